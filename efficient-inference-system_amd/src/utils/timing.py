"""Wall-clock timing of a code section with device synchronisation on both ends.

Same contract as src/utils/timing.py:11-21 of the reference: on "cuda" the whole device is
synchronised before the start and before the end stamp, so the elapsed time covers all work the
section queued. This elapsed time is what the serving schedulers advance their virtual clock by.
"""
import time
from contextlib import contextmanager

import torch


class _TimerResult:
    def __init__(self):
        self.elapsed_ms = 0.0


def _is_gpu(device) -> bool:
    if isinstance(device, torch.device):
        return device.type == "cuda"
    return str(device).startswith("cuda")


@contextmanager
def timed_section(device: str = "cpu"):
    result = _TimerResult()
    gpu = _is_gpu(device) and torch.cuda.is_available()
    if gpu:
        torch.cuda.synchronize()
    start = time.perf_counter()
    yield result
    if gpu:
        torch.cuda.synchronize()
    end = time.perf_counter()
    result.elapsed_ms = (end - start) * 1000.0
