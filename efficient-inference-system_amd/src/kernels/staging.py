"""Host->device uploads of small int32 metadata through a persistent pinned ring.

Allocating fresh pinned memory for every upload (torch's `pin_memory()`) costs far more than the
copy itself when the previous buffers are still in flight. Here each device owns a ring of pinned
slots; an upload copies into the next slot, enqueues an asynchronous copy on the current stream
and records an event, and a slot is reused only after its event has completed (normally long
before the ring wraps).
"""
from __future__ import annotations

import numpy as np
import torch

_SLOT_BYTES = 256 * 1024
_SLOTS = 32


class _PinnedRing:
    def __init__(self, device: torch.device):
        self.device = device
        self.host = torch.empty(_SLOTS * _SLOT_BYTES, dtype=torch.uint8, pin_memory=True)
        self.host_np = self.host.numpy()
        self.events: list[torch.cuda.Event | None] = [None] * _SLOTS
        self.next = 0

    def upload_into(self, arr: np.ndarray, dst: torch.Tensor) -> None:
        """Asynchronous copy of arr into the first arr.nbytes bytes of the device tensor dst
        (contiguous), through the next pinned slot."""
        nbytes = arr.nbytes
        if nbytes > _SLOT_BYTES:
            dst.view(-1).view(torch.uint8)[:nbytes].copy_(torch.from_numpy(arr.view(np.uint8).reshape(-1)).pin_memory(),
                                                          non_blocking=True)
            return
        i = self.next
        self.next = (i + 1) % _SLOTS
        ev = self.events[i]
        if ev is not None:
            ev.synchronize()
        self.host_np[i * _SLOT_BYTES:i * _SLOT_BYTES + nbytes] = arr.view(np.uint8).reshape(-1)
        dst.view(-1).view(torch.uint8)[:nbytes].copy_(self.host[i * _SLOT_BYTES:i * _SLOT_BYTES + nbytes],
                                                      non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self.events[i] = ev

    def upload(self, arr: np.ndarray) -> torch.Tensor:
        nbytes = arr.nbytes
        if nbytes > _SLOT_BYTES:
            return torch.from_numpy(arr).pin_memory().to(self.device, non_blocking=True)
        i = self.next
        self.next = (i + 1) % _SLOTS
        ev = self.events[i]
        if ev is not None:
            ev.synchronize()
        view = self.host_np[i * _SLOT_BYTES:i * _SLOT_BYTES + nbytes]
        view[:] = arr.view(np.uint8).reshape(-1)
        src = self.host[i * _SLOT_BYTES:i * _SLOT_BYTES + nbytes]
        out = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        out.copy_(src, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self.events[i] = ev
        return out.view(torch.from_numpy(arr[:0]).dtype)


_rings: dict[int, _PinnedRing] = {}


def upload(arr: np.ndarray, device: torch.device) -> torch.Tensor:
    """Asynchronously copy a contiguous numpy array to `device`; returns a flat device tensor of
    the same dtype, valid in stream order on the current stream."""
    arr = np.ascontiguousarray(arr)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ring = _rings.get(idx)
    if ring is None:
        ring = _rings[idx] = _PinnedRing(torch.device("cuda", idx))
    return ring.upload(arr)


def upload_into(arr: np.ndarray, dst: torch.Tensor) -> None:
    """Asynchronously copy a contiguous numpy array into the leading bytes of the contiguous
    device tensor dst (on the current stream), without an intermediate device buffer."""
    arr = np.ascontiguousarray(arr)
    if not dst.is_contiguous() or dst.numel() * dst.element_size() < arr.nbytes:
        raise ValueError("upload_into: destination must be contiguous and large enough")
    device = dst.device
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ring = _rings.get(idx)
    if ring is None:
        ring = _rings[idx] = _PinnedRing(torch.device("cuda", idx))
    ring.upload_into(arr, dst)
