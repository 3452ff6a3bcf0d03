"""pa_hbm_read_probe on the device: it reads the whole buffer and, for a buffer of zeros, leaves
its sink untouched (its single conditional store never fires)."""
import pytest
import torch

from src.kernels import _lib

pytestmark = pytest.mark.gpu


def test_read_probe_reads_and_writes_nothing_for_zeros(device):
    lib = _lib.load()
    buf = torch.zeros(64 << 20, dtype=torch.uint8, device=device)
    wgs = 1024
    sink = torch.full((wgs,), 7, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    for n in (buf.numel(), buf.numel() - 16 * 1000, 16):  # whole, ragged tail, one vector
        _lib.check(lib.pa_hbm_read_probe(buf.data_ptr(), n, sink.data_ptr(), wgs, stream), "pa_hbm_read_probe")
    torch.cuda.synchronize()
    assert bool((sink == 7).all())
