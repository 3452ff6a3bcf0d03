"""The bandwidth probes on the device: pa_hbm_read_probe reads the whole buffer in every shape it
builds and pa_hbm_chunk_read_probe every chunk its order names, and for a buffer of zeros neither
writes its sink (their single conditional store never fires)."""
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
    for threads in (256, 512, 1024):
        for depth in (1, 4, 8):
            for n in (buf.numel(), buf.numel() - 16 * 1000, 16):  # whole, ragged tail, one vector
                _lib.check(lib.pa_hbm_read_probe(buf.data_ptr(), n, sink.data_ptr(), wgs, threads, depth, stream),
                           "pa_hbm_read_probe")
    torch.cuda.synchronize()
    assert bool((sink == 7).all())


def test_chunk_read_probe_follows_its_order_and_writes_nothing_for_zeros(device):
    lib = _lib.load()
    chunks = 4096  # 16 MiB of 4 KB chunks
    buf = torch.zeros(chunks * 4096, dtype=torch.uint8, device=device)
    g = torch.Generator().manual_seed(3)
    order = torch.randperm(chunks, generator=g).to(torch.int32)
    order[5] = -1  # out-of-range ids are skipped
    order[9] = chunks
    order = order.to(device)
    wgs = 256
    sink = torch.full((wgs,), 7, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream(device).cuda_stream
    for depth in (1, 2, 4):
        for n in (chunks, chunks - 3, 1):
            _lib.check(lib.pa_hbm_chunk_read_probe(buf.data_ptr(), order.data_ptr(), n, sink.data_ptr(), wgs, depth,
                                                   stream), "pa_hbm_chunk_read_probe")
    torch.cuda.synchronize()
    assert bool((sink == 7).all())
