"""pa_decode_noalloc (arrival counters and split-K records in the library's fixed per-device
scratch array) against pa_decode with a caller workspace, called through the C ABI: same kernels,
so the outputs must be bit-identical. Two calls in a row, the second with a smaller batch, so the second reads records
the first left behind in the shared array only if it were wrong. Also checked against the
oracle (fp32 within 1e-4, bf16 KV within 1e-4 of the oracle on the same bf16 values)."""
import math

import numpy as np
import pytest
import torch

import oracle
from src import workloads
from src.kernels import _lib

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 16 << 20  # PA_DECODE_NOALLOC_SCRATCH_BYTES in include/paged_hip.h


def lib():
    return _lib.load()


def make(device, seed, lens, H, Hd, kv_dtype):
    g = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(L / 16) for L in lens)
    N = need + 5
    perm = torch.randperm(N, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / 16)
        lists.append(perm[pos:pos + n])
        pos += n
    B = len(lens)
    q = torch.randn(B, H, 1, Hd, generator=g).to(device)
    k = torch.randn(N, H, 16, Hd, generator=g).to(kv_dtype).to(device)
    v = torch.randn(N, H, 16, Hd, generator=g).to(kv_dtype).to(device)
    return workloads._batch(q, k, v, lists, list(lens), [1] * B, device)


def call(lb, b, split_blocks, noalloc):
    B, H, _, Hd = b.q.shape
    out = torch.full_like(b.q, float("nan"))
    pt = b.page_table
    max_pages = pt.shape[1]
    stream = torch.cuda.current_stream(b.q.device).cuda_stream
    common = (b.q.data_ptr(), b.q.stride(0), b.q.stride(1),
              out.data_ptr(), out.stride(0), out.stride(1), _lib.PA_DTYPE_F32,
              b.k_pool.data_ptr(), b.v_pool.data_ptr(), _lib.dtype_code(b.k_pool.dtype), b.k_pool.shape[0],
              pt.data_ptr(), pt.stride(0), max_pages,
              b.seq_lens_t.data_ptr(), b.cur_lens_t.data_ptr(), None,
              B, H, Hd, 16, 1.0 / math.sqrt(Hd), split_blocks)
    if noalloc:
        st = lb.pa_decode_noalloc(*common, stream)
    else:
        need = lb.pa_decode_workspace_size(B, H, Hd, max_pages, split_blocks)
        ws = torch.zeros(max(need, 1), dtype=torch.uint8, device=b.q.device)  # arrival counters start at zero
        st = lb.pa_decode(*common, ws.data_ptr(), need, stream)
        torch.cuda.synchronize()
        del ws
    _lib.check(st, "pa_decode_noalloc" if noalloc else "pa_decode")
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("kv_dtype,Hd", [(torch.bfloat16, 128), (torch.float32, 64)])
def test_noalloc_matches_workspace_entry_point(device, kv_dtype, Hd):
    lb = lib()
    H = 8
    cases = [
        # (seed, lengths, split_blocks): the first call needs 4 x 8 x 16 split records, the second
        # a smaller batch with fewer splits per request
        (11, [4000, 2500, 3100, 1800], 16),
        (12, [700, 1300], 16),
    ]
    for seed, lens, split in cases:
        print(f"noalloc decode: kv={kv_dtype} Hd={Hd} lens={lens} split_blocks={split}", flush=True)
        b = make(device, seed, lens, H, Hd, kv_dtype)
        need = lb.pa_decode_workspace_size(len(lens), H, Hd, b.page_table.shape[1], split)
        assert 0 < need <= SCRATCH_BYTES
        got = call(lb, b, split, noalloc=True)
        want = call(lb, b, split, noalloc=False)
        assert torch.equal(got, want)
        ref = oracle.paged_attention(b.q.cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                     b.cur_lens)
        assert float(np.abs(got.cpu().numpy() - ref).max()) <= 1e-4


def test_noalloc_without_split_and_over_the_limit(device):
    lb = lib()
    b = make(device, 13, [300, 900, 40], 8, 64, torch.float32)
    got = call(lb, b, 0, noalloc=True)  # no split: the scratch is not touched
    assert torch.equal(got, call(lb, b, 0, noalloc=False))
    # 64 requests x 64 heads x 2048 pages in 1-block splits need far more than the array: the
    # call is refused on the host before anything is launched. Every pointer is a real device
    # buffer of the stated size, and every request is empty (length 0, a page table of -1), so a
    # launch, had the host check been skipped, would only write zeros into `out` (no split record
    # is written for an empty request) and the assertion on `out` below would report it.
    B, H, Hd, pages = 64, 64, 128, 2048
    assert lb.pa_decode_workspace_size(B, H, Hd, pages, 1) > SCRATCH_BYTES
    q = torch.zeros(B, H, 1, Hd, device=device)
    out = torch.full_like(q, float("nan"))
    k = torch.zeros(1, H, 16, Hd, dtype=torch.bfloat16, device=device)
    v = torch.zeros_like(k)
    pt = torch.full((B, pages), -1, dtype=torch.int32, device=device)
    lens = torch.zeros(B, dtype=torch.int32, device=device)
    cur = torch.ones(B, dtype=torch.int32, device=device)
    st = lb.pa_decode_noalloc(q.data_ptr(), q.stride(0), q.stride(1), out.data_ptr(), out.stride(0), out.stride(1),
                              _lib.PA_DTYPE_F32, k.data_ptr(), v.data_ptr(), _lib.PA_DTYPE_BF16, k.shape[0],
                              pt.data_ptr(), pt.stride(0), pages, lens.data_ptr(), cur.data_ptr(), None,
                              B, H, Hd, 16, 0.1, 1, torch.cuda.current_stream(device).cuda_stream)
    torch.cuda.synchronize()
    assert st == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"fixed scratch" in lb.pa_last_error_message()
    assert bool(torch.isnan(out).all()), "the refused call must not launch"
