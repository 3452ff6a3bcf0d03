"""HIP paged DECODE attention vs the oracle (fp32 within 1e-4; bf16 KV within 2e-2 of the fp32
result on the unrounded values and within 1e-4 of the oracle on the same bf16 values)."""
import math
import os

import numpy as np
import pytest
import torch

import oracle
from src import workloads
from src.kernels import _lib
from src.kernels.hip_paged_attention import paged_attention_decode_hip

pytestmark = pytest.mark.gpu
NTHREADS = min(16, os.cpu_count() or 1)


def run(batch, **kw):
    return paged_attention_decode_hip(batch.q, batch.k_pool, batch.v_pool, batch.page_table, batch.seq_lens_t,
                                      batch.cur_lens_t, **kw)


def oracle_out(batch):
    return oracle.paged_attention(batch.q.cpu(), batch.k_pool.cpu(), batch.v_pool.cpu(), batch.block_lists,
                                  batch.seq_lens, batch.cur_lens, nthreads=NTHREADS)


def make_batch(device, seed, lens, curs, H, Hd, bs=16, kv_dtype=torch.float32, io_dtype=torch.float32, spare=7):
    g = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(L / bs) for L in lens)
    N = need + spare
    perm = torch.randperm(N, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / bs)
        lists.append(perm[pos:pos + n])
        pos += n
    B = len(lens)
    q = torch.randn(B, H, 1, Hd, generator=g).to(io_dtype).to(device)
    k = torch.randn(N, H, bs, Hd, generator=g).to(kv_dtype).to(device)
    v = torch.randn(N, H, bs, Hd, generator=g).to(kv_dtype).to(device)
    return workloads._batch(q, k, v, lists, list(lens), list(curs), device)


def max_err(got, want):
    return float(np.abs(got.float().cpu().numpy() - want).max()) if want.size else 0.0


def test_single_decode_config(device):
    b = workloads.single_decode(seed=0, device=device)
    print("single decode: B=1 H=8 Hd=64 L=128", flush=True)
    assert max_err(run(b), oracle_out(b)) <= 1e-4


@pytest.mark.parametrize("layer", range(6))
def test_ragged_decode_config(device, layer):
    b = workloads.ragged_decode(seed=0, layer=layer, device=device)
    print(f"ragged decode layer {layer}: lens={b.seq_lens}", flush=True)
    assert max_err(run(b), oracle_out(b)) <= 1e-4


@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("io_dtype", [torch.float32, torch.bfloat16])
def test_decode_fast_kernel_variants(device, kv_dtype, head_dim, io_dtype):
    lens = [1, 15, 16, 17, 100, 257, 700, 1500]
    b = make_batch(device, 3, lens, [1] * len(lens), H=4, Hd=head_dim, kv_dtype=kv_dtype, io_dtype=io_dtype)
    print(f"decode variant kv={kv_dtype} hd={head_dim} io={io_dtype}", flush=True)
    got = run(b)
    assert got.dtype == io_dtype
    want = oracle.paged_attention(b.q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)
    tol = 1e-4 if io_dtype == torch.float32 else 1e-2  # bf16 output rounding: |out| <= ~4, ulp 2^-6
    assert max_err(got, want) <= tol


def test_bf16_kv_against_unrounded_fp32(device):
    lens = [33, 400, 1024, 3000]
    b32 = make_batch(device, 4, lens, [1] * 4, H=8, Hd=128, kv_dtype=torch.float32)
    want = oracle_out(b32)
    got = paged_attention_decode_hip(b32.q, b32.k_pool.to(torch.bfloat16), b32.v_pool.to(torch.bfloat16),
                                     b32.page_table, b32.seq_lens_t, b32.cur_lens_t)
    assert max_err(got, want) <= 2e-2


@pytest.mark.parametrize("split_blocks", [1, 3, 16, 32, 129])
def test_split_path_matches_oracle_and_unsplit(device, split_blocks):
    lens = [5, 64, 200, 1000, 2049]
    b = make_batch(device, 5, lens, [1] * 5, H=3, Hd=64)
    print(f"split decode split_blocks={split_blocks}", flush=True)
    got = run(b, split_blocks=split_blocks)
    assert max_err(got, oracle_out(b)) <= 1e-4
    assert max_err(got, run(b, split_blocks=0).cpu().numpy()) <= 1e-5
    # the merge order is fixed, so a second call reproduces the first bit for bit
    assert torch.equal(got, run(b, split_blocks=split_blocks))


@pytest.mark.parametrize("io_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("split_blocks", [1, 5, 64])
def test_split_path_hd128_bf16_kv(device, split_blocks, io_dtype):
    # 1-block splits give 190 records for the longest request (merged 64 per pass), 64-block
    # splits one or two; lengths 0 and 16 leave a single split that writes the output itself
    lens = [0, 16, 17, 1023, 3031]
    b = make_batch(device, 11, lens, [1] * 5, H=4, Hd=128, kv_dtype=torch.bfloat16, io_dtype=io_dtype)
    print(f"split decode hd128 bf16 KV split_blocks={split_blocks} io={io_dtype}", flush=True)
    got = run(b, split_blocks=split_blocks)
    want = oracle.paged_attention(b.q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)
    tol = 1e-4 if io_dtype == torch.float32 else 1e-2
    assert max_err(got, want) <= tol
    assert max_err(got, run(b, split_blocks=0).float().cpu().numpy()) <= (1e-5 if io_dtype == torch.float32 else 1e-2)
    assert torch.count_nonzero(got[0]).item() == 0


@pytest.mark.parametrize("Hd,bs", [(16, 8), (32, 16), (96, 16), (64, 32), (80, 4)])
def test_generic_kernel_shapes(device, Hd, bs):
    lens = [1, 9, 40, 130]
    b = make_batch(device, 6, lens, [1] * 4, H=2, Hd=Hd, bs=bs)
    print(f"generic decode Hd={Hd} bs={bs}", flush=True)
    assert max_err(run(b), oracle_out(b)) <= 1e-4


def test_edge_lengths_and_current_lengths(device):
    # empty request, single key, block edges; current_lengths 0 (attend all), >1 (fewer keys),
    # > seq_len (no key -> zeros)
    lens = [0, 1, 15, 16, 17, 33, 50, 64]
    curs = [1, 1, 0, 2, 17, 40, 3, 1]
    b = make_batch(device, 7, lens, curs, H=2, Hd=64)
    got = run(b)
    want = oracle_out(b)
    assert max_err(got, want) <= 1e-4
    assert torch.count_nonzero(got[0]).item() == 0 and torch.count_nonzero(got[5]).item() == 0


def test_strided_views_like_the_model(device):
    B, H, Hd = 4, 8, 64
    base = make_batch(device, 8, [70, 16, 300, 5], [1] * 4, H=H, Hd=Hd)
    x = torch.randn(B, 1, H * Hd, device=device)
    q = x.view(B, 1, H, Hd).transpose(1, 2)  # the model's [B, H, T, Hd] view
    assert q.stride() == (H * Hd, Hd, H * Hd, 1)
    out = paged_attention_decode_hip(q, base.k_pool, base.v_pool, base.page_table, base.seq_lens_t, base.cur_lens_t)
    assert out.stride() == q.stride()
    want = oracle.paged_attention(q.cpu().contiguous(), base.k_pool.cpu(), base.v_pool.cpu(), base.block_lists,
                                  base.seq_lens, base.cur_lens)
    assert max_err(out, want) <= 1e-4


def test_order_does_not_change_results(device):
    lens = [300, 20, 1000, 64, 513]
    b = make_batch(device, 9, lens, [1] * 5, H=4, Hd=128, kv_dtype=torch.bfloat16)
    order = torch.tensor(sorted(range(5), key=lambda i: -lens[i]), dtype=torch.int32, device=device)
    a1 = run(b)
    a2 = run(b, order=order)
    assert torch.equal(a1, a2)


def test_negative_page_entries_are_skipped(device):
    b = make_batch(device, 10, [64, 64], [1, 1], H=2, Hd=64)
    pt = b.page_table.clone()
    pt[0, 1] = -1  # keys 16..31 of request 0 are skipped, like the reference kernels skip -1 pages
    got = paged_attention_decode_hip(b.q, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t)
    # equivalent request: drop block 1 and shorten by 16 keys
    k = b.k_pool.cpu()
    want0 = oracle.paged_attention(b.q[:1].cpu(), k, b.v_pool.cpu(), [[b.block_lists[0][0]] + b.block_lists[0][2:]],
                                   [48], [1])
    assert max_err(got[:1], want0) <= 1e-4
    assert max_err(got[1:], oracle_out(b)[1:]) <= 1e-4


def test_large_ragged_decode_parity(device):
    """Full large ragged decode (B=256, 32x128, bf16 KV): every request against the oracle on the
    same bf16 values, 32 requests at a time (their blocks gathered to the host)."""
    b = workloads.large_decode(seed=0, device=device)
    print(f"large decode: B={b.batch} total tokens={sum(b.seq_lens)} pool={b.k_pool.shape[0]}", flush=True)
    got = run(b)
    torch.cuda.synchronize()
    lens = b.seq_lens
    worst = 0.0
    for c0 in range(0, b.batch, 32):
        rows = list(range(c0, min(c0 + 32, b.batch)))
        ids = torch.tensor([i for r in rows for i in b.block_lists[r]], device=device, dtype=torch.long)
        k = oracle._np(b.k_pool.index_select(0, ids).cpu())
        v = oracle._np(b.v_pool.index_select(0, ids).cpu())
        lists, pos = [], 0
        for r in rows:
            lists.append(list(range(pos, pos + len(b.block_lists[r]))))
            pos += len(b.block_lists[r])
        want = oracle.paged_attention(b.q[c0:c0 + len(rows)].cpu(), k, v, lists, lens[c0:c0 + len(rows)],
                                      [1] * len(rows), nthreads=NTHREADS)
        err = max_err(got[c0:c0 + len(rows)], want)
        worst = max(worst, err)
        print(f"  requests {c0}..{rows[-1]} (L {min(lens[r] for r in rows)}..{max(lens[r] for r in rows)}): "
              f"max err {err:.2e}", flush=True)
        assert err <= 1e-4
        del k, v
    print(f"  all {b.batch} requests: max err {worst:.2e}", flush=True)
    del b
    torch.cuda.empty_cache()


def test_large_ragged_decode_bf16_against_unrounded_fp32(device):
    """Large ragged decode shape (32 heads x 128, block 16, lengths of the 256-request batch) on 16
    of its requests chosen from the shortest to the longest (the 32k one included): K and V are
    drawn in fp32, the kernel runs on their bf16 rounding, and each request is compared with the
    oracle on the UNROUNDED fp32 values (bf16-KV tolerance 2e-2) and on the same bf16 values
    (1e-4)."""
    lens_all = workloads.large_decode_lengths(0)
    by_len = sorted(range(len(lens_all)), key=lambda i: lens_all[i])
    rows = sorted({by_len[round(j * (len(by_len) - 1) / 15)] for j in range(16)})
    assert len(rows) == 16 and max(lens_all[r] for r in rows) == max(lens_all)
    b = workloads.large_decode(seed=0, device=device, rows=rows, kv_dtype=torch.float32)
    print(f"large decode vs unrounded fp32: requests {rows}, lengths {b.seq_lens}", flush=True)
    kb, vb = b.k_pool.to(torch.bfloat16), b.v_pool.to(torch.bfloat16)
    got = paged_attention_decode_hip(b.q, kb, vb, b.page_table, b.seq_lens_t, b.cur_lens_t)
    torch.cuda.synchronize()
    # only the blocks the requests use go to the host, renumbered in list order
    ids = torch.tensor([i for x in b.block_lists for i in x], device=device, dtype=torch.long)
    lists, pos = [], 0
    for x in b.block_lists:
        lists.append(list(range(pos, pos + len(x))))
        pos += len(x)
    q = b.q.cpu()
    want32 = oracle.paged_attention(q, oracle._np(b.k_pool.index_select(0, ids)),
                                    oracle._np(b.v_pool.index_select(0, ids)), lists, b.seq_lens, b.cur_lens,
                                    nthreads=NTHREADS)
    want16 = oracle.paged_attention(q, oracle._np(kb.index_select(0, ids)), oracle._np(vb.index_select(0, ids)),
                                    lists, b.seq_lens, b.cur_lens, nthreads=NTHREADS)
    g = got.float().cpu().numpy()
    e32 = np.abs(g - want32).reshape(len(rows), -1).max(axis=1)
    e16 = np.abs(g - want16).reshape(len(rows), -1).max(axis=1)
    for r, L, a, c in zip(rows, b.seq_lens, e32, e16):
        print(f"  request {r:3d} L={L:5d}: max err vs unrounded fp32 {a:.2e}, vs same bf16 values {c:.2e}",
              flush=True)
    print(f"  worst: {e32.max():.2e} vs unrounded fp32 (bound 2e-2), {e16.max():.2e} vs bf16 values (1e-4)",
          flush=True)
    assert float(e32.max()) <= 2e-2
    assert float(e16.max()) <= 1e-4
    del b, kb, vb
    torch.cuda.empty_cache()


def test_in_launch_split_merge_shares_one_workspace_across_shapes_and_graph_replays(device):
    """Splits of at most 8 per (request, head) are merged in the launch by the split that arrives
    last, counted in the workspace's leading arrival counters. Calls of different shapes (and
    merge modes: more than 8 splits take the merge launch) share the decode workspace; each must
    match the oracle and leave every counter at zero, also when replayed from a graph with eager
    calls of other shapes in between."""
    from src.kernels.hip_paged_attention import _workspaces

    cases = [
        (make_batch(device, 31, [130, 1000, 17, 600, 257, 990, 1, 700], [1] * 8, H=8, Hd=64), 16),  # <= 4 splits
        (make_batch(device, 32, [3000, 40, 2049], [1] * 3, H=4, Hd=128, kv_dtype=torch.bfloat16), 32),  # <= 6
        (make_batch(device, 33, [1500, 900], [1] * 2, H=3, Hd=64), 8),  # 12 splits: merge launch
    ]
    wants = [oracle_out(b) for b, _ in cases]

    def counters_zero():
        ws = _workspaces.get((device.index if device.index is not None else 0, "decode"))
        return ws is None or int(ws[:256 << 10].view(torch.int32).abs().sum()) == 0

    for rep in range(2):
        for (b, split), want in zip(cases, wants):
            print(f"in-launch merge rep {rep}: lens {b.seq_lens} split {split}", flush=True)
            assert max_err(run(b, split_blocks=split), want) <= 1e-4
            torch.cuda.synchronize()
            assert counters_zero()
    b, split = cases[0]
    out = torch.empty_like(b.q)
    call = lambda: run(b, split_blocks=split, out=out)
    call()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for rep in range(3):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert max_err(out, wants[0]) <= 1e-4, rep
        assert counters_zero()
        b2, split2 = cases[1 + rep % 2]
        assert max_err(run(b2, split_blocks=split2), wants[1 + rep % 2]) <= 1e-4
        torch.cuda.synchronize()
        assert counters_zero()


def test_captured_graph_keeps_its_workspace_when_a_larger_one_is_needed(device):
    """A graph captured with a split decode records its workspace's address; a later call that
    needs a larger workspace makes the wrapper allocate a new one, and the old one must stay
    allocated: after fresh allocations are filled with other data, the graph still replays to the
    oracle's result and leaves its counters at zero."""
    from src.kernels import hip_paged_attention as hpa

    small = make_batch(device, 41, [300, 900, 650, 128], [1] * 4, H=8, Hd=64)
    big = make_batch(device, 42, [3000, 2900, 2800, 2700, 2600, 2500, 2400, 2300], [1] * 8, H=32, Hd=128,
                     kv_dtype=torch.bfloat16)
    want_small = oracle_out(small)
    idx = device.index if device.index is not None else 0
    prev = hpa._workspaces.pop((idx, "decode"), None)  # start from a fresh (1 MiB) workspace
    if prev is not None:
        hpa._retired_workspaces.append(prev)
    out = torch.empty_like(small.q)
    call = lambda: run(small, split_blocks=16, out=out)
    call()  # allocates the workspace this graph records
    torch.cuda.synchronize()
    old = hpa._workspaces[(idx, "decode")]
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    need = _lib.load().pa_decode_workspace_size(8, 32, 128, big.page_table.shape[1], 16)
    assert need > old.numel()  # the big call grows the workspace
    print(f"workspace {old.numel()} -> {need} bytes", flush=True)
    assert max_err(run(big, split_blocks=16), oracle_out(big)) <= 2e-2
    torch.cuda.synchronize()
    assert hpa._workspaces[(idx, "decode")].data_ptr() != old.data_ptr()
    filler = [torch.full((old.numel() // 4,), 7.0, device=device) for _ in range(4)]  # reuses freed memory, if any
    torch.cuda.synchronize()
    for rep in range(2):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert max_err(out, want_small) <= 1e-4, rep
        assert int(old[:256 << 10].view(torch.int32).abs().sum()) == 0
    del filler
