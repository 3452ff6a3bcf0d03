"""HIP chunked-PREFILL attention vs the oracle (fp32 KV within 1e-4, bf16 KV within 2e-2),
including the reference's padded-row semantics and the append-then-attend order."""
import math
import os
import random

import numpy as np
import pytest
import torch

import oracle
from src import workloads
from src.cache.paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState
from src.kernels.hip_paged_attention import paged_attention_decode_hip, paged_attention_prefill_hip
from src.kernels.paged_attention import paged_attention

pytestmark = pytest.mark.gpu
NTHREADS = min(16, os.cpu_count() or 1)


def max_err(got, want):
    return float(np.abs(got.float().cpu().numpy() - want).max()) if want.size else 0.0


def make_prefill(device, seed, ctx, curs, T, H, Hd, bs=16, kv_dtype=torch.float32):
    """Requests whose cache holds ctx[b] + curs[b] tokens (the chunk already appended)."""
    g = torch.Generator().manual_seed(seed)
    lens = [c0 + c for c0, c in zip(ctx, curs)]
    need = sum(math.ceil(L / bs) for L in lens)
    N = need + 3
    perm = torch.randperm(N, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / bs)
        lists.append(perm[pos:pos + n])
        pos += n
    B = len(lens)
    q = torch.randn(B, H, T, Hd, generator=g).to(device)
    k = torch.randn(N, H, bs, Hd, generator=g).to(kv_dtype).to(device)
    v = torch.randn(N, H, bs, Hd, generator=g).to(kv_dtype).to(device)
    return workloads._batch(q, k, v, lists, lens, list(curs), device)


def run(b, **kw):
    return paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t, **kw)


def oracle_out(b):
    return oracle.paged_attention(b.q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)


# seed 0 draws four 256-token chunks; seeds 2 and 4 mix 128- and 256-token chunks, so rows past a
# 128-token chunk are padded rows inside the 256-row batch (the reference's padded-row semantics)
@pytest.mark.parametrize("seed,kv_dtype,tol", [(0, torch.float32, 1e-4), (2, torch.float32, 1e-4),
                                               (4, torch.float32, 1e-4), (2, torch.bfloat16, 2e-2)])
def test_chunked_prefill_config(device, seed, kv_dtype, tol):
    w = workloads.chunked_prefill(seed=seed, device=device, kv_dtype=kv_dtype)
    B = len(w["prev_lens"])
    print(f"chunked prefill seed={seed} kv={kv_dtype} ctx={w['prev_lens']} chunk={w['chunk_lens']}", flush=True)
    pool = LayerBlockPool(block_size=16, initial_blocks=w["k_pool"].shape[0], growth_factor=2.0, dtype=kv_dtype)
    pool.ensure_initialized(8, 64, torch.float32, device)
    pool.k_blocks.copy_(w["k_pool"])
    pool.v_blocks.copy_(w["v_pool"])
    before_k, before_v = pool.k_blocks.cpu(), pool.v_blocks.cpu()
    states = []
    for lst, c0 in zip(w["block_lists"], w["prev_lens"]):
        nctx = math.ceil(c0 / 16)
        states.append(PagedKVCacheState(pool=pool, block_ids=list(lst[:nctx]), seq_len=c0))
    # the chunk's blocks come from the free list; hand the workload's block choice to the states
    # by making exactly those ids the next ones popped
    chunk_ids = [lst[math.ceil(c0 / 16):] for lst, c0 in zip(w["block_lists"], w["prev_lens"])]
    order = [i for ids in chunk_ids for i in ids]
    pool.free_block_ids = [i for i in range(pool.capacity_blocks) if i not in set(order)] + order[::-1]
    batch = BatchedPagedKVCache(states=states, pool=pool)
    cur = torch.tensor(w["chunk_lens"])
    batch.append_batch(w["k_new"], w["v_new"], current_lengths=cur)
    assert [s.block_ids for s in states] == w["block_lists"]
    # append is bit-exact against the oracle
    nk, nv = oracle._np(before_k).copy(), oracle._np(before_v).copy()
    oracle.append(w["k_new"].cpu(), w["v_new"].cpu(), nk, nv, w["block_lists"], w["prev_lens"], w["chunk_lens"])
    assert np.array_equal(oracle._np(pool.k_blocks.cpu()), nk) and np.array_equal(oracle._np(pool.v_blocks.cpu()), nv)
    out = paged_attention("hip_paged", w["q"], batch, cur)
    want = oracle.paged_attention(w["q"].cpu(), nk, nv, w["block_lists"], w["seq_lens"], w["chunk_lens"],
                                  nthreads=NTHREADS)
    err = max_err(out, want)
    print(f"  max err {err:.2e}", flush=True)
    assert err <= tol


@pytest.mark.parametrize("seed", [0, 2])
@pytest.mark.parametrize("kv_dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_kv_staging_lds_and_registers_agree(device, monkeypatch, seed, kv_dtype, tol):
    """The 16-row kernel's two KV stagings (LDS-direct copies into a per-wavefront ring, or loads
    straight into the operand registers) run the same products in the same order: bit-identical
    outputs on the chunked-prefill workload, unsplit and split (down to one block per split), and
    within tolerance of the oracle."""
    w = workloads.chunked_prefill(seed=seed, device=device, kv_dtype=kv_dtype)
    lists = w["block_lists"]
    b = workloads._batch(w["q"], w["k_pool"], w["v_pool"], lists, w["seq_lens"], w["chunk_lens"], device)
    print(f"kv staging seed={seed} kv={kv_dtype} ctx={w['prev_lens']} chunk={w['chunk_lens']}", flush=True)
    outs = {}
    for staging in ("lds", "regs"):
        monkeypatch.setenv("PAGED_HIP_PREFILL_STAGING", staging)
        for split in (0, 1, 3):
            outs[staging, split] = run(b, split_blocks=split)
    for split in (0, 1, 3):
        assert torch.equal(outs["lds", split], outs["regs", split]), split
    err = max_err(outs["lds", 0], oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= tol


@pytest.mark.parametrize("kv_dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
def test_kv_staging_over_several_page_table_chunks(device, monkeypatch, kv_dtype, tol):
    """Contexts of 4.4k and 5.1k tokens, unsplit: each wavefront walks 69-80 blocks, so the walk
    restarts at a second 64-entry page-table chunk of 5-16 blocks. Both stagings bit-identical
    and within tolerance of the oracle."""
    b = make_prefill(device, 5, [4400, 5090], [32, 21], 32, 2, 64, kv_dtype=kv_dtype)
    print(f"kv staging long contexts kv={kv_dtype}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "tile")
    outs = {}
    for staging in ("lds", "regs"):
        monkeypatch.setenv("PAGED_HIP_PREFILL_STAGING", staging)
        outs[staging] = run(b, split_blocks=0)
    assert torch.equal(outs["lds"], outs["regs"])
    err = max_err(outs["lds"], oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= tol


@pytest.mark.parametrize("kv_dtype", [torch.float32, torch.bfloat16])
def test_kv_staging_on_a_large_grid(device, monkeypatch, kv_dtype):
    """8 requests x 8 heads x 256 rows (1024 workgroups, past the grid where fp32 KV switches to
    register staging): both stagings bit-identical and within tolerance of the oracle."""
    b = workloads.large_prefill(seed=3, device=device, batch=8, heads=8, head_dim=64, chunk=256, ctx_lo=0,
                                ctx_hi=768, kv_dtype=kv_dtype)
    print(f"kv staging large grid kv={kv_dtype}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_STAGING", "lds")
    lds = run(b)
    monkeypatch.setenv("PAGED_HIP_PREFILL_STAGING", "regs")
    regs = run(b)
    assert torch.equal(lds, regs)
    monkeypatch.delenv("PAGED_HIP_PREFILL_STAGING")
    assert torch.equal(run(b), regs if kv_dtype == torch.float32 else lds)
    err = max_err(lds, oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= (1e-4 if kv_dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("seed", [0, 2, 4])
def test_split_step_kernel_chunked(device, monkeypatch, seed):
    """The split-step kernel (8 wavefronts per 32-row tile, each taking every 8th 32-key step
    through its own LDS ring, states merged in LDS) on the chunked-prefill workload with bf16 KV,
    against the oracle on the same bf16 values."""
    w = workloads.chunked_prefill(seed=seed, device=device, kv_dtype=torch.bfloat16)
    b = workloads._batch(w["q"], w["k_pool"], w["v_pool"], w["block_lists"], w["seq_lens"], w["chunk_lens"], device)
    print(f"split-step seed={seed} ctx={w['prev_lens']} chunk={w['chunk_lens']}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "split")
    err = max_err(run(b), oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= 2e-2


@pytest.mark.parametrize("T,ctx,curs", [
    (40, [0, 37, 300], [40, 1, 25]),         # rows past T in the last tile, a one-token chunk
    (8, [16, 0], [8, 3]),                    # one partial tile, an empty context
    (96, [700, 0, 33], [96, 80, 17]),        # padded rows, contexts off block boundaries
    (64, [9000], [64]),                      # 286 steps: two 32-step chunks per wavefront
])
@pytest.mark.parametrize("io_dtype", [torch.float32, torch.bfloat16])
def test_split_step_kernel_ragged(device, monkeypatch, T, ctx, curs, io_dtype):
    """The split-step kernel forced on ragged shapes with bf16 KV, fp32 and bf16 q/out."""
    b = make_prefill(device, 17, ctx, curs, T, 8, 64, kv_dtype=torch.bfloat16)
    if io_dtype == torch.bfloat16:
        b = workloads._batch(b.q.to(torch.bfloat16), b.k_pool, b.v_pool, b.block_lists, b.seq_lens, b.cur_lens, device)
    print(f"split-step ragged T={T} ctx={ctx} curs={curs} io={io_dtype}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "split")
    err = max_err(run(b), oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= (2e-2 if io_dtype == torch.float32 else 3e-2)


@pytest.mark.parametrize("seed", range(12))
def test_split_step_kernel_random(device, monkeypatch, seed):
    """Random batches through the split-step kernel: 1-4 requests, 1-8 heads, chunks of 1-300 rows
    with empty, partial, full and over-long current lengths, contexts up to 1500 tokens."""
    r = random.Random(5000 + seed)
    B, H, T = r.randint(1, 4), r.randint(1, 8), r.randint(1, 300)
    ctx = [r.choice([0, r.randint(0, 1500), 16 * r.randint(0, 90)]) for _ in range(B)]
    curs = [r.choice([T, T, r.randint(0, T), 0, T + 3]) for _ in range(B)]
    io_dtype = r.choice([torch.float32, torch.bfloat16])
    print(f"split-step random seed={seed} B={B} H={H} T={T} ctx={ctx} curs={curs} io={io_dtype}", flush=True)
    b = make_prefill(device, 300 + seed, ctx, curs, T, H, 64, kv_dtype=torch.bfloat16)
    if io_dtype == torch.bfloat16:
        b = workloads._batch(b.q.to(torch.bfloat16), b.k_pool, b.v_pool, b.block_lists, b.seq_lens, b.cur_lens, device)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "split")
    err = max_err(run(b), oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= (2e-2 if io_dtype == torch.float32 else 3e-2)


def test_split_step_kernel_negative_pages_and_strided_views(device, monkeypatch):
    """-1 page-table entries past a request's blocks and strided q/out views (the layout the model
    passes) through the split-step kernel."""
    H, Hd, T = 8, 64, 48
    b = make_prefill(device, 19, [130, 20], [48, 30], T, H, Hd, kv_dtype=torch.bfloat16)
    qv = b.q.transpose(1, 2).contiguous().transpose(1, 2)  # [B, H, T, Hd] view of [B, T, H, Hd]
    pt = torch.cat([b.page_table, torch.full((2, 3), -1, dtype=torch.int32, device=device)], dim=1)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "split")
    out = paged_attention_prefill_hip(qv, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t)
    err = max_err(out, oracle_out(b))
    print(f"split-step strided max err {err:.2e}", flush=True)
    assert err <= 2e-2


def test_kv_staging_head_dim_128(device, monkeypatch):
    """bf16 KV at head_dim 128 through the 16-row kernel: LDS and register staging bit-identical and
    within tolerance of the oracle (2 requests x 16 heads, 256-token chunks over 1-2k contexts)."""
    b = workloads.large_prefill(seed=7, device=device, batch=2, heads=16, head_dim=128, chunk=256, ctx_lo=1024,
                                ctx_hi=2048, kv_dtype=torch.bfloat16)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "tile")
    print("kv staging head_dim 128", flush=True)
    outs = {}
    for staging in ("lds", "regs"):
        monkeypatch.setenv("PAGED_HIP_PREFILL_STAGING", staging)
        outs[staging] = run(b)
    assert torch.equal(outs["lds"], outs["regs"])
    err = max_err(outs["lds"], oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= 2e-2


def test_wrappers_reject_mismatched_out(device):
    b = make_prefill(device, 23, [32, 0], [20, 5], T=20, H=2, Hd=64)
    for bad in (torch.empty(2, 2, 19, 64, device=device), torch.empty(2, 2, 20, 64, device=device, dtype=torch.bfloat16),
                torch.empty(2, 2, 64, 20, device=device).transpose(2, 3), torch.empty(2, 2, 20, 64)):
        with pytest.raises(ValueError, match="out"):
            run(b, out=bad)
    d = make_prefill(device, 24, [40], [1], T=1, H=2, Hd=64)
    with pytest.raises(ValueError, match="out"):
        paged_attention_decode_hip(d.q, d.k_pool, d.v_pool, d.page_table, d.seq_lens_t, d.cur_lens_t,
                                   out=torch.empty(1, 2, 1, 32, device=device))
    ok = torch.empty_like(b.q)
    assert run(b, out=ok) is ok


@pytest.mark.parametrize("kv_dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_prefill_variants(device, kv_dtype, tol, head_dim):
    ctx = [0, 16, 100, 7, 300]
    curs = [40, 33, 1, 17, 0]  # chunk lengths; rows >= cur are padded rows
    T = 40
    b = make_prefill(device, 21, ctx, curs, T=T, H=3, Hd=head_dim, kv_dtype=kv_dtype)
    print(f"prefill variant kv={kv_dtype} hd={head_dim}", flush=True)
    err = max_err(run(b), oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= tol


def test_bf16_prefill_against_unrounded_fp32(device):
    b = make_prefill(device, 22, [200, 64], [130, 256], T=256, H=4, Hd=128)
    want = oracle_out(b)
    got = paged_attention_prefill_hip(b.q, b.k_pool.to(torch.bfloat16), b.v_pool.to(torch.bfloat16), b.page_table,
                                      b.seq_lens_t, b.cur_lens_t)
    assert max_err(got, want) <= 2e-2


@pytest.mark.parametrize("Hd,bs", [(16, 8), (64, 8), (48, 16)])
def test_prefill_generic_shapes(device, Hd, bs):
    b = make_prefill(device, 23, [0, 20, 5], [9, 4, 12], T=12, H=2, Hd=Hd, bs=bs)
    assert max_err(run(b), oracle_out(b)) <= 1e-4


def test_prefill_last_row_equals_decode(device):
    b = make_prefill(device, 24, [50, 0, 31], [20, 20, 20], T=20, H=2, Hd=64)
    pre = run(b)
    dec = paged_attention_decode_hip(b.q[:, :, -1:].contiguous(), b.k_pool, b.v_pool, b.page_table, b.seq_lens_t,
                                     torch.ones_like(b.cur_lens_t))
    assert float((pre[:, :, -1:] - dec).abs().max()) <= 1e-5


def test_prefill_strided_views_and_tiles(device):
    B, H, T, Hd = 2, 4, 70, 64
    b = make_prefill(device, 25, [16, 3], [70, 65], T=T, H=H, Hd=Hd)
    x = torch.randn(B, T, H * Hd, device=device)
    q = x.view(B, T, H, Hd).transpose(1, 2)
    out = paged_attention_prefill_hip(q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    assert out.stride() == q.stride()
    want = oracle.paged_attention(q.cpu().contiguous(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens)
    assert max_err(out, want) <= 1e-4


@pytest.mark.parametrize("kv_dtype,tol", [(torch.float32, 1e-4), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("split_blocks", [1, 3, 16])
def test_prefill_split_k(device, kv_dtype, tol, head_dim, split_blocks):
    """Split-K prefill (splits, then the merge kernel) against the oracle and the unsplit kernel,
    with tiles whose block count is below, at and above the split size, an empty request and
    padded rows; a second call must reproduce the first bit for bit (fixed merge order)."""
    ctx = [0, 16, 300, 7, 600, 0]
    curs = [40, 33, 1, 17, 0, 0]
    T = 40
    b = make_prefill(device, 26, ctx, curs, T=T, H=3, Hd=head_dim, kv_dtype=kv_dtype)
    print(f"split prefill kv={kv_dtype} hd={head_dim} split_blocks={split_blocks}", flush=True)
    got = run(b, split_blocks=split_blocks)
    err = max_err(got, oracle_out(b))
    print(f"  max err {err:.2e}", flush=True)
    assert err <= tol
    # bf16 KV rounds the softmax weights relative to the running max, which depends on the split
    assert float((got - run(b, split_blocks=0)).abs().max()) <= (1e-5 if kv_dtype == torch.float32 else 5e-3)
    assert torch.equal(got, run(b, split_blocks=split_blocks))


def test_prefill_split_then_other_shapes_share_the_workspace(device):
    """Split calls of different shapes and kinds in sequence share one workspace."""
    b1 = make_prefill(device, 27, [500, 200, 37], [64, 64, 5], T=64, H=8, Hd=64)
    b2 = make_prefill(device, 28, [900], [16], T=16, H=2, Hd=128)
    want1, want2 = oracle_out(b1), oracle_out(b2)
    for _ in range(2):
        assert max_err(run(b1, split_blocks=4), want1) <= 1e-4
        dec = paged_attention_decode_hip(b1.q[:, :, -1:].contiguous(), b1.k_pool, b1.v_pool, b1.page_table,
                                         b1.seq_lens_t, torch.ones_like(b1.cur_lens_t), split_blocks=2)
        # every request's last row attends all of its keys, as the decode row does
        assert float((dec - run(b1, split_blocks=0)[:, :, -1:]).abs().max()) <= 1e-5
        assert max_err(run(b2, split_blocks=5), want2) <= 1e-4


# ---- wide-tile bf16 kernel (128 query rows per workgroup, KV staged through LDS) -------------

@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("io_dtype,kv_dtype", [(torch.float32, torch.bfloat16), (torch.bfloat16, torch.bfloat16),
                                               (torch.float32, torch.float32), (torch.bfloat16, torch.float32)])
def test_wide_prefill_forced_small(device, monkeypatch, head_dim, io_dtype, kv_dtype):
    """The wide kernels (bf16 and fp32 KV) on ragged requests: contexts 0 / unaligned / long, chunk
    rows padded (C < T), T not a multiple of 128 nor of 32, an empty request; against the oracle
    on the same KV values and against the 16-row kernel."""
    ctx = [0, 37, 700, 16, 0, 1200]
    curs = [150, 150, 3, 90, 0, 150]
    T = 150
    b = make_prefill(device, 31, ctx, curs, T=T, H=3, Hd=head_dim, kv_dtype=kv_dtype)
    q = b.q.to(io_dtype)
    print(f"wide prefill hd={head_dim} io={io_dtype} kv={kv_dtype}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "wide")
    got = paged_attention_prefill_hip(q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "tile")
    tile = paged_attention_prefill_hip(q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    want = oracle.paged_attention(q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)
    err = max_err(got, want)
    print(f"  max err vs oracle {err:.2e}, vs 16-row kernel {float((got - tile).abs().max()):.2e}", flush=True)
    if kv_dtype == torch.float32:
        tol, tile_tol = (1e-4, 1e-5) if io_dtype == torch.float32 else (1e-2, 1e-2)  # bf16 output rounding
    else:
        tol, tile_tol = (2e-2, 5e-3) if io_dtype == torch.float32 else (3e-2, 2e-2)
    assert err <= tol
    assert float((got.float() - tile.float()).abs().max()) <= tile_tol


@pytest.mark.parametrize("B,kv_dtype", [(40, torch.bfloat16), (90, torch.bfloat16), (90, torch.float32)])
def test_wide_prefill_work_orders(device, monkeypatch, B, kv_dtype):
    """Many ragged requests: with B * tiles <= 256 (40 x 3) every workgroup ranks the (request,
    tile) units longest-first; above (90 x 3) the kernel keeps its fixed order. Every request and
    head must be computed exactly once either way: against the oracle and the 16-row kernel."""
    g = torch.Generator().manual_seed(B)
    ctx = torch.randint(0, 200, (B,), generator=g).tolist()
    curs = torch.randint(0, 301, (B,), generator=g).tolist()
    b = make_prefill(device, 33 + B, ctx, curs, T=300, H=2, Hd=64, kv_dtype=kv_dtype)
    print(f"wide prefill work order B={B} kv={kv_dtype}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "wide")
    got = run(b)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "tile")
    tile = run(b)
    want = oracle_out(b)
    tol, tile_tol = (2e-2, 5e-3) if kv_dtype == torch.bfloat16 else (1e-4, 1e-5)
    assert max_err(got, want) <= tol
    assert float((got - tile).abs().max()) <= tile_tol


@pytest.mark.parametrize("head_dim", [64, 128])
def test_wide_prefill_long_page_tables(device, monkeypatch, head_dim):
    """Contexts of 2-5k tokens (130-330 blocks: the wide kernel reads its page-table entries 64 at
    a time, so every request crosses several of those windows), with -1 entries in different
    windows: against the 16-row kernel everywhere and the oracle on one request."""
    ctx = [5000, 2100, 4000]
    curs = [150, 40, 130]
    b = make_prefill(device, 34 + head_dim, ctx, curs, T=150, H=2, Hd=head_dim, kv_dtype=torch.bfloat16)
    pt = b.page_table.clone()
    for r, cols in ((0, (3, 70, 200, 311)), (2, (64, 65, 190))):
        pt[r, list(cols)] = -1
    print(f"wide prefill long page tables hd={head_dim}", flush=True)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "wide")
    got = paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "tile")
    tile = paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t)
    assert float((got - tile).abs().max()) <= 5e-3
    want = oracle.paged_attention(b.q[1:2].cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists[1:2],
                                  b.seq_lens[1:2], b.cur_lens[1:2], nthreads=NTHREADS)
    assert max_err(got[1:2], want) <= 2e-2


def test_wide_prefill_negative_pages_and_strided_views(device, monkeypatch):
    """A -1 page entry skips its 16 keys in the wide kernel as in the 16-row kernel; q/out are
    the model's transposed views; the untouched request matches the oracle."""
    B, H, T, Hd = 2, 4, 96, 128
    b = make_prefill(device, 32, [300, 40], [96, 96], T=T, H=H, Hd=Hd, kv_dtype=torch.bfloat16)
    pt = b.page_table.clone()
    pt[0, 3] = -1
    x = torch.randn(B, T, H * Hd, device=device)
    q = x.view(B, T, H, Hd).transpose(1, 2)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "wide")
    got = paged_attention_prefill_hip(q, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t)
    assert got.stride() == q.stride()
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", "tile")
    tile = paged_attention_prefill_hip(q, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t)
    full = paged_attention_prefill_hip(q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    assert float((got - tile).abs().max()) <= 5e-3
    assert float((got[0] - full[0]).abs().max()) > 1e-2  # the skipped keys did matter
    want = oracle.paged_attention(q[1:].cpu().contiguous(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists[1:],
                                  b.seq_lens[1:], b.cur_lens[1:], nthreads=NTHREADS)
    assert max_err(got[1:], want) <= 2e-2


def _check_large_request(b, out, r, tol):
    """Every head of request r of a large-prefill batch against the oracle."""
    ids = torch.tensor(b.block_lists[r], device=b.q.device, dtype=torch.long)
    k = b.k_pool.index_select(0, ids).cpu()
    v = b.v_pool.index_select(0, ids).cpu()
    want = oracle.paged_attention(b.q[r:r + 1].cpu(), k, v, [list(range(len(b.block_lists[r])))],
                                  [b.seq_lens[r]], [b.cur_lens[r]], nthreads=NTHREADS)
    err = max_err(out[r:r + 1], want)
    print(f"  request {r} (L={b.seq_lens[r]}, all {b.q.shape[1]} heads): max err {err:.2e}", flush=True)
    assert err <= tol


def test_large_prefill_fp32_parity(device):
    """The large-prefill workload with fp32 KV (the wide fp32 kernel at this size): one request,
    all 32 heads x 512 rows, against the oracle within 1e-4."""
    b = workloads.large_prefill(seed=1, device=device, kv_dtype=torch.float32)
    out = paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    print(f"large fp32 prefill ctx={b.extra['prev_lens']}", flush=True)
    _check_large_request(b, out, 3, 1e-4)


def test_large_prefill_parity(device):
    """The MFMA-utilisation workload at full size (8 requests x 32 heads x 128, chunk 512 over
    1-4k contexts, bf16 KV) through the default dispatch (the wide kernel at this size); two
    requests, every head, against the oracle on the same bf16 values."""
    from src.kernels.hip_paged_attention import cu_count
    b = workloads.large_prefill(seed=0, device=device)
    print(f"large prefill ctx={b.extra['prev_lens']}", flush=True)
    out = paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    assert 8 * 32 * 4 >= 2 * cu_count(device)  # the wide kernel's grid rule holds at this size
    for r in (0, 5):
        _check_large_request(b, out, r, 2e-2)


@pytest.mark.parametrize("ctx,kernel", [(2048, "split"), (256, "tile")])
def test_split_step_kernel_two_rounds_by_context(device, monkeypatch, ctx, kernel):
    """4 requests x 8 heads x 64, 512-token chunks, bf16 KV: 512 split-step units (two per CU on
    MI355X). The default dispatch takes the split-step kernel for two rounds once the widest
    request spans 96 pages (a 2k context), the 16-row kernel below that: its output equals the
    forced kernel's bit for bit, and two requests match the oracle."""
    from src.kernels.hip_paged_attention import cu_count
    b = workloads.large_prefill(seed=7, device=device, batch=4, heads=8, head_dim=64, chunk=512,
                                ctx_lo=ctx, ctx_hi=ctx)
    units, cus = 4 * 8 * (512 // 32), cu_count(device)
    if not cus < units <= 2 * cus:
        pytest.skip(f"{units} units is not one to two rounds on {cus} CUs")
    print(f"split-step two rounds ctx={ctx} pages={b.page_table.shape[1]} expect {kernel}", flush=True)
    out = run(b)
    monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", kernel)
    assert torch.equal(out, run(b))
    for r in (0, 3):
        _check_large_request(b, out, r, 2e-2)
