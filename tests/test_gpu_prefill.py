"""HIP chunked-PREFILL attention vs the oracle (fp32 KV within 1e-4, bf16 KV within 2e-2),
including the reference's padded-row semantics and the append-then-attend order."""
import math
import os

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


def run(b):
    return paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)


def oracle_out(b):
    return oracle.paged_attention(b.q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)


def test_chunked_prefill_config(device):
    w = workloads.chunked_prefill(seed=0, device=device)
    B = len(w["prev_lens"])
    print(f"chunked prefill ctx={w['prev_lens']} chunk={w['chunk_lens']}", flush=True)
    pool = LayerBlockPool(block_size=16, initial_blocks=w["k_pool"].shape[0], growth_factor=2.0)
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
    assert err <= 1e-4


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
