"""Seeded random sweep of the HIP attention entry points against the oracle.

Each case draws batch size, heads, head_dim (the MFMA/fast shapes 64 and 128 with block 16, or a
generic shape), block size, cached lengths (with the block-edge and empty cases mixed in),
current_lengths (including 0 and values past the query length or the cached length), KV and
q/out dtypes, the split size and, for prefill, the kernel choice (16-row or wide tiles). The case
is printed before it runs, so a failure names its seed and shape.

Tolerances: fp32 arithmetic against the fp64 oracle on the same (possibly bf16-rounded) pool
values 1e-4; the bf16 MFMA prefill (q and softmax weights rounded to bf16) 2e-2; bf16 outputs
1e-2 more (|out| <= ~4, bf16 ulp 2^-6).
"""
import math
import os
import random

import numpy as np
import pytest
import torch

import oracle
from src import workloads
from src.kernels.hip_paged_attention import paged_attention_decode_hip, paged_attention_prefill_hip

pytestmark = pytest.mark.gpu
NTHREADS = min(16, os.cpu_count() or 1)


def _lengths(r: random.Random, B: int, bs: int, hi: int) -> list[int]:
    special = [0, 1, bs - 1, bs, bs + 1, 2 * bs]
    return [r.choice(special) if r.random() < 0.3 else r.randint(0, hi) for _ in range(B)]


def _shape(r: random.Random):
    if r.random() < 0.7:
        return r.choice([64, 128]), 16, True
    return r.choice([16, 32, 48, 80, 96, 160]), r.choice([4, 8, 16, 32]), False


def _build(device, seed, lens, curs, T, H, Hd, bs, kv_dtype, io_dtype):
    g = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(L / bs) for L in lens)
    N = need + 5
    perm = torch.randperm(N, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / bs)
        lists.append(perm[pos:pos + n])
        pos += n
    B = len(lens)
    q = torch.randn(B, H, T, Hd, generator=g).to(io_dtype).to(device)
    k = torch.randn(N, H, bs, Hd, generator=g).to(kv_dtype).to(device)
    v = torch.randn(N, H, bs, Hd, generator=g).to(kv_dtype).to(device)
    return workloads._batch(q, k, v, lists, list(lens), list(curs), device)


def _oracle(b):
    return oracle.paged_attention(b.q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)


def _err(got, want):
    return float(np.abs(got.float().cpu().numpy() - want).max()) if want.size else 0.0


@pytest.mark.parametrize("seed", range(40))
def test_decode_random_cases(device, seed):
    r = random.Random(1000 + seed)
    Hd, bs, fast = _shape(r)
    B, H = r.randint(1, 9), r.randint(1, 6)
    lens = _lengths(r, B, bs, 700)
    curs = [r.choice([1, 1, 1, 0, 2, 5]) for _ in range(B)]
    kv_dtype = r.choice([torch.float32, torch.bfloat16])
    io_dtype = r.choice([torch.float32, torch.bfloat16])
    split = r.choice([0, 0, 1, 2, 5, 16]) if fast else 0
    print(f"decode seed={seed} B={B} H={H} Hd={Hd} bs={bs} kv={kv_dtype} io={io_dtype} split={split} "
          f"lens={lens} curs={curs}", flush=True)
    b = _build(device, seed, lens, curs, 1, H, Hd, bs, kv_dtype, io_dtype)
    got = paged_attention_decode_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t,
                                     split_blocks=split)
    assert got.dtype == io_dtype and got.shape == b.q.shape
    tol = 1e-4 + (1e-2 if io_dtype == torch.bfloat16 else 0.0)
    assert _err(got, _oracle(b)) <= tol


@pytest.mark.parametrize("seed", range(40))
def test_prefill_random_cases(device, monkeypatch, seed):
    r = random.Random(2000 + seed)
    Hd, bs, fast = _shape(r)
    B, H = r.randint(1, 6), r.randint(1, 5)
    T = r.randint(2, 48)
    ctx = _lengths(r, B, bs, 300)
    curs = [r.choice([T, T, r.randint(0, T), 0, T + 3]) for _ in range(B)]
    lens = [c0 + min(c, T) for c0, c in zip(ctx, curs)]  # the cache after appending the chunk
    kv_dtype = r.choice([torch.float32, torch.bfloat16])
    io_dtype = r.choice([torch.float32, torch.bfloat16])
    kernel = r.choice(["", "tile", "wide", "split"]) if fast else ""
    split = r.choice([0, 0, 1, 3]) if fast and kernel != "wide" else 0
    staging = r.choice(["", "lds", "regs"])  # the 16-row kernel's KV staging at head_dim 64
    if kernel:
        monkeypatch.setenv("PAGED_HIP_PREFILL_KERNEL", kernel)
    if staging:
        monkeypatch.setenv("PAGED_HIP_PREFILL_STAGING", staging)
    print(f"prefill seed={seed} B={B} H={H} T={T} Hd={Hd} bs={bs} kv={kv_dtype} io={io_dtype} "
          f"kernel={kernel or 'auto'} staging={staging or 'auto'} split={split} ctx={ctx} curs={curs}", flush=True)
    b = _build(device, seed, lens, curs, T, H, Hd, bs, kv_dtype, io_dtype)
    got = paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t,
                                      split_blocks=split)
    assert got.dtype == io_dtype and got.shape == b.q.shape
    tol = 2e-2 if (fast and kv_dtype == torch.bfloat16) else 1e-4
    if io_dtype == torch.bfloat16:
        tol += 1e-2
    assert _err(got, _oracle(b)) <= tol
