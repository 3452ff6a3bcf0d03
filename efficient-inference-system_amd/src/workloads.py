"""Seeded synthetic inputs for the paged-attention benchmark workloads.

  single_decode   1 request, 8 heads x 64, 128 cached tokens in 16-token blocks: 8 blocks drawn
                  by a seeded permutation from a 64-block pool; fp32.
  ragged_decode   8 requests, 8 heads x 64, context lengths uniform in [128, 1024], 4096-block
                  pool, disjoint seeded block sets; fp32; one instance per model layer (6).
  chunked_prefill 4 requests, 8 heads x 64, cached context uniform in [0, 768] aligned to 16
                  plus a new chunk of 128 or 256 tokens; shuffled 4096-block pool; fp32.
  large_decode    256 requests, 32 heads x 128, lengths log-uniform in [512, 32768] (request b
                  drawn from seed + b), pool = ceil(1.1 * blocks needed), shuffled block lists;
                  bf16 KV (N(0,1) drawn in fp32, rounded to nearest even), fp32 q.
  large_prefill   8 requests, 32 heads x 128, cached context uniform in [1024, 4096] aligned to 16
                  plus a new 512-token chunk already in the cache; pool = ceil(1.1 * blocks
                  needed), shuffled block lists; bf16 KV, fp32 q (the MFMA-utilisation workload).
Q, K and V are i.i.d. N(0, 1). Block lists are drawn on the host with torch.Generator; pool
contents are drawn on the target device. Each workload also carries its algorithmic HBM bytes:
K and V rows read, q read and output written (fp32), page-table entries and two int32 lengths.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

BLOCK = 16


@dataclass
class PagedBatch:
    q: torch.Tensor                      # [B, H, T, Hd]
    k_pool: torch.Tensor                 # [N, H, 16, Hd]
    v_pool: torch.Tensor
    block_lists: list[list[int]]
    seq_lens: list[int]                  # cached length after the append (the attention's L)
    cur_lens: list[int]                  # current_lengths (1 for decode)
    page_table: torch.Tensor             # int32 [B, max_pages], -1 padded, on the pool's device
    seq_lens_t: torch.Tensor             # int32 [B]
    cur_lens_t: torch.Tensor             # int32 [B]
    extra: dict = field(default_factory=dict)

    @property
    def batch(self) -> int:
        return self.q.shape[0]

    def decode_bytes(self) -> int:
        """Algorithmic HBM bytes of one decode call over this batch."""
        _, H, _, Hd = self.q.shape
        s_kv = self.k_pool.element_size()
        total = 0
        for L in self.seq_lens:
            total += H * (2 * L * Hd * s_kv + 2 * Hd * 4) + 4 * math.ceil(L / BLOCK) + 8
        return total


def _page_table(block_lists: list[list[int]], device) -> torch.Tensor:
    max_pages = max((len(x) for x in block_lists), default=0)
    pt = torch.full((len(block_lists), max_pages), -1, dtype=torch.int32)
    for i, row in enumerate(block_lists):
        if row:
            pt[i, : len(row)] = torch.tensor(row, dtype=torch.int32)
    return pt.to(device)


def _fill_normal(t: torch.Tensor, gen: torch.Generator, chunk_elems: int = 1 << 28) -> None:
    """Fill t with N(0,1) drawn in fp32 and rounded to t's dtype, chunk by chunk."""
    flat = t.view(-1)
    for s in range(0, flat.numel(), chunk_elems):
        e = min(s + chunk_elems, flat.numel())
        flat[s:e] = torch.randn(e - s, generator=gen, device=t.device, dtype=torch.float32).to(t.dtype)


def _device_gen(device, seed: int) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def _batch(q, k_pool, v_pool, block_lists, seq_lens, cur_lens, device) -> PagedBatch:
    return PagedBatch(
        q=q, k_pool=k_pool, v_pool=v_pool, block_lists=block_lists, seq_lens=seq_lens, cur_lens=cur_lens,
        page_table=_page_table(block_lists, device),
        seq_lens_t=torch.tensor(seq_lens, dtype=torch.int32, device=device),
        cur_lens_t=torch.tensor(cur_lens, dtype=torch.int32, device=device),
    )


def single_decode(seed: int = 0, device="cpu") -> PagedBatch:
    g = torch.Generator().manual_seed(seed)
    H, Hd, L, pool_blocks = 8, 64, 128, 64
    block_ids = torch.randperm(pool_blocks, generator=g)[: L // BLOCK].tolist()
    dg = _device_gen(device, seed + 1)
    q = torch.empty(1, H, 1, Hd, device=device)
    k = torch.empty(pool_blocks, H, BLOCK, Hd, device=device)
    v = torch.empty_like(k)
    for t in (q, k, v):
        _fill_normal(t, dg)
    return _batch(q, k, v, [block_ids], [L], [1], device)


def ragged_decode(seed: int = 0, layer: int = 0, device="cpu", batch: int = 8, heads: int = 8, head_dim: int = 64,
                  pool_blocks: int = 4096, min_len: int = 128, max_len: int = 1024,
                  kv_dtype: torch.dtype = torch.float32) -> PagedBatch:
    g = torch.Generator().manual_seed(seed * 1000 + layer)
    lens = torch.randint(min_len, max_len + 1, (batch,), generator=g).tolist()
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / BLOCK)
        lists.append(perm[pos:pos + n])
        pos += n
    if pos > pool_blocks:
        raise ValueError("pool too small for the drawn lengths")
    dg = _device_gen(device, seed * 1000 + layer + 7)
    q = torch.empty(batch, heads, 1, head_dim, device=device)
    k = torch.empty(pool_blocks, heads, BLOCK, head_dim, device=device, dtype=kv_dtype)
    v = torch.empty_like(k)
    for t in (q, k, v):
        _fill_normal(t, dg)
    return _batch(q, k, v, lists, lens, [1] * batch, device)


def large_decode_lengths(seed: int = 0, batch: int = 256, lo: int = 512, hi: int = 32768) -> list[int]:
    lens = []
    for b in range(batch):
        g = torch.Generator().manual_seed(seed + b)
        u = torch.rand(1, generator=g, dtype=torch.float64).item()
        lens.append(int(round(math.exp(math.log(lo) + u * (math.log(hi) - math.log(lo))))))
    return lens


def large_decode(seed: int = 0, device="cpu", batch: int = 256, heads: int = 32, head_dim: int = 128,
                 lo: int = 512, hi: int = 32768, kv_dtype: torch.dtype = torch.bfloat16,
                 rows: list[int] | None = None) -> PagedBatch:
    """The large ragged decode batch. With `rows`, only those requests of the batch (their
    lengths, in that order) over a pool sized and shuffled for them alone; the pool and q values
    are then drawn afresh, not taken from the full batch."""
    lens = large_decode_lengths(seed, batch, lo, hi)
    if rows is not None:
        lens = [lens[r] for r in rows]
        batch = len(lens)
    need = sum(math.ceil(L / BLOCK) for L in lens)
    pool_blocks = math.ceil(1.1 * need)
    g = torch.Generator().manual_seed(seed + 100003)
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / BLOCK)
        lists.append(perm[pos:pos + n])
        pos += n
    dg = _device_gen(device, seed + 200003)
    q = torch.empty(batch, heads, 1, head_dim, device=device)
    k = torch.empty(pool_blocks, heads, BLOCK, head_dim, device=device, dtype=kv_dtype)
    v = torch.empty_like(k)
    for t in (q, k, v):
        _fill_normal(t, dg)
    return _batch(q, k, v, lists, lens, [1] * batch, device)


def chunked_prefill(seed: int = 0, device="cpu", batch: int = 4, heads: int = 8, head_dim: int = 64,
                    pool_blocks: int = 4096, kv_dtype: torch.dtype = torch.float32) -> dict:
    """Cached context + new chunk per request. Returns a dict with the pre-append batch
    (block_lists already holding the chunk's blocks), prev lengths, chunk lengths, the new
    chunk's K/V [B, H, maxC, Hd] and q [B, H, maxC, Hd]."""
    g = torch.Generator().manual_seed(seed)
    ctx = [16 * int(x) for x in torch.randint(0, 49, (batch,), generator=g).tolist()]
    chunk = [128 if int(x) == 0 else 256 for x in torch.randint(0, 2, (batch,), generator=g).tolist()]
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    lists, pos = [], 0
    for c0, c in zip(ctx, chunk):
        n = math.ceil((c0 + c) / BLOCK)
        lists.append(perm[pos:pos + n])
        pos += n
    T = max(chunk)
    dg = _device_gen(device, seed + 11)
    q = torch.empty(batch, heads, T, head_dim, device=device)
    k_new = torch.empty(batch, heads, T, head_dim, device=device)
    v_new = torch.empty_like(k_new)
    k = torch.empty(pool_blocks, heads, BLOCK, head_dim, device=device, dtype=kv_dtype)
    v = torch.empty_like(k)
    for t in (q, k_new, v_new, k, v):
        _fill_normal(t, dg)
    return {
        "q": q, "k_new": k_new, "v_new": v_new, "k_pool": k, "v_pool": v, "block_lists": lists,
        "prev_lens": ctx, "chunk_lens": chunk, "seq_lens": [c0 + c for c0, c in zip(ctx, chunk)],
    }


def prefill_flops(prev_lens: list[int], chunk_lens: list[int], heads: int, head_dim: int) -> int:
    """Useful FLOPs of causal chunked prefill (QK^T and PV over attended keys of real rows)."""
    return sum(4 * heads * head_dim * (c * c0 + c * (c + 1) // 2) for c0, c in zip(prev_lens, chunk_lens))


def prefill_flops_with_padding(prev_lens: list[int], chunk_lens: list[int], query_len: int, heads: int,
                               head_dim: int) -> int:
    """FLOPs over every row of a [B, H, query_len] batch, the padded rows past a shorter chunk
    included: padded row i of request b attends to all of its seq_len keys, as in the reference
    (src/kernels/reference_paged_attention.py:33-42), so a kernel computes them too."""
    total = 0
    for c0, c in zip(prev_lens, chunk_lens):
        L = c0 + c
        total += c * c0 + c * (c + 1) // 2 + (query_len - c) * L
    return 4 * heads * head_dim * total


def large_prefill(seed: int = 0, device="cpu", batch: int = 8, heads: int = 32, head_dim: int = 128,
                  chunk: int = 512, ctx_lo: int = 1024, ctx_hi: int = 4096,
                  kv_dtype: torch.dtype = torch.bfloat16) -> PagedBatch:
    """Chunked prefill after the chunk's append: seq_lens = context + chunk, cur_lens = chunk."""
    g = torch.Generator().manual_seed(seed + 300007)
    ctx = [BLOCK * int(x) for x in torch.randint(ctx_lo // BLOCK, ctx_hi // BLOCK + 1, (batch,), generator=g).tolist()]
    lens = [c0 + chunk for c0 in ctx]
    need = sum(math.ceil(L / BLOCK) for L in lens)
    pool_blocks = math.ceil(1.1 * need)
    perm = torch.randperm(pool_blocks, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / BLOCK)
        lists.append(perm[pos:pos + n])
        pos += n
    dg = _device_gen(device, seed + 400009)
    q = torch.empty(batch, heads, chunk, head_dim, device=device)
    k = torch.empty(pool_blocks, heads, BLOCK, head_dim, device=device, dtype=kv_dtype)
    v = torch.empty_like(k)
    for t in (q, k, v):
        _fill_normal(t, dg)
    b = _batch(q, k, v, lists, lens, [chunk] * batch, device)
    b.extra["prev_lens"] = ctx
    return b
