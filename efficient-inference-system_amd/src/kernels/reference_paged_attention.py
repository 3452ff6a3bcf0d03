"""The "paged_reference" backend: torch paged attention with the reference's semantics.

Behaviour of src/kernels/reference_paged_attention.py:10-59 of the reference: for request b,
head h and query row i, with L = state.seq_len and C = current_lengths[b], the row attends key
positions t < L with t <= (L - C) + i, read from pool blocks state.block_ids[t // block_size] at
offset t % block_size; the output is softmax(q.k / sqrt(head_dim)) weighted V, and a row with no
key stays zero. The reference loops over (request, head, row, key) in Python; here each request's
keys are gathered once and the rows are computed with batched matmuls, on whatever device the
tensors live. It is a selectable backend of the product (as in the reference), and is not used by
the "hip_paged" path.
"""
from __future__ import annotations

import math

import torch

from src.cache.paged_kv import BatchedPagedKVCache


def _current_lengths_list(current_lengths, batch_size: int, query_len: int) -> list[int]:
    if current_lengths is None:
        return [query_len] * batch_size
    if isinstance(current_lengths, int):
        return [current_lengths] * batch_size
    return [int(x) for x in current_lengths.reshape(-1).tolist()]


def paged_attention_reference(
    q: torch.Tensor,
    kv_cache: BatchedPagedKVCache,
    current_lengths: int | torch.Tensor | None,
) -> torch.Tensor:
    batch_size, num_heads, query_len, head_dim = q.shape
    out = torch.zeros_like(q)
    cur = _current_lengths_list(current_lengths, batch_size, query_len)
    scale = 1.0 / math.sqrt(head_dim)
    pool = kv_cache.pool
    for batch_idx, state in enumerate(kv_cache.states):
        seq_len = state.seq_len
        if seq_len <= 0:
            continue
        past_len = seq_len - cur[batch_idx]
        bs = state.pool.block_size
        nblocks = (seq_len + bs - 1) // bs
        ids = torch.tensor(state.block_ids[:nblocks], dtype=torch.long, device=state.pool.k_blocks.device)
        if ids.numel() < nblocks:
            raise IndexError(f"request {batch_idx}: {ids.numel()} blocks cannot hold {seq_len} tokens")
        # [nblocks, H, bs, Hd] -> [H, nblocks*bs, Hd] -> first seq_len keys
        k = state.pool.k_blocks.index_select(0, ids).permute(1, 0, 2, 3).reshape(num_heads, nblocks * bs, head_dim)
        v = state.pool.v_blocks.index_select(0, ids).permute(1, 0, 2, 3).reshape(num_heads, nblocks * bs, head_dim)
        k = k[:, :seq_len].to(q.dtype).contiguous()
        v = v[:, :seq_len].to(q.dtype).contiguous()
        qb = q[batch_idx].contiguous()  # [H, T, Hd]
        scores = torch.matmul(qb, k.transpose(1, 2).contiguous()) * scale  # [H, T, L]
        rows = torch.arange(query_len, device=q.device).view(query_len, 1)
        keys = torch.arange(seq_len, device=q.device).view(1, seq_len)
        allowed = keys <= (past_len + rows)  # [T, L]
        scores = scores.masked_fill(~allowed.view(1, query_len, seq_len), float("-inf"))
        weights = torch.softmax(scores, dim=-1)
        has_key = allowed.any(dim=1).view(1, query_len, 1)
        weights = torch.where(has_key, weights, torch.zeros_like(weights))
        out[batch_idx] = torch.matmul(weights, v)
    del pool
    return out
