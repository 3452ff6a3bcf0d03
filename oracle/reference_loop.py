"""ORACLE — test infrastructure only.

The reference's CPU paged attention as written: a Python loop over (request, head, query row,
key) with torch.dot / torch.softmax per row (src/kernels/reference_paged_attention.py:10-59).
Inputs are plain tensors and per-request block lists instead of cache objects. It is slow
(microseconds per key); use it only on tiny shapes and to time the reference's own CPU path.
"""
from __future__ import annotations

import math

import torch


def paged_attention_loop(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                         block_lists: list[list[int]], seq_lens: list[int], cur_lens: list[int]) -> torch.Tensor:
    batch_size, num_heads, query_len, head_dim = q.shape
    block_size = k_pool.shape[2]
    out = torch.zeros_like(q)
    scale = 1.0 / math.sqrt(head_dim)
    for b in range(batch_size):
        seq_len = seq_lens[b]
        past_len = seq_len - cur_lens[b]
        for h in range(num_heads):
            for i in range(query_len):
                query_abs_pos = past_len + i
                scores, values = [], []
                for t in range(seq_len):
                    if t > query_abs_pos:
                        break
                    blk = block_lists[b][t // block_size]
                    off = t % block_size
                    k_vec = k_pool[blk, h, off, :].to(q.dtype)
                    v_vec = v_pool[blk, h, off, :].to(q.dtype)
                    scores.append(torch.dot(q[b, h, i], k_vec) * scale)
                    values.append(v_vec)
                if not scores:
                    continue
                weights = torch.softmax(torch.stack(scores), dim=0)
                out[b, h, i] = torch.sum(weights.unsqueeze(-1) * torch.stack(values, dim=0), dim=0)
    return out
