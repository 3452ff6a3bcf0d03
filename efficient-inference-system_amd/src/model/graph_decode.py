"""HIP-graph replay of one decode step of TinyTransformerLM on the "hip_paged" backend.

A decode step of the small model is ~100 kernel launches of a few microseconds each, so in eager
mode the host (Python and the framework's dispatch) is the bottleneck. This runner captures the
whole step once per batch size and replays it:

  outside the graph (host):  the cache bookkeeping of every layer (block allocation in the
                             reference's LIFO order, seq_len += 1), one upload of the batch's block
                             lists in CSR form into a static device buffer, and copies of the token
                             ids and positions into static buffers;
  inside the graph (device): metadata packing (page table, lengths, slots), then per layer
                             LayerNorm, q/k/v projections, KV scatter into the pool, paged decode
                             attention, output projection, MLP and residuals; final LayerNorm and
                             lm_head.

It is used only when every layer's cache holds the same block lists and every pool the same free
list, which the model guarantees (all layers allocate in lockstep), so one metadata pack serves
all layers exactly as in eager mode. A graph holds the pool tensors' addresses, so it is captured
again when a pool is reallocated (growth or reset). The page table is packed at a fixed width of
ceil(max_seq_len / block_size) pages; unused entries are -1.
Set PAGED_HIP_GRAPHS=0 to run the eager forward instead.
"""
from __future__ import annotations

import math
import os

import torch

from src.cache.paged_kv import BatchedPagedKVCache
from src.kernels.hip_paged_attention import (
    _workspace, default_split_blocks, kv_append_hip, pack_metadata_hip, paged_attention_decode_hip)
from src.kernels import _lib
from src.kernels.staging import upload


def graphs_enabled() -> bool:
    return os.environ.get("PAGED_HIP_GRAPHS", "1") != "0"


class _Captured:
    def __init__(self, model, B: int, pages: int, device: torch.device, pools):
        H, Hd = model.num_heads, model.head_dim
        self.B = B
        self.pages = pages
        self.ids = torch.zeros((B, 1), dtype=torch.long, device=device)
        self.pos = torch.zeros((B,), dtype=torch.long, device=device)
        self.csr = torch.zeros((3 * B + 1 + B * pages,), dtype=torch.int32, device=device)
        self.cur = torch.ones((B,), dtype=torch.int32, device=device)
        self.split_blocks = default_split_blocks(B, H, pages, device)
        ws_bytes = _lib.load().pa_decode_workspace_size(B, H, Hd, pages, self.split_blocks)
        # Allocated outside the capture and referenced here, so the address the graph records
        # stays valid for the graph's lifetime.
        self.ws = _workspace(device, ws_bytes) if ws_bytes else None
        self.signature = _pool_signature(pools)
        self.graph = None
        self.logits = None


def _pool_signature(pools) -> tuple:
    return tuple((p.k_blocks.data_ptr(), p.v_blocks.data_ptr(), p.k_blocks.shape[0], p.k_blocks.dtype) for p in pools)


def _lockstep(kv_caches: list[BatchedPagedKVCache]) -> bool:
    """True when all layers hold identical states and pools (so allocations stay identical)."""
    first = kv_caches[0]
    p0 = first.pool
    if p0.k_blocks is None:
        return False
    for cache in kv_caches[1:]:
        p = cache.pool
        if p.k_blocks is None or p.capacity_blocks != p0.capacity_blocks or p.free_block_ids != p0.free_block_ids:
            return False
        if len(cache.states) != len(first.states):
            return False
        for a, b in zip(cache.states, first.states):
            if a.seq_len != b.seq_len or a.block_ids != b.block_ids:
                return False
    return True


class GraphedDecodeStep:
    def __init__(self, model):
        self.model = model
        self.captured: dict[int, _Captured] = {}

    def usable(self, input_ids: torch.Tensor, kv_caches) -> bool:
        m = self.model
        return (
            graphs_enabled()
            and input_ids.is_cuda
            and input_ids.dim() == 2 and input_ids.shape[1] == 1
            and not m.training
            and m.attention_backend == "hip_paged"
            and all(b.attn.attention_backend == "hip_paged" for b in m.blocks)
            and isinstance(kv_caches, list) and len(kv_caches) == len(m.blocks)
            and all(isinstance(c, BatchedPagedKVCache) for c in kv_caches)
            and _lockstep(kv_caches)
        )

    # ------------------------------------------------------------------------------------------
    def _static_forward(self, cap: _Captured, pools) -> torch.Tensor:
        m = self.model
        B = cap.B
        bs = m.kv_block_size
        csr = cap.csr
        pt, seq32, _, slots = pack_metadata_hip(
            csr[3 * B + 1:], csr[0:B + 1], csr[B + 1:2 * B + 1], csr[2 * B + 1:3 * B + 1],
            query_len=1, block_size=bs, max_pages=cap.pages, with_slots=True,
        )
        x = m.token_emb(cap.ids) + m.pos_emb(cap.pos.view(B, 1))
        for blk, pool in zip(m.blocks, pools):
            a = blk.attn
            h = blk.ln1(x)
            q = a._split_heads(a.q_proj(h))
            k_new = a._split_heads(a.k_proj(h))
            v_new = a._split_heads(a.v_proj(h))
            kv_append_hip(k_new, v_new, pool.k_blocks, pool.v_blocks, slots)
            o = paged_attention_decode_hip(q, pool.k_blocks, pool.v_blocks, pt, seq32, cap.cur,
                                           split_blocks=cap.split_blocks)
            x = x + a.out_proj(a._merge_heads(o))
            x = x + blk.mlp(blk.ln2(x))
        return m.lm_head(m.ln_f(x))

    def _capture(self, cap: _Captured, pools) -> None:
        # Warm-up on a side stream (initialises library handles); it performs the same step the
        # replay will (same inputs, same slots), so the cache contents are unaffected.
        side = torch.cuda.Stream(device=cap.ids.device)
        side.wait_stream(torch.cuda.current_stream(cap.ids.device))
        with torch.cuda.stream(side):
            self._static_forward(cap, pools)
        torch.cuda.current_stream(cap.ids.device).wait_stream(side)
        # Each graph keeps its own private memory pool (a step's intermediates are small), so
        # dropping graphs after a pool reallocation never leaves a shared pool half-released.
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cap.logits = self._static_forward(cap, pools)
        cap.graph = g

    # ------------------------------------------------------------------------------------------
    def __call__(self, input_ids: torch.Tensor, positions: torch.Tensor, kv_caches: list[BatchedPagedKVCache]):
        m = self.model
        B = input_ids.shape[0]
        device = input_ids.device
        pools = [c.pool for c in kv_caches]
        app = [1] * B
        prev = None
        for cache in kv_caches:
            p = cache.host_append(app, 1, m.num_heads, m.head_dim, pools[0].dtype, device)
            prev = p if prev is None else prev
        buf, max_pages = kv_caches[0].csr_buffer(prev, app)
        pages = max(math.ceil(m.max_seq_len / m.kv_block_size), max_pages)
        sig = _pool_signature(pools)
        cap = self.captured.get(B)
        if cap is None or cap.signature != sig or cap.pages < max_pages:
            if cap is not None and cap.signature != sig:
                self.captured.clear()  # every graph holds the old pool addresses
            cap = _Captured(m, B, pages, device, pools)
            self.captured[B] = cap
        staged = upload(buf, device)
        cap.csr[: buf.size].copy_(staged)
        cap.ids.copy_(input_ids)
        cap.pos.copy_(positions.view(B))
        if cap.graph is None:
            self._capture(cap, pools)
        cap.graph.replay()
        return cap.logits.clone()
