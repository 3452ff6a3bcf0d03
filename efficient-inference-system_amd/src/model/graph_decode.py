"""HIP-graph replay of TinyTransformerLM cached steps on the "hip_paged" backend.

A cached step of the small model is ~100 kernel launches of a few microseconds each, so in eager
mode the host (Python and the framework's dispatch) is the bottleneck. This runner captures a
whole step once per (batch size, query-length bucket) and replays it:

  outside the graph (host):  the cache bookkeeping of every layer (block allocation in the
                             reference's LIFO order, seq_len advance), then the step descriptor:
                             token ids, first positions, current lengths, greedy rows and, per
                             request, only the part of its block list that its row of the device
                             block-table mirror does not hold yet (normally the blocks this step
                             opened). The descriptor is pinned host memory the device reads
                             directly, so a step issues no copy call;
  inside the graph (device): one launch reads the descriptor, updates the mirror rows and builds
                             the page table, lengths and the slot of every new token, staging the
                             ids, positions and lengths into device buffers; then per layer
                             LayerNorm, q/k/v projections, KV scatter into the pool, paged
                             attention (decode kernel for one-token steps, chunked-prefill kernel
                             otherwise), output projection, MLP and residuals; final LayerNorm and
                             lm_head; and the greedy argmax of each request's selected row.

The mirror (int32 [rows, width] on the device) keeps every live request's block list between
steps; the host keeps a shadow copy and, each step, sends a request's list from the first entry
that differs from the shadow (the whole list for a request new to its row), so host-to-device
traffic is O(blocks opened) per step and a block list edited by hand is still sent correctly.
Requests own rows by the identity of their first layer's cache state; a row returns to the free
list when that state is garbage collected, and the least recently used row is taken over when
none is free.

Steps of at most FUSED_STEP_ROWS rows (B * bucketed T: every decode step, and prefill chunks up
to 1024 rows) run the layers through the fused kernels (src/kernels/hip_linear.py) when the model's
shapes allow: per layer one launch for LayerNorm + q/k/v projections + KV append, the attention
(decode or chunked prefill kernel), one for the output projection + residual, one for LayerNorm +
fc1 + GELU, one for fc2 + residual; then LayerNorm + lm_head. Steps of at most 16 rows of an fp32
model (every decode step at batch <= 16) fold the last two into one launch: the output projection
writes x1 into the MLP's input buffer and over the residual stream, and each fc1 column tile of
the MLP launch adds its share of fc2 to the residual stream with atomic adds (four launches per
layer; PAGED_HIP_DECODE_FOLD=0 keeps five). A fused launch reads its weight tile
once per 16 rows, so above a per-layer row count (FUSED_ROWS) that layer runs through torch
instead. Set PAGED_HIP_FUSED_DECODE=0 to use the torch layers throughout.

Query lengths T > 1 are padded up to a bucket (16, 32, 64, then every 32 to 256) with token id 0 and the
logits of the real rows are returned. Padded rows are never appended to the cache (their slots
are -1) and no real row reads them, so real rows are computed exactly as in eager mode; padded
rows' positions are clamped to the position table.

The runner is used only when every layer's cache holds the same block lists and every pool the
same free list, which the model guarantees (all layers allocate in lockstep), so one metadata
pack serves all layers as in eager mode. Kernels address the pools through the model's per-layer
KVStorage, whose device addresses survive pool growth and pool resets; a graph is captured again
only if a storage is reallocated. Set PAGED_HIP_GRAPHS=0 to run the eager forward instead.
"""
from __future__ import annotations

import math
import os
import weakref

import numpy as np
import torch

from src.cache.paged_kv import BatchedPagedKVCache, KVStorage
from src.kernels import _lib, hip_linear
from src.kernels.hip_paged_attention import (
    _stream_ptr, _workspace, argmax_rows_hip, default_prefill_split_blocks, default_split_blocks, kv_append_hip,
    pack_metadata_mirror_hip, paged_attention_decode_hip, paged_attention_prefill_hip)
from src.kernels.staging import MappedHostWords

try:  # native host bookkeeping (csrc/host/paged_host.cpp): same results as the Python below
    from src.cache import _paged_host as _host
except ImportError:  # not built: the Python versions run
    _host = None

# Query-length buckets of captured prefill steps: padded rows cost as much as real ones, so above
# 64 rows the buckets are 32 rows apart.
T_BUCKETS = (16, 32, 64, 96, 128, 160, 192, 224, 256)

# Largest step (rows = B * bucketed T) for which each fused launch beats torch's layers, per
# dtype. Measured in HIP-graph replay on MI355X (fused vs torch, us), d_model 512, d_ff 2048,
# vocab 5000, with the library's choice between its 16-row and tiled kernels:
#   LayerNorm + q/k/v + append  fp32 11.8 at 256 rows, 32.5 vs 40.4 at 1024, 47.2 vs 46.4 at 1536
#                               (torch without the append); bf16 22.1 vs 33.4 at 1024
#   out_proj + residual         fp32 8.6 vs 11.0 at 1024, 12.6 vs 13.0 at 1536; bf16 5.0 vs 8.0 at 1024
#   LayerNorm + fc1 + GELU      fp32 29.4 vs 31.4 at 768, 39.0 vs 33.6 at 1024; bf16 13.5 vs 14.5
#                               at 512, 19.4 vs 16.7 at 768
#   fc2 + residual              fp32 23.7 vs 24.0 at 1024, 34.3 vs 31.9 at 1536; bf16 10.6 vs 11.0
#                               at 1024, 15.5 vs 12.7 at 1536
#   LayerNorm + lm_head         fp32 10.7 vs 11.8 at 48, 15.8 vs 11.8 at 64; bf16 9.1 vs 10.4 at 64,
#                               13.6 vs 11.2 at 96
FUSED_ROWS = {
    torch.float32: {"qkv": 1024, "out_proj": 1024, "fc1": 768, "fc2": 1024, "lm_head": 48},
    torch.bfloat16: {"qkv": 1024, "out_proj": 1024, "fc1": 512, "fc2": 1024, "lm_head": 64},
}
FUSED_STEP_ROWS = 1024  # steps above this run the torch layers throughout


def graphs_enabled() -> bool:
    return os.environ.get("PAGED_HIP_GRAPHS", "1") != "0"


def fused_decode_enabled() -> bool:
    return os.environ.get("PAGED_HIP_FUSED_DECODE", "1") != "0"


def folded_decode_enabled() -> bool:
    """Four launches per layer in steps of at most 16 rows (fc2 folded into the fc1 launch);
    PAGED_HIP_DECODE_FOLD=0 keeps five."""
    return os.environ.get("PAGED_HIP_DECODE_FOLD", "1") != "0"


def bucket_for(T: int) -> int | None:
    if T == 1:
        return 1
    for b in T_BUCKETS:
        if T <= b:
            return b
    return None


def _pool_tensors(pool):
    """The tensors kernels address: the fixed storage when the pool has one, else its view."""
    if pool.storage is not None and pool.storage.k is not None:
        return pool.storage.k, pool.storage.v
    return pool.k_blocks, pool.v_blocks


def _signature(pools) -> tuple:
    """What a captured step's recorded pool addresses depend on: for storage-backed pools, the
    storages and their allocation count (a view that grows inside its storage keeps its address);
    otherwise every pool tensor's address, length and dtype."""
    if all(p.storage is not None and p.storage.k is not None for p in pools):
        return ("storage", KVStorage.allocations) + tuple(id(p.storage) for p in pools)
    sig = []
    for p in pools:
        k, v = _pool_tensors(p)
        sig.append((k.data_ptr(), v.data_ptr(), k.shape[0], k.dtype))
    return tuple(sig)


def _lockstep(kv_caches: list[BatchedPagedKVCache], max_new_blocks: int) -> bool:
    """_lockstep_py through the native module when it is built."""
    if _host is not None:
        return _host.lockstep(kv_caches, max_new_blocks)
    return _lockstep_py(kv_caches, max_new_blocks)


def _lockstep_py(kv_caches: list[BatchedPagedKVCache], max_new_blocks: int) -> bool:
    """True when all layers hold identical states and pools, so this step's allocations are the
    same in every layer and one metadata pack serves them all. Block lists are compared whole;
    of the free lists, the lengths and the last max_new_blocks ids: a step pops at most that many
    ids from the end of each list (LIFO), and deeper ids are compared in a later step before they
    can be popped (releases push onto the end)."""
    first = kv_caches[0]
    p0 = first.pool
    if p0.k_blocks is None:
        return False
    f0 = p0.free_block_ids
    n0 = len(f0)
    tail0 = f0[n0 - max_new_blocks:] if max_new_blocks < n0 else f0
    states0 = first.states
    for cache in kv_caches[1:]:
        p = cache.pool
        if p.k_blocks is None or p.capacity_blocks != p0.capacity_blocks:
            return False
        f = p.free_block_ids
        if len(f) != n0 or (f[n0 - max_new_blocks:] if max_new_blocks < n0 else f) != tail0:
            return False
        states = cache.states
        if len(states) != len(states0):
            return False
        for a, b in zip(states, states0):
            if a.seq_len != b.seq_len or a.block_ids != b.block_ids:
                return False
    return True


def _step_metadata_py(states, rows, prev, app, cur, sel, shadow, shadow_len, desc, layout) -> tuple[int, int]:
    """Python restatement of the native step_metadata: write the int32 part of a step's
    descriptor (current lengths, greedy rows, mirror rows, first changed page, list lengths,
    lengths before the append, appended counts, and each request's block-list update against its
    mirror row's shadow at a fixed stride) and update the shadow. desc is a flat int32 array;
    layout = (o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, stride) word offsets
    and the update stride. Returns (update count, longest block list)."""
    o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, stride = layout
    R, W = shadow.shape
    n_upd = max_pages = 0
    for b, st in enumerate(states):
        row = rows[b]
        if not 0 <= row < R:
            raise ValueError(f"mirror row {row} outside [0, {R})")
        desc[o_cur + b], desc[o_sel + b], desc[o_mrow + b] = cur[b], sel[b], row
        desc[o_prev + b], desc[o_app + b] = prev[b], app[b]
        ids = st.block_ids
        n = len(ids)
        if n > W:
            raise ValueError(f"a request holds {n} blocks, more than the mirror width {W}")
        max_pages = max(max_pages, n)
        known = min(max(int(shadow_len[row]), 0), n)
        f = 0
        while f < known and ids[f] == shadow[row, f]:
            f += 1
        if n - f > stride:
            raise ValueError("descriptor update area too small")
        shadow[row, f:n] = ids[f:n]
        u = o_upd + b * stride
        desc[u:u + n - f] = ids[f:n]
        n_upd += n - f
        shadow_len[row] = n
        desc[o_first + b], desc[o_npages + b] = f, n
    return n_upd, max_pages


class _BlockTableMirror:
    """The device block-table mirror (int32 [rows, width]), its host shadow and the assignment of
    rows to requests (by the identity of the request's first-layer cache state)."""

    def __init__(self, rows: int, width: int, device: torch.device):
        self.rows, self.width = rows, width
        self.dev = torch.full((rows, width), -1, dtype=torch.int32, device=device)
        self.shadow = np.full((rows, width), -1, dtype=np.int32)
        self.shadow_len = np.zeros((rows,), dtype=np.int32)
        self._row_of: dict[int, int] = {}
        self._owner: list = [None] * rows     # weakref to the state owning the row
        self._used = [0] * rows              # step stamp of the row's last use
        self._free = list(range(rows - 1, -1, -1))
        self._stamp = 0

    def _drop(self, row: int) -> None:
        ref = self._owner[row]
        if ref is not None:
            for key, r in list(self._row_of.items()):
                if r == row:
                    del self._row_of[key]
                    break
        self._owner[row] = None
        self.shadow_len[row] = 0

    def _on_state_gone(self, row: int, ref) -> None:
        if self._owner[row] is ref:
            self._drop(row)
            self._free.append(row)

    def rows_for(self, states) -> list[int] | None:
        """One row per state (distinct states), or None when there are more states than rows."""
        if len(states) > self.rows:
            return None
        self._stamp += 1
        stamp = self._stamp
        out = []
        for st in states:
            r = self._row_of.get(id(st))
            if r is None or self._owner[r] is None or self._owner[r]() is not st:
                r = self._take(stamp)
                self._owner[r] = weakref.ref(st, lambda ref, row=r, me=weakref.ref(self): (
                    me() is not None and me()._on_state_gone(row, ref)))
                self._row_of[id(st)] = r
                self.shadow_len[r] = 0
            self._used[r] = stamp
            out.append(r)
        return out

    def _take(self, stamp: int) -> int:
        if self._free:
            return self._free.pop()
        victim = min((r for r in range(self.rows) if self._used[r] != stamp), key=lambda r: self._used[r])
        self._drop(victim)
        return victim

    def forget(self, rows: list[int]) -> None:
        """The device copy of these rows is unknown (a step failed after its descriptor was
        written): resend them whole next time."""
        for r in rows:
            self.shadow_len[r] = 0


class _Captured:
    def __init__(self, model, B: int, Tb: int, pages: int, device: torch.device, pools, mirror_width: int,
                 tokens_only: bool = False):
        H, Hd = model.num_heads, model.head_dim
        self.B, self.Tb, self.pages = B, Tb, pages
        # A graph whose callers take only the tokens computes ln_f + lm_head for each request's
        # greedy row alone (the other rows' logits are never read), with the argmax folded into
        # that launch (token keys, reset to all ones by the staging copy of every step).
        self.select_head = tokens_only and hip_linear.model_supported(model)
        # Step descriptor (int32 words of pinned host memory the device reads):
        #   [ids int64 B*Tb | first positions int64 B | current lengths B | greedy rows B | padding |
        #    token keys, one 128-byte line per request, all ones (select_head only)]
        #     staged into the device buffer `stage` by the metadata launch;
        #   [mirror rows B | first changed page B | list lengths B | lengths before B | appended B |
        #    update ids, mirror width words per request]  read by that launch in place.
        o_pos = 2 * B * Tb
        o_cur = o_pos + 2 * B
        o_sel = o_cur + B
        ks = hip_linear.KEY_STRIDE
        o_key = -(-(o_sel + B) // (2 * ks)) * (2 * ks)  # each request's key on its own 128-byte line
        self.stage_words = o_key + (2 * B * ks if self.select_head else 0)
        o_mrow = self.stage_words
        o_first, o_npages = o_mrow + B, o_mrow + 2 * B
        o_prev = o_npages + B
        o_app = o_prev + B
        o_upd = o_app + B
        self.layout = (o_cur, o_sel, o_mrow, o_first, o_npages, o_prev, o_app, o_upd, mirror_width)
        self.desc = MappedHostWords(o_upd + B * mirror_width, device)
        w = self.desc.words
        w[o_key:self.stage_words] = -1
        self.ids_host = w[0:o_pos].view(np.int64).reshape(B, Tb)
        self.pos_host = w[o_pos:o_cur].view(np.int64)
        addr = self.desc.device_addr
        self.desc_addrs = {"mirror_row": addr(o_mrow), "first_page": addr(o_first), "num_pages": addr(o_npages),
                           "update_ids": addr(o_upd), "update_stride": mirror_width, "prev_lens": addr(o_prev),
                           "append_lens": addr(o_app), "stage_src": addr(0)}
        self.stage = torch.zeros((self.stage_words,), dtype=torch.int32, device=device)
        self.ids = self.stage[0:o_pos].view(torch.int64).view(B, Tb)
        self.pos = self.stage[o_pos:o_cur].view(torch.int64)
        self.cur = self.stage[o_cur:o_sel]
        self.rows = self.stage[o_sel:o_sel + B]
        if self.select_head:
            self.keys = self.stage[o_key:self.stage_words].view(torch.int64).view(B, ks)[:, 0]
            self.tokens = hip_linear.token_keys_to_tokens(self.keys)
        else:
            self.keys = None
            self.tokens = torch.zeros((B,), dtype=torch.int64, device=device)
        self.last_sel: list[int] = [0] * B
        lib = _lib.load()
        if Tb == 1:
            self.split_blocks = default_split_blocks(B, H, pages, device)
            ws_bytes = lib.pa_decode_workspace_size(B, H, Hd, pages, self.split_blocks)
        else:
            self.split_blocks = default_prefill_split_blocks(B, H, Tb, pages, device, pools[0].dtype)
            ws_bytes = lib.pa_prefill_workspace_size(B, H, Tb, Hd, pages, self.split_blocks)
        # Allocated outside the capture and referenced here, so the address the graph records
        # stays valid for the graph's lifetime.
        self.ws = _workspace(device, ws_bytes, "decode" if Tb == 1 else "prefill") if ws_bytes else None
        self.fused = B * Tb <= FUSED_STEP_ROWS and fused_decode_enabled() and hip_linear.model_supported(model)
        # Steps of at most 16 rows of an fp32 model (every decode step at batch <= 16): per layer
        # four launches, the MLP in one (fc1 column tiles adding their fc2 shares with atomic adds).
        self.folded = (self.fused and B * Tb <= hip_linear.MLP_MAX_ROWS and folded_decode_enabled()
                       and hip_linear.mlp_supported(model))
        emb_dt = model.token_emb.weight.dtype
        self.embed_fused = (fused_decode_enabled() and emb_dt in hip_linear.DTYPES
                            and model.pos_emb.weight.dtype == emb_dt
                            and model.token_emb.embedding_dim % (4 if emb_dt == torch.float32 else 8) == 0)
        self.signature = _signature(pools)
        self.graph = None
        self.logits = None

    def release(self) -> None:
        """Drop the graph, then free the step descriptor it reads (after its last replay)."""
        self.desc.wait()
        self.graph = None
        self.desc.close()


class GraphedStep:
    def __init__(self, model):
        self.model = model
        self.captured: dict[tuple[int, int, bool], _Captured] = {}
        self.captures = 0
        self._attns = None
        self.mirror: _BlockTableMirror | None = None
        # the embedding weight, read per call only for its device (a Parameter keeps its identity
        # across .to() and load_state_dict)
        self._weight = model.token_emb.weight

    def usable(self, input_ids, kv_caches) -> bool:
        """Whether a step over input_ids ([B, T], device tensor or host data) and these per-layer
        caches can replay a graph: a HIP model in eval mode on the hip_paged backend, batched
        caches of every layer in lockstep, and T within the largest bucket."""
        m = self.model
        if self._attns is None or len(self._attns) != len(m.blocks):
            self._attns = [b.attn for b in m.blocks]  # plain attribute reads below, per call
        if not (self._weight.is_cuda and graphs_enabled() and len(input_ids.shape) == 2 and not m.training
                and m.attention_backend == "hip_paged"
                and all(a.attention_backend == "hip_paged" for a in self._attns)
                and isinstance(kv_caches, list) and len(kv_caches) == len(self._attns)
                and all(isinstance(c, BatchedPagedKVCache) for c in kv_caches)):
            return False
        B, T = input_ids.shape
        if bucket_for(T) is None:
            return False
        states0 = kv_caches[0].states
        if len({id(st) for st in states0}) != len(states0):
            return False  # a request twice in one batch: its mirror row would be written twice
        # a request appending up to T tokens opens at most ceil(T / block) + 1 new blocks
        return _lockstep(kv_caches, B * (-(-T // m.kv_block_size) + 1))

    # ------------------------------------------------------------------------------------------
    def _static_forward(self, cap: _Captured, pools) -> torch.Tensor:
        m = self.model
        B, Tb = cap.B, cap.Tb
        pt, seq32, _, slots = pack_metadata_mirror_hip(
            self.mirror.dev, cap.desc_addrs, batch=B, query_len=Tb, block_size=m.kv_block_size,
            max_pages=cap.pages, stage_dst=cap.stage, stage_words=cap.stage_words)
        if cap.embed_fused:
            x = hip_linear.embed_rows_hip(cap.ids, cap.pos, m.token_emb, m.pos_emb).view(B, Tb, -1)
        else:
            steps = torch.arange(Tb, device=cap.ids.device).view(1, Tb)
            positions = torch.clamp(cap.pos.view(B, 1) + steps, max=m.max_seq_len - 1)
            x = m.token_emb(cap.ids) + m.pos_emb(positions)
        if cap.fused:
            x = self._fused_layers(cap, pools, x.view(B * Tb, -1), pt, seq32, slots)
        else:
            x = self._torch_layers(cap, pools, x, pt, seq32, slots).reshape(B * Tb, -1)
        if cap.select_head:
            return hip_linear.linear_select_rows_hip(x, Tb, cap.rows, m.lm_head, ln=m.ln_f, token_keys=cap.keys)
        if cap.fused and B * Tb <= FUSED_ROWS[x.dtype]["lm_head"]:
            logits = hip_linear.linear_rows_hip(x, m.lm_head, ln=m.ln_f)
        else:
            logits = m.lm_head(m.ln_f(x))
        logits = logits.view(B, Tb, -1)
        argmax_rows_hip(logits, cap.rows, out=cap.tokens)
        return logits

    def _torch_layers(self, cap: _Captured, pools, x, pt, seq32, slots) -> torch.Tensor:
        m = self.model
        Tb = cap.Tb
        for blk, pool in zip(m.blocks, pools):
            k_pool, v_pool = _pool_tensors(pool)
            a = blk.attn
            h = blk.ln1(x)
            q = a.heads(a.q_proj(h))
            k_new = a.heads(a.k_proj(h))
            v_new = a.heads(a.v_proj(h))
            kv_append_hip(k_new, v_new, k_pool, v_pool, slots)
            if Tb == 1:
                o = paged_attention_decode_hip(q, k_pool, v_pool, pt, seq32, cap.cur, split_blocks=cap.split_blocks)
            else:
                o = paged_attention_prefill_hip(q, k_pool, v_pool, pt, seq32, cap.cur,
                                                split_blocks=cap.split_blocks)
            x = x + a.out_proj(a.merge_heads(o))
            x = x + blk.mlp(blk.ln2(x))
        return x

    def _fused_layers(self, cap: _Captured, pools, x, pt, seq32, slots) -> torch.Tensor:
        """The layers of a step through the fused kernels; x is [B * Tb, d_model] with at most
        FUSED_STEP_ROWS rows. Layers whose FUSED_ROWS limit the step exceeds run through torch."""
        m = self.model
        B, Tb = cap.B, cap.Tb
        lim = FUSED_ROWS[x.dtype]
        rows = B * Tb
        fc1_fused, fc2_fused = rows <= lim["fc1"], rows <= lim["fc2"]
        # Folded MLP: x stays the residual buffer; out_proj writes x1 into x1_buf (the MLP's input)
        # and into x itself, and the MLP launch adds fc2's output (fc1 tile by fc1 tile) to x.
        x1_buf = torch.empty_like(x) if cap.folded else None
        for blk, pool in zip(m.blocks, pools):
            k_pool, v_pool = _pool_tensors(pool)
            a = blk.attn
            q = hip_linear.qkv_append_hip(x, blk.ln1, a, k_pool, v_pool, slots)
            q4 = q.view(B, Tb, a.num_heads, a.head_dim).transpose(1, 2)
            if Tb == 1:
                o = paged_attention_decode_hip(q4, k_pool, v_pool, pt, seq32, cap.cur, split_blocks=cap.split_blocks)
            else:
                o = paged_attention_prefill_hip(q4, k_pool, v_pool, pt, seq32, cap.cur, split_blocks=cap.split_blocks)
            o2 = o.transpose(1, 2).reshape(rows, a.d_model)
            if cap.folded:
                hip_linear.linear_rows_hip(o2, a.out_proj, residual=x, out=x1_buf, copy_to=x)
                hip_linear.mlp_rows_hip(x1_buf, blk.ln2, blk.mlp[0], blk.mlp[2], x)
                continue
            x1 = hip_linear.linear_rows_hip(o2, a.out_proj, residual=x)
            if fc1_fused:
                h = hip_linear.linear_rows_hip(x1, blk.mlp[0], ln=blk.ln2, gelu=True)
            else:
                h = blk.mlp[1](blk.mlp[0](blk.ln2(x1)))
            if fc2_fused:
                x = hip_linear.linear_rows_hip(h, blk.mlp[2], residual=x1)
            else:
                x = blk.mlp[2](h) + x1
        return x

    def _capture(self, cap: _Captured, pools) -> None:
        # Warm-up on a side stream (initialises library handles); it performs the same step the
        # replay will (same inputs, same slots), so the cache contents are unaffected.
        dev = cap.ids.device
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            self._static_forward(cap, pools)
        torch.cuda.current_stream(dev).wait_stream(side)
        # Each graph keeps its own private memory pool (a step's intermediates are small), so
        # dropping graphs never leaves a shared pool half-released.
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            cap.logits = self._static_forward(cap, pools)
        cap.graph = g
        self.captures += 1

    def _drop_captures(self) -> None:
        for cap in self.captured.values():
            cap.release()
        self.captured.clear()

    # ------------------------------------------------------------------------------------------
    def _mirror_for(self, B: int, pages: int, device: torch.device) -> _BlockTableMirror:
        """The mirror, (re)allocated when a step needs more rows or a wider row than it has; a new
        mirror has a new device address, so every graph is captured again."""
        mir = self.mirror
        if mir is None or B > mir.rows or pages > mir.width:
            rows = max(64, 2 * B, mir.rows if mir is not None else 0)
            width = max(pages, mir.width if mir is not None else 0)
            self._drop_captures()
            self.mirror = mir = _BlockTableMirror(rows, width, device)
        return mir

    def __call__(self, input_ids, positions, current_lengths: list[int], kv_caches, rows: list[int] | None = None,
                 want_logits: bool = True):
        """One cached step, replayed from a captured graph that ends in a greedy argmax.

        input_ids: [B, T] token ids as host data (numpy array or CPU tensor); positions: int, or
        each request's first position as host data; current_lengths: host list (the reference's
        current_lengths, before clamping); rows: per request, the logits row whose argmax becomes
        its token (None: row 0; the tokens then mean nothing).
        Returns (logits [B, T, vocab] or None when want_logits is False, tokens): tokens is an
        integer [B] device tensor owned by the graph (int64; int32 when the argmax is folded into
        the head's launch), overwritten by the next step of this batch size and bucket. The caller checks ids and positions first (the model's
        check_token_inputs), before any cache state changes."""
        m = self.model
        B, T = input_ids.shape
        Tb = bucket_for(T)
        device = self._weight.device
        pools = [c.pool for c in kv_caches]
        app = [max(min(c, T), 0) for c in current_lengths]
        if _host is not None:
            prev = _host.host_append(kv_caches, app, m.num_heads, m.head_dim, pools[0].dtype, device)
        else:
            prev = None
            for cache in kv_caches:
                p = cache.host_append(app, T, m.num_heads, m.head_dim, pools[0].dtype, device)
                prev = p if prev is None else prev
        states0 = kv_caches[0].states
        max_pages = _host.max_blocks(states0) if _host is not None else \
            max((len(st.block_ids) for st in states0), default=0)
        pages = max(-(-m.max_seq_len // m.kv_block_size), max_pages)
        mirror = self._mirror_for(B, pages, device)
        sig = _signature(pools)
        key = (B, Tb, bool(want_logits))
        cap = self.captured.get(key)
        if cap is None or cap.signature != sig or cap.pages < max_pages:
            if cap is not None and cap.signature != sig:
                self._drop_captures()  # every graph holds the old storage addresses
            elif cap is not None:
                cap.release()  # replaced by one with more pages
            cap = _Captured(m, B, Tb, pages, device, pools, mirror.width, tokens_only=not want_logits)
            self.captured[key] = cap
        mrows = mirror.rows_for(states0)
        cap.desc.wait()  # the previous replay of this graph has read its descriptor
        try:
            sel = list(rows) if rows is not None else [0] * B
            step = _host.step_metadata if _host is not None else _step_metadata_py
            step(states0, mrows, prev, app, current_lengths, sel, mirror.shadow, mirror.shadow_len,
                 cap.desc.words, cap.layout)
            ids = input_ids.numpy() if isinstance(input_ids, torch.Tensor) else input_ids
            if T == Tb:
                cap.ids_host[:] = ids
            else:
                cap.ids_host[:, :T] = ids
                cap.ids_host[:, T:] = 0
            cap.pos_host[:] = positions.numpy() if isinstance(positions, torch.Tensor) else positions
            if cap.graph is None:
                self._capture(cap, pools)
            cap.graph.replay()
            cap.desc.mark(_stream_ptr(device))
        except BaseException:
            mirror.forget(mrows)
            raise
        return (cap.logits[:, :T].clone() if want_logits else None), cap.tokens
