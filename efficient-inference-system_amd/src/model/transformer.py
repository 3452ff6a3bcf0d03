"""Decoder-only LM with per-layer paged KV pools (src/model/transformer.py of the reference).

TinyTransformerLM: token + learned position embeddings, pre-LayerNorm blocks (attention, GELU
MLP), final LayerNorm, bias-free lm_head; one LayerBlockPool per layer, created lazily, each a
view of a per-layer KVStorage the model keeps (fixed device addresses). Module and parameter
names match the reference so state dicts load across the two. On the "hip_paged" backend, cached
steps over per-layer batched caches (decode steps and prefill chunks up to 256 tokens) replay
captured HIP graphs (src/model/graph_decode.py); everything else runs eagerly.
"""
import numpy as np
import torch
import torch.nn as nn

from src.cache.paged_kv import BatchedPagedKVCache, KVStorage, LayerBlockPool, PagedKVCacheState

try:  # native host checks (csrc/host/paged_host.cpp); the Python versions below run without it
    from src.cache import _paged_host as _host
except ImportError:
    _host = None
from src.config import ATTENTION_BACKENDS
from src.model.attention import CausalSelfAttention


class TransformerBlock(nn.Module):
    def __init__(self, d_model: int, num_heads: int, d_ff: int, dropout: float = 0.0, attention_backend: str = "hip_paged"):
        super().__init__()
        self.ln1 = nn.LayerNorm(d_model)
        self.attn = CausalSelfAttention(d_model, num_heads, dropout, attention_backend=attention_backend)
        self.ln2 = nn.LayerNorm(d_model)
        self.mlp = nn.Sequential(
            nn.Linear(d_model, d_ff),
            nn.GELU(),
            nn.Linear(d_ff, d_model),
            nn.Dropout(dropout),
        )

    def forward(self, x, kv_cache=None, use_cache: bool = False, current_lengths=None):
        attn_out, kv_cache = self.attn(self.ln1(x), kv_cache=kv_cache, use_cache=use_cache, current_lengths=current_lengths)
        x = x + attn_out
        x = x + self.mlp(self.ln2(x))
        return x, kv_cache


class TinyTransformerLM(nn.Module):
    def __init__(
        self,
        vocab_size: int,
        d_model: int,
        num_heads: int,
        num_layers: int,
        d_ff: int,
        max_seq_len: int,
        dropout: float = 0.0,
        attention_backend: str = "hip_paged",
        kv_block_size: int = 16,
        kv_pool_initial_blocks: int = 64,
        kv_pool_growth_factor: float = 2.0,
        enable_attention_correctness_checks: bool = False,
        kv_cache_dtype: torch.dtype | None = None,
        kv_pool_reserve_blocks: int | None = None,
    ):
        super().__init__()
        if attention_backend not in ATTENTION_BACKENDS:
            raise ValueError(f"Unsupported attention backend: {attention_backend}")
        self.vocab_size = vocab_size
        self.max_seq_len = max_seq_len
        self.attention_backend = attention_backend
        self.kv_block_size = kv_block_size
        self.kv_pool_initial_blocks = kv_pool_initial_blocks
        self.kv_pool_growth_factor = kv_pool_growth_factor
        self.enable_attention_correctness_checks = enable_attention_correctness_checks
        self.kv_cache_dtype = kv_cache_dtype
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.token_emb = nn.Embedding(vocab_size, d_model)
        self.pos_emb = nn.Embedding(max_seq_len, d_model)
        self.blocks = nn.ModuleList(
            [TransformerBlock(d_model, num_heads, d_ff, dropout, attention_backend=attention_backend) for _ in range(num_layers)]
        )
        self.ln_f = nn.LayerNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        self.layer_block_pools: list[LayerBlockPool] | None = None
        # Physical KV storage per layer, kept across pool resets (pools are prefix views of it):
        # None = ceil(max_seq_len / block) * 32 blocks, 0 = plain pools that reallocate on growth.
        if kv_pool_reserve_blocks is None:
            kv_pool_reserve_blocks = max(kv_pool_initial_blocks, 32 * -(-max_seq_len // kv_block_size))
        self._kv_storages = [KVStorage(kv_pool_reserve_blocks) for _ in range(num_layers)] if kv_pool_reserve_blocks else None
        self._graph_step = None

    def _ensure_layer_block_pools(self) -> list[LayerBlockPool]:
        if self.layer_block_pools is None:
            self.layer_block_pools = [
                LayerBlockPool(
                    block_size=self.kv_block_size,
                    initial_blocks=self.kv_pool_initial_blocks,
                    growth_factor=self.kv_pool_growth_factor,
                    dtype=self.kv_cache_dtype,
                    storage=self._kv_storages[i] if self._kv_storages else None,
                )
                for i in range(len(self.blocks))
            ]
        return self.layer_block_pools

    def reset_paged_cache_pools(self) -> None:
        self.layer_block_pools = None

    def _graph_runner(self):
        """Lazily created HIP-graph runner for cached steps (see graph_decode.py)."""
        if self._graph_step is None:
            from src.model.graph_decode import GraphedStep

            self._graph_step = GraphedStep(self)
        return self._graph_step

    @torch.no_grad()
    def prepare_graphs(self, max_batch: int, device, want_logits: bool = False) -> int:
        """Capture the HIP graphs of cached steps ahead of time: for every batch size up to
        max_batch, one prefill chunk per length bucket and one decode step, on throwaway
        requests that are released afterwards. want_logits selects the graphs of steps that return
        logits (forward, greedy_step(return_logits=True)) instead of those that return only the
        greedy tokens. Leaves fresh pools; returns the captures made."""
        from src.model.graph_decode import T_BUCKETS

        device = torch.device(device)
        if device.type != "cuda" or self.attention_backend != "hip_paged" or self._kv_storages is None:
            return 0
        runner = self._graph_runner()
        before = runner.captures
        for B in range(1, max_batch + 1):
            pools = self._ensure_layer_block_pools()
            per_request, pos = None, 0
            for T in (16,) + tuple(T_BUCKETS) + (1,):
                if per_request is None or pos + T > self.max_seq_len:
                    # fresh requests once the current ones would outgrow the position table (the
                    # first step of new requests runs eagerly and initialises nothing new)
                    if per_request is not None:
                        for r in range(B):
                            self.release_request_caches(per_request[r])
                    per_request, pos = self.create_request_kv_caches(B), 0
                    if T > 16 and pos + 16 <= self.max_seq_len:
                        self._prepare_step(per_request, pools, B, 16, pos, device, want_logits)
                        pos += 16
                if pos + T > self.max_seq_len:
                    continue
                self._prepare_step(per_request, pools, B, T, pos, device, want_logits)
                pos += T
            for r in range(B):
                self.release_request_caches(per_request[r])
        torch.cuda.synchronize(device)
        self.reset_paged_cache_pools()
        return runner.captures - before

    def _prepare_step(self, per_request, pools, B, T, pos, device, want_logits) -> None:
        caches = [BatchedPagedKVCache([per_request[r][l] for r in range(B)], pools[l]) for l in range(len(self.blocks))]
        ids = torch.zeros((B, T), dtype=torch.long, device=device)
        if want_logits:
            self(ids, kv_caches=caches, use_cache=True, position_offset=pos, current_lengths=T)
        else:
            self.greedy_step(ids, caches, position_offset=pos, current_lengths=[T] * B)

    def create_request_kv_caches(self, batch_size: int) -> list[list[PagedKVCacheState]]:
        pools = self._ensure_layer_block_pools()
        return [[PagedKVCacheState(pool=pools[layer_idx]) for layer_idx in range(len(self.blocks))] for _ in range(batch_size)]

    def release_request_caches(self, request_caches) -> None:
        if request_caches is None:
            return
        for cache in request_caches:
            if isinstance(cache, PagedKVCacheState):
                cache.release()

    def release_kv_caches(self, kv_caches) -> None:
        if kv_caches is None:
            return
        for cache in kv_caches:
            if isinstance(cache, BatchedPagedKVCache):
                for state in cache.states:
                    state.release()
            elif isinstance(cache, PagedKVCacheState):
                cache.release()

    def set_attention_backend(self, backend_name: str) -> None:
        if backend_name not in ATTENTION_BACKENDS:
            raise ValueError(f"Unsupported attention backend: {backend_name}")
        self.attention_backend = backend_name
        for block in self.blocks:
            block.attn.attention_backend = backend_name

    def paged_memory_stats(self) -> dict[str, int]:
        pools = self.layer_block_pools or []
        reserved = sum(pool.reserved_bytes() for pool in pools)
        allocated = reserved - sum(pool.bytes_per_block() * len(pool.free_block_ids) for pool in pools)
        return {
            "allocated_kv_block_bytes": allocated,
            "reserved_kv_bytes": reserved,
            "free_kv_pool_bytes": max(reserved - allocated, 0),
        }

    def check_token_inputs(self, input_ids, positions, T: int) -> None:
        """Raise IndexError where the embedding lookups of an eager forward would: a token id
        outside [0, vocab_size) or a row position (first position + t, t < T) outside
        [0, max_seq_len). Used before GPU steps, where the graph path clamps instead and an eager
        lookup would fault the device rather than raise. Host data is checked on the host;
        device tensors cost one device->host read."""
        dev_ids = isinstance(input_ids, torch.Tensor) and input_ids.is_cuda
        dev_pos = isinstance(positions, torch.Tensor) and positions.is_cuda
        if _host is not None and not isinstance(input_ids, torch.Tensor) and not isinstance(positions, torch.Tensor):
            try:  # int64 arrays, sequences and ints: one native pass
                _host.check_tokens(input_ids, positions, T, self.vocab_size, self.max_seq_len)
                return
            except TypeError:
                pass  # other element types: the general path below
        if dev_ids or dev_pos:
            parts = ([input_ids.min(), input_ids.max()] if dev_ids and input_ids.numel() else []) + \
                    ([positions.min(), positions.max()] if dev_pos and positions.numel() else [])
            vals = torch.stack([t.to(torch.int64) for t in parts]).tolist() if parts else []
        if dev_ids:
            lo_id, hi_id = (vals[0], vals[1]) if input_ids.numel() else (0, 0)
            vals = vals[2:] if input_ids.numel() else vals
        else:
            ids = input_ids.numpy() if isinstance(input_ids, torch.Tensor) else np.asarray(input_ids)
            lo_id, hi_id = (int(ids.min()), int(ids.max())) if ids.size else (0, 0)
        if isinstance(positions, int):
            lo_pos = hi_pos = positions
        elif dev_pos:
            lo_pos, hi_pos = (vals[0], vals[1]) if positions.numel() else (0, 0)
        elif isinstance(positions, list):
            lo_pos, hi_pos = (min(positions), max(positions)) if positions else (0, 0)
        else:
            p = positions.numpy() if isinstance(positions, torch.Tensor) else np.asarray(positions)
            lo_pos, hi_pos = (int(p.min()), int(p.max())) if p.size else (0, 0)
        if lo_id < 0 or hi_id >= self.vocab_size:
            raise IndexError(f"token id out of range [0, {self.vocab_size}): min {lo_id}, max {hi_id}")
        if T > 0 and (lo_pos < 0 or hi_pos + T - 1 >= self.max_seq_len):
            raise IndexError(f"positions {lo_pos}..{hi_pos + T - 1} outside the position table "
                             f"[0, {self.max_seq_len})")

    @staticmethod
    def _host_step_inputs(input_ids, positions):
        """Token ids and first positions of a graph step as host data (a graph step takes them
        from pinned host memory): device tensors are read back in one copy."""
        on_dev = [isinstance(x, torch.Tensor) and x.is_cuda for x in (input_ids, positions)]
        if on_dev[0] and on_dev[1]:
            n = input_ids.numel()
            both = torch.cat([input_ids.reshape(-1).to(torch.int64), positions.reshape(-1).to(torch.int64)]).cpu()
            return both[:n].view(input_ids.shape).numpy(), both[n:].numpy()
        ids = input_ids.cpu() if on_dev[0] else input_ids
        pos = positions.cpu() if on_dev[1] else positions
        if isinstance(ids, torch.Tensor):
            ids = ids.to(torch.int64).numpy()
        if isinstance(pos, torch.Tensor):
            pos = pos.reshape(-1).to(torch.int64).numpy()
        return ids, pos

    @staticmethod
    def _host_lengths(current_lengths, B: int, T: int) -> list[int]:
        if current_lengths is None:
            return [T] * B
        if isinstance(current_lengths, int):
            return [current_lengths] * B
        if isinstance(current_lengths, torch.Tensor):
            return [int(x) for x in current_lengths.reshape(-1).tolist()]
        return [int(x) for x in current_lengths]

    @torch.no_grad()
    def greedy_step(self, input_ids, kv_caches, position_offset=0, current_lengths=None, select_rows=None,
                    return_logits: bool = False):
        """One cached step that also picks every request's next token greedily.

        input_ids: [B, T] token ids, host data (tensor or numpy array) or a device tensor;
        position_offset: int, or each request's first position (host data or tensor);
        current_lengths: as forward() (None, int, tensor) or a host list;
        select_rows: per request, the logits row whose argmax is its next token (default: its last
        real row, current_lengths - 1; negative rows count from the end as torch indexing does).
        Returns (tokens, logits, caches): tokens an integer [B] tensor on the model's device
        (int64; on the graph path a buffer the next step of the same shape overwrites, read it
        before that: int32 when the argmax is folded into the lm_head launch), logits
        [B, T, vocab] when return_logits else None, and the per-layer caches as forward() returns
        them. On the hip_paged backend with batched caches the step replays a captured graph
        that ends in the greedy selection, so only the token ids need to leave the device."""
        B, T = input_ids.shape
        cur = self._host_lengths(current_lengths, B, T)
        rows = list(select_rows) if select_rows is not None else [c - 1 for c in cur]
        if len(rows) != B or any(not -T <= r < T for r in rows):
            raise IndexError(f"select_rows {rows} out of range for {B} requests of {T} rows")
        rows = [r % T for r in rows]
        runner = self._graph_runner()
        if kv_caches is not None and runner.usable(input_ids, kv_caches):
            ids_h, pos_h = self._host_step_inputs(input_ids, position_offset)
            self.check_token_inputs(ids_h, pos_h, T)
            logits, tokens = runner(ids_h, pos_h, cur, kv_caches, rows=rows, want_logits=return_logits)
            return tokens, logits, list(kv_caches)
        device = self.token_emb.weight.device
        if device.type == "cuda":
            self.check_token_inputs(input_ids, position_offset, T)
        ids = torch.as_tensor(input_ids, dtype=torch.long).to(device)
        pos = position_offset if isinstance(position_offset, int) else \
            torch.as_tensor(position_offset, dtype=torch.long).to(device)
        logits, caches = self(ids, kv_caches=kv_caches, use_cache=True, position_offset=pos,
                              current_lengths=torch.tensor(cur, dtype=torch.long))
        picked = logits[torch.arange(B, device=device), torch.tensor(rows, device=device)]
        return torch.argmax(picked, dim=-1), (logits if return_logits else None), caches

    def forward(
        self,
        input_ids: torch.Tensor,
        kv_caches=None,
        use_cache: bool = False,
        position_offset: int | torch.Tensor = 0,
        current_lengths: int | torch.Tensor | None = None,
    ):
        B, T = input_ids.shape
        device = input_ids.device
        if use_cache and kv_caches is not None and input_ids.is_cuda:
            runner = self._graph_runner()
            if runner.usable(input_ids, kv_caches):
                ids_h, pos_h = self._host_step_inputs(input_ids, position_offset)
                self.check_token_inputs(ids_h, pos_h, T)
                cur = self._host_lengths(current_lengths, B, T)
                logits, _ = runner(ids_h, pos_h, cur, kv_caches)
                return logits, list(kv_caches)
        if input_ids.is_cuda:
            self.check_token_inputs(input_ids, position_offset, T)
        if isinstance(position_offset, int):
            positions = torch.arange(position_offset, position_offset + T, device=device).unsqueeze(0).expand(B, T)
        else:
            positions = position_offset.view(B, 1) + torch.arange(T, device=device).view(1, T)
        x = self.token_emb(input_ids) + self.pos_emb(positions)

        if use_cache and kv_caches is None:
            per_request = self.create_request_kv_caches(B)
            if B > 1:
                pools = self._ensure_layer_block_pools()
                kv_caches = [
                    BatchedPagedKVCache(states=[per_request[r][layer_idx] for r in range(B)], pool=pools[layer_idx])
                    for layer_idx in range(len(self.blocks))
                ]
            else:
                kv_caches = [per_request[0][layer_idx] for layer_idx in range(len(self.blocks))]

        # A device tensor of per-request lengths is read on the host by every layer's append;
        # convert it once here (a single device->host copy) and pass the list down.
        if isinstance(current_lengths, torch.Tensor) and use_cache:
            current_lengths_host = current_lengths
            if current_lengths.is_cuda:
                current_lengths_host = current_lengths.cpu()
        else:
            current_lengths_host = current_lengths

        new_caches = [] if use_cache else None
        for i, block in enumerate(self.blocks):
            cache_i = kv_caches[i] if use_cache else None
            x, cache_i = block(x, kv_cache=cache_i, use_cache=use_cache, current_lengths=current_lengths_host)
            if use_cache:
                new_caches.append(cache_i)
        x = self.ln_f(x)
        logits = self.lm_head(x)
        return logits, new_caches
