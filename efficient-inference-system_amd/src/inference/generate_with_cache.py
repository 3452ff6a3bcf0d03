"""Batched greedy generation through the paged KV cache.

Interface and result keys of the reference's generate_with_cache
(src/inference/generate_with_cache.py:112-260): the prompts are right-padded rows of prompt_ids
with their real lengths in prompt_lengths (default: the full width) and max_new_tokens is an int,
a list or a tensor of per-request limits.

The generation is a loop of model.greedy_step() calls, each timed with the device synchronised on
both sides (the argmax is inside the timed step, as in the reference):
  - one prefill step over every prompt (current_lengths = the prompt lengths), whose token for
    request r comes from the logits row prompt_length - 1; a request with a limit of 0 takes none;
  - then one decode step per round over the requests still below their limit, each feeding its
    last token at position prompt_length + generated - 1. The per-layer states of the active
    requests are batched afresh every round; a request's states persist across rounds.
On the hip_paged backend every decode round replays a captured graph that ends in the argmax, so
a round reads back only the active requests' token ids.
"""
from __future__ import annotations

import numpy as np
import torch

from src.cache.paged_kv import BatchedPagedKVCache, PagedKVCacheState
from src.utils.timing import timed_section


def _per_request(values, batch_size: int, default: int) -> list[int]:
    if values is None:
        return [default] * batch_size
    if isinstance(values, int):
        return [values] * batch_size
    if isinstance(values, torch.Tensor):
        values = values.reshape(-1).tolist()
    return [int(v) for v in values]


class _Generation:
    """Per-request host state of one generate_with_cache call."""

    def __init__(self, prompt_ids: torch.Tensor, lengths: list[int], limits: list[int]):
        self.prompt_ids = prompt_ids
        self.lengths = lengths
        self.limits = limits
        self.tokens: list[list[int]] = [[] for _ in lengths]
        self.layer_states: list[list] | None = None  # [request][layer]

    def active(self) -> list[int]:
        return [r for r, (toks, lim) in enumerate(zip(self.tokens, self.limits)) if len(toks) < lim]

    def take(self, requests: list[int], tokens: list[int]) -> None:
        for r, t in zip(requests, tokens):
            self.tokens[r].append(int(t))

    def keep_states(self, layer_caches, batch_size: int) -> None:
        """Per-request states from the per-layer caches the prefill step returned."""
        self.layer_states = [[] for _ in range(batch_size)]
        for cache in layer_caches:
            states = cache.states if isinstance(cache, BatchedPagedKVCache) else [cache] * batch_size
            for r in range(batch_size):
                self.layer_states[r].append(states[r])

    def batched(self, requests: list[int]) -> list[BatchedPagedKVCache] | None:
        """Per-layer batched caches over the given requests' states."""
        if self.layer_states is None or not requests:
            return None
        out = []
        for layer in zip(*(self.layer_states[r] for r in requests)):
            pool = next((s.pool for s in layer if s is not None), None)
            if pool is None:
                raise ValueError("Paged request caches must be initialized before stacking.")
            out.append(BatchedPagedKVCache([s if isinstance(s, PagedKVCacheState) else PagedKVCacheState(pool=pool)
                                            for s in layer], pool))
        return out

    def adopt(self, requests: list[int], layer_caches) -> None:
        if self.layer_states is None or layer_caches is None:
            return
        for layer, cache in enumerate(layer_caches):
            for i, r in enumerate(requests):
                self.layer_states[r][layer] = cache.states[i] if isinstance(cache, BatchedPagedKVCache) else cache

    def kv_bytes(self, model) -> tuple[int, int, int]:
        if self.layer_states is None:
            return 0, 0, 0
        live = sum(s.live_bytes() for states in self.layer_states for s in states if isinstance(s, PagedKVCacheState))
        stats = model.paged_memory_stats() if hasattr(model, "paged_memory_stats") else {}
        reserved = stats.get("reserved_kv_bytes", live)
        return live, reserved, max(reserved - live, 0)


def _memory(device: torch.device) -> tuple[int, int]:
    if device.type == "cuda" and torch.cuda.is_available():
        return int(torch.cuda.memory_allocated(device)), int(torch.cuda.max_memory_allocated(device))
    return 0, 0


@torch.no_grad()
def generate_with_cache(model, prompt_ids: torch.Tensor, max_new_tokens, prompt_lengths: torch.Tensor | None = None):
    device = prompt_ids.device
    B, width = prompt_ids.shape
    gen = _Generation(prompt_ids, _per_request(prompt_lengths, B, width), _per_request(max_new_tokens, B, 0))

    if max(gen.limits, default=0) <= 0:
        return {
            "generated_ids": [prompt_ids[r, :gen.lengths[r]].clone() for r in range(B)],
            "prefill_time_ms": 0.0, "decode_times_ms": [], "per_generated_token_times_ms": [],
            "total_time_ms": 0.0, "avg_generated_token_time_ms": 0.0, "avg_decode_only_token_time_ms": 0.0,
            "cache_bytes": 0, "kv_caches": None, "num_generated_tokens": 0,
            "generated_tokens_per_request": [0] * B,
        }

    with timed_section(device=device) as prefill_timer:
        tokens, _, caches = model.greedy_step(prompt_ids, None, position_offset=0,
                                              current_lengths=torch.tensor(gen.lengths, dtype=torch.long),
                                              select_rows=[n - 1 for n in gen.lengths])
    first = tokens.tolist()
    gen.take([r for r in range(B) if gen.limits[r] > 0], [first[r] for r in range(B) if gen.limits[r] > 0])
    gen.keep_states(caches, B)

    step_times: list[float] = []
    step_sizes: list[int] = []
    while True:
        active = gen.active()
        if not active:
            break
        last = np.asarray([[gen.tokens[r][-1]] for r in active], dtype=np.int64)
        positions = [gen.lengths[r] + len(gen.tokens[r]) - 1 for r in active]
        batched = gen.batched(active)
        with timed_section(device=device) as timer:
            tokens, _, batched = model.greedy_step(last, batched, position_offset=positions, current_lengths=1)
        step_times.append(timer.elapsed_ms)
        step_sizes.append(len(active))
        gen.adopt(active, batched)
        gen.take(active, tokens.tolist())

    live, reserved, fragmentation = gen.kv_bytes(model)
    allocated, peak = _memory(device)
    per_token = [prefill_timer.elapsed_ms] + step_times
    produced = [len(t) for t in gen.tokens]
    total_ms = sum(per_token)
    generated_ids = [torch.cat([prompt_ids[r, :gen.lengths[r]].clone(),
                                torch.tensor(gen.tokens[r], device=device, dtype=prompt_ids.dtype)])
                     for r in range(B)]
    return {
        "generated_ids": generated_ids,
        "prefill_time_ms": prefill_timer.elapsed_ms,
        "decode_times_ms": step_times,
        "decode_tokens_per_step": step_sizes,
        "per_generated_token_times_ms": per_token,
        "total_time_ms": total_ms,
        "avg_generated_token_time_ms": total_ms / sum(produced) if sum(produced) else 0.0,
        "avg_decode_only_token_time_ms": sum(step_times) / sum(step_sizes) if sum(step_sizes) else 0.0,
        "cache_bytes": reserved if reserved > 0 else live,
        "live_kv_bytes": live,
        "reserved_kv_bytes": reserved,
        "fragmentation_bytes": fragmentation,
        "workspace_bytes": 0,
        "gpu_allocated_bytes": allocated,
        "gpu_peak_allocated_bytes": peak,
        "kv_caches": gen.batched(list(range(B))),
        "num_generated_tokens": max(produced),
        "generated_tokens_per_request": produced,
        "decode_kernel_tokens": sum(step_sizes),
        "backend_name": getattr(model, "attention_backend", "hip_paged"),
    }
