"""Batched greedy generation through the paged KV cache.

Mirrors src/inference/generate_with_cache.py:112-260 of the reference: one prefill forward over
the padded prompts with current_lengths = prompt lengths, the first token from each request's
last prompt position, then one decode forward per step over the requests that still need tokens
(each step restacks the active requests' per-layer cache states). Returns the same result keys.
"""
import torch

from src.cache.paged_kv import BatchedPagedKVCache, PagedKVCacheState
from src.utils.timing import timed_section


def _normalize_prompt_lengths(prompt_ids: torch.Tensor, prompt_lengths: torch.Tensor | None) -> torch.Tensor:
    if prompt_lengths is None:
        return torch.full((prompt_ids.shape[0],), prompt_ids.shape[1], device=prompt_ids.device, dtype=torch.long)
    return prompt_lengths.to(device=prompt_ids.device, dtype=torch.long)


def _normalize_decode_limits(batch_size: int, device: torch.device, max_new_tokens) -> torch.Tensor:
    if isinstance(max_new_tokens, int):
        return torch.full((batch_size,), max_new_tokens, device=device, dtype=torch.long)
    if isinstance(max_new_tokens, torch.Tensor):
        return max_new_tokens.to(device=device, dtype=torch.long)
    return torch.tensor(max_new_tokens, device=device, dtype=torch.long)


def _extract_request_caches(kv_caches, batch_size: int):
    """Per-request, per-layer cache states from the per-layer caches a forward returned."""
    if kv_caches is None:
        return None
    request_caches = [[] for _ in range(batch_size)]
    for layer_cache in kv_caches:
        if isinstance(layer_cache, BatchedPagedKVCache):
            for request_idx, state in enumerate(layer_cache.states):
                request_caches[request_idx].append(state)
        else:
            for request_idx in range(batch_size):
                request_caches[request_idx].append(layer_cache)
    return request_caches


def _stack_request_caches(request_caches, request_indices: list[int]):
    """Per-layer BatchedPagedKVCache over the given requests."""
    if request_caches is None or not request_indices:
        return None
    num_layers = len(request_caches[request_indices[0]])
    stacked = []
    for layer_idx in range(num_layers):
        entries = [request_caches[r][layer_idx] for r in request_indices]
        sample = next((e for e in entries if e is not None), None)
        if sample is None:
            raise ValueError("Paged request caches must be initialized before stacking.")
        states = [e if isinstance(e, PagedKVCacheState) else PagedKVCacheState(pool=sample.pool) for e in entries]
        stacked.append(BatchedPagedKVCache(states=states, pool=sample.pool))
    return stacked


def _scatter_request_caches(request_caches, request_indices: list[int], kv_caches) -> None:
    if request_caches is None or kv_caches is None:
        return
    for layer_idx, layer_cache in enumerate(kv_caches):
        if isinstance(layer_cache, BatchedPagedKVCache):
            for local_idx, request_idx in enumerate(request_indices):
                request_caches[request_idx][layer_idx] = layer_cache.states[local_idx]
        else:
            for request_idx in request_indices:
                request_caches[request_idx][layer_idx] = layer_cache


def _cache_metric_totals(request_caches, model=None) -> tuple[int, int, int]:
    if request_caches is None:
        return 0, 0, 0
    live = sum(c.live_bytes() for caches in request_caches for c in caches if isinstance(c, PagedKVCacheState))
    pool_stats = model.paged_memory_stats() if model is not None and hasattr(model, "paged_memory_stats") else {}
    reserved = pool_stats.get("reserved_kv_bytes", live)
    return live, reserved, max(reserved - live, 0)


def _gpu_bytes(device: torch.device) -> tuple[int, int]:
    if device.type == "cuda" and torch.cuda.is_available():
        return int(torch.cuda.memory_allocated(device)), int(torch.cuda.max_memory_allocated(device))
    return 0, 0


@torch.no_grad()
def generate_with_cache(model, prompt_ids: torch.Tensor, max_new_tokens, prompt_lengths: torch.Tensor | None = None):
    device = prompt_ids.device
    batch_size = prompt_ids.shape[0]
    prompt_lengths = _normalize_prompt_lengths(prompt_ids, prompt_lengths)
    decode_limits = _normalize_decode_limits(batch_size, device, max_new_tokens)
    prompt_len_host = [int(x) for x in prompt_lengths.tolist()]
    limits_host = [int(x) for x in decode_limits.tolist()]

    if max(limits_host, default=0) <= 0:
        return {
            "generated_ids": [prompt_ids[idx, : prompt_len_host[idx]].clone() for idx in range(batch_size)],
            "prefill_time_ms": 0.0,
            "decode_times_ms": [],
            "per_generated_token_times_ms": [],
            "total_time_ms": 0.0,
            "avg_generated_token_time_ms": 0.0,
            "avg_decode_only_token_time_ms": 0.0,
            "cache_bytes": 0,
            "kv_caches": None,
            "num_generated_tokens": 0,
            "generated_tokens_per_request": [0] * batch_size,
        }

    with timed_section(device=device) as prefill_timer:
        logits, kv_caches = model(prompt_ids, use_cache=True, position_offset=0, current_lengths=prompt_lengths)
        last_prompt_logits = logits[torch.arange(batch_size, device=device), prompt_lengths - 1, :]
        next_tokens = torch.argmax(last_prompt_logits, dim=-1)

    prefill_time_ms = prefill_timer.elapsed_ms
    decode_times_ms: list[float] = []
    decode_tokens_per_step: list[int] = []
    per_generated_token_times_ms = [prefill_time_ms]
    generated_tokens_per_request = [0] * batch_size
    generated_token_ids: list[list[int]] = [[] for _ in range(batch_size)]
    last_tokens: list[int | None] = [None] * batch_size

    first = next_tokens.tolist()
    for r in range(batch_size):
        if limits_host[r] > 0:
            generated_token_ids[r].append(int(first[r]))
            generated_tokens_per_request[r] = 1
            last_tokens[r] = int(first[r])

    request_caches = _extract_request_caches(kv_caches, batch_size)
    for _ in range(1, max(limits_host)):
        active = [r for r in range(batch_size) if generated_tokens_per_request[r] < limits_host[r]]
        if not active:
            break
        decode_input = torch.tensor([[last_tokens[r]] for r in active], device=device, dtype=torch.long)
        current_pos = torch.tensor(
            [prompt_len_host[r] + generated_tokens_per_request[r] - 1 for r in active], device=device, dtype=torch.long
        )
        active_caches = _stack_request_caches(request_caches, active)
        with timed_section(device=device) as timer:
            logits, active_caches = model(
                decode_input, kv_caches=active_caches, use_cache=True, position_offset=current_pos, current_lengths=1
            )
            next_tokens = torch.argmax(logits[:, -1, :], dim=-1)
        decode_times_ms.append(timer.elapsed_ms)
        decode_tokens_per_step.append(len(active))
        per_generated_token_times_ms.append(timer.elapsed_ms)
        _scatter_request_caches(request_caches, active, active_caches)
        for local_idx, r in enumerate(next_tokens.tolist()):
            req = active[local_idx]
            generated_token_ids[req].append(int(r))
            generated_tokens_per_request[req] += 1
            last_tokens[req] = int(r)

    final_request_caches = _stack_request_caches(request_caches, list(range(batch_size)))
    live_kv_bytes, reserved_kv_bytes, fragmentation_bytes = _cache_metric_totals(request_caches, model=model)
    gpu_allocated_bytes, gpu_peak_allocated_bytes = _gpu_bytes(device)
    total_time_ms = sum(per_generated_token_times_ms)
    total_generated_tokens = sum(generated_tokens_per_request)
    decode_kernel_tokens = sum(decode_tokens_per_step)
    generated_ids = [
        torch.cat(
            [
                prompt_ids[idx, : prompt_len_host[idx]].clone(),
                torch.tensor(generated_token_ids[idx], device=device, dtype=prompt_ids.dtype),
            ]
        )
        for idx in range(batch_size)
    ]
    return {
        "generated_ids": generated_ids,
        "prefill_time_ms": prefill_time_ms,
        "decode_times_ms": decode_times_ms,
        "decode_tokens_per_step": decode_tokens_per_step,
        "per_generated_token_times_ms": per_generated_token_times_ms,
        "total_time_ms": total_time_ms,
        "avg_generated_token_time_ms": total_time_ms / total_generated_tokens if total_generated_tokens > 0 else 0.0,
        "avg_decode_only_token_time_ms": sum(decode_times_ms) / decode_kernel_tokens if decode_kernel_tokens > 0 else 0.0,
        "cache_bytes": reserved_kv_bytes if reserved_kv_bytes > 0 else live_kv_bytes,
        "live_kv_bytes": live_kv_bytes,
        "reserved_kv_bytes": reserved_kv_bytes,
        "fragmentation_bytes": fragmentation_bytes,
        "workspace_bytes": 0,
        "gpu_allocated_bytes": gpu_allocated_bytes,
        "gpu_peak_allocated_bytes": gpu_peak_allocated_bytes,
        "kv_caches": final_request_caches,
        "num_generated_tokens": max(generated_tokens_per_request),
        "generated_tokens_per_request": generated_tokens_per_request,
        "decode_kernel_tokens": decode_kernel_tokens,
        "backend_name": getattr(model, "attention_backend", "hip_paged"),
    }
