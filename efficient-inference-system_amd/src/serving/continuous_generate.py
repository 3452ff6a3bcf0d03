"""Continuous-batching executors: run one scheduler iteration's prefill chunk or decode step on a
paged-KV model and pick each request's next token greedily.

The two entry points keep the reference's names, positional arguments and event keys
(src/serving/continuous_generate.py:82-276), since ContinuousBatchingScheduler and the benchmark
harness call them that way and read those keys:

    run_prefill_chunk(model, requests, chunk_size, device, start_time_ms, event_id) -> event
    run_decode_step(model, requests, device, start_time_ms, event_id) -> event

Each call goes through three stages of a StepExecutor:

  plan     (host)  the step's token ids as a host array padded with id 0 to the group's longest
                   chunk, each request's first position, its real token count (current_lengths)
                   and the logits row its next token is read from (its last real row);
  execute  (timed) one model.greedy_step(): on the hip_paged backend a captured HIP graph whose
                   last kernel is the argmax, so no [B, T, vocab] logits leave the device; only
                   the B token ids are read back, after the timed region;
  commit   (host)  tokens appended, phase transitions (prefill -> decode -> finished), first-token
                   and finish times on the scheduler's virtual clock, and the event record.

As in the reference, the batch runtime that advances the virtual clock is the timed model step,
which here includes the on-device argmax (part of the captured step). A StepExecutor can also
keep each step's logits and report every step to an observer, which is what the end-to-end
parity test uses to replay the same steps on another backend.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

from src.cache.paged_kv import BatchedPagedKVCache, PagedKVCacheState
from src.utils.timing import timed_section


@dataclass
class StepPlan:
    """Host-side description of one model step over a group of requests."""
    phase: str                    # "prefill" or "decode"
    requests: list
    token_ids: np.ndarray         # int64 [B, T], right-padded with id 0
    positions: int | list[int]    # first position: shared (prefill) or per request (decode)
    lengths: list[int]            # real tokens per request (the model's current_lengths)
    rows: list[int]               # logits row of each request's next token

    @property
    def padded_len(self) -> int:
        return int(self.token_ids.shape[1])


def plan_prefill(requests: list, chunk_size: int) -> StepPlan | None:
    """The next chunk of a group with equal prompt progress: up to chunk_size prompt tokens per
    request. None when no request has prompt tokens left."""
    start = requests[0].prompt_tokens_processed
    if any(r.prompt_tokens_processed != start for r in requests):
        raise ValueError("run_prefill_chunk expects requests with the same prompt progress.")
    lengths = [max(min(chunk_size, r.prompt_len - start), 0) for r in requests]
    width = max(lengths)
    if width <= 0:
        return None
    ids = np.zeros((len(requests), width), dtype=np.int64)
    for row, (r, n) in zip(ids, zip(requests, lengths)):
        row[:n] = r.prompt_ids[start:start + n].cpu().numpy()
    return StepPlan("prefill", requests, ids, start, lengths, [n - 1 for n in lengths])


def plan_decode(requests: list) -> StepPlan:
    """One token per request: its last generated token at position prompt_len + generated - 1."""
    ids = np.asarray([[r.generated_token_ids[-1]] for r in requests], dtype=np.int64)
    positions = [r.prompt_len + r.num_generated_tokens - 1 for r in requests]
    return StepPlan("decode", requests, ids, positions, [1] * len(requests), [0] * len(requests))


def _layer_batches(model, requests: list) -> list[BatchedPagedKVCache]:
    """Per-layer batched caches over the requests' per-layer states, creating the states of
    requests that have none yet (a request's states persist across its steps)."""
    fresh = [r for r in requests if r.kv_caches is None]
    for r, caches in zip(fresh, model.create_request_kv_caches(len(fresh)) if fresh else []):
        r.kv_caches = caches
    batches = []
    for layer in zip(*(r.kv_caches for r in requests)):
        pool = next((c.pool for c in layer if c is not None), None)
        if pool is None:
            raise ValueError("Paged request caches must be initialized before batching.")
        states = [c if isinstance(c, PagedKVCacheState) else PagedKVCacheState(pool=pool) for c in layer]
        batches.append(BatchedPagedKVCache(states=states, pool=pool))
    return batches


def _adopt(requests: list, layer_caches) -> None:
    """Point each request at its per-layer state in the caches the model step returned."""
    if layer_caches is None:
        return
    for i, r in enumerate(requests):
        r.kv_caches = [c.states[i] if isinstance(c, BatchedPagedKVCache) else c for c in layer_caches]


def _kv_accounting(model, requests: list) -> dict:
    live = sum(c.live_bytes() for r in requests for c in (r.kv_caches or ()) if isinstance(c, PagedKVCacheState))
    reserved = model.paged_memory_stats().get("reserved_kv_bytes", live) if hasattr(model, "paged_memory_stats") \
        else live
    return {"live_kv_bytes": live, "reserved_kv_bytes": reserved, "fragmentation_bytes": max(reserved - live, 0)}


def _device_memory(device) -> dict:
    on_gpu = str(device).startswith("cuda") and torch.cuda.is_available()
    return {"gpu_allocated_bytes": int(torch.cuda.memory_allocated()) if on_gpu else 0,
            "gpu_peak_allocated_bytes": int(torch.cuda.max_memory_allocated()) if on_gpu else 0}


def _kv_bytes_per_token(model) -> int:
    """KV bytes one token occupies over all layers (K and V rows of d_model elements)."""
    elem = next(model.parameters()).element_size()
    return 2 * len(model.blocks) * model.blocks[0].attn.d_model * elem


class StepExecutor:
    """Runs planned steps on `model`. keep_logits: also return each step's logits (for tests;
    on the graph path this copies them out of the graph); observer(plan, tokens, logits, event):
    called after every step."""

    def __init__(self, model, device, keep_logits: bool = False, observer=None):
        self.model = model
        self.device = device
        self.keep_logits = keep_logits
        self.observer = observer

    def _execute(self, plan: StepPlan) -> tuple[list[int], torch.Tensor | None, float]:
        caches = _layer_batches(self.model, plan.requests)
        with timed_section(device=self.device) as timer:
            tokens, logits, caches = self.model.greedy_step(
                plan.token_ids, caches, position_offset=plan.positions, current_lengths=plan.lengths,
                select_rows=plan.rows, return_logits=self.keep_logits)
        tokens = [int(t) for t in tokens.tolist()]  # the step's only device->host read
        _adopt(plan.requests, caches)
        return tokens, logits, timer.elapsed_ms

    def run(self, plan: StepPlan, start_time_ms: float, event_id: int) -> dict:
        tokens, logits, runtime = self._execute(plan)
        finish = start_time_ms + runtime
        completed, emitted = [], 0
        for r, tok, n in zip(plan.requests, tokens, plan.lengths):
            if r.start_time_ms is None:
                r.start_time_ms, r.batch_id = start_time_ms, event_id
            r.scheduler_mode = "continuous"
            if plan.phase == "prefill":
                r.prompt_tokens_processed += n
                if r.prompt_tokens_processed < r.prompt_len:
                    r.phase = "prefill"
                    continue
                if r.first_token_time_ms is None:
                    r.first_token_time_ms = finish
            r.generated_token_ids.append(tok)
            emitted += 1
            if r.num_generated_tokens >= r.max_new_tokens:
                r.phase, r.finish_time_ms = "finished", finish
                completed.append(r)
            else:
                r.phase = "decode"
        event = self._event(plan, runtime, completed, emitted)
        if self.observer is not None:
            self.observer(plan, tokens, logits, event)
        return event

    def _event(self, plan: StepPlan, runtime: float, completed: list, emitted: int) -> dict:
        reqs = plan.requests
        n = len(reqs)
        real = sum(plan.lengths)
        prefill = plan.phase == "prefill"
        waste = n * plan.padded_len - real if prefill else 0
        event = {
            "batch_runtime_ms": runtime,
            "requests_completed": completed,
            "batch_size": n,
            "tokens_scheduled": real,
            "phase": plan.phase,
            "prompt_len": max(r.prompt_len for r in reqs),
            "max_new_tokens": max(r.max_new_tokens for r in reqs),
            "prefill_tokens": real if prefill else 0,
            "decode_tokens": emitted,
            "decode_kernel_tokens": 0 if prefill else n,
            "prefill_runtime_ms": runtime if prefill else 0.0,
            "decode_runtime_ms": 0.0 if prefill else runtime,
            "decode_ms_per_token": 0.0 if prefill else runtime / max(n, 1),
            # split-K workspaces of captured steps are allocated at capture, none per step
            "workspace_bytes": 0,
            "backend_name": getattr(self.model, "attention_backend", "hip_paged"),
            "padding_waste_tokens": waste,
            "padding_waste_bytes_est": waste * _kv_bytes_per_token(self.model),
            "padding_waste_pct": 100.0 * waste / (n * plan.padded_len) if prefill else 0.0,
        }
        event.update(_kv_accounting(self.model, reqs))
        event.update(_device_memory(self.device))
        return event


_IDLE = {"batch_runtime_ms": 0.0, "requests_completed": []}


@torch.no_grad()
def run_prefill_chunk(model, requests: list, chunk_size: int, device: str, start_time_ms: float,
                      event_id: int, executor: StepExecutor | None = None) -> dict:
    """One prefill chunk for a group of requests with equal prompt progress; requests whose
    prompt completes emit their first token."""
    if not requests:
        return dict(_IDLE)
    plan = plan_prefill(requests, chunk_size)
    if plan is None:
        return dict(_IDLE)
    return (executor or StepExecutor(model, device)).run(plan, start_time_ms, event_id)


@torch.no_grad()
def run_decode_step(model, requests: list, device: str, start_time_ms: float, event_id: int,
                    executor: StepExecutor | None = None) -> dict:
    """One decode step: one new token for every request in the group."""
    if not requests:
        return dict(_IDLE)
    return (executor or StepExecutor(model, device)).run(plan_decode(requests), start_time_ms, event_id)
