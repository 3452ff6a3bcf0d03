"""Continuous-batching scheduler on a virtual clock (src/serving/scheduler.py:254-465 of the reference).

Policy, step for step as in the reference:
  - requests are sorted by arrival; an idle scheduler jumps the clock to the next arrival;
  - arrivals up to the current time join a FIFO waiting queue, and up to max_batch_size of them
    are admitted to the active set;
  - each iteration first runs ONE decode step for every active request in the decode phase, then
    spends the remaining token budget (max_tokens_per_iteration minus the decode tokens) on prefill:
    repeatedly pick the group of prefill-phase requests with equal prompt progress that is largest,
    ties going to the group with the earliest arrival, and give it a chunk of
    min(prefill_chunk_size, budget // group size) tokens per request;
  - after every executor call the clock advances by the call's measured runtime, finished requests
    are released and retired, and new arrivals are admitted.
Executors are injected callables returning a dict with batch_runtime_ms, tokens_scheduled,
requests_completed, batch_size, prompt_len, max_new_tokens, phase and optional accounting keys;
one event record per call is returned alongside the completed requests.
"""
from __future__ import annotations

_OPTIONAL_KEYS_INT = (
    "prefill_tokens", "decode_tokens", "decode_kernel_tokens", "live_kv_bytes", "reserved_kv_bytes",
    "fragmentation_bytes", "workspace_bytes", "gpu_allocated_bytes", "gpu_peak_allocated_bytes",
    "padding_waste_tokens", "padding_waste_bytes_est",
)
_OPTIONAL_KEYS_FLOAT = ("prefill_runtime_ms", "decode_runtime_ms", "decode_ms_per_token", "padding_waste_pct")


class ContinuousBatchingScheduler:
    """Continuous batching with strict decode priority and chunked, progress-grouped prefill."""

    def __init__(self, max_batch_size: int, prefill_chunk_size: int, max_tokens_per_iteration: int):
        self.max_batch_size = max_batch_size
        self.prefill_chunk_size = prefill_chunk_size
        self.max_tokens_per_iteration = max_tokens_per_iteration

    def _enqueue_arrivals(self, requests: list, next_request_idx: int, current_time_ms: float, waiting: list) -> int:
        while next_request_idx < len(requests) and requests[next_request_idx].arrival_time_ms <= current_time_ms:
            waiting.append(requests[next_request_idx])
            next_request_idx += 1
        return next_request_idx

    def _admit_waiting(self, waiting: list, active: list) -> None:
        while waiting and len(active) < self.max_batch_size:
            active.append(waiting.pop(0))

    def _build_prefill_groups(self, active: list) -> dict[int, list]:
        groups: dict[int, list] = {}
        for req in active:
            if req.phase == "prefill":
                groups.setdefault(req.prompt_tokens_processed, []).append(req)
        return groups

    def _select_prefill_group(self, groups: dict[int, list]) -> int:
        return max(groups, key=lambda k: (len(groups[k]), -min(r.arrival_time_ms for r in groups[k])))

    def _event(self, event_id: int, finish_time_ms: float, res: dict) -> dict:
        runtime = res["batch_runtime_ms"]
        record = {
            "batch_id": event_id,
            "dispatch_time_ms": finish_time_ms - runtime,
            "finish_time_ms": finish_time_ms,
            "batch_size": res["batch_size"],
            "batch_runtime_ms": runtime,
            "prompt_len": res["prompt_len"],
            "max_new_tokens": res["max_new_tokens"],
            "tokens_generated_total": res["tokens_scheduled"],
            "scheduler_mode": "continuous",
            "scheduling_policy_value": self.prefill_chunk_size,
            "phase": res["phase"],
            "tokens_scheduled": res["tokens_scheduled"],
            "tokens_per_s": 1000.0 * res["tokens_scheduled"] / runtime if runtime > 0 else 0.0,
            "active_requests": res["batch_size"],
        }
        for key in _OPTIONAL_KEYS_INT:
            record[key] = res.get(key, 0)
        for key in _OPTIONAL_KEYS_FLOAT:
            record[key] = res.get(key, 0.0)
        record["backend_name"] = res.get("backend_name", "hip_paged")
        return record

    def run(self, requests: list, prefill_executor, decode_executor, release_request_cache=None) -> tuple[list, list[dict]]:
        requests = sorted(requests, key=lambda r: r.arrival_time_ms)
        waiting: list = []
        active: list = []
        completed: list = []
        events: list[dict] = []
        now = 0.0
        next_idx = 0
        event_id = 0
        total = len(requests)

        def retire(res: dict) -> None:
            for done in res["requests_completed"]:
                if release_request_cache is not None:
                    release_request_cache(done)
                active.remove(done)
                completed.append(done)

        while len(completed) < total:
            if not waiting and not active and next_idx < total:
                now = max(now, requests[next_idx].arrival_time_ms)
            next_idx = self._enqueue_arrivals(requests, next_idx, now, waiting)
            self._admit_waiting(waiting, active)
            if not active:
                continue

            used = 0
            decode_group = [req for req in active if req.phase == "decode"]
            if decode_group:
                res = decode_executor(decode_group, now, event_id)
                now += res["batch_runtime_ms"]
                used += res["tokens_scheduled"]
                retire(res)
                events.append(self._event(event_id, now, res))
                event_id += 1
                next_idx = self._enqueue_arrivals(requests, next_idx, now, waiting)
                self._admit_waiting(waiting, active)

            budget = max(self.max_tokens_per_iteration - used, 0)
            while budget > 0:
                groups = self._build_prefill_groups(active)
                if not groups:
                    break
                group = groups[self._select_prefill_group(groups)]
                group_budget = min(self.prefill_chunk_size, max(budget // max(len(group), 1), 0))
                if group_budget <= 0:
                    break
                res = prefill_executor(group, group_budget, now, event_id)
                now += res["batch_runtime_ms"]
                budget -= res["tokens_scheduled"]
                retire(res)
                events.append(self._event(event_id, now, res))
                event_id += 1
                next_idx = self._enqueue_arrivals(requests, next_idx, now, waiting)
                self._admit_waiting(waiting, active)

        completed.sort(key=lambda r: r.request_id)
        return completed, events
