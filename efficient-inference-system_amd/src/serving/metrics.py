"""Run summaries (src/serving/metrics.py of the reference) plus p50 first-token latency.

percentile() is linear interpolation between order statistics (metrics.py:4-16): rank =
(n - 1) * p / 100. summarize_run() keeps every key of the reference (throughput_tokens_per_s =
sum of max_new_tokens / makespan, makespan = last finish - first arrival) and adds
p50_first_token_latency_ms, which the reference does not compute.
"""
from src.utils.metrics import mean


def percentile(values: list[float], p: float) -> float:
    if not values:
        return 0.0
    values = sorted(values)
    if len(values) == 1:
        return values[0]
    rank = (len(values) - 1) * (p / 100.0)
    lower = int(rank)
    upper = min(lower + 1, len(values) - 1)
    weight = rank - lower
    return values[lower] * (1.0 - weight) + values[upper] * weight


def summarize_run(
    completed_requests: list,
    batch_records: list[dict],
    arrival_rate_rps: float,
    max_batch_size: int,
    batch_timeout_ms: float,
    scheduler_mode: str,
    scheduling_policy_value: float,
    run_idx: int,
) -> dict:
    latencies = [r.latency_ms for r in completed_requests]
    waits = [r.wait_time_ms for r in completed_requests]
    services = [r.service_time_ms for r in completed_requests]
    ttfts = [r.first_token_latency_ms for r in completed_requests if r.first_token_time_ms is not None]
    prompt_lengths = [r.prompt_len for r in completed_requests]
    decode_lengths = [r.max_new_tokens for r in completed_requests]
    if completed_requests:
        makespan_ms = max(r.finish_time_ms for r in completed_requests) - min(r.arrival_time_ms for r in completed_requests)
    else:
        makespan_ms = 0.0
    total_generated_tokens = sum(decode_lengths)
    num_completed = len(completed_requests)
    throughput_rps = num_completed / (makespan_ms / 1000.0) if makespan_ms > 0 else 0.0
    throughput_tokens_per_s = total_generated_tokens / (makespan_ms / 1000.0) if makespan_ms > 0 else 0.0

    def col(key, default=0):
        return [b.get(key, default) for b in batch_records]

    realized_batch_sizes = [b["batch_size"] for b in batch_records]
    batch_runtimes = [b["batch_runtime_ms"] for b in batch_records]
    live_kv = col("live_kv_bytes")
    reserved_kv = col("reserved_kv_bytes")
    frag = col("fragmentation_bytes")
    workspace = col("workspace_bytes")
    gpu_alloc = col("gpu_allocated_bytes")
    gpu_peak = col("gpu_peak_allocated_bytes")
    prefill_runtime_total = sum(col("prefill_runtime_ms", 0.0))
    decode_runtime_total = sum(col("decode_runtime_ms", 0.0))
    decode_kernel_tokens_total = sum(col("decode_kernel_tokens"))
    total_runtime_ms = sum(batch_runtimes)
    return {
        "run_idx": run_idx,
        "scheduler_mode": scheduler_mode,
        "scheduling_policy_value": scheduling_policy_value,
        "arrival_rate_rps": arrival_rate_rps,
        "max_batch_size": max_batch_size,
        "batch_timeout_ms": batch_timeout_ms,
        "num_requests": num_completed,
        "num_batches": len(batch_records),
        "throughput_rps": throughput_rps,
        "throughput_tokens_per_s": throughput_tokens_per_s,
        "mean_event_tokens_per_s": mean(col("tokens_per_s", 0.0)),
        "mean_latency_ms": mean(latencies),
        "p50_latency_ms": percentile(latencies, 50),
        "p95_latency_ms": percentile(latencies, 95),
        "p99_latency_ms": percentile(latencies, 99),
        "mean_wait_ms": mean(waits),
        "p95_wait_ms": percentile(waits, 95),
        "mean_service_ms": mean(services),
        "mean_first_token_latency_ms": mean(ttfts),
        "p50_first_token_latency_ms": percentile(ttfts, 50),
        "p95_first_token_latency_ms": percentile(ttfts, 95),
        "mean_prompt_len": mean(prompt_lengths),
        "min_prompt_len": min(prompt_lengths) if prompt_lengths else 0,
        "max_prompt_len": max(prompt_lengths) if prompt_lengths else 0,
        "mean_max_new_tokens": mean(decode_lengths),
        "min_max_new_tokens": min(decode_lengths) if decode_lengths else 0,
        "max_max_new_tokens": max(decode_lengths) if decode_lengths else 0,
        "mean_batch_size": mean(realized_batch_sizes),
        "max_batch_size_realized": max(realized_batch_sizes) if realized_batch_sizes else 0,
        "mean_batch_runtime_ms": mean(batch_runtimes),
        "mean_tokens_scheduled": mean(col("tokens_scheduled")),
        "mean_active_requests": mean(col("active_requests")),
        "mean_decode_ms_per_token": decode_runtime_total / decode_kernel_tokens_total if decode_kernel_tokens_total > 0 else 0.0,
        "prefill_runtime_ms_total": prefill_runtime_total,
        "decode_runtime_ms_total": decode_runtime_total,
        "prefill_runtime_share": prefill_runtime_total / total_runtime_ms if total_runtime_ms > 0 else 0.0,
        "decode_runtime_share": decode_runtime_total / total_runtime_ms if total_runtime_ms > 0 else 0.0,
        "mean_padding_waste_tokens": mean(col("padding_waste_tokens")),
        "total_padding_waste_tokens": sum(col("padding_waste_tokens")),
        "mean_padding_waste_bytes_est": mean(col("padding_waste_bytes_est")),
        "total_padding_waste_bytes_est": sum(col("padding_waste_bytes_est")),
        "mean_padding_waste_pct": mean(col("padding_waste_pct", 0.0)),
        "mean_live_kv_bytes": mean(live_kv),
        "max_live_kv_bytes": max(live_kv) if live_kv else 0,
        "mean_reserved_kv_bytes": mean(reserved_kv),
        "max_reserved_kv_bytes": max(reserved_kv) if reserved_kv else 0,
        "mean_fragmentation_bytes": mean(frag),
        "max_fragmentation_bytes": max(frag) if frag else 0,
        "mean_workspace_bytes": mean(workspace),
        "max_workspace_bytes": max(workspace) if workspace else 0,
        "mean_gpu_allocated_bytes": mean(gpu_alloc),
        "max_gpu_allocated_bytes": max(gpu_alloc) if gpu_alloc else 0,
        "max_gpu_peak_allocated_bytes": max(gpu_peak) if gpu_peak else 0,
        "prefill_tokens_total": sum(col("prefill_tokens")),
        "decode_tokens_total": sum(col("decode_tokens")),
        "decode_kernel_tokens_total": decode_kernel_tokens_total,
        "backend_name": batch_records[0].get("backend_name", "hip_paged") if batch_records else "hip_paged",
    }


def requests_to_rows(completed_requests, arrival_rate_rps, max_batch_size, batch_timeout_ms, scheduler_mode,
                     scheduling_policy_value, run_idx) -> list[dict]:
    common = {
        "run_idx": run_idx,
        "scheduler_mode": scheduler_mode,
        "scheduling_policy_value": scheduling_policy_value,
        "arrival_rate_rps": arrival_rate_rps,
        "max_batch_size": max_batch_size,
        "batch_timeout_ms": batch_timeout_ms,
    }
    return [
        {
            **common,
            "request_id": r.request_id,
            "batch_id": r.batch_id,
            "workload_name": r.workload_name,
            "prompt_len": r.prompt_len,
            "max_new_tokens": r.max_new_tokens,
            "arrival_time_ms": r.arrival_time_ms,
            "start_time_ms": r.start_time_ms,
            "finish_time_ms": r.finish_time_ms,
            "first_token_time_ms": r.first_token_time_ms,
            "first_token_latency_ms": r.first_token_latency_ms,
            "wait_time_ms": r.wait_time_ms,
            "service_time_ms": r.service_time_ms,
            "latency_ms": r.latency_ms,
        }
        for r in completed_requests
    ]


def batches_to_rows(batch_records, arrival_rate_rps, max_batch_size, batch_timeout_ms, scheduler_mode,
                    scheduling_policy_value, run_idx) -> list[dict]:
    common = {
        "run_idx": run_idx,
        "scheduler_mode": scheduler_mode,
        "scheduling_policy_value": scheduling_policy_value,
        "arrival_rate_rps": arrival_rate_rps,
        "max_batch_size": max_batch_size,
        "batch_timeout_ms": batch_timeout_ms,
    }
    return [{**common, **record} for record in batch_records]
