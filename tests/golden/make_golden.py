"""Write the golden fixtures under tests/golden/ by running the reference (jacobzhang22/
efficient-inference-system, mounted at /root/reference) in this container.

Only functions that no closed form or invariant pins are recorded here:
  loadgen_trace.json   src/serving/loadgen.py:14-85 — the exact Poisson trace for a seed depends
                       on the order of the random.Random and torch.Generator draws;
  scheduler_events.json src/serving/scheduler.py:254-465 with tests/golden/fake_executors.py —
                       the continuous scheduler's event sequence, request timings and
                       summarize_run (src/serving/metrics.py:19-133) of that run;
  model_logits.json    src/model/transformer.py + src/model/attention.py through
                       src/inference/generate_with_cache.py on the CPU ("paged_reference"):
                       logits and greedy tokens of a small model with formula-set weights;
  executor_run.json    the real continuous-batching executors (src/serving/continuous_generate.py:
                       82-276) driven by ContinuousBatchingScheduler over a short trace on a small
                       model on the CPU, with the executors' timer replaced by a fixed 1 ms per
                       call so the event sequence does not depend on the machine: every event,
                       every request's generated tokens and timings, the release order and the
                       pools' final free lists.
Run from any directory: python tests/golden/make_golden.py. The reference must not be on the
path of anything else; this script imports it as the package `src`.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
sys.path.insert(0, "/root/reference")
sys.path.insert(0, str(HERE))

import torch  # noqa: E402

from fake_executors import EVENT_FIELDS, REQUEST_FIELDS, make_executors  # noqa: E402
from src.config import RequestWorkloadProfile, default_serving_request_mix  # noqa: E402
from src.inference.generate_with_cache import generate_with_cache  # noqa: E402
from src.model.transformer import TinyTransformerLM  # noqa: E402
from src.serving.loadgen import generate_requests  # noqa: E402
from src.serving.metrics import summarize_run  # noqa: E402
from src.serving.scheduler import ContinuousBatchingScheduler  # noqa: E402

BENCH_MIX = [  # the end-to-end benchmark's mix (differs from default_serving_request_mix)
    ("short_qa", 16, 64, 16, 64, 0.4),
    ("chat_turn", 64, 256, 32, 128, 0.3),
    ("rag_answer", 256, 640, 64, 128, 0.2),
    ("long_summary", 512, 896, 96, 128, 0.1),
]


def trace_record(reqs) -> list[dict]:
    return [
        {
            "request_id": r.request_id, "arrival_time_ms": r.arrival_time_ms, "prompt_len": r.prompt_len,
            "max_new_tokens": r.max_new_tokens, "workload_name": r.workload_name,
            "prompt_head": r.prompt_ids[:4].tolist(), "prompt_tail": r.prompt_ids[-4:].tolist(),
            "prompt_sum": int(r.prompt_ids.sum()),
        }
        for r in reqs
    ]


def loadgen_fixture() -> dict:
    bench = [RequestWorkloadProfile(*p) for p in BENCH_MIX]
    return {
        "bench_mix_200_at_32rps_seed42": trace_record(generate_requests(200, 32.0, 5000, workload_profiles=bench, seed=42)),
        "default_mix_30_at_8rps_seed7": trace_record(
            generate_requests(30, 8.0, 5000, workload_profiles=default_serving_request_mix(), seed=7)),
        "fixed_10_at_4rps_seed3": trace_record(generate_requests(10, 4.0, 128, prompt_len=24, max_new_tokens=5, seed=3)),
    }


def request_record(r) -> dict:
    rec = {k: getattr(r, k) for k in REQUEST_FIELDS}
    rec["generated_count"] = len(r.generated_token_ids)
    rec["generated_sum"] = sum(r.generated_token_ids)
    return rec


def scheduler_fixture() -> dict:
    out = {}
    for name, n, rate, seed, max_batch, chunk, budget in (
        ("bench_mix_24_at_32rps", 24, 32.0, 42, 8, 256, 1536),
        ("bench_mix_16_at_200rps_tight", 16, 200.0, 5, 4, 64, 200),
    ):
        bench = [RequestWorkloadProfile(*p) for p in BENCH_MIX]
        reqs = generate_requests(n, rate, 5000, workload_profiles=bench, seed=seed)
        prefill, decode = make_executors()
        released = []
        sched = ContinuousBatchingScheduler(max_batch_size=max_batch, prefill_chunk_size=chunk,
                                            max_tokens_per_iteration=budget)
        done, events = sched.run(reqs, prefill, decode, release_request_cache=lambda r: released.append(r.request_id))
        summary = summarize_run(done, events, rate, max_batch, 0.0, "continuous", chunk, 0)
        out[name] = {
            "args": {"n": n, "rate": rate, "seed": seed, "max_batch": max_batch, "chunk": chunk, "budget": budget},
            "event_fields": list(EVENT_FIELDS),
            "events": [[e[k] for k in EVENT_FIELDS] for e in events],
            "requests": [request_record(r) for r in done],
            "released_order": released,
            "summary": {k: v for k, v in summary.items() if isinstance(v, (int, float, str))},
        }
    return out


def set_weights(model, seed: int = 1234, scale: float = 0.2) -> None:
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name in sorted(model.state_dict()):
            p = model.state_dict()[name]
            p.copy_(torch.randn(p.shape, generator=g) * scale)


def model_fixture() -> dict:
    model = TinyTransformerLM(vocab_size=128, d_model=64, num_heads=4, num_layers=2, d_ff=128, max_seq_len=128,
                              attention_backend="paged_reference", kv_block_size=8, kv_pool_initial_blocks=8,
                              kv_pool_growth_factor=2.0).eval()
    set_weights(model)
    prompt = torch.randint(0, 128, (2, 24), generator=torch.Generator().manual_seed(5))
    lens = torch.tensor([24, 17])
    gen = generate_with_cache(model, prompt, max_new_tokens=[3, 5], prompt_lengths=lens)
    model.reset_paged_cache_pools()
    with torch.no_grad():
        logits, caches = model(prompt, use_cache=True, position_offset=0, current_lengths=lens)
        prefill_last = logits[torch.arange(2), lens - 1]
        step_tokens = torch.tensor([[3], [9]])
        logits2, caches = model(step_tokens, kv_caches=caches, use_cache=True, position_offset=lens, current_lengths=1)
        decode_logits = logits2[:, -1]
        padded_rows = logits[1, 17:24]  # rows past request 1's length (reference padded-row semantics)
    model.reset_paged_cache_pools()
    with torch.no_grad():  # two-chunk prefill: 10 tokens, then the rest
        c1, caches = model(prompt[:, :10], use_cache=True, position_offset=0, current_lengths=torch.tensor([10, 10]))
        c2, caches = model(prompt[:, 10:], kv_caches=caches, use_cache=True, position_offset=10,
                           current_lengths=torch.tensor([14, 7]))
        chunked_last = c2[torch.arange(2), torch.tensor([13, 6])]
    return {
        "config": {"vocab": 128, "d_model": 64, "heads": 4, "layers": 2, "d_ff": 128, "max_seq": 128, "block": 8,
                   "initial_blocks": 8, "weight_seed": 1234, "weight_scale": 0.2, "prompt_seed": 5},
        "prompt": prompt.tolist(), "prompt_lengths": lens.tolist(), "max_new_tokens": [3, 5],
        "generated_ids": [g.tolist() for g in gen["generated_ids"]],
        "generated_tokens_per_request": gen["generated_tokens_per_request"],
        "reserved_kv_bytes": gen["reserved_kv_bytes"], "live_kv_bytes": gen["live_kv_bytes"],
        "prefill_last_logits": prefill_last.tolist(), "decode_step_tokens": [3, 9],
        "decode_step_logits": decode_logits.tolist(), "padded_row_logits": padded_rows.tolist(),
        "chunked_prefill_last_logits": chunked_last.tolist(),
    }


EXECUTOR_MIX = [  # small prompts and decodes so chunks, groups and pool growth all occur
    ("short", 5, 20, 2, 6, 0.5),
    ("mid", 21, 45, 3, 9, 0.35),
    ("long", 46, 70, 4, 8, 0.15),
]


class _FixedTimer:
    """Stand-in for timed_section: every timed call takes exactly 1 ms."""

    def __init__(self, *args, **kwargs):
        self.elapsed_ms = 1.0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.elapsed_ms = 1.0
        return False


def executor_fixture() -> dict:
    import src.serving.continuous_generate as cg

    cg.timed_section = _FixedTimer
    model = TinyTransformerLM(vocab_size=128, d_model=64, num_heads=4, num_layers=2, d_ff=128, max_seq_len=128,
                              attention_backend="paged_reference", kv_block_size=8, kv_pool_initial_blocks=8,
                              kv_pool_growth_factor=2.0).eval()
    set_weights(model)
    mix = [RequestWorkloadProfile(*p) for p in EXECUTOR_MIX]
    reqs = generate_requests(14, 400.0, 128, workload_profiles=mix, seed=11)
    sched = ContinuousBatchingScheduler(max_batch_size=4, prefill_chunk_size=16, max_tokens_per_iteration=40)
    released = []

    def release(r):
        released.append(r.request_id)
        model.release_request_caches(r.kv_caches)

    with torch.no_grad():
        done, events = sched.run(
            reqs,
            prefill_executor=lambda b, c, t, e: cg.run_prefill_chunk(model, b, c, "cpu", t, e),
            decode_executor=lambda b, t, e: cg.run_decode_step(model, b, "cpu", t, e),
            release_request_cache=release)
    fields = ["batch_id", "dispatch_time_ms", "finish_time_ms", "batch_size", "phase", "tokens_scheduled",
              "prompt_len", "max_new_tokens", "prefill_tokens", "decode_tokens", "decode_kernel_tokens",
              "live_kv_bytes", "reserved_kv_bytes", "fragmentation_bytes", "padding_waste_tokens",
              "padding_waste_bytes_est", "padding_waste_pct", "prefill_runtime_ms", "decode_runtime_ms",
              "decode_ms_per_token"]
    return {
        "config": {"vocab": 128, "d_model": 64, "heads": 4, "layers": 2, "d_ff": 128, "max_seq": 128, "block": 8,
                   "initial_blocks": 8, "weight_seed": 1234, "weight_scale": 0.2, "mix": EXECUTOR_MIX,
                   "requests": 14, "rate": 400.0, "seed": 11, "max_batch": 4, "chunk": 16, "budget": 40},
        "event_fields": fields,
        "events": [[e[k] for k in fields] for e in events],
        "requests": [{"request_id": r.request_id, "generated_token_ids": list(r.generated_token_ids),
                      "start_time_ms": r.start_time_ms, "first_token_time_ms": r.first_token_time_ms,
                      "finish_time_ms": r.finish_time_ms, "batch_id": r.batch_id} for r in done],
        "released_order": released,
        "free_lists": [list(p.free_block_ids) for p in model.layer_block_pools],
        "capacity_blocks": [p.capacity_blocks for p in model.layer_block_pools],
    }


def main() -> None:
    torch.set_num_threads(1)
    for name, fn in (("loadgen_trace.json", loadgen_fixture), ("scheduler_events.json", scheduler_fixture),
                     ("model_logits.json", model_fixture), ("executor_run.json", executor_fixture)):
        data = fn()
        (HERE / name).write_text(json.dumps(data, indent=None, separators=(",", ":")) + "\n")
        print(f"wrote {name} ({(HERE / name).stat().st_size} bytes)")


if __name__ == "__main__":
    main()
