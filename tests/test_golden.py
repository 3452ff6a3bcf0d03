"""This implementation against the golden fixtures written from the reference by
tests/golden/make_golden.py: the Poisson trace, the continuous scheduler's event sequence and
summary under deterministic executors, and a small model's logits and greedy tokens."""
import json
import math
import sys
from pathlib import Path

import pytest
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"
sys.path.insert(0, str(GOLDEN))

from fake_executors import EVENT_FIELDS, REQUEST_FIELDS, make_executors  # noqa: E402
from src.config import RequestWorkloadProfile, benchmark_serving_request_mix, default_serving_request_mix  # noqa: E402
from src.inference.generate_with_cache import generate_with_cache  # noqa: E402
from src.model.transformer import TinyTransformerLM  # noqa: E402
from src.serving.loadgen import generate_requests  # noqa: E402
from src.serving.metrics import percentile, summarize_run  # noqa: E402
from src.serving.scheduler import ContinuousBatchingScheduler  # noqa: E402


def load(name):
    return json.loads((GOLDEN / name).read_text())


def trace_record(reqs):
    return [
        {
            "request_id": r.request_id, "arrival_time_ms": r.arrival_time_ms, "prompt_len": r.prompt_len,
            "max_new_tokens": r.max_new_tokens, "workload_name": r.workload_name,
            "prompt_head": r.prompt_ids[:4].tolist(), "prompt_tail": r.prompt_ids[-4:].tolist(),
            "prompt_sum": int(r.prompt_ids.sum()),
        }
        for r in reqs
    ]


def test_benchmark_mix_matches_the_benchmark_definition():
    mix = benchmark_serving_request_mix()
    assert [(p.name, p.prompt_len_min, p.prompt_len_max, p.max_new_tokens_min, p.max_new_tokens_max, p.weight)
            for p in mix] == [
        ("short_qa", 16, 64, 16, 64, 0.4), ("chat_turn", 64, 256, 32, 128, 0.3),
        ("rag_answer", 256, 640, 64, 128, 0.2), ("long_summary", 512, 896, 96, 128, 0.1)]


def test_loadgen_trace_matches_reference():
    g = load("loadgen_trace.json")
    assert trace_record(generate_requests(200, 32.0, 5000, workload_profiles=benchmark_serving_request_mix(), seed=42)) \
        == g["bench_mix_200_at_32rps_seed42"]
    assert trace_record(generate_requests(30, 8.0, 5000, workload_profiles=default_serving_request_mix(), seed=7)) \
        == g["default_mix_30_at_8rps_seed7"]
    assert trace_record(generate_requests(10, 4.0, 128, prompt_len=24, max_new_tokens=5, seed=3)) \
        == g["fixed_10_at_4rps_seed3"]


@pytest.mark.parametrize("scenario", ["bench_mix_24_at_32rps", "bench_mix_16_at_200rps_tight"])
def test_scheduler_event_sequence_matches_reference(scenario):
    g = load("scheduler_events.json")[scenario]
    a = g["args"]
    reqs = generate_requests(a["n"], a["rate"], 5000, workload_profiles=benchmark_serving_request_mix(), seed=a["seed"])
    prefill, decode = make_executors()
    released = []
    sched = ContinuousBatchingScheduler(max_batch_size=a["max_batch"], prefill_chunk_size=a["chunk"],
                                        max_tokens_per_iteration=a["budget"])
    done, events = sched.run(reqs, prefill, decode, release_request_cache=lambda r: released.append(r.request_id))
    assert g["event_fields"] == list(EVENT_FIELDS)
    assert [[e[k] for k in EVENT_FIELDS] for e in events] == g["events"]
    got_reqs = []
    for r in done:
        rec = {k: getattr(r, k) for k in REQUEST_FIELDS}
        rec["generated_count"] = len(r.generated_token_ids)
        rec["generated_sum"] = sum(r.generated_token_ids)
        got_reqs.append(rec)
    assert got_reqs == g["requests"]
    assert released == g["released_order"]
    summary = summarize_run(done, events, a["rate"], a["max_batch"], 0.0, "continuous", a["chunk"], 0)
    for key, want in g["summary"].items():
        if key == "backend_name":
            continue
        assert summary[key] == pytest.approx(want, rel=1e-12, abs=1e-12), key
    ttft = sorted(r.first_token_latency_ms for r in done)
    assert summary["p50_first_token_latency_ms"] == pytest.approx(percentile(ttft, 50))


def test_percentile_is_linear_interpolation():
    import numpy as np

    rng = np.random.default_rng(0)
    for n in (1, 2, 5, 17, 200):
        xs = rng.normal(size=n).tolist()
        for p in (0, 1, 50, 95, 99, 100):
            assert percentile(xs, p) == pytest.approx(float(np.percentile(xs, p, method="linear")), abs=1e-12)
    assert percentile([], 50) == 0.0


def set_weights(model, seed=1234, scale=0.2):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name in sorted(model.state_dict()):
            p = model.state_dict()[name]
            p.copy_(torch.randn(p.shape, generator=g) * scale)


def golden_model(backend, device):
    m = TinyTransformerLM(vocab_size=128, d_model=64, num_heads=4, num_layers=2, d_ff=128, max_seq_len=128,
                          attention_backend=backend, kv_block_size=8, kv_pool_initial_blocks=8,
                          kv_pool_growth_factor=2.0).eval()
    set_weights(m)
    return m.to(device)


def check_model(backend, device, atol):
    g = load("model_logits.json")
    m = golden_model(backend, device)
    prompt = torch.tensor(g["prompt"], device=device)
    assert prompt.tolist() == torch.randint(0, 128, (2, 24), generator=torch.Generator().manual_seed(5)).tolist()
    lens = torch.tensor(g["prompt_lengths"], device=device)
    gen = generate_with_cache(m, prompt, max_new_tokens=g["max_new_tokens"], prompt_lengths=lens)
    assert [x.tolist() for x in gen["generated_ids"]] == g["generated_ids"]
    assert gen["generated_tokens_per_request"] == g["generated_tokens_per_request"]
    assert gen["reserved_kv_bytes"] == g["reserved_kv_bytes"] and gen["live_kv_bytes"] == g["live_kv_bytes"]
    m.reset_paged_cache_pools()
    with torch.no_grad():
        logits, caches = m(prompt, use_cache=True, position_offset=0, current_lengths=lens)
        got = logits[torch.arange(2, device=device), lens - 1]
        assert (got.cpu() - torch.tensor(g["prefill_last_logits"])).abs().max().item() <= atol
        assert (logits[1, 17:24].cpu() - torch.tensor(g["padded_row_logits"])).abs().max().item() <= atol
        step = torch.tensor([[3], [9]], device=device)
        logits2, caches = m(step, kv_caches=caches, use_cache=True, position_offset=lens, current_lengths=1)
        assert (logits2[:, -1].cpu() - torch.tensor(g["decode_step_logits"])).abs().max().item() <= atol
    m.reset_paged_cache_pools()
    with torch.no_grad():
        c1, caches = m(prompt[:, :10], use_cache=True, position_offset=0,
                       current_lengths=torch.tensor([10, 10], device=device))
        c2, caches = m(prompt[:, 10:], kv_caches=caches, use_cache=True, position_offset=10,
                       current_lengths=torch.tensor([14, 7], device=device))
        got = c2[torch.arange(2, device=device), torch.tensor([13, 6], device=device)]
        assert (got.cpu() - torch.tensor(g["chunked_prefill_last_logits"])).abs().max().item() <= atol


def test_model_logits_and_tokens_match_reference_cpu():
    check_model("paged_reference", torch.device("cpu"), atol=1e-5)


@pytest.mark.gpu
def test_model_logits_and_tokens_match_reference_hip(device):
    check_model("hip_paged", device, atol=1e-4)
