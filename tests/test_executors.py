"""The continuous-batching executors (run_prefill_chunk / run_decode_step) driven by the scheduler,
against the reference's own executors: tests/golden/executor_run.json was recorded by running the
reference's src/serving/continuous_generate.py:82-276 with its scheduler on a small model over a
short trace (tests/golden/make_golden.py), with the executors' timer fixed at 1 ms per call so the
event sequence does not depend on the machine.

Checked: every event's phase, batch size, token counts, KV accounting and times; each request's
generated token ids and timings; the release order; the pools' final free lists and capacities.
On the CPU through the "paged_reference" backend, and on the GPU through "hip_paged" (captured
graphs with the on-device argmax, and the eager path)."""
import json
from pathlib import Path

import pytest
import torch

import src.serving.continuous_generate as cg
from src.config import RequestWorkloadProfile
from src.model.transformer import TinyTransformerLM
from src.serving.loadgen import generate_requests
from src.serving.scheduler import ContinuousBatchingScheduler

GOLDEN = json.loads((Path(__file__).resolve().parent / "golden" / "executor_run.json").read_text())


class FixedTimer:
    def __init__(self, *args, **kwargs):
        self.elapsed_ms = 1.0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.elapsed_ms = 1.0
        return False


def set_weights(model, seed=1234, scale=0.2):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name in sorted(model.state_dict()):
            p = model.state_dict()[name]
            p.copy_(torch.randn(p.shape, generator=g) * scale)


def run_trace(backend, device, monkeypatch):
    monkeypatch.setattr(cg, "timed_section", FixedTimer)
    c = GOLDEN["config"]
    model = TinyTransformerLM(vocab_size=c["vocab"], d_model=c["d_model"], num_heads=c["heads"],
                              num_layers=c["layers"], d_ff=c["d_ff"], max_seq_len=c["max_seq"],
                              attention_backend=backend, kv_block_size=c["block"],
                              kv_pool_initial_blocks=c["initial_blocks"], kv_pool_growth_factor=2.0).eval()
    set_weights(model, c["weight_seed"], c["weight_scale"])
    model = model.to(device)
    mix = [RequestWorkloadProfile(*p) for p in c["mix"]]
    reqs = generate_requests(c["requests"], c["rate"], c["vocab"], workload_profiles=mix, seed=c["seed"])
    sched = ContinuousBatchingScheduler(max_batch_size=c["max_batch"], prefill_chunk_size=c["chunk"],
                                        max_tokens_per_iteration=c["budget"])
    released = []

    def release(r):
        released.append(r.request_id)
        model.release_request_caches(r.kv_caches)

    dev = str(device)
    done, events = sched.run(
        reqs,
        prefill_executor=lambda b, ch, t, e: cg.run_prefill_chunk(model, b, ch, dev, t, e),
        decode_executor=lambda b, t, e: cg.run_decode_step(model, b, dev, t, e),
        release_request_cache=release)
    return model, done, events, released


def check_against_golden(model, done, events, released):
    fields = GOLDEN["event_fields"]
    assert len(events) == len(GOLDEN["events"])
    for i, (ev, want) in enumerate(zip(events, GOLDEN["events"])):
        for k, w in zip(fields, want):
            if isinstance(w, float):
                assert ev[k] == pytest.approx(w, abs=1e-9), (i, k)
            else:
                assert ev[k] == w, (i, k, ev[k], w)
    assert [r.request_id for r in done] == [r["request_id"] for r in GOLDEN["requests"]]
    for r, want in zip(done, GOLDEN["requests"]):
        assert r.generated_token_ids == want["generated_token_ids"], r.request_id
        for k in ("start_time_ms", "first_token_time_ms", "finish_time_ms"):
            assert getattr(r, k) == pytest.approx(want[k], abs=1e-9), (r.request_id, k)
        assert r.batch_id == want["batch_id"]
        assert r.phase == "finished"
    assert released == GOLDEN["released_order"]
    assert [list(p.free_block_ids) for p in model.layer_block_pools] == GOLDEN["free_lists"]
    assert [p.capacity_blocks for p in model.layer_block_pools] == GOLDEN["capacity_blocks"]


def test_executors_match_reference_run_cpu(monkeypatch):
    check_against_golden(*run_trace("paged_reference", torch.device("cpu"), monkeypatch))


def test_executor_plans():
    from src.serving.request import InferenceRequest

    reqs = [InferenceRequest(i, 0.0, n, 3, torch.arange(100, 100 + n)) for i, n in enumerate((5, 12, 9))]
    plan = cg.plan_prefill(reqs, 8)
    assert plan.lengths == [5, 8, 8] and plan.rows == [4, 7, 7] and plan.positions == 0
    assert plan.token_ids.tolist()[0] == [100, 101, 102, 103, 104, 0, 0, 0]
    for r, n in zip(reqs, plan.lengths):
        r.prompt_tokens_processed = n
    with pytest.raises(ValueError, match="same prompt progress"):
        cg.plan_prefill(reqs, 8)
    reqs[0].generated_token_ids = [7]
    reqs[0].prompt_tokens_processed = 5
    d = cg.plan_decode(reqs[:1])
    assert d.token_ids.tolist() == [[7]] and d.positions == [5] and d.lengths == [1] and d.rows == [0]
    assert cg.run_decode_step(None, [], "cpu", 0.0, 0) == {"batch_runtime_ms": 0.0, "requests_completed": []}


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_executors_match_reference_run_hip(device, monkeypatch, graphs):
    monkeypatch.setenv("PAGED_HIP_GRAPHS", graphs)
    print(f"executor trace on hip_paged, graphs={graphs}", flush=True)
    model, done, events, released = run_trace("hip_paged", device, monkeypatch)
    check_against_golden(model, done, events, released)
    if graphs == "1":
        assert model._graph_step is not None and model._graph_step.captures > 0
