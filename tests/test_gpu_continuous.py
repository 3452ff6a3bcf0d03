"""End-to-end continuous batching on the benchmark model and trace, on the GPU.

Model: vocab 5000, d_model 512, 8 heads, 6 layers, d_ff 2048, max_seq_len 1024, KV block 16,
weights N(0, 0.02), biases 0, LayerNorms (1, 0). Trace: all 200 requests of the Poisson trace at
32 req/s (seed 42, the benchmark mix). Scheduler: max batch 8, chunk 256,
1536-token budget. The hip_paged model runs the real executors with its captured graphs (bucketed
chunks, on-device argmax, pool growth), with the executors' timer fixed at 3 ms per call so that
the scheduler's decisions do not depend on the box's speed.

Every step is replayed, in lockstep and teacher-forced (the same token ids, positions and
lengths), on a copy of the model on the "paged_reference" backend with its own caches:
  - logits of every row of every step within 1e-4;
  - each request's per-layer block lists and every pool's free list identical after every step
    and every release;
  - each greedy token equal to the argmax of the reference's logits row (unless that row's top
    two logits are within 2e-4, where fp32 rounding may legitimately pick either).
A second scheduler run of the reference model through the same executors must then produce the
same event sequence (phases, batch sizes, token counts, KV accounting) and the same tokens, except
for requests whose tokens the lockstep run found at a near-tie.
"""
import copy

import pytest
import torch

import src.serving.continuous_generate as cg
from src.cache.paged_kv import BatchedPagedKVCache
from src.config import benchmark_serving_request_mix
from src.model.transformer import TinyTransformerLM
from src.serving.loadgen import generate_requests
from src.serving.scheduler import ContinuousBatchingScheduler

pytestmark = pytest.mark.gpu

N_REQUESTS = 200
TIE = 2e-4


class StepTimer:
    """Deterministic executor timer: 3 ms per call, so the virtual clock admits arrivals the same
    way on every box, and slowly enough that requests overlap (batches of up to 8 requests and
    mixed prefill groups; at the GPU's real step times of ~0.2 ms this arrival rate leaves most
    requests alone in the batch)."""

    def __init__(self, *args, **kwargs):
        self.elapsed_ms = 3.0

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def benchmark_model(backend, device):
    torch.manual_seed(42)
    m = TinyTransformerLM(vocab_size=5000, d_model=512, num_heads=8, num_layers=6, d_ff=2048, max_seq_len=1024,
                          attention_backend=backend, kv_block_size=16, kv_pool_initial_blocks=64,
                          kv_pool_growth_factor=2.0)
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, (torch.nn.Linear, torch.nn.Embedding)):
                mod.weight.normal_(0.0, 0.02)
                if getattr(mod, "bias", None) is not None:
                    mod.bias.zero_()
            elif isinstance(mod, torch.nn.LayerNorm):
                mod.weight.fill_(1.0)
                mod.bias.zero_()
    return m.to(device).eval()


def trace():
    reqs = generate_requests(200, 32.0, 5000, workload_profiles=benchmark_serving_request_mix(), seed=42)
    return sorted(reqs, key=lambda r: r.arrival_time_ms)[:N_REQUESTS]


def run(model, device, observer=None, on_release=None, keep_logits=False):
    sched = ContinuousBatchingScheduler(max_batch_size=8, prefill_chunk_size=256, max_tokens_per_iteration=1536)
    ex = cg.StepExecutor(model, str(device), keep_logits=keep_logits, observer=observer)

    def release(r):
        if on_release is not None:
            on_release(r)
        model.release_request_caches(r.kv_caches)

    with torch.no_grad():
        done, events = sched.run(
            trace(),
            prefill_executor=lambda b, c, t, e: cg.run_prefill_chunk(model, b, c, str(device), t, e, executor=ex),
            decode_executor=lambda b, t, e: cg.run_decode_step(model, b, str(device), t, e, executor=ex),
            release_request_cache=release)
    return done, events


EVENT_KEYS = ("phase", "batch_size", "tokens_scheduled", "prefill_tokens", "decode_tokens", "decode_kernel_tokens",
              "prompt_len", "max_new_tokens", "live_kv_bytes", "reserved_kv_bytes", "fragmentation_bytes",
              "padding_waste_tokens", "dispatch_time_ms", "finish_time_ms")


@pytest.mark.timeout(900)
def test_continuous_batching_benchmark_model_lockstep(device, monkeypatch):
    monkeypatch.setattr(cg, "timed_section", StepTimer)
    hip = benchmark_model("hip_paged", device)
    ref = benchmark_model("paged_reference", device)
    ref.load_state_dict(copy.deepcopy(hip.state_dict()))
    captured = hip.prepare_graphs(8, device, want_logits=True)
    print(f"C4 lockstep: {N_REQUESTS} requests, {captured} graphs captured ahead", flush=True)

    ref_states: dict[int, list] = {}
    stats = {"steps": 0, "max_err": 0.0, "prefill_steps": 0, "near_ties": set(), "tokens": 0, "near_tie_tokens": 0,
             "near_tie_flips": 0}

    def ref_pools():
        return ref._ensure_layer_block_pools()

    def compare_pools():
        for lh, lr in zip(hip.layer_block_pools, ref.layer_block_pools):
            assert lh.free_block_ids == lr.free_block_ids
            assert lh.capacity_blocks == lr.capacity_blocks

    def observe(plan, tokens, logits, event):
        ids = [r.request_id for r in plan.requests]
        for rid in ids:
            if rid not in ref_states:
                ref_states[rid] = ref.create_request_kv_caches(1)[0]
        pools = ref_pools()
        caches = [BatchedPagedKVCache([ref_states[rid][l] for rid in ids], pools[l]) for l in range(len(pools))]
        pos = plan.positions if isinstance(plan.positions, int) else torch.tensor(plan.positions, device=device)
        with torch.no_grad():
            want, _ = ref(torch.from_numpy(plan.token_ids).to(device), kv_caches=caches, use_cache=True,
                          position_offset=pos, current_lengths=torch.tensor(plan.lengths))
        err = (logits - want).abs().max().item()
        stats["max_err"] = max(stats["max_err"], err)
        stats["steps"] += 1
        stats["prefill_steps"] += plan.phase == "prefill"
        assert err <= 1e-4, (stats["steps"], plan.phase, ids, err)
        for b, (req, rid) in enumerate(zip(plan.requests, ids)):
            for l in range(len(pools)):
                assert req.kv_caches[l].block_ids == ref_states[rid][l].block_ids, (rid, l)
                assert req.kv_caches[l].seq_len == ref_states[rid][l].seq_len, (rid, l)
            row = want[b, plan.rows[b]]
            top2 = torch.topk(row, 2).values
            if (top2[0] - top2[1]).item() < TIE:
                stats["near_ties"].add(rid)
                stats["near_tie_tokens"] += 1
                stats["near_tie_flips"] += int(tokens[b]) != int(torch.argmax(row))
            else:
                assert tokens[b] == int(torch.argmax(row)), (rid, plan.phase)
            stats["tokens"] += 1
        compare_pools()
        if stats["steps"] % 500 == 0:
            print(f"  step {stats['steps']}: {stats['tokens']} tokens checked, max logits err {stats['max_err']:.2e}",
                  flush=True)

    def on_release(r):
        ref.release_request_caches(ref_states.pop(r.request_id))

    done, events = run(hip, device, observer=observe, on_release=on_release, keep_logits=True)
    compare_pools()
    print(f"C4 lockstep: {stats['steps']} steps ({stats['prefill_steps']} prefill), {stats['tokens']} tokens "
          f"checked, max logits err {stats['max_err']:.2e}, {stats['near_tie_tokens']} near-tie tokens "
          f"({stats['near_tie_flips']} of them not the reference's argmax) in requests {sorted(stats['near_ties'])}, "
          f"pool capacity {hip.layer_block_pools[0].capacity_blocks} blocks, "
          f"graph captures {hip._graph_step.captures}", flush=True)
    assert len(done) == N_REQUESTS and all(r.num_generated_tokens == r.max_new_tokens for r in done)
    assert stats["prefill_steps"] > 0 and stats["steps"] > stats["prefill_steps"]
    assert hip.layer_block_pools[0].capacity_blocks > 64  # the pools grew during the run
    assert any(e["phase"] == "prefill" and e["batch_size"] > 1 for e in events)

    # the reference model through the same executors: same events, same tokens
    ref.reset_paged_cache_pools()
    ref_done, ref_events = run(ref, device)
    assert len(ref_events) == len(events)
    for i, (a, b) in enumerate(zip(events, ref_events)):
        for k in EVENT_KEYS:
            assert a[k] == b[k], (i, k, a[k], b[k])
    for a, b in zip(done, ref_done):
        assert a.request_id == b.request_id
        if a.request_id not in stats["near_ties"]:
            assert a.generated_token_ids == b.generated_token_ids, a.request_id
