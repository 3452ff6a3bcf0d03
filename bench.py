"""Benchmark of the MI355X paged-attention backend.

One step = one paged-decode attention call (libpaged_hip `pa_decode`) over the large ragged
decode batch: 256 requests, 32 heads x 128, block 16, context lengths log-uniform in
[512, 32768], bf16 KV with fp32 accumulation, pool = 1.1 x the blocks needed, shuffled block
lists; Q, K, V i.i.d. N(0, 1). All inputs are resident in HBM before timing. `value` is the
achieved HBM bandwidth in GB/s: algorithmic bytes per call (K/V rows read, q read and output
written in fp32, page-table entries, two int32 lengths per request) / mean call time, timed with
HIP events on the stream the kernel is launched on.

Also reported on the same line:
  roofline       the decode kernel against MI355X's 8 TB/s HBM peak (and HBM traffic per launch
                 when a counter summary is available under profiles/);
  cpu_baseline   the oracle (C restatement of the reference's paged attention, fp64
                 accumulation) on a bounded sample of the same batch, on this host's cores;
  continuous_batching  the end-to-end run: decoder LM (vocab 5000, d_model 512, 8 heads,
                 6 layers, d_ff 2048, KV block 16, fp32, weights N(0, 0.02)), 200 Poisson requests
                 at 32 req/s, max batch 8, prefill chunk 256, 1536-token iteration budget, greedy;
                 tokens/s and p50 TTFT on the scheduler's virtual clock, plus wall time.
Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-e2e]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import re
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "efficient-inference-system_amd"))
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
METRIC = "paged decode attn HBM GB/s (% peak); continuous-batching tokens/sec, p50 TTFT"


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def pmc_traffic_bytes() -> float | None:
    """HBM bytes per decode launch from the committed counter summary, if present."""
    p = REPO / "profiles" / "decode_large_ragged_pmc.txt"
    if not p.exists():
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text(), re.M)
    return float(m.group(1)) if m else None


def time_decode(batch, steps: int, warmup: int):
    import torch

    from src.kernels.hip_paged_attention import paged_attention_decode_hip

    dev = batch.q.device
    order = torch.tensor(sorted(range(batch.batch), key=lambda i: -batch.seq_lens[i]), dtype=torch.int32, device=dev)
    out = torch.empty_like(batch.q)

    def step():
        paged_attention_decode_hip(batch.q, batch.k_pool, batch.v_pool, batch.page_table, batch.seq_lens_t,
                                   batch.cur_lens_t, order=order, out=out)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    return start.elapsed_time(end) / steps, wall_ms / steps, out


def cpu_baseline(batch, target_s: float = 6.0) -> dict:
    """Oracle on the first n requests of the batch (n sized for ~target_s per run), median of 3."""
    import torch

    import oracle

    nthreads = cpu_threads()
    lens = batch.seq_lens

    def sample(n):
        ks, vs, lists, pos = [], [], [], 0
        for r in range(n):
            ids = torch.tensor(batch.block_lists[r], device=batch.q.device, dtype=torch.long)
            ks.append(batch.k_pool.index_select(0, ids).cpu())
            vs.append(batch.v_pool.index_select(0, ids).cpu())
            lists.append(list(range(pos, pos + len(ids))))
            pos += len(ids)
        return (batch.q[:n].cpu(), oracle._np(torch.cat(ks)), oracle._np(torch.cat(vs)), lists, lens[:n], [1] * n)

    def run(args):
        t0 = time.perf_counter()
        oracle.paged_attention(*args, nthreads=nthreads)
        return time.perf_counter() - t0

    probe = sample(2)
    rate = sum(lens[:2]) / max(run(probe), 1e-6)  # tokens (x all heads) per second
    n, tokens = 0, 0
    while n < batch.batch and tokens < rate * target_s and n < 64:
        tokens += lens[n]
        n += 1
    args = sample(n)
    times = sorted(run(args) for _ in range(3))
    t = statistics.median(times)
    H, Hd = batch.q.shape[1], batch.q.shape[3]
    nbytes = sum(H * (2 * L * Hd * batch.k_pool.element_size() + 2 * Hd * 4) + 4 * math.ceil(L / 16) + 8 for L in lens[:n])
    return {
        "value": nbytes / t / 1e9,
        "unit": "GB/s",
        "cores": nthreads,
        "kind": "port",
        "sample": f"requests 0..{n - 1} of the same batch ({sum(lens[:n])} tokens x {H} heads x {Hd}, bf16 KV); "
                  f"oracle C restatement, fp64 accumulation, OpenMP over (request, head); median of 3 runs "
                  f"({t:.2f} s each)",
        "seconds_per_run": t,
    }


def init_weights_normal(model, std: float = 0.02) -> None:
    import torch

    with torch.no_grad():
        for mod in model.modules():
            if isinstance(mod, (torch.nn.Linear, torch.nn.Embedding)):
                mod.weight.normal_(0.0, std)
                if getattr(mod, "bias", None) is not None:
                    mod.bias.zero_()
            elif isinstance(mod, torch.nn.LayerNorm):
                mod.weight.fill_(1.0)
                mod.bias.zero_()


def continuous_batching(device) -> dict:
    import torch

    from src.config import benchmark_serving_request_mix
    from src.inference.generate_with_cache import generate_with_cache
    from src.model.transformer import TinyTransformerLM
    from src.serving.continuous_generate import run_decode_step, run_prefill_chunk
    from src.serving.loadgen import generate_requests
    from src.serving.metrics import summarize_run
    from src.serving.scheduler import ContinuousBatchingScheduler

    torch.manual_seed(42)
    model = TinyTransformerLM(vocab_size=5000, d_model=512, num_heads=8, num_layers=6, d_ff=2048, max_seq_len=1024,
                              attention_backend="hip_paged", kv_block_size=16, kv_pool_initial_blocks=64,
                              kv_pool_growth_factor=2.0).to(device).eval()
    init_weights_normal(model)
    # warm-up as the reference harness does: one batched generate, then fresh pools
    generate_with_cache(model, torch.randint(0, 5000, (8, 512), device=device), max_new_tokens=[2] * 8)
    torch.cuda.synchronize()
    model.reset_paged_cache_pools()
    reqs = generate_requests(200, 32.0, 5000, workload_profiles=benchmark_serving_request_mix(), seed=42)
    sched = ContinuousBatchingScheduler(max_batch_size=8, prefill_chunk_size=256, max_tokens_per_iteration=1536)
    dev = str(device)
    t0 = time.perf_counter()
    with torch.no_grad():
        done, events = sched.run(
            reqs,
            prefill_executor=lambda b, c, t, e: run_prefill_chunk(model, b, c, dev, t, e),
            decode_executor=lambda b, t, e: run_decode_step(model, b, dev, t, e),
            release_request_cache=lambda r: model.release_request_caches(r.kv_caches),
        )
    wall = time.perf_counter() - t0
    s = summarize_run(done, events, 32.0, 8, 0.0, "continuous", 256, 0)
    return {
        "tokens_per_s": s["throughput_tokens_per_s"],
        "p50_ttft_ms": s["p50_first_token_latency_ms"],
        "mean_ttft_ms": s["mean_first_token_latency_ms"],
        "p95_ttft_ms": s["p95_first_token_latency_ms"],
        "requests": s["num_requests"],
        "generated_tokens": sum(r.max_new_tokens for r in done),
        "decode_ms_per_token": s["mean_decode_ms_per_token"],
        "events": s["num_batches"],
        "wall_s": wall,
        "clock": "scheduler virtual clock (sum of measured forward times), as the reference",
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    from src import workloads

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    log("building the large ragged decode batch (B=256, 32x128, bf16 KV)")
    batch = workloads.large_decode(seed=0, device=dev)
    nbytes = batch.decode_bytes()
    log(f"pool blocks={batch.k_pool.shape[0]} tokens={sum(batch.seq_lens)} algorithmic bytes/call={nbytes}")
    ms, wall_ms, _ = time_decode(batch, args.steps, args.warmup)
    gbs = nbytes / (ms * 1e-3) / 1e9
    log(f"decode: {ms:.3f} ms/call (events), {wall_ms:.3f} ms/call (wall), {gbs:.1f} GB/s")

    traffic = pmc_traffic_bytes()
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16-kv/f32-acc",
        "data": "synthetic",
        "config": {
            "workload": "large ragged paged decode: 256 requests, 32 heads x 128, block 16, lengths log-uniform "
                        "[512, 32768], bf16 KV, fp32 q/out, pool 1.1x, shuffled block tables",
            "batch": batch.batch,
            "tokens": sum(batch.seq_lens),
            "bytes_per_step": nbytes,
        },
        "pct_peak_hbm": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {
            "bound": "hbm",
            "achieved": round(gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
    }
    if not args.no_cpu_baseline:
        log("CPU baseline (oracle on a sample of the batch)")
        result["cpu_baseline"] = cpu_baseline(batch)
    del batch
    torch.cuda.empty_cache()
    if not args.no_e2e:
        log("end-to-end continuous batching (200 requests, 32 req/s)")
        result["continuous_batching"] = continuous_batching(dev)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
