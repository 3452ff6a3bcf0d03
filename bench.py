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
                 when a counter summary is available under profiles/), and against what this box
                 delivers to a plain streaming read and to a copy, measured right after;
  cpu_baseline   the oracle (C restatement of the reference's paged attention, fp64
                 accumulation) over the same batch on this host's cores, plus the rate of the
                 reference's own per-token torch loop on a small slice of it;
  secondary      the single fp32 decode (1 request, 128 tokens), the ragged fp32 decode (8 requests
                 x 6 layers), the chunked prefill (4 requests, fp32 and bf16 KV), the large
                 prefill (8 requests x 32 heads x 128, 512-token chunks over 1-4k contexts, bf16 and
                 fp32 KV) and a mid-size bf16 prefill (4 requests x 32 heads x 128, 256-token
                 chunks, with the 16-row kernel timed beside the default dispatch); MFMA
                 utilisation against the fp32 / bf16 matrix peaks; for the first three
                 also the same-run CPU times of one call (the oracle, and the reference's per-key
                 torch loop, whole or on a scaled sample);
  continuous_batching  the end-to-end run: decoder LM (vocab 5000, d_model 512, 8 heads,
                 6 layers, d_ff 2048, KV block 16, fp32, weights N(0, 0.02)), 200 Poisson requests
                 at 32 req/s, max batch 8, prefill chunk 256, 1536-token iteration budget, greedy;
                 tokens/s and p50 TTFT on the scheduler's virtual clock, plus wall time;
  continuous_batching_bf16_model  the same trace and weights with the model in bf16 (weights,
                 activations and KV; the decode steps through the bf16 fused kernels), GPU only;
  continuous_batching_saturated  the fp32 model on the same request mix with every request
                 arriving at once (the serving path's capacity at max batch 8), GPU only.
Usage: python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-e2e]
                       [--no-secondary] [--no-decode] [--calibrate-copy] [--no-box-calibration]
                       [--e2e-model fp32|bf16|both]
                       [--only GROUP[,GROUP...]]
(--no-decode skips the headline decode measurement and --only restricts the secondary workloads to
the named groups; both are for profiling one workload alone.)
"""
from __future__ import annotations

import argparse
import contextlib
import json
import math
import os
import re
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


def affinity_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads() -> int:
    """Threads for the CPU baselines: every core this process may run on, capped by the host's
    per-process thread allotment when one is set (OMP_NUM_THREADS; a shared GPU host allots each
    one-GPU job a share of its cores and sets it)."""
    n = affinity_cores()
    allot = os.environ.get("OMP_NUM_THREADS", "")
    if allot.isdigit() and int(allot) > 0:
        n = min(n, int(allot))
    return max(1, n)


def cpu_info() -> dict:
    """What the CPU baselines ran on: the CPU model, the cores this process may use, and the
    threads the baselines used."""
    model = "unknown"
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"cpu_model": model, "affinity_cores": affinity_cores(), "threads": cpu_threads(),
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS")}


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


def cpu_baseline(batch, chunk: int = 32) -> dict:
    """The oracle over the whole batch on this host's cores: requests are copied to host memory
    `chunk` at a time and only the oracle's compute is timed (one run per chunk)."""
    import torch

    import oracle

    nthreads = cpu_threads()
    lens = batch.seq_lens
    total_s = 0.0
    for c0 in range(0, batch.batch, chunk):
        rows = range(c0, min(c0 + chunk, batch.batch))
        ids = torch.tensor([i for r in rows for i in batch.block_lists[r]], device=batch.q.device, dtype=torch.long)
        k = oracle._np(batch.k_pool.index_select(0, ids).cpu())
        v = oracle._np(batch.v_pool.index_select(0, ids).cpu())
        lists, pos = [], 0
        for r in rows:
            lists.append(list(range(pos, pos + len(batch.block_lists[r]))))
            pos += len(batch.block_lists[r])
        q = batch.q[c0:c0 + len(rows)].cpu()
        t0 = time.perf_counter()
        oracle.paged_attention(q, k, v, lists, lens[c0:c0 + len(rows)], [1] * len(rows), nthreads=nthreads)
        total_s += time.perf_counter() - t0
        del k, v
    H, Hd = batch.q.shape[1], batch.q.shape[3]
    return {
        "value": batch.decode_bytes() / total_s / 1e9,
        "unit": "GB/s",
        "cores": nthreads,
        "host": cpu_info(),
        "kind": "port",
        "sample": f"the whole batch ({batch.batch} requests, {sum(lens)} tokens x {H} heads x {Hd}, bf16 KV), "
                  f"copied to host {chunk} requests at a time; oracle C restatement of the reference's paged "
                  f"attention, fp64 accumulation, OpenMP over (request, head); compute time {total_s:.2f} s",
        "seconds": total_s,
    }


def reference_loop_rate(batch, requests: int = 8, tokens: int = 2048) -> dict:
    """The reference's own CPU path (its per-key torch loop, restated in oracle/reference_loop.py)
    on the first `requests` requests, each cut to its first `tokens` keys, all heads: seconds per
    (key x head), and the time the whole batch would take at that rate."""
    import torch

    from oracle.reference_loop import paged_attention_loop

    torch.set_num_threads(cpu_threads())
    rows = list(range(min(requests, batch.batch)))
    cut = [min(tokens, batch.seq_lens[r]) for r in rows]
    lists, ids, pos = [], [], 0
    for r, n in zip(rows, cut):
        nblk = (n + 15) // 16
        ids += batch.block_lists[r][:nblk]
        lists.append(list(range(pos, pos + nblk)))
        pos += nblk
    idx = torch.tensor(ids, device=batch.q.device, dtype=torch.long)
    k = batch.k_pool.index_select(0, idx).float().cpu()
    v = batch.v_pool.index_select(0, idx).float().cpu()
    q = batch.q[:len(rows)].cpu()
    t0 = time.perf_counter()
    paged_attention_loop(q, k, v, lists, cut, [1] * len(rows))
    dt = time.perf_counter() - t0
    per = dt / (sum(cut) * q.shape[1])
    whole = per * sum(batch.seq_lens) * q.shape[1]
    return {"seconds_per_key_head": per,
            "sample": f"requests 0..{len(rows) - 1} cut to their first {tokens} keys ({sum(cut)} keys) x "
                      f"{q.shape[1]} heads: {dt:.2f} s",
            "extrapolated_batch_seconds": whole,
            "extrapolated_GBps": batch.decode_bytes() / whole / 1e9, "threads": torch.get_num_threads()}


def _median_s(fn, reps: int = 3) -> float:
    """One untimed call, then the median wall time of `reps` calls (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _attended(seq_lens, cur_lens, T: int) -> int:
    """(query row, key) pairs the reference loop visits per head: row i of request b attends the
    keys t <= L_b - C_b + i, all L_b keys for padded rows."""
    return sum(min(L, L - C + i + 1) for L, C in zip(seq_lens, cur_lens) for i in range(T))


def cpu_call_times(q, k_pool, v_pool, block_lists, seq_lens, cur_lens, loop_request: int | None = None) -> dict:
    """Same-run CPU timings of one attention call on host copies of its inputs: the oracle (C
    restatement, fp64 accumulation, all host threads) and the reference's own per-key torch loop,
    each one untimed call then the median of 3. With `loop_request` set, the loop runs on that
    request's head 0 only and its time is scaled by the ratio of attended (row, key) pairs."""
    import torch

    import oracle
    from oracle.reference_loop import paged_attention_loop

    nthreads = cpu_threads()
    torch.set_num_threads(nthreads)
    q, k_pool, v_pool = q.cpu(), k_pool.cpu(), v_pool.cpu()
    B, H, T, _ = q.shape
    kn, vn = oracle._np(k_pool), oracle._np(v_pool)
    oracle_s = _median_s(lambda: oracle.paged_attention(q, kn, vn, block_lists, seq_lens, cur_lens,
                                                        nthreads=nthreads))
    total_pairs = H * _attended(seq_lens, cur_lens, T)
    if loop_request is None:
        loop_s = _median_s(lambda: paged_attention_loop(q, k_pool, v_pool, block_lists, seq_lens, cur_lens))
        sample = "the whole call"
        scale = 1.0
    else:
        r = loop_request
        qs, ks, vs = q[r:r + 1, :1], k_pool[:, :1], v_pool[:, :1]
        lists, sl, cl = [block_lists[r]], [seq_lens[r]], [cur_lens[r]]
        loop_s = _median_s(lambda: paged_attention_loop(qs, ks, vs, lists, sl, cl))
        part = _attended(sl, cl, T)
        scale = total_pairs / part
        sample = f"request {r}, head 0 ({part} of {total_pairs} row-key pairs), scaled by the pair count"
    return {
        "oracle_ms": round(1e3 * oracle_s, 3),
        "reference_loop_ms": round(1e3 * loop_s * scale, 1),
        "reference_loop_sample": sample,
        "threads": nthreads,
    }


def time_call(fn, steps: int, warmup: int = 2) -> float:
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_cold_prefill(q, k_pool, v_pool, page_table, seq_lens, cur_lens, copies: int, replays: int = 3) -> float:
    """Milliseconds per chunked-prefill call with its KV out of every cache: the call's blocks
    are copied into `copies` disjoint block sets of a larger pool (random contents) and one HIP
    graph runs the call once per set, each with its own page table, so that no set is read again
    before all the others (copies x working set well beyond the 256 MB MALL and the L2s)."""
    import torch

    from src.kernels.hip_paged_attention import paged_attention_prefill_hip

    dev = q.device
    used = sorted(set(int(x) for x in page_table.flatten().tolist() if x >= 0))
    n = len(used)
    lut = torch.full((k_pool.shape[0],), -1, dtype=torch.int64, device=dev)
    lut[torch.tensor(used, device=dev)] = torch.arange(n, device=dev)
    local = torch.where(page_table >= 0, lut[page_table.long().clamp(min=0)], -1)
    big_k = torch.empty((copies * n,) + tuple(k_pool.shape[1:]), dtype=k_pool.dtype, device=dev)
    big_v = torch.empty_like(big_k)
    gen = torch.Generator(device=dev)
    gen.manual_seed(77)
    for t in (big_k, big_v):
        t.copy_(torch.randn(t.shape, generator=gen, device=dev, dtype=torch.float32).to(t.dtype))
    tables = [torch.where(local >= 0, local + c * n, -1).to(torch.int32).contiguous() for c in range(copies)]
    out = torch.empty_like(q)
    fns = [lambda pt=pt: paged_attention_prefill_hip(q, big_k, big_v, pt, seq_lens, cur_lens, out=out)
           for pt in tables]
    ms = time_graph_calls(fns, replays)
    del big_k, big_v
    torch.cuda.empty_cache()
    return ms


def time_graph_calls(fns, replays: int = 5) -> float:
    """Milliseconds per call of one HIP graph that runs the callables in `fns` back to back."""
    import torch

    for fn in fns[:1]:
        fn()  # eager first: workspaces are allocated outside the capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fns[0]()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for fn in fns:
            fn()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (replays * len(fns))


def time_graph_call(fn, calls: int = 20, replays: int = 5) -> float:
    """Milliseconds per call of `fn` replayed from one HIP graph of `calls` back-to-back calls (the
    way the serving loop replays its decode steps): no Python or launch cost per call."""
    import torch

    fn()  # eager first: workspaces are allocated outside the capture
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls):
            fn()
    g.replay()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(replays):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (replays * calls)


SECONDARY = ("single_decode", "ragged_decode", "chunked_prefill", "large_prefill", "mid_prefill",
             "long_prompt_prefill")


def secondary_workloads(device, steps: int, with_cpu: bool = True, only=SECONDARY) -> dict:
    """Single decode, ragged fp32 decode (8 requests x 6 layers), chunked prefill (fp32 and bf16
    KV), large and mid-size prefill (the groups named in `only`); with `with_cpu`, the same-run CPU
    timings of the first three."""
    res = {}
    if "single_decode" in only:
        _single_decode(res, device, steps, with_cpu)
    if "ragged_decode" in only:
        _ragged_decode(res, device, steps, with_cpu)
    if "chunked_prefill" in only:
        _chunked_prefill(res, device, steps, with_cpu)
    if "large_prefill" in only:
        _large_prefill(res, device, steps)
    if "mid_prefill" in only:
        _mid_prefill(res, device, steps)
    if "long_prompt_prefill" in only:
        _long_prompt_prefill(res, device, steps)
    return res


def _single_decode(res, device, steps, with_cpu):
    from src import workloads
    from src.kernels.hip_paged_attention import paged_attention_decode_hip

    b = workloads.single_decode(seed=0, device=device)
    call = lambda: paged_attention_decode_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    ms = time_call(call, steps)
    gms = time_graph_call(call)
    res["single_decode_fp32"] = {
        "workload": "1 request, 8 heads x 64, 128 cached tokens in 8 of 64 shuffled blocks, fp32",
        "us_per_call": round(1e3 * ms, 2), "us_per_call_graph": round(1e3 * gms, 2),
        "bytes_per_call": b.decode_bytes(), "GBps_graph": round(b.decode_bytes() / (gms * 1e-3) / 1e9, 1),
        "note": "us_per_call: eager back-to-back calls through the Python wrapper (host-bound at this size); "
                "us_per_call_graph: the same call replayed from a HIP graph",
    }
    if with_cpu:
        log("CPU timings: single decode")
        res["single_decode_fp32"]["cpu"] = cpu_call_times(b.q, b.k_pool, b.v_pool, b.block_lists, b.seq_lens,
                                                          b.cur_lens)


def _ragged_decode(res, device, steps, with_cpu):
    from src import workloads
    from src.kernels.hip_paged_attention import paged_attention_decode_hip

    per_layer, cpu_layers = [], []
    for layer in range(6):
        b = workloads.ragged_decode(seed=0, layer=layer, device=device)
        call = lambda: paged_attention_decode_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
        ms = time_call(call, steps)
        gms = time_graph_call(call)
        per_layer.append((ms, b.decode_bytes(), gms))
        if with_cpu:
            log(f"CPU timings: ragged decode layer {layer}")
            cpu_layers.append(cpu_call_times(b.q, b.k_pool, b.v_pool, b.block_lists, b.seq_lens, b.cur_lens))
        del b
    ms_tot = sum(m for m, _, _ in per_layer)
    by_tot = sum(x for _, x, _ in per_layer)
    g_tot = sum(g for _, _, g in per_layer)
    res["ragged_decode_fp32_6_layers"] = {
        "workload": "8 requests, 8 heads x 64, lengths U[128,1024], 4096-block pool, fp32, one call per layer",
        "us_per_layer": round(1e3 * ms_tot / 6, 2), "GBps": round(by_tot / (ms_tot * 1e-3) / 1e9, 1),
        "us_per_layer_graph": round(1e3 * g_tot / 6, 2), "GBps_graph": round(by_tot / (g_tot * 1e-3) / 1e9, 1),
        "bytes_per_layer": by_tot // 6,
    }
    if with_cpu:
        res["ragged_decode_fp32_6_layers"]["cpu"] = {
            "oracle_ms_per_layer": round(sum(c["oracle_ms"] for c in cpu_layers) / 6, 3),
            "reference_loop_ms_per_layer": round(sum(c["reference_loop_ms"] for c in cpu_layers) / 6, 1),
            "reference_loop_sample": "every layer's whole call",
            "threads": cpu_layers[0]["threads"],
        }


@contextlib.contextmanager
def _env(var, value):
    """Set an environment variable the library reads at each call for the calls inside the block."""
    prev = os.environ.get(var)
    os.environ[var] = value
    try:
        yield
    finally:
        if prev is None:
            del os.environ[var]
        else:
            os.environ[var] = prev


def _forced_prefill_kernel(name):
    """Force pa_prefill's kernel choice (tile | split | wide) for the calls inside the block."""
    return _env("PAGED_HIP_PREFILL_KERNEL", name)


def _chunked_prefill(res, device, steps, with_cpu):
    import torch

    from src import workloads
    from src.kernels.hip_paged_attention import kv_append_hip, pack_metadata_hip, paged_attention_prefill_hip

    for kv_dtype, tag in ((torch.float32, "fp32"), (torch.bfloat16, "bf16kv")):
        w = workloads.chunked_prefill(seed=0, device=device, kv_dtype=kv_dtype)
        B = len(w["prev_lens"])
        T = w["q"].shape[2]
        lists = w["block_lists"]
        max_pages = max(len(x) for x in lists)
        flat = [i for x in lists for i in x]
        offs = [0]
        for x in lists:
            offs.append(offs[-1] + len(x))
        i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=device)
        pt, s32, _, slots = pack_metadata_hip(i32(flat), i32(offs), i32(w["prev_lens"]), i32(w["chunk_lens"]),
                                              query_len=T, block_size=16, max_pages=max_pages)
        cur = i32(w["chunk_lens"])
        append_ms = time_call(lambda: kv_append_hip(w["k_new"], w["v_new"], w["k_pool"], w["v_pool"], slots), steps)
        attn = lambda: paged_attention_prefill_hip(w["q"], w["k_pool"], w["v_pool"], pt, s32, cur)
        attn_ms = time_call(attn, steps)
        graph_ms = time_graph_call(attn)
        cold_ms = time_cold_prefill(w["q"], w["k_pool"], w["v_pool"], pt, s32, cur, copies=64)
        flops = workloads.prefill_flops(w["prev_lens"], w["chunk_lens"], 8, 64)
        peak = 157.3 if tag == "fp32" else 2500.0
        tfs = flops / (attn_ms * 1e-3) / 1e12
        res[f"chunked_prefill_{tag}"] = {
            "workload": f"4 requests, 8 heads x 64, context {w['prev_lens']} + chunk {w['chunk_lens']}, "
                        f"{'fp32' if tag == 'fp32' else 'bf16'} KV",
            "attention_us": round(1e3 * attn_ms, 2), "append_us": round(1e3 * append_ms, 2),
            "attention_us_graph": round(1e3 * graph_ms, 2), "attention_us_cold": round(1e3 * cold_ms, 2),
            "timing": "attention_us: the same call repeated eagerly through the Python wrapper (its ~12 MB of KV "
                      "stay in L2/MALL, as right after the chunk's append in a serving step); attention_us_graph: "
                      "the same call replayed 20 times from a HIP graph (no launch cost between calls, the way "
                      "serving steps run it); attention_us_cold: the call over 64 disjoint copies of its blocks "
                      "in one graph (~0.4-0.75 GB, beyond the 256 MB MALL)",
            "useful_gflop": round(flops / 1e9, 4), "TFLOPs": round(tfs, 2),
            "TFLOPs_graph": round(flops / (graph_ms * 1e-3) / 1e12, 2),
            "TFLOPs_cold": round(flops / (cold_ms * 1e-3) / 1e12, 2),
            "mfma_peak_TFLOPs": peak, "mfma_frac": round(tfs / peak, 4),
            "mfma_frac_graph": round(flops / (graph_ms * 1e-3) / 1e12 / peak, 4),
        }
        if tag == "bf16kv":  # the default choice here is the split-step kernel; the 16-row one beside it
            with _forced_prefill_kernel("tile"):
                res[f"chunked_prefill_{tag}"]["attention_us_graph_16row_kernel"] = round(1e3 * time_graph_call(attn), 2)
            res[f"chunked_prefill_{tag}"]["kernel"] = ("split-step (8 wavefronts share one 32-row tile's 32-key steps, "
                                                       "one workgroup per CU)")
        else:
            res[f"chunked_prefill_{tag}"]["kernel"] = "16-row tiles (4 wavefronts per tile, KV staged through LDS)"
        if with_cpu:  # the pools already hold the appended chunks
            log(f"CPU timings: chunked prefill ({tag})")
            res[f"chunked_prefill_{tag}"]["cpu"] = cpu_call_times(
                w["q"], w["k_pool"], w["v_pool"], lists, w["seq_lens"], w["chunk_lens"], loop_request=0)
        del w
        res[f"chunked_prefill_{tag}"]["mixed_chunks"] = _chunked_prefill_mix(device, kv_dtype, steps, peak)


def _chunked_prefill_mix(device, kv_dtype, steps, peak):
    """The same configuration at seed 2, whose chunks are a 128/256 mix (seed 0 draws four
    256-token chunks): attention time, eager and in graph replay."""
    from src import workloads
    from src.kernels.hip_paged_attention import kv_append_hip, paged_attention_prefill_hip

    w = workloads.chunked_prefill(seed=2, device=device, kv_dtype=kv_dtype)
    lists = w["block_lists"]
    pt, s32, cur, slots = _prefill_metadata(device, lists, w["prev_lens"], w["chunk_lens"], w["q"].shape[2])
    kv_append_hip(w["k_new"], w["v_new"], w["k_pool"], w["v_pool"], slots)
    attn = lambda: paged_attention_prefill_hip(w["q"], w["k_pool"], w["v_pool"], pt, s32, cur)
    attn_ms = time_call(attn, steps)
    graph_ms = time_graph_call(attn)
    flops = workloads.prefill_flops(w["prev_lens"], w["chunk_lens"], 8, 64)
    padded = workloads.prefill_flops_with_padding(w["prev_lens"], w["chunk_lens"], w["q"].shape[2], 8, 64)
    return {
        "workload": f"seed 2: context {w['prev_lens']} + chunk {w['chunk_lens']}",
        "attention_us": round(1e3 * attn_ms, 2), "attention_us_graph": round(1e3 * graph_ms, 2),
        "useful_gflop": round(flops / 1e9, 4),
        "gflop_with_padded_rows": round(padded / 1e9, 4),
        "padded_rows": "rows past a 128-token chunk in the 256-row batch attend to all of their request's keys, "
                       "as in the reference, so the kernel computes them; useful_gflop counts real rows only",
        "TFLOPs_graph": round(flops / (graph_ms * 1e-3) / 1e12, 2),
        "mfma_frac_graph": round(flops / (graph_ms * 1e-3) / 1e12 / peak, 4),
        "mfma_frac_graph_with_padded_rows": round(padded / (graph_ms * 1e-3) / 1e12 / peak, 4),
    }


def _prefill_metadata(device, lists, prev_lens, chunk_lens, T):
    """Page table, sequence lengths, chunk lengths and append slots of a chunked-prefill batch,
    packed on the device (the chunk's blocks already in the lists)."""
    import torch

    from src.kernels.hip_paged_attention import pack_metadata_hip

    flat = [i for x in lists for i in x]
    offs = [0]
    for x in lists:
        offs.append(offs[-1] + len(x))
    i32 = lambda a: torch.tensor(a, dtype=torch.int32, device=device)
    pt, s32, _, slots = pack_metadata_hip(i32(flat), i32(offs), i32(prev_lens), i32(chunk_lens),
                                          query_len=T, block_size=16, max_pages=max(len(x) for x in lists))
    return pt, s32, i32(chunk_lens), slots


def _large_prefill(res, device, steps):
    import torch

    from src import workloads
    from src.kernels.hip_paged_attention import PREFILL_BALANCED, paged_attention_prefill_hip

    for kv_dtype, tag in ((torch.bfloat16, "bf16kv"), (torch.float32, "fp32")):
        b = workloads.large_prefill(seed=0, device=device, kv_dtype=kv_dtype)
        H, Hd = b.q.shape[1], b.q.shape[3]
        flops = workloads.prefill_flops(b.extra["prev_lens"], b.cur_lens, H, Hd)
        call = lambda: paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
        ms = time_call(call, max(3, steps // 2))
        graph_ms = time_graph_call(call, calls=10 if tag == "bf16kv" else 4, replays=3)
        peak = 157.3 if tag == "fp32" else 2500.0
        tfs = flops / (ms * 1e-3) / 1e12
        res[f"large_prefill_{tag}"] = {
            "workload": f"{b.batch} requests, {H} heads x {Hd}, context {b.extra['prev_lens']} + chunk 512 each, "
                        f"{'bf16' if tag == 'bf16kv' else 'fp32'} KV, fp32 q/out "
                        "(wide-tile kernel: 128 query rows per workgroup, KV staged through LDS)",
            "attention_us": round(1e3 * ms, 1), "attention_us_graph": round(1e3 * graph_ms, 1),
            "timing": "attention_us: eager calls through the Python wrapper, averaged (host gaps between calls); "
                      "attention_us_graph: the same call replayed back to back from a HIP graph, with no gap between "
                      "launches (sustained load)",
            "useful_gflop": round(flops / 1e9, 2), "TFLOPs": round(tfs, 1),
            "TFLOPs_graph": round(flops / (graph_ms * 1e-3) / 1e12, 1),
            "mfma_peak_TFLOPs": peak, "mfma_frac": round(tfs / peak, 4),
            "mfma_frac_graph": round(flops / (graph_ms * 1e-3) / 1e12 / peak, 4),
        }
        if tag == "bf16kv":
            # The balanced launch (a resident grid, KV steps dealt out evenly, cut tiles merged in
            # the launch), which the library's policy does not take at this size, forced and timed
            # beside the default one on the same batch.
            bal = lambda: paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t,
                                                      b.cur_lens_t, split_blocks=PREFILL_BALANCED)
            with _env("PAGED_HIP_PREFILL_BALANCE", "force"):
                bal_ms = time_call(bal, max(3, steps // 2))
            res[f"large_prefill_{tag}"]["attention_us_balanced_launch"] = round(1e3 * bal_ms, 1)
        del b
        torch.cuda.empty_cache()


def _long_prompt_prefill(res, device, steps):
    import torch

    from src import workloads
    from src.kernels.hip_paged_attention import paged_attention_prefill_hip

    # One long prompt: 1 request x 32 heads x 128, a 512-token chunk over an 8k context (128
    # tiles of 128 rows, half a tile per CU), bf16 and fp32 KV; and the benchmark model's head
    # shape (8 heads x 64), a 128-token chunk over a 32k context (8 tiles), bf16 and fp32 KV. The default
    # call takes the balanced launch on each; the unbalanced dispatch (the 16-row kernel at these
    # tile counts) is timed beside it.
    for kv_dtype, tag, peak, H, Hd, chunk, ctx, per_cu in (
            (torch.bfloat16, "bf16kv", 2500.0, 32, 128, 512, 8192, "two workgroups"),
            (torch.float32, "fp32", 157.3, 32, 128, 512, 8192, "two workgroups"),
            (torch.bfloat16, "bf16kv_head_dim_64", 2500.0, 8, 64, 128, 32768, "one workgroup"),
            (torch.float32, "fp32_head_dim_64", 157.3, 8, 64, 128, 32768, "one workgroup")):
        b = workloads.large_prefill(seed=16, device=device, batch=1, heads=H, head_dim=Hd, chunk=chunk,
                                    ctx_lo=ctx, ctx_hi=ctx, kv_dtype=kv_dtype)
        flops = workloads.prefill_flops(b.extra["prev_lens"], b.cur_lens, H, Hd)
        call = lambda: paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
        reps = steps if kv_dtype == torch.bfloat16 else max(3, steps // 4)
        ms = time_call(call, reps)
        with _env("PAGED_HIP_PREFILL_BALANCE", "off"):
            ms_plain = time_call(call, reps)
        tfs = flops / (ms * 1e-3) / 1e12
        res[f"long_prompt_prefill_{tag}"] = {
            "workload": f"1 request, {H} heads x {Hd}, context {b.extra['prev_lens'][0]} + chunk {chunk}, "
                        f"{'bf16' if kv_dtype == torch.bfloat16 else 'fp32'} KV, fp32 q/out "
                        f"(default dispatch: the balanced launch, {per_cu} per CU)",
            "attention_us": round(1e3 * ms, 1), "attention_us_unbalanced": round(1e3 * ms_plain, 1),
            "useful_gflop": round(flops / 1e9, 2), "TFLOPs": round(tfs, 1), "mfma_peak_TFLOPs": peak,
            "mfma_frac": round(tfs / peak, 4),
        }
        del b
        torch.cuda.empty_cache()


def _mid_prefill(res, device, steps):
    import torch

    from src import workloads
    from src.kernels.hip_paged_attention import paged_attention_prefill_hip

    # A mid-size prefill: 4 x 32 heads x 128 with 256-token chunks is one 128-row unit per CU, where
    # the dispatch takes the wide kernel for bf16 KV; the 16-row kernel is timed beside it.
    b = workloads.large_prefill(seed=0, device=device, batch=4, chunk=256, ctx_lo=512, ctx_hi=1536)
    H, Hd = b.q.shape[1], b.q.shape[3]
    flops = workloads.prefill_flops(b.extra["prev_lens"], b.cur_lens, H, Hd)
    call = lambda: paged_attention_prefill_hip(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    ms = time_call(call, steps)
    with _forced_prefill_kernel("tile"):
        ms_tile = time_call(call, steps)
    cold_ms = time_cold_prefill(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t, copies=12)
    tfs = flops / (ms * 1e-3) / 1e12
    res["mid_prefill_bf16kv"] = {
        "workload": f"{b.batch} requests, {H} heads x {Hd}, context {b.extra['prev_lens']} + chunk 256 each, "
                    "bf16 KV, fp32 q/out (default dispatch: wide-tile kernel, one unit per CU)",
        "attention_us": round(1e3 * ms, 1), "attention_us_16row_kernel": round(1e3 * ms_tile, 1),
        "attention_us_cold": round(1e3 * cold_ms, 1),
        "timing": "attention_us: the same call repeated (~85 MB of KV, largely MALL-resident); attention_us_cold: "
                  "the call over 12 disjoint copies of its blocks in one graph (~1 GB)",
        "useful_gflop": round(flops / 1e9, 2), "TFLOPs": round(tfs, 1), "mfma_peak_TFLOPs": 2500.0,
        "mfma_frac": round(tfs / 2500.0, 4),
    }
    del b
    torch.cuda.empty_cache()


def calibration_copy(device, nbytes: int = 1 << 32) -> None:
    """A plain device copy of known size (reads and writes nbytes), for scaling HBM counters."""
    import torch

    src = torch.empty(nbytes, dtype=torch.uint8, device=device)
    dst = torch.empty_like(src)
    src.fill_(1)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    log(f"calibration copy: 3 x {nbytes} bytes read and written")


def box_bandwidth(device, nbytes: int = 4 << 30, reps: int = 10) -> dict:
    """What this box's HBM delivers, measured in the same process right after the decode timing,
    with the decode kernel's 16-byte non-temporal loads: a streaming read of `nbytes`
    (pa_hbm_read_probe, the best over 4 grid sizes x 3 workgroup sizes x 1, 4 or 8 loads in
    flight per lane), the same bytes as 4 KB chunks in a random order, as a paged KV pool is read
    (pa_hbm_chunk_read_probe, the best over 4 grid sizes x 1, 2 or 4 chunks in flight per
    workgroup), and torch's device copy of nbytes / 2 (counted as read + write bytes). HIP events
    on the stream the kernels run on."""
    import torch

    from src.kernels import _lib

    lib = _lib.load()
    cus = torch.cuda.get_device_properties(device).multi_processor_count
    stream = torch.cuda.current_stream(device)
    buf = torch.zeros(nbytes, dtype=torch.uint8, device=device)
    sink = torch.zeros(16 * cus, dtype=torch.int32, device=device)
    best = (0.0, "")
    for per_cu in (1, 2, 4, 8):
        for threads in (256, 512, 1024):
            for depth in (1, 4, 8):
                wgs = cus * per_cu
                call = lambda: _lib.check(lib.pa_hbm_read_probe(buf.data_ptr(), nbytes, sink.data_ptr(), wgs, threads,
                                                                depth, stream.cuda_stream), "pa_hbm_read_probe")
                ms = time_call(call, reps)
                best = max(best, (nbytes / (ms * 1e-3) / 1e9,
                                  f"{wgs} workgroups of {threads}, {depth} loads in flight per lane"))
    chunks = nbytes // 4096
    order = torch.randperm(chunks, generator=torch.Generator().manual_seed(4096)).to(torch.int32).to(device)
    best_chunk = (0.0, "")
    for per_cu in (2, 4, 8, 16):
        for depth in (1, 2, 4):
            wgs = cus * per_cu
            call = lambda: _lib.check(lib.pa_hbm_chunk_read_probe(buf.data_ptr(), order.data_ptr(), chunks,
                                                                  sink.data_ptr(), wgs, depth, stream.cuda_stream),
                                      "pa_hbm_chunk_read_probe")
            ms = time_call(call, reps)
            best_chunk = max(best_chunk, (chunks * 4096 / (ms * 1e-3) / 1e9,
                                          f"{wgs} workgroups of 256, {depth} chunks in flight per workgroup"))
    del buf, order, sink
    half = nbytes // 2
    a = torch.zeros(half, dtype=torch.uint8, device=device)
    b = torch.empty_like(a)
    ms = time_call(lambda: b.copy_(a), reps)
    copy = 2 * half / (ms * 1e-3) / 1e9
    del a, b
    torch.cuda.empty_cache()
    return {"read_probe_GBps": round(best[0], 1), "read_probe_shape": best[1],
            "paged_read_probe_GBps": round(best_chunk[0], 1), "paged_read_probe_shape": best_chunk[1],
            "copy_GBps": round(copy, 1), "bytes": nbytes}


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


def continuous_batching(device, backend: str = "hip_paged", warmup: bool = True, dtype=None,
                        rate: float = 32.0) -> dict:
    """The end-to-end benchmark trace through the continuous scheduler on `device` (model weights
    and activations in `dtype`, default fp32; Poisson arrivals at `rate` requests per second)."""
    import torch

    from src.config import benchmark_serving_request_mix
    from src.inference.generate_with_cache import generate_with_cache
    from src.model.transformer import TinyTransformerLM
    from src.serving.continuous_generate import run_decode_step, run_prefill_chunk
    from src.serving.loadgen import generate_requests
    from src.serving.metrics import summarize_run
    from src.serving.scheduler import ContinuousBatchingScheduler

    # The weights are drawn on the host (CPU generator, seed 42) and then moved, so the GPU run and
    # the CPU baseline run the same model.
    torch.manual_seed(42)
    model = TinyTransformerLM(vocab_size=5000, d_model=512, num_heads=8, num_layers=6, d_ff=2048, max_seq_len=1024,
                              attention_backend=backend, kv_block_size=16, kv_pool_initial_blocks=64,
                              kv_pool_growth_factor=2.0)
    init_weights_normal(model)
    model = model.to(device).eval()
    if dtype is not None:
        model = model.to(dtype)
    graphs_prepared = 0
    if warmup:  # as the reference harness: one batched generate, then fresh pools
        generate_with_cache(model, torch.randint(0, 5000, (8, 512), device=device), max_new_tokens=[2] * 8)
        if device.type == "cuda":
            torch.cuda.synchronize()
        model.reset_paged_cache_pools()
        # capture the HIP graphs of cached steps (batch sizes 1..8, chunk buckets, decode) here,
        # outside the timed run
        graphs_prepared = model.prepare_graphs(8, device)
    reqs = generate_requests(200, rate, 5000, workload_profiles=benchmark_serving_request_mix(), seed=42)
    sched = ContinuousBatchingScheduler(max_batch_size=8, prefill_chunk_size=256, max_tokens_per_iteration=1536)
    dev = str(device) if device.type == "cuda" else "cpu"
    t0 = time.perf_counter()
    with torch.no_grad():
        done, events = sched.run(
            reqs,
            prefill_executor=lambda b, c, t, e: run_prefill_chunk(model, b, c, dev, t, e),
            decode_executor=lambda b, t, e: run_decode_step(model, b, dev, t, e),
            release_request_cache=lambda r: model.release_request_caches(r.kv_caches),
        )
    wall = time.perf_counter() - t0
    s = summarize_run(done, events, rate, 8, 0.0, "continuous", 256, 0)
    return {
        "tokens_per_s": s["throughput_tokens_per_s"],
        "p50_ttft_ms": s["p50_first_token_latency_ms"],
        "mean_ttft_ms": s["mean_first_token_latency_ms"],
        "p95_ttft_ms": s["p95_first_token_latency_ms"],
        "requests": s["num_requests"],
        "generated_tokens": sum(r.max_new_tokens for r in done),
        "decode_ms_per_token": s["mean_decode_ms_per_token"],
        "prefill_runtime_ms_total": s["prefill_runtime_ms_total"],
        "decode_runtime_ms_total": s["decode_runtime_ms_total"],
        "events": s["num_batches"],
        "wall_s": wall,
        "graphs_captured_in_warmup": graphs_prepared,
        "graphs_captured_in_run": (model._graph_step.captures - graphs_prepared) if model._graph_step else 0,
        "_tokens": {r.request_id: list(r.generated_token_ids) for r in done},
    }


def token_agreement(a: dict, b: dict) -> dict:
    """Per-request agreement of two runs' greedy tokens (request id -> generated ids). A request's
    greedy tokens depend only on its own prompt, so two runs agree request by request even when
    they batched the requests differently; they may part at a near-tie of two logits, after which
    the rest of that request differs."""
    same = [rid for rid in a if a[rid] == b.get(rid)]
    firsts = []
    for rid in a:
        x, y = a[rid], b.get(rid, [])
        if x != y:
            firsts.append(next((i for i, (u, v) in enumerate(zip(x, y)) if u != v), min(len(x), len(y))))
    total = sum(len(x) for x in a.values())
    agree = sum(sum(1 for u, v in zip(a[rid], b.get(rid, [])) if u == v) for rid in a)
    return {"requests": len(a), "requests_identical": len(same), "tokens": total, "tokens_equal": agree,
            "first_difference_positions": sorted(firsts)}


def continuous_batching_pair(device, with_cpu: bool = True) -> dict:
    """GPU run (hip_paged) and the same-run CPU baseline (torch paged_reference on the host cores)."""
    import torch

    gpu = continuous_batching(device, "hip_paged")
    gpu_tokens = gpu.pop("_tokens")
    if not with_cpu:
        return gpu
    torch.set_num_threads(cpu_threads())
    log(f"continuous batching on the CPU ({torch.get_num_threads()} threads)")
    cpu = continuous_batching(torch.device("cpu"), "paged_reference", warmup=False)
    gpu["token_agreement_with_cpu"] = token_agreement(gpu_tokens, cpu.pop("_tokens"))
    cpu["threads"] = torch.get_num_threads()
    cpu["host"] = cpu_info()
    cpu["kind"] = "port: this package's paged_reference backend (vectorised torch) on the CPU, same trace and weights"
    gpu["clock"] = "scheduler virtual clock (sum of measured forward times), as the reference"
    gpu["cpu_baseline"] = cpu
    return gpu


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-decode", action="store_true", help="skip the headline decode (profiling runs)")
    ap.add_argument("--only", default=",".join(SECONDARY),
                    help="comma-separated secondary workload groups to run: " + ", ".join(SECONDARY))
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a copy kernel of known size (scales HBM counters in a profiling run)")
    ap.add_argument("--no-box-calibration", action="store_true",
                    help="skip the read-probe and copy bandwidth measured after the decode timing")
    ap.add_argument("--e2e-model", choices=("fp32", "bf16", "both"), default="both",
                    help="end-to-end runs: the fp32 model (with its CPU baseline), the bf16 model, or both")
    args = ap.parse_args()
    only = tuple(x for x in args.only.split(",") if x)
    unknown = sorted(set(only) - set(SECONDARY))
    if unknown:
        print(f"bench.py: unknown --only groups {unknown}; choose from {', '.join(SECONDARY)}", file=sys.stderr)
        return 2
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the library has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        return 2

    import torch

    from src import workloads

    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        return 2
    dev = torch.device("cuda:0")
    result = {
        "metric": METRIC,
        "value": None,
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16-kv/f32-acc",
        "data": "synthetic",
    }
    if not args.no_decode:
        log("building the large ragged decode batch (B=256, 32x128, bf16 KV)")
        batch = workloads.large_decode(seed=0, device=dev)
        nbytes = batch.decode_bytes()
        log(f"pool blocks={batch.k_pool.shape[0]} tokens={sum(batch.seq_lens)} algorithmic bytes/call={nbytes}")
        ms, wall_ms, _ = time_decode(batch, args.steps, args.warmup)
        gbs = nbytes / (ms * 1e-3) / 1e9
        log(f"decode: {ms:.3f} ms/call (events), {wall_ms:.3f} ms/call (wall), {gbs:.1f} GB/s")
        # Measured after the decode timing: right after a heavy copy the same decode calls measured
        # ~4% slower on one box, so the calibration must not run ahead of the timed region.
        box = None
        if not args.no_box_calibration:
            box = box_bandwidth(dev)
            log(f"box: read probe {box['read_probe_GBps']} GB/s, 4 KB chunks in random order "
                f"{box['paged_read_probe_GBps']} GB/s, copy {box['copy_GBps']} GB/s")
        result.update({
            "value": round(gbs, 2),
            "ms_per_step": round(ms, 4),
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
                "traffic": pmc_traffic_bytes(),
            },
        })
        if box is not None:
            # the same kernel against what this box's HBM delivers to a streaming read, to the
            # paged pool's access pattern (4 KB slabs in random order) and to a copy, so a slower
            # box and a slower kernel can be told apart
            result["roofline"].update({
                "hbm_read_probe_GBps": box["read_probe_GBps"],
                "frac_vs_read_probe": round(gbs / box["read_probe_GBps"], 4),
                "hbm_paged_read_probe_GBps": box["paged_read_probe_GBps"],
                "frac_vs_paged_read_probe": round(gbs / box["paged_read_probe_GBps"], 4),
                "hbm_copy_GBps": box["copy_GBps"],
                "frac_vs_copy": round(gbs / box["copy_GBps"], 4),
                "calibration": f"read probe: {box['bytes']} bytes read once in order with 16-byte non-temporal loads, "
                               f"best of 36 shapes ({box['read_probe_shape']}); paged read probe: the same bytes as "
                               f"4 KB chunks in a random order, best of 12 shapes ({box['paged_read_probe_shape']}); "
                               f"copy: torch copy of {box['bytes'] // 2} bytes, read + write counted",
            })
        if not args.no_cpu_baseline:
            log("CPU baseline (oracle over the batch)")
            result["cpu_baseline"] = cpu_baseline(batch)
            result["cpu_reference_loop"] = reference_loop_rate(batch)
        del batch
        torch.cuda.empty_cache()
    if args.calibrate_copy:
        calibration_copy(dev)
    if not args.no_secondary:
        log("secondary workloads (single and ragged fp32 decode, chunked, large and mid-size prefill)")
        result["secondary"] = secondary_workloads(dev, args.steps, with_cpu=not args.no_cpu_baseline, only=only)
    if not args.no_e2e:
        if args.e2e_model in ("fp32", "both"):
            log("end-to-end continuous batching (200 requests, 32 req/s)")
            result["continuous_batching"] = continuous_batching_pair(dev, with_cpu=not args.no_cpu_baseline)
        if args.e2e_model in ("bf16", "both"):
            log("end-to-end continuous batching with the model in bf16")
            bf = continuous_batching(dev, dtype=torch.bfloat16)
            bf.pop("_tokens")
            bf["model_dtype"] = "bf16 (weights, activations, KV pools; fp32 accumulation)"
            result["continuous_batching_bf16_model"] = bf
        if args.e2e_model in ("fp32", "both"):
            # The benchmark rate (32 req/s) bounds the GPU's tokens/s by the arrivals; with every
            # request arriving at once the same scheduler (max batch 8) shows the serving path's
            # capacity, comparable with the CPU baseline's compute-bound rate above.
            log("end-to-end continuous batching, saturated (200 requests arriving at once)")
            sat = continuous_batching(dev, rate=1.0e6)
            sat.pop("_tokens")
            sat["arrivals"] = "the same 200-request mix, Poisson at 1e6 req/s (all within ~1 ms)"
            result["continuous_batching_saturated"] = sat
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
