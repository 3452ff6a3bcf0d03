"""The balanced launch of the wide prefill kernels (bf16 and fp32 KV, head_dim 128 and 64;
split_blocks < 0): the tiles' KV steps dealt out evenly over a grid of resident workgroups, tiles cut between
workgroups merged in the same launch by the piece that finishes last; and the library's policy
for when to take it. Checked against the oracle on the same KV values (bf16 KV 2e-2, fp32 KV
1e-4) and against the unbalanced launch, on repeated calls (the arrival counters must be left at
zero), in a HIP graph, and on ragged shapes whose tiles are cut into many pieces."""
import os

import numpy as np
import pytest
import torch

import oracle
from src import workloads
from src.kernels import _lib
from src.kernels.hip_paged_attention import PREFILL_BALANCED, cu_count, paged_attention_prefill_hip
from test_gpu_prefill import _check_large_request, make_prefill, max_err

pytestmark = pytest.mark.gpu
NTHREADS = min(16, os.cpu_count() or 1)


@pytest.fixture
def forced(monkeypatch):
    """The balanced launch wherever it can run, also where the library's policy would not take it
    (these tests use large grids to cut tiles into many pieces)."""
    monkeypatch.setenv("PAGED_HIP_PREFILL_BALANCE", "force")


def _prefill(b, q=None, page_table=None, **kw):
    q = b.q if q is None else q
    pt = b.page_table if page_table is None else page_table
    return paged_attention_prefill_hip(q, b.k_pool, b.v_pool, pt, b.seq_lens_t, b.cur_lens_t, **kw)


def _balanced_applies(b):
    B, H, T, Hd = b.q.shape
    return _lib.load().pa_prefill_workspace_size(B, H, T, Hd, b.page_table.shape[1], PREFILL_BALANCED) > 0


def test_balanced_large_prefill(device, forced):
    """The large-prefill workload (8 x 32 heads x 128, chunk 512 over 1-4k contexts): three calls
    in a row agree with each other up to the pieces' summation order and with the unbalanced
    launch; requests 0 (shortest) and 6 (longest, its tiles cut between workgroups) against the
    oracle on every head."""
    b = workloads.large_prefill(seed=0, device=device)
    assert _balanced_applies(b)
    print(f"balanced large prefill ctx={b.extra['prev_lens']} cus={cu_count(device)}", flush=True)
    plain = _prefill(b, split_blocks=0)
    outs = [_prefill(b, split_blocks=PREFILL_BALANCED) for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs:
        d = float((o - plain).abs().max())
        print(f"  vs unbalanced: max diff {d:.2e}", flush=True)
        assert d <= 5e-3
        assert torch.equal(o, outs[0])  # the same pieces merge in the same order every call
    for r in (0, 6):
        _check_large_request(b, outs[-1], r, 2e-2)


def test_balanced_large_prefill_head_dim_64(device, forced):
    """8 requests x 32 heads x 64, chunk 512 over 1-4k contexts, bf16 KV (64-key steps): three
    calls bit-identical, within 5e-3 of the unbalanced launch, requests 0 and 6 against the oracle
    on every head."""
    b = workloads.large_prefill(seed=3, device=device, head_dim=64)
    assert _balanced_applies(b)
    print(f"balanced large prefill head_dim 64 ctx={b.extra['prev_lens']}", flush=True)
    plain = _prefill(b, split_blocks=0)
    outs = [_prefill(b, split_blocks=PREFILL_BALANCED) for _ in range(3)]
    torch.cuda.synchronize()
    for o in outs:
        d = float((o - plain).abs().max())
        print(f"  vs unbalanced: max diff {d:.2e}", flush=True)
        assert d <= 5e-3
        assert torch.equal(o, outs[0])
    for r in (0, 6):
        _check_large_request(b, outs[-1], r, 2e-2)


@pytest.mark.parametrize("kv_dtype,Hd", [(torch.bfloat16, 128), (torch.float32, 128), (torch.bfloat16, 64),
                                         (torch.float32, 64)])
@pytest.mark.parametrize("io_dtype", [torch.float32, torch.bfloat16])
def test_balanced_ragged_requests(device, forced, io_dtype, kv_dtype, Hd):
    """6 requests x 32 heads, T = 300 (three tiles, the last one partial): an empty request, a
    request of 3 new tokens behind a 4000-token context (one long pair cut over many gangs), rows
    padded past short chunks; every request against the oracle, the whole batch against the
    unbalanced launch, twice in a row."""
    ctx = [0, 37, 4000, 16, 0, 1200]
    curs = [300, 150, 3, 90, 0, 300]
    b = make_prefill(device, 41, ctx, curs, T=300, H=32, Hd=Hd, kv_dtype=kv_dtype)
    assert _balanced_applies(b)
    q = b.q.to(io_dtype)
    print(f"balanced ragged io={io_dtype} kv={kv_dtype} head_dim={Hd}", flush=True)
    plain = _prefill(b, q=q, split_blocks=0)
    got = _prefill(b, q=q, split_blocks=PREFILL_BALANCED)
    again = _prefill(b, q=q, split_blocks=PREFILL_BALANCED)
    torch.cuda.synchronize()
    assert torch.equal(got, again)
    if kv_dtype == torch.float32:
        # bf16 output: half an ulp of outputs up to ~4 is ~1.6e-2 against the fp64 oracle
        tol_plain, tol = (2e-5, 1e-4) if io_dtype == torch.float32 else (1e-2, 3e-2)
    else:
        tol_plain, tol = (5e-3, 2e-2) if io_dtype == torch.float32 else (2e-2, 3e-2)
    d = float((got.float() - plain.float()).abs().max())
    want = oracle.paged_attention(q.float().cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens,
                                  b.cur_lens, nthreads=NTHREADS)
    err = max_err(got, want)
    print(f"  max err vs oracle {err:.2e}, vs unbalanced {d:.2e}", flush=True)
    assert d <= tol_plain
    assert err <= tol
    assert float(got[4].abs().max()) == 0.0  # the empty request


@pytest.mark.parametrize("Hd", [128, 64])
def test_balanced_many_heads_and_one_long_request(device, forced, Hd):
    """64 heads (8 pairs per die and request), one 6000-token context among three short ones (its
    pairs are cut over several gangs each), -1 page entries inside cut tiles: against the
    unbalanced launch everywhere and the oracle on the short requests."""
    ctx = [6000, 100, 300]
    curs = [512, 512, 200]
    b = make_prefill(device, 42, ctx, curs, T=512, H=64, Hd=Hd, kv_dtype=torch.bfloat16)
    assert _balanced_applies(b)
    pt = b.page_table.clone()
    pt[0, [5, 130, 131, 300]] = -1
    print(f"balanced 64 heads, one long request, head_dim {Hd}", flush=True)
    plain = _prefill(b, page_table=pt, split_blocks=0)
    got = _prefill(b, page_table=pt, split_blocks=PREFILL_BALANCED)
    torch.cuda.synchronize()
    d = float((got - plain).abs().max())
    print(f"  vs unbalanced: max diff {d:.2e}", flush=True)
    assert d <= 5e-3
    full = _prefill(b, split_blocks=PREFILL_BALANCED)
    assert float((got[0] - full[0]).abs().max()) > 1e-2  # the skipped keys did matter
    want = oracle.paged_attention(b.q[1:].cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists[1:],
                                  b.seq_lens[1:], b.cur_lens[1:], nthreads=NTHREADS)
    assert max_err(full[1:], want) <= 2e-2


def test_balanced_needs_its_workspace(device, forced):
    """Asked for the balanced launch with a workspace smaller than pa_prefill_workspace_size, the
    call fails on the host with PA_ERR_WORKSPACE and launches nothing."""
    b = workloads.large_prefill(seed=0, device=device, batch=5, ctx_lo=1024, ctx_hi=1024)
    B, H, T, Hd = b.q.shape
    lib = _lib.load()
    need = lib.pa_prefill_workspace_size(B, H, T, Hd, b.page_table.shape[1], PREFILL_BALANCED)
    if need == 0:
        pytest.skip("the balanced launch does not apply on this device at 5 x 32 x 4 tiles")
    ws = torch.zeros(need // 2, dtype=torch.uint8, device=device)
    out = torch.empty_like(b.q)
    st = lib.pa_prefill(b.q.data_ptr(), b.q.stride(0), b.q.stride(1), b.q.stride(2),
                        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), _lib.dtype_code(b.q.dtype),
                        b.k_pool.data_ptr(), b.v_pool.data_ptr(), _lib.dtype_code(b.k_pool.dtype),
                        b.k_pool.shape[0], b.page_table.data_ptr(), b.page_table.stride(0),
                        b.page_table.shape[1], b.seq_lens_t.data_ptr(), b.cur_lens_t.data_ptr(),
                        B, H, T, Hd, 16, float(Hd) ** -0.5, PREFILL_BALANCED, ws.data_ptr(), need // 2, 0)
    assert st == _lib.PA_ERR_WORKSPACE
    assert "workspace" in lib.pa_last_error_message().decode()


@pytest.mark.parametrize("Hd", [128, 64])
def test_balanced_launch_in_a_graph(device, forced, Hd):
    """The balanced launch captured in a HIP graph (its counters are reset by the kernel, no memset
    in the graph): three replays, each after eager calls of the same launch on other inputs, each
    bit-identical to the eager result on the graph's inputs."""
    b = workloads.large_prefill(seed=0, device=device, batch=5, head_dim=Hd, ctx_lo=1024, ctx_hi=2048)
    other = workloads.large_prefill(seed=9, device=device, batch=5, head_dim=Hd, ctx_lo=1024, ctx_hi=2048)
    assert _balanced_applies(b) and _balanced_applies(other)
    print(f"balanced launch in a graph, head_dim {Hd}", flush=True)
    out = torch.empty_like(b.q)
    call = lambda: _prefill(b, split_blocks=PREFILL_BALANCED, out=out)
    want = _prefill(b, split_blocks=PREFILL_BALANCED).clone()  # eager; allocates the workspace
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for r in range(3):
        _prefill(other, split_blocks=PREFILL_BALANCED)  # eager work between the replays
        torch.cuda.synchronize()
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {r}"


@pytest.mark.parametrize("kv_dtype,tol_plain,tol", [(torch.bfloat16, 5e-3, 2e-2), (torch.float32, 2e-5, 1e-4)])
def test_policy_takes_the_balanced_launch_on_a_long_context(device, monkeypatch, kv_dtype, tol_plain, tol):
    """One request x 32 heads x 128, a 512-token chunk over an 8k context (128 tiles, half a tile
    per CU): the default call takes the balanced launch (two workgroups per CU) and matches the
    oracle on every head and the unbalanced launch; PAGED_HIP_PREFILL_BALANCE=off declines it."""
    b = workloads.large_prefill(seed=16, device=device, batch=1, chunk=512, ctx_lo=8192, ctx_hi=8192,
                                kv_dtype=kv_dtype)
    if 2 * 128 > cu_count(device):
        pytest.skip("fewer than 256 compute units")
    assert _balanced_applies(b)
    print(f"policy: balanced launch on 1 x 32 heads, chunk 512 over 8k, kv={kv_dtype}", flush=True)
    got = _prefill(b)  # default split_blocks: PREFILL_BALANCED
    monkeypatch.setenv("PAGED_HIP_PREFILL_BALANCE", "off")
    assert not _balanced_applies(b)
    plain = _prefill(b)
    torch.cuda.synchronize()
    d = float((got - plain).abs().max())
    print(f"  vs unbalanced: max diff {d:.2e}", flush=True)
    assert d <= tol_plain
    _check_large_request(b, got, 0, tol)


def test_policy_declines_short_contexts_and_sizes_its_grid(device, monkeypatch):
    """A 128-token chunk over 4k (32 tiles x 132 steps, under 8192 tile-steps): no balanced launch.
    Over 16k it is taken with one workgroup per CU (two would cut each tile 16 ways)."""
    monkeypatch.delenv("PAGED_HIP_PREFILL_BALANCE", raising=False)
    lib = _lib.load()
    cus = cu_count(device)
    assert lib.pa_prefill_workspace_size(1, 32, 128, 128, (4096 + 128 + 15) // 16, PREFILL_BALANCED) == 0  # both dtypes
    need = lib.pa_prefill_workspace_size(1, 32, 128, 128, (16384 + 128 + 15) // 16, PREFILL_BALANCED)
    if 2 * 32 > cus or 4 * 32 >= cus:
        pytest.skip("the per-CU rule differs at this CU count")
    record = 4 * 17 * 64 * 4 * 4  # four wavefronts x 17 groups x 64 lanes x 16 bytes
    assert need == (64 << 10) + cus * 2 * record  # grid = one workgroup per CU


@pytest.mark.parametrize("kv_dtype,tol_plain,tol", [(torch.bfloat16, 5e-3, 2e-2), (torch.float32, 2e-5, 1e-4)])
def test_policy_takes_the_balanced_launch_at_head_dim_64(device, monkeypatch, kv_dtype, tol_plain, tol):
    """One request x 8 heads x 64, a 128-token chunk over a 32k context (8 tiles of 514 64-key
    steps with bf16 KV, 1028 32-key steps with fp32 KV): the default call takes the balanced launch
    and matches the unbalanced launch and the oracle on every head; 32 heads with a 512-token chunk
    over 2k (128 tiles x 40 or 80 steps) do not take it with either KV dtype."""
    monkeypatch.delenv("PAGED_HIP_PREFILL_BALANCE", raising=False)
    b = workloads.large_prefill(seed=17, device=device, batch=1, heads=8, head_dim=64, chunk=128,
                                ctx_lo=32768, ctx_hi=32768, kv_dtype=kv_dtype)
    if 2 * 8 > cu_count(device):
        pytest.skip("fewer than 16 compute units")
    assert _balanced_applies(b)
    lib = _lib.load()
    assert lib.pa_prefill_workspace_size(1, 32, 512, 64, (2048 + 512) // 16, PREFILL_BALANCED) == 0
    print(f"policy: balanced launch on 1 x 8 heads x 64, chunk 128 over 32k, kv={kv_dtype}", flush=True)
    got = _prefill(b)
    monkeypatch.setenv("PAGED_HIP_PREFILL_BALANCE", "off")
    plain = _prefill(b)
    torch.cuda.synchronize()
    d = float((got - plain).abs().max())
    print(f"  vs unbalanced: max diff {d:.2e}", flush=True)
    assert d <= tol_plain
    _check_large_request(b, got, 0, tol)
