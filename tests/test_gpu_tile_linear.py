"""The tiled linear kernel (steps of more than 16 rows: 32-row x 16/32-column tiles, K split over
4 wavefronts streaming 128-byte row slices through LDS rings) against float64 references, at the
shapes it takes (in_features 256-2048, out_features a multiple of 16), partial row tiles, both
column-tile widths, every epilogue (LayerNorm, bias, GELU, residual, second copy, K/V scatter),
fp32 and bf16; and against the 16-row kernel on the same calls."""
import pytest
import torch
import torch.nn as nn

from src.kernels import hip_linear
from test_gpu_linear import _Attn, assert_bf16_close, ref_linear, ref_linear_bf16

pytestmark = pytest.mark.gpu


def _layer(device, K, N, seed, dtype=torch.float32):
    torch.manual_seed(seed)
    lin = nn.Linear(K, N).to(device)
    ln = nn.LayerNorm(K).to(device)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.1)
    return lin.to(dtype), ln.to(dtype)


@pytest.mark.parametrize("K", [256, 512, 1024, 2048])
@pytest.mark.parametrize("M,N", [(17, 512), (33, 2048), (100, 512), (256, 2048), (1024, 512)])
def test_tiled_linear_fp32(device, K, M, N):
    lin, ln = _layer(device, K, N, K + M + N)
    x = torch.randn(M, K, device=device) * 2 + 0.3
    r = torch.randn(M, N, device=device)
    use_ln = K <= 1024  # (fp32 at 1024: the statistics pass reads each row in two halves)
    print(f"tiled fp32 K={K} M={M} N={N} ln={use_ln}", flush=True)
    got = hip_linear.linear_rows_hip(x, lin, ln=ln if use_ln else None, gelu=use_ln, residual=r)
    err = (got.double().cpu() - ref_linear(x, lin, ln if use_ln else None, use_ln, r)).abs().max().item()
    assert err <= 5e-5, err


@pytest.mark.parametrize("kernel", ["auto", "tiled"])
@pytest.mark.parametrize("K", [256, 512, 1024, 2048])
@pytest.mark.parametrize("M,N", [(20, 512), (64, 2048), (300, 512)])
def test_tiled_linear_bf16(device, monkeypatch, K, M, N, kernel):
    if kernel == "tiled":
        monkeypatch.setenv("PAGED_HIP_LINEAR_KERNEL", "tiled")
    lin, ln = _layer(device, K, N, 50 + K + M, torch.bfloat16)
    x = (torch.randn(M, K, device=device) * 2 + 0.3).to(torch.bfloat16)
    r = torch.randn(M, N, device=device).to(torch.bfloat16)
    use_ln = K <= 1024
    print(f"tiled bf16 K={K} M={M} N={N} ln={use_ln} kernel={kernel}", flush=True)
    got = hip_linear.linear_rows_hip(x, lin, ln=ln if use_ln else None, gelu=use_ln, residual=r)
    assert_bf16_close(got, ref_linear_bf16(x, lin, ln if use_ln else None, use_ln, r))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_tiled_and_16row_kernels_agree(device, monkeypatch, dtype):
    lin, ln = _layer(device, 512, 2048, 77, dtype)
    x = torch.randn(96, 512, device=device).to(dtype)
    outs = {}
    for kernel in ("tiled", "small"):
        monkeypatch.setenv("PAGED_HIP_LINEAR_KERNEL", kernel)
        outs[kernel] = hip_linear.linear_rows_hip(x, lin, ln=ln, gelu=True).float()
    tol = 1e-5 if dtype == torch.float32 else 2e-2
    assert (outs["tiled"] - outs["small"]).abs().max().item() <= tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("ln_on", [True, False])
def test_tiled_column_widths_agree(device, monkeypatch, dtype, ln_on):
    """16- and 32-column tiles run the same per-column products in the same order: bit-identical
    outputs (q/k/v-sized layer with LayerNorm, and without)."""
    lin, ln = _layer(device, 512, 1536, 79, dtype)
    x = torch.randn(160, 512, device=device).to(dtype)
    monkeypatch.setenv("PAGED_HIP_LINEAR_KERNEL", "tiled")
    outs = {}
    for cols in ("16", "32"):
        monkeypatch.setenv("PAGED_HIP_TILE_COLUMNS", cols)
        outs[cols] = hip_linear.linear_rows_hip(x, lin, ln=ln if ln_on else None, gelu=ln_on)
    assert torch.equal(outs["16"], outs["32"])


def test_tiled_strided_rows_and_copy(device):
    lin, _ = _layer(device, 512, 512, 78)
    big = torch.randn(70, 600, device=device)
    x = big[:, 40:552]  # row stride 600 (16-byte aligned start)
    res = torch.randn(70, 512, device=device)
    want = ref_linear(x, lin, residual=res)
    out = torch.full((70, 520), 7.0, device=device)
    hip_linear.linear_rows_hip(x, lin, residual=res, out=out[:, :512], copy_to=res)
    assert (out[:, 512:] == 7.0).all()
    assert torch.equal(out[:, :512], res)
    assert (res.double().cpu() - want).abs().max().item() <= 2e-5


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_tiled_qkv_append(device, pool_dtype):
    """q/k/v + KV scatter of a 64-row chunk through the tiled kernel: q within 2e-5 of fp64, K/V
    rows in exactly their slots."""
    torch.manual_seed(21)
    d, h, M, bs, nblk = 512, 8, 64, 16, 8
    attn = _Attn(d, h).to(device)
    ln = nn.LayerNorm(d).to(device)
    x = torch.randn(M, d, device=device)
    k_pool = torch.zeros(nblk, h, bs, d // h, device=device, dtype=pool_dtype)
    v_pool = torch.zeros_like(k_pool)
    slots = torch.tensor([(3 * bs + i) if i < 60 else -1 for i in range(M)], dtype=torch.int32, device=device)
    q = hip_linear.qkv_append_hip(x, ln, attn, k_pool, v_pool, slots)
    xn = nn.functional.layer_norm(x.double().cpu(), (d,), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    assert (q.double().cpu() - ref_linear(xn, attn.q_proj)).abs().max().item() <= 2e-5
    kref = ref_linear(xn, attn.k_proj).float().view(M, h, d // h)
    tol = 2e-5 if pool_dtype == torch.float32 else 1e-2
    got = k_pool.cpu().float()
    for i in range(M):
        s = int(slots[i])
        if s >= 0:
            assert (got[s // bs, :, s % bs] - kref[i]).abs().max().item() <= tol
    assert got[3 * bs // bs + 4:].abs().sum() == 0  # blocks past the written slots stay empty
