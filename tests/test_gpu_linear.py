"""Decode-step linear kernels (pa_linear_rows, pa_qkv_append) against float64 torch on the CPU:
LayerNorm prologue, bias / GELU / residual epilogues, every supported in_features, ragged
out_features, 1..2048 rows, and the K/V scatter into fp32 and bf16 pools (bit-exact placement,
skipped slots untouched)."""
import pytest
import torch
import torch.nn as nn

from src.kernels import hip_linear

pytestmark = pytest.mark.gpu


def ref_linear(x, lin, ln=None, gelu=False, residual=None):
    x = x.double().cpu()
    if ln is not None:
        x = nn.functional.layer_norm(x, (x.shape[1],), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    y = x @ lin.weight.double().cpu().t()
    if lin.bias is not None:
        y = y + lin.bias.double().cpu()
    if gelu:
        y = nn.functional.gelu(y)
    if residual is not None:
        y = y + residual.double().cpu()
    return y


@pytest.mark.parametrize("K", [128, 256, 512, 1024, 2048])
@pytest.mark.parametrize("M", [1, 3, 16, 17, 40, 64, 200, 1024, 2048])
def test_linear_rows_shapes(device, K, M):
    torch.manual_seed(K + M)
    N = 300 if K != 512 else 5000  # out_features not a multiple of 16 (partial last tile)
    lin = nn.Linear(K, N).to(device)
    x = torch.randn(M, K, device=device)
    got = hip_linear.linear_rows_hip(x, lin)
    err = (got.double().cpu() - ref_linear(x, lin)).abs().max().item()
    print(f"linear K={K} M={M} N={N}: max err {err:.2e}", flush=True)
    assert err <= 2e-5


@pytest.mark.parametrize("use_ln,gelu,res,bias", [(True, False, False, True), (True, True, False, True),
                                                  (False, False, True, True), (True, True, True, False)])
def test_linear_rows_fusions(device, use_ln, gelu, res, bias):
    torch.manual_seed(7)
    M, K, N = 5, 512, 2048
    lin = nn.Linear(K, N, bias=bias).to(device)
    ln = nn.LayerNorm(K).to(device)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.1)
    x = torch.randn(M, K, device=device) * 3 + 0.5
    r = torch.randn(M, N, device=device) if res else None
    got = hip_linear.linear_rows_hip(x, lin, ln=ln if use_ln else None, gelu=gelu, residual=r)
    want = ref_linear(x, lin, ln if use_ln else None, gelu, r)
    assert (got.double().cpu() - want).abs().max().item() <= 2e-5


def test_linear_rows_strided_rows_and_out(device):
    torch.manual_seed(8)
    lin = nn.Linear(256, 64).to(device)
    big = torch.randn(6, 400, device=device)
    x = big[:, 8:264]  # row stride 400, 16-byte aligned start
    out = torch.full((6, 80), 7.0, device=device)
    hip_linear.linear_rows_hip(x, lin, out=out[:, :64])
    assert (out[:, 64:] == 7.0).all()
    assert (out[:, :64].double().cpu() - ref_linear(x, lin)).abs().max().item() <= 2e-5


def test_linear_rows_rejects_bad_shapes(device):
    lin = nn.Linear(96, 32).to(device)
    with pytest.raises(Exception):
        hip_linear.linear_rows_hip(torch.randn(2, 96, device=device), lin)  # in_features 96 unsupported
    lin = nn.Linear(128, 32).to(device)
    with pytest.raises(ValueError):
        hip_linear.linear_rows_hip(torch.randn(2049, 128, device=device), lin)  # more than 2048 rows


class _Attn(nn.Module):
    def __init__(self, d, h):
        super().__init__()
        self.num_heads, self.head_dim, self.d_model = h, d // h, d
        self.q_proj, self.k_proj, self.v_proj = nn.Linear(d, d), nn.Linear(d, d), nn.Linear(d, d)


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("d,h,M", [(512, 8, 22), (128, 2, 22), (512, 8, 300)])
def test_qkv_append(device, pool_dtype, d, h, M):
    torch.manual_seed(9)
    bs = 16
    nblk = 12 if M <= 22 else 40  # 22 rows: two row tiles; 300 rows: 19, the last one partial
    attn = _Attn(d, h).to(device)
    ln = nn.LayerNorm(d).to(device)
    x = torch.randn(M, d, device=device)
    k_pool = torch.zeros(nblk, h, bs, d // h, device=device, dtype=pool_dtype)
    v_pool = torch.zeros_like(k_pool)
    head = [5 * bs + 3, -1, 0, 11 * bs + 15, 12 * bs, 2 * bs + 7]  # 12 * bs: outside a 12-block pool
    rest = [6 * bs + i for i in range(16)] if M == 22 else [13 * bs + i for i in range(M - len(head))]
    slots = torch.tensor(head + rest, dtype=torch.int32, device=device)
    q = hip_linear.qkv_append_hip(x, ln, attn, k_pool, v_pool, slots)
    xn = nn.functional.layer_norm(x.double().cpu(), (d,), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    assert (q.double().cpu() - ref_linear(xn, attn.q_proj)).abs().max().item() <= 2e-5
    kref = ref_linear(xn, attn.k_proj).float()
    vref = ref_linear(xn, attn.v_proj).float()
    want_k = torch.zeros(nblk, h, bs, d // h, dtype=pool_dtype)
    want_v = torch.zeros_like(want_k)
    for m, s in enumerate(slots.tolist()):
        if s < 0 or s // bs >= nblk:
            continue  # skipped rows (negative slot, block out of range)
        want_k[s // bs, :, s % bs] = kref[m].view(h, d // h).to(pool_dtype)
        want_v[s // bs, :, s % bs] = vref[m].view(h, d // h).to(pool_dtype)
    got_k, got_v = k_pool.cpu(), v_pool.cpu()
    written = want_k.abs().sum(dim=(1, 3)) > 0
    assert torch.equal(got_k.abs().sum(dim=(1, 3)) > 0, written)  # exactly the target slots
    tol = 2e-5 if pool_dtype == torch.float32 else 1e-2
    assert (got_k.float() - want_k.float()).abs().max().item() <= tol
    assert (got_v.float() - want_v.float()).abs().max().item() <= tol


def test_embed_rows(device):
    """Token + position embedding of a [B, T] step, positions clamped to the table like the
    graph step's padded rows; an out-of-vocabulary id gives a zero token row."""
    torch.manual_seed(10)
    tok, pos = nn.Embedding(300, 128).to(device), nn.Embedding(64, 128).to(device)
    ids = torch.randint(0, 300, (3, 20), device=device)
    ids[1, 4] = 300
    p0 = torch.tensor([0, 30, 55], device=device)
    got = hip_linear.embed_rows_hip(ids, p0, tok, pos).cpu()
    want = torch.empty(3 * 20, 128)
    for b in range(3):
        for t in range(20):
            i = int(ids[b, t])
            row = tok.weight[i].cpu() if i < 300 else torch.zeros(128)
            want[b * 20 + t] = row + pos.weight[min(int(p0[b]) + t, 63)].cpu()
    assert torch.equal(got, want)


@pytest.mark.parametrize("K", [128, 1024, 2048])
def test_linear_rows_layernorm_every_width(device, K):
    """The LayerNorm prologue at every kernel width (preloaded parameters up to 1024, read after
    the statistics at 2048), with rows of different means and scales."""
    torch.manual_seed(K)
    M, N = 7, 96
    lin = nn.Linear(K, N).to(device)
    ln = nn.LayerNorm(K, eps=1e-5).to(device)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.2)
        ln.bias.normal_(0.0, 0.2)
    x = torch.randn(M, K, device=device) * torch.linspace(0.1, 10, M, device=device).view(M, 1) + 3.0
    got = hip_linear.linear_rows_hip(x, lin, ln=ln, gelu=True)
    assert (got.double().cpu() - ref_linear(x, lin, ln, True)).abs().max().item() <= 5e-5


# ---- bf16 weights and activations ------------------------------------------------------------

def bf16_round(t):
    return t.to(torch.bfloat16).double()


def ref_linear_bf16(x, lin, ln=None, gelu=False, residual=None):
    """fp64 arithmetic on the bf16 operands, with the rounding points of the fused kernel: the
    LayerNorm output rounded to bf16 (as torch's bf16 LayerNorm), one rounding of the result."""
    x = x.double().cpu()
    if ln is not None:
        x = bf16_round(nn.functional.layer_norm(x, (x.shape[1],), ln.weight.double().cpu(), ln.bias.double().cpu(),
                                                ln.eps))
    y = x @ lin.weight.double().cpu().t()
    if lin.bias is not None:
        y = y + lin.bias.double().cpu()
    if gelu:
        y = nn.functional.gelu(y)
    if residual is not None:
        y = y + residual.double().cpu()
    return y


def assert_bf16_close(got, want):
    """Within one bf16 rounding of the result (2^-8 relative) plus fp32-accumulation slack."""
    err = (got.double().cpu() - want).abs()
    bound = 2.0 ** -8 * want.abs() + 2e-3 * want.abs().max().clamp_min(1e-3)
    assert bool((err <= bound).all()), float((err - bound).max())


@pytest.mark.parametrize("K", [128, 256, 512, 1024, 2048])
@pytest.mark.parametrize("M", [1, 16, 40, 64, 200])
def test_linear_rows_bf16_shapes(device, K, M):
    torch.manual_seed(100 + K + M)
    N = 300
    lin = nn.Linear(K, N).to(device).to(torch.bfloat16)
    x = torch.randn(M, K, device=device).to(torch.bfloat16)
    got = hip_linear.linear_rows_hip(x, lin)
    assert got.dtype == torch.bfloat16
    assert_bf16_close(got, ref_linear_bf16(x, lin))


@pytest.mark.parametrize("K", [128, 512, 2048])
@pytest.mark.parametrize("use_ln,gelu,res", [(True, False, False), (True, True, False), (False, False, True),
                                             (True, True, True)])
def test_linear_rows_bf16_fusions(device, K, use_ln, gelu, res):
    torch.manual_seed(7 + K)
    M, N = 9, 1000
    lin = nn.Linear(K, N).to(device).to(torch.bfloat16)
    ln = nn.LayerNorm(K).to(device)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.1)
    ln = ln.to(torch.bfloat16)
    x = (torch.randn(M, K, device=device) * 3 + 0.5).to(torch.bfloat16)
    r = torch.randn(M, N, device=device).to(torch.bfloat16) if res else None
    got = hip_linear.linear_rows_hip(x, lin, ln=ln if use_ln else None, gelu=gelu, residual=r)
    assert_bf16_close(got, ref_linear_bf16(x, lin, ln if use_ln else None, gelu, r))


def test_linear_rows_rejects_mixed_dtypes(device):
    lin = nn.Linear(128, 32).to(device).to(torch.bfloat16)
    with pytest.raises(ValueError):
        hip_linear.linear_rows_hip(torch.randn(2, 128, device=device), lin)  # fp32 rows, bf16 weights


@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_qkv_append_bf16(device, pool_dtype):
    torch.manual_seed(19)
    d, h, M, bs, nblk = 512, 8, 22, 16, 12
    attn = _Attn(d, h).to(device).to(torch.bfloat16)
    ln = nn.LayerNorm(d).to(device).to(torch.bfloat16)
    x = torch.randn(M, d, device=device).to(torch.bfloat16)
    k_pool = torch.zeros(nblk, h, bs, d // h, device=device, dtype=pool_dtype)
    v_pool = torch.zeros_like(k_pool)
    slots = torch.tensor([5 * bs + 3, -1, 0, 11 * bs + 15, 12 * bs, 2 * bs + 7] + [6 * bs + i for i in range(16)],
                         dtype=torch.int32, device=device)
    q = hip_linear.qkv_append_hip(x, ln, attn, k_pool, v_pool, slots)
    assert q.dtype == torch.bfloat16
    assert_bf16_close(q, ref_linear_bf16(x, attn.q_proj, ln))
    kref = ref_linear_bf16(x, attn.k_proj, ln)
    vref = ref_linear_bf16(x, attn.v_proj, ln)
    for m, s in enumerate(slots.tolist()):
        if s < 0 or s // bs >= nblk:
            continue
        for pool, ref in ((k_pool, kref), (v_pool, vref)):
            got = pool[s // bs, :, s % bs].reshape(-1).unsqueeze(0)
            assert_bf16_close(got, ref[m].unsqueeze(0))
    written = (k_pool.float().abs().sum(dim=(1, 3)) > 0).cpu()
    want = torch.zeros(nblk, bs, dtype=torch.bool)
    for s in slots.tolist():
        if 0 <= s and s // bs < nblk:
            want[s // bs, s % bs] = True
    assert torch.equal(written, want)


def test_embed_rows_bf16(device):
    """bf16 tables: each row is the fp32 sum of the two bf16 vectors, rounded once (bit-exact)."""
    torch.manual_seed(11)
    tok = nn.Embedding(300, 128).to(device).to(torch.bfloat16)
    pos = nn.Embedding(64, 128).to(device).to(torch.bfloat16)
    ids = torch.randint(0, 300, (2, 9), device=device)
    ids[0, 3] = -1
    p0 = torch.tensor([0, 60], device=device)
    got = hip_linear.embed_rows_hip(ids, p0, tok, pos).cpu()
    assert got.dtype == torch.bfloat16
    want = torch.empty(18, 128, dtype=torch.bfloat16)
    for b in range(2):
        for t in range(9):
            i = int(ids[b, t])
            row = tok.weight[i].float().cpu() if 0 <= i < 300 else torch.zeros(128)
            want[b * 9 + t] = (row + pos.weight[min(int(p0[b]) + t, 63)].float().cpu()).to(torch.bfloat16)
    assert torch.equal(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("groups,group_rows", [(1, 1), (3, 7), (8, 1), (8, 256), (5, 33)])
def test_linear_select_rows(device, dtype, groups, group_rows):
    """pa_linear_select_rows computes each group's selected row, bit-identical to pa_linear_rows on
    that row alone (same kernel, same per-row arithmetic), and within 2e-5 of float64 torch for fp32;
    negative rows count from the group's end, out-of-range rows are clamped into the group."""
    torch.manual_seed(groups * 100 + group_rows)
    K, N = 512, 5000
    lin = nn.Linear(K, N).to(device=device, dtype=dtype)
    ln = nn.LayerNorm(K).to(device=device, dtype=dtype)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.1)
    x = torch.randn(groups * group_rows, K, device=device).to(dtype)
    g = torch.Generator().manual_seed(groups + group_rows)
    rows = torch.randint(-group_rows, group_rows, (groups,), generator=g, dtype=torch.int32)
    if groups >= 3:
        rows[0], rows[1] = group_rows + 5, -group_rows - 3  # clamped to the group's last / first row
    eff = [min(max(r + group_rows if r < 0 else r, 0), group_rows - 1) for r in rows.tolist()]
    picked = torch.stack([x[gi * group_rows + r] for gi, r in enumerate(eff)])
    got = hip_linear.linear_select_rows_hip(x, group_rows, rows.to(device), lin, ln=ln)
    assert got.shape == (groups, N)
    same = hip_linear.linear_rows_hip(picked.contiguous(), lin, ln=ln)
    assert torch.equal(got, same)
    if dtype == torch.float32:
        assert (got.double().cpu() - ref_linear(picked, lin, ln)).abs().max().item() <= 2e-5


def test_linear_select_rows_rejects_bad_arguments(device):
    lin = nn.Linear(256, 64).to(device)
    x = torch.randn(12, 256, device=device)
    rows = torch.zeros(3, dtype=torch.int32, device=device)
    with pytest.raises(ValueError):
        hip_linear.linear_select_rows_hip(x, 5, rows, lin)  # 3 groups of 5 rows > 12 rows
    with pytest.raises(ValueError):
        hip_linear.linear_select_rows_hip(x, 4, rows.long(), lin)
    with pytest.raises(ValueError):
        hip_linear.linear_select_rows_hip(x, 4, rows.cpu(), lin)
    with pytest.raises(ValueError):
        hip_linear.linear_select_rows_hip(x, 4, rows, lin, out=torch.empty(3, 32, device=device))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("K", [128, 256, 512, 1024, 2048])
@pytest.mark.parametrize("M,N", [(1, 300), (5, 40), (8, 1536), (16, 5000)])
def test_linear_lds_staging_matches_registers(device, monkeypatch, dtype, K, M, N):
    """One-tile launches (<= 16 rows) stage their weight and activation slices through LDS: the
    same products in the same order as loading the operands straight into registers, so the
    outputs are bit-identical (LayerNorm + GELU + residual, narrow and wide layers, and the
    row-selecting head over strided groups)."""
    torch.manual_seed(K + M + N)
    lin = nn.Linear(K, N).to(device, dtype)
    ln = nn.LayerNorm(K).to(device, dtype)
    with torch.no_grad():
        ln.weight.uniform_(0.5, 1.5)
        ln.bias.uniform_(-0.2, 0.2)
    x = torch.randn(M, K, device=device, dtype=dtype)
    res = torch.randn(M, N, device=device, dtype=dtype)
    xs = torch.randn(M * 7, K, device=device, dtype=dtype)  # M groups of 7 rows
    rows = torch.tensor([(3 * g) % 7 - (g % 2) * 7 for g in range(M)], dtype=torch.int32, device=device)
    print(f"linear staging dtype={dtype} K={K} M={M} N={N}", flush=True)
    outs = {}
    for staging in ("lds", "regs"):
        if staging == "regs":
            monkeypatch.setenv("PAGED_HIP_LINEAR_STAGING", "regs")
        outs[staging] = (hip_linear.linear_rows_hip(x, lin),
                         hip_linear.linear_rows_hip(x, lin, ln=ln, gelu=True, residual=res),
                         hip_linear.linear_select_rows_hip(xs, 7, rows, lin, ln=ln))
    for a, b in zip(outs["lds"], outs["regs"]):
        assert torch.equal(a, b)
    err = (outs["lds"][1].double().cpu() - ref_linear(x, lin, ln=ln, gelu=True, residual=res)).abs().max().item()
    assert err <= (2e-5 if dtype == torch.float32 else 0.1)


@pytest.mark.parametrize("key_stride", [1, hip_linear.KEY_STRIDE])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("case", ["plain", "ties", "zeros", "nan"])
def test_linear_select_rows_folds_the_argmax(device, dtype, case, key_stride):
    """pa_linear_select_rows with token_keys: the low word of each group's key is torch.argmax of
    the group's output row as stored (first index of the maximum; -0.0 == +0.0; the first NaN
    wins), the outputs themselves unchanged; exact ties planted by duplicated weight rows. Keys
    packed or one 128-byte line apart; the words between strided keys stay untouched."""
    torch.manual_seed(11)
    K, N, groups, rows = 512, 5000, 6, 9
    lin = nn.Linear(K, N).to(device, dtype)
    ln = nn.LayerNorm(K).to(device, dtype)
    with torch.no_grad():
        if case == "ties":
            for dst, src in ((4000, 17), (4001, 17), (10, 4999)):  # same column values -> exact ties
                lin.weight[dst] = lin.weight[src]
                lin.bias[dst] = lin.bias[src]
            lin.bias[17] += 50.0
            lin.bias[4000] += 50.0
            lin.bias[4001] += 50.0  # columns 17, 4000 and 4001 tie at the top: 17 wins
        if case == "zeros":
            lin.weight.zero_()
            lin.bias.copy_(-torch.rand(N, device=device).to(dtype) - 1.0)
            lin.bias[3000] = -0.0
            lin.bias[200] = 0.0  # +0.0 (column 200) and -0.0 (column 3000) tie at the top: 200 wins
        if case == "nan":
            lin.bias[2500] = float("nan")
            lin.bias[4100] = float("nan")  # the first NaN column wins
    x = torch.randn(groups * rows, K, device=device, dtype=dtype)
    idx = torch.tensor([r % rows - (r % 2) * rows for r in range(groups)], dtype=torch.int32, device=device)
    key_buf = torch.full((groups, key_stride), -1, dtype=torch.int64, device=device)
    key_buf[:, 1:] = 7
    keys = key_buf[:, 0]
    print(f"folded argmax dtype={dtype} case={case} key stride={key_stride}", flush=True)
    out = hip_linear.linear_select_rows_hip(x, rows, idx, lin, ln=ln, token_keys=keys)
    plain = hip_linear.linear_select_rows_hip(x, rows, idx, lin, ln=ln)
    assert torch.equal(out, plain) if case != "nan" else torch.equal(out.isnan(), plain.isnan())
    tokens = hip_linear.token_keys_to_tokens(keys).tolist()
    want = torch.argmax(plain.float().cpu(), dim=1).tolist()
    assert tokens == want
    assert bool((key_buf[:, 1:] == 7).all())
    if case == "ties":
        assert want == [17] * groups
    if case == "zeros":
        assert want == [200] * groups
    if case == "nan":
        assert want == [2500] * groups
