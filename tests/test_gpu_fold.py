"""The folded decode-step launches against float64 references: pa_mlp_rows (LayerNorm + fc1 +
GELU + fc2 + residual of at most 16 rows, accumulated with atomic adds) and pa_linear_rows writing
its rows a second time over its residual; then whole graph steps of the model folded (four
launches per layer) against the same steps unfolded (five launches) and against the eager
forward."""
import pytest
import torch
import torch.nn as nn

from src.cache.paged_kv import BatchedPagedKVCache
from src.kernels import hip_linear
from src.model.transformer import TinyTransformerLM

pytestmark = pytest.mark.gpu


def ref_mlp(x, ln, fc1, fc2, residual):
    x = x.double().cpu()
    h = nn.functional.layer_norm(x, (x.shape[1],), ln.weight.double().cpu(), ln.bias.double().cpu(), ln.eps)
    h = nn.functional.gelu(h @ fc1.weight.double().cpu().t() + fc1.bias.double().cpu())
    y = h @ fc2.weight.double().cpu().t() + fc2.bias.double().cpu()
    return y + residual.double().cpu() if residual is not None else y


@pytest.mark.parametrize("d,ff", [(512, 2048), (128, 256), (256, 512)])
@pytest.mark.parametrize("M", [1, 3, 8, 16])
def test_mlp_rows(device, d, ff, M):
    torch.manual_seed(d + ff + M)
    ln = nn.LayerNorm(d).to(device)
    fc1, fc2 = nn.Linear(d, ff).to(device), nn.Linear(ff, d).to(device)
    with torch.no_grad():
        ln.weight.normal_(1.0, 0.1)
        ln.bias.normal_(0.0, 0.1)
    x = torch.randn(M, d, device=device) * 2 + 0.3
    out = torch.zeros(M, d, device=device)
    print(f"mlp rows d={d} ff={ff} M={M}", flush=True)
    hip_linear.mlp_rows_hip(x, ln, fc1, fc2, out, residual=x)
    err = (out.double().cpu() - ref_mlp(x, ln, fc1, fc2, x)).abs().max().item()
    assert err <= 5e-5, err
    # without residual, into a strided, pre-zeroed slice: rows past M stay untouched
    big = torch.full((M + 2, d + 16), 7.0, device=device)
    big[:M, :d] = 0
    hip_linear.mlp_rows_hip(x, ln, fc1, fc2, big[:M, :d])
    assert (big[M:] == 7.0).all() and (big[:, d:] == 7.0).all()
    assert (big[:M, :d].double().cpu() - ref_mlp(x, ln, fc1, fc2, None)).abs().max().item() <= 5e-5


def test_mlp_rows_rejects_bad_arguments(device):
    ln, fc1, fc2 = nn.LayerNorm(512).to(device), nn.Linear(512, 2048).to(device), nn.Linear(2048, 512).to(device)
    out = torch.zeros(17, 512, device=device)
    with pytest.raises(ValueError):
        hip_linear.mlp_rows_hip(torch.randn(17, 512, device=device), ln, fc1, fc2, out)  # more than 16 rows
    with pytest.raises(ValueError):
        hip_linear.mlp_rows_hip(torch.randn(2, 512, device=device).bfloat16(), ln, fc1, fc2, out)  # fp32 only


def test_linear_rows_copy_to_residual_in_place(device):
    """out_proj's launch in a folded step writes x1 = x + o W^T + b to a buffer and back over its
    residual x (each element read and written by one thread)."""
    torch.manual_seed(4)
    proj = nn.Linear(512, 512).to(device)
    o = torch.randn(7, 512, device=device)
    x = torch.randn(7, 512, device=device)
    want = (o.double().cpu() @ proj.weight.double().cpu().t() + proj.bias.double().cpu() + x.double().cpu())
    x1 = torch.empty_like(x)
    hip_linear.linear_rows_hip(o, proj, residual=x, out=x1, copy_to=x)
    assert torch.equal(x1, x)
    assert (x1.double().cpu() - want).abs().max().item() <= 2e-5


def _model(device, d=128, heads=2, layers=3, ff=256, seed=0):
    torch.manual_seed(seed)
    return TinyTransformerLM(vocab_size=300, d_model=d, num_heads=heads, num_layers=layers, d_ff=ff, max_seq_len=256,
                             attention_backend="hip_paged", kv_block_size=16, kv_pool_initial_blocks=4,
                             kv_pool_growth_factor=2.0).to(device).eval()


@pytest.mark.parametrize("d,heads,ff", [(128, 2, 256), (512, 8, 2048)])
def test_folded_decode_steps_match_unfolded_and_eager(device, monkeypatch, d, heads, ff):
    """The same prompts, a 16-row chunk and decode steps through three models with equal weights:
    graphs with folded layers, graphs with five launches per layer, and the eager forward; logits
    within 1e-5 and identical block lists at every step, over batch-size changes and pool growth."""
    models = {name: _model(device, d, heads, 3, ff) for name in ("fold", "five", "eager")}
    for m in models.values():
        m.load_state_dict(models["fold"].state_dict())
    B = 5
    g = torch.Generator().manual_seed(3)
    prompt = torch.randint(0, 300, (B, 37), generator=g).to(device)
    lens = torch.tensor([37, 20, 33, 5, 29], device=device)
    states = {}
    with torch.no_grad():
        for name, m in models.items():
            _, caches = m(prompt, use_cache=True, position_offset=0, current_lengths=lens)
            states[name] = [[c.states[r] for c in caches] for r in range(B)]
    pos = lens.clone()
    # one prefill chunk of 3 tokens for a single request: a 16-row step (bucket 16), folded too
    chunk = torch.randint(0, 300, (1, 3), generator=g).to(device)
    outs = {}
    for name, m in models.items():
        monkeypatch.setenv("PAGED_HIP_GRAPHS", "0" if name == "eager" else "1")
        monkeypatch.setenv("PAGED_HIP_DECODE_FOLD", "0" if name == "five" else "1")
        caches = [BatchedPagedKVCache([states[name][1][l]], states[name][1][l].pool) for l in range(3)]
        with torch.no_grad():
            outs[name], _ = m(chunk, kv_caches=caches, use_cache=True, position_offset=pos[1:2],
                              current_lengths=torch.tensor([3]))
    for other in ("five", "eager"):
        assert (outs["fold"] - outs[other]).abs().max().item() <= 1e-5, other
    pos[1] += 3
    rows = list(range(B))
    for step in range(40):
        if step == 15:
            rows = [0, 2, 4]
        tok = torch.randint(0, 300, (len(rows), 1), generator=g).to(device)
        outs = {}
        for name, m in models.items():
            monkeypatch.setenv("PAGED_HIP_GRAPHS", "0" if name == "eager" else "1")
            monkeypatch.setenv("PAGED_HIP_DECODE_FOLD", "0" if name == "five" else "1")
            caches = [BatchedPagedKVCache([states[name][r][l] for r in rows], states[name][rows[0]][l].pool)
                      for l in range(3)]
            with torch.no_grad():
                logits, _ = m(tok, kv_caches=caches, use_cache=True, position_offset=pos[rows],
                              current_lengths=torch.ones(len(rows), dtype=torch.long))
            outs[name] = logits
        for other in ("five", "eager"):
            err = (outs["fold"] - outs[other]).abs().max().item()
            assert err <= 1e-5, (step, other, err)
        for r in rows:
            for l in range(3):
                assert states["fold"][r][l].block_ids == states["eager"][r][l].block_ids
        pos[rows] += 1
    caps = models["fold"]._graph_step.captured
    assert all(c.folded for (Bk, Tb, _), c in caps.items()) and any(Tb == 16 for (Bk, Tb, _) in caps)
    assert not any(c.folded for c in models["five"]._graph_step.captured.values())
