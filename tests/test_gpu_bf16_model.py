"""The decoder with bf16 weights and activations (model.to(torch.bfloat16)) on the "hip_paged"
backend: bf16 q/out through the attention kernels, bf16 KV pools, bf16 matrix-core GEMMs.
Graph-replayed steps (decode steps and short chunks through the fused bf16 decode-step kernels)
and eager steps of the same model (torch layers) against the "paged_reference" backend of the
same bf16 model, teacher-forced on the same tokens (within 0.03: the fused kernels round once per
layer output where torch rounds after every op), and against the fp32 model on the same weights
(bf16 rounding of every activation: logits within 0.05, most greedy tokens equal)."""
import pytest
import torch

from src.cache.paged_kv import BatchedPagedKVCache
from src.model.transformer import TinyTransformerLM

pytestmark = pytest.mark.gpu


def build(device, seed=5):
    torch.manual_seed(seed)
    m = TinyTransformerLM(vocab_size=300, d_model=256, num_heads=4, num_layers=3, d_ff=512, max_seq_len=256,
                          attention_backend="hip_paged", kv_block_size=16, kv_pool_initial_blocks=8).to(device).eval()
    with torch.no_grad():
        for mod in m.modules():
            if isinstance(mod, (torch.nn.Linear, torch.nn.Embedding)):
                mod.weight.normal_(0.0, 0.02)
    return m


def stack(caches_per_request, rows):
    layers = len(caches_per_request[0])
    return [BatchedPagedKVCache([caches_per_request[r][l] for r in rows], caches_per_request[rows[0]][l].pool)
            for l in range(layers)]


def run(m, prompt, lens, steps, monkeypatch, graphs):
    """Prefill, a second (bucketed) chunk, then decode steps on a fixed token sequence (the same for
    every model compared, so a near-tie argmax cannot send two models down different paths);
    returns the logits of every step."""
    B = prompt.shape[0]
    monkeypatch.setenv("PAGED_HIP_GRAPHS", "1" if graphs else "0")
    out = []
    with torch.no_grad():
        logits, caches = m(prompt, use_cache=True, position_offset=0, current_lengths=lens)
        out.append(logits.float())
        per = [[c.states[r] for c in caches] for r in range(B)]
        pos = lens.clone()
        chunk = torch.randint(0, 300, (B, 20), generator=torch.Generator().manual_seed(1)).to(prompt.device)
        logits, _ = m(chunk, kv_caches=stack(per, list(range(B))), use_cache=True, position_offset=pos,
                      current_lengths=torch.tensor([20] * B))
        out.append(logits.float())
        pos += 20
        toks = torch.randint(0, 300, (steps, B, 1), generator=torch.Generator().manual_seed(3)).to(prompt.device)
        for i in range(steps):
            logits, _ = m(toks[i], kv_caches=stack(per, list(range(B))), use_cache=True, position_offset=pos)
            out.append(logits.float())
            pos += 1
    return out


def test_bf16_model_graph_matches_eager_and_fp32(device, monkeypatch):
    B = 3
    prompt = torch.randint(0, 300, (B, 37), generator=torch.Generator().manual_seed(2)).to(device)
    lens = torch.tensor([37, 25, 30], device=device)
    ref32 = build(device)
    ref32.set_attention_backend("paged_reference")
    ref16 = build(device).to(torch.bfloat16)
    ref16.set_attention_backend("paged_reference")
    eager16 = build(device).to(torch.bfloat16)
    graph16 = build(device).to(torch.bfloat16)
    print("bf16 model: fp32 and bf16 paged_reference, bf16 hip_paged eager and graphs", flush=True)
    want = run(ref32, prompt, lens, 12, monkeypatch, graphs=False)
    r16 = run(ref16, prompt, lens, 12, monkeypatch, graphs=False)
    e16 = run(eager16, prompt, lens, 12, monkeypatch, graphs=False)
    g16 = run(graph16, prompt, lens, 12, monkeypatch, graphs=True)
    # the torch backend of the same bf16 model, teacher-forced on the same tokens
    for i, (r, e, g) in enumerate(zip(r16, e16, g16)):
        assert (e - r).abs().max().item() <= 3e-2, ("eager", i)
        assert (g - r).abs().max().item() <= 3e-2, ("graph", i)
    assert eager16.layer_block_pools[0].k_blocks.dtype == torch.bfloat16
    assert graph16._graph_step is not None and graph16._graph_step.captures >= 2, "the graph path was not used"
    assert any(c.fused for c in graph16._graph_step.captured.values()), "the bf16 fused kernels were not used"
    agree = total = 0
    for i, (w, e, g) in enumerate(zip(want, e16, g16)):
        # the fused kernels round once per layer output where the torch layers round after the
        # LayerNorm, the product, the activation and the residual: a few bf16 ulps per layer
        assert (e - g).abs().max().item() <= 3e-2, i
        err = (e - w).abs().max().item()
        assert err <= 5e-2, (i, err)
        agree += int((e[:, -1].argmax(-1) == w[:, -1].argmax(-1)).sum())
        total += B
    print(f"  argmax of the last position equal to the fp32 model's: {agree}/{total}", flush=True)
    assert agree >= 0.8 * total
