"""The HIP-graph cached steps (decode and bucketed prefill chunks) against the eager forward:
same logits within 1e-5, identical block lists and free lists, KV pools within 1e-5, across
batch-size changes, pool growth and eager work and synchronisations between replays."""
import pytest
import torch

from src.cache.paged_kv import BatchedPagedKVCache
from src.model.transformer import TinyTransformerLM

pytestmark = pytest.mark.gpu


def make(device, seed=0):
    torch.manual_seed(seed)
    m = TinyTransformerLM(vocab_size=300, d_model=128, num_heads=2, num_layers=3, d_ff=256, max_seq_len=256,
                          attention_backend="hip_paged", kv_block_size=16, kv_pool_initial_blocks=4,
                          kv_pool_growth_factor=2.0).to(device).eval()
    return m


def stack(caches_per_request, rows):
    layers = len(caches_per_request[0])
    return [BatchedPagedKVCache([caches_per_request[r][l] for r in rows], caches_per_request[rows[0]][l].pool)
            for l in range(layers)]


def test_graph_decode_matches_eager(device, monkeypatch):
    eager, graphed = make(device), make(device)
    graphed.load_state_dict(eager.state_dict())
    B = 3
    prompt = torch.randint(0, 300, (B, 40), device=device)
    lens = torch.tensor([40, 23, 31], device=device)
    per = {}
    with torch.no_grad():
        for name, m in (("eager", eager), ("graph", graphed)):
            _, caches = m(prompt, use_cache=True, position_offset=0, current_lengths=lens)
            per[name] = [[c.states[r] for c in caches] for r in range(B)]
    # chunked prefill steps through graphs (T=40 -> bucket 64, 16, 3 -> bucket 16), then decode
    pos = lens.clone()
    for T, cur in ((40, [40, 17, 40]), (16, [16, 16, 0]), (3, [3, 1, 2])):
        chunk = torch.randint(0, 300, (B, T), device=device)
        outs = {}
        with torch.no_grad():
            for name, m in (("eager", eager), ("graph", graphed)):
                monkeypatch.setenv("PAGED_HIP_GRAPHS", "0" if name == "eager" else "1")
                logits, _ = m(chunk, kv_caches=stack(per[name], [0, 1, 2]), use_cache=True, position_offset=pos,
                              current_lengths=torch.tensor(cur))
                outs[name] = logits
        assert outs["graph"].shape == outs["eager"].shape == (B, T, 300)
        err = (outs["eager"] - outs["graph"]).abs().max().item()
        assert err <= 1e-5, (T, err)
        pos += torch.tensor(cur, device=device)
    rows = [0, 1, 2]
    tok = torch.randint(0, 300, (B, 1), device=device)
    for step in range(60):
        if step == 25:
            rows = [0, 2]  # request 1 leaves the batch: a different batch size / graph
        r = torch.tensor(rows, device=device)
        outs = {}
        with torch.no_grad():
            for name, m in (("eager", eager), ("graph", graphed)):
                monkeypatch.setenv("PAGED_HIP_GRAPHS", "0" if name == "eager" else "1")
                logits, _ = m(tok[r], kv_caches=stack(per[name], rows), use_cache=True, position_offset=pos[r])
                outs[name] = logits
        torch.cuda.synchronize()
        err = (outs["eager"] - outs["graph"]).abs().max().item()
        assert err <= 1e-5, (step, err)
        pos[r] += 1
        tok = torch.randint(0, 300, (B, 1), device=device)  # eager work between replays
        torch.cuda.synchronize()
    runner = graphed._graph_step
    assert runner is not None and runner.captures >= 2, "the graph path was not used"
    for le, lg in zip(eager.layer_block_pools, graphed.layer_block_pools):
        assert le.capacity_blocks == lg.capacity_blocks > 4  # grew during decode
        assert le.free_block_ids == lg.free_block_ids
        # Prefill chunks run padded to their bucket, so the K/V projections are GEMMs of another
        # M and may round differently in the last bits; the scatter itself copies exactly.
        assert torch.allclose(le.k_blocks, lg.k_blocks, rtol=0, atol=1e-5)
        assert torch.allclose(le.v_blocks, lg.v_blocks, rtol=0, atol=1e-5)
    for re_, rg in zip(per["eager"], per["graph"]):
        for se, sg in zip(re_, rg):
            assert se.block_ids == sg.block_ids and se.seq_len == sg.seq_len


def test_graph_decode_bf16_kv_cache_matches_eager(device, monkeypatch):
    """A model whose pools store bf16 KV (kv_cache_dtype) through the fused decode kernels (K/V
    rounded to bf16 by the q/k/v + append launch) against the eager forward (torch projections,
    then the append kernel's rounding): logits within 1e-2 (the two fp32 projections may round a
    K/V element to neighbouring bf16 values)."""
    def build():
        torch.manual_seed(3)
        return TinyTransformerLM(vocab_size=300, d_model=256, num_heads=4, num_layers=2, d_ff=512, max_seq_len=256,
                                 attention_backend="hip_paged", kv_block_size=16, kv_pool_initial_blocks=8,
                                 kv_cache_dtype=torch.bfloat16).to(device).eval()
    eager, graphed = build(), build()
    graphed.load_state_dict(eager.state_dict())
    B = 4
    prompt = torch.randint(0, 300, (B, 30), device=device)
    per = {}
    with torch.no_grad():
        for name, m in (("eager", eager), ("graph", graphed)):
            monkeypatch.setenv("PAGED_HIP_GRAPHS", "0")
            _, caches = m(prompt, use_cache=True, position_offset=0, current_lengths=30)
            per[name] = [[c.states[r] for c in caches] for r in range(B)]
        assert graphed.layer_block_pools[0].k_blocks.dtype == torch.bfloat16
        pos = torch.full((B,), 30, device=device)
        tok = torch.randint(0, 300, (B, 1), device=device)
        for step in range(20):
            outs = {}
            for name, m in (("eager", eager), ("graph", graphed)):
                monkeypatch.setenv("PAGED_HIP_GRAPHS", "0" if name == "eager" else "1")
                logits, _ = m(tok, kv_caches=stack(per[name], list(range(B))), use_cache=True, position_offset=pos)
                outs[name] = logits
            err = (outs["eager"] - outs["graph"]).abs().max().item()
            assert err <= 1e-2, (step, err)
            pos += 1
            tok = torch.randint(0, 300, (B, 1), device=device)
    assert graphed._graph_step is not None and graphed._graph_step.captures >= 1
    assert any(c.fused for c in graphed._graph_step.captured.values()), "the fused decode kernels were not used"


def test_tokens_only_graphs_select_the_greedy_rows(device):
    """greedy_step without logits replays graphs that compute ln_f + lm_head only for each request's
    greedy row (pa_linear_select_rows): the same tokens as the argmax of the full logits of a
    twin model's logits graphs (unless a row's top two logits are within 1e-4), and the same block
    lists, over prefill chunks in several buckets and decode steps."""
    full, sel = make(device, seed=3), make(device, seed=3)
    sel.load_state_dict(full.state_dict())
    B = 3
    per = {}
    for name, m in (("full", full), ("sel", sel)):
        per[name] = m.create_request_kv_caches(B)
    pos = [0, 0, 0]
    steps = [(40, [40, 17, 40]), (100, [100, 64, 3]), (16, [16, 16, 0])] + [(1, [1, 1, 1])] * 20
    ties = 0
    g = torch.Generator().manual_seed(9)
    for T, cur in steps:
        ids = torch.randint(0, 300, (B, T), generator=g)
        with torch.no_grad():
            tf, logits, _ = full.greedy_step(ids, stack(per["full"], [0, 1, 2]), position_offset=list(pos),
                                             current_lengths=cur, return_logits=True)
            ts, none, _ = sel.greedy_step(ids, stack(per["sel"], [0, 1, 2]), position_offset=list(pos),
                                          current_lengths=cur)
        assert none is None
        tf, ts = tf.tolist(), ts.tolist()
        for b in range(B):
            row = logits[b, (cur[b] - 1) % T]
            top2 = torch.topk(row, 2).values
            assert tf[b] == int(torch.argmax(row))
            if (top2[0] - top2[1]).item() < 1e-4:
                ties += 1
            else:
                assert ts[b] == tf[b], (T, b)
        pos = [p + c for p, c in zip(pos, cur)]
    assert ties <= 2
    caps = sel._graph_step.captured
    assert any(not k[2] and c.select_head for k, c in caps.items()), "the row-selecting graphs were not used"
    for rf, rs in zip(per["full"], per["sel"]):
        for a, b in zip(rf, rs):
            assert a.block_ids == b.block_ids and a.seq_len == b.seq_len


def test_dropped_graphs_free_their_descriptors(device, monkeypatch):
    """Graphs dropped for a new storage or mirror release their pinned step descriptors (after
    their last replay); the steps that follow capture again and still match the eager forward."""
    graphed, eager = make(device, seed=5), make(device, seed=5)
    eager.load_state_dict(graphed.state_dict())
    B = 2
    caches = {"graph": graphed.create_request_kv_caches(B), "eager": eager.create_request_kv_caches(B)}
    g = torch.Generator().manual_seed(4)
    pos = torch.zeros(B, dtype=torch.long)
    old = []
    for step, T in enumerate((20, 1, 1, 16, 1, 1)):
        if step == 3:
            runner = graphed._graph_step
            old = list(runner.captured.values())
            assert old and all(c.desc.host_ptr is not None for c in old)
            runner._drop_captures()
            assert not runner.captured and all(c.desc.host_ptr is None and c.graph is None for c in old)
        ids = torch.randint(0, 300, (B, T), generator=g).to(device)
        outs = {}
        with torch.no_grad():
            for name, m in (("eager", eager), ("graph", graphed)):
                monkeypatch.setenv("PAGED_HIP_GRAPHS", "0" if name == "eager" else "1")
                outs[name], _ = m(ids, kv_caches=stack(caches[name], [0, 1]), use_cache=True,
                                  position_offset=pos.to(device), current_lengths=torch.tensor([T] * B))
        assert (outs["eager"] - outs["graph"]).abs().max().item() <= 1e-5, step
        pos += T
    runner = graphed._graph_step
    assert runner.captured and all(c.desc.host_ptr is not None for c in runner.captured.values())


def test_step_descriptors_are_freed_with_the_model(device):
    """Each captured step owns pinned, mapped descriptor words and an event; dropping the model
    without releasing its graphs frees them when the captures are collected."""
    import gc

    from src.kernels.staging import MappedHostWords

    words = MappedHostWords(64, device)
    fin = words._finalizer
    del words
    gc.collect()
    assert not fin.alive

    m = make(device)
    with torch.no_grad():
        assert m.prepare_graphs(2, device) > 0
    fins = [cap.desc._finalizer for cap in m._graph_step.captured.values()]
    assert fins and all(f.alive for f in fins)
    del m
    gc.collect()
    torch.cuda.synchronize()
    assert not any(f.alive for f in fins)
