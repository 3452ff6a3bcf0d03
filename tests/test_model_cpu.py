"""Model-level behaviour on the CPU with the torch backend: the reference's CPU tests
(tests/test_paged_attention.py:42-55 of the reference), backend validation, and the product's
"paged_reference" backend checked against the oracle."""
import numpy as np
import pytest
import torch

import oracle
from src.cache.paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState
from src.config import ModelConfig
from src.inference.generate_with_cache import generate_with_cache
from src.kernels.paged_attention import paged_attention
from src.model.transformer import TinyTransformerLM


def build_tiny_model(backend_name: str, device: str) -> TinyTransformerLM:
    cfg = ModelConfig(vocab_size=128, d_model=64, num_heads=4, num_layers=2, d_ff=128, max_seq_len=128,
                      attention_backend=backend_name, kv_block_size=8, kv_pool_initial_blocks=8,
                      kv_pool_growth_factor=2.0)
    model = TinyTransformerLM(
        vocab_size=cfg.vocab_size, d_model=cfg.d_model, num_heads=cfg.num_heads, num_layers=cfg.num_layers,
        d_ff=cfg.d_ff, max_seq_len=cfg.max_seq_len, dropout=cfg.dropout, attention_backend=cfg.attention_backend,
        kv_block_size=cfg.kv_block_size, kv_pool_initial_blocks=cfg.kv_pool_initial_blocks,
        kv_pool_growth_factor=cfg.kv_pool_growth_factor,
        enable_attention_correctness_checks=cfg.enable_attention_correctness_checks,
    ).to(device)
    model.eval()
    return model


def test_chunked_prefill_then_decode_runs():
    model = build_tiny_model("paged_reference", "cpu")
    prompt = torch.randint(0, 128, (2, 24))
    result = generate_with_cache(model, prompt, max_new_tokens=[3, 4])
    assert result["generated_tokens_per_request"] == [3, 4]
    assert result["reserved_kv_bytes"] > 0


def test_reference_shapes_match_single_and_batched():
    prompt = torch.randint(0, 128, (2, 16))
    model = build_tiny_model("paged_reference", "cpu")
    paged = generate_with_cache(model, prompt, max_new_tokens=[2, 2])
    assert len(paged["generated_ids"]) == 2
    for ids in paged["generated_ids"]:
        assert len(tuple(ids.shape)) == 1


def test_unknown_backend_rejected_everywhere():
    with pytest.raises(ValueError):
        build_tiny_model("triton_paged", "cpu")
    model = build_tiny_model("paged_reference", "cpu")
    with pytest.raises(ValueError):
        model.set_attention_backend("nope")
    pool = LayerBlockPool(4, 4, 2.0)
    with pytest.raises(ValueError):
        paged_attention("nope", torch.zeros(1, 1, 1, 4), BatchedPagedKVCache([PagedKVCacheState(pool)], pool), None)


def test_hip_backend_refuses_cpu_tensors():
    model = build_tiny_model("hip_paged", "cpu")
    with pytest.raises(ValueError, match="HIP device"):
        generate_with_cache(model, torch.randint(0, 128, (1, 8)), max_new_tokens=[1])


@pytest.mark.parametrize("T,curs", [(1, [1, 1, 1]), (6, [6, 2, 0]), (3, [3, 3, 5])])
def test_torch_backend_matches_oracle(T, curs):
    g = torch.Generator().manual_seed(21)
    H, Hd, bs = 2, 8, 4
    pool = LayerBlockPool(block_size=bs, initial_blocks=4, growth_factor=2.0)
    states = [PagedKVCacheState(pool=pool) for _ in range(3)]
    batch = BatchedPagedKVCache(states=states, pool=pool)
    batch.append_batch(torch.randn(3, H, 9, Hd, generator=g), torch.randn(3, H, 9, Hd, generator=g),
                       current_lengths=torch.tensor([9, 4, 7]))
    batch.append_batch(torch.randn(3, H, T, Hd, generator=g), torch.randn(3, H, T, Hd, generator=g),
                       current_lengths=torch.tensor(curs))
    q = torch.randn(3, H, T, Hd, generator=g)
    got = paged_attention("paged_reference", q, batch, torch.tensor(curs)).numpy()
    want = oracle.paged_attention(q, pool.k_blocks, pool.v_blocks, [s.block_ids for s in states],
                                  [s.seq_len for s in states], curs)
    np.testing.assert_allclose(got, want, atol=2e-6, rtol=0)


def test_state_dict_names_match_reference_layout():
    model = build_tiny_model("paged_reference", "cpu")
    keys = set(model.state_dict())
    for name in ("token_emb.weight", "pos_emb.weight", "blocks.0.ln1.weight", "blocks.0.attn.q_proj.weight",
                 "blocks.0.attn.out_proj.bias", "blocks.1.mlp.0.weight", "blocks.1.mlp.2.bias", "ln_f.bias",
                 "lm_head.weight"):
        assert name in keys
    assert "lm_head.bias" not in keys


@pytest.mark.parametrize("native", [True, False])
def test_token_and_position_checks(native, monkeypatch):
    """check_token_inputs raises IndexError exactly where the eager embedding lookups would, for
    the native host check and the Python one."""
    import numpy as np

    import src.model.transformer as tr

    if not native:
        monkeypatch.setattr(tr, "_host", None)
    elif tr._host is None:
        pytest.skip("native host module not built")
    model = build_tiny_model("paged_reference", "cpu")  # vocab 128, max_seq_len 128
    ok_ids = np.array([[0, 127], [5, 6]], dtype=np.int64)
    model.check_token_inputs(ok_ids, 0, 2)
    model.check_token_inputs(ok_ids, [0, 126], 2)
    model.check_token_inputs([[1], [2]], [10, 127], 1)
    model.check_token_inputs(np.array([[3]], dtype=np.int32), np.array([5], dtype=np.int32), 1)
    for ids, pos, T in ((np.array([[128]]), 0, 1), ([[-1]], 0, 1), (ok_ids, [0, 127], 2), (ok_ids, -1, 2),
                        ([[1]], np.array([128], dtype=np.int64), 1)):
        with pytest.raises(IndexError):
            model.check_token_inputs(ids, pos, T)
        with pytest.raises(IndexError):  # eager lookups agree
            ids_t = torch.as_tensor(np.asarray(ids), dtype=torch.long)
            p = torch.as_tensor(np.asarray(pos), dtype=torch.long).view(-1, 1) + torch.arange(T).view(1, T)
            model.token_emb(ids_t) + model.pos_emb(p.expand(ids_t.shape[0], T))
