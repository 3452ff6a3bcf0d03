"""Model-level parity of the hip_paged backend with the torch backend on the GPU: the reference's
only backend-parity test (token equality, tests/test_paged_attention.py:57-66 of the reference),
plus teacher-forced logits, since greedy tokens of a random-init model are fragile to 1e-6 noise."""
import pytest
import torch

from src.inference.generate_with_cache import generate_with_cache
from src.model.transformer import TinyTransformerLM

pytestmark = pytest.mark.gpu


def tiny_model(backend, device):
    m = TinyTransformerLM(vocab_size=128, d_model=64, num_heads=4, num_layers=2, d_ff=128, max_seq_len=128,
                          attention_backend=backend, kv_block_size=8, kv_pool_initial_blocks=8,
                          kv_pool_growth_factor=2.0).to(device)
    return m.eval()


def test_reference_and_hip_agree_on_small_case(device):
    torch.manual_seed(0)
    prompt = torch.randint(0, 128, (2, 16), device=device)
    ref_model = tiny_model("paged_reference", device)
    hip_model = tiny_model("hip_paged", device)
    hip_model.load_state_dict(ref_model.state_dict())
    ref = generate_with_cache(ref_model, prompt, max_new_tokens=[2, 2])
    hip = generate_with_cache(hip_model, prompt, max_new_tokens=[2, 2])
    for a, b in zip(ref["generated_ids"], hip["generated_ids"]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("kv_block_size,d_model,heads", [(8, 64, 4), (16, 512, 8)])
def test_teacher_forced_logits_match(device, kv_block_size, d_model, heads):
    torch.manual_seed(1)
    models = {}
    for backend in ("paged_reference", "hip_paged"):
        models[backend] = TinyTransformerLM(vocab_size=500, d_model=d_model, num_heads=heads, num_layers=3,
                                            d_ff=4 * d_model, max_seq_len=256, attention_backend=backend,
                                            kv_block_size=kv_block_size, kv_pool_initial_blocks=4).to(device).eval()
    models["hip_paged"].load_state_dict(models["paged_reference"].state_dict())
    B = 3
    prompt = torch.randint(0, 500, (B, 50), device=device)
    lens = torch.tensor([50, 37, 12], device=device)
    decode_tokens = torch.randint(0, 500, (B, 6), device=device)
    outs = {}
    with torch.no_grad():
        for name, m in models.items():
            logits, caches = m(prompt, use_cache=True, position_offset=0, current_lengths=lens)
            steps = [logits[torch.arange(B, device=device), lens - 1]]
            for s in range(decode_tokens.shape[1]):
                logits, caches = m(decode_tokens[:, s:s + 1], kv_caches=caches, use_cache=True,
                                   position_offset=lens + s, current_lengths=1)
                steps.append(logits[:, -1])
            outs[name] = torch.stack(steps)
    err = (outs["hip_paged"] - outs["paged_reference"]).abs().max().item()
    print(f"teacher-forced logits max err {err:.2e}", flush=True)
    assert err <= 1e-4
