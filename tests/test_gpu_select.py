"""pa_argmax_rows (greedy token selection on the device) against torch.argmax on the CPU: exact
indices, including ties (first index), NaN (the first NaN wins), all -inf rows, -0.0 against 0.0,
bf16 logits, negative row indices and vocabularies smaller and larger than the workgroup."""
import pytest
import torch

from src.kernels.hip_paged_attention import argmax_rows_hip

pytestmark = pytest.mark.gpu


def want(logits, rows):
    B, T, _ = logits.shape
    return torch.stack([torch.argmax(logits[b, rows[b] % T].float()) for b in range(B)])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,T,V", [(1, 1, 5000), (8, 1, 5000), (4, 256, 5000), (3, 7, 100), (2, 3, 1), (5, 2, 1025)])
def test_argmax_rows_matches_torch(device, dtype, B, T, V):
    g = torch.Generator().manual_seed(B * 1000 + T * 10 + V)
    logits = torch.randn(B, T, V, generator=g).to(dtype)
    rows = torch.randint(-T, T, (B,), generator=g, dtype=torch.int32)
    got = argmax_rows_hip(logits.to(device), rows.to(device))
    assert got.cpu().tolist() == want(logits, rows.tolist()).tolist()


def test_argmax_rows_special_values(device):
    V = 3000
    rows = []
    r = torch.zeros(V)
    r[[17, 900, 2999]] = 5.0  # ties: first index
    rows.append(r)
    r = torch.full((V,), -float("inf"))  # all -inf: index 0
    rows.append(r)
    r = torch.randn(V, generator=torch.Generator().manual_seed(3))
    r[[1500, 40]] = float("nan")  # NaN above every number: the first NaN
    rows.append(r)
    r = torch.full((V,), -1.0)
    r[7] = -0.0
    r[5] = 0.0  # -0.0 == 0.0: the first of the two
    rows.append(r)
    r = torch.full((V,), -3.0)
    r[V - 1] = float("inf")
    rows.append(r)
    logits = torch.stack(rows).view(len(rows), 1, V)
    got = argmax_rows_hip(logits.to(device), None).cpu().tolist()
    assert got == [torch.argmax(x).item() for x in rows] == [17, 0, 40, 5, V - 1]


def test_argmax_rows_rejects_bad_layouts(device):
    logits = torch.randn(2, 4, 64, device=device)
    with pytest.raises(ValueError):
        argmax_rows_hip(logits.transpose(1, 2), None)
    with pytest.raises(ValueError):
        argmax_rows_hip(logits, torch.zeros(2, dtype=torch.int64, device=device))
