"""Pins of the oracle (oracle/paged_oracle.c) before it is trusted to check the HIP kernels.

The reference ships no golden vectors for its attention op, so the oracle is pinned by:
  1. closed form: softmax(Q K^T / sqrt(d) + mask) V on the dense K/V gathered with torch indexing,
     computed by torch.nn.functional.scaled_dot_product_attention in float64, with the reference's
     mask (key t allowed for row i iff t < L and t <= L - C + i);
  2. invariants: physical block relabelling, single key -> its value row, identical keys -> mean of
     V, empty rows -> zeros, decode == last row of the matching prefill, padded rows i >= C attend
     every cached key;
  3. the reference's literal per-token loop (oracle/reference_loop.py) on tiny shapes;
  4. planted mistakes: each `mutation` of the oracle must fail check 1.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle
from oracle.reference_loop import paged_attention_loop


def _case(seed, B, H, T, Hd, bs, lens, curs, pool_blocks=None, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    need = sum(math.ceil(L / bs) for L in lens)
    N = pool_blocks or need + 5
    perm = torch.randperm(N, generator=g).tolist()
    lists, pos = [], 0
    for L in lens:
        n = math.ceil(L / bs)
        lists.append(perm[pos:pos + n])
        pos += n
    q = torch.randn(B, H, T, Hd, generator=g)
    k = torch.randn(N, H, bs, Hd, generator=g).to(dtype)
    v = torch.randn(N, H, bs, Hd, generator=g).to(dtype)
    return q, k, v, lists, list(lens), list(curs)


def closed_form(q, k, v, lists, lens, curs):
    """Dense gather + SDPA in float64 (independent of the oracle's code)."""
    B, H, T, Hd = q.shape
    bs = k.shape[2]
    out = torch.zeros(B, H, T, Hd, dtype=torch.float64)
    for b in range(B):
        L, C = lens[b], curs[b]
        if L == 0:
            continue
        pos = torch.arange(L)
        blocks = torch.tensor(lists[b], dtype=torch.long)[pos // bs]
        kd = k.double()[blocks, :, pos % bs, :].permute(1, 0, 2)  # [H, L, Hd]
        vd = v.double()[blocks, :, pos % bs, :].permute(1, 0, 2)
        rows = torch.arange(T).view(T, 1)
        allowed = pos.view(1, L) <= (L - C + rows)
        has = allowed.any(dim=1)
        o = F.scaled_dot_product_attention(q[b].double(), kd, vd, attn_mask=allowed)
        out[b] = torch.where(has.view(1, T, 1), o, torch.zeros_like(o))
    return out.numpy()


CASES = [
    # (seed, B, H, T, Hd, bs, lens, curs)
    (1, 1, 8, 1, 64, 16, [128], [1]),
    (2, 3, 2, 1, 16, 8, [1, 37, 64], [1, 1, 1]),
    (3, 2, 2, 7, 8, 4, [13, 7], [7, 3]),          # prefill with a padded row set (C < T)
    (4, 2, 3, 5, 8, 4, [5, 20], [5, 5]),          # chunk == whole sequence / with context
    (5, 3, 1, 4, 8, 4, [6, 6, 6], [0, 9, 2]),      # C = 0, C > L (empty rows), C < T
    (6, 2, 2, 1, 32, 16, [0, 17], [1, 1]),         # empty request
]


@pytest.mark.parametrize("case", CASES)
def test_oracle_matches_closed_form(case):
    q, k, v, lists, lens, curs = _case(*case)
    got = oracle.paged_attention(q, k, v, lists, lens, curs)
    want = closed_form(q, k, v, lists, lens, curs)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


@pytest.mark.parametrize("case", CASES[:5])
def test_oracle_matches_reference_loop(case):
    q, k, v, lists, lens, curs = _case(*case)
    got = oracle.paged_attention(q, k, v, lists, lens, curs)
    want = paged_attention_loop(q, k, v, lists, lens, curs).numpy()
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-5)


@pytest.mark.parametrize("mutation", [1, 2, 3, 4])
def test_planted_mistakes_are_caught(mutation):
    q, k, v, lists, lens, curs = _case(7, 2, 2, 6, 8, 4, [23, 10], [6, 4])
    want = closed_form(q, k, v, lists, lens, curs)
    got = oracle.paged_attention(q, k, v, lists, lens, curs, mutation=mutation)
    assert np.abs(got - want).max() > 1e-3


def test_block_relabelling_invariance():
    q, k, v, lists, lens, curs = _case(8, 2, 2, 3, 8, 4, [30, 11], [3, 2])
    base = oracle.paged_attention(q, k, v, lists, lens, curs)
    N = k.shape[0]
    perm = torch.randperm(N, generator=torch.Generator().manual_seed(9))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(N)
    k2, v2 = k[perm], v[perm]  # physical block j of k2 is old block perm[j]
    lists2 = [[int(inv[i]) for i in row] for row in lists]
    np.testing.assert_array_equal(oracle.paged_attention(q, k2, v2, lists2, lens, curs), base)


def test_single_key_returns_value_row():
    q, k, v, lists, lens, curs = _case(10, 1, 4, 1, 16, 8, [1], [1])
    got = oracle.paged_attention(q, k, v, lists, lens, curs)
    np.testing.assert_allclose(got[0, :, 0, :], v[lists[0][0], :, 0, :].numpy(), atol=0, rtol=0)


def test_identical_keys_give_mean_of_values():
    q, k, v, lists, lens, curs = _case(11, 1, 2, 1, 8, 4, [10], [1])
    k[:] = k[lists[0][0], :, 0:1, :]
    got = oracle.paged_attention(q, k, v, lists, lens, curs)
    pos = torch.arange(10)
    blocks = torch.tensor(lists[0])[pos // 4]
    mean_v = v[blocks, :, pos % 4, :].double().mean(dim=0).numpy()
    np.testing.assert_allclose(got[0, :, 0, :], mean_v, atol=1e-6)


def test_decode_equals_last_prefill_row_and_padded_rows_see_all_keys():
    q, k, v, lists, lens, curs = _case(12, 2, 2, 6, 8, 4, [25, 14], [4, 6])
    pre = oracle.paged_attention(q, k, v, lists, lens, curs)
    for b, C in enumerate(curs):
        dec = oracle.paged_attention(q[b:b + 1, :, C - 1:C], k, v, [lists[b]], [lens[b]], [1])
        np.testing.assert_allclose(pre[b:b + 1, :, C - 1:C], dec, atol=1e-6)
        # a padded row (i >= C) attends every cached key: same as a decode query with C = 1
        for i in range(C, q.shape[2]):
            full = oracle.paged_attention(q[b:b + 1, :, i:i + 1], k, v, [lists[b]], [lens[b]], [1])
            np.testing.assert_allclose(pre[b:b + 1, :, i:i + 1], full, atol=1e-6)


def test_bf16_pool_equals_upcast_pool():
    q, k, v, lists, lens, curs = _case(13, 2, 2, 1, 16, 8, [40, 9], [1, 1], dtype=torch.bfloat16)
    got = oracle.paged_attention(q, k, v, lists, lens, curs)
    want = oracle.paged_attention(q, k.float(), v.float(), lists, lens, curs)
    np.testing.assert_array_equal(got, want)


def test_bf16_rounding_matches_torch():
    x = torch.randn(4096, generator=torch.Generator().manual_seed(14)) * 100
    x[:4] = torch.tensor([1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, -2.5, 0.0])  # ties round to even
    bits = oracle.f32_to_bf16_bits(x)
    np.testing.assert_array_equal(bits, x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))


def test_missing_block_is_an_error():
    q, k, v, lists, lens, curs = _case(15, 1, 1, 1, 8, 4, [9], [1])
    with pytest.raises(IndexError):
        oracle.paged_attention(q, k, v, [lists[0][:1]], lens, curs)
