"""Host-side pieces of bench.py: the attended-pair count that scales the reference loop's sample,
the CPU timing helper on a tiny case, and the one-GPU refusal."""
import subprocess
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, str(REPO / "efficient-inference-system_amd"))

import bench  # noqa: E402
from src import workloads  # noqa: E402


def _brute_pairs(seq_lens, cur_lens, T):
    # the reference loop's own break rule (src/kernels/reference_paged_attention.py:36-42): key t is visited
    # while t <= L - C + i
    n = 0
    for L, C in zip(seq_lens, cur_lens):
        for i in range(T):
            for t in range(L):
                if t > L - C + i:
                    break
                n += 1
    return n


@pytest.mark.parametrize("case", [
    ([128], [1], 1),
    ([300, 17, 1024], [1, 1, 1], 1),
    ([176 + 256, 608 + 128], [256, 128], 256),   # the second request has 128 padded rows
    ([5, 40], [5, 3], 8),
])
def test_attended_pairs(case):
    seq_lens, cur_lens, T = case
    assert bench._attended(seq_lens, cur_lens, T) == _brute_pairs(seq_lens, cur_lens, T)


def test_attended_pairs_closed_forms():
    lens = [128, 700, 1024]
    assert bench._attended(lens, [1, 1, 1], 1) == sum(lens)
    ctx, chunk = [176, 608, 672, 368], [256] * 4
    # unpadded causal prefill: C*ctx + C(C+1)/2 pairs per request, the useful-FLOP count / (4 H Hd)
    assert bench._attended([a + c for a, c in zip(ctx, chunk)], chunk, 256) \
        == workloads.prefill_flops(ctx, chunk, 1, 1) // 4


def test_cpu_call_times_single_decode():
    b = workloads.single_decode(seed=0, device="cpu")
    r = bench.cpu_call_times(b.q, b.k_pool, b.v_pool, b.block_lists, b.seq_lens, b.cur_lens)
    assert r["oracle_ms"] > 0 and r["reference_loop_ms"] > 0 and r["threads"] >= 1
    assert r["reference_loop_sample"] == "the whole call"


def test_bench_refuses_more_than_one_gpu():
    p = subprocess.run([sys.executable, str(REPO / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 2
    assert "one GPU" in p.stderr


def test_token_agreement_counts():
    a = {0: [5, 6, 7], 1: [1, 2, 3, 4], 2: [9]}
    b = {0: [5, 6, 7], 1: [1, 2, 8, 8], 2: [9]}
    r = bench.token_agreement(a, b)
    assert r == {"requests": 3, "requests_identical": 2, "tokens": 8, "tokens_equal": 6,
                 "first_difference_positions": [2]}
    assert bench.token_agreement(a, a)["requests_identical"] == 3
    # a request missing from the second run counts as different from its first token
    assert bench.token_agreement({3: [1, 2]}, {})["first_difference_positions"] == [0]


@pytest.mark.parametrize("prev,chunks,T", [([704, 384, 736, 480], [128, 256, 128, 256], 256),
                                          ([0, 16], [5, 32], 32), ([176, 608], [256, 256], 256)])
def test_prefill_flops_with_padding(prev, chunks, T):
    """4 * H * Hd FLOPs per attended (row, key) pair over every row of the padded batch: the
    brute-force count of the reference loop's visited pairs; equal to the useful count when no
    row is padded."""
    want = 4 * 8 * 64 * _brute_pairs([p + c for p, c in zip(prev, chunks)], chunks, T)
    assert workloads.prefill_flops_with_padding(prev, chunks, T, 8, 64) == want
    if all(c == T for c in chunks):
        assert want == workloads.prefill_flops(prev, chunks, 8, 64)
