"""The ctypes binding a maintainer of the reference would add (the "Option B" Python block of the
integration guide at the repository root, read from that file) is executed verbatim and checked
against the oracle, so the published binding stays correct."""
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from src import workloads
from src.kernels import _lib

pytestmark = pytest.mark.gpu
DOC = Path(__file__).resolve().parents[1] / "INTEGRATION.md"


def load_stub():
    text = DOC.read_text()
    block = re.search(r"## Option B.*?```python\n(.*?)```", text, re.S).group(1)
    block = block.replace('"/path/to/libpaged_hip.so"', repr(str(_lib.LIB_PATH)))
    ns = {}
    exec(compile(block, str(DOC), "exec"), ns)
    return ns["paged_attention_hip"]


def test_integration_stub_decode_and_prefill(device):
    fn = load_stub()
    b = workloads.ragged_decode(seed=3, layer=0, device=device)
    got = fn(b.q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, b.cur_lens_t)
    want = oracle.paged_attention(b.q.cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens, b.cur_lens)
    assert np.abs(got.cpu().numpy() - want).max() <= 1e-4
    q = torch.randn(b.batch, 8, 5, 64, device=device)
    cur = torch.full((b.batch,), 5, dtype=torch.int32, device=device)
    got = fn(q, b.k_pool, b.v_pool, b.page_table, b.seq_lens_t, cur)
    want = oracle.paged_attention(q.cpu(), b.k_pool.cpu(), b.v_pool.cpu(), b.block_lists, b.seq_lens, [5] * b.batch)
    assert np.abs(got.cpu().numpy() - want).max() <= 1e-4
