"""The native host bookkeeping of graph steps (csrc/host/paged_host.cpp) against the Python code it
replaces: graph_decode._lockstep_py, BatchedPagedKVCache.host_append and .csr_buffer. Same
results, same pool mutations (LIFO ids, growth, mutation counter), same errors, no leaked
references."""
import copy
import random
import tracemalloc

import numpy as np
import pytest
import torch

from src.cache.paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState
from src.model import graph_decode

host = pytest.importorskip("src.cache._paged_host", reason="native host module not built (run __graft_entry__.build())")


def _layers(n_layers, lens, bs=4, initial=8, seed=0):
    """n_layers identical layer caches holding requests of the given lengths (fp32 CPU pools)."""
    out = []
    for _ in range(n_layers):
        pool = LayerBlockPool(block_size=bs, initial_blocks=initial, growth_factor=2.0)
        states = [PagedKVCacheState(pool=pool) for _ in lens]
        batch = BatchedPagedKVCache(states=states, pool=pool)
        T = max(lens) if lens else 1
        g = torch.Generator().manual_seed(seed)
        k = torch.randn(len(lens), 1, T, 2, generator=g)
        batch.append_batch(k, k.clone(), current_lengths=list(lens))
        out.append(batch)
    return out


def _snapshot(layers):
    return [([(s.seq_len, list(s.block_ids)) for s in c.states], list(c.pool.free_block_ids), c.pool.capacity_blocks,
             c.pool.mutations) for c in layers]


def test_lockstep_matches_python_on_perturbations():
    layers = _layers(3, [6, 3, 11])
    r = random.Random(0)
    for trial in range(300):
        mnb = r.choice([0, 1, 4, 8, 100])
        assert host.lockstep(layers, mnb) == graph_decode._lockstep_py(layers, mnb)
        # perturb one thing, compare, undo
        which = r.randrange(4)
        li = r.randrange(1, 3)
        c = layers[li]
        if which == 0 and c.pool.free_block_ids:
            i, j = r.randrange(len(c.pool.free_block_ids)), r.randrange(len(c.pool.free_block_ids))
            f = c.pool.free_block_ids
            f[i], f[j] = f[j], f[i]
            assert host.lockstep(layers, mnb) == graph_decode._lockstep_py(layers, mnb)
            f[i], f[j] = f[j], f[i]
        elif which == 1:
            s = c.states[r.randrange(len(c.states))]
            s.seq_len += 1
            assert host.lockstep(layers, mnb) is False and graph_decode._lockstep_py(layers, mnb) is False
            s.seq_len -= 1
        elif which == 2:
            s = c.states[r.randrange(len(c.states))]
            if s.block_ids:
                s.block_ids[-1] += 1
                assert host.lockstep(layers, mnb) is False
                s.block_ids[-1] -= 1
        else:
            c.pool.free_block_ids.append(10_000)
            assert host.lockstep(layers, mnb) is False and graph_decode._lockstep_py(layers, mnb) is False
            c.pool.free_block_ids.pop()
    assert host.lockstep(layers, 4)
    layers[1].pool.k_blocks = None  # an uninitialised pool never runs in lockstep
    assert host.lockstep(layers, 4) is False and graph_decode._lockstep_py(layers, 4) is False


def test_host_append_matches_python_with_allocation_and_growth():
    r = random.Random(1)
    for trial in range(40):
        lens = [r.randint(0, 13) for _ in range(r.randint(1, 5))]
        a = _layers(3, lens, bs=4, initial=r.choice([4, 8, 16]), seed=trial)
        b = copy.deepcopy(a)
        assert _snapshot(a) == _snapshot(b)
        for step in range(6):
            T = r.choice([1, 1, 3, 9])
            app = [max(min(r.choice([0, 1, T, T + 2, 5]), T), 0) for _ in lens]
            prev_native = host.host_append(a, app, 1, 2, torch.float32, torch.device("cpu"))
            prev_py = None
            for cache in b:
                p = cache.host_append(app, T, 1, 2, torch.float32, torch.device("cpu"))
                prev_py = p if prev_py is None else prev_py
            assert prev_native == prev_py
            assert _snapshot(a) == _snapshot(b)  # states, free lists, growth and mutation counts
            raw, mp = host.csr(a[0].states, prev_native, app)
            want, want_mp = b[0].csr_buffer(prev_py, app)
            assert mp == want_mp
            assert np.array_equal(np.frombuffer(raw, dtype=np.int32), want)


def test_host_append_initialises_empty_pools():
    pool = LayerBlockPool(block_size=4, initial_blocks=3, growth_factor=2.0)
    batch = BatchedPagedKVCache(states=[PagedKVCacheState(pool=pool)], pool=pool)
    assert pool.k_blocks is None
    prev = host.host_append([batch], [5], 2, 8, torch.float32, torch.device("cpu"))
    assert prev == [0] and pool.k_blocks is not None and pool.k_blocks.shape == (3, 2, 4, 8)
    assert batch.states[0].seq_len == 5 and batch.states[0].block_ids == [2, 1]
    # nothing appended: the pool is not touched
    pool2 = LayerBlockPool(block_size=4, initial_blocks=3, growth_factor=2.0)
    batch2 = BatchedPagedKVCache(states=[PagedKVCacheState(pool=pool2)], pool=pool2)
    assert host.host_append([batch2], [0], 2, 8, torch.float32, torch.device("cpu")) == [0]
    assert pool2.k_blocks is None


def test_host_append_errors_match_python():
    a = _layers(1, [5, 2])
    other = LayerBlockPool(block_size=4, initial_blocks=4, growth_factor=2.0)
    a[0].states[1].pool = other
    with pytest.raises(ValueError, match="must share its pool"):
        host.host_append(a, [1, 1], 1, 2, torch.float32, torch.device("cpu"))
    b = _layers(1, [5, 2])
    b[0].states[0].block_ids.append(99)
    with pytest.raises(ValueError, match=r"block_ids \(3 blocks\) does not match seq_len 5 at block size 4"):
        host.host_append(b, [1, 1], 1, 2, torch.float32, torch.device("cpu"))
    with pytest.raises(ValueError, match=r"block_ids \(3 blocks\) does not match seq_len 5 at block size 4"):
        b[0].host_append([1, 1], 1, 1, 2, torch.float32, torch.device("cpu"))


def test_csr_edge_cases():
    raw, mp = host.csr([], [], [])
    assert np.frombuffer(raw, dtype=np.int32).tolist() == [0] and mp == 0
    a = _layers(1, [0, 7, 0])
    prev = [s.seq_len for s in a[0].states]
    raw, mp = host.csr(a[0].states, prev, [0, 0, 0])
    want, want_mp = a[0].csr_buffer(prev, [0, 0, 0])
    assert np.array_equal(np.frombuffer(raw, dtype=np.int32), want) and mp == want_mp == 2
    with pytest.raises(ValueError):
        host.csr(a[0].states, prev[:2], [0, 0, 0])
    with pytest.raises(OverflowError):
        host.csr(a[0].states, [0, 2 ** 40, 0], [0, 0, 0])


def test_no_leaked_references():
    layers = _layers(6, [9, 4, 17, 1])
    app = [0, 0, 0, 0]
    prev = [s.seq_len for s in layers[0].states]
    for _ in range(200):  # warm caches of the allocator
        host.lockstep(layers, 8)
        host.host_append(layers, app, 1, 2, torch.float32, torch.device("cpu"))
        host.csr(layers[0].states, prev, app)
    tracemalloc.start()
    before = tracemalloc.get_traced_memory()[0]
    for _ in range(5000):
        host.lockstep(layers, 8)
        host.host_append(layers, app, 1, 2, torch.float32, torch.device("cpu"))
        host.csr(layers[0].states, prev, app)
    grown = tracemalloc.get_traced_memory()[0] - before
    tracemalloc.stop()
    assert grown < 64 * 1024, grown
