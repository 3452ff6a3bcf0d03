"""Paged KV cache host logic on the CPU: the reference's own three tests
(tests/test_paged_kv.py:9-40 of the reference) plus allocation order, growth, append contents and
page tables checked against the oracle's restatements."""
import random

import numpy as np
import pytest
import torch

import oracle
from src.cache.paged_kv import BatchedPagedKVCache, LayerBlockPool, PagedKVCacheState


# --- the reference's tests, restated -------------------------------------------------------------
def test_allocator_growth_and_reuse():
    pool = LayerBlockPool(block_size=4, initial_blocks=1, growth_factor=2.0)
    state = PagedKVCacheState(pool=pool)
    k = torch.randn(1, 2, 6, 8)
    v = torch.randn(1, 2, 6, 8)
    state.append(k, v, length=6)
    assert pool.capacity_blocks >= 2
    allocated = list(state.block_ids)
    state.release()
    reused = pool.allocate_block()
    assert reused in allocated


def test_block_boundary_append():
    pool = LayerBlockPool(block_size=4, initial_blocks=2, growth_factor=2.0)
    state = PagedKVCacheState(pool=pool)
    state.append(torch.randn(1, 2, 5, 8), torch.randn(1, 2, 5, 8), length=5)
    assert state.seq_len == 5
    assert len(state.block_ids) == 2


def test_batched_page_table_handles_heterogeneous_lengths():
    pool = LayerBlockPool(block_size=4, initial_blocks=4, growth_factor=2.0)
    states = [PagedKVCacheState(pool=pool) for _ in range(2)]
    batch = BatchedPagedKVCache(states=states, pool=pool)
    k = torch.randn(2, 2, 4, 8)
    v = torch.randn(2, 2, 4, 8)
    batch.append_batch(k, v, current_lengths=torch.tensor([4, 2]))
    page_table = batch.page_table_tensor(device=k.device)
    seq_lens = batch.seq_lens_tensor(device=k.device)
    assert tuple(page_table.shape) == (2, 1)
    assert seq_lens.tolist() == [4, 2]


# --- allocation order and growth ----------------------------------------------------------------
def test_lifo_order_and_growth_match_oracle_allocator():
    rng = random.Random(5)
    pool = LayerBlockPool(block_size=4, initial_blocks=3, growth_factor=1.5)
    pool.ensure_initialized(2, 8, torch.float32, "cpu")
    ref = oracle.LifoAllocator(initial_blocks=3, growth_factor=1.5)
    ref.ensure()
    held, held_ref = [], []
    for _ in range(400):
        if held and rng.random() < 0.4:
            k = rng.randrange(len(held))
            ids = held.pop(k)
            ids_ref = held_ref.pop(k)
            pool.release_blocks(ids)
            ref.release(ids_ref)
        else:
            n = rng.randint(1, 5)
            held.append([pool.allocate_block() for _ in range(n)])
            held_ref.append([ref.allocate() for _ in range(n)])
        assert held == held_ref
        assert pool.capacity_blocks == ref.capacity
        assert pool.free_block_ids == ref.free
    assert pool.k_blocks.shape[0] == pool.capacity_blocks


def test_first_allocation_is_highest_id_and_release_zeroes():
    pool = LayerBlockPool(block_size=4, initial_blocks=8, growth_factor=2.0)
    state = PagedKVCacheState(pool=pool)
    state.append(torch.ones(1, 2, 9, 8), torch.ones(1, 2, 9, 8), length=9)
    assert state.block_ids == [7, 6, 5]
    assert float(pool.k_blocks[[7, 6, 5]].abs().sum()) > 0
    state.release()
    assert float(pool.k_blocks.abs().sum()) == 0.0 and float(pool.v_blocks.abs().sum()) == 0.0
    assert pool.free_block_ids[-3:] == [7, 6, 5]
    assert pool.allocate_block() == 5


# --- append contents vs the oracle, bit for bit ---------------------------------------------------
@pytest.mark.parametrize("pool_dtype", [torch.float32, torch.bfloat16])
def test_batched_append_matches_oracle_bitwise(pool_dtype):
    g = torch.Generator().manual_seed(3)
    B, H, Hd, bs = 5, 3, 8, 4
    pool = LayerBlockPool(block_size=bs, initial_blocks=2, growth_factor=2.0, dtype=pool_dtype)
    states = [PagedKVCacheState(pool=pool) for _ in range(B)]
    ref_lists = [[] for _ in range(B)]
    ref_lens = [0] * B
    for step in range(4):
        T = [7, 1, 5, 3][step]
        k = torch.randn(B, H, T, Hd, generator=g)
        v = torch.randn(B, H, T, Hd, generator=g)
        cur = torch.tensor([T, T - 1, 0, T + 3, 1])[:B]
        batch = BatchedPagedKVCache(states=states, pool=pool)
        out = batch.append_batch(k, v, current_lengths=cur)
        assert out.dtype == torch.long
        app = [max(min(int(c), T), 0) for c in cur]
        prev = list(ref_lens)
        for b in range(B):
            ref_lens[b] += app[b]
        assert out.tolist() == ref_lens
        assert [s.seq_len for s in states] == ref_lens
        for b in range(B):
            assert len(states[b].block_ids) == (ref_lens[b] + bs - 1) // bs
        ref_lists = [list(s.block_ids) for s in states]
        np_dtype = np.float32 if pool_dtype == torch.float32 else np.uint16
        kp = np.zeros((pool.capacity_blocks, H, bs, Hd), dtype=np_dtype)
        vp = np.zeros_like(kp)
        if step == 0:
            ref_pool = (kp, vp)
        else:
            old_k, old_v = ref_pool
            kp[: old_k.shape[0]] = old_k
            vp[: old_v.shape[0]] = old_v
            ref_pool = (kp, vp)
        oracle.append(k, v, kp, vp, ref_lists, prev, app)
        assert np.array_equal(oracle._np(pool.k_blocks), kp)
        assert np.array_equal(oracle._np(pool.v_blocks), vp)


def test_page_table_matches_oracle():
    pool = LayerBlockPool(block_size=4, initial_blocks=4, growth_factor=2.0)
    lists = [[3, 1], [], [0, 2, 5, 6], [7]]
    states = [PagedKVCacheState(pool=pool, block_ids=list(x), seq_len=4 * len(x)) for x in lists]
    batch = BatchedPagedKVCache(states=states, pool=pool)
    pt = batch.page_table_tensor(device="cpu")
    assert pt.dtype == torch.int32
    assert np.array_equal(pt.numpy(), oracle.page_table(lists))
    assert batch.seq_lens_tensor(device="cpu").tolist() == [8, 0, 16, 4]


def test_empty_page_table_shape():
    pool = LayerBlockPool(block_size=4, initial_blocks=4, growth_factor=2.0)
    batch = BatchedPagedKVCache(states=[PagedKVCacheState(pool=pool) for _ in range(3)], pool=pool)
    assert tuple(batch.page_table_tensor(device="cpu").shape) == (3, 0)


def test_uninitialized_pool_errors_like_reference():
    pool = LayerBlockPool(block_size=4, initial_blocks=1, growth_factor=2.0)
    with pytest.raises(ValueError):
        pool._grow(1)
    with pytest.raises(ValueError):
        BatchedPagedKVCache(states=[None])


def test_byte_accounting():
    pool = LayerBlockPool(block_size=4, initial_blocks=2, growth_factor=2.0)
    state = PagedKVCacheState(pool=pool)
    state.append(torch.randn(1, 2, 5, 8), torch.randn(1, 2, 5, 8), length=5)
    assert pool.bytes_per_block() == 2 * 2 * 4 * 8 * 4
    assert state.live_bytes() == 5 * 2 * 8 * 2 * 4
    assert state.reserved_bytes() == 2 * pool.bytes_per_block()
    assert state.fragmentation_bytes() == state.reserved_bytes() - state.live_bytes()
    assert pool.reserved_bytes() == pool.capacity_blocks * pool.bytes_per_block()


# --- storage-backed pools keep the reference's logical behaviour ----------------------------------
def test_storage_backed_pool_matches_plain_pool():
    from src.cache.paged_kv import KVStorage

    g = torch.Generator().manual_seed(31)
    storage = KVStorage(reserve_blocks=5)
    plain = LayerBlockPool(block_size=4, initial_blocks=2, growth_factor=2.0)
    backed = LayerBlockPool(block_size=4, initial_blocks=2, growth_factor=2.0, storage=storage)
    sp = [PagedKVCacheState(pool=plain) for _ in range(3)]
    sb = [PagedKVCacheState(pool=backed) for _ in range(3)]
    for step in range(6):
        T = [9, 3, 7, 1, 12, 4][step]
        k = torch.randn(3, 2, T, 8, generator=g)
        v = torch.randn(3, 2, T, 8, generator=g)
        cur = torch.tensor([T, max(T - 2, 0), T])
        BatchedPagedKVCache(sp, plain).append_batch(k, v, cur)
        BatchedPagedKVCache(sb, backed).append_batch(k, v, cur)
        if step == 3:
            sp[1].release()
            sb[1].release()
        assert [s.block_ids for s in sp] == [s.block_ids for s in sb]
        assert plain.capacity_blocks == backed.capacity_blocks and plain.free_block_ids == backed.free_block_ids
        assert torch.equal(plain.k_blocks, backed.k_blocks) and torch.equal(plain.v_blocks, backed.v_blocks)
        assert backed.reserved_bytes() == plain.reserved_bytes()
        assert backed.k_blocks.data_ptr() == storage.k.data_ptr()
    assert storage.blocks >= backed.capacity_blocks > 5  # outgrew the reservation once


def test_storage_reuse_starts_from_zeroed_blocks():
    from src.cache.paged_kv import KVStorage

    storage = KVStorage(reserve_blocks=16)
    first = LayerBlockPool(block_size=4, initial_blocks=4, growth_factor=2.0, storage=storage)
    st = PagedKVCacheState(pool=first)
    st.append(torch.ones(1, 2, 14, 8), torch.ones(1, 2, 14, 8), length=14)  # held, never released
    ptr = storage.k.data_ptr()
    second = LayerBlockPool(block_size=4, initial_blocks=4, growth_factor=2.0, storage=storage)
    second.ensure_initialized(2, 8, torch.float32, "cpu")
    assert second.k_blocks.data_ptr() == ptr
    assert float(second.k_blocks.abs().sum()) == 0.0 and float(second.v_blocks.abs().sum()) == 0.0
    assert second.free_block_ids == [0, 1, 2, 3] and second.capacity_blocks == 4


def test_graph_lockstep_check():
    """The graph step's lockstep test over per-layer caches: identical layers pass; a different
    block list, free-list length or free-list tail (the ids a step may pop) fails; a difference
    deeper in the free lists than the step can reach is left to later steps."""
    from src.model.graph_decode import _lockstep

    def layer():
        pool = LayerBlockPool(block_size=4, initial_blocks=32, growth_factor=2.0)
        states = [PagedKVCacheState(pool=pool), PagedKVCacheState(pool=pool)]
        batch = BatchedPagedKVCache(states=states, pool=pool)
        k = torch.zeros(2, 1, 6, 2)
        batch.append_batch(k, k.clone(), current_lengths=[6, 3])
        return batch

    layers = [layer() for _ in range(3)]
    assert _lockstep(layers, 4)
    free = layers[2].pool.free_block_ids
    free[0], free[1] = free[1], free[0]  # deep in the list: no step of <= 4 pops reaches it
    assert _lockstep(layers, 4)
    assert not _lockstep(layers, len(free))  # a step that could pop every id sees the difference
    free[0], free[1] = free[1], free[0]
    free[-1], free[-2] = free[-2], free[-1]  # the next ids to be popped differ
    assert not _lockstep(layers, 4)
    free[-1], free[-2] = free[-2], free[-1]
    layers[1].states[0].block_ids[0] += 1
    assert not _lockstep(layers, 4)
    layers[1].states[0].block_ids[0] -= 1
    layers[1].pool.free_block_ids.pop()
    assert not _lockstep(layers, 4)
