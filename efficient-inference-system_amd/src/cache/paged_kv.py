"""Paged KV cache: per-layer block pools, per-request block lists, batched views.

Same classes, attributes and allocation order as src/cache/paged_kv.py of the reference:
  - LayerBlockPool (:9-93): pool tensors [num_blocks, H, block_size, head_dim], lazily created on
    the first append with the dtype/device of the new keys; growth by
    max(min_extra, initial if empty else ceil(capacity * (growth_factor - 1))) zero blocks appended
    with torch.cat; a LIFO free list (ids pushed in increasing order, popped from the end);
    released blocks are zeroed before they return to the free list.
  - PagedKVCacheState (:96-137): a request's block id list and cached length.
  - BatchedPagedKVCache (:140-206): a batch of states over one pool; append_batch clamps each
    request's new-token count to [0, T] and returns the new lengths as int64.

On a HIP device, BatchedPagedKVCache.append_batch does the allocation bookkeeping on the host
(the block lists stay Python lists, as in the reference) and the data movement on the device:
one pinned host->device copy of the batch's block lists in CSR form, one metadata-packing launch
(page table, lengths, slot of every new token) and one scatter launch for K and V. The packed
page table and lengths are kept for the paged_attention call that follows. Because every layer
of a model sees the same allocation sequence, consecutive layers usually pack identical metadata;
the last packed result per device is reused when the host-side CSR buffer is byte-identical.

Additions beyond the reference: LayerBlockPool(dtype=...) to store KV in another dtype than the
model (bf16 under an fp32 model), LayerBlockPool(storage=KVStorage) to keep the pool's tensors as
views of fixed physical storage (the logical capacity, growth steps, free list and zeroing are
unchanged; only the device addresses stay put), LayerBlockPool.release_blocks (one zeroing launch
for many blocks), LayerBlockPool.mutations (allocation/release counter) and
BatchedPagedKVCache.device_metadata().
"""
from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field

import numpy as np
import torch


class KVStorage:
    """Physical K/V storage a pool's tensors are prefix views of, so their device addresses stay
    fixed while the pool grows and across pools that reuse it (a model keeps one per layer).
    Holds `blocks` physical blocks; replaced by a larger allocation only when a pool outgrows it."""

    # Bumped by every (re)allocation of any storage: a step captured against storages whose
    # addresses it recorded stays valid while this count is unchanged.
    allocations = 0

    def __init__(self, reserve_blocks: int):
        self.reserve_blocks = reserve_blocks
        self.k: torch.Tensor | None = None
        self.v: torch.Tensor | None = None

    @property
    def blocks(self) -> int:
        return 0 if self.k is None else self.k.shape[0]

    def fits(self, shape_tail: tuple, dtype: torch.dtype, device: torch.device, blocks: int) -> bool:
        return (self.k is not None and tuple(self.k.shape[1:]) == shape_tail and self.k.dtype == dtype
                and self.k.device == device and self.k.shape[0] >= blocks)

    def ensure(self, shape_tail: tuple, dtype: torch.dtype, device: torch.device, blocks: int,
               keep: int = 0) -> None:
        """Make room for `blocks` blocks, keeping the first `keep` blocks' contents."""
        if self.fits(shape_tail, dtype, device, blocks):
            return
        compatible = (self.k is not None and tuple(self.k.shape[1:]) == shape_tail and self.k.dtype == dtype
                      and self.k.device == device)
        n = max(blocks, self.reserve_blocks, 2 * self.blocks if compatible else 0)
        new_k = torch.zeros((n, *shape_tail), dtype=dtype, device=device)
        new_v = torch.zeros_like(new_k)
        if compatible and keep:
            new_k[:keep].copy_(self.k[:keep])
            new_v[:keep].copy_(self.v[:keep])
        self.k, self.v = new_k, new_v
        KVStorage.allocations += 1


class LayerBlockPool:
    def __init__(
        self,
        block_size: int,
        initial_blocks: int,
        growth_factor: float,
        dtype: torch.dtype | None = None,
        storage: KVStorage | None = None,
    ):
        self.block_size = block_size
        self.initial_blocks = initial_blocks
        self.growth_factor = growth_factor
        self.k_blocks: torch.Tensor | None = None
        self.v_blocks: torch.Tensor | None = None
        self.num_heads: int | None = None
        self.head_dim: int | None = None
        self.dtype: torch.dtype | None = None
        self.device: torch.device | None = None
        self.free_block_ids: list[int] = []
        self.capacity_blocks = 0
        self.kv_dtype = dtype
        self.mutations = 0
        self.storage = storage

    def ensure_initialized(
        self,
        num_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device,
    ) -> None:
        if self.k_blocks is not None:
            return
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.dtype = self.kv_dtype if self.kv_dtype is not None else dtype
        self.device = torch.device(device)
        self._grow(self.initial_blocks)

    def _grow(self, min_extra_blocks: int) -> None:
        if self.num_heads is None or self.head_dim is None or self.dtype is None or self.device is None:
            raise ValueError("Pool must be initialized before growth.")
        grow_by = max(
            min_extra_blocks,
            self.initial_blocks
            if self.capacity_blocks == 0
            else int(math.ceil(self.capacity_blocks * (self.growth_factor - 1.0))),
        )
        grow_by = max(grow_by, 1)
        if self.storage is not None:
            # Same logical growth, as a longer view of fixed storage: the new blocks are zeroed
            # (the storage may hold an earlier pool's data) and existing blocks keep their place.
            tail = (self.num_heads, self.block_size, self.head_dim)
            old_cap = self.capacity_blocks
            self.storage.ensure(tail, self.dtype, self.device, old_cap + grow_by, keep=old_cap)
            self.storage.k[old_cap:old_cap + grow_by].zero_()
            self.storage.v[old_cap:old_cap + grow_by].zero_()
            self.k_blocks = self.storage.k[: old_cap + grow_by]
            self.v_blocks = self.storage.v[: old_cap + grow_by]
        else:
            new_k = torch.zeros(grow_by, self.num_heads, self.block_size, self.head_dim, dtype=self.dtype,
                                device=self.device)
            new_v = torch.zeros_like(new_k)
            if self.k_blocks is None:
                self.k_blocks = new_k
                self.v_blocks = new_v
            else:
                self.k_blocks = torch.cat([self.k_blocks, new_k], dim=0)
                self.v_blocks = torch.cat([self.v_blocks, new_v], dim=0)
        start = self.capacity_blocks
        self.capacity_blocks += grow_by
        self.free_block_ids.extend(range(start, self.capacity_blocks))

    def allocate_block(self) -> int:
        if not self.free_block_ids:
            self._grow(1)
        self.mutations += 1
        return self.free_block_ids.pop()

    def release_block(self, block_id: int) -> None:
        if self.k_blocks is None or self.v_blocks is None:
            return
        self.k_blocks[block_id].zero_()
        self.v_blocks[block_id].zero_()
        self.free_block_ids.append(block_id)
        self.mutations += 1

    def release_blocks(self, block_ids: list[int]) -> None:
        """Release several blocks: the same zeroing and free-list order as calling
        release_block for each id in turn, with one device launch on a HIP pool."""
        if self.k_blocks is None or self.v_blocks is None or not block_ids:
            return
        if self.k_blocks.is_cuda:
            from src.kernels.hip_paged_attention import zero_blocks_hip

            from src.kernels.staging import upload

            ids = upload(np.asarray(block_ids, dtype=np.int32), self.k_blocks.device)
            zero_blocks_hip(self.k_blocks, self.v_blocks, ids)
        else:
            idx = torch.tensor(block_ids, dtype=torch.long)
            self.k_blocks[idx] = 0
            self.v_blocks[idx] = 0
        self.free_block_ids.extend(block_ids)
        self.mutations += 1

    def bytes_per_block(self) -> int:
        if self.k_blocks is None:
            return 0
        return 2 * self.k_blocks[0].numel() * self.k_blocks.element_size()

    def reserved_bytes(self) -> int:
        return self.capacity_blocks * self.bytes_per_block()


@dataclass
class PagedKVCacheState:
    pool: LayerBlockPool
    block_ids: list[int] = field(default_factory=list)
    seq_len: int = 0

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor, length: int) -> None:
        if length <= 0:
            return
        if k_new.is_cuda:
            BatchedPagedKVCache(states=[self], pool=self.pool).append_batch(k_new, v_new, current_lengths=[length])
            return
        # Host bookkeeping shared with the device path (the reference's block order), then one
        # scatter per pool: the token at position p goes to slot p % block_size of block
        # block_ids[p // block_size].
        _, num_heads, query_len, head_dim = k_new.shape
        if length > query_len:
            raise ValueError(f"append of {length} tokens from {query_len} new rows")
        start = BatchedPagedKVCache(states=[self], pool=self.pool).host_append(
            [length], query_len, num_heads, head_dim, k_new.dtype, k_new.device)[0]
        bs = self.pool.block_size
        pos = torch.arange(start, start + length)
        blocks = torch.tensor(self.block_ids, dtype=torch.long)[pos // bs]
        for pool_blocks, new in ((self.pool.k_blocks, k_new), (self.pool.v_blocks, v_new)):
            pool_blocks[blocks, :, pos % bs, :] = new[0, :, :length, :].transpose(0, 1).to(pool_blocks.dtype)

    def release(self) -> None:
        self.pool.release_blocks(list(self.block_ids))
        self.block_ids.clear()
        self.seq_len = 0

    def live_bytes(self) -> int:
        if self.pool.k_blocks is None:
            return 0
        kb = self.pool.k_blocks
        return self.seq_len * kb.shape[1] * kb.shape[3] * 2 * kb.element_size()

    def reserved_bytes(self) -> int:
        return len(self.block_ids) * self.pool.bytes_per_block()

    def fragmentation_bytes(self) -> int:
        return self.reserved_bytes() - self.live_bytes()


def _host_lengths(current_lengths, count: int, query_len: int) -> list[int]:
    if current_lengths is None:
        return [query_len] * count
    if isinstance(current_lengths, int):
        return [current_lengths] * count
    if isinstance(current_lengths, torch.Tensor):
        return [int(x) for x in current_lengths.tolist()]
    return [int(x) for x in current_lengths]


def _device_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


def _same_device(a: torch.device, b: torch.device) -> bool:
    return a.type == b.type and (a.type != "cuda" or _device_index(a) == _device_index(b))


# Last metadata packed on each device: (host CSR bytes, query_len, block_size, max_pages) -> tensors.
_last_pack: dict[tuple, tuple] = {}


class BatchedPagedKVCache:
    def __init__(self, states: list[PagedKVCacheState], pool: LayerBlockPool | None = None):
        self.states = states
        if pool is not None:
            self.pool = pool
        else:
            non_null = next((state for state in states if state is not None), None)
            if non_null is None:
                raise ValueError("BatchedPagedKVCache needs a pool when all states are uninitialized.")
            self.pool = non_null.pool
        self._meta: tuple | None = None  # (signature, page_table, seq_lens int32)

    # ------------------------------------------------------------------------------------------
    def _signature(self) -> tuple:
        return (
            self.pool.mutations,
            len(self.states),
            tuple(s.seq_len for s in self.states),
            tuple(len(s.block_ids) for s in self.states),
        )

    def _pack(self, device: torch.device, query_len: int, prev: list[int], app: list[int], with_slots: bool):
        """Upload the batch's block lists (CSR) and build page table / lengths / slots on device."""
        from src.kernels.hip_paged_attention import pack_metadata_hip

        B = len(self.states)
        buf, max_pages = self.csr_buffer(prev, app)
        dev_index = _device_index(device)
        key = (dev_index, buf.tobytes(), query_len, self.pool.block_size, max_pages, with_slots)
        hit = _last_pack.get(dev_index)
        if hit is not None and hit[0] == key:
            return hit[1]
        from src.kernels.staging import upload

        dev = upload(buf, device)
        result = pack_metadata_hip(
            dev[3 * B + 1:], dev[0:B + 1], dev[B + 1:2 * B + 1], dev[2 * B + 1:3 * B + 1],
            query_len=query_len, block_size=self.pool.block_size, max_pages=max_pages, with_slots=with_slots,
        )
        _last_pack[dev_index] = (key, result)
        return result

    def device_metadata(self, device: torch.device) -> tuple[torch.Tensor, torch.Tensor]:
        """(page_table int32 [B, max_pages], seq_lens int32 [B]) on `device`, reusing what the last
        append_batch packed when no state changed since."""
        device = torch.device(device)
        sig = self._signature()
        if self._meta is not None and self._meta[0] == sig and _same_device(self._meta[1].device, device):
            return self._meta[1], self._meta[2]
        prev = [s.seq_len for s in self.states]
        page_table, seq32, _, _ = self._pack(device, 0, prev, [0] * len(self.states), False)
        self._meta = (sig, page_table, seq32)
        return page_table, seq32

    def invalidate_metadata(self) -> None:
        """Drop cached device metadata (needed only after editing block_ids lists by hand)."""
        self._meta = None

    # ------------------------------------------------------------------------------------------
    def append_batch(
        self,
        k_new: torch.Tensor,
        v_new: torch.Tensor,
        current_lengths: int | torch.Tensor | None = None,
    ) -> torch.Tensor:
        T = k_new.shape[2]
        lengths = _host_lengths(current_lengths, len(self.states), T)
        if not k_new.is_cuda:
            updated = []
            for batch_idx, state in enumerate(self.states):
                state.append(
                    k_new[batch_idx:batch_idx + 1],
                    v_new[batch_idx:batch_idx + 1],
                    max(min(lengths[batch_idx], T), 0),
                )
                updated.append(state.seq_len)
            return torch.tensor(updated, dtype=torch.long, device=k_new.device)
        return self._append_batch_device(k_new, v_new, lengths)

    def host_append(self, app: list[int], query_len: int, num_heads: int, head_dim: int, dtype: torch.dtype,
                    device: torch.device) -> list[int]:
        """Host half of a device append of app[b] (already clamped to [0, T]) new tokens per
        request: initialises the pool if needed, allocates blocks in the reference's order and
        advances seq_len. Returns the lengths before the append."""
        pool = self.pool
        bs = pool.block_size
        if any(app):
            pool.ensure_initialized(num_heads, head_dim, dtype, device)
        prev = []
        for state, n in zip(self.states, app):
            p = state.seq_len
            prev.append(p)
            if n <= 0:
                continue
            if state.pool is not pool:
                raise ValueError("all states of a BatchedPagedKVCache must share its pool")
            if len(state.block_ids) != (p + bs - 1) // bs:
                raise ValueError(
                    f"block_ids ({len(state.block_ids)} blocks) does not match seq_len {p} at block size {bs}"
                )
            for _ in range((p + n + bs - 1) // bs - len(state.block_ids)):
                state.block_ids.append(pool.allocate_block())
            state.seq_len = p + n
        return prev

    def csr_buffer(self, prev: list[int], app: list[int]) -> tuple[np.ndarray, int]:
        """int32 [row_offsets B+1 | prev B | app B | block ids] of the batch, and max_pages."""
        B = len(self.states)
        counts = [len(s.block_ids) for s in self.states]
        total = sum(counts)
        buf = np.empty(3 * B + 1 + total, dtype=np.int32)
        buf[0] = 0
        np.cumsum(counts, out=buf[1:B + 1])
        buf[B + 1:2 * B + 1] = prev
        buf[2 * B + 1:3 * B + 1] = app
        if total:
            buf[3 * B + 1:] = np.fromiter(itertools.chain.from_iterable([s.block_ids for s in self.states]),
                                          dtype=np.int32, count=total)
        return buf, max(counts, default=0)

    def _append_batch_device(self, k_new: torch.Tensor, v_new: torch.Tensor, lengths: list[int]) -> torch.Tensor:
        from src.kernels.hip_paged_attention import kv_append_hip

        B, H, T, Hd = k_new.shape
        pool = self.pool
        app = [max(min(n, T), 0) for n in lengths]
        prev = self.host_append(app, T, H, Hd, k_new.dtype, k_new.device)
        page_table, seq32, seq64, slots = self._pack(k_new.device, T, prev, app, True)
        if any(app):
            kv_append_hip(k_new, v_new, pool.k_blocks, pool.v_blocks, slots)
        self._meta = (self._signature(), page_table, seq32)
        return seq64

    # ------------------------------------------------------------------------------------------
    def page_table_tensor(self, device: torch.device | None = None) -> torch.Tensor:
        device = torch.device(device) if device is not None else self.pool.device
        max_pages = max((len(state.block_ids) for state in self.states), default=0)
        if device is not None and device.type == "cuda":
            return self.device_metadata(device)[0]
        if max_pages == 0:
            return torch.empty((len(self.states), 0), dtype=torch.int32, device=device)
        page_table = torch.full((len(self.states), max_pages), -1, dtype=torch.int32, device=device)
        for row_idx, state in enumerate(self.states):
            if state.block_ids:
                page_table[row_idx, : len(state.block_ids)] = torch.tensor(state.block_ids, dtype=torch.int32, device=device)
        return page_table

    def seq_lens_tensor(self, device: torch.device | None = None) -> torch.Tensor:
        device = torch.device(device) if device is not None else self.pool.device
        if device is not None and device.type == "cuda":
            return self.device_metadata(device)[1]
        return torch.tensor([state.seq_len for state in self.states], dtype=torch.int32, device=device)

    def live_bytes(self) -> int:
        return sum(state.live_bytes() for state in self.states)

    def reserved_bytes(self) -> int:
        return sum(state.reserved_bytes() for state in self.states)

    def fragmentation_bytes(self) -> int:
        return sum(state.fragmentation_bytes() for state in self.states)
