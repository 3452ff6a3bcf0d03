"""ORACLE — test infrastructure only.

CPU restatements of the reference's paged-attention path, used to check the HIP kernels. Only
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import this package; product
code never does.

Contents:
  - libpaged_oracle.so (paged_oracle.c): attention, append and page-table restatements in C with
    double accumulation (file:line citations in the C header), wrapped by paged_attention(),
    append() and page_table() below;
  - reference_loop.py: the reference's per-token torch loop
    (src/kernels/reference_paged_attention.py:10-59), for tiny cases;
  - LifoAllocator: the reference pool's id order (src/cache/paged_kv.py:44-85).
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "libpaged_oracle.so"

_lib = None


def build() -> Path:
    """Compile paged_oracle.c with the committed Makefile (gcc, OpenMP)."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "libpaged_oracle.so"], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
        l.oracle_paged_attention.restype = ctypes.c_int
        l.oracle_paged_attention.argtypes = [vp, vp, vp, ctypes.c_int, i64, vp, vp, vp, vp,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_int, vp, ctypes.c_int, ctypes.c_int]
        l.oracle_append.restype = ctypes.c_int
        l.oracle_append.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                    vp, vp, ctypes.c_int, i64, ctypes.c_int, vp, vp, vp, vp]
        l.oracle_page_table.restype = None
        l.oracle_page_table.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
        l.oracle_f32_to_bf16.restype = None
        l.oracle_f32_to_bf16.argtypes = [vp, vp, i64]
        _lib = l
    return _lib


def _np(x, dtype=None) -> np.ndarray:
    """numpy view of a CPU array-like; torch bfloat16 tensors become uint16 bit patterns."""
    try:
        import torch

        if isinstance(x, torch.Tensor):
            x = x.detach().cpu()
            if x.dtype == torch.bfloat16:
                x = x.contiguous().view(torch.int16).numpy().view(np.uint16)
            else:
                x = x.contiguous().numpy()
    except ImportError:
        pass
    a = np.ascontiguousarray(x)
    if dtype is not None and a.dtype != dtype:
        a = a.astype(dtype)
    return a


def csr(block_lists: list[list[int]]) -> tuple[np.ndarray, np.ndarray]:
    """(flat int32 ids, int32 row offsets [B+1]) of per-request block lists."""
    offsets = np.zeros(len(block_lists) + 1, dtype=np.int32)
    offsets[1:] = np.cumsum([len(x) for x in block_lists])
    flat = np.fromiter((i for row in block_lists for i in row), dtype=np.int32, count=int(offsets[-1]))
    return flat, offsets


def _pool_dtype_code(pool: np.ndarray) -> int:
    if pool.dtype == np.float32:
        return 0
    if pool.dtype == np.uint16:
        return 1
    raise TypeError(f"pool must be float32 or bf16 (uint16 bits), got {pool.dtype}")


def paged_attention(q, k_pool, v_pool, block_lists, seq_lens, cur_lens, *, nthreads: int = 0,
                    mutation: int = 0) -> np.ndarray:
    """Oracle attention. q [B, H, T, Hd] float32; pools [N, H, bs, Hd] float32 or bf16 bits;
    block_lists per request; returns float32 [B, H, T, Hd]."""
    qn = _np(q, np.float32)
    kp, vp = _np(k_pool), _np(v_pool)
    B, H, T, Hd = qn.shape
    N, Hp, bs, Hdp = kp.shape
    assert (Hp, Hdp) == (H, Hd) and vp.shape == kp.shape and vp.dtype == kp.dtype
    ids, offs = csr(block_lists)
    sl = _np(seq_lens, np.int32)
    cl = _np(cur_lens, np.int32)
    out = np.zeros_like(qn)
    status = lib().oracle_paged_attention(
        qn.ctypes.data, kp.ctypes.data, vp.ctypes.data, _pool_dtype_code(kp), N,
        ids.ctypes.data if ids.size else None, offs.ctypes.data, sl.ctypes.data, cl.ctypes.data,
        B, H, T, Hd, bs, out.ctypes.data, nthreads, mutation,
    )
    if status != 0:
        raise IndexError("oracle: a key position has no valid block in its request's block list")
    return out


def append(k_new, v_new, k_pool: np.ndarray, v_pool: np.ndarray, block_lists, prev_lens, current_lengths) -> None:
    """Oracle append into numpy pools in place (block_lists already hold the new blocks)."""
    kn, vn = _np(k_new, np.float32), _np(v_new, np.float32)
    B, H, T, Hd = kn.shape
    assert k_pool.flags.c_contiguous and v_pool.flags.c_contiguous
    ids, offs = csr(block_lists)
    pl = _np(prev_lens, np.int32)
    cl = _np(current_lengths, np.int32)
    status = lib().oracle_append(
        kn.ctypes.data, vn.ctypes.data, B, H, T, Hd, k_pool.ctypes.data, v_pool.ctypes.data,
        _pool_dtype_code(k_pool), k_pool.shape[0], k_pool.shape[2],
        ids.ctypes.data if ids.size else None, offs.ctypes.data, pl.ctypes.data, cl.ctypes.data,
    )
    if status != 0:
        raise IndexError("oracle: append position has no valid block")


def page_table(block_lists) -> np.ndarray:
    ids, offs = csr(block_lists)
    max_pages = max((len(x) for x in block_lists), default=0)
    out = np.empty((len(block_lists), max_pages), dtype=np.int32)
    if max_pages:
        lib().oracle_page_table(ids.ctypes.data if ids.size else None, offs.ctypes.data, len(block_lists), max_pages,
                                out.ctypes.data)
    return out


def f32_to_bf16_bits(x) -> np.ndarray:
    a = _np(x, np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().oracle_f32_to_bf16(a.ctypes.data, out.ctypes.data, a.size)
    return out


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


class LifoAllocator:
    """Block-id order of the reference pool (src/cache/paged_kv.py:44-85): growth appends ids
    start..capacity-1 to the free list, allocation pops the last id, release appends."""

    def __init__(self, initial_blocks: int, growth_factor: float):
        self.initial = initial_blocks
        self.growth = growth_factor
        self.capacity = 0
        self.free: list[int] = []

    def _grow(self, min_extra: int) -> None:
        import math

        by = max(min_extra, self.initial if self.capacity == 0 else int(math.ceil(self.capacity * (self.growth - 1.0))))
        by = max(by, 1)
        self.free.extend(range(self.capacity, self.capacity + by))
        self.capacity += by

    def ensure(self) -> None:
        if self.capacity == 0:
            self._grow(self.initial)

    def allocate(self) -> int:
        if not self.free:
            self._grow(1)
        return self.free.pop()

    def release(self, ids: list[int]) -> None:
        self.free.extend(ids)
