"""Loader and ctypes signatures for libpaged_hip.so (declared in include/paged_hip.h).

The library is built in-tree by `efficient-inference-system_amd/build_lib.py`. There is no
fallback: if the library is missing or fails to load, every "hip_paged" call raises.
torch is imported first so the library binds to the HIP runtime torch already mapped.
"""
from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library links against)

LIB_PATH = Path(os.environ.get("PAGED_HIP_LIB", Path(__file__).resolve().parents[2] / "libpaged_hip.so"))

PA_DTYPE_F32 = 0
PA_DTYPE_BF16 = 1

PA_OK = 0
PA_ERR_INVALID_ARGUMENT = 1
PA_ERR_UNSUPPORTED = 2
PA_ERR_WORKSPACE = 3
PA_ERR_HIP = 4

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_int = ctypes.c_int
_f32 = ctypes.c_float
_size_t = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/paged_hip.h one to one.
SIGNATURES: dict[str, tuple] = {
    "pa_version": (_int, []),
    "pa_last_error_message": (ctypes.c_char_p, []),
    "pa_decode": (
        _int,
        [_c_void_p, _i64, _i64,  # q, strides b, h
         _c_void_p, _i64, _i64, _int,  # out, strides b, h, io dtype
         _c_void_p, _c_void_p, _int, _i64,  # k pool, v pool, kv dtype, num_blocks
         _c_void_p, _i64, _i32,  # page table, stride, max_pages
         _c_void_p, _c_void_p, _c_void_p,  # seq_lens, cur_lens, order
         _i32, _i32, _i32, _i32,  # batch, heads, head_dim, block_size
         _f32, _i32,  # scale, split_blocks
         _c_void_p, _size_t, _c_void_p],  # workspace, bytes, stream
    ),
    "pa_decode_workspace_size": (_size_t, [_i32, _i32, _i32, _i32, _i32]),
    "pa_decode_noalloc": (
        _int,
        [_c_void_p, _i64, _i64,  # q, strides b, h
         _c_void_p, _i64, _i64, _int,  # out, strides b, h, io dtype
         _c_void_p, _c_void_p, _int, _i64,  # k pool, v pool, kv dtype, num_blocks
         _c_void_p, _i64, _i32,  # page table, stride, max_pages
         _c_void_p, _c_void_p, _c_void_p,  # seq_lens, cur_lens, order
         _i32, _i32, _i32, _i32,  # batch, heads, head_dim, block_size
         _f32, _i32, _c_void_p],  # scale, split_blocks, stream
    ),
    "pa_prefill": (
        _int,
        [_c_void_p, _i64, _i64, _i64,
         _c_void_p, _i64, _i64, _i64, _int,
         _c_void_p, _c_void_p, _int, _i64,
         _c_void_p, _i64, _i32,
         _c_void_p, _c_void_p,
         _i32, _i32, _i32, _i32, _i32,
         _f32, _i32,  # scale, split_blocks
         _c_void_p, _size_t, _c_void_p],  # workspace, bytes, stream
    ),
    "pa_prefill_workspace_size": (_size_t, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "pa_kv_append": (
        _int,
        [_c_void_p, _c_void_p, _i64, _i64, _i64, _int,
         _c_void_p, _c_void_p, _int, _i64,
         _c_void_p,
         _i32, _i32, _i32, _i32, _i32, _c_void_p],
    ),
    "pa_pack_metadata": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _i32, _i32, _i32, _i32,
         _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p],
    ),
    "pa_pack_metadata_mirror": (
        _int,
        [_c_void_p, _i64, _i32,  # mirror, stride, rows
         _c_void_p, _c_void_p,  # mirror row, first page
         _c_void_p, _c_void_p, _i64,  # num pages, update ids, update stride
         _c_void_p, _c_void_p,  # prev lens, append lens
         _i32, _i32, _i32, _i32,  # batch, query_len, block_size, max_pages
         _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p,  # page table, stride, seq32, seq64, slots
         _c_void_p, _c_void_p, _i32, _c_void_p],  # stage src, stage dst, stage words, stream
    ),
    "pa_linear_rows": (
        _int,
        [_c_void_p, _i64, _i32, _i32,  # x, stride, rows, in_features
         _c_void_p, _c_void_p, _i32,  # weight, bias, out_features
         _c_void_p, _c_void_p, _f32,  # LayerNorm weight, bias, eps
         _i32, _c_void_p, _i64,  # activation, residual, stride
         _c_void_p, _i64, _c_void_p, _i64,  # out, stride, out copy, stride
         _int, _c_void_p],  # dtype, stream
    ),
    "pa_linear_select_rows": (
        _int,
        [_c_void_p, _i64, _i32, _i32, _c_void_p,  # x, stride, groups, group rows, row index
         _i32, _c_void_p, _c_void_p, _i32,  # in_features, weight, bias, out_features
         _c_void_p, _c_void_p, _f32,  # LayerNorm weight, bias, eps
         _i32, _c_void_p, _i64, _c_void_p, _i64,  # activation, out, stride, token keys, key stride
         _int, _c_void_p],  # dtype, stream
    ),
    "pa_qkv_append": (
        _int,
        [_c_void_p, _i64, _i32, _i32,  # x, stride, rows, d_model
         _c_void_p, _c_void_p, _f32,  # LayerNorm weight, bias, eps
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,  # wq, bq, wk, bk, wv, bv
         _c_void_p, _i64,  # q_out, stride
         _c_void_p, _c_void_p, _int, _i64,  # k pool, v pool, pool dtype, num_blocks
         _c_void_p, _i32, _i32, _i32, _int, _c_void_p],  # slots, heads, head_dim, block_size, dtype, stream
    ),
    "pa_mlp_rows": (
        _int,
        [_c_void_p, _i64, _i32, _i32,  # x, stride, rows, d_model
         _c_void_p, _c_void_p, _f32,  # LayerNorm weight, bias, eps
         _c_void_p, _c_void_p, _i32, _i32,  # fc1 weight, bias, d_ff, activation
         _c_void_p, _c_void_p,  # fc2 weight, bias
         _c_void_p, _i64,  # residual, stride
         _c_void_p, _i64, _int, _c_void_p],  # out (accumulated), stride, dtype, stream
    ),
    "pa_embed_rows": (
        _int,
        [_c_void_p, _c_void_p, _i32, _i32,  # ids, pos_start, batch, query_len
         _c_void_p, _i64, _c_void_p, _i32,  # token table, vocab, position table, max_pos
         _i32, _c_void_p, _i64, _int, _c_void_p],  # d_model, out, out stride, dtype, stream
    ),
    "pa_argmax_rows": (
        _int,
        [_c_void_p, _i64, _i32, _i32,  # logits, row stride, batch, rows per request
         _c_void_p, _i32, _int, _c_void_p, _c_void_p],  # row index, vocab, dtype, tokens, stream
    ),
    "pa_hbm_read_probe": (_int, [_c_void_p, _size_t, _c_void_p, _i32, _i32, _i32, _c_void_p]),
    "pa_hbm_chunk_read_probe": (_int, [_c_void_p, _c_void_p, _i32, _c_void_p, _i32, _i32, _c_void_p]),
    "pa_zero_blocks": (
        _int,
        [_c_void_p, _c_void_p, _int, _i64, _i32, _i32, _i32, _c_void_p, _i32, _c_void_p],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class PagedHipError(RuntimeError):
    """A libpaged_hip entry point returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Load (once) and return the library with argtypes set; raises if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"libpaged_hip.so not found at {LIB_PATH}; build it with "
                    "`python efficient-inference-system_amd/build_lib.py` (hipcc, gfx950)"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != PA_OK:
        msg = load().pa_last_error_message()
        text = msg.decode() if msg else ""
        exc = ValueError if status == PA_ERR_INVALID_ARGUMENT else PagedHipError
        raise exc(f"{what} failed with status {status}: {text}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return PA_DTYPE_F32
    if dtype == torch.bfloat16:
        return PA_DTYPE_BF16
    raise TypeError(f"libpaged_hip supports float32 and bfloat16 tensors, got {dtype}")
