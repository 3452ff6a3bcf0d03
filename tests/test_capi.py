"""The C-ABI library loads and exports exactly what include/paged_hip.h declares (no GPU needed:
these tests only resolve symbols and call the pure host functions)."""
import ctypes
import re
from pathlib import Path

import pytest

from src.kernels import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "paged_hip.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        import importlib.util

        spec = importlib.util.spec_from_file_location("build_lib", _lib.LIB_PATH.parent / "build_lib.py")
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _lib.load()


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted([
        "pa_argmax_rows", "pa_decode", "pa_decode_noalloc", "pa_decode_workspace_size", "pa_embed_rows",
        "pa_hbm_chunk_read_probe", "pa_hbm_read_probe", "pa_kv_append", "pa_last_error_message",
        "pa_linear_rows", "pa_linear_select_rows", "pa_mlp_rows",
        "pa_pack_metadata", "pa_pack_metadata_mirror", "pa_prefill", "pa_prefill_workspace_size", "pa_qkv_append", "pa_version",
        "pa_zero_blocks",
    ])


def test_noalloc_scratch_size_is_stated_in_the_header():
    text = HEADER.read_text()
    assert re.search(r"#define PA_DECODE_NOALLOC_SCRATCH_BYTES \(\(size_t\)16 << 20\)", text)
    assert re.search(r"#define PA_DECODE_COUNTER_BYTES \(\(size_t\)256 << 10\)", text)


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr), name


def test_ctypes_signatures_cover_the_header():
    assert sorted(_lib.SIGNATURES) == declared_functions()


def test_host_only_entry_points(lib):
    assert lib.pa_version() == 100
    # no split -> no workspace; a split of 16 blocks over 64 pages -> 4 partial records per (b, h)
    assert lib.pa_decode_workspace_size(8, 8, 64, 64, 0) == 0
    # (arrival counters first: a fixed 256 KiB region; then the records)
    assert lib.pa_decode_workspace_size(8, 8, 64, 64, 16) == (256 << 10) + 8 * 8 * 4 * (64 + 2) * 4
    assert lib.pa_decode_workspace_size(8, 8, 64, 16, 16) == 0
    # prefill: 4 requests x 8 heads x 16 tiles of 16 rows, 58 pages in splits of 16 -> 4 splits
    # (arrival counters first: a fixed 64 KiB region; then the records)
    assert lib.pa_prefill_workspace_size(4, 8, 256, 64, 58, 0) == 0
    assert lib.pa_prefill_workspace_size(4, 8, 256, 64, 58, 16) == (64 << 10) + 4 * 8 * 16 * 4 * 16 * (64 + 2) * 4
    assert lib.pa_prefill_workspace_size(4, 8, 256, 64, 16, 16) == 0
    assert lib.pa_prefill_workspace_size(4, 8, 256, 96, 58, 16) == 0  # no tuned kernel: no split
    # the balanced launch sizes its grid from the device's compute units (none here: no workspace);
    # it never applies to other head_dims or to head counts that are not a multiple of 8
    assert lib.pa_prefill_workspace_size(8, 32, 512, 64, 300, -1) == 0
    assert lib.pa_prefill_workspace_size(8, 32, 512, 96, 300, -1) == 0
    assert lib.pa_prefill_workspace_size(8, 12, 512, 128, 300, -1) == 0  # heads not a multiple of 8


def test_argument_errors_are_reported_without_a_device(lib):
    # invalid sizes are rejected on the host before any HIP call
    st = lib.pa_decode(None, 0, 0, None, 0, 0, 0, None, None, 0, 0, None, 0, 0, None, None, None,
                       1, 0, 64, 16, 1.0, 0, None, 0, None)
    assert st == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"bad sizes" in lib.pa_last_error_message()
    st = lib.pa_kv_append(None, None, 0, 0, 0, 7, None, None, 0, 0, None, 1, 1, 1, 1, 1, None)
    assert st == _lib.PA_ERR_INVALID_ARGUMENT
    # the read probes: whole 16-byte vectors only, at least one workgroup, the shapes they build;
    # nothing to read is a no-op (these calls launch nothing)
    assert lib.pa_hbm_read_probe(0x10000, 24, 0x10000, 8, 512, 8, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"multiple of 16" in lib.pa_last_error_message()
    assert lib.pa_hbm_read_probe(0x10000, 32, 0x10000, 0, 512, 8, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_hbm_read_probe(0x10000, 32, 0x10000, 8, 128, 8, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_hbm_read_probe(0x10000, 32, 0x10000, 8, 512, 2, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_hbm_read_probe(0x10000, 0, 0x10000, 8, 512, 8, None) == _lib.PA_OK
    assert lib.pa_hbm_chunk_read_probe(0x10000, None, 4, 0x10000, 8, 1, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_hbm_chunk_read_probe(0x10000, 0x10000, -1, 0x10000, 8, 1, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_hbm_chunk_read_probe(0x10000, 0x10000, 4, 0x10000, 8, 8, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert lib.pa_hbm_chunk_read_probe(0x10000, 0x10000, 0, 0x10000, 8, 1, None) == _lib.PA_OK
    # zero-sized work is a no-op success
    assert lib.pa_prefill(None, 0, 0, 0, None, 0, 0, 0, 0, None, None, 0, 0, None, 0, 0, None, None,
                          0, 8, 4, 64, 16, 1.0, 0, None, 0, None) == _lib.PA_OK


def test_decode_step_layer_entry_points_check_arguments_on_the_host(lib):
    """pa_linear_rows / pa_qkv_append / pa_embed_rows reject bad arguments before any HIP call
    (the pointers below are never dereferenced: every case fails or returns on the host)."""
    A = 0x10000  # a 16-byte aligned stand-in address
    F32, BF16 = _lib.PA_DTYPE_F32, _lib.PA_DTYPE_BF16
    lin = lib.pa_linear_rows
    # more than 1024 rows
    assert lin(A, 512, 2049, 512, A, None, 512, None, None, 0.0, 0, None, 0, A, 512, None, 0, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"rows must be in [0, 2048]" in lib.pa_last_error_message()
    # unknown activation
    assert lin(A, 512, 4, 512, A, None, 512, None, None, 0.0, 2, None, 0, A, 512, None, 0, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    # unknown element type
    assert lin(A, 512, 4, 512, A, None, 512, None, None, 0.0, 0, None, 0, A, 512, None, 0, 7, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"bad dtype" in lib.pa_last_error_message()
    # misaligned activations
    assert lin(A + 4, 512, 4, 512, A, None, 512, None, None, 0.0, 0, None, 0, A, 512, None, 0, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    # bf16 rows must start on 16-byte boundaries: a row stride of 516 bf16 values does not
    assert lin(A, 516, 4, 512, A, None, 512, None, None, 0.0, 0, None, 0, A, 512, None, 0, BF16, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"multiple of 8" in lib.pa_last_error_message()
    # LayerNorm weight without bias
    assert lin(A, 512, 4, 512, A, None, 512, A, None, 1e-5, 0, None, 0, A, 512, None, 0, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    # in_features without a kernel
    assert lin(A, 96, 4, 96, A, None, 32, None, None, 0.0, 0, None, 0, A, 32, None, 0, F32, None) == _lib.PA_ERR_UNSUPPORTED
    assert b"in_features" in lib.pa_last_error_message()
    # no rows: nothing to do
    assert lin(None, 0, 0, 512, None, None, 512, None, None, 0.0, 0, None, 0, None, 0, None, 0, BF16, None) == _lib.PA_OK
    # the row-selecting form: group_rows must be positive, row_index present, at most 2048 groups
    sel = lib.pa_linear_select_rows
    assert sel(A, 512, 2, 0, A, 512, A, None, 512, None, None, 0.0, 0, A, 512, None, 1, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"group_rows" in lib.pa_last_error_message()
    assert sel(A, 512, 2, 4, None, 512, A, None, 512, None, None, 0.0, 0, A, 512, None, 1, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert sel(A, 512, 2049, 4, A, 512, A, None, 512, None, None, 0.0, 0, A, 512, None, 1, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert sel(A, 96, 2, 4, A, 96, A, None, 32, None, None, 0.0, 0, A, 32, None, 1, F32, None) == _lib.PA_ERR_UNSUPPORTED
    assert sel(None, 0, 0, 4, None, 512, None, None, 512, None, None, 0.0, 0, None, 0, None, 1, F32, None) == _lib.PA_OK
    # greedy-token keys must be 8-byte aligned
    assert sel(A, 512, 2, 4, A, 512, A, None, 512, None, None, 0.0, 0, A, 512, A + 4, 1, F32, None) \
        == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"token_keys" in lib.pa_last_error_message()
    # and their stride positive
    assert sel(A, 512, 2, 4, A, 512, A, None, 512, None, None, 0.0, 0, A, 512, A, 0, F32, None) \
        == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"token_keys_stride" in lib.pa_last_error_message()
    # q/k/v: d_model must be heads x head_dim
    qkv = lib.pa_qkv_append
    assert qkv(A, 512, 2, 512, None, None, 0.0, A, None, A, None, A, None, A, 512, A, A, 0, 8, A, 8, 32, 16,
               F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"d_model" in lib.pa_last_error_message()
    assert qkv(A, 512, 2049, 512, None, None, 0.0, A, None, A, None, A, None, A, 512, A, A, 0, 8, A, 8, 64, 16,
               F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert b"rows must be in [0, 2048]" in lib.pa_last_error_message()
    assert qkv(A, 512, 2, 512, None, None, 0.0, A, None, A, None, A, None, A, 512, A, A, 0, 8, A, 8, 64, 16,
               5, None) == _lib.PA_ERR_INVALID_ARGUMENT
    # embedding rows must be whole 16-byte vectors: 4 fp32 or 8 bf16 values
    emb = lib.pa_embed_rows
    assert emb(A, A, 2, 3, A, 100, A, 64, 6, A, 8, F32, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert emb(A, A, 2, 3, A, 100, A, 64, 12, A, 16, BF16, None) == _lib.PA_ERR_INVALID_ARGUMENT
    assert emb(A, A, 0, 3, A, 100, A, 64, 8, A, 8, F32, None) == _lib.PA_OK
