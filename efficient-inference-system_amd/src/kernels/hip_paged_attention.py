"""torch-facing wrappers over the libpaged_hip C ABI (HIP kernels for gfx950).

These replace the reference's Triton launch wrappers with the same argument meaning:
  paged_attention_decode_hip  <- paged_attention_decode_triton  (triton_paged_attention.py:179-217)
  paged_attention_prefill_hip <- paged_attention_prefill_triton (triton_paged_attention.py:220-258)
and add the device-side cache operations the reference does with per-request Python loops:
  kv_append_hip      <- PagedKVCacheState.append slice copies   (src/cache/paged_kv.py:102-120)
  pack_metadata_hip  <- page_table_tensor / seq_lens_tensor      (src/cache/paged_kv.py:174-197)
  zero_blocks_hip    <- LayerBlockPool.release_block zero_()     (src/cache/paged_kv.py:80-85)
  argmax_rows_hip    <- torch.argmax(logits[b, row]).item()      (src/serving/continuous_generate.py:145,238)

All work is enqueued on torch's current stream; nothing here synchronises. Every tensor must live
on a HIP device: there is no CPU path.
"""
from __future__ import annotations

import math

import torch

from src.kernels import _lib

_workspaces: dict[tuple[int, str], torch.Tensor] = {}
_retired_workspaces: list[torch.Tensor] = []
_cu_counts: dict[int, int] = {}


# torch's raw current-stream lookup (one C call, ~0.1 us) where this build of torch has it; the
# public torch.cuda.current_stream(device).cuda_stream builds a Stream object per call (~2 us).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_ptr(device: torch.device) -> int:
    """The current HIP stream of `device` as a raw pointer."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise ValueError(f"{name}: the hip_paged backend needs tensors on a HIP device, got {t.device}")


def _require_i32(name: str, t: torch.Tensor) -> None:
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor (got {t.dtype}, contiguous={t.is_contiguous()})")


def cu_count(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _cu_counts:
        _cu_counts[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _cu_counts[idx]


def _workspace(device: torch.device, nbytes: int, kind: str) -> torch.Tensor:
    """The device's split-K workspace for `kind` ("decode" or "prefill"), at least `nbytes` long.
    Both kinds start with arrival counters of the in-launch merges, which must be zero before first
    use and stay zero between calls: workspaces are zero-filled when allocated, and the two kinds
    are kept apart (their layouts differ). A workspace replaced by a larger one stays allocated
    for the life of the process: a HIP graph a caller captured may hold its address."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = _workspaces.get((idx, kind))
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _retired_workspaces.append(ws)
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _workspaces[(idx, kind)] = ws
    return ws


def default_split_blocks(batch: int, num_heads: int, max_pages: int, device: torch.device) -> int:
    """KV blocks per decode split: 0 (no split) when (request, head) pairs alone fill the GPU or
    the context is at most 256 tokens; 16 blocks when contexts are at most 1024 tokens and the
    pairs fill at most one workgroup per compute unit (at most 4 splits, merged inside the launch:
    8 requests x 8 heads fp32 at 128-1024 tokens, graph replay, 10.4-11.7 us per layer unsplit,
    7.8-8.1 us split); otherwise enough splits for about two workgroups per compute unit, 16 to
    32 blocks each when there are at most 128 pairs, at least 16 blocks above that. Measured
    (graph replay, MI355X): 1-4 requests x 32 heads x 128 bf16 at 8k tokens 26 / 36 / 64 us with
    32-block splits against 74 / 75 / 83 us unsplit."""
    units = batch * num_heads
    target = 2 * cu_count(device)
    if units == 0 or units >= target or max_pages <= 16:
        return 0
    if max_pages <= 64:
        return 16 if units <= cu_count(device) else 0
    splits = math.ceil(target / units)
    blocks = max(16, math.ceil(max_pages / splits))
    if units <= 128:
        blocks = min(blocks, 32)
    return 0 if blocks >= max_pages else blocks


# split_blocks value asking pa_prefill for its balanced launch where the library's policy finds it
# faster (head_dim 128 or 64, heads a multiple of 8: few 128-row tiles over long contexts); other calls
# run unsplit. PAGED_HIP_PREFILL_BALANCE=force / off overrides the policy.
PREFILL_BALANCED = -1


def default_prefill_split_blocks(batch: int, num_heads: int, query_len: int, max_pages: int,
                                 device: torch.device, kv_dtype: torch.dtype | None = None) -> int:
    """split_blocks for a prefill call: PREFILL_BALANCED, so that the library takes the balanced
    launch where it measured faster on MI355X (1 x 32 heads x 128, 512-token chunk over an 8k
    context: bf16 KV 159 -> 96 us, fp32 KV 807 -> 574 us; 1 x 8 heads x 64, 128-token chunk over
    32k: bf16 KV 147 -> 44-47 us, fp32 KV 365 -> 120-123 us) and runs unsplit elsewhere. Fixed split-K
    (split_blocks > 0) is never the default: its second (merge) launch costs more than the load
    balance it buys, from the chunked-prefill workload (4 x 8 heads, 16-row tiles over up to 58
    blocks: 24.5 us unsplit, 32-95 us split) up to 8 x 32 heads with 512-token chunks. Callers may
    still pass split_blocks explicitly. (kv_dtype: accepted for callers that pass it; the policy
    lives in the library.)"""
    return PREFILL_BALANCED


def _check_out(name: str, out: torch.Tensor, q: torch.Tensor) -> None:
    """A caller-supplied output must look like q: the kernels write q's dtype through out's
    b/h/t strides, with unit stride along head_dim."""
    if not out.is_cuda or out.device != q.device:
        raise ValueError(f"{name}: out must be on {q.device}, got {out.device}")
    if out.shape != q.shape or out.dtype != q.dtype:
        raise ValueError(f"{name}: out must match q's shape {tuple(q.shape)} and dtype {q.dtype}, "
                         f"got {tuple(out.shape)} {out.dtype}")
    if out.stride(3) != 1:
        raise ValueError(f"{name}: out must have unit stride along head_dim")


def _check_pool(name: str, k_pool: torch.Tensor, v_pool: torch.Tensor) -> None:
    if k_pool.dim() != 4 or k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype:
        raise ValueError(f"{name}: K/V pools must share shape [num_blocks, H, block_size, head_dim] and dtype")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError(f"{name}: K/V pools must be contiguous")


def paged_attention_decode_hip(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    current_lengths: torch.Tensor,
    *,
    order: torch.Tensor | None = None,
    split_blocks: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Decode attention for q [B, H, 1, Hd]; returns a tensor shaped and strided like q."""
    _require_gpu("paged_attention_decode_hip", q, k_pool, v_pool, page_table, seq_lens, current_lengths)
    _check_pool("paged_attention_decode_hip", k_pool, v_pool)
    B, H, T, Hd = q.shape
    if T != 1:
        raise ValueError(f"decode expects query_len 1, got {T}")
    if q.stride(3) != 1:
        q = q.contiguous()
    nblk, Hp, bs, Hdp = k_pool.shape
    if (Hp, Hdp) != (H, Hd):
        raise ValueError(f"pool heads/head_dim {Hp}/{Hdp} do not match q {H}/{Hd}")
    _require_i32("page_table", page_table)
    _require_i32("seq_lens", seq_lens)
    _require_i32("current_lengths", current_lengths)
    if order is not None:
        _require_i32("order", order)
    if out is None:
        out = torch.empty_like(q)
    _check_out("paged_attention_decode_hip", out, q)
    max_pages = page_table.shape[1] if page_table.dim() == 2 else 0
    pt_stride = page_table.stride(0) if page_table.dim() == 2 and B > 0 else max_pages
    if split_blocks is None:
        split_blocks = default_split_blocks(B, H, max_pages, q.device)
    lib = _lib.load()
    ws_bytes = lib.pa_decode_workspace_size(B, H, Hd, max_pages, split_blocks)
    ws_ptr = _workspace(q.device, ws_bytes, "decode").data_ptr() if ws_bytes else None
    status = lib.pa_decode(
        q.data_ptr(), q.stride(0), q.stride(1),
        out.data_ptr(), out.stride(0), out.stride(1), _lib.dtype_code(q.dtype),
        k_pool.data_ptr(), v_pool.data_ptr(), _lib.dtype_code(k_pool.dtype), nblk,
        page_table.data_ptr() if max_pages else None, pt_stride, max_pages,
        seq_lens.data_ptr(), current_lengths.data_ptr(), order.data_ptr() if order is not None else None,
        B, H, Hd, bs,
        1.0 / math.sqrt(Hd), split_blocks,
        ws_ptr, ws_bytes, _stream_ptr(q.device),
    )
    _lib.check(status, "pa_decode")
    return out


def paged_attention_prefill_hip(
    q: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    page_table: torch.Tensor,
    seq_lens: torch.Tensor,
    current_lengths: torch.Tensor,
    *,
    split_blocks: int | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Chunked causal prefill attention for q [B, H, T, Hd]; returns a tensor shaped like q.
    split_blocks: KV blocks per split-K workgroup (0: none; PREFILL_BALANCED: the balanced launch
    where the library finds it faster; None: default_prefill_split_blocks)."""
    _require_gpu("paged_attention_prefill_hip", q, k_pool, v_pool, page_table, seq_lens, current_lengths)
    _check_pool("paged_attention_prefill_hip", k_pool, v_pool)
    B, H, T, Hd = q.shape
    if q.stride(3) != 1:
        q = q.contiguous()
    nblk, Hp, bs, Hdp = k_pool.shape
    if (Hp, Hdp) != (H, Hd):
        raise ValueError(f"pool heads/head_dim {Hp}/{Hdp} do not match q {H}/{Hd}")
    _require_i32("page_table", page_table)
    _require_i32("seq_lens", seq_lens)
    _require_i32("current_lengths", current_lengths)
    if out is None:
        out = torch.empty_like(q)
    _check_out("paged_attention_prefill_hip", out, q)
    max_pages = page_table.shape[1] if page_table.dim() == 2 else 0
    pt_stride = page_table.stride(0) if page_table.dim() == 2 and B > 0 else max_pages
    if split_blocks is None:
        split_blocks = default_prefill_split_blocks(B, H, T, max_pages, q.device, k_pool.dtype)
    lib = _lib.load()
    ws_bytes = lib.pa_prefill_workspace_size(B, H, T, Hd, max_pages, split_blocks) if bs == 16 else 0
    ws_ptr = _workspace(q.device, ws_bytes, "prefill").data_ptr() if ws_bytes else None
    status = lib.pa_prefill(
        q.data_ptr(), q.stride(0), q.stride(1), q.stride(2),
        out.data_ptr(), out.stride(0), out.stride(1), out.stride(2), _lib.dtype_code(q.dtype),
        k_pool.data_ptr(), v_pool.data_ptr(), _lib.dtype_code(k_pool.dtype), nblk,
        page_table.data_ptr() if max_pages else None, pt_stride, max_pages,
        seq_lens.data_ptr(), current_lengths.data_ptr(),
        B, H, T, Hd, bs,
        1.0 / math.sqrt(Hd), split_blocks,
        ws_ptr, ws_bytes, _stream_ptr(q.device),
    )
    _lib.check(status, "pa_prefill")
    return out


def kv_append_hip(
    k_new: torch.Tensor,
    v_new: torch.Tensor,
    k_pool: torch.Tensor,
    v_pool: torch.Tensor,
    slot_mapping: torch.Tensor,
) -> None:
    """Scatter k_new/v_new [B, H, T, Hd] rows into pool slots (slot_mapping int32 [B*T], -1 = skip)."""
    _require_gpu("kv_append_hip", k_new, v_new, k_pool, v_pool, slot_mapping)
    _check_pool("kv_append_hip", k_pool, v_pool)
    _require_i32("slot_mapping", slot_mapping)
    B, H, T, Hd = k_new.shape
    if v_new.shape != k_new.shape or v_new.dtype != k_new.dtype:
        raise ValueError("k_new and v_new must have the same shape and dtype")
    if k_new.stride() != v_new.stride() or k_new.stride(3) != 1:
        k_new = k_new.contiguous()
        v_new = v_new.contiguous()
    if slot_mapping.numel() != B * T:
        raise ValueError(f"slot_mapping has {slot_mapping.numel()} entries, expected {B * T}")
    nblk, Hp, bs, Hdp = k_pool.shape
    if (Hp, Hdp) != (H, Hd):
        raise ValueError(f"pool heads/head_dim {Hp}/{Hdp} do not match new rows {H}/{Hd}")
    status = _lib.load().pa_kv_append(
        k_new.data_ptr(), v_new.data_ptr(), k_new.stride(0), k_new.stride(1), k_new.stride(2),
        _lib.dtype_code(k_new.dtype),
        k_pool.data_ptr(), v_pool.data_ptr(), _lib.dtype_code(k_pool.dtype), nblk,
        slot_mapping.data_ptr(), B, H, T, Hd, bs, _stream_ptr(k_new.device),
    )
    _lib.check(status, "pa_kv_append")


def pack_metadata_hip(
    block_ids: torch.Tensor,
    row_offsets: torch.Tensor,
    prev_lens: torch.Tensor,
    append_lens: torch.Tensor,
    *,
    query_len: int,
    block_size: int,
    max_pages: int,
    with_slots: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor | None]:
    """Build (page_table int32 [B, max_pages], seq_lens int32 [B], seq_lens int64 [B],
    slot_mapping int32 [B*query_len] or None) on the device from CSR block lists."""
    _require_gpu("pack_metadata_hip", block_ids, row_offsets, prev_lens, append_lens)
    for name, t in (("block_ids", block_ids), ("row_offsets", row_offsets), ("prev_lens", prev_lens),
                    ("append_lens", append_lens)):
        _require_i32(name, t)
    B = prev_lens.numel()
    dev = prev_lens.device
    page_table = torch.empty((B, max_pages), dtype=torch.int32, device=dev)
    seq32 = torch.empty((B,), dtype=torch.int32, device=dev)
    seq64 = torch.empty((B,), dtype=torch.int64, device=dev)
    slots = torch.empty((B * query_len,), dtype=torch.int32, device=dev) if with_slots else None
    status = _lib.load().pa_pack_metadata(
        block_ids.data_ptr() if block_ids.numel() else None, row_offsets.data_ptr(),
        prev_lens.data_ptr(), append_lens.data_ptr(),
        B, query_len, block_size, max_pages,
        page_table.data_ptr() if max_pages else None, max_pages, seq32.data_ptr(), seq64.data_ptr(),
        slots.data_ptr() if slots is not None else None, _stream_ptr(dev),
    )
    _lib.check(status, "pa_pack_metadata")
    return page_table, seq32, seq64, slots


def zero_blocks_hip(k_pool: torch.Tensor, v_pool: torch.Tensor, block_ids: torch.Tensor) -> None:
    """Zero the K and V tiles of the given pool blocks (int32 ids on device) in one launch."""
    _require_gpu("zero_blocks_hip", k_pool, v_pool, block_ids)
    _check_pool("zero_blocks_hip", k_pool, v_pool)
    _require_i32("block_ids", block_ids)
    nblk, H, bs, Hd = k_pool.shape
    status = _lib.load().pa_zero_blocks(
        k_pool.data_ptr(), v_pool.data_ptr(), _lib.dtype_code(k_pool.dtype), nblk, H, bs, Hd,
        block_ids.data_ptr(), block_ids.numel(), _stream_ptr(k_pool.device),
    )
    _lib.check(status, "pa_zero_blocks")


def argmax_rows_hip(logits: torch.Tensor, row_index: torch.Tensor | None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy tokens of a step: out[b] = argmax_v logits[b, row_index[b], v] (int64 [B]) for
    logits [B, T, V] with unit stride along V and rows of one request adjacent (row_index int32
    [B] on the device, negative values count from the end; None means row 0). torch.argmax's
    rules: first index of the maximum, NaN above every number."""
    _require_gpu("argmax_rows_hip", logits)
    if logits.dim() != 3 or logits.stride(2) != 1 or logits.stride(0) != logits.shape[1] * logits.stride(1):
        raise ValueError("argmax_rows_hip: logits must be [B, T, V] with unit stride along V and adjacent rows")
    B, T, V = logits.shape
    if row_index is not None:
        _require_gpu("argmax_rows_hip", row_index)
        _require_i32("row_index", row_index)
        if row_index.numel() < B:
            raise ValueError(f"row_index has {row_index.numel()} entries, expected {B}")
    if out is None:
        out = torch.empty((B,), dtype=torch.int64, device=logits.device)
    elif out.dtype != torch.int64 or not out.is_contiguous() or out.numel() < B or not out.is_cuda:
        raise ValueError("argmax_rows_hip: out must be a contiguous int64 device tensor of at least B entries")
    status = _lib.load().pa_argmax_rows(
        logits.data_ptr(), logits.stride(1), B, T,
        row_index.data_ptr() if row_index is not None else None, V, _lib.dtype_code(logits.dtype),
        out.data_ptr(), _stream_ptr(logits.device),
    )
    _lib.check(status, "pa_argmax_rows")
    return out


def pack_metadata_mirror_hip(
    mirror: torch.Tensor,
    desc_addrs: dict,
    *,
    batch: int,
    query_len: int,
    block_size: int,
    max_pages: int,
    stage_dst: torch.Tensor | None = None,
    stage_words: int = 0,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """pa_pack_metadata_mirror: (page_table int32 [B, max_pages], seq_lens int32 [B], seq_lens int64
    [B], slot_mapping int32 [B * query_len]) from the device block-table mirror (int32 [rows,
    width], updated in place) and a step descriptor given as device addresses (pinned host memory
    the device reads, or device memory) under the keys mirror_row, first_page, num_pages,
    update_ids, prev_lens, append_lens and, with stage_words > 0, stage_src, plus the int
    update_stride (words between two requests' update ids); stage_words int32 words are copied
    from stage_src into stage_dst by the same launch."""
    _require_gpu("pack_metadata_mirror_hip", mirror)
    if mirror.dtype != torch.int32 or mirror.dim() != 2 or mirror.stride(1) != 1:
        raise ValueError("mirror must be an int32 [rows, width] tensor with unit column stride")
    if stage_words:
        if stage_dst is None or stage_dst.dtype != torch.int32 or not stage_dst.is_contiguous() \
                or stage_dst.numel() < stage_words or stage_dst.device != mirror.device:
            raise ValueError("stage_dst must be a contiguous int32 device tensor of at least stage_words words")
    dev = mirror.device
    page_table = torch.empty((batch, max_pages), dtype=torch.int32, device=dev)
    seq32 = torch.empty((batch,), dtype=torch.int32, device=dev)
    seq64 = torch.empty((batch,), dtype=torch.int64, device=dev)
    slots = torch.empty((batch * query_len,), dtype=torch.int32, device=dev)
    d = desc_addrs
    status = _lib.load().pa_pack_metadata_mirror(
        mirror.data_ptr(), mirror.stride(0), mirror.shape[0],
        d["mirror_row"], d["first_page"], d["num_pages"], d["update_ids"], d["update_stride"],
        d["prev_lens"], d["append_lens"],
        batch, query_len, block_size, max_pages,
        page_table.data_ptr() if max_pages else None, max_pages, seq32.data_ptr(), seq64.data_ptr(),
        slots.data_ptr() if slots.numel() else None,
        d.get("stage_src") if stage_words else None, stage_dst.data_ptr() if stage_words else None, stage_words,
        _stream_ptr(dev),
    )
    _lib.check(status, "pa_pack_metadata_mirror")
    return page_table, seq32, seq64, slots
