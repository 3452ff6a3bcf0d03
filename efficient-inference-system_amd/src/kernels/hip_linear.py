"""torch-facing wrappers of the decode-step linear kernels of libpaged_hip (fp32, <= 64 rows).

  linear_rows_hip  act(LayerNorm(x) W^T + b) + residual in one launch     (pa_linear_rows)
  qkv_append_hip   LayerNorm, q/k/v projections and the KV append of a cached attention layer in
                   one launch; returns q                                     (pa_qkv_append)
  embed_rows_hip   token + clamped position embedding of a [B, T] step       (pa_embed_rows)

They stand in for the nn.LayerNorm / nn.Linear / nn.GELU calls and the append of the
reference's cached forward (src/model/transformer.py:30-35, src/model/attention.py:46-64) on
one-token steps and short prefill chunks. All work is enqueued on torch's current stream; tensors must be on a HIP device.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from src.kernels import _lib

MAX_ROWS = 64
SUPPORTED_FEATURES = (128, 256, 512, 1024, 2048)


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _ptr(t: torch.Tensor | None) -> int | None:
    return t.data_ptr() if t is not None else None


def _rows(x: torch.Tensor, name: str) -> None:
    if not x.is_cuda or x.dtype != torch.float32 or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"{name} must be a float32 [rows, features] tensor with unit column stride on a HIP device")


def supported(linear: nn.Linear) -> bool:
    return (linear.weight.dtype == torch.float32 and linear.weight.is_contiguous()
            and linear.in_features in SUPPORTED_FEATURES)


def linear_rows_hip(x: torch.Tensor, linear: nn.Linear, *, ln: nn.LayerNorm | None = None, gelu: bool = False,
                    residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """out[m] = act(LN(x[m]) W^T + b) + residual[m] for the rows of x (at most 64)."""
    _rows(x, "x")
    M, K = x.shape
    if K != linear.in_features:
        raise ValueError(f"x has {K} features, the layer takes {linear.in_features}")
    N = linear.out_features
    if out is None:
        out = torch.empty((M, N), dtype=torch.float32, device=x.device)
    _rows(out, "out")
    if residual is not None:
        _rows(residual, "residual")
    status = _lib.load().pa_linear_rows(
        x.data_ptr(), x.stride(0), M, K,
        linear.weight.data_ptr(), _ptr(linear.bias), N,
        _ptr(ln.weight if ln is not None else None), _ptr(ln.bias if ln is not None else None),
        float(ln.eps) if ln is not None else 0.0,
        1 if gelu else 0, _ptr(residual), residual.stride(0) if residual is not None else 0,
        out.data_ptr(), out.stride(0), _stream(x.device),
    )
    _lib.check(status, "pa_linear_rows")
    return out


def qkv_append_hip(x: torch.Tensor, ln: nn.LayerNorm, attn, k_pool: torch.Tensor, v_pool: torch.Tensor,
                   slot_mapping: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """q = LN(x) Wq^T + bq for the rows of x; the K and V rows go straight into their pool slots."""
    _rows(x, "x")
    M, D = x.shape
    if out is None:
        out = torch.empty((M, D), dtype=torch.float32, device=x.device)
    nblk, H, bs, Hd = k_pool.shape
    if slot_mapping.dtype != torch.int32 or slot_mapping.numel() < M or not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be a contiguous int32 tensor with one entry per row")
    if k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype or not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("K/V pools must be contiguous with equal shapes and dtypes")
    status = _lib.load().pa_qkv_append(
        x.data_ptr(), x.stride(0), M, D,
        _ptr(ln.weight if ln is not None else None), _ptr(ln.bias if ln is not None else None),
        float(ln.eps) if ln is not None else 0.0,
        attn.q_proj.weight.data_ptr(), _ptr(attn.q_proj.bias), attn.k_proj.weight.data_ptr(), _ptr(attn.k_proj.bias),
        attn.v_proj.weight.data_ptr(), _ptr(attn.v_proj.bias),
        out.data_ptr(), out.stride(0),
        k_pool.data_ptr(), v_pool.data_ptr(), _lib.dtype_code(k_pool.dtype), nblk,
        slot_mapping.data_ptr(), H, Hd, bs, _stream(x.device),
    )
    _lib.check(status, "pa_qkv_append")
    return out


def embed_rows_hip(ids: torch.Tensor, pos_start: torch.Tensor, token_emb: nn.Embedding, pos_emb: nn.Embedding,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """[B*T, d] rows token_emb(ids[b, t]) + pos_emb(min(pos_start[b] + t, max_pos - 1))."""
    if ids.dtype != torch.int64 or pos_start.dtype != torch.int64 or not ids.is_contiguous():
        raise ValueError("ids and pos_start must be int64 (ids contiguous [B, T])")
    if not (pos_start.is_contiguous() and pos_start.numel() == ids.shape[0]):
        raise ValueError("pos_start must be a contiguous [B] tensor")
    for name, t in (("token_emb", token_emb.weight), ("pos_emb", pos_emb.weight)):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"{name} weight must be a contiguous float32 table")
    B, T = ids.shape
    d = token_emb.embedding_dim
    if out is None:
        out = torch.empty((B * T, d), dtype=torch.float32, device=ids.device)
    status = _lib.load().pa_embed_rows(
        ids.data_ptr(), pos_start.data_ptr(), B, T, token_emb.weight.data_ptr(), token_emb.num_embeddings,
        pos_emb.weight.data_ptr(), pos_emb.num_embeddings, d, out.data_ptr(), out.stride(0), _stream(ids.device),
    )
    _lib.check(status, "pa_embed_rows")
    return out


def model_supported(model) -> bool:
    """True when every linear layer of the model's cached step fits the fused decode kernels."""
    for blk in model.blocks:
        a = blk.attn
        fc1, act, fc2 = blk.mlp[0], blk.mlp[1], blk.mlp[2]
        layers = (a.q_proj, a.k_proj, a.v_proj, a.out_proj, fc1, fc2)
        if not all(supported(l) for l in layers):
            return False
        if not isinstance(act, nn.GELU) or act.approximate != "none":
            return False
        if not all(_ln_supported(n) for n in (blk.ln1, blk.ln2)):
            return False
    return supported(model.lm_head) and _ln_supported(model.ln_f)


def _ln_supported(n) -> bool:
    return (isinstance(n, nn.LayerNorm) and n.elementwise_affine and n.bias is not None
            and n.weight.dtype == torch.float32 and tuple(n.normalized_shape) == (n.weight.numel(),))
