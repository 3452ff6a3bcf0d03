"""torch-facing wrappers of the decode-step linear kernels of libpaged_hip (fp32 or bf16, <= 2048 rows).

  linear_rows_hip  act(LayerNorm(x) W^T + b) + residual in one launch     (pa_linear_rows)
  linear_select_rows_hip  the same without residual for one selected row per group of rows
                   (a step's greedy rows), optionally with the greedy argmax  (pa_linear_select_rows)
  qkv_append_hip   LayerNorm, q/k/v projections and the KV append of a cached attention layer in
                   one launch; returns q                                     (pa_qkv_append)
  embed_rows_hip   token + clamped position embedding of a [B, T] step       (pa_embed_rows)
  mlp_rows_hip     LayerNorm + fc1 + GELU + fc2 (+ residual) of at most 16 fp32 rows in one
                   launch, accumulated into a zeroed output                  (pa_mlp_rows)

They stand in for the nn.LayerNorm / nn.Linear / nn.GELU calls and the append of the
reference's cached forward (src/model/transformer.py:30-35, src/model/attention.py:46-64) on
one-token steps and short prefill chunks, for a model in fp32 or in bf16 (weights and activations of
one dtype; products accumulate in fp32). All work is enqueued on torch's current stream; tensors
must be on a HIP device.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from src.kernels import _lib
from src.kernels.hip_paged_attention import _stream_ptr

MAX_ROWS = 2048  # rows per call accepted by the library
SUPPORTED_FEATURES = (128, 256, 512, 1024, 2048)


def _stream(device: torch.device) -> int:
    return _stream_ptr(device)


def _ptr(t: torch.Tensor | None) -> int | None:
    return t.data_ptr() if t is not None else None


DTYPES = (torch.float32, torch.bfloat16)


def _rows(x: torch.Tensor, name: str, dtype: torch.dtype | None = None) -> None:
    if not x.is_cuda or x.dtype not in DTYPES or x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"{name} must be a float32 or bfloat16 [rows, features] tensor with unit column stride "
                         "on a HIP device")
    if dtype is not None and x.dtype != dtype:
        raise ValueError(f"{name} is {x.dtype}, the layer computes in {dtype}")


def _same_dtype(dtype: torch.dtype, *tensors) -> None:
    for t in tensors:
        if t is not None and t.dtype != dtype:
            raise ValueError(f"all operands must be {dtype}, got a {t.dtype} tensor")


def supported(linear: nn.Linear) -> bool:
    return (linear.weight.dtype in DTYPES and linear.weight.is_contiguous()
            and (linear.bias is None or linear.bias.dtype == linear.weight.dtype)
            and linear.in_features in SUPPORTED_FEATURES)


def linear_rows_hip(x: torch.Tensor, linear: nn.Linear, *, ln: nn.LayerNorm | None = None, gelu: bool = False,
                    residual: torch.Tensor | None = None, out: torch.Tensor | None = None,
                    copy_to: torch.Tensor | None = None) -> torch.Tensor:
    """out[m] = act(LN(x[m]) W^T + b) + residual[m] for the rows of x (at most 2048); x, the layer's
    parameters, residual and out share one dtype (float32 or bfloat16). copy_to: the same rows are
    also written there (it may be residual itself)."""
    _rows(x, "x")
    dt = x.dtype
    M, K = x.shape
    if K != linear.in_features:
        raise ValueError(f"x has {K} features, the layer takes {linear.in_features}")
    _same_dtype(dt, linear.weight, linear.bias, ln.weight if ln is not None else None,
                ln.bias if ln is not None else None)
    N = linear.out_features
    if out is None:
        out = torch.empty((M, N), dtype=dt, device=x.device)
    _rows(out, "out", dt)
    if residual is not None:
        _rows(residual, "residual", dt)
    if copy_to is not None:
        _rows(copy_to, "copy_to", dt)
        if copy_to.shape[0] < M or copy_to.shape[1] < N:
            raise ValueError(f"copy_to must hold {M} rows of {N} features")
    status = _lib.load().pa_linear_rows(
        x.data_ptr(), x.stride(0), M, K,
        linear.weight.data_ptr(), _ptr(linear.bias), N,
        _ptr(ln.weight if ln is not None else None), _ptr(ln.bias if ln is not None else None),
        float(ln.eps) if ln is not None else 0.0,
        1 if gelu else 0, _ptr(residual), residual.stride(0) if residual is not None else 0,
        out.data_ptr(), out.stride(0), _ptr(copy_to), copy_to.stride(0) if copy_to is not None else 0,
        _lib.dtype_code(dt), _stream(x.device),
    )
    _lib.check(status, "pa_linear_rows")
    return out


def linear_select_rows_hip(x: torch.Tensor, group_rows: int, row_index: torch.Tensor, linear: nn.Linear, *,
                           ln: nn.LayerNorm | None = None, gelu: bool = False,
                           out: torch.Tensor | None = None, token_keys: torch.Tensor | None = None) -> torch.Tensor:
    """out[g] = act(LN(x[g * group_rows + r_g]) W^T + b) with r_g = row_index[g] (negative values
    count from the group's end; clamped into the group), for the len(row_index) groups of rows of
    x; x, the layer's parameters and out share one dtype (float32 or bfloat16).

    token_keys (int64 [groups] device tensor, any positive stride, holding -1, i.e. all bits set):
    the same launch folds in each group's greedy token; afterwards the low 32-bit word of
    token_keys[g] holds torch.argmax(out[g]) (see token_keys_to_tokens). Every workgroup sends one
    atomic per group, so keys one 128-byte line apart (a stride of KEY_STRIDE) are faster for
    several groups."""
    _rows(x, "x")
    dt = x.dtype
    M, K = x.shape
    if K != linear.in_features:
        raise ValueError(f"x has {K} features, the layer takes {linear.in_features}")
    if (row_index.dtype != torch.int32 or row_index.dim() != 1 or not row_index.is_contiguous()
            or row_index.device != x.device):
        raise ValueError("row_index must be a contiguous 1-d int32 tensor on x's device")
    groups = row_index.numel()
    if group_rows <= 0 or groups * group_rows > M:
        raise ValueError(f"{groups} groups of {group_rows} rows do not fit in x's {M} rows")
    _same_dtype(dt, linear.weight, linear.bias, ln.weight if ln is not None else None,
                ln.bias if ln is not None else None)
    N = linear.out_features
    if out is None:
        out = torch.empty((groups, N), dtype=dt, device=x.device)
    _rows(out, "out", dt)
    if out.shape[0] < groups or out.shape[1] != N:
        raise ValueError(f"out must hold {groups} rows of {N} features")
    if token_keys is not None and (token_keys.dtype != torch.int64 or token_keys.dim() != 1 or token_keys.numel() < groups
                                   or token_keys.stride(0) < 1 or token_keys.device != x.device):
        raise ValueError("token_keys must be a positively strided int64 [groups] tensor on x's device")
    status = _lib.load().pa_linear_select_rows(
        x.data_ptr(), x.stride(0), groups, group_rows, row_index.data_ptr(), K,
        linear.weight.data_ptr(), _ptr(linear.bias), N,
        _ptr(ln.weight if ln is not None else None), _ptr(ln.bias if ln is not None else None),
        float(ln.eps) if ln is not None else 0.0,
        1 if gelu else 0, out.data_ptr(), out.stride(0), _ptr(token_keys),
        token_keys.stride(0) if token_keys is not None else 1, _lib.dtype_code(dt), _stream(x.device),
    )
    _lib.check(status, "pa_linear_select_rows")
    return out


KEY_STRIDE = 16  # int64 elements: one 128-byte line per group's token key


def token_keys_to_tokens(token_keys: torch.Tensor) -> torch.Tensor:
    """The greedy tokens folded into token_keys by linear_select_rows_hip: the low 32-bit word of
    each key (a strided int32 view of the same memory, no copy)."""
    words = torch.empty(0, dtype=torch.int32, device=token_keys.device)
    return words.set_(token_keys.untyped_storage(), 2 * token_keys.storage_offset(), (token_keys.numel(),),
                      (2 * token_keys.stride(0),))


def qkv_append_hip(x: torch.Tensor, ln: nn.LayerNorm, attn, k_pool: torch.Tensor, v_pool: torch.Tensor,
                   slot_mapping: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """q = LN(x) Wq^T + bq for the rows of x; the K and V rows go straight into their pool slots
    (converted to the pool dtype). x, the projections, LayerNorm and q share one dtype."""
    _rows(x, "x")
    dt = x.dtype
    M, D = x.shape
    _same_dtype(dt, ln.weight if ln is not None else None, ln.bias if ln is not None else None,
                *(t for l in (attn.q_proj, attn.k_proj, attn.v_proj) for t in (l.weight, l.bias)))
    if out is None:
        out = torch.empty((M, D), dtype=dt, device=x.device)
    _rows(out, "out", dt)
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
        slot_mapping.data_ptr(), H, Hd, bs, _lib.dtype_code(dt), _stream(x.device),
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
    dt = token_emb.weight.dtype
    for name, t in (("token_emb", token_emb.weight), ("pos_emb", pos_emb.weight)):
        if t.dtype not in DTYPES or t.dtype != dt or not t.is_contiguous():
            raise ValueError(f"{name} weight must be a contiguous float32 or bfloat16 table (both of one dtype)")
    B, T = ids.shape
    d = token_emb.embedding_dim
    if out is None:
        out = torch.empty((B * T, d), dtype=dt, device=ids.device)
    _rows(out, "out", dt)
    status = _lib.load().pa_embed_rows(
        ids.data_ptr(), pos_start.data_ptr(), B, T, token_emb.weight.data_ptr(), token_emb.num_embeddings,
        pos_emb.weight.data_ptr(), pos_emb.num_embeddings, d, out.data_ptr(), out.stride(0), _lib.dtype_code(dt),
        _stream(ids.device),
    )
    _lib.check(status, "pa_embed_rows")
    return out


MLP_MAX_ROWS = 16
MLP_FEATURES = (128, 256, 512)


def mlp_supported(model) -> bool:
    """True when the model's MLP blocks fit pa_mlp_rows: fp32, d_model 128/256/512, d_ff a
    multiple of 16 (on top of model_supported)."""
    return (model.lm_head.weight.dtype == torch.float32 and model_supported(model)
            and all(blk.mlp[0].in_features in MLP_FEATURES and blk.mlp[0].out_features % 16 == 0
                    and blk.mlp[2].out_features == blk.mlp[0].in_features for blk in model.blocks))


def mlp_rows_hip(x: torch.Tensor, ln: nn.LayerNorm, fc1: nn.Linear, fc2: nn.Linear, out: torch.Tensor, *,
                 residual: torch.Tensor | None = None, gelu: bool = True) -> torch.Tensor:
    """out[m] += fc2(act(fc1(LN(x[m])))) + residual[m] for the (at most 16) rows of x, fp32, in one
    launch: the fc1 column tiles add their shares of fc2 to `out` with atomic adds (so the sum's
    order, and its last bits, vary from run to run). `out` holds the starting value: zeros, or
    the residual rows themselves (then pass residual=None)."""
    _rows(x, "x", torch.float32)
    M, D = x.shape
    if M > MLP_MAX_ROWS:
        raise ValueError(f"mlp_rows_hip takes at most {MLP_MAX_ROWS} rows, got {M}")
    if fc1.in_features != D or fc2.in_features != fc1.out_features or fc2.out_features != D:
        raise ValueError("fc1 must map d_model -> d_ff and fc2 d_ff -> d_model")
    _same_dtype(torch.float32, ln.weight, ln.bias, fc1.weight, fc1.bias, fc2.weight, fc2.bias)
    _rows(out, "out", torch.float32)
    if out.shape[0] < M or out.shape[1] != D:
        raise ValueError(f"out must hold {M} rows of {D} features")
    if residual is not None:
        _rows(residual, "residual", torch.float32)
    status = _lib.load().pa_mlp_rows(
        x.data_ptr(), x.stride(0), M, D, ln.weight.data_ptr(), ln.bias.data_ptr(), float(ln.eps),
        fc1.weight.data_ptr(), _ptr(fc1.bias), fc1.out_features, 1 if gelu else 0,
        fc2.weight.data_ptr(), _ptr(fc2.bias), _ptr(residual), residual.stride(0) if residual is not None else 0,
        out.data_ptr(), out.stride(0), _lib.PA_DTYPE_F32, _stream(x.device),
    )
    _lib.check(status, "pa_mlp_rows")
    return out


def model_supported(model) -> bool:
    """True when every linear layer of the model's cached step fits the fused decode kernels (all
    parameters of one dtype, float32 or bfloat16)."""
    dt = model.lm_head.weight.dtype
    if any(p.dtype != dt for p in model.parameters()):
        return False
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
            and n.weight.dtype in DTYPES and n.bias.dtype == n.weight.dtype
            and tuple(n.normalized_shape) == (n.weight.numel(),))
