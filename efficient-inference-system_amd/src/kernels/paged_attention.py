"""Backend dispatch for paged attention: the drop-in boundary of the hot path.

Same signature and contract as src/kernels/paged_attention.py:13-51 of the reference:
`paged_attention(backend, q [B, H, T, Hd], kv_cache, current_lengths) -> [B, H, T, Hd]`, called
after `kv_cache.append_batch(...)`. current_lengths is normalised to an int32 device tensor
(None -> T, int -> that value, tensor -> cast), then query_len 1 goes to the decode kernel and
anything longer to the chunked-prefill kernel.

Backends: "paged_reference" (torch, any device) and "hip_paged" (libpaged_hip.so on a HIP device).
Unlike the reference, which silently sends CPU tensors to its torch loop, "hip_paged" refuses
tensors that are not on a HIP device, so a run of this backend always executes the HIP kernels.
"""
from __future__ import annotations

import torch

from src.cache.paged_kv import BatchedPagedKVCache
from src.config import ATTENTION_BACKENDS
from src.kernels.reference_paged_attention import paged_attention_reference
from src.kernels.staging import upload

_const_lengths: dict[tuple, torch.Tensor] = {}
_last_host_lengths: dict[str, tuple] = {}


def _lengths_tensor(current_lengths, batch_size: int, query_len: int, device: torch.device) -> torch.Tensor:
    if current_lengths is None or isinstance(current_lengths, int):
        value = query_len if current_lengths is None else current_lengths
        key = (device.index if device.index is not None else torch.cuda.current_device(), batch_size, value)
        t = _const_lengths.get(key)
        if t is None:
            t = torch.full((batch_size,), value, device=device, dtype=torch.int32)
            _const_lengths[key] = t
        return t
    if not current_lengths.is_cuda:
        # Host lengths (the model passes them this way, the same tensor to every layer): one
        # asynchronous upload per tensor version, reused by the following layers.
        key = (id(current_lengths), current_lengths._version, device.index)
        hit = _last_host_lengths.get("last")
        if hit is not None and hit[0] == key and hit[1] is current_lengths:
            return hit[2]
        dev = upload(current_lengths.to(torch.int32).contiguous().numpy(), device)
        _last_host_lengths["last"] = (key, current_lengths, dev)
        return dev
    return current_lengths.to(device=device, dtype=torch.int32).contiguous()


def paged_attention(
    backend: str,
    q: torch.Tensor,
    kv_cache: BatchedPagedKVCache,
    current_lengths: int | torch.Tensor | None,
) -> torch.Tensor:
    if backend not in ATTENTION_BACKENDS:
        raise ValueError(f"Unsupported paged attention backend: {backend}")

    if backend == "paged_reference":
        return paged_attention_reference(q=q, kv_cache=kv_cache, current_lengths=current_lengths)

    if not q.is_cuda:
        raise ValueError(
            "the hip_paged backend runs on a HIP device only; got q on "
            f"{q.device} (select 'paged_reference' for CPU tensors)"
        )
    from src.kernels.hip_paged_attention import paged_attention_decode_hip, paged_attention_prefill_hip

    pool = kv_cache.pool
    batch_size, _, query_len, _ = q.shape
    if pool.k_blocks is None:
        return torch.zeros_like(q)
    page_table, seq_lens = kv_cache.device_metadata(q.device)
    cur = _lengths_tensor(current_lengths, batch_size, query_len, q.device)
    if query_len == 1:
        return paged_attention_decode_hip(q, pool.k_blocks, pool.v_blocks, page_table, seq_lens, cur)
    return paged_attention_prefill_hip(q, pool.k_blocks, pool.v_blocks, page_table, seq_lens, cur)
