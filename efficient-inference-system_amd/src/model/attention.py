"""Self-attention of the decoder blocks, over the paged KV cache when caching.

Interface of the reference's CausalSelfAttention (src/model/attention.py:9-78): the same
constructor, the four projections q_proj / k_proj / v_proj / out_proj and the dropout module (so
state dicts load across the two), and forward(x, kv_cache, use_cache, current_lengths) returning
(output, cache).

Cached calls follow the paged contract: the step's keys and values enter the cache first
(append_batch, which clamps each request's new-token count to [0, T]), and only then is the
query attended over everything cached, through paged_attention() and the configured backend; a
lone PagedKVCacheState is served as a one-request batch and handed back as the state itself.
Uncached calls are dense causal attention over the call's own tokens.

Head layout: [B, T, d_model] activations are viewed as [B, H, T, head_dim] without a copy
(heads), which is the strided q layout the paged kernels take; attention outputs come back in that
layout and merge_heads flattens them again for out_proj.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from src.cache.paged_kv import BatchedPagedKVCache, PagedKVCacheState
from src.kernels.paged_attention import paged_attention


class CausalSelfAttention(nn.Module):
    def __init__(self, d_model: int, num_heads: int, dropout: float = 0.0, attention_backend: str = "hip_paged"):
        super().__init__()
        if d_model % num_heads:
            raise AssertionError(f"d_model {d_model} is not a multiple of num_heads {num_heads}")
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.attention_backend = attention_backend
        for name in ("q_proj", "k_proj", "v_proj", "out_proj"):
            setattr(self, name, nn.Linear(d_model, d_model))
        self.dropout = nn.Dropout(dropout)

    def heads(self, x: torch.Tensor) -> torch.Tensor:
        """[B, T, d_model] -> [B, H, T, head_dim] view (strides T*d_model, head_dim, d_model, 1)."""
        return x.unflatten(-1, (self.num_heads, self.head_dim)).transpose(1, 2)

    def merge_heads(self, x: torch.Tensor) -> torch.Tensor:
        """[B, H, T, head_dim] -> contiguous [B, T, d_model]."""
        return x.transpose(1, 2).flatten(2).contiguous()

    def _paged(self, q, k, v, kv_cache, current_lengths):
        if isinstance(kv_cache, PagedKVCacheState):
            batch, single = BatchedPagedKVCache(states=[kv_cache], pool=kv_cache.pool), True
        elif isinstance(kv_cache, BatchedPagedKVCache):
            batch, single = kv_cache, len(kv_cache.states) == 1
        else:
            raise ValueError("Paged cached attention requires initialized paged cache state.")
        batch.append_batch(k, v, current_lengths=current_lengths)
        attended = paged_attention(backend=self.attention_backend, q=q, kv_cache=batch,
                                   current_lengths=current_lengths)
        return attended, (batch.states[0] if single else batch)

    def _dense_causal(self, q, k, v):
        # fp32 scores and softmax, one causal mask over the call's own T tokens
        p = self.dropout.p if self.training else 0.0
        return F.scaled_dot_product_attention(q, k, v, dropout_p=p, is_causal=True)

    def forward(
        self,
        x: torch.Tensor,
        kv_cache: PagedKVCacheState | BatchedPagedKVCache | None = None,
        use_cache: bool = False,
        current_lengths: int | torch.Tensor | None = None,
    ) -> tuple[torch.Tensor, PagedKVCacheState | BatchedPagedKVCache | None]:
        q, k, v = (self.heads(proj(x)) for proj in (self.q_proj, self.k_proj, self.v_proj))
        if use_cache:
            attended, cache = self._paged(q, k, v, kv_cache, current_lengths)
        else:
            attended, cache = self._dense_causal(q, k, v), None
        return self.out_proj(self.merge_heads(attended)), cache
