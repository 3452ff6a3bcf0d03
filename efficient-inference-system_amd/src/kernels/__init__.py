from .paged_attention import paged_attention
