"""Configuration dataclasses (src/config.py:1-140 of the reference), with the HIP backend.

Differences from the reference, all additive:
  - the default attention backend is "hip_paged" (the reference's is "triton_paged");
  - ModelConfig.kv_cache_dtype (None = the model dtype) selects a bf16 KV pool under an fp32 model;
  - benchmark_serving_request_mix() is the request mix of the end-to-end continuous-batching
    benchmark (200 Poisson requests at 32 req/s), which differs from default_serving_request_mix().
"""
from dataclasses import dataclass, field

import torch


@dataclass(frozen=True)
class RequestWorkloadProfile:
    name: str
    prompt_len_min: int
    prompt_len_max: int
    max_new_tokens_min: int
    max_new_tokens_max: int
    weight: float

    @property
    def prompt_len(self) -> int:
        return self.prompt_len_min

    @property
    def max_new_tokens(self) -> int:
        return self.max_new_tokens_min


def default_serving_request_mix() -> list[RequestWorkloadProfile]:
    """The reference's chat-serving mixture (src/config.py:23-63)."""
    return [
        RequestWorkloadProfile("short_qa", 48, 160, 16, 48, 0.35),
        RequestWorkloadProfile("chat_turn", 128, 320, 32, 96, 0.35),
        RequestWorkloadProfile("rag_answer", 256, 640, 64, 160, 0.20),
        RequestWorkloadProfile("long_summary", 512, 768, 96, 256, 0.10),
    ]


def benchmark_serving_request_mix() -> list[RequestWorkloadProfile]:
    """Mix of the end-to-end continuous-batching benchmark; lengths uniform, inclusive."""
    return [
        RequestWorkloadProfile("short_qa", 16, 64, 16, 64, 0.4),
        RequestWorkloadProfile("chat_turn", 64, 256, 32, 128, 0.3),
        RequestWorkloadProfile("rag_answer", 256, 640, 64, 128, 0.2),
        RequestWorkloadProfile("long_summary", 512, 896, 96, 128, 0.1),
    ]


ATTENTION_BACKENDS = frozenset({"paged_reference", "hip_paged"})


@dataclass
class ModelConfig:
    vocab_size: int = 5000
    d_model: int = 512
    num_heads: int = 8
    num_layers: int = 6
    d_ff: int = 2048
    max_seq_len: int = 1024
    dropout: float = 0.0
    attention_backend: str = "hip_paged"
    kv_block_size: int = 16
    kv_pool_initial_blocks: int = 64
    kv_pool_growth_factor: float = 2.0
    enable_attention_correctness_checks: bool = False
    kv_cache_dtype: torch.dtype | None = None


@dataclass
class ExperimentConfig:
    prompt_lengths: list[int] = field(default_factory=lambda: [128, 256, 512, 768])
    max_new_tokens: int = 128
    batched_backend_batch_size: int = 8
    repeats: int = 3
    seed: int = 42
    batch_size: int = 1
    output_dir: str = "results/kv_cache_analysis"
    warmup_runs: int = 1

    @property
    def device(self) -> str:
        return "cuda" if torch.cuda.is_available() else "cpu"


@dataclass
class SchedulingExperimentConfig:
    arrival_rates: list[float] = field(default_factory=lambda: [4.0, 8.0, 16.0, 24.0, 32.0, 36.0, 44.0, 52.0])
    max_batch_sizes: list[int] = field(default_factory=lambda: [1, 4, 8])
    scheduler_modes: list[str] = field(default_factory=lambda: ["continuous"])
    batch_timeouts_ms: list[float] = field(default_factory=lambda: [0.0, 10.0, 20.0])
    prefill_chunk_sizes: list[int] = field(default_factory=lambda: [128, 256])
    max_tokens_per_iteration: int = 1536
    num_requests: int = 200
    prompt_len: int = 256
    max_new_tokens: int = 16
    heterogeneous_requests: bool = True
    request_workload_profiles: list[RequestWorkloadProfile] = field(default_factory=list)
    repeats: int = 3
    seed: int = 42
    output_dir: str = "results/batching"
    attention_backend: str = "hip_paged"
    kv_block_size: int = 16
    kv_pool_initial_blocks: int = 64
    kv_pool_growth_factor: float = 2.0
    enable_attention_correctness_checks: bool = False

    @property
    def device(self) -> str:
        return "cuda" if torch.cuda.is_available() else "cpu"

    def resolved_request_workload_profiles(self) -> list[RequestWorkloadProfile]:
        if self.heterogeneous_requests:
            return self.request_workload_profiles if self.request_workload_profiles else default_serving_request_mix()
        return [
            RequestWorkloadProfile(
                name="fixed",
                prompt_len_min=self.prompt_len,
                prompt_len_max=self.prompt_len,
                max_new_tokens_min=self.max_new_tokens,
                max_new_tokens_max=self.max_new_tokens,
                weight=1.0,
            )
        ]
