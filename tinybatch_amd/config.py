"""Engine configuration (counterpart of src/tinybatch/config.py:7-35).

The model is a random-initialised Qwen2 of the configured shape (no
checkpoint or tokenizer is loaded: requests are token ids), run in bf16 on the
GPU by default.
"""
from __future__ import annotations

from dataclasses import dataclass, field


@dataclass
class EngineConfig:
    device: str = "cuda"
    dtype: str = "bfloat16"
    # paged KV cache
    block_size: int = 16
    num_blocks: int = 512
    enable_prefix_caching: bool = True
    # scheduler
    max_batch_tokens: int = 2048
    max_running: int = 32
    max_model_len: int = 4096
    # "recompute": a preempted sequence restarts from its prompt (the reference,
    # scheduler.py:141-149); "swap": its KV blocks go to pinned host memory
    # (K3 gather) and come back (K3 scatter) when blocks are free again
    preemption: str = "recompute"
    # sampling defaults
    max_new_tokens: int = 256
    temperature: float = 0.0
    top_p: float = 1.0
    stop_token_ids: tuple = field(default_factory=tuple)
    # decode-only steps replay a captured HIP graph per batch-size bucket
    decode_graphs: bool = True
    # steady greedy decode queues step N+1 before step N's tokens reach the host
    # (the host's scheduling and packing then overlap the GPU's step)
    pipeline_decode: bool = True
    # random-init weights
    seed: int = 0

    def kv_pool_tokens(self) -> int:
        return self.block_size * self.num_blocks
