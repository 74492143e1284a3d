"""tinybatch_amd — MI355X (gfx950) paged KV-cache data path for tinybatch.

Hand-written HIP kernels behind a C ABI (include/tinybatch_amd.h):
K1 KV append, K2 fused paged attention, K3 block copy/gather; a drop-in
PagedKVCache (src/tinybatch/kv_cache.py of the reference) on top.
"""
from .metadata import StepMetadata, build_step_metadata
from .kv_cache import PagedKVCache
from . import ops

__all__ = ["PagedKVCache", "StepMetadata", "build_step_metadata", "ops"]
