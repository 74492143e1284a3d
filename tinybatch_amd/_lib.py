"""ctypes binding of libtinybatch_amd.so (the C ABI in include/tinybatch_amd.h).

The library must be built (``python -m tinybatch_amd.build``); there is no
fallback path: every op raises if the library or a GPU is missing.
torch is imported first so that the library's ``libamdhip64.so.7`` dependency
binds to the HIP runtime torch already loaded (same SONAME) and both share one
runtime, one device context and torch's streams.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the library, see above)

from .build import LIB_PATH

TB_OK = 0
TB_ERR_INVALID_ARG = -1
TB_ERR_UNSUPPORTED = -2
TB_ERR_LAUNCH = -3
TB_ERR_SCRATCH = -4
TB_ERR_INDEX = -5

DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

c_i32, c_i64, c_f32, c_sz, c_vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes); mirrors include/tinybatch_amd.h
SIGNATURES = {
    "tb_status_string": (ctypes.c_char_p, [c_i32]),
    "tb_kv_append": (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_kv_append_rope": (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_vp, c_vp, c_i32,
                                  c_i32, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_linear": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_linear_partials": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_linear_silu_mul": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_linear_argmax_workspace_bytes": (c_sz, [c_i32, c_i32]),
    "tb_linear_argmax": (c_i32, [c_vp, c_i64, c_vp, c_i32, c_i32, c_i32, c_vp, c_sz, c_vp, c_i32, c_vp]),
    "tb_rms_norm_partials": (c_i32, [c_vp, c_i32, c_vp, c_i64, c_vp, c_vp, c_i64, c_i32, c_i32, c_f32, c_i32,
                                     c_vp]),
    "tb_kv_gather": (c_i32, [c_vp, c_i64, c_vp, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_attention_partition_tokens": (c_i32, [c_i32, c_i32]),
    "tb_paged_attention_workspace_bytes": (c_sz, [c_i32, c_i32, c_i32]),
    "tb_paged_attention": (c_i32, [
        c_vp, c_i64,            # q, q_row_stride
        c_vp, c_i64,            # pool, num_blocks
        c_vp, c_i64,            # out, out_row_stride
        c_vp, c_i32,            # block_tables, max_blocks_per_seq
        c_vp, c_i32,            # work_items, num_work_items
        c_vp, c_i32,            # prefill_tiles, num_prefill_tiles
        c_vp, c_i32,            # row_part_offsets, num_rows
        c_vp, c_i32,            # split_rows, num_split_rows
        c_i32, c_i32, c_i32,    # max_parts_per_row, partition_tokens, total_partitions
        c_i32, c_i32, c_i32, c_i32,  # num_heads, num_kv_heads, head_dim, block_size
        c_f32, c_i32,           # scale, dtype
        c_vp, c_i64, c_vp, c_i64,  # k_new, k_row_stride, v_new, v_row_stride
        c_vp, c_sz,             # workspace, workspace_bytes
        c_vp,                   # device_counts
        c_vp, c_vp, c_i32,      # rope_cos, rope_sin, rope_max_position
        c_vp,                   # stream
    ]),
    "tb_step_metadata_counts": (c_i32, [c_vp, c_i32, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_build_step_metadata": (c_i32, [
        c_vp, c_i32, c_vp, c_vp, c_i32,      # query_start_loc, num_seqs, context_lens, positions, num_tokens
        c_vp, c_i32, c_i64, c_i32,           # block_tables, max_blocks_per_seq, num_blocks, block_size
        c_i32, c_i32, c_i32,                 # partition_tokens, rows_per_item, tile_prefill
        c_vp, c_vp,                          # slot_mapping, row_part_offsets
        c_vp, c_i32, c_vp, c_i32, c_vp, c_i32,   # work items, tiles, split rows (+ capacities)
        c_vp,                                # counts
    ]),
    "tb_paged_decode": (c_i32, [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,   # q, q stride, pool, num_blocks, out, out stride
        c_i32, c_vp, c_i32, c_i32, c_i32,        # num_seqs, plan, plan_workgroups, plan_waves, plan_stride
        c_i32, c_i32, c_i32, c_i32, c_f32, c_i32,   # heads, kv heads, head_dim, block_size, scale, dtype
        c_vp, c_i64, c_vp, c_i64,                # k_new, k stride, v_new, v stride
        c_vp, c_sz, c_i32,                       # workspace, bytes, max_pieces
        c_vp, c_i32, c_vp,                       # arrivals, arrival_units, violations
        c_vp, c_vp, c_i32, c_vp,                 # rope cos, sin, max position, stream
    ]),
    "tb_paged_decode_piece_bytes": (c_sz, [c_i32, c_i32, c_i32]),
    "tb_paged_decode_workspace_bytes": (c_sz, [c_i32, c_i32, c_i32, c_i32]),
    "tb_decode_defaults": (c_i32, [c_i32, c_vp, c_vp]),
    "tb_decode_variant_supported": (c_i32, [c_i32, c_i32]),
    "tb_decode_unit_cost": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp]),
    "tb_decode_plan_shape": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "tb_decode_plan_words": (c_sz, [c_i32, c_i32]),
    "tb_build_decode_plan": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32, c_i32, c_i64, c_i32, c_i32, c_i32,
                                     c_i32, c_i32, c_vp, c_sz]),
    "tb_decode_xcc_probe": (c_i32, [c_i32, c_vp, c_vp]),
    "tb_build_decode_segments": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32,
                                         c_i32, c_vp, c_vp, c_i32, c_vp, c_vp, c_vp]),
    "tb_expand_decode_plan": (c_i32, [c_vp, c_i32, c_vp, c_i32, c_i32, c_i64, c_i32, c_i32, c_i32, c_i32, c_vp,
                                      c_vp, c_vp]),
    "tb_paged_prefill": (c_i32, [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,   # q, q stride, pool, num_blocks, out, out stride
        c_vp, c_i32, c_vp, c_i32, c_i32,         # block tables, max_nb, work, num_work, max_tiles
        c_i32, c_i32, c_i32, c_i32, c_f32, c_i32,   # heads, kv heads, head_dim, block_size, scale, dtype
        c_vp, c_i64, c_vp, c_i64,                # k_new, k stride, v_new, v stride (fused append, may be NULL)
        c_vp, c_vp, c_i32, c_vp]),               # rope cos, sin, max position, stream
    "tb_prefill_stream_max_context": (c_i32, [c_i32]),
    "tb_prefill_stream_max_group": (c_i32, [c_i32]),
    "tb_prefill_work_count": (c_i32, [c_vp, c_i32, c_i32]),
    "tb_build_prefill_work": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_vp, c_i32, c_vp]),
    "tb_paged_attention_noalloc": (c_i32, [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32,
        c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_i32, c_f32, c_i32, c_vp, c_i64, c_vp, c_i64,
        c_vp,                   # device_counts (no workspace arguments)
        c_vp, c_vp, c_i32, c_vp,
    ]),
    "tb_paged_attention_merged": (c_i32, [
        c_vp, c_i64, c_vp, c_i64, c_vp, c_i64,   # q, stride, pool, num_blocks, out, stride
        c_vp, c_i32, c_vp, c_i32, c_vp, c_i32,   # block_tables, max_nb, work_items, n, row_part_offsets, rows
        c_i32, c_i32, c_i32,                     # max_parts_per_row, partition_tokens, total_partitions
        c_i32, c_i32, c_i32, c_i32, c_f32, c_i32,   # heads, kv heads, head_dim, block_size, scale, dtype
        c_vp, c_i64, c_vp, c_i64,                # k_new, stride, v_new, stride
        c_vp, c_sz,                              # workspace, bytes
        c_vp, c_i32, c_vp, c_i32, c_vp,          # slot_map, slot_count, arrivals, arrival_units, violations
        c_vp, c_vp, c_i32, c_vp,                 # rope cos, sin, max position, stream
    ]),
    "tb_xcd_slot_map_slots": (c_i32, [c_vp, c_i32, c_i32, c_i32]),
    "tb_build_xcd_slot_map": (c_i32, [c_vp, c_i32, c_i32, c_i32, c_vp, c_i32]),
    "tb_block_copy": (c_i32, [c_vp, c_i32, c_i64, c_vp, c_vp, c_i32, c_i64, c_vp]),
    "tb_block_gather": (c_i32, [c_vp, c_i64, c_vp, c_i32, c_vp, c_i64, c_vp]),
    "tb_block_scatter": (c_i32, [c_vp, c_vp, c_i64, c_vp, c_i32, c_i64, c_vp]),
    "tb_rms_norm": (c_i32, [c_vp, c_i64, c_vp, c_i64, c_vp, c_vp, c_i64, c_i32, c_i32, c_f32, c_i32, c_vp]),
    "tb_rope_qk": (c_i32, [c_vp, c_i64, c_vp, c_vp, c_vp, c_i32, c_vp, c_vp, c_i32, c_i32, c_i32, c_i32, c_i32,
                           c_vp]),
    "tb_silu_mul": (c_i32, [c_vp, c_i64, c_vp, c_i64, c_i32, c_i32, c_i32, c_vp]),
}

_LIB: ctypes.CDLL | None = None


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    with open("/proc/self/maps") as f:
        for line in f:
            if "libamdhip64" in line:
                paths.add(os.path.realpath(line.split()[-1]))
    return paths


def lib() -> ctypes.CDLL:
    """Load (once) and return the library; raises if it has not been built."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m tinybatch_amd.build` "
            "(there is no CPU fallback for the paged KV-cache kernels)")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    runtimes = _hip_runtimes_mapped()
    if len(runtimes) > 1:
        raise RuntimeError(f"two HIP runtimes are mapped in this process: {sorted(runtimes)}")
    _LIB = handle
    return handle


def check(status: int, what: str) -> None:
    if status != TB_OK:
        msg = lib().tb_status_string(status).decode()
        raise RuntimeError(f"{what} failed: {msg} (status {status})")


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu_tensor(name: str, t: torch.Tensor) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a GPU tensor (no CPU fallback); got device {t.device}")
