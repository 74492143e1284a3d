"""Functional wrappers over the C ABI: argument checks, then one ctypes call.

Every function launches on the current torch stream of the tensors' device
and returns without synchronising. Temporary device arguments (block-id
lists, pointer arrays) come from torch's caching allocator on that same
stream, so their reuse is ordered after the kernel that reads them. Errors are raised on the host before any
launch: shape/dtype/device mismatches as ValueError/TypeError, out-of-range
block ids or positions as IndexError (as the reference's tensor indexing
would), and a rejected launch as RuntimeError.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib
from .metadata import StepMetadata

_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def _ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _check_pool(pool: torch.Tensor) -> tuple[int, int, int, int]:
    _lib.require_gpu_tensor("pool", pool)
    if pool.dim() != 5 or pool.shape[1] != 2:
        raise ValueError(f"pool must be [num_blocks, 2, kv_heads, block_size, head_dim], got {tuple(pool.shape)}")
    if not pool.is_contiguous():
        raise ValueError("pool must be contiguous")
    if pool.dtype not in _lib.DTYPE_CODE:
        raise TypeError(f"unsupported pool dtype {pool.dtype}")
    nb, _, hkv, bs, d = pool.shape
    return nb, hkv, bs, d


class Rope:
    """RoPE tables for the fused rotations: fp32 cos / sin [max_position, head_dim / 2]
    on the GPU (the angles of the reference's _rope, model.py:74-76)."""

    def __init__(self, cos: torch.Tensor, sin: torch.Tensor):
        for name, t in (("cos", cos), ("sin", sin)):
            _lib.require_gpu_tensor(name, t)
            if t.dtype != torch.float32 or t.dim() != 2 or not t.is_contiguous():
                raise TypeError(f"rope {name} must be a contiguous fp32 [max_position, head_dim/2] tensor")
        if cos.shape != sin.shape:
            raise ValueError("rope cos and sin differ in shape")
        self.cos, self.sin = cos, sin
        self.max_position, self.half = cos.shape

    def check(self, head_dim: int, device: torch.device) -> None:
        if 2 * self.half != head_dim:
            raise ValueError(f"rope tables are for head_dim {2 * self.half}, not {head_dim}")
        if self.cos.device != device:
            raise ValueError("rope tables are on another device")


def _rows_view(name: str, t: torch.Tensor, n_heads: int, d: int) -> int:
    """Validate a [T, n_heads, D] (or [T, n_heads*D]) tensor with contiguous rows; return its row stride."""
    if t.dim() == 3:
        if t.shape[1] != n_heads or t.shape[2] != d:
            raise ValueError(f"{name} must be [T, {n_heads}, {d}], got {tuple(t.shape)}")
        if t.stride(2) != 1 or t.stride(1) != d:
            raise ValueError(f"{name} must have contiguous [heads, head_dim] rows")
    elif t.dim() == 2:
        if t.shape[1] != n_heads * d:
            raise ValueError(f"{name} must be [T, {n_heads * d}], got {tuple(t.shape)}")
        if t.stride(1) != 1:
            raise ValueError(f"{name} must have contiguous rows")
    else:
        raise ValueError(f"{name} must be 2-D or 3-D, got {t.dim()}-D")
    return t.stride(0) if t.shape[0] > 1 else n_heads * d


def kv_append(pool: torch.Tensor, k: torch.Tensor, v: torch.Tensor, slot_mapping: torch.Tensor,
              rope: Rope | None = None, positions: torch.Tensor | None = None) -> None:
    """K1: pool[slot] <- (k, v) for every token with slot >= 0 (reference kv_cache.py:25-38).
    With ``rope`` (and int64 device ``positions``) k is rotated at its position on the way
    (tb_kv_append_rope: the reference's _rope of k, model.py:72-80, folded into the write)."""
    nb, hkv, bs, d = _check_pool(pool)
    for name, t in (("k", k), ("v", v)):
        _lib.require_gpu_tensor(name, t)
        if t.dtype != pool.dtype:
            raise TypeError(f"{name} dtype {t.dtype} != pool dtype {pool.dtype}")
    ks = _rows_view("k", k, hkv, d)
    vs = _rows_view("v", v, hkv, d)
    T = k.shape[0]
    if v.shape[0] != T or slot_mapping.numel() != T:
        raise ValueError("k, v and slot_mapping disagree on the number of tokens")
    if slot_mapping.dtype != torch.int32 or not slot_mapping.is_cuda or not slot_mapping.is_contiguous():
        raise TypeError("slot_mapping must be a contiguous int32 GPU tensor")
    if rope is None:
        st = _lib.lib().tb_kv_append(k.data_ptr(), ks, v.data_ptr(), vs, pool.data_ptr(), nb,
                                     slot_mapping.data_ptr(), T, hkv, d, bs,
                                     _lib.DTYPE_CODE[pool.dtype], _lib.stream_handle(pool.device))
        _lib.check(st, "tb_kv_append")
        return
    rope.check(d, pool.device)
    if (positions is None or positions.dtype != torch.int64 or not positions.is_cuda
            or not positions.is_contiguous() or positions.numel() != T):
        raise TypeError("rope needs positions: a contiguous int64 GPU tensor with one entry per token")
    st = _lib.lib().tb_kv_append_rope(k.data_ptr(), ks, v.data_ptr(), vs, pool.data_ptr(), nb,
                                      slot_mapping.data_ptr(), positions.data_ptr(), rope.cos.data_ptr(),
                                      rope.sin.data_ptr(), rope.max_position, T, hkv, d, bs,
                                      _lib.DTYPE_CODE[pool.dtype], _lib.stream_handle(pool.device))
    _lib.check(st, "tb_kv_append_rope")


def kv_gather(pool: torch.Tensor, table: torch.Tensor, context_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Contiguous K, V [context_len, kv_heads, head_dim] of one sequence (reference kv_cache.py:40-45)."""
    nb, hkv, bs, d = _check_pool(pool)
    if table.dtype != torch.int32 or not table.is_cuda or not table.is_contiguous():
        raise TypeError("table must be a contiguous int32 GPU tensor")
    k_out = torch.empty(context_len, hkv, d, device=pool.device, dtype=pool.dtype)
    v_out = torch.empty_like(k_out)
    st = _lib.lib().tb_kv_gather(pool.data_ptr(), nb, table.data_ptr(), int(context_len), k_out.data_ptr(),
                                 v_out.data_ptr(), hkv, d, bs, _lib.DTYPE_CODE[pool.dtype],
                                 _lib.stream_handle(pool.device))
    _lib.check(st, "tb_kv_gather")
    return k_out, v_out


def heads_per_group(dtype: torch.dtype, num_heads: int, num_kv_heads: int) -> int:
    """Query heads one work item serves (the C dispatch uses the same rule)."""
    rep = num_heads // num_kv_heads
    cap = 16 if dtype in (torch.float16, torch.bfloat16) else 8
    return max(t for t in range(1, cap + 1) if rep % t == 0)


def rows_per_item(dtype: torch.dtype, num_heads: int, num_kv_heads: int) -> int:
    """Consecutive query rows one 16-bit work item serves: its MFMA operand holds
    16 (row, head) columns. fp32 items serve one row."""
    if dtype not in (torch.float16, torch.bfloat16):
        return 1
    return max(1, 16 // heads_per_group(dtype, num_heads, num_kv_heads))


def partition_tokens(dtype: torch.dtype, head_dim: int) -> int:
    """Default attention partition length (positions per wave) for this element type."""
    return int(_lib.lib().tb_attention_partition_tokens(_lib.DTYPE_CODE[dtype], head_dim))


def workspace_for(meta: StepMetadata, num_heads: int, head_dim: int,
                  device: torch.device) -> torch.Tensor | None:
    """Split-row partials buffer, grown on demand and cached per device and stream:
    calls on one stream are ordered, so consecutive calls can share it; calls on two
    streams may overlap in time, so each stream has its own."""
    if meta.max_parts_per_row <= 1:
        return None
    need = int(_lib.lib().tb_paged_attention_workspace_bytes(meta.total_partitions, num_heads, head_dim))
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < need:
        ws = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


class DecodeDevice:
    """Launch facts of the decode kernel on one GPU: one workgroup per CU, and the XCD
    count under which a unit's partials are written and merged inside one XCD. The XCD
    count is the CU count / 32 (the CUs of one XCD); the decode kernel is used only if
    a probe launch shows workgroup g running on XCD g mod that count, with distinct
    XCDs in between (merge_in_kernel), and steps go to the work-item kernel otherwise."""

    def __init__(self, device: torch.device):
        props = torch.cuda.get_device_properties(device)
        cus = int(props.multi_processor_count)
        self.device = device
        self.workgroups = cus
        nx = cus // 32 if cus % 32 == 0 and cus >= 32 else 1
        self.num_xcds, self.merge_in_kernel = self._verify(device, cus, nx)
        # the error count of the in-launch merges (tb_paged_decode, tb_paged_attention_merged):
        # nonzero after a call whose outputs cannot be trusted (a unit's partials on two
        # XCDs, a malformed plan, a refused fused append); ordinary tensors even when the
        # device is first used under inference mode (they are updated in place later)
        with torch.inference_mode(False):
            self.violations = torch.zeros(1, dtype=torch.int32, device=device)
            self._host_errors = torch.zeros(1, dtype=torch.int32).pin_memory()

    def errors_async(self) -> torch.Tensor:
        """Queue a copy of the error count on the current stream into pinned host memory;
        the returned tensor holds it once the stream passes that point (read it after the
        next synchronisation, e.g. the step's token copy)."""
        self._host_errors.copy_(self.violations, non_blocking=True)
        return self._host_errors

    def errors(self) -> int:
        """The error count now (synchronises the device)."""
        return int(self.violations.item())

    def disable_merges(self) -> None:
        """After a nonzero error count: no more in-launch merges on this device (every
        later step goes to the work-item kernel, whose split rows a separate kernel
        merges), and the count back to zero."""
        self.merge_in_kernel = False
        self.violations.zero_()
        for key in [k for k in _DECODE_WORKSPACES if k[0] == self.device.index]:
            del _DECODE_WORKSPACES[key]      # arrival counters a failed call may have left nonzero

    @staticmethod
    def _verify(device, cus: int, nx: int) -> tuple[int, bool]:
        g = 8 * cus
        out = torch.full((g,), -1, dtype=torch.int32, device=device)
        with torch.cuda.device(device):
            _lib.check(_lib.lib().tb_decode_xcc_probe(g, out.data_ptr(), _lib.stream_handle(device)),
                       "tb_decode_xcc_probe")
        x = out.cpu().numpy()
        if nx <= 1:
            return 1, bool(np.all(x == x[0]))
        ok = len(set(x[:nx].tolist())) == nx and bool(np.all(x == np.tile(x[:nx], g // nx)))
        return (nx, True) if ok else (1, False)


_DECODE_DEVICES: dict[int, DecodeDevice] = {}
_DECODE_WORKSPACES: dict[tuple[int, int], "DecodeBuffers"] = {}


def decode_device(device: torch.device) -> DecodeDevice:
    """The device's DecodeDevice (built on first use: a probe launch and a synchronisation,
    so not while a graph is being captured)."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    d = _DECODE_DEVICES.get(key)
    if d is None:
        d = _DECODE_DEVICES[key] = DecodeDevice(torch.device("cuda", key))
    return d


# Decode-only steps with at least this many K/V bytes per call go to the streaming
# decode kernel (tb_paged_decode); smaller steps to the work-item kernel, whose
# fixed cost per call is lower. Measured on the Qwen 0.5B layer geometry (fp16,
# block 16, 24 rotating pools), us per call streaming / work items: 8 sequences
# (12 MB of K/V) 11.3 / 10.2, 16 (22 MB) 11.7 / 12.3, 24 (30 MB) 12.2 / 13.1,
# 48 (57 MB) 15.6 / 18.2 (eight-wave form). With the four-wave default: 8 sequences
# 10.9 / 9.7 (16 units), 16 sequences 10.8 / 11.9, and the engine's decode shape
# (bf16, 32 sequences of 400..770 positions, 9.5 MB) 8.3 / 8.5 against the merged
# items: the crossover now lies near 8 MiB at >= 32 units. The threshold stays
# at 16 MiB: below it the gain is <= 2%, and lower would also split the engine's
# mixed steps, whose prefill shapes were not measured split.
DECODE_KERNEL_MIN_BYTES = 16 << 20


def prefill_route(dtype: torch.dtype, num_heads: int, num_kv_heads: int, head_dim: int,
                  device: torch.device | None = None):
    """The PrefillRoute (build_step_metadata's prefill_route) that sends whole prefill
    sequences to tb_paged_prefill for this geometry, or None where that kernel does not
    serve it (fp32, head dims other than 64 / 128, too many query heads per kv head).
    With ``device``, the work of one (sequence, kv head) is placed on one of its XCDs
    when the device runs workgroup g on XCD g mod the XCD count (DecodeDevice)."""
    from .metadata import PrefillRoute

    if dtype not in (torch.float16, torch.bfloat16) or num_kv_heads <= 0 or num_heads % num_kv_heads:
        return None
    lib = _lib.lib()
    max_ctx = int(lib.tb_prefill_stream_max_context(head_dim))
    if max_ctx <= 0 or num_heads // num_kv_heads > int(lib.tb_prefill_stream_max_group(head_dim)) \
            or num_kv_heads > 127:
        return None
    xcds = 1
    if device is not None and device.type == "cuda":
        d = decode_device(device)
        xcds = d.num_xcds if d.merge_in_kernel else 1
    return PrefillRoute(num_kv_heads, head_dim, max_ctx, xcds)


def decode_kernel_preferred(meta: StepMetadata, *, num_kv_heads: int, head_dim: int, dtype: torch.dtype,
                            min_bytes: int = DECODE_KERNEL_MIN_BYTES) -> bool:
    """Whether a step is served faster by the streaming decode kernel: a decode-only
    step (row b = sequence b) in fp16 / bf16 reading at least ``min_bytes`` of K/V
    (DECODE_KERNEL_MIN_BYTES by default), with at least 32 (sequence, kv head) units (a unit stays on one XCD, so
    fewer units leave XCDs idle). The plan must then be attached (attach_decode_plan)
    before meta.to()."""
    if not meta.rows_are_seqs or dtype not in (torch.float16, torch.bfloat16):
        return False
    if meta.num_seqs * num_kv_heads < 32:
        return False
    kv_bytes = int(meta.row_ctx_np[:meta.num_seqs].astype(np.int64).sum()) * num_kv_heads * head_dim * 2 * 2
    return kv_bytes >= min_bytes


def decode_waves_for(meta: StepMetadata, *, num_kv_heads: int, head_dim: int) -> int | None:
    """The decode kernel variant (waves per workgroup) for a decode-only step: None, the
    library's default for the head dim (tb_decode_defaults). At head dim 64 that is four
    waves with two tile pairs in flight each; same-box graph runs on the Qwen layer
    (fp16, 64 sequences, 24 pools, us per call four / six / eight waves): 17.94 / 18.23 /
    18.10 on one box, 17.59 / - / 18.05 on another (bench.py --decode-waves picks another)."""
    return None


def attach_decode_plan(meta: StepMetadata, *, num_heads: int, num_kv_heads: int, head_dim: int,
                       dtype: torch.dtype, device: torch.device, waves: int | None = None,
                       unit_cost: int | None = None, on_device: bool = True) -> bool:
    """metadata.attach_decode_plan with this device's workgroups and XCDs (by default the
    plan's entries are written on the device by meta.to: the host assigns the tiles
    only); False (the
    step stays with the work-item kernel) when the device's workgroup placement is not
    the one the kernel's in-XCD merges assume. ``waves`` None: the library's default
    variant (decode_waves_for)."""
    from .metadata import attach_decode_plan as attach

    d = decode_device(device)
    if not d.merge_in_kernel or d.num_xcds <= 1:
        return False
    if waves is None:
        waves = decode_waves_for(meta, num_kv_heads=num_kv_heads, head_dim=head_dim)
    return attach(meta, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim, dtype=dtype,
                  workgroups=d.workgroups, num_xcds=d.num_xcds, waves=waves, unit_cost=unit_cost,
                  on_device=on_device)


def attach_split_parts(meta: StepMetadata, positions, seq_slices, block_tables, context_lens, *, num_heads: int,
                       num_kv_heads: int, head_dim: int, dtype: torch.dtype, device: torch.device,
                       rows: int | None = None) -> bool:
    """For a mixed step of whole prefills (that tb_paged_prefill serves) on one side
    and decode rows on the other (metadata.split_step_parts), attach the two
    sub-steps to ``meta`` (before meta.to()) when the decode side is one the
    streaming decode kernel serves faster (decode_kernel_preferred):
    paged_attention then runs tb_paged_prefill on the prefill rows and
    tb_paged_decode on the decode rows, in place of one launch of prefill tiles
    and decode work items. Returns whether it did."""
    from .metadata import split_step_parts

    route = prefill_route(dtype, num_heads, num_kv_heads, head_dim, device)
    if route is None or meta.decode_only or context_lens is None:
        return False
    # the decode side's size first (the sub-steps are only built when it qualifies)
    dec_ctx = [int(c) for (b, e), c in zip(seq_slices, context_lens) if int(e) - int(b) == 1]
    if len(dec_ctx) * num_kv_heads < 32 or \
            sum(dec_ctx) * num_kv_heads * head_dim * 2 * 2 < DECODE_KERNEL_MIN_BYTES:
        return False
    if rows is None:                 # query rows per work item, as the full step's metadata
        rows = rows_per_item(dtype, num_heads, num_kv_heads)
    parts = split_step_parts(positions, seq_slices, block_tables, context_lens, block_size=meta.block_size,
                             num_blocks=meta.num_blocks, partition_tokens=meta.partition_tokens,
                             rows_per_item=rows, prefill_route=route)
    if parts is None:
        return False
    dec = next(m for _, _, m in parts if m.decode_only)
    if not decode_kernel_preferred(dec, num_kv_heads=num_kv_heads, head_dim=head_dim, dtype=dtype):
        return False
    if not attach_decode_plan(dec, num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                              dtype=dtype, device=device):
        return False
    meta.parts = parts
    return True


def attach_xcd_slot_map(meta: StepMetadata, *, num_heads: int, num_kv_heads: int, dtype: torch.dtype,
                        device: torch.device) -> bool:
    """metadata.attach_xcd_slot_map with this device's XCDs, when the device runs workgroup
    g on XCD g mod the XCD count (DecodeDevice); before meta.to(). Returns whether the
    step's split rows will be merged inside the launch."""
    from .metadata import attach_xcd_slot_map as attach

    d = decode_device(device)
    if not d.merge_in_kernel or d.num_xcds <= 1:
        return False
    return attach(meta, num_heads=num_heads, num_kv_heads=num_kv_heads, dtype=dtype, num_xcds=d.num_xcds)


def decode_workspace_bytes(meta: StepMetadata, num_heads: int, num_kv_heads: int, head_dim: int) -> int:
    return int(_lib.lib().tb_paged_decode_workspace_bytes(meta.decode_pieces, num_heads, num_kv_heads, head_dim))


class DecodeBuffers:
    """The decode kernel's partials workspace and its arrival counters (128 bytes per
    unit, zero between calls: every call leaves them zero)."""

    def __init__(self, device: torch.device, piece_bytes: int, units: int):
        self.pieces = torch.empty(max(piece_bytes, 1 << 16), dtype=torch.uint8, device=device)
        self.units = max(units, 256)
        self.arrivals = torch.zeros(self.units * 16, dtype=torch.int64, device=device)


def decode_buffers(device: torch.device, piece_bytes: int, units: int) -> DecodeBuffers:
    """Cached per device and stream (calls on one stream are ordered; calls on two
    streams must not share counters); grown on demand, new counters zeroed."""
    key = (device.index if device.index is not None else torch.cuda.current_device(),
           torch.cuda.current_stream(device).cuda_stream)
    b = _DECODE_WORKSPACES.get(key)
    if b is None or b.pieces.numel() < piece_bytes or b.units < units:
        b = DecodeBuffers(device, max(piece_bytes, 0 if b is None else b.pieces.numel()),
                          max(units, 0 if b is None else b.units))
        _DECODE_WORKSPACES[key] = b
    return b


def paged_decode(q: torch.Tensor, pool: torch.Tensor, meta: StepMetadata, *, num_heads: int,
                 scale: float | None = None, out: torch.Tensor | None = None,
                 k_new: torch.Tensor | None = None, v_new: torch.Tensor | None = None,
                 workspace: "DecodeBuffers | None" = None, rope: Rope | None = None) -> torch.Tensor:
    """tb_paged_decode: the decode kernel for a step whose metadata carries a decode plan
    (attach_decode_plan). Arguments and result as paged_attention; ``workspace`` is a
    DecodeBuffers (by default one cached per device and stream)."""
    nb, hkv, bs, d = _check_pool(pool)
    if meta.decode_plan is None:
        raise ValueError("metadata has no uploaded decode plan (attach_decode_plan, then meta.to(device))")
    if meta.num_blocks > nb:
        raise ValueError(f"the decode plan indexes a pool of {meta.num_blocks} blocks; this pool holds {nb}")
    _lib.require_gpu_tensor("q", q)
    if q.dtype != pool.dtype or q.dtype not in (torch.float16, torch.bfloat16):
        raise TypeError("the decode kernel takes fp16 / bf16 q in the pool dtype")
    qs = _rows_view("q", q, num_heads, d)
    B = meta.num_seqs
    if q.shape[0] != B:
        raise ValueError(f"q has {q.shape[0]} rows, the decode step {B}")
    if out is None:
        out = torch.empty(B, num_heads * d, device=q.device, dtype=q.dtype)
    _lib.require_gpu_tensor("out", out)
    if out.dtype != q.dtype or out.shape[0] != B:
        raise ValueError("out must match q's dtype and row count")
    os_ = _rows_view("out", out, num_heads, d)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if rope is not None:
        rope.check(d, q.device)
    ksp = vsp = None
    ks = vs = 0
    if k_new is not None or v_new is not None:
        if k_new is None or v_new is None:
            raise ValueError("k_new and v_new go together")
        sm = meta.slot_mapping_np
        if sm.size and np.any(sm[:B] < 0):
            raise ValueError("two decode rows write one pool slot; the fused append cannot serve the "
                             "step: append with kv_append, then call paged_attention without k_new")
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            _lib.require_gpu_tensor(name, t)
            if t.dtype != pool.dtype or t.shape[0] != B:
                raise ValueError(f"{name} must be [B, kv_heads, head_dim] in the pool dtype")
        ks = _rows_view("k_new", k_new, hkv, d)
        vs = _rows_view("v_new", v_new, hkv, d)
        ksp, vsp = k_new.data_ptr(), v_new.data_ptr()
    dev = decode_device(q.device)
    need = decode_workspace_bytes(meta, num_heads, hkv, d)
    bufs = workspace if workspace is not None else decode_buffers(q.device, need, meta.decode_units)
    if bufs.pieces.numel() < need or bufs.units < meta.decode_units:
        raise ValueError("decode buffers too small for the step")
    st = _lib.lib().tb_paged_decode(
        q.data_ptr(), qs, pool.data_ptr(), nb, out.data_ptr(), os_, B, meta.decode_plan.data_ptr(),
        meta.decode_workgroups, meta.decode_waves, meta.decode_stride, num_heads, hkv, d, bs, float(scale),
        _lib.DTYPE_CODE[q.dtype], ksp, ks, vsp, vs, bufs.pieces.data_ptr(), bufs.pieces.numel(), meta.decode_pieces,
        bufs.arrivals.data_ptr(), bufs.units, dev.violations.data_ptr(),
        None if rope is None else rope.cos.data_ptr(), None if rope is None else rope.sin.data_ptr(),
        0 if rope is None else rope.max_position, _lib.stream_handle(q.device))
    _lib.check(st, "tb_paged_decode")
    return out


def paged_attention(q: torch.Tensor, pool: torch.Tensor, meta: StepMetadata, *, num_heads: int,
                    scale: float | None = None, out: torch.Tensor | None = None,
                    k_new: torch.Tensor | None = None, v_new: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None, rope: Rope | None = None,
                    noalloc: bool = False) -> torch.Tensor:
    """K2: paged attention of every query row of the step (reference model.py:130-147).

    q: [T, num_heads, head_dim]; returns out [T, num_heads * head_dim] in q's dtype
    (rows outside every sequence slice are left untouched). With k_new/v_new
    ([T, kv_heads, head_dim]) the kernel also appends each decode row's new
    K/V (fused append); this requires a decode-only step. With ``rope`` q (and
    k_new) hold the projections before rotation: each row is rotated at its
    position row_ctx - 1 inside the kernels (model.py:72-80,125 folded in).
    With ``noalloc`` the call allocates nothing on the device: ``out`` must be
    given and the split-row partials go to the library's static per-GPU scratch
    (tb_paged_attention_noalloc; calls that overlap in time on one GPU race).
    """
    if meta.decode_plan is not None and not noalloc and q.dtype in (torch.float16, torch.bfloat16):
        return paged_decode(q, pool, meta, num_heads=num_heads, scale=scale, out=out, k_new=k_new, v_new=v_new,
                            rope=rope)
    if meta.parts is not None and not noalloc:
        # a split mixed step (attach_split_parts): each sub-step on its own rows; with
        # k_new / v_new each side appends its own rows (K rotated first with ``rope``)
        _lib.require_gpu_tensor("q", q)
        d = pool.shape[-1]
        if q.shape[0] != meta.num_tokens:
            raise ValueError(f"q has {q.shape[0]} rows, metadata describes {meta.num_tokens}")
        if out is None:
            out = torch.empty(q.shape[0], num_heads * d, device=q.device, dtype=q.dtype)
        elif out.shape[0] != q.shape[0]:
            raise ValueError("out must match q's row count")
        fused = k_new is not None or v_new is not None
        if fused and (k_new is None or v_new is None or k_new.shape[0] != q.shape[0] or v_new.shape[0] != q.shape[0]):
            raise ValueError("k_new and v_new go together, one row per row of q")
        if fused:
            # a slot written by rows of both parts: each part's own slot mapping cannot
            # see it, the whole step's can (the superseded writer holds -1)
            sm = meta.slot_mapping_np
            if sm.size and np.any((sm < 0) & (meta.row_ctx_np > 0)):
                raise ValueError("two rows of the step write one pool slot; the fused append cannot serve "
                                 "the step: append with kv_append, then call paged_attention without k_new")
        for r0, r1, m in meta.parts:
            paged_attention(q[r0:r1], pool, m, num_heads=num_heads, scale=scale, out=out[r0:r1], rope=rope,
                            k_new=k_new[r0:r1] if fused else None, v_new=v_new[r0:r1] if fused else None)
        return out
    nb, hkv, bs, d = _check_pool(pool)
    _lib.require_gpu_tensor("q", q)
    if q.dtype != pool.dtype:
        raise TypeError(f"q dtype {q.dtype} != pool dtype {pool.dtype}")
    if num_heads % hkv:
        raise ValueError(f"num_heads {num_heads} is not a multiple of kv heads {hkv}")
    if meta.block_size != bs:
        raise ValueError(f"metadata block_size {meta.block_size} != pool block_size {bs}")
    qs = _rows_view("q", q, num_heads, d)
    T = q.shape[0]
    if T != meta.num_tokens:
        raise ValueError(f"q has {T} rows, metadata describes {meta.num_tokens}")
    if out is None:
        if noalloc:
            raise ValueError("noalloc: pass the output buffer (out=...)")
        out = torch.empty(T, num_heads * d, device=q.device, dtype=q.dtype)
    else:
        _lib.require_gpu_tensor("out", out)
        if out.dtype != q.dtype or out.shape[0] != T:
            raise ValueError("out must match q's dtype and row count")
    os_ = _rows_view("out", out, num_heads, d)
    if meta.work is None:
        raise ValueError("metadata has not been uploaded (call meta.to(device))")
    if meta.num_prefill_tiles and q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("prefill tiles need fp16/bf16; build fp32 metadata with tile_prefill=False")
    if meta.rows_per_item > rows_per_item(q.dtype, num_heads, hkv):
        raise ValueError(f"metadata groups {meta.rows_per_item} rows per item; this geometry allows "
                         f"{rows_per_item(q.dtype, num_heads, hkv)}")
    if scale is None:
        scale = 1.0 / math.sqrt(d)   # scaled_dot_product_attention's default (model.py:140,146)
    if rope is not None:
        rope.check(d, q.device)
    ksp = vsp = None
    ks = vs = 0
    prefill_fused = False
    if k_new is not None or v_new is not None:
        if k_new is None or v_new is None:
            raise ValueError("k_new and v_new go together")
        if meta.num_prefill_work and not meta.num_work_items and not meta.num_prefill_tiles:
            # whole prefill sequences only: tb_paged_prefill reads their new rows from
            # k_new / v_new (K rotated in the kernel with ``rope``) and stores them
            prefill_fused = True
        elif not meta.decode_only or meta.num_prefill_tiles or meta.num_prefill_work:
            raise ValueError("fused append needs a decode-only step (one query row per sequence) or a step of "
                             "whole prefills only")
        sm = meta.slot_mapping_np
        if sm.size and np.any((sm < 0) & (meta.row_ctx_np > 0)):
            # a superseded writer of a shared slot: the kernel would store and read each
            # row's own K/V where the reference's last writer wins (kv_cache.py:33-38)
            raise ValueError("two decode rows write one pool slot; the fused append cannot serve the "
                             "step: append with kv_append, then call paged_attention without k_new")
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            _lib.require_gpu_tensor(name, t)
            if t.dtype != pool.dtype or t.shape[0] != T:
                raise ValueError(f"{name} must be [T, kv_heads, head_dim] in the pool dtype")
        ks = _rows_view("k_new", k_new, hkv, d)
        vs = _rows_view("v_new", v_new, hkv, d)
        ksp, vsp = k_new.data_ptr(), v_new.data_ptr()
    head = (q.data_ptr(), qs, pool.data_ptr(), nb, out.data_ptr(), os_,
            meta.block_tables.data_ptr(), meta.max_blocks_per_seq,
            meta.work.data_ptr(), meta.num_work_items,
            meta.prefill_tiles.data_ptr(), meta.num_prefill_tiles,
            meta.row_part_off.data_ptr(), T,
            meta.split_rows.data_ptr(), meta.num_split_rows,
            max(meta.max_parts_per_row, 1), meta.partition_tokens, meta.total_partitions,
            num_heads, hkv, d, bs, float(scale), _lib.DTYPE_CODE[q.dtype],
            *((None, 0, None, 0) if prefill_fused else (ksp, ks, vsp, vs)))
    tail = (_ptr(meta.device_counts),
            None if rope is None else rope.cos.data_ptr(), None if rope is None else rope.sin.data_ptr(),
            0 if rope is None else rope.max_position, _lib.stream_handle(q.device))
    if meta.num_prefill_work:   # whole prefill sequences first (their K/V are appended already)
        if meta.prefill_work is None:
            raise ValueError("metadata has not been uploaded (call meta.to(device))")
        _lib.check(_lib.lib().tb_paged_prefill(
            q.data_ptr(), qs, pool.data_ptr(), nb, out.data_ptr(), os_, meta.block_tables.data_ptr(),
            meta.max_blocks_per_seq, meta.prefill_work.data_ptr(), meta.num_prefill_work, meta.prefill_max_tiles,
            num_heads, hkv, d, bs, float(scale), _lib.DTYPE_CODE[q.dtype],
            *((ksp, ks, vsp, vs) if prefill_fused else (None, 0, None, 0)), *tail[1:]), "tb_paged_prefill")
    if noalloc:
        if workspace is not None:
            raise ValueError("noalloc takes no workspace")
        _lib.check(_lib.lib().tb_paged_attention_noalloc(*head, *tail), "tb_paged_attention_noalloc")
        return out
    if workspace is None:
        workspace = workspace_for(meta, num_heads, d, q.device)
    ws = workspace
    ws_bytes = 0 if ws is None else ws.numel() * ws.element_size()
    if meta.slot_map is not None:   # split rows merged inside the launch (attach_xcd_slot_map)
        dev = decode_device(q.device)
        bufs = decode_buffers(q.device, 0, T * hkv)
        _lib.check(_lib.lib().tb_paged_attention_merged(
            q.data_ptr(), qs, pool.data_ptr(), nb, out.data_ptr(), os_,
            meta.block_tables.data_ptr(), meta.max_blocks_per_seq, meta.work.data_ptr(), meta.num_work_items,
            meta.row_part_off.data_ptr(), T, max(meta.max_parts_per_row, 1), meta.partition_tokens,
            meta.total_partitions, num_heads, hkv, d, bs, float(scale), _lib.DTYPE_CODE[q.dtype], ksp, ks, vsp, vs,
            _ptr(ws), ws_bytes, meta.slot_map.data_ptr(), int(meta.slot_map.numel()), bufs.arrivals.data_ptr(),
            bufs.units, dev.violations.data_ptr(), *tail[1:]), "tb_paged_attention_merged")
        return out
    _lib.check(_lib.lib().tb_paged_attention(*head, _ptr(ws), ws_bytes, *tail), "tb_paged_attention")
    return out


def _block_ids(name: str, ids, num_blocks: int, device) -> torch.Tensor:
    arr = np.asarray(ids.cpu() if isinstance(ids, torch.Tensor) else ids, dtype=np.int64).reshape(-1)
    if arr.size and (arr.min() < 0 or arr.max() >= num_blocks):
        raise IndexError(f"{name} holds a block id outside [0, {num_blocks})")
    return torch.from_numpy(arr.astype(np.int32)).to(device)


class BlockCopyPlan:
    """A validated copy round over a fixed set of layer pools: ids and pool pointers
    live on the device, so ``launch`` makes no host round trip and can be
    captured in a HIP graph (the pools must stay allocated while it is in use)."""

    def __init__(self, pools: list[torch.Tensor], src, dst):
        if not pools:
            raise ValueError("no layer pools")
        nb = pools[0].shape[0]
        for p in pools:
            _check_pool(p)
            if p.shape != pools[0].shape or p.dtype != pools[0].dtype or p.device != pools[0].device:
                raise ValueError("all layer pools must share shape, dtype and device")
        s_np = np.asarray(src.cpu() if isinstance(src, torch.Tensor) else src, dtype=np.int64).reshape(-1)
        d_np = np.asarray(dst.cpu() if isinstance(dst, torch.Tensor) else dst, dtype=np.int64).reshape(-1)
        if s_np.size != d_np.size:
            raise ValueError("src and dst differ in length")
        if d_np.size != np.unique(d_np).size:
            raise ValueError("dst block ids must be distinct")
        if np.intersect1d(s_np, d_np).size:
            raise ValueError("a dst block is also a src block; split the copy into rounds")
        self.device = pools[0].device
        self.num_blocks = nb
        self.num_layers = len(pools)
        self.num_pairs = int(s_np.size)
        self.block_bytes = pools[0][0].numel() * pools[0].element_size()
        self.src = _block_ids("src", s_np, nb, self.device)
        self.dst = _block_ids("dst", d_np, nb, self.device)
        self.ptrs = torch.tensor([p.data_ptr() for p in pools], dtype=torch.int64).to(self.device)

    def launch(self) -> None:
        st = _lib.lib().tb_block_copy(self.ptrs.data_ptr(), self.num_layers, self.num_blocks, self.src.data_ptr(),
                                      self.dst.data_ptr(), self.num_pairs, self.block_bytes,
                                      _lib.stream_handle(self.device))
        _lib.check(st, "tb_block_copy")


def block_copy(pools: list[torch.Tensor], src, dst) -> None:
    """K3: pool_l[dst[i]] <- pool_l[src[i]] for every layer pool l, one launch."""
    if not pools:
        return
    BlockCopyPlan(pools, src, dst).launch()


def block_gather(pool: torch.Tensor, blocks, staging: torch.Tensor) -> None:
    """staging[i] <- pool[blocks[i]] (swap out); staging: [n, *pool.shape[1:]] device or pinned host."""
    nb, _, _, _ = _check_pool(pool)
    b_t = _block_ids("blocks", blocks, nb, pool.device)
    n = b_t.numel()
    if staging.dtype != pool.dtype or staging.numel() < n * pool[0].numel() or not staging.is_contiguous():
        raise ValueError("staging must be a contiguous buffer of n blocks in the pool dtype")
    st = _lib.lib().tb_block_gather(pool.data_ptr(), nb, b_t.data_ptr(), n, staging.data_ptr(),
                                    pool[0].numel() * pool.element_size(), _lib.stream_handle(pool.device))
    _lib.check(st, "tb_block_gather")


def block_scatter(staging: torch.Tensor, pool: torch.Tensor, blocks) -> None:
    """pool[blocks[i]] <- staging[i] (swap in)."""
    nb, _, _, _ = _check_pool(pool)
    b_t = _block_ids("blocks", blocks, nb, pool.device)
    n = b_t.numel()
    if staging.dtype != pool.dtype or staging.numel() < n * pool[0].numel() or not staging.is_contiguous():
        raise ValueError("staging must be a contiguous buffer of n blocks in the pool dtype")
    if b_t.numel() != torch.unique(b_t).numel():
        raise ValueError("blocks must be distinct")
    st = _lib.lib().tb_block_scatter(staging.data_ptr(), pool.data_ptr(), nb, b_t.data_ptr(), n,
                                     pool[0].numel() * pool.element_size(), _lib.stream_handle(pool.device))
    _lib.check(st, "tb_block_scatter")
