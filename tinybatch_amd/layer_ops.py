"""Host wrappers of the fused layer kernels (tb_rms_norm, tb_rope_qk, tb_silu_mul).

They replace the PyTorch op chains of the reference's layer
(src/tinybatch/model.py:65-80,115-154) with one launch each; see
include/tinybatch_amd.h for the exact arithmetic.
"""
from __future__ import annotations

import torch

from . import _lib


def _row_stride(name: str, t: torch.Tensor, width: int) -> int:
    _lib.require_gpu_tensor(name, t)
    if t.dim() != 2 or t.shape[1] < width or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D tensor with contiguous rows of >= {width} elements")
    return t.stride(0) if t.shape[0] > 1 else t.shape[1]


def rms_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, *, residual: torch.Tensor | None = None,
             out: torch.Tensor | None = None) -> torch.Tensor:
    """RMSNorm of x's rows (model.py:65-69). With ``residual``: residual += x
    first (in place) and the sum is normalised (the residual add of model.py:149,154)."""
    rows, dim = x.shape
    xs = _row_stride("x", x, dim)
    if weight.shape != (dim,) or weight.dtype != x.dtype or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [dim] tensor of x's dtype")
    rs = 0
    if residual is not None:
        rs = _row_stride("residual", residual, dim)
        if residual.shape != x.shape or residual.dtype != x.dtype:
            raise ValueError("residual must match x")
    if out is None:
        out = torch.empty(rows, dim, dtype=x.dtype, device=x.device)
    os_ = _row_stride("out", out, dim)
    st = _lib.lib().tb_rms_norm(x.data_ptr(), xs, None if residual is None else residual.data_ptr(), rs,
                                weight.data_ptr(), out.data_ptr(), os_, rows, dim, float(eps),
                                _lib.DTYPE_CODE[x.dtype], _lib.stream_handle(x.device))
    _lib.check(st, "tb_rms_norm")
    return out


def rope_qk(qkv: torch.Tensor, positions: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, num_heads: int,
            num_kv_heads: int, head_dim: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Rotated q [T, Hq, D] and k [T, Hkv, D] from the q|k|v rows of the qkv GEMM (model.py:72-80)."""
    T = qkv.shape[0]
    rs = _row_stride("qkv", qkv, (num_heads + num_kv_heads) * head_dim)
    if positions.dtype != torch.int64 or not positions.is_cuda or positions.numel() != T:
        raise TypeError("positions must be an int64 GPU tensor with one entry per row")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != torch.float32 or not t.is_cuda or not t.is_contiguous() or t.shape[1] != head_dim // 2:
            raise TypeError(f"{name} must be a contiguous fp32 GPU table [max_position, head_dim/2]")
    q = torch.empty(T, num_heads, head_dim, dtype=qkv.dtype, device=qkv.device)
    k = torch.empty(T, num_kv_heads, head_dim, dtype=qkv.dtype, device=qkv.device)
    st = _lib.lib().tb_rope_qk(qkv.data_ptr(), rs, positions.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                               cos.shape[0], q.data_ptr(), k.data_ptr(), T, num_heads, num_kv_heads, head_dim,
                               _lib.DTYPE_CODE[qkv.dtype], _lib.stream_handle(qkv.device))
    _lib.check(st, "tb_rope_qk")
    return q, k


def silu_mul(gate_up: torch.Tensor, d_ff: int) -> torch.Tensor:
    """silu(gate) * up for gate_up rows [gate | up] (model.py:152-154)."""
    T = gate_up.shape[0]
    rs = _row_stride("gate_up", gate_up, 2 * d_ff)
    out = torch.empty(T, d_ff, dtype=gate_up.dtype, device=gate_up.device)
    st = _lib.lib().tb_silu_mul(gate_up.data_ptr(), rs, out.data_ptr(), d_ff, T, d_ff,
                                _lib.DTYPE_CODE[gate_up.dtype], _lib.stream_handle(gate_up.device))
    _lib.check(st, "tb_silu_mul")
    return out


def _linear_operands(x: torch.Tensor, weight: torch.Tensor) -> tuple[int, int, int]:
    if x.dim() != 2 or weight.dim() != 2 or x.shape[1] != weight.shape[1]:
        raise ValueError("x must be [rows, in_features] and weight [out_features, in_features]")
    for name, t in (("x", x), ("weight", weight)):
        _lib.require_gpu_tensor(name, t)
        if t.dtype != x.dtype or t.stride(-1) != 1:
            raise ValueError(f"{name} must share x's dtype and have contiguous rows")
    if not weight.is_contiguous():
        raise ValueError("weight must be contiguous")
    rows, k = x.shape
    return rows, weight.shape[0], x.stride(0) if rows > 1 else k


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None,
           out: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear for decode-sized batches (rows <= 64, fp16/bf16; tb_linear): the
    weight is streamed once, fp32 accumulation, one rounding (model.py:121-154)."""
    rows, n, xs = _linear_operands(x, weight)
    k = x.shape[1]
    if bias is not None and (bias.dtype != x.dtype or bias.shape != (n,) or not bias.is_contiguous()):
        raise ValueError("bias must be a contiguous [out_features] tensor in x's dtype")
    if out is None:
        out = torch.empty(rows, n, device=x.device, dtype=x.dtype)
    st = _lib.lib().tb_linear(x.data_ptr(), xs, weight.data_ptr(),
                              None if bias is None else bias.data_ptr(), out.data_ptr(),
                              out.stride(0) if rows > 1 else n, rows, n, k, _lib.DTYPE_CODE[x.dtype],
                              _lib.stream_handle(x.device))
    _lib.check(st, "tb_linear")
    return out


def linear_partials(x: torch.Tensor, weight: torch.Tensor, splits: int) -> torch.Tensor:
    """Split-K pieces of F.linear(x, weight) (no bias; tb_linear_partials): float32
    [splits, rows, out_features] whose sum over dim 0 is the product, for
    rms_norm_partials to add, round and normalise (model.py:149,154)."""
    rows, n, xs = _linear_operands(x, weight)
    parts = torch.empty(splits, rows, n, device=x.device, dtype=torch.float32)
    st = _lib.lib().tb_linear_partials(x.data_ptr(), xs, weight.data_ptr(), parts.data_ptr(), splits, rows, n,
                                       x.shape[1], _lib.DTYPE_CODE[x.dtype], _lib.stream_handle(x.device))
    _lib.check(st, "tb_linear_partials")
    return parts


def linear_silu_mul(x: torch.Tensor, w_gate_up: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """silu(x W_gate^T) * (x W_up^T) for the merged [2 d_ff, in] gate/up weight
    (model.py:151-154; tb_linear_silu_mul): the bits of linear() then silu_mul()."""
    rows, n, xs = _linear_operands(x, w_gate_up)
    d_ff = n // 2
    if n % 2:
        raise ValueError("w_gate_up must hold gate and up rows (an even row count)")
    if out is None:
        out = torch.empty(rows, d_ff, device=x.device, dtype=x.dtype)
    st = _lib.lib().tb_linear_silu_mul(x.data_ptr(), xs, w_gate_up.data_ptr(), out.data_ptr(),
                                       out.stride(0) if rows > 1 else d_ff, rows, d_ff, x.shape[1],
                                       _lib.DTYPE_CODE[x.dtype], _lib.stream_handle(x.device))
    _lib.check(st, "tb_linear_silu_mul")
    return out


def linear_argmax(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
                  workspace: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight).argmax(-1) (int64 [rows]) without the logits: the LM
    head with greedy sampling fused (tb_linear_argmax; model.py:157-158,
    engine.py:145-151)."""
    rows, n, xs = _linear_operands(x, weight)
    L = _lib.lib()
    need = L.tb_linear_argmax_workspace_bytes(rows, n)
    if workspace is None:
        workspace = torch.empty(max(need, 8), dtype=torch.uint8, device=x.device)
    if workspace.numel() * workspace.element_size() < need or not workspace.is_contiguous():
        raise ValueError(f"workspace must be a contiguous tensor of >= {need} bytes")
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=x.device)
    if out.dtype != torch.int64 or out.shape != (rows,) or not out.is_contiguous():
        raise ValueError("out must be a contiguous int64 [rows] tensor")
    st = L.tb_linear_argmax(x.data_ptr(), xs, weight.data_ptr(), rows, n, x.shape[1], workspace.data_ptr(),
                            workspace.numel() * workspace.element_size(), out.data_ptr(),
                            _lib.DTYPE_CODE[x.dtype], _lib.stream_handle(x.device))
    _lib.check(st, "tb_linear_argmax")
    return out


def rms_norm_partials(partials: torch.Tensor, weight: torch.Tensor, eps: float, *,
                      residual: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """rms_norm() of x = partials.sum(0) rounded to weight's dtype (tb_rms_norm_partials):
    the projection output of linear_partials, then the residual add and RMSNorm."""
    _lib.require_gpu_tensor("partials", partials)
    if partials.dim() != 3 or partials.dtype != torch.float32 or not partials.is_contiguous():
        raise ValueError("partials must be a contiguous float32 [splits, rows, dim] tensor")
    splits, rows, dim = partials.shape
    _lib.require_gpu_tensor("weight", weight)
    if weight.shape != (dim,) or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous [dim] tensor")
    rs = 0
    if residual is not None:
        rs = _row_stride("residual", residual, dim)
        if residual.shape != (rows, dim) or residual.dtype != weight.dtype:
            raise ValueError("residual must be [rows, dim] in weight's dtype")
    if out is None:
        out = torch.empty(rows, dim, dtype=weight.dtype, device=weight.device)
    os_ = _row_stride("out", out, dim)
    st = _lib.lib().tb_rms_norm_partials(partials.data_ptr(), splits,
                                         None if residual is None else residual.data_ptr(), rs,
                                         weight.data_ptr(), out.data_ptr(), os_, rows, dim, float(eps),
                                         _lib.DTYPE_CODE[weight.dtype], _lib.stream_handle(weight.device))
    _lib.check(st, "tb_rms_norm_partials")
    return out
