// Model-side fused elementwise kernels of the engine's Qwen2 layer.
//
// The reference's layer (src/tinybatch/model.py:115-154) runs RMSNorm, RoPE and
// SwiGLU as chains of PyTorch elementwise ops (8, ~20 and 2 launches per
// layer); in a decode step of a few dozen tokens each launch costs more than
// its arithmetic. One launch each here, with the reference's fp32 arithmetic:
//   tb_rms_norm  : [h = x + residual;] out = (h * rsqrt(mean(h^2) + eps)) * w  (model.py:65-69,149)
//   tb_rope_qk   : rotate-half RoPE of q and k, straight from the qkv GEMM rows  (model.py:72-80,125)
//   tb_silu_mul  : silu(gate) * up of the gate/up GEMM rows                       (model.py:151-154)
//   tb_rms_norm_partials : tb_rms_norm whose x is the sum of split-K partials of
//                  the projection before it (o_proj, down_proj: model.py:149,154)
// Rounding follows the PyTorch ops they replace: the residual sum and silu(g)
// are rounded to the element type before their next use. The norm's two
// products are single v_mul_f32s (mul_rn): left to the compiler, the second
// one and the rounding to fp16 fused into one mixed-precision FMA in some of
// the norm kernels and not in others (one rounding instead of two, a 1-ulp
// difference in rare elements).
#include "tb_common.h"

namespace tb {

template <typename T>
__device__ __forceinline__ float to_f(T x) { return (float)x; }
template <typename T>
__device__ __forceinline__ T from_f(float x) { return (T)x; }

// ---- RMSNorm (+ residual add) ------------------------------------------------
// One workgroup of 256 threads per row; thread t owns elements t, t + 256, ...
// (dim <= 256 * 16). The row sum of squares is reduced in fp32.
constexpr int NORM_THREADS = 256;
constexpr int NORM_MAX_PER_THREAD = 16;

template <typename T>
__global__ __launch_bounds__(NORM_THREADS) void rms_norm_kernel(const T* x, int64_t xs, T* res, int64_t rs,
                                                               const T* w, T* out, int64_t os, int dim,
                                                               float eps) {
  __shared__ float part[NORM_THREADS / 64];
  const int row = blockIdx.x;
  const T* xr = x + row * xs;
  T* rr = res ? res + row * rs : nullptr;
  float h[NORM_MAX_PER_THREAD];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < NORM_MAX_PER_THREAD; ++k) {
    const int i = threadIdx.x + k * NORM_THREADS;
    h[k] = 0.f;
    if (i < dim) {
      float v = to_f(xr[i]);
      if (rr) {
        const T sum = from_f<T>(v + to_f(rr[i]));   // h = h + delta, rounded like the tensor add
        rr[i] = sum;
        v = to_f(sum);
      }
      h[k] = v;
      ss += v * v;
    }
  }
  ss += __shfl_xor(ss, 1);
  ss += __shfl_xor(ss, 2);
  ss += __shfl_xor(ss, 4);
  ss += __shfl_xor(ss, 8);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < NORM_THREADS / 64; ++k) tot += part[k];
  const float inv = rsqrtf(__fdiv_rn(tot, (float)dim) + eps);   // the mean correctly rounded (every norm kernel alike)
  T* orow = out + row * os;
#pragma unroll
  for (int k = 0; k < NORM_MAX_PER_THREAD; ++k) {
    const int i = threadIdx.x + k * NORM_THREADS;
    if (i < dim) orow[i] = from_f<T>(mul_rn(mul_rn(h[k], inv), to_f(w[i])));
  }
}

// ---- RMSNorm of split-K partial sums (+ residual add) ---------------------------
// x = T(sum over s of partials[s][row]) is the projection output (the split-K
// pieces of tb_linear_partials, added in split order and rounded once, like
// F.linear's output); then the residual add and RMSNorm of rms_norm_kernel.
// One wave (one workgroup) per row, so that the row's partials (S x dim x 4
// bytes, 28 KB for 8 pieces of 896) stream through a CU of their own: four
// rows per workgroup measured 3.7 us a launch for 8 pieces of 32 rows, one
// row 3.0 us.
// Lane owns the 8-element chunks lane, lane + 64, ... (CH of them), every
// load issued before any use.
template <typename T, int S, int CH>
__global__ __launch_bounds__(64) void rms_norm_partials_kernel(const float* __restrict__ part, int rows, int dim,
                                                                T* res, int64_t rs, const T* __restrict__ w,
                                                                T* out, int64_t os, float eps) {
  const int row = blockIdx.x, lane = threadIdx.x;
  struct x8 {
    T v[8];
  };
  const int chunks = dim >> 3;
  const int64_t plane = (int64_t)rows * dim;
  float4_t p[CH][S][2];
  vec16 rv[CH], wv[CH];
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const int c = min(lane + 64 * i, chunks - 1);       // lanes past the row repeat its last chunk, unused
    const float* src = part + (int64_t)row * dim + 8 * c;
#pragma unroll
    for (int s = 0; s < S; ++s) {
      p[i][s][0] = *reinterpret_cast<const float4_t*>(src + s * plane);
      p[i][s][1] = *reinterpret_cast<const float4_t*>(src + s * plane + 4);
    }
    if (res) rv[i] = ld16(res + row * rs + 8 * c);
    wv[i] = ld16(w + 8 * c);
  }
  float h[CH][8];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    const bool mine = lane + 64 * i < chunks;
    const x8 r = __builtin_bit_cast(x8, rv[i]);
    x8 sum;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float acc = p[i][0][e >> 2][e & 3];
#pragma unroll
      for (int s = 1; s < S; ++s) acc += p[i][s][e >> 2][e & 3];
      float v = to_f(from_f<T>(acc));                  // the projection's output rounding
      if (res) {
        sum.v[e] = from_f<T>(v + to_f(r.v[e]));        // h = h + delta, rounded like the tensor add
        v = to_f(sum.v[e]);
      }
      h[i][e] = v;
      if (mine) ss += v * v;
    }
    if (res && mine) st16(res + row * rs + 8 * (lane + 64 * i), __builtin_bit_cast(vec16, sum));
  }
  ss += __shfl_xor(ss, 1);
  ss += __shfl_xor(ss, 2);
  ss += __shfl_xor(ss, 4);
  ss += __shfl_xor(ss, 8);
  ss += __shfl_xor(ss, 16);
  ss += __shfl_xor(ss, 32);
  const float inv = rsqrtf(__fdiv_rn(ss, (float)dim) + eps);    // the mean correctly rounded (every norm kernel alike)
#pragma unroll
  for (int i = 0; i < CH; ++i) {
    if (lane + 64 * i >= chunks) continue;
    const x8 wt = __builtin_bit_cast(x8, wv[i]);
    x8 o;
#pragma unroll
    for (int e = 0; e < 8; ++e) o.v[e] = from_f<T>(mul_rn(mul_rn(h[i][e], inv), to_f(wt.v[e])));
    st16(out + row * os + 8 * (lane + 64 * i), __builtin_bit_cast(vec16, o));
  }
}

template <typename T, int S>
static void launch_norm_partials_ch(int ch, dim3 grid, const float* part, int rows, int dim, T* res, int64_t rs,
                                    const T* w, T* out, int64_t os, float eps, hipStream_t stream) {
  switch (ch) {
    case 1: hipLaunchKernelGGL((rms_norm_partials_kernel<T, S, 1>), grid, dim3(64), 0, stream, part, rows, dim, res, rs, w, out, os, eps); break;
    case 2: hipLaunchKernelGGL((rms_norm_partials_kernel<T, S, 2>), grid, dim3(64), 0, stream, part, rows, dim, res, rs, w, out, os, eps); break;
    case 4: hipLaunchKernelGGL((rms_norm_partials_kernel<T, S, 4>), grid, dim3(64), 0, stream, part, rows, dim, res, rs, w, out, os, eps); break;
    default: hipLaunchKernelGGL((rms_norm_partials_kernel<T, S, 8>), grid, dim3(64), 0, stream, part, rows, dim, res, rs, w, out, os, eps); break;
  }
}

template <typename T>
static void launch_norm_partials(int splits, int ch, const float* part, int rows, int dim, T* res, int64_t rs,
                                 const T* w, T* out, int64_t os, float eps, hipStream_t stream) {
  const dim3 grid(rows);
  switch (splits) {
    case 1: launch_norm_partials_ch<T, 1>(ch, grid, part, rows, dim, res, rs, w, out, os, eps, stream); break;
    case 2: launch_norm_partials_ch<T, 2>(ch, grid, part, rows, dim, res, rs, w, out, os, eps, stream); break;
    case 4: launch_norm_partials_ch<T, 4>(ch, grid, part, rows, dim, res, rs, w, out, os, eps, stream); break;
    default: launch_norm_partials_ch<T, 8>(ch, grid, part, rows, dim, res, rs, w, out, os, eps, stream); break;
  }
}

// ---- RoPE of q and k ------------------------------------------------------------
// Thread per (row, head, i < D/2): x1 = x[i], x2 = x[i + D/2];
// out = (x1 c - x2 s, x2 c + x1 s) with c, s the fp32 tables at the row's
// position (each product rounded on its own, as the separate tensor ops do).
template <typename T>
__global__ __launch_bounds__(256) void rope_qk_kernel(const T* qkv, int64_t row_stride, const int64_t* positions,
                                                      const float* cos_t, const float* sin_t, int max_position,
                                                      T* q_out, T* k_out, int rows, int hq, int hkv, int d) {
  const int half = d >> 1;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = (int64_t)(hq + hkv) * half;
  if (idx >= (int64_t)rows * per_row) return;
  const int row = (int)(idx / per_row);
  const int rem = (int)(idx - (int64_t)row * per_row);
  const int head = rem / half, i = rem - head * half;
  int64_t p = positions[row];
  p = p < 0 ? 0 : (p >= max_position ? max_position - 1 : p);   // the host validates positions
  const float c = cos_t[p * half + i], s = sin_t[p * half + i];
  const T* src = qkv + row * row_stride + (int64_t)head * d;     // q heads, then k heads
  const float x1 = to_f(src[i]), x2 = to_f(src[i + half]);
  const float o1 = mul_rn(x1, c) - mul_rn(x2, s);   // each product rounded on its own
  const float o2 = mul_rn(x2, c) + mul_rn(x1, s);
  T* dst = head < hq ? q_out + ((int64_t)row * hq + head) * d : k_out + ((int64_t)row * hkv + head - hq) * d;
  dst[i] = from_f<T>(o1);
  dst[i + half] = from_f<T>(o2);
}

// ---- SwiGLU gate ------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(const T* gu, int64_t row_stride, T* out, int64_t os,
                                                       int rows, int d_ff) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)rows * d_ff) return;
  const int row = (int)(idx / d_ff), i = (int)(idx - (int64_t)row * d_ff);
  const float g = to_f(gu[row * row_stride + i]);
  const T act = from_f<T>(g / (1.f + expf(-g)));                 // F.silu, rounded to the element type
  out[row * os + i] = from_f<T>(to_f(act) * to_f(gu[row * row_stride + d_ff + i]));
}

}  // namespace tb

extern "C" int32_t tb_rms_norm(const void* x, int64_t x_row_stride, void* residual, int64_t residual_row_stride,
                               const void* weight, void* out, int64_t out_row_stride, int32_t rows, int32_t dim,
                               float eps, int32_t dtype, hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(rows >= 0 && dim > 0 && dim <= NORM_THREADS * NORM_MAX_PER_THREAD);
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(x && weight && out);
  TB_CHECK_ARG(x_row_stride >= dim && out_row_stride >= dim && (!residual || residual_row_stride >= dim));
  const dim3 grid(rows), block(NORM_THREADS);
  switch (dtype) {
    case TB_DTYPE_F32:
      hipLaunchKernelGGL(rms_norm_kernel<float>, grid, block, 0, stream, (const float*)x, x_row_stride,
                         (float*)residual, residual_row_stride, (const float*)weight, (float*)out, out_row_stride,
                         dim, eps);
      break;
    case TB_DTYPE_F16:
      hipLaunchKernelGGL(rms_norm_kernel<_Float16>, grid, block, 0, stream, (const _Float16*)x, x_row_stride,
                         (_Float16*)residual, residual_row_stride, (const _Float16*)weight, (_Float16*)out,
                         out_row_stride, dim, eps);
      break;
    case TB_DTYPE_BF16:
      hipLaunchKernelGGL(rms_norm_kernel<__bf16>, grid, block, 0, stream, (const __bf16*)x, x_row_stride,
                         (__bf16*)residual, residual_row_stride, (const __bf16*)weight, (__bf16*)out,
                         out_row_stride, dim, eps);
      break;
    default: return TB_ERR_INVALID_ARG;
  }
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_rope_qk(const void* qkv, int64_t row_stride, const int64_t* positions, const float* cos_table,
                              const float* sin_table, int32_t max_position, void* q_out, void* k_out, int32_t rows,
                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                              hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(rows >= 0 && num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && head_dim % 2 == 0);
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(qkv && positions && cos_table && sin_table && q_out && k_out && max_position > 0);
  TB_CHECK_ARG(row_stride >= (int64_t)(num_heads + num_kv_heads) * head_dim);
  const int64_t n = (int64_t)rows * (num_heads + num_kv_heads) * (head_dim / 2);
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  switch (dtype) {
    case TB_DTYPE_F32:
      hipLaunchKernelGGL(rope_qk_kernel<float>, grid, block, 0, stream, (const float*)qkv, row_stride, positions,
                         cos_table, sin_table, max_position, (float*)q_out, (float*)k_out, rows, num_heads,
                         num_kv_heads, head_dim);
      break;
    case TB_DTYPE_F16:
      hipLaunchKernelGGL(rope_qk_kernel<_Float16>, grid, block, 0, stream, (const _Float16*)qkv, row_stride,
                         positions, cos_table, sin_table, max_position, (_Float16*)q_out, (_Float16*)k_out, rows,
                         num_heads, num_kv_heads, head_dim);
      break;
    case TB_DTYPE_BF16:
      hipLaunchKernelGGL(rope_qk_kernel<__bf16>, grid, block, 0, stream, (const __bf16*)qkv, row_stride, positions,
                         cos_table, sin_table, max_position, (__bf16*)q_out, (__bf16*)k_out, rows, num_heads,
                         num_kv_heads, head_dim);
      break;
    default: return TB_ERR_INVALID_ARG;
  }
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_silu_mul(const void* gate_up, int64_t row_stride, void* out, int64_t out_row_stride,
                               int32_t rows, int32_t d_ff, int32_t dtype, hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(rows >= 0 && d_ff > 0);
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(gate_up && out && row_stride >= 2 * (int64_t)d_ff && out_row_stride >= d_ff);
  const int64_t n = (int64_t)rows * d_ff;
  const dim3 grid((unsigned)((n + 255) / 256)), block(256);
  switch (dtype) {
    case TB_DTYPE_F32:
      hipLaunchKernelGGL(silu_mul_kernel<float>, grid, block, 0, stream, (const float*)gate_up, row_stride,
                         (float*)out, out_row_stride, rows, d_ff);
      break;
    case TB_DTYPE_F16:
      hipLaunchKernelGGL(silu_mul_kernel<_Float16>, grid, block, 0, stream, (const _Float16*)gate_up, row_stride,
                         (_Float16*)out, out_row_stride, rows, d_ff);
      break;
    case TB_DTYPE_BF16:
      hipLaunchKernelGGL(silu_mul_kernel<__bf16>, grid, block, 0, stream, (const __bf16*)gate_up, row_stride,
                         (__bf16*)out, out_row_stride, rows, d_ff);
      break;
    default: return TB_ERR_INVALID_ARG;
  }
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_rms_norm_partials(const float* partials, int32_t splits, void* residual,
                                        int64_t residual_row_stride, const void* weight, void* out,
                                        int64_t out_row_stride, int32_t rows, int32_t dim, float eps, int32_t dtype,
                                        hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(rows >= 0 && dim > 0);
  if (dtype != TB_DTYPE_F16 && dtype != TB_DTYPE_BF16) return TB_ERR_UNSUPPORTED;
  if (dim % 8 != 0 || dim > 64 * 8 * 8) return TB_ERR_UNSUPPORTED;
  if (splits != 1 && splits != 2 && splits != 4 && splits != 8) return TB_ERR_UNSUPPORTED;
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(partials && weight && out && out_row_stride >= dim && out_row_stride % 8 == 0);
  TB_CHECK_ARG(!residual || (residual_row_stride >= dim && residual_row_stride % 8 == 0));
  TB_CHECK_ARG((((uintptr_t)partials | (uintptr_t)weight | (uintptr_t)out | (uintptr_t)residual) & 15u) == 0);
  const int chunks = dim / 8;
  const int ch = chunks <= 64 ? 1 : chunks <= 128 ? 2 : chunks <= 256 ? 4 : 8;
  if (dtype == TB_DTYPE_F16)
    launch_norm_partials<_Float16>(splits, ch, partials, rows, dim, (_Float16*)residual, residual_row_stride,
                                   (const _Float16*)weight, (_Float16*)out, out_row_stride, eps, stream);
  else
    launch_norm_partials<__bf16>(splits, ch, partials, rows, dim, (__bf16*)residual, residual_row_stride,
                                 (const __bf16*)weight, (__bf16*)out, out_row_stride, eps, stream);
  TB_RETURN_LAUNCH_STATUS();
}
