// Skinny linear layer for decode-sized batches (the engine's projections,
// reference src/tinybatch/model.py:121-124,149-154: F.linear with weights
// [N][K], K contiguous):
//   Y[M][N] = X[M][K] . W[N][K]^T (+ bias[N]),   M <= 64.
// At decode batch sizes the weight is the whole cost (N*K*2 bytes read once,
// X and Y are a few KB), so the kernel is a weight stream: every workgroup owns
// 16 output columns and splits K over its four waves; a wave issues the loads
// of its whole K range (up to KB 32-wide k-slices per pass) before its MFMAs.
//   v_mfma_f32_16x16x32_{f16,bf16}: A = X rows (m-tile of 16), B = W rows read
//   straight from HBM (lane l: W[n0 + l%16][k + 8(l/16) .. +8], 16 bytes),
//   C/D lane l: Y[m0 + 4(l/16) + j][n0 + l%16].
// The four waves' partial sums meet in LDS; the output is rounded once to the
// element type (after the bias add, as F.linear's single GEMM does).
#include "tb_common.h"

namespace tb {

typedef _Float16 lin_half8 __attribute__((ext_vector_type(8)));
typedef __bf16 lin_bf168 __attribute__((ext_vector_type(8)));

template <typename Tag>
struct lin_math;
template <>
struct lin_math<f16_t> {
  typedef _Float16 scalar_t;
  static __device__ __forceinline__ float4_t mfma(const vec16& a, const vec16& b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(lin_half8, a), __builtin_bit_cast(lin_half8, b),
                                                  c, 0, 0, 0);
  }
};
template <>
struct lin_math<bf16_t> {
  typedef __bf16 scalar_t;
  static __device__ __forceinline__ float4_t mfma(const vec16& a, const vec16& b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(lin_bf168, a), __builtin_bit_cast(lin_bf168, b),
                                                   c, 0, 0, 0);
  }
};

constexpr int LIN_WAVES = 4;
constexpr int LIN_KB = 8;   // k-slices of 32 loaded per pass

template <typename Tag, int MT>
__global__ __launch_bounds__(64 * LIN_WAVES) void linear_kernel(const char* __restrict__ x, int64_t x_row_bytes,
                                                                const char* __restrict__ w, const char* __restrict__ bias,
                                                                char* __restrict__ y, int64_t y_row_bytes, int M, int K) {
  using L = lin_math<Tag>;
  typedef typename L::scalar_t T;
  __shared__ float red[LIN_WAVES][MT][64][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int slices = K / 32;
  const int per_wave = (slices + LIN_WAVES - 1) / LIN_WAVES;
  const int s_begin = wave * per_wave;
  const int s_end = min(slices, s_begin + per_wave);

  const char* wrow = w + (int64_t)(n0 + lc) * K * 2 + 16 * lg;   // B operand: this lane's W row, 8 k per slice
  const char* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = x + (int64_t)min(16 * mt + lc, M - 1) * x_row_bytes + 16 * lg;

  float4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = s_begin; s0 < s_end; s0 += LIN_KB) {
    vec16 wb[LIN_KB], xb[MT][LIN_KB];
#pragma unroll
    for (int i = 0; i < LIN_KB; ++i) {
      const int s = min(s0 + i, s_end - 1);          // past the range: a repeat that is not used
      wb[i] = ld16_stream(wrow + (int64_t)s * 64);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xb[mt][i] = ld16(xrow[mt] + (int64_t)s * 64);
    }
#pragma unroll
    for (int i = 0; i < LIN_KB; ++i) {
      if (s0 + i < s_end) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = L::mfma(xb[mt][i], wb[i], acc[mt]);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][mt][lane][j] = acc[mt][j];
  __syncthreads();
  // thread t: output element (row m, column n0 + c) for t = m * 16 + c
  for (int t = threadIdx.x; t < MT * 256; t += 64 * LIN_WAVES) {
    const int m = t >> 4, c = t & 15;
    if (m >= M) continue;
    const int mt = m >> 4, r = m & 15;
    const int l = 16 * (r >> 2) + c, j = r & 3;          // the D lane and element holding (r, c)
    float v = 0.f;
#pragma unroll
    for (int wv = 0; wv < LIN_WAVES; ++wv) v += red[wv][mt][l][j];
    if (bias) v += (float)reinterpret_cast<const T*>(bias)[n0 + c];
    reinterpret_cast<T*>(y + (int64_t)m * y_row_bytes)[n0 + c] = (T)v;
  }
}

template <typename Tag>
static void launch_linear(const void* x, int64_t xrb, const void* w, const void* bias, void* y, int64_t yrb, int M,
                          int N, int K, hipStream_t stream) {
  const dim3 grid(N / 16), block(64 * LIN_WAVES);
  const char *xc = (const char*)x, *wc = (const char*)w, *bc = (const char*)bias;
  char* yc = (char*)y;
  switch ((M + 15) / 16) {
    case 1: hipLaunchKernelGGL((linear_kernel<Tag, 1>), grid, block, 0, stream, xc, xrb, wc, bc, yc, yrb, M, K); break;
    case 2: hipLaunchKernelGGL((linear_kernel<Tag, 2>), grid, block, 0, stream, xc, xrb, wc, bc, yc, yrb, M, K); break;
    case 3: hipLaunchKernelGGL((linear_kernel<Tag, 3>), grid, block, 0, stream, xc, xrb, wc, bc, yc, yrb, M, K); break;
    default: hipLaunchKernelGGL((linear_kernel<Tag, 4>), grid, block, 0, stream, xc, xrb, wc, bc, yc, yrb, M, K); break;
  }
}

}  // namespace tb

extern "C" int32_t tb_linear(const void* x, int64_t x_row_stride, const void* w, const void* bias, void* y,
                             int64_t y_row_stride, int32_t rows, int32_t out_features, int32_t in_features,
                             int32_t dtype, hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(rows >= 0 && out_features > 0 && in_features > 0);
  if (dtype != TB_DTYPE_F16 && dtype != TB_DTYPE_BF16) return TB_ERR_UNSUPPORTED;
  if (rows > 64 || out_features % 16 != 0 || in_features % 32 != 0) return TB_ERR_UNSUPPORTED;
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(x && w && y);
  TB_CHECK_ARG(x_row_stride >= in_features && y_row_stride >= out_features);
  TB_CHECK_ARG((((uintptr_t)x | (uintptr_t)w) & 15u) == 0 && (x_row_stride * 2) % 16 == 0);
  if (dtype == TB_DTYPE_F16)
    launch_linear<f16_t>(x, x_row_stride * 2, w, bias, y, y_row_stride * 2, rows, out_features, in_features, stream);
  else
    launch_linear<bf16_t>(x, x_row_stride * 2, w, bias, y, y_row_stride * 2, rows, out_features, in_features, stream);
  TB_RETURN_LAUNCH_STATUS();
}
