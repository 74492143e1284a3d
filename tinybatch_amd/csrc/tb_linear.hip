// Skinny linear layers for decode-sized batches (the engine's projections,
// reference src/tinybatch/model.py:121-124,149-154: F.linear with weights
// [N][K], K contiguous):
//   Y[M][N] = X[M][K] . W[N][K]^T (+ bias[N]),   M <= 64.
// At decode batch sizes the weight is the whole cost (N*K*2 bytes read once,
// X and Y are a few KB), so the kernels are weight streams: a workgroup owns
// NT tiles of 16 output columns and one K range, which its waves split; a wave
// issues the loads of its whole K share (up to KB 32-wide k-slices per pass)
// before its MFMAs.
//   v_mfma_f32_16x16x32_{f16,bf16}: A = X rows (m-tile of 16), B = W rows read
//   straight from HBM (lane l: W[n0 + l%16][k + 8(l/16) .. +8], 16 bytes),
//   C/D lane l: Y[m0 + 4(l/16) + j][n0 + l%16].
// One load instruction reads 64 bytes of each of 16 W rows; the other half of
// each 128-byte line is the next k-slice's load. W therefore goes through
// plain loads that keep the line: non-temporal ones measured 5-25% slower
// (the 151936 x 896 LM head at one row: 64.6 vs 50.6 us).
// The waves' partial sums meet in LDS. Three epilogues:
//   round   : Y = T(sum + bias), one rounding as F.linear's single GEMM;
//   partial : fp32 sums of one K range to partials[split][M][N] (the split-K
//             pieces; tb_rms_norm_partials adds them in split order, rounds
//             once and continues with the residual add and RMSNorm);
//   silu    : the workgroup's two tiles are gate columns c and up columns
//             d_ff + c of the merged gate/up weight; Y = silu(T(gate)) * T(up)
//             with the roundings of F.linear followed by tb_silu_mul
//             (model.py:151-154).
// A tile's sum does not depend on the epilogue or on NT: for equal K ranges
// and wave counts the silu epilogue gives the bits of the round epilogue
// followed by tb_silu_mul.
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

constexpr int LIN_KB = 8;   // k-slices of 32 loaded per pass
enum { LIN_ROUND = 0, LIN_PARTIAL = 1, LIN_SILU = 2 };

struct lin_args {
  const char* x;
  int64_t x_row_bytes;
  const char* w;              // [N][K]
  const char* bias;           // [N] or null (round epilogue only)
  void* y;                    // round / silu: [M][y_row_stride] of T; partial: float [splits][M][N]
  int64_t y_row_stride;       // elements
  int M, N, K;                // K range s of gridDim.y: k-slices [s*K/32/splits, (s+1)*K/32/splits)
};

template <typename Tag, int MT, int NT, int WAVES, int MODE>
__global__ __launch_bounds__(64 * WAVES) void linear_kernel(lin_args a) {
  using L = lin_math<Tag>;
  typedef typename L::scalar_t T;
  __shared__ float red[WAVES][MT][NT][64][4];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  // silu: tiles j < NT/2 are gate columns, tile j + NT/2 the up columns d_ff later
  constexpr int OUT_TILES = MODE == LIN_SILU ? NT / 2 : NT;
  static_assert(MODE != LIN_SILU || NT % 2 == 0, "silu pairs gate and up tiles");
  int n0[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
    n0[j] = (j / OUT_TILES) * (a.N >> 1) + (blockIdx.x * OUT_TILES + j % OUT_TILES) * 16;
  const int slices = a.K / 32;
  const int k_begin = (int)blockIdx.y * slices / (int)gridDim.y;
  const int k_end = ((int)blockIdx.y + 1) * slices / (int)gridDim.y;
  const int per_wave = (k_end - k_begin + WAVES - 1) / WAVES;
  const int s_begin = k_begin + wave * per_wave;
  const int s_end = min(k_end, s_begin + per_wave);

  const char* wrow[NT];       // B operand: this lane's W row, 8 k per slice
#pragma unroll
  for (int j = 0; j < NT; ++j) wrow[j] = a.w + (int64_t)(n0[j] + lc) * a.K * 2 + 16 * lg;
  const char* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = a.x + (int64_t)min(16 * mt + lc, a.M - 1) * a.x_row_bytes + 16 * lg;

  float4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mt][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = s_begin; s0 < s_end; s0 += LIN_KB) {
    vec16 wb[NT][LIN_KB], xb[MT][LIN_KB];
#pragma unroll
    for (int i = 0; i < LIN_KB; ++i) {
      const int s = min(s0 + i, s_end - 1);          // past the range: a repeat that is not used
#pragma unroll
      for (int j = 0; j < NT; ++j) wb[j][i] = ld16(wrow[j] + (int64_t)s * 64);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) xb[mt][i] = ld16(xrow[mt] + (int64_t)s * 64);
    }
#pragma unroll
    for (int i = 0; i < LIN_KB; ++i) {
      if (s0 + i < s_end) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < NT; ++j) acc[mt][j] = L::mfma(xb[mt][i], wb[j][i], acc[mt][j]);
      }
    }
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[wave][mt][j][lane][e] = acc[mt][j][e];
  __syncthreads();
  // thread t: output element (row m, tile j, column c)
  for (int t = threadIdx.x; t < MT * 256 * OUT_TILES; t += 64 * WAVES) {
    const int c = t & 15, j = (t >> 4) % OUT_TILES, m = t / (16 * OUT_TILES);
    if (m >= a.M) continue;
    const int mt = m >> 4, r = m & 15;
    const int l = 16 * (r >> 2) + c, e = r & 3;          // the D lane and element holding (r, c)
    float v0 = 0.f, v1 = 0.f;
#pragma unroll
    for (int wv = 0; wv < WAVES; ++wv) v0 += red[wv][mt][j][l][e];
    if constexpr (MODE == LIN_ROUND) {
      if (a.bias) v0 += (float)reinterpret_cast<const T*>(a.bias)[n0[j] + c];
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_row_stride + n0[j] + c] = (T)v0;
    } else if constexpr (MODE == LIN_PARTIAL) {
      reinterpret_cast<float*>(a.y)[((int64_t)blockIdx.y * a.M + m) * a.N + n0[j] + c] = v0;
    } else {
#pragma unroll
      for (int wv = 0; wv < WAVES; ++wv) v1 += red[wv][mt][j + OUT_TILES][l][e];
      const float g = (float)(T)v0, u = (float)(T)v1;    // the gate/up GEMM's roundings
      const T act = (T)(g / (1.f + expf(-g)));           // F.silu, rounded to the element type
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_row_stride + n0[j] + c] = (T)((float)act * u);
    }
  }
}

// Launch shape: NT tiles per workgroup, WAVES waves splitting each K range,
// `splits` K ranges (partial epilogue only).
struct lin_shape {
  int nt, waves, splits;
};

template <typename Tag, int MODE, int MT, int NT>
static int launch_waves(const lin_args& a, dim3 grid, int waves, hipStream_t stream) {
  if (waves == 8) {
    if constexpr (8 * MT * NT <= 64) {
      hipLaunchKernelGGL((linear_kernel<Tag, MT, NT, 8, MODE>), grid, dim3(512), 0, stream, a);
      return 0;
    }
    return -1;
  }
  hipLaunchKernelGGL((linear_kernel<Tag, MT, NT, 4, MODE>), grid, dim3(256), 0, stream, a);
  return 0;
}

template <typename Tag, int MODE, int MT>
static int launch_nt(const lin_args& a, dim3 grid, const lin_shape& s, hipStream_t stream) {
  if (s.nt == 4) return launch_waves<Tag, MODE, MT, 4>(a, grid, s.waves, stream);
  if (s.nt == 2) return launch_waves<Tag, MODE, MT, 2>(a, grid, s.waves, stream);
  if constexpr (MODE != LIN_SILU) return launch_waves<Tag, MODE, MT, 1>(a, grid, s.waves, stream);
  return -1;
}

template <typename Tag, int MODE>
static int launch_linear(const lin_args& a, const lin_shape& s, hipStream_t stream) {
  const int tiles = a.N / 16 / s.nt;
  const dim3 grid(tiles, s.splits);
  switch ((a.M + 15) / 16) {
    case 1: return launch_nt<Tag, MODE, 1>(a, grid, s, stream);
    case 2: return launch_nt<Tag, MODE, 2>(a, grid, s, stream);
    case 3: return launch_nt<Tag, MODE, 3>(a, grid, s, stream);
    default: return launch_nt<Tag, MODE, 4>(a, grid, s, stream);
  }
}

template <int MODE>
static int launch_dtype(const lin_args& a, const lin_shape& s, int32_t dtype, hipStream_t stream) {
  if (dtype == TB_DTYPE_F16) return launch_linear<f16_t, MODE>(a, s, stream);
  return launch_linear<bf16_t, MODE>(a, s, stream);
}

// Launch shapes measured at the engine's decode shapes (0.5B dims, 1..32 rows,
// 24 layers of weights rotating). Every workgroup reads all of X (M x K) from
// L2 for its NT tiles, so the X reads per weight byte are M / (16 NT): more
// tiles per workgroup pay off once rows grow (gate/up at 32 rows: 12.2 us
// with one tile, 10.7 with four), fewer and larger workgroups cost where the
// grid gets small (gate/up at 1 row: 6.7 vs 8.1 us).
static lin_shape round_shape() { return lin_shape{1, 4, 1}; }
static lin_shape partial_shape(int M, int N, int splits) {
  return lin_shape{M > 8 && (N / 16) % 2 == 0 ? 2 : 1, 4, splits};
}
static lin_shape silu_shape(int d_ff) { return lin_shape{(d_ff / 16) % 2 == 0 ? 4 : 2, 4, 1}; }

static int32_t check_common(const void* x, int64_t x_row_stride, const void* w, int32_t rows, int32_t out_features,
                            int32_t in_features, int32_t dtype) {
  if (rows < 0 || out_features <= 0 || in_features <= 0) return TB_ERR_INVALID_ARG;
  if (dtype != TB_DTYPE_F16 && dtype != TB_DTYPE_BF16) return TB_ERR_UNSUPPORTED;
  if (rows > 64 || out_features % 16 != 0 || in_features % 32 != 0) return TB_ERR_UNSUPPORTED;
  if (rows == 0) return TB_OK;
  if (!x || !w || x_row_stride < in_features) return TB_ERR_INVALID_ARG;
  if ((((uintptr_t)x | (uintptr_t)w) & 15u) != 0 || (x_row_stride * 2) % 16 != 0) return TB_ERR_INVALID_ARG;
  return TB_OK;
}

}  // namespace tb

extern "C" int32_t tb_linear(const void* x, int64_t x_row_stride, const void* w, const void* bias, void* y,
                             int64_t y_row_stride, int32_t rows, int32_t out_features, int32_t in_features,
                             int32_t dtype, hipStream_t stream) {
  using namespace tb;
  const int32_t st = check_common(x, x_row_stride, w, rows, out_features, in_features, dtype);
  if (st != TB_OK || rows == 0) return st;
  TB_CHECK_ARG(y && y_row_stride >= out_features);
  const lin_args a{(const char*)x, x_row_stride * 2, (const char*)w, (const char*)bias, y, y_row_stride,
                   rows, out_features, in_features};
  if (launch_dtype<LIN_ROUND>(a, round_shape(), dtype, stream)) return TB_ERR_UNSUPPORTED;
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_linear_partials(const void* x, int64_t x_row_stride, const void* w, float* partials,
                                      int32_t splits, int32_t rows, int32_t out_features, int32_t in_features,
                                      int32_t dtype, hipStream_t stream) {
  using namespace tb;
  const int32_t st = check_common(x, x_row_stride, w, rows, out_features, in_features, dtype);
  if (st != TB_OK) return st;
  TB_CHECK_ARG(splits >= 1 && splits <= 64 && splits <= in_features / 32);
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(partials);
  const lin_args a{(const char*)x, x_row_stride * 2, (const char*)w, nullptr, partials, 0,
                   rows, out_features, in_features};
  if (launch_dtype<LIN_PARTIAL>(a, partial_shape(rows, out_features, splits), dtype, stream))
    return TB_ERR_UNSUPPORTED;
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_linear_silu_mul(const void* x, int64_t x_row_stride, const void* w_gate_up, void* y,
                                      int64_t y_row_stride, int32_t rows, int32_t d_ff, int32_t in_features,
                                      int32_t dtype, hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(d_ff > 0 && d_ff <= (1 << 29));
  const int32_t st = check_common(x, x_row_stride, w_gate_up, rows, 2 * d_ff, in_features, dtype);
  if (st != TB_OK) return st;
  if (d_ff % 16 != 0) return TB_ERR_UNSUPPORTED;
  if (rows == 0) return TB_OK;
  TB_CHECK_ARG(y && y_row_stride >= d_ff);
  const lin_args a{(const char*)x, x_row_stride * 2, (const char*)w_gate_up, nullptr, y, y_row_stride,
                   rows, 2 * d_ff, in_features};
  if (launch_dtype<LIN_SILU>(a, silu_shape(d_ff), dtype, stream)) return TB_ERR_UNSUPPORTED;
  TB_RETURN_LAUNCH_STATUS();
}
