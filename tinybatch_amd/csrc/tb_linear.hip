// Skinny linear layers for decode-sized batches (the engine's projections,
// reference src/tinybatch/model.py:121-124,149-154: F.linear with weights
// [N][K], K contiguous):
//   Y[M][N] = X[M][K] . W[N][K]^T (+ bias[N]),   M <= 64.
// At decode batch sizes the weight is the whole cost (N*K*2 bytes read once,
// X and Y are a few KB), so the kernels are weight streams. A workgroup of
// four waves owns TW tiles of 16 output columns and one K range; the
// 4 / TW waves of a tile split the range between them.
//   v_mfma_f32_16x16x32_{f16,bf16}: A = X rows (m-tile of 16) from LDS,
//   B = W rows straight from HBM (lane l: W[n0 + l%16][k + 8(l/16) .. +8]),
//   C/D lane l: Y[m0 + 4(l/16) + j][n0 + l%16].
// X reaches LDS by row-contiguous direct loads (global_load_lds, consecutive
// lanes along a row, whole 128-byte lines per instruction) and is read from
// there in the MFMA layout; the row pitch is 1 mod 16 units of 16 bytes, so
// the 16 rows one read touches fall in 16 different bank groups. Reading X
// from memory in the MFMA layout (16 rows x 64 bytes per instruction, half of
// each line) had cost as much as the weight stream itself: for the 9728 x 896
// gate/up weight at 32 rows, 9.5 us against 6.1 us for the same bytes read
// row-contiguously, 4.8 us for the weight alone (load-pattern probe).
// W keeps the MFMA-layout loads into registers (all of a wave's loads for the
// K range in flight at once); the other half of each of their lines is the
// next k-slice's load, so they are plain loads that keep the line
// (non-temporal ones measured 5-25% slower).
// Three epilogues, after the tile's waves meet in LDS:
//   round   : Y = T(sum + bias), one rounding as F.linear's single GEMM;
//   partial : fp32 sums of one K range to partials[split][M][N] (the split-K
//             pieces; tb_rms_norm_partials adds them in split order, rounds
//             once and continues with the residual add and RMSNorm);
//   silu    : tiles j < TW/2 are gate columns, tile j + TW/2 the up columns
//             d_ff later (merged gate/up weight); Y = silu(T(gate)) * T(up)
//             with the roundings of F.linear followed by tb_silu_mul
//             (model.py:151-154);
//   silu8   : the same with 8 features per workgroup: lanes 0-7 of the one
//             tile load gate rows, lanes 8-15 the up rows of the same
//             features, so twice the workgroups share the weight stream;
//   argmax  : the LM head followed by greedy sampling (model.py:157-158,
//             engine.py:145-151): per row, the largest T(sum) of the
//             workgroup's columns and its index go to a workspace slot, and
//             argmax_rows_kernel picks each row's winner over the slots.
//             Order: NaN above everything, -0 equal to +0, the first index
//             among equals (torch.argmax over the rounded logits).
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

enum { LIN_ROUND = 0, LIN_PARTIAL = 1, LIN_SILU = 2, LIN_ARGMAX = 3, LIN_SILU8 = 4 };
constexpr int LIN_WAVES = 4;

// A workgroup walks its K range in windows of up to SP = 28 k-slices (d_model
// 896 in one window): every wave issues all of its W loads for the window,
// then X of the window is staged (one chunk up to 32 rows: staging it in two
// halves to fit more workgroups on a CU measured slower, the second round
// trip costing more than the occupancy gained; 33..64 rows in chunks of 14).
constexpr int LIN_SP = 28;
template <int MT>
struct lin_pass {
  static constexpr int CH = MT <= 2 ? 28 : 14;
  static __host__ __device__ constexpr int pitch(int slices) { return (4 * slices + 15) / 16 * 16 + 1; }
  static constexpr int lds_bytes(int nt) {
    const int staged = (16 * MT * pitch(CH) + 63) / 64 * 1024;
    return staged > 4096 * MT * nt ? staged : 4096 * MT * nt;
  }
};

// Argmax candidates as one 64-bit key: the value's order in the high word (a
// total order of floats with NaN on top and -0 = +0), the complement of the
// column in the low word, so that the larger key is the larger value and,
// among equals, the smaller column.
__device__ __forceinline__ uint64_t argmax_key(float v, int col) {
  uint32_t k;
  if (v != v) {
    k = 0xFFFFFFFFu;
  } else {
    const int b = __float_as_int(v == 0.f ? 0.f : v);
    k = (uint32_t)(b >= 0 ? b : b ^ 0x7FFFFFFF) ^ 0x80000000u;
  }
  return ((uint64_t)k << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)col);
}
__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
  const uint32_t lo = __shfl_xor((uint32_t)v, m), hi = __shfl_xor((uint32_t)(v >> 32), m);
  return ((uint64_t)hi << 32) | lo;
}

struct lin_args {
  const char* x;
  int64_t x_row_bytes;
  const char* w;              // [N][K]
  const char* bias;           // [N] or null (round epilogue only)
  void* y;                    // round / silu: [M][y_row_stride] of T; partial: float [splits][M][N]
  int64_t y_row_stride;       // elements
  int M, N, K;                // K range s of gridDim.y: k-slices [s*K/32/splits, (s+1)*K/32/splits)
};

// Four waves split the K range; each wave computes all NT tiles of the
// workgroup over its share, reading its X fragment from LDS once for them.
template <typename Tag, int MT, int NT, int MODE>
__global__ __launch_bounds__(64 * LIN_WAVES) void linear_kernel(lin_args a) {
  using L = lin_math<Tag>;
  using PS = lin_pass<MT>;
  typedef typename L::scalar_t T;
  constexpr int KB = (LIN_SP + LIN_WAVES - 1) / LIN_WAVES;   // k-slices per wave per window
  constexpr int OUT_TILES = MODE == LIN_SILU ? NT / 2 : NT;
  constexpr int ROWS = 16 * MT;
  static_assert(MODE != LIN_SILU || NT % 2 == 0, "silu pairs gate and up tiles");
  constexpr bool HALF = MODE == LIN_SILU8;
  static_assert(!HALF || NT == 1, "silu8: one tile of 8 gate and 8 up columns");
  __shared__ __align__(16) char lds[PS::lds_bytes(NT)];
  // wave-uniform in a scalar register: the K-share tests below become scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  int n0[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j)
    n0[j] = HALF ? (int)blockIdx.x * 8
                 : (MODE == LIN_SILU ? (j / OUT_TILES) * (a.N >> 1) : 0) + (blockIdx.x * OUT_TILES + j % OUT_TILES) * 16;
  const int slices = a.K / 32;
  const int k_begin = (int)blockIdx.y * slices / (int)gridDim.y;
  const int range = ((int)blockIdx.y + 1) * slices / (int)gridDim.y - k_begin;
  const char* wrow[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) {
    const int wr = HALF ? (lc < 8 ? n0[j] + lc : (a.N >> 1) + n0[j] + lc - 8) : n0[j] + lc;   // this lane's W row
    wrow[j] = a.w + (int64_t)wr * a.K * 2 + (int64_t)k_begin * 64 + 16 * lg;
  }
  const char* const xk = a.x + (int64_t)k_begin * 64;

  float4_t acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mt][j] = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int w0 = 0; w0 < range; w0 += LIN_SP) {         // windows and chunks: the same in every wave
    const int wn = min(LIN_SP, range - w0);
    const int per = (wn + LIN_WAVES - 1) / LIN_WAVES;
    const int sb = wave * per, se = min(wn, sb + per);  // this wave's slices of the window
    vec16 wb[NT][KB];
#pragma unroll
    for (int i = 0; i < KB; ++i)
      if (sb + i < se) {
#pragma unroll
        for (int j = 0; j < NT; ++j) wb[j][i] = ld16(wrow[j] + (int64_t)(w0 + sb + i) * 64);
      }
    for (int x0 = 0; x0 < wn; x0 += PS::CH) {
      const int xn = min(PS::CH, wn - x0);
      const int P = PS::pitch(xn), units = ROWS * P, used = 4 * xn;
      if (w0 + x0 > 0) __syncthreads();                 // the last chunk's X reads are done
      // X rows [0, ROWS) x the chunk's slices -> LDS unit r * P + c (unit = 16 bytes);
      // load q covers units 64 q .. 64 q + 63, lane order along the rows.
      {
        int p = wave * 64 + lane;
        int r = p / P, c = p - r * P;
        const int dr = 256 / P, dc = 256 - dr * P;
        const char* const xc = xk + (int64_t)(w0 + x0) * 64;
        for (int q = wave; q * 64 < units; q += LIN_WAVES) {
          const bool real = r < ROWS && c < used;
          const char* src = real ? xc + (int64_t)min(r, a.M - 1) * a.x_row_bytes + 16 * c : a.x;
          __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                           (__attribute__((address_space(3))) void*)(lds + 1024 * q), 16, 0, 0);
          c += dc;
          r += dr;
          if (c >= P) {
            c -= P;
            ++r;
          }
        }
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      // the wave's X fragments of this chunk first (all LDS reads in flight), then the MFMAs
      vec16 xa[KB][MT];
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        const int sl = sb + i;
        if (sl < se && sl >= x0 && sl < x0 + xn) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            xa[i][mt] = *reinterpret_cast<const vec16*>(lds + 16 * ((16 * mt + lc) * P + 4 * (sl - x0) + lg));
        }
      }
#pragma unroll
      for (int i = 0; i < KB; ++i) {
        const int sl = sb + i;
        if (sl < se && sl >= x0 && sl < x0 + xn) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < NT; ++j) acc[mt][j] = L::mfma(xa[i][mt], wb[j][i], acc[mt][j]);
        }
      }
    }
  }
  __syncthreads();                                      // X reads done: the area holds the sums now
  float* red = reinterpret_cast<float*>(lds);           // [wave][mt][tile][lane][4]
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) red[(((wave * MT + mt) * NT + j) * 64 + lane) * 4 + e] = acc[mt][j][e];
  __syncthreads();
  if constexpr (HALF) {
    // thread t: output (row m, feature n0 + c); gate in column c, up in column c + 8
    for (int t = threadIdx.x; t < MT * 128; t += 64 * LIN_WAVES) {
      const int c = t & 7, m = t >> 3;
      if (m >= a.M) continue;
      const int mt = m >> 4, r = m & 15;
      const int l = 16 * (r >> 2) + c, e = r & 3;
      float gs = 0.f, us = 0.f;
#pragma unroll
      for (int wv = 0; wv < LIN_WAVES; ++wv) {
        gs += red[((wv * MT + mt) * 64 + l) * 4 + e];
        us += red[((wv * MT + mt) * 64 + l + 8) * 4 + e];
      }
      const float g = (float)(T)gs, u = (float)(T)us;   // the gate/up GEMM's roundings
      const T act = (T)(g / (1.f + expf(-g)));
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_row_stride + n0[0] + c] = (T)((float)act * u);
    }
    return;
  }
  // thread t: output element (row m, tile j, column c); the waves' K shares added in order
  for (int t = threadIdx.x; t < MT * 256 * OUT_TILES; t += 64 * LIN_WAVES) {
    const int c = t & 15, j = (t >> 4) % OUT_TILES, m = t / (16 * OUT_TILES);
    if (m >= a.M) continue;
    const int mt = m >> 4, r = m & 15;
    const int l = 16 * (r >> 2) + c, e = r & 3;          // the D lane and element holding (r, c)
    auto tile_sum = [&](int tile) {
      float v = 0.f;
#pragma unroll
      for (int wv = 0; wv < LIN_WAVES; ++wv) v += red[(((wv * MT + mt) * NT + tile) * 64 + l) * 4 + e];
      return v;
    };
    const float v0 = tile_sum(j);
    if constexpr (MODE == LIN_ROUND) {
      const float b = a.bias ? (float)reinterpret_cast<const T*>(a.bias)[n0[j] + c] : 0.f;
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_row_stride + n0[j] + c] = (T)(v0 + b);
    } else if constexpr (MODE == LIN_PARTIAL) {
      reinterpret_cast<float*>(a.y)[((int64_t)blockIdx.y * a.M + m) * a.N + n0[j] + c] = v0;
    } else if constexpr (MODE == LIN_ARGMAX) {
      // the row's 16 NT columns sit in 16 NT consecutive lanes (16 NT divides 64)
      uint64_t key = argmax_key((float)(T)v0, n0[j] + c);
#pragma unroll
      for (int sh = 1; sh < 16 * NT; sh <<= 1) key = max_u64(key, shfl_xor_u64(key, sh));
      if ((t & (16 * NT - 1)) == 0) reinterpret_cast<uint64_t*>(a.y)[(int64_t)m * gridDim.x + blockIdx.x] = key;
    } else {
      const float g = (float)(T)v0, u = (float)(T)tile_sum(j + OUT_TILES);   // the gate/up GEMM's roundings
      const T act = (T)(g / (1.f + expf(-g)));           // F.silu, rounded to the element type
      reinterpret_cast<T*>(a.y)[(int64_t)m * a.y_row_stride + n0[j] + c] = (T)((float)act * u);
    }
  }
}

// Row r's winner over its n candidate keys (one workgroup per row).
__global__ __launch_bounds__(256) void argmax_rows_kernel(const uint64_t* __restrict__ keys, int n,
                                                          int64_t* __restrict__ ids) {
  __shared__ uint64_t part[4];
  const uint64_t* row = keys + (int64_t)blockIdx.x * n;
  uint64_t best = 0;
  for (int i = threadIdx.x; i < n; i += 256) best = max_u64(best, row[i]);
#pragma unroll
  for (int sh = 1; sh < 64; sh <<= 1) best = max_u64(best, shfl_xor_u64(best, sh));
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    best = max_u64(max_u64(part[0], part[1]), max_u64(part[2], part[3]));
    ids[blockIdx.x] = (int64_t)(0xFFFFFFFFu - (uint32_t)best);
  }
}

// Launch shape: NT tiles per workgroup, `splits` K ranges (partial epilogue only).
struct lin_shape {
  int tw, splits;
};

template <typename Tag, int MODE, int MT>
static int launch_tw(const lin_args& a, dim3 grid, int tw, hipStream_t stream) {
  if constexpr (MODE == LIN_SILU8) {
    if (tw != 1) return -1;
    hipLaunchKernelGGL((linear_kernel<Tag, MT, 1, MODE>), grid, dim3(256), 0, stream, a);
  } else {
    if (tw == 4) hipLaunchKernelGGL((linear_kernel<Tag, MT, 4, MODE>), grid, dim3(256), 0, stream, a);
    else if (tw == 2) hipLaunchKernelGGL((linear_kernel<Tag, MT, 2, MODE>), grid, dim3(256), 0, stream, a);
    else if constexpr (MODE != LIN_SILU) hipLaunchKernelGGL((linear_kernel<Tag, MT, 1, MODE>), grid, dim3(256), 0, stream, a);
    else return -1;
  }
  return 0;
}

template <typename Tag, int MODE>
static int launch_linear(const lin_args& a, const lin_shape& s, hipStream_t stream) {
  if (s.tw != 1 && s.tw != 2 && s.tw != 4) return -1;
  const dim3 grid(a.N / 16 / s.tw, s.splits);
  switch ((a.M + 15) / 16) {
    case 1: return launch_tw<Tag, MODE, 1>(a, grid, s.tw, stream);
    case 2: return launch_tw<Tag, MODE, 2>(a, grid, s.tw, stream);
    case 3: return launch_tw<Tag, MODE, 3>(a, grid, s.tw, stream);
    default: return launch_tw<Tag, MODE, 4>(a, grid, s.tw, stream);
  }
}

template <int MODE>
static int launch_dtype(const lin_args& a, const lin_shape& s, int32_t dtype, hipStream_t stream) {
  if (dtype == TB_DTYPE_F16) return launch_linear<f16_t, MODE>(a, s, stream);
  return launch_linear<bf16_t, MODE>(a, s, stream);
}

// Launch shapes, measured at the engine's decode shapes (0.5B dims, 1..32 rows,
// 24 layers of weights rotating). The weight stream is bound by how evenly
// the 16-column tiles spread over the 256 CUs, so one tile per workgroup
// (the most workgroups) wins for q/k/v and for the split-K pieces up to 16
// rows; with more rows every workgroup's X staging weighs more and two or
// four tiles per workgroup share it (gate/up at 32 rows: 10.1 us with one
// tile pair, 9.8 with two pairs; down 5.6 -> 5.2 us with two tiles). Gate/up
// up to 16 rows takes 8 features per workgroup (silu8: 608 workgroups instead
// of 304 at d_ff 4864, 8.6 -> 7.0 us at 1 row, 9.0 -> 7.7 at 16); above 16
// rows the doubled X staging makes it slower (9.8 -> 10.2 us at 32).
static lin_shape round_shape() { return lin_shape{1, 1}; }
static lin_shape partial_shape(int M, int N, int K, int splits) {
  const int range = K / 32 / splits;
  return lin_shape{M > 16 && range >= 16 && (N / 16) % 2 == 0 ? 2 : 1, splits};
}
static lin_shape silu_shape(int M, int d_ff) {
  return lin_shape{M > 16 && (d_ff / 16) % 2 == 0 ? 4 : 2, 1};
}
// LM head (151936 x 896): two tiles per workgroup up to 16 rows, four above.
static lin_shape argmax_shape(int M, int N) {
  const int tiles = N / 16;
  if (M > 16 && tiles % 4 == 0) return lin_shape{4, 1};
  return lin_shape{tiles % 2 == 0 ? 2 : 1, 1};
}

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
  if (launch_dtype<LIN_PARTIAL>(a, partial_shape(rows, out_features, in_features, splits), dtype, stream))
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
  const int st8 = rows <= 16 ? launch_dtype<LIN_SILU8>(a, lin_shape{1, 1}, dtype, stream)
                             : launch_dtype<LIN_SILU>(a, silu_shape(rows, d_ff), dtype, stream);
  if (st8) return TB_ERR_UNSUPPORTED;
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" size_t tb_linear_argmax_workspace_bytes(int32_t rows, int32_t out_features) {
  if (rows <= 0 || out_features <= 0) return 0;
  return (size_t)rows * (size_t)(out_features / 16) * sizeof(uint64_t);
}

extern "C" int32_t tb_linear_argmax(const void* x, int64_t x_row_stride, const void* w, int32_t rows,
                                    int32_t out_features, int32_t in_features, void* workspace,
                                    size_t workspace_bytes, int64_t* ids, int32_t dtype, hipStream_t stream) {
  using namespace tb;
  const int32_t st = check_common(x, x_row_stride, w, rows, out_features, in_features, dtype);
  if (st != TB_OK || rows == 0) return st;
  TB_CHECK_ARG(workspace && ids && ((uintptr_t)workspace & 7u) == 0);
  TB_CHECK_ARG(workspace_bytes >= tb_linear_argmax_workspace_bytes(rows, out_features));
  const lin_shape shape = argmax_shape(rows, out_features);
  const lin_args a{(const char*)x, x_row_stride * 2, (const char*)w, nullptr, workspace, 0,
                   rows, out_features, in_features};
  if (launch_dtype<LIN_ARGMAX>(a, shape, dtype, stream)) return TB_ERR_UNSUPPORTED;
  hipLaunchKernelGGL(argmax_rows_kernel, dim3(rows), dim3(256), 0, stream, (const uint64_t*)workspace,
                     out_features / 16 / shape.tw, ids);
  TB_RETURN_LAUNCH_STATUS();
}
