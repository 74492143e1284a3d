// Shared device helpers for the paged KV-cache kernels (gfx950 / CDNA4).
//
// Pool layout (kept verbatim from the reference, src/tinybatch/kv_cache.py:1-7,17-20):
//   pool[num_blocks][2][num_kv_heads][block_size][head_dim], axis 1: 0 = K, 1 = V.
//   Element (blk, kv, h, s, d) lives at (((blk*2 + kv)*Hkv + h)*BS + s)*D + d.
// A (block, kv head) K or V tile [BS x D] is therefore contiguous, which is what
// every kernel here streams with 16-byte vector loads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tinybatch_amd.h"

namespace tb {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// 16 bytes moved per lane per vector load/store.
struct alignas(16) vec16 {
  uint32_t w[4];
};

__device__ __forceinline__ vec16 ld16(const void* p) {
  const uint4 v = *reinterpret_cast<const uint4*>(p);
  vec16 r;
  r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  return r;
}

// Streamed once (K/V rows): non-temporal hint, the line is not kept in L2.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ vec16 ld16_stream(const void* p) {
  const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
  vec16 r;
  r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
  return r;
}

__device__ __forceinline__ void st16(void* p, const vec16& r) {
  uint4 v;
  v.x = r.w[0]; v.y = r.w[1]; v.z = r.w[2]; v.w = r.w[3];
  *reinterpret_cast<uint4*>(p) = v;
}

__device__ __forceinline__ vec16 zero16() {
  vec16 r;
  r.w[0] = r.w[1] = r.w[2] = r.w[3] = 0u;
  return r;
}

// ---- element traits -------------------------------------------------------
struct f32_t {};
struct f16_t {};
struct bf16_t {};

template <typename Tag> struct elem;
template <> struct elem<f32_t> {
  using type = float;
  static constexpr int bytes = 4;
};
template <> struct elem<f16_t> {
  using type = _Float16;
  static constexpr int bytes = 2;
};
template <> struct elem<bf16_t> {
  using type = __bf16;
  static constexpr int bytes = 2;
};

__device__ __forceinline__ float bits_to_f32(uint32_t u) { return __uint_as_float(u); }

// ---- cross-lane helpers ---------------------------------------------------
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xf, 0xf, false));
}

// DPP control words (GCN/CDNA encoding).
constexpr int DPP_QUAD_XOR1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141; // lane i <- lane 7-i inside each 8-lane half row
constexpr int DPP_ROW_MIRROR = 0x140;      // lane i <- lane 15-i inside each 16-lane row
constexpr int DPP_ROW_ROR8 = 0x128;        // lane i <- lane (i+8)%16 inside a row, i.e. xor 8

// Sum over aligned groups of N consecutive lanes; every lane of a group ends
// with the group total. Pairings: xor1, xor2, then mirrors, which pair each
// lane with a lane of the other half once the halves are already reduced.
template <int N>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(N == 1 || N == 2 || N == 4 || N == 8 || N == 16 || N == 32 || N == 64, "group");
  if constexpr (N >= 2) x += dpp<DPP_QUAD_XOR1>(x);
  if constexpr (N >= 4) x += dpp<DPP_QUAD_XOR2>(x);
  if constexpr (N >= 8) x += dpp<DPP_ROW_HALF_MIRROR>(x);
  if constexpr (N >= 16) x += dpp<DPP_ROW_MIRROR>(x);
  if constexpr (N >= 32) x += __shfl_xor(x, 16);
  if constexpr (N >= 64) x += __shfl_xor(x, 32);
  return x;
}

template <int MASK>
__device__ __forceinline__ float lane_xor(float x) {
  if constexpr (MASK == 1) return dpp<DPP_QUAD_XOR1>(x);
  else if constexpr (MASK == 2) return dpp<DPP_QUAD_XOR2>(x);
  else if constexpr (MASK == 8) return dpp<DPP_ROW_ROR8>(x);
  else return __shfl_xor(x, MASK);
}

// Reduce across lanes that differ only in the bits >= FIRST (lane groups of
// FIRST consecutive lanes hold the same "column"): max and sum variants.
template <int FIRST>
__device__ __forceinline__ float cross_group_max(float x) {
  if constexpr (FIRST <= 1) x = fmaxf(x, lane_xor<1>(x));
  if constexpr (FIRST <= 2) x = fmaxf(x, lane_xor<2>(x));
  if constexpr (FIRST <= 4) x = fmaxf(x, lane_xor<4>(x));
  if constexpr (FIRST <= 8) x = fmaxf(x, lane_xor<8>(x));
  if constexpr (FIRST <= 16) x = fmaxf(x, lane_xor<16>(x));
  if constexpr (FIRST <= 32) x = fmaxf(x, lane_xor<32>(x));
  return x;
}

template <int FIRST>
__device__ __forceinline__ float cross_group_sum(float x) {
  if constexpr (FIRST <= 1) x += lane_xor<1>(x);
  if constexpr (FIRST <= 2) x += lane_xor<2>(x);
  if constexpr (FIRST <= 4) x += lane_xor<4>(x);
  if constexpr (FIRST <= 8) x += lane_xor<8>(x);
  if constexpr (FIRST <= 16) x += lane_xor<16>(x);
  if constexpr (FIRST <= 32) x += lane_xor<32>(x);
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// gfx950 LDS transpose read (ds_read_b64_tr_b16). Within each group of 16
// lanes, lane i receives element (i & 3) of the 8-byte LDS rows addressed by
// lanes (i >> 2) + 4j, j = 0..3, in that order. With lane s of a group
// pointing at row r0 + (s >> 2), elements 4 (s & 3) .. 4 (s & 3) + 3 of a
// row-major 16-bit matrix, lane i gets column i of rows r0 .. r0 + 3: the
// k-contiguous operand layout of a 16x16x32 MFMA, read from row-major data.
typedef short short4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const void* p) {
  const short4_t r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) short4_t*)(const_cast<void*>(p)));
  return __builtin_bit_cast(uint2, r);
}

// Reductions across the 16-lane rows of a wave on the VALU (gfx950 permlane
// swaps, no LDS round trip): combine lane l with lane l ^ 16 / l ^ 32.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

}  // namespace tb

// Status helpers shared by the C entry points.
#define TB_CHECK_ARG(cond)               \
  do {                                   \
    if (!(cond)) return TB_ERR_INVALID_ARG; \
  } while (0)

#define TB_RETURN_LAUNCH_STATUS()                        \
  do {                                                   \
    hipError_t _e = hipGetLastError();                   \
    return _e == hipSuccess ? TB_OK : TB_ERR_LAUNCH;      \
  } while (0)
