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

// Cache policy of a buffer load that must see stores other CUs of this XCD (or this
// wave, just before) made to the L2: SC1 set, device scope, so the load misses in
// the CU's vector L1 and is served by the L2. SC0 alone (workgroup scope) may still
// hit a stale L1 line.
constexpr int LOAD_DEVICE_SCOPE = 16;

__device__ __forceinline__ void st16(void* p, const vec16& r) {
  uint4 v;
  v.x = r.w[0]; v.y = r.w[1]; v.z = r.w[2]; v.w = r.w[3];
  *reinterpret_cast<uint4*>(p) = v;
}

// Stores of a kernel's results (outputs, appended rows, copied blocks), written
// through this XCD's L2 at device scope (SC1). A plain store leaves the line
// dirty in the L2. The L2 then writes it back at the kernel's end, and the
// kernel completes only after that write-back. A written-through line goes to
// memory while the kernel still runs. Same bits either way.
// Measured, same box:
// - the 1024-block copy over 24 pools: 73.0 against 86.9 us;
// - the prefill rows of 8 x 512 bf16: 11.9 against 12.5 us per layer.
// The 16-byte form is one vector store instruction; the compiler does not count
// it in its own waits, so any later wait it makes only waits longer.
__device__ __forceinline__ void st16_through(void* p, const vec16& r) {
  const u32x4_t v = {r.w[0], r.w[1], r.w[2], r.w[3]};
  asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}
template <typename T>
__device__ __forceinline__ void st8_through(void* p, const T& r) {
  static_assert(sizeof(T) == 8, "an 8-byte value");
  __hip_atomic_store(reinterpret_cast<uint64_t*>(p), __builtin_bit_cast(uint64_t, r), __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
// An 8- or 16-byte value (four 16-bit or four 32-bit elements) written through.
template <typename T>
__device__ __forceinline__ void st_through(void* p, const T& r) {
  static_assert(sizeof(T) == 8 || sizeof(T) == 16, "an 8- or 16-byte value");
  if constexpr (sizeof(T) == 8) {
    st8_through(p, r);
  } else {
    const u32x4_t v = __builtin_bit_cast(u32x4_t, r);
    asm volatile("global_store_dwordx4 %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
  }
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

// Maxima of softmax scores (MFMA results or -inf, never NaN): IEEE-754 maximum
// needs no quieting of its inputs, so a pair or triple is one v_maximum3_f32 (a
// plain fmaxf in IEEE mode first quiets every input with an extra v_max). Written
// with builtins, never inline asm: the compiler inserts the wait states between an
// MFMA and a VALU read of its result only for reads it can see, and an asm max
// placed right after an MFMA reads the accumulator's previous contents.
__device__ __forceinline__ float max_f32(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}

// Reductions across the 16-lane rows of a wave on the VALU (gfx950 permlane
// swaps, no LDS round trip): combine lane l with lane l ^ 16 / l ^ 32.
__device__ __forceinline__ float max_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return max_f32(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// A product rounded on its own to fp32: a multiply the compiler may not contract
// into a following add (HIP's __fmul_rn is a plain multiply, and whether it is
// fused into an FMA depends on where it is inlined), nor fold with a following
// conversion to fp16 into one v_fma_mixlo (a single rounding). The multiply is an
// ordinary instruction, so the compiler sees its operand reads (the wait states
// after v_rsq and the like); the empty asm only hides the product's origin from
// the folds and executes nothing.
__device__ __forceinline__ float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  float p = a * b;
  asm("" : "+v"(p));
  return p;
}

// Rotate-half RoPE (reference src/tinybatch/model.py:72-80) of one 16-byte
// chunk pair of a head row: x1 holds dims i .. i+n-1 of the first half, x2 the
// same dims of the second half, c / s point at the fp32 cos / sin table entries
// of dims i .. of the position (n = 16 / sizeof(T)):
//   x1' = x1 c - x2 s,  x2' = x2 c + x1 s,
// each product rounded on its own as the separate tensor ops round it, the
// result rounded to the element type (the arithmetic of tb_rope_qk).
template <typename T>
__device__ __forceinline__ void rope_pair(vec16& x1, vec16& x2, const float* c, const float* s) {
  constexpr int N = 16 / sizeof(T);
  T a[N], b[N];
  __builtin_memcpy(a, &x1, 16);
  __builtin_memcpy(b, &x2, 16);
  float cv[N], sv[N];
#pragma unroll
  for (int q = 0; q < N; q += 4) {
    const float4 c4 = *reinterpret_cast<const float4*>(c + q);
    const float4 s4 = *reinterpret_cast<const float4*>(s + q);
    cv[q] = c4.x; cv[q + 1] = c4.y; cv[q + 2] = c4.z; cv[q + 3] = c4.w;
    sv[q] = s4.x; sv[q + 1] = s4.y; sv[q + 2] = s4.z; sv[q + 3] = s4.w;
  }
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float u = (float)a[e], w = (float)b[e];
    a[e] = (T)(mul_rn(u, cv[e]) - mul_rn(w, sv[e]));
    b[e] = (T)(mul_rn(w, cv[e]) + mul_rn(u, sv[e]));
  }
  __builtin_memcpy(&x1, a, 16);
  __builtin_memcpy(&x2, b, 16);
}

// RoPE tables of a call: fp32 cos / sin [max_position][head_dim / 2]; the
// position is clamped into the table (the host validates positions).
struct rope_tables {
  const float* cos;
  const float* sin;
  int32_t max_position;
  __device__ __forceinline__ int64_t row(int64_t p, int half) const {
    p = p < 0 ? 0 : (p >= max_position ? max_position - 1 : p);
    return p * half;
  }
};

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
