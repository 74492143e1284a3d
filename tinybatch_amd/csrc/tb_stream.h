// Shared pieces of the streaming kernels (decode and prefill), gfx950: the
// 16x16x32 MFMA of a 16-bit type with its 8-value operand packing, direct
// global->LDS loads issued as asm with explicit vm-count waits, the swizzled
// 16-position K / V tile layout in LDS, and the asm block that reads a pair of
// such tiles as MFMA operands.
#pragma once

#include "tb_common.h"

namespace tb {

typedef _Float16 shalf8_t __attribute__((ext_vector_type(8)));
typedef __bf16 sbf168_t __attribute__((ext_vector_type(8)));
typedef unsigned int su32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int su32x4_t __attribute__((ext_vector_type(4)));

template <typename Tag>
struct smath;
template <>
struct smath<f16_t> {
  typedef _Float16 scalar_t;
  static __device__ __forceinline__ float4_t mfma32(su32x4_t a, su32x4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(shalf8_t, a), __builtin_bit_cast(shalf8_t, b), c,
                                                   0, 0, 0);
  }
  // 8 probabilities as the B operand of the 16x16x32 product
  static __device__ __forceinline__ su32x4_t pack8(const float (&p)[8]) {
    shalf8_t h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (_Float16)p[i];
    return __builtin_bit_cast(su32x4_t, h);
  }
};
template <>
struct smath<bf16_t> {
  typedef __bf16 scalar_t;
  static __device__ __forceinline__ float4_t mfma32(su32x4_t a, su32x4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(sbf168_t, a), __builtin_bit_cast(sbf168_t, b),
                                                    c, 0, 0, 0);
  }
  static __device__ __forceinline__ su32x4_t pack8(const float (&p)[8]) {
    sbf168_t h;
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (__bf16)p[i];
    return __builtin_bit_cast(su32x4_t, h);
  }
};

// The LDS layout of a 16-position tile: K row r keeps its 16-byte chunk c in
// slot c ^ (r & 7), so the A-operand reads (16 rows x 16 bytes per 16 lanes) cover
// every bank; V row r keeps chunk c in slot c ^ 2 (r & 3), so do the transpose
// reads (4 rows x 32 bytes per 16 lanes). The swizzle is applied on the global
// side of the direct loads: the lane that fills LDS slot c of row r reads chunk
// c ^ swizzle(r).
__device__ __forceinline__ int stream_kswz(int r) { return r & 7; }
__device__ __forceinline__ int stream_vswz(int r) { return 2 * (r & 3); }

__device__ __forceinline__ uint32_t s_lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One direct global->LDS load of a wave: lane l's 16 bytes at src go to
// lds_dst + 16 l (lds_dst wave-uniform, in M0). Issued as asm, so the compiler,
// which cannot tell which LDS a direct load writes, sees none and never makes an
// LDS access wait for one; every wait for these loads is explicit (s_vm_wait_le).
// The s_nop is the wait state an M0 write needs before a direct load.
__device__ __forceinline__ void s_dma16(const void* src, const void* lds_dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(s_lds_addr(lds_dst)) : "memory");
}

// The same with a wave-uniform base (SGPRs) and a per-lane 32-bit byte offset.
__device__ __forceinline__ void s_dma16_s(uint32_t off, const void* base, const void* lds_dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt" ::"v"(off), "s"(base), "{m0}"(s_lds_addr(lds_dst))
               : "memory");
}

// The same without the non-temporal hint, for bytes that other workgroups read
// again soon (the lines stay in the L2). The prefill kernel's K/V range with the
// hint measured 12.6-12.8 against 12.2-12.4 us per layer on 8 x 512 bf16 rows.
__device__ __forceinline__ void s_dma16_l2(uint32_t off, const void* base, const void* lds_dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(s_lds_addr(lds_dst))
               : "memory");
}

// The same with a per-lane 64-bit address and no non-temporal hint.
__device__ __forceinline__ void s_dma16_l2p(const void* src, const void* lds_dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(s_lds_addr(lds_dst)) : "memory");
}

// Wait until at most n vector memory instructions of this wave are outstanding
// (they complete in issue order); n is wave-uniform.
template <int LO, int HI>
__device__ __forceinline__ void s_vm_wait_range(int n) {
  if constexpr (LO == HI) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LO) : "memory");
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID)
      s_vm_wait_range<LO, MID>(n);
    else
      s_vm_wait_range<MID + 1, HI>(n);
  }
}
__device__ __forceinline__ void s_vm_wait_le(int n) { s_vm_wait_range<0, 63>(n < 0 ? 0 : (n > 63 ? 63 : n)); }

// The reads of a step's two ring slots (A and B; the same slot twice for a one-tile
// step) in one asm block that ends complete: K rows of both (A operand) and the
// transposed V rows of both (the lo and hi halves of the P.V operand).
template <int KS, int NSL>
struct step_reads2;
template <>
struct step_reads2<2, 4> {
  static __device__ __forceinline__ void run(const uint32_t (&ka)[4], const uint32_t (&va)[4], const uint32_t (&vb)[4],
                                             su32x4_t (&k)[4], su32x2_t (&lo)[4], su32x2_t (&hi)[4]) {
    asm volatile(
        "ds_read_b128 %0, %12\n\tds_read_b128 %1, %13\n\tds_read_b128 %2, %14\n\tds_read_b128 %3, %15\n\t"
        "ds_read_b64_tr_b16 %4, %16\n\tds_read_b64_tr_b16 %5, %17\n\t"
        "ds_read_b64_tr_b16 %6, %18\n\tds_read_b64_tr_b16 %7, %19\n\t"
        "ds_read_b64_tr_b16 %8, %20\n\tds_read_b64_tr_b16 %9, %21\n\t"
        "ds_read_b64_tr_b16 %10, %22\n\tds_read_b64_tr_b16 %11, %23\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(lo[0]), "=&v"(lo[1]), "=&v"(lo[2]), "=&v"(lo[3]),
          "=&v"(hi[0]), "=&v"(hi[1]), "=&v"(hi[2]), "=&v"(hi[3])
        : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]),
          "v"(vb[0]), "v"(vb[1]), "v"(vb[2]), "v"(vb[3])
        : "memory");
  }
};
template <>
struct step_reads2<4, 8> {
  static __device__ __forceinline__ void run(const uint32_t (&ka)[8], const uint32_t (&va)[8], const uint32_t (&vb)[8],
                                             su32x4_t (&k)[8], su32x2_t (&lo)[8], su32x2_t (&hi)[8]) {
    asm volatile(
        "ds_read_b128 %0, %24\n\tds_read_b128 %1, %25\n\tds_read_b128 %2, %26\n\tds_read_b128 %3, %27\n\t"
        "ds_read_b128 %4, %28\n\tds_read_b128 %5, %29\n\tds_read_b128 %6, %30\n\tds_read_b128 %7, %31\n\t"
        "ds_read_b64_tr_b16 %8, %32\n\tds_read_b64_tr_b16 %9, %33\n\t"
        "ds_read_b64_tr_b16 %10, %34\n\tds_read_b64_tr_b16 %11, %35\n\t"
        "ds_read_b64_tr_b16 %12, %36\n\tds_read_b64_tr_b16 %13, %37\n\t"
        "ds_read_b64_tr_b16 %14, %38\n\tds_read_b64_tr_b16 %15, %39\n\t"
        "ds_read_b64_tr_b16 %16, %40\n\tds_read_b64_tr_b16 %17, %41\n\t"
        "ds_read_b64_tr_b16 %18, %42\n\tds_read_b64_tr_b16 %19, %43\n\t"
        "ds_read_b64_tr_b16 %20, %44\n\tds_read_b64_tr_b16 %21, %45\n\t"
        "ds_read_b64_tr_b16 %22, %46\n\tds_read_b64_tr_b16 %23, %47\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]), "=&v"(k[6]), "=&v"(k[7]),
          "=&v"(lo[0]), "=&v"(lo[1]), "=&v"(lo[2]), "=&v"(lo[3]), "=&v"(lo[4]), "=&v"(lo[5]), "=&v"(lo[6]), "=&v"(lo[7]),
          "=&v"(hi[0]), "=&v"(hi[1]), "=&v"(hi[2]), "=&v"(hi[3]), "=&v"(hi[4]), "=&v"(hi[5]), "=&v"(hi[6]), "=&v"(hi[7])
        : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(ka[4]), "v"(ka[5]), "v"(ka[6]), "v"(ka[7]),
          "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "v"(va[4]), "v"(va[5]), "v"(va[6]), "v"(va[7]),
          "v"(vb[0]), "v"(vb[1]), "v"(vb[2]), "v"(vb[3]), "v"(vb[4]), "v"(vb[5]), "v"(vb[6]), "v"(vb[7])
        : "memory");
  }
};

}  // namespace tb
