// K2 for decode steps (one query row per sequence), fp16 / bf16.
//
// Replaces, for the decode rows of Qwen2Paged.forward (reference
// src/tinybatch/model.py:130-147), the per-sequence gather
// (kv_cache.py:40-45), repeat_interleave (model.py:135-137) and SDPA over the
// whole context (a decode row sees every position, model.py:142-146), with
// the fused append of the row's new K/V (kv_cache.py:25-38) when k_new is given.
//
// Decomposition (tb_build_decode_plan): a unit is one sequence's K/V rows of
// one kv head, cut into 16-position tiles. Units are packed onto the XCDs by
// tile count, each XCD's tiles are split evenly over the persistent
// workgroups that run on it (workgroup g on XCD g % num_xcds), and a
// workgroup's range is cut at unit boundaries into segments. Every workgroup
// therefore streams the same number of bytes, which keeps every CU's memory
// pipeline busy until the end of the launch (a one-shot grid of fixed work
// items left CUs idle while others still had data in flight).
//
// Inside a workgroup each wave takes a contiguous share of every segment and
// streams its tiles through a ring of RING tile slots in LDS, filled by direct
// global->LDS loads (no registers) issued RING tiles ahead of their use. A
// pair of tiles (32 positions) is one step:
//   S^T[pos][head] = K[pos][:] . Q[head][:]  v_mfma_f32_16x16x32, A = K rows (LDS),
//                                            B = q (registers, per segment)
//   O[head][d]   += P[head][pos] . V[pos][d] A = P (the S^T registers, repacked),
//                                            B = V rows (LDS transpose reads)
// with the online softmax state (max, sum, O) of every head kept per wave.
// At a segment's end the waves merge their states in LDS. A unit held whole by
// one segment writes its output; a unit cut into several segments leaves one
// partial (unnormalised O, max, sum) per segment, and the workgroup whose
// partial arrives last merges them all (log-sum-exp) and writes the output.
// All of a unit's partials are written and read inside one XCD, whose L2 every
// CU of the XCD shares: plain stores (acknowledged by the L2 before the arrival
// is counted) and L1-bypassing loads suffice, with no cache write-back. The
// arrival word of a unit counts pieces per XCD (8-bit fields), so a piece that
// ran on another XCD is detected and reported in `violations`. Without the
// XCD assumption (merge_in_kernel = 0) every partial is written and
// decode_combine_kernel merges them after the launch.
#include "tb_common.h"

namespace tb {

typedef _Float16 dhalf8_t __attribute__((ext_vector_type(8)));
typedef __bf16 dbf168_t __attribute__((ext_vector_type(8)));

template <typename Tag>
struct dmath;
template <>
struct dmath<f16_t> {
  typedef _Float16 scalar_t;
  typedef dhalf8_t vec8_t;
  static __device__ __forceinline__ float4_t mfma(vec8_t a, vec8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct dmath<bf16_t> {
  typedef __bf16 scalar_t;
  typedef dbf168_t vec8_t;
  static __device__ __forceinline__ float4_t mfma(vec8_t a, vec8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

struct decode_args {
  const char* q;            // [B][Hq][D]
  int64_t q_row_bytes;
  char* pool;               // [NB][2][Hkv][BS][D]
  int64_t num_blocks;
  char* out;                // [B][Hq*D]
  int64_t out_row_bytes;
  const int32_t* block_tables;
  int32_t max_nb;
  const int32_t* context_lens;   // [B]
  const int32_t* plan;      // tb_build_decode_plan layout
  char* pieces;             // partials: piece_bytes each
  uint32_t pieces_bytes;    // bytes addressable through the buffer resource
  int32_t piece_bytes;
  unsigned long long* arrivals;   // one per unit, 128 bytes apart, zero between launches (caller's buffer)
  uint32_t* violations;     // incremented when a unit's pieces ran on more than one XCD
  int32_t num_heads, num_kv_heads, rep;
  int32_t log2_bs;
  float scale_log2e;
  const char* k_new;        // fused append (may be null)
  int64_t k_new_row_bytes;
  const char* v_new;
  int64_t v_new_row_bytes;
  rope_tables rope;
  int32_t merge_in_kernel;
};

template <int D>
struct dshape {
  static constexpr int RB = 2 * D;             // bytes per K or V row
  static constexpr int TB = 16 * RB;           // bytes of a 16-position K (or V) tile
  static constexpr int VCOLS = RB / 16;        // 16-byte chunks per row
  static constexpr int TLD = TB / 1024;        // direct loads per tile, of K and of V each
  static constexpr int LPT = 2 * TLD;          // vector memory instructions per tile
  static constexpr int KS = D / 32;            // k-slices of q.k
  static constexpr int NSL = D / 16;           // 16-dim slices of O
  static constexpr int NW = 4;                 // waves per workgroup
  static constexpr int RING = D == 64 ? 6 : 3; // tile slots per wave (a step takes 2)
  static constexpr int TMAX = D == 64 ? 1024 : 2048;   // tiles per workgroup (block ids in LDS)
  static constexpr int SEGCAP = 64;            // segment records per workgroup
  static constexpr int QBYTES = D == 64 ? 32768 : 16384;   // q rows of the workgroup's segments
  static constexpr int HMAX = 8;               // query heads per kv head
  static constexpr int SLOT = 2 * TB;          // K tile then V tile
  static constexpr int RING_BYTES = NW * RING * SLOT;
  static constexpr int MERGE_BYTES = 2 * NW * HMAX * D * 4;   // two areas: segments alternate
  static constexpr int ML_BYTES = 2 * NW * 16 * 8;
  static constexpr int LDS = RING_BYTES + MERGE_BYTES + ML_BYTES + TMAX * 4 + SEGCAP * 20 + QBYTES;
  static_assert(LDS <= 160 * 1024, "LDS budget of a workgroup");
  static_assert(LPT * (RING - 1) <= 63, "vmcnt range");
  // K row r keeps its 16-byte chunk c in slot c ^ (r & 7): the A-operand reads
  // (16 rows x 16 bytes per 16 lanes) then cover every bank. V row r keeps c in
  // slot c ^ 2 (r & 3): the transpose reads (4 rows x 32 bytes per 16 lanes) too.
  static __device__ __forceinline__ int kswz(int r) { return r & 7; }
  static __device__ __forceinline__ int vswz(int r) { return 2 * (r & 3); }
};

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));

// The transpose reads of one step's V operand (both tiles, every 16-dim slice),
// issued together and complete when the block ends (lgkmcnt(0) inside it). As
// separate intrinsics each would wait for every direct global->LDS load of the
// wave in flight (the compiler cannot tell which ring slot a read depends on),
// which would drain the prefetch ring at every step; the ring's own waits
// (vmcnt) already cover the slots read here. Outputs are early-clobber.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}
// The A-operand reads of one step's K rows (both tiles, every k-slice), the same way.
typedef unsigned int u32x4_t_ __attribute__((ext_vector_type(4)));
template <int KS>
struct k_reads;
template <>
struct k_reads<2> {
  static __device__ __forceinline__ void run(const uint32_t (&ad)[4], u32x4_t_ (&k)[4]) {
    asm volatile(
        "ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3])
        : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3])
        : "memory");
  }
};
template <>
struct k_reads<4> {
  static __device__ __forceinline__ void run(const uint32_t (&ad)[8], u32x4_t_ (&k)[8]) {
    asm volatile(
        "ds_read_b128 %0, %8\n\tds_read_b128 %1, %9\n\tds_read_b128 %2, %10\n\tds_read_b128 %3, %11\n\t"
        "ds_read_b128 %4, %12\n\tds_read_b128 %5, %13\n\tds_read_b128 %6, %14\n\tds_read_b128 %7, %15\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]), "=&v"(k[6]), "=&v"(k[7])
        : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7])
        : "memory");
  }
};

template <int NSL>
struct v_reads;
template <>
struct v_reads<4> {
  static __device__ __forceinline__ void run(const uint32_t (&lo)[4], const uint32_t (&hi)[4], u32x2_t (&a)[4],
                                             u32x2_t (&b)[4]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %8\n\tds_read_b64_tr_b16 %1, %9\n\t"
        "ds_read_b64_tr_b16 %2, %10\n\tds_read_b64_tr_b16 %3, %11\n\t"
        "ds_read_b64_tr_b16 %4, %12\n\tds_read_b64_tr_b16 %5, %13\n\t"
        "ds_read_b64_tr_b16 %6, %14\n\tds_read_b64_tr_b16 %7, %15\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
        : "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(hi[0]), "v"(hi[1]), "v"(hi[2]), "v"(hi[3])
        : "memory");
  }
};
template <>
struct v_reads<8> {
  static __device__ __forceinline__ void run(const uint32_t (&lo)[8], const uint32_t (&hi)[8], u32x2_t (&a)[8],
                                             u32x2_t (&b)[8]) {
    asm volatile(
        "ds_read_b64_tr_b16 %0, %16\n\tds_read_b64_tr_b16 %1, %17\n\t"
        "ds_read_b64_tr_b16 %2, %18\n\tds_read_b64_tr_b16 %3, %19\n\t"
        "ds_read_b64_tr_b16 %4, %20\n\tds_read_b64_tr_b16 %5, %21\n\t"
        "ds_read_b64_tr_b16 %6, %22\n\tds_read_b64_tr_b16 %7, %23\n\t"
        "ds_read_b64_tr_b16 %8, %24\n\tds_read_b64_tr_b16 %9, %25\n\t"
        "ds_read_b64_tr_b16 %10, %26\n\tds_read_b64_tr_b16 %11, %27\n\t"
        "ds_read_b64_tr_b16 %12, %28\n\tds_read_b64_tr_b16 %13, %29\n\t"
        "ds_read_b64_tr_b16 %14, %30\n\tds_read_b64_tr_b16 %15, %31\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(a[4]), "=&v"(a[5]), "=&v"(a[6]), "=&v"(a[7]),
          "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]), "=&v"(b[6]), "=&v"(b[7])
        : "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(lo[4]), "v"(lo[5]), "v"(lo[6]), "v"(lo[7]),
          "v"(hi[0]), "v"(hi[1]), "v"(hi[2]), "v"(hi[3]), "v"(hi[4]), "v"(hi[5]), "v"(hi[6]), "v"(hi[7])
        : "memory");
  }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t pieces_rsrc(char* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(base, 0, bytes, 0x00020000);
}

// Wait until at most N vector memory instructions of this wave are outstanding
// (they complete in issue order).
template <int LPT>
__device__ __forceinline__ void wait_tiles_ahead(int ahead) {
  switch (ahead) {
    case 0: asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); break;
    case 1: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPT) : "memory"); break;
    case 2: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(2 * LPT) : "memory"); break;
    case 3: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * LPT) : "memory"); break;
    case 4: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(4 * LPT) : "memory"); break;
    default: asm volatile("s_waitcnt vmcnt(%0)" ::"n"(5 * LPT) : "memory"); break;
  }
}

// A unit's partials merged (log-sum-exp) by one wave and written as its output:
//   out = sum_k 2^(m_k - M) acc_k / sum_k 2^(m_k - M) l_k,  M = max_k m_k
// Piece layout: acc [rep][D] fp32, then (m, l) [rep] float2. Every lane owns up
// to CPL float4 columns; pieces are read in batches of 4 whose loads are all in
// flight. AUX is the load cache policy (1: L1 bypass, for partials that other
// CUs of this XCD wrote during this launch).
template <typename Tag, int D, int AUX>
__device__ __forceinline__ void merge_unit(const decode_args& a, int unit, int np, int base, int lane) {
  typedef typename dmath<Tag>::scalar_t scalar_t;
  constexpr int CPL = (dshape<D>::HMAX * D / 4 + 63) / 64;
  constexpr int BATCH = 4;
  const int b = unit / a.num_kv_heads, h = unit - b * a.num_kv_heads;
  const auto rs = pieces_rsrc(a.pieces, a.pieces_bytes);
  const int n4 = a.rep * D / 4;
  const uint32_t ml_off = (uint32_t)(a.rep * D * 4);
  float Mx[CPL], L[CPL];
  float4_t o[CPL];
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    Mx[q] = -INFINITY;
    L[q] = 0.f;
    o[q] = float4_t{0.f, 0.f, 0.f, 0.f};
  }
  for (int k0 = 0; k0 < np; k0 += BATCH) {
    float2 ml[BATCH][CPL];
    float4_t v[BATCH][CPL];
#pragma unroll
    for (int k = 0; k < BATCH; ++k)
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int c = lane + 64 * q;
        const int head = (4 * c) / D;
        if (k0 + k < np && c < n4) {
          const uint32_t p = (uint32_t)(base + k0 + k) * a.piece_bytes;
          ml[k][q] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, p + ml_off + 8 * head, 0, AUX));
          v[k][q] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, p + 16 * c, 0, AUX));
        } else {
          ml[k][q] = make_float2(-INFINITY, 0.f);
          v[k][q] = float4_t{0.f, 0.f, 0.f, 0.f};
        }
      }
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      float mb = Mx[q];
#pragma unroll
      for (int k = 0; k < BATCH; ++k) mb = fmaxf(mb, ml[k][q].x);
      const float keep = fast_exp2(Mx[q] - mb);   // 0 while Mx = -inf
      L[q] *= keep;
      o[q] *= keep;
#pragma unroll
      for (int k = 0; k < BATCH; ++k) {
        const float w = ml[k][q].y > 0.f ? fast_exp2(ml[k][q].x - mb) : 0.f;
        L[q] = fmaf(ml[k][q].y, w, L[q]);
        o[q] += v[k][q] * w;
      }
      Mx[q] = mb;
    }
  }
#pragma unroll
  for (int q = 0; q < CPL; ++q) {
    const int c = lane + 64 * q;
    if (c >= n4) continue;
    const float inv = 1.f / L[q];
    typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
    s4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = (scalar_t)(o[q][j] * inv);
    *reinterpret_cast<s4_t*>(a.out + b * a.out_row_bytes + ((int64_t)h * a.rep * D + 4 * c) * 2) = r;
  }
}

template <typename Tag, int D>
__global__ __launch_bounds__(64 * dshape<D>::NW) void paged_decode_kernel(const decode_args a) {
  using S = dshape<D>;
  using M = dmath<Tag>;
  typedef typename M::vec8_t vec8_t;
  typedef typename M::scalar_t scalar_t;
  constexpr int RB = S::RB, TB = S::TB, VCOLS = S::VCOLS, TLD = S::TLD, LPT = S::LPT, KS = S::KS;
  constexpr int NSL = S::NSL, NW = S::NW, RING = S::RING, SLOT = S::SLOT, HMAX = S::HMAX;
  // the ring (target of the direct loads) and the other areas are separate arrays, so the
  // compiler sees that reads of the latter do not depend on loads into the ring
  __shared__ __align__(16) char ring[S::RING_BYTES];
  __shared__ __align__(16) char lds[S::LDS - S::RING_BYTES];
  float* const acc_lds = reinterpret_cast<float*>(lds);                              // [2][NW][HMAX][D]
  float2* const ml_lds = reinterpret_cast<float2*>(lds + S::MERGE_BYTES);            // [2][NW][16]
  int32_t* const blk_lds = reinterpret_cast<int32_t*>(lds + S::MERGE_BYTES + S::ML_BYTES);
  int4* const seg_lds = reinterpret_cast<int4*>(blk_lds + S::TMAX);                 // (unit, t0, t1, slot)
  int32_t* const sctx_lds = reinterpret_cast<int32_t*>(seg_lds + S::SEGCAP);         // the segment's context
  char* const q_lds = reinterpret_cast<char*>(sctx_lds + S::SEGCAP);                 // [segment][rep][D]

  // wave-uniform values (the wave index, the segment records and everything derived
  // from them) are made scalar, so the loop control and the waits stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int G = a.plan[0];
  const int32_t* const wg_first = a.plan + 8;
  const int4* const segs = reinterpret_cast<const int4*>(wg_first + (G + 1 + 3) / 4 * 4);
  if ((int)blockIdx.x >= G) return;              // a grid larger than the plan's
  const int s0 = wg_first[blockIdx.x], s1 = wg_first[blockIdx.x + 1];
  const int nseg = s1 - s0;
  const int rep = a.rep;
  // the plan builder keeps every workgroup within its LDS areas; a plan that does not
  // is not served (nothing is read or written)
  if (nseg <= 0 || nseg > S::SEGCAP || nseg * rep * RB > S::QBYTES) return;
  const int32_t* const unit_rec = reinterpret_cast<const int32_t*>(segs + a.plan[1]);   // after S segments

  // ---- segments, their contexts and q rows, and the block id of every tile, into LDS ----
  for (int i = threadIdx.x; i < nseg; i += 64 * NW) {
    const int4 sg = segs[s0 + i];
    seg_lds[i] = sg;
    sctx_lds[i] = a.context_lens[sg.x / a.num_kv_heads];
  }
  {
    constexpr int C16 = RB / 16;               // 16-byte chunks of a head row
    const int per_seg = rep * C16;
    for (int f = threadIdx.x; f < nseg * per_seg; f += 64 * NW) {
      const int i = f / per_seg, w = f - i * per_seg;
      const int u = segs[s0 + i].x;
      const int b = u / a.num_kv_heads, h = u - b * a.num_kv_heads;
      const vec16 x = ld16(a.q + b * a.q_row_bytes + (int64_t)h * rep * RB + 16 * w);
      *reinterpret_cast<vec16*>(q_lds + (int64_t)i * rep * RB + 16 * w) = x;
    }
  }
  __syncthreads();
  auto seg_at = [&](int i) {                     // segment record i, wave-uniform
    const int4 v = seg_lds[i];
    return make_int4(__builtin_amdgcn_readfirstlane(v.x), __builtin_amdgcn_readfirstlane(v.y),
                     __builtin_amdgcn_readfirstlane(v.z), __builtin_amdgcn_readfirstlane(v.w));
  };
  auto seg_len = [&](int i) {
    const int4 v = seg_lds[i];
    return __builtin_amdgcn_readfirstlane(v.z - v.y);
  };
  int range = 0;                                 // tiles of the workgroup
  for (int i = 0; i < nseg; ++i) range += seg_len(i);
  if (range > S::TMAX) return;                   // uniform: every thread read the same records
  const int bs = 1 << a.log2_bs;
  for (int j = threadIdx.x; j < range; j += 64 * NW) {
    int i = 0, off = j;
    while (off >= seg_lds[i].z - seg_lds[i].y) {
      off -= seg_lds[i].z - seg_lds[i].y;
      ++i;
    }
    const int u = seg_lds[i].x, t = seg_lds[i].y + off;
    const int b = u / a.num_kv_heads;
    int blk = a.block_tables[(int64_t)b * a.max_nb + ((16 * t) >> a.log2_bs)];
    if (blk < 0 || blk >= a.num_blocks) blk = 0;   // the host validates tables; stay inside the pool
    blk_lds[j] = blk;
  }
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  xcc &= 7;                                      // arrival fields: 8 XCDs of 8 bits
  __syncthreads();

  const int64_t tile_bytes = (int64_t)bs * RB;                 // one kv head's K (or V) rows of a block
  const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * tile_bytes;
  const int64_t v_off = (int64_t)a.num_kv_heads * tile_bytes;
  const bool fused = a.k_new != nullptr;
  char* const my_ring = ring + wave * RING * SLOT;

  // This wave's share of segment i: tiles [lo, hi) of the segment, a contiguous NW-th;
  // `base` is the segment's first tile in the workgroup's range.
  auto share = [&](int i, int& lo, int& hi, int& base) {
    base = 0;
    for (int k = 0; k < i; ++k) base += seg_len(k);
    const int n = seg_len(i);
    lo = n * wave / NW;
    hi = n * (wave + 1) / NW;
  };

  // ---- loads: the wave's tiles in order, RING slots ahead ----
  int ls = 0, lt = 0, lhi = 0, lbase = 0;        // load cursor: segment, tile (segment-relative), end, base
  share(0, lt, lhi, lbase);
  auto advance_load = [&]() {
    while (ls < nseg && lt >= lhi) {
      ++ls;
      if (ls < nseg) share(ls, lt, lhi, lbase);
    }
  };
  advance_load();
  int issued = 0, islot = 0;                     // tiles issued; the slot the next one fills
  auto issue_next = [&]() {
    if (ls >= nseg) return;
    const int4 sg = seg_at(ls);
    const int u = sg.x, t = sg.y + lt;
    const int b = u / a.num_kv_heads, h = u - b * a.num_kv_heads;
    const int ctx = __builtin_amdgcn_readfirstlane(sctx_lds[ls]);
    const int blk = __builtin_amdgcn_readfirstlane(blk_lds[lbase + lt]);
    const int p0 = 16 * t;
    const char* kbase = a.pool + (int64_t)blk * blk_bytes + (int64_t)h * tile_bytes + (int64_t)(p0 & (bs - 1)) * RB;
    const char* kn = fused ? a.k_new + b * a.k_new_row_bytes + (int64_t)h * RB : nullptr;
    const char* vn = fused ? a.v_new + b * a.v_new_row_bytes + (int64_t)h * RB : nullptr;
    char* const dst = my_ring + islot * SLOT;
#pragma unroll
    for (int j = 0; j < TLD; ++j) {
      const int f = 64 * j + lane;                // 16-byte slot of the tile
      const int r = f / VCOLS, cs = f % VCOLS;
      int p = p0 + r;
      if (p >= ctx) p = ctx - 1;                  // rows past the context read a valid row (masked)
      const int rr = p - p0;
      const bool newest = fused && p == ctx - 1;
      const int ck = cs ^ S::kswz(r), cv = cs ^ S::vswz(r);
      const char* ks = newest ? kn + 16 * ck : kbase + rr * RB + 16 * ck;
      const char* vs = newest ? vn + 16 * cv : kbase + v_off + rr * RB + 16 * cv;
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)ks,
                                       (__attribute__((address_space(3))) void*)(dst + 1024 * j), 16, 0, 2);
      __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)vs,
                                       (__attribute__((address_space(3))) void*)(dst + TB + 1024 * j), 16, 0, 2);
    }
    ++issued;
    islot = islot + 1 == RING ? 0 : islot + 1;
    ++lt;
    advance_load();
  };
  for (int r = 0; r < RING; ++r) issue_next();

  // ---- consume ----
  int consumed = 0, cslot = 0;                   // tiles consumed; the slot of the next one
  for (int i = 0; i < nseg; ++i) {
    const int4 sg = seg_at(i);
    const int u = sg.x;
    const int b = u / a.num_kv_heads, h = u - b * a.num_kv_heads;
    const int ctx = __builtin_amdgcn_readfirstlane(sctx_lds[i]);
    const int head0 = h * rep;
    const int newest = ctx - 1;
    int lo, hi, sbase;
    share(i, lo, hi, sbase);
    const int n = hi - lo;                        // this wave's tiles of the segment
    // q (B operand): lane (lc, lg) holds q[b][head0 + lc][32 s + 8 lg .. + 8]; heads past rep are 0
    vec16 qb[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = zero16();
    if (lc < rep && n > 0) {
      const char* qrow = q_lds + ((int64_t)i * rep + lc) * RB + 16 * lg;
#pragma unroll
      for (int s = 0; s < KS; ++s) qb[s] = *reinterpret_cast<const vec16*>(qrow + 64 * s);
      if (a.rope.cos) {   // slice s (dims 32 s + 8 lg ..) pairs with slice s + KS/2
        const int64_t rr = a.rope.row(newest, D / 2) + 8 * lg;
#pragma unroll
        for (int s = 0; s < KS / 2; ++s)
          rope_pair<scalar_t>(qb[s], qb[s + KS / 2], a.rope.cos + rr + 32 * s, a.rope.sin + rr + 32 * s);
      }
    }
    float m_run = -INFINITY;     // max of head lc (base-2 domain)
    float l_part = 0.f;          // this lane's share of head lc's sum
    float4_t acc[NSL];           // O[head 4 lg + j][16 nn + lc]
#pragma unroll
    for (int nn = 0; nn < NSL; ++nn) acc[nn] = float4_t{0.f, 0.f, 0.f, 0.f};

    for (int k = 0; k < n; k += 2) {
      const bool two = k + 1 < n;
      wait_tiles_ahead<LPT>(issued - consumed - (two ? 2 : 1));   // this step's tiles have landed
      const int ia = sbase + lo + k;              // the step's first tile in the range
      const int cslot2 = cslot + 1 == RING ? 0 : cslot + 1;
      const char* ta = my_ring + cslot * SLOT;
      const char* tb2 = two ? my_ring + cslot2 * SLOT : ta;
      const int pa0 = 16 * (sg.y + lo + k), pb0 = pa0 + 16;
      // fused append: the unit's newest row was loaded from k_new / v_new; with RoPE its K
      // is rotated in place before the scores read it; either way it goes to its pool slot
      if (fused) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
          const int pt0 = tt == 0 ? pa0 : pb0;
          if ((tt == 0 || two) && newest >= pt0 && newest < pt0 + 16) {   // wave-uniform
            char* kt = const_cast<char*>(tt == 0 ? ta : tb2);
            const int r = newest - pt0;
            if (a.rope.cos && lane < VCOLS / 2) {
              char* c1 = kt + r * RB + 16 * (lane ^ S::kswz(r));
              char* c2 = kt + r * RB + 16 * ((lane + VCOLS / 2) ^ S::kswz(r));
              vec16 x1 = *reinterpret_cast<vec16*>(c1), x2 = *reinterpret_cast<vec16*>(c2);
              const int64_t rr = a.rope.row(newest, D / 2) + 8 * lane;
              rope_pair<scalar_t>(x1, x2, a.rope.cos + rr, a.rope.sin + rr);
              *reinterpret_cast<vec16*>(c1) = x1;
              *reinterpret_cast<vec16*>(c2) = x2;
            }
            if (lane < 2 * VCOLS) {   // LDS accesses of a wave run in order: the rotated row is read
              const int c = lane % VCOLS;
              const bool is_v = lane >= VCOLS;
              const vec16 x = *reinterpret_cast<const vec16*>(
                  kt + (is_v ? TB : 0) + r * RB + 16 * (c ^ (is_v ? S::vswz(r) : S::kswz(r))));
              const int nblk = __builtin_amdgcn_readfirstlane(blk_lds[ia + tt]);   // a tile lies in one block
              char* dst = a.pool + (int64_t)nblk * blk_bytes + (int64_t)h * tile_bytes + (is_v ? v_off : 0) +
                          (int64_t)(newest & (bs - 1)) * RB + 16 * c;
              st16(dst, x);
            }
          }
        }
      }
      // S^T for both tiles (A = K rows from LDS)
      uint32_t kad[2 * KS];
      u32x4_t_ kv[2 * KS];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt)
#pragma unroll
        for (int s = 0; s < KS; ++s)
          kad[tt * KS + s] = lds_addr((tt == 0 ? ta : tb2) + lc * RB + 16 * ((4 * s + lg) ^ S::kswz(lc)));
      k_reads<KS>::run(kad, kv);
      float4_t sc[2];
#pragma unroll
      for (int tt = 0; tt < 2; ++tt) {
        sc[tt] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < KS; ++s)
          sc[tt] = M::mfma(__builtin_bit_cast(vec8_t, kv[tt * KS + s]), __builtin_bit_cast(vec8_t, qb[s]), sc[tt]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[0][j] = (pa0 + 4 * lg + j) < ctx ? sc[0][j] * a.scale_log2e : -INFINITY;
        sc[1][j] = (two && (pb0 + 4 * lg + j) < ctx) ? sc[1][j] * a.scale_log2e : -INFINITY;
      }
      float cm = max3_f32(max_f32(sc[0][0], sc[0][1]), sc[0][2], sc[0][3]);
      cm = max3_f32(cm, max_f32(sc[1][0], sc[1][1]), max_f32(sc[1][2], sc[1][3]));
      cm = max_xor32(max_xor16(cm));             // max of head lc over the step's positions (finite)
      const float m_new = fmaxf(m_run, cm);
      const float alpha = fast_exp2(m_run - m_new);   // 0 while m_run = -inf
      m_run = m_new;
      l_part *= alpha;
      // the O rows of this lane are heads 4 lg + j, whose factors sit in lanes 4 lg + j
      float al[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) al[j] = __shfl(alpha, 4 * lg + j);
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[nn][j] *= al[j];
      vec8_t pa;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float p0v = fast_exp2(sc[0][j] - m_new), p1v = fast_exp2(sc[1][j] - m_new);
        l_part += p0v + p1v;
        pa[j] = (scalar_t)p0v;
        pa[4 + j] = (scalar_t)p1v;
      }
      // O += P.V: k index 8 lg + j <-> row 4 lg + j of tile a (j < 4) or of tile b (j >= 4)
      const int rv = 4 * lg + (lc >> 2);
      const int half8 = 8 * (lc & 1);
      uint32_t alo[NSL], ahi[NSL];
      u32x2_t vlo[NSL], vhi[NSL];
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) {
        const int c = ((lc & 3) >> 1) + 2 * nn;
        const int off = TB + rv * RB + 16 * (c ^ S::vswz(rv)) + half8;
        alo[nn] = lds_addr(ta + off);
        ahi[nn] = lds_addr(tb2 + off);
      }
      v_reads<NSL>::run(alo, ahi, vlo, vhi);
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) {
        vec16 vb;
        vb.w[0] = vlo[nn].x; vb.w[1] = vlo[nn].y; vb.w[2] = vhi[nn].x; vb.w[3] = vhi[nn].y;
        acc[nn] = M::mfma(pa, __builtin_bit_cast(vec8_t, vb), acc[nn]);
      }
      // the step's slots are read (the LDS reads have returned): refill them
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      consumed += two ? 2 : 1;
      cslot = two ? (cslot2 + 1 == RING ? 0 : cslot2 + 1) : cslot2;
      issue_next();
      if (two) issue_next();
    }

    // ---- the waves' states of this segment, merged in LDS (area i % 2) ----
    float2* const mlb = ml_lds + (i & 1) * NW * 16;
    float* const accb = acc_lds + (i & 1) * NW * HMAX * D;
    float l_w = l_part + __shfl_xor(l_part, 16);
    l_w += __shfl_xor(l_w, 32);
    if (lg == 0) mlb[wave * 16 + lc] = make_float2(m_run, l_w);
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int hh = 4 * lg + j;
      if (hh >= rep) continue;
      float Mh = mlb[hh].x;
#pragma unroll
      for (int w = 1; w < NW; ++w) Mh = fmaxf(Mh, mlb[w * 16 + hh].x);
      const float mw = mlb[wave * 16 + hh].x;
      const float f = mw != -INFINITY ? fast_exp2(mw - Mh) : 0.f;
      float* dst = accb + (wave * HMAX + hh) * D + lc;
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) dst[16 * nn] = acc[nn][j] * f;
    }
    __syncthreads();
    // wave 0 finishes the segment: output, or a partial and the unit's arrival
    if (wave == 0) {
      const int slot = sg.w;
      const auto rs = pieces_rsrc(a.pieces, a.pieces_bytes);
      for (int idx = lane; idx < rep * D; idx += 64) {
        const int hh = idx / D, d = idx - hh * D;
        float Mh = mlb[hh].x;
#pragma unroll
        for (int w = 1; w < NW; ++w) Mh = fmaxf(Mh, mlb[w * 16 + hh].x);
        float L = 0.f, o = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
          const float2 ml = mlb[w * 16 + hh];
          if (ml.y > 0.f) L = fmaf(ml.y, fast_exp2(ml.x - Mh), L);   // idle waves hold (-inf, 0)
          o += accb[(w * HMAX + hh) * D + d];
        }
        if (slot < 0) {
          reinterpret_cast<scalar_t*>(a.out + b * a.out_row_bytes)[(int64_t)(head0 + hh) * D + d] = (scalar_t)(o / L);
        } else {
          const uint32_t p = (uint32_t)slot * a.piece_bytes;
          __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), rs, p + 4 * idx, 0, 0);
          if (d == 0)
            __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, make_float2(Mh, L)), rs,
                                                  p + rep * D * 4 + 8 * hh, 0, 0);
        }
      }
      if (slot >= 0 && a.merge_in_kernel) {
        // the partial is in this XCD's L2 (its stores acknowledged) before the arrival counts it
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        const int np = unit_rec[2 * u], pbase = unit_rec[2 * u + 1];
        const unsigned long long mine = 1ull << (8 * xcc);
        unsigned long long prev = 0;
        if (lane == 0)
          prev = __hip_atomic_fetch_add(a.arrivals + 16 * (int64_t)u, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        prev = __shfl(prev, 0);
        const unsigned long long now = prev + mine;
        int arrived = 0;
#pragma unroll
        for (int x = 0; x < 8; ++x) arrived += (int)((now >> (8 * x)) & 0xFF);
        if (arrived == np) {                       // the last piece: merge them all
          if (now != ((unsigned long long)np << (8 * xcc)) && lane == 0)
            __hip_atomic_fetch_add(a.violations, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          merge_unit<Tag, D, 1>(a, u, np, pbase, lane);
          if (lane == 0)
            __hip_atomic_store(a.arrivals + 16 * (int64_t)u, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      }
    }
  }
}

// Partials merged after the launch (merge_in_kernel = 0): one wave per split unit.
template <typename Tag, int D>
__global__ __launch_bounds__(64) void decode_combine_kernel(const decode_args a) {
  const int u = blockIdx.x;
  const int G = a.plan[0];
  const int32_t* const wg_first = a.plan + 8;
  const int32_t* const unit_rec = wg_first + (G + 1 + 3) / 4 * 4 + 4 * a.plan[1];
  if (u >= a.plan[2]) return;                     // grids may be sized for a capacity
  const int np = unit_rec[2 * u], pbase = unit_rec[2 * u + 1];
  if (np <= 1) return;
  merge_unit<Tag, D, 0>(a, u, np, pbase, threadIdx.x);
}

template <typename Tag, int D>
static void launch_decode(const decode_args& a, int wgs, int units, hipStream_t stream) {
  hipLaunchKernelGGL((paged_decode_kernel<Tag, D>), dim3(wgs), dim3(64 * dshape<D>::NW), 0, stream, a);
  if (!a.merge_in_kernel && units > 0)
    hipLaunchKernelGGL((decode_combine_kernel<Tag, D>), dim3(units), dim3(64), 0, stream, a);
}

__global__ void xcc_probe_kernel(int32_t* out) {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)(x & 0xF);
}

}  // namespace tb

extern "C" int32_t tb_decode_limits(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t* max_tiles_per_wg, int32_t* max_segments_per_wg,
                                    int32_t* waves_per_wg) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return TB_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return TB_ERR_UNSUPPORTED;
  const int rep = num_heads / num_kv_heads;
  if (rep > tb::dshape<64>::HMAX) return TB_ERR_UNSUPPORTED;
  const bool d64 = head_dim == 64;
  const int tmax = d64 ? tb::dshape<64>::TMAX : tb::dshape<128>::TMAX;
  const int segcap = d64 ? tb::dshape<64>::SEGCAP : tb::dshape<128>::SEGCAP;
  const int qbytes = d64 ? tb::dshape<64>::QBYTES : tb::dshape<128>::QBYTES;
  const int by_q = qbytes / (rep * 2 * head_dim);
  if (max_tiles_per_wg) *max_tiles_per_wg = tmax;
  if (max_segments_per_wg) *max_segments_per_wg = by_q < segcap ? by_q : segcap;
  if (waves_per_wg) *waves_per_wg = d64 ? tb::dshape<64>::NW : tb::dshape<128>::NW;
  return TB_OK;
}

extern "C" size_t tb_paged_decode_piece_bytes(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim) {
  if (num_heads <= 0 || num_kv_heads <= 0 || head_dim <= 0 || num_heads % num_kv_heads) return 0;
  const size_t rep = (size_t)(num_heads / num_kv_heads);
  return (rep * head_dim * 4 + rep * 8 + 127) / 128 * 128;
}

extern "C" size_t tb_paged_decode_workspace_bytes(int32_t max_pieces, int32_t num_heads, int32_t num_kv_heads,
                                                  int32_t head_dim) {
  if (max_pieces < 0) return 0;
  return (size_t)max_pieces * tb_paged_decode_piece_bytes(num_heads, num_kv_heads, head_dim);
}

extern "C" int32_t tb_decode_xcc_probe(int32_t workgroups, int32_t* out, hipStream_t stream) {
  if (workgroups <= 0 || !out) return TB_ERR_INVALID_ARG;
  hipLaunchKernelGGL(tb::xcc_probe_kernel, dim3(workgroups), dim3(64), 0, stream, out);
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_paged_decode(const void* q, int64_t q_row_stride, void* pool, int64_t num_blocks, void* out,
                                   int64_t out_row_stride, const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int32_t* context_lens, int32_t num_seqs, const int32_t* plan,
                                   int32_t plan_workgroups, int32_t max_units, int32_t num_heads,
                                   int32_t num_kv_heads, int32_t head_dim, int32_t block_size, float scale,
                                   int32_t dtype, const void* k_new, int64_t k_row_stride, const void* v_new,
                                   int64_t v_row_stride, void* workspace, size_t workspace_bytes,
                                   int32_t max_pieces, unsigned long long* arrivals, int32_t arrival_units,
                                   int32_t merge_in_kernel, uint32_t* violations,
                                   const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                                   hipStream_t stream) {
  using namespace tb;
  if (dtype != TB_DTYPE_F16 && dtype != TB_DTYPE_BF16) return TB_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0);
  const int rep = num_heads / num_kv_heads;
  if (rep > dshape<64>::HMAX) return TB_ERR_UNSUPPORTED;
  if (block_size < 16 || (block_size & (block_size - 1))) return TB_ERR_UNSUPPORTED;
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  TB_CHECK_ARG(num_seqs >= 0 && plan_workgroups > 0 && max_units >= num_seqs * num_kv_heads && max_pieces >= 0);
  if (num_seqs == 0) return TB_OK;
  TB_CHECK_ARG(q && pool && out && block_tables && context_lens && plan && max_blocks_per_seq > 0 && num_blocks > 0);
  TB_CHECK_ARG((((uintptr_t)q | (uintptr_t)pool | (uintptr_t)out) & 15u) == 0);
  TB_CHECK_ARG(q_row_stride >= (int64_t)num_heads * head_dim && out_row_stride >= (int64_t)num_heads * head_dim);
  TB_CHECK_ARG((q_row_stride * 2) % 16 == 0 && (out_row_stride * 2) % 16 == 0);
  const size_t piece = tb_paged_decode_piece_bytes(num_heads, num_kv_heads, head_dim);
  const size_t need = tb_paged_decode_workspace_bytes(max_pieces, num_heads, num_kv_heads, head_dim);
  TB_CHECK_ARG(max_pieces == 0 || (workspace != nullptr && workspace_bytes >= need));
  TB_CHECK_ARG((((uintptr_t)workspace) & 127u) == 0);
  TB_CHECK_ARG((size_t)max_pieces * piece < ((size_t)1 << 31));
  if (merge_in_kernel) {
    TB_CHECK_ARG(violations != nullptr && arrivals != nullptr && arrival_units >= max_units);
    TB_CHECK_ARG((((uintptr_t)arrivals) & 127u) == 0);
  }
  if (rope_cos || rope_sin) {
    TB_CHECK_ARG(rope_cos && rope_sin && rope_max_position > 0);
    TB_CHECK_ARG((((uintptr_t)rope_cos | (uintptr_t)rope_sin) & 15u) == 0);
  }
  if (k_new || v_new) {
    TB_CHECK_ARG(k_new && v_new);
    TB_CHECK_ARG(k_row_stride >= (int64_t)num_kv_heads * head_dim && v_row_stride >= (int64_t)num_kv_heads * head_dim);
    TB_CHECK_ARG((((uintptr_t)k_new | (uintptr_t)v_new) & 15u) == 0);
    TB_CHECK_ARG((k_row_stride * 2) % 16 == 0 && (v_row_stride * 2) % 16 == 0);
  }
  decode_args a;
  a.q = (const char*)q;
  a.q_row_bytes = q_row_stride * 2;
  a.pool = (char*)pool;
  a.num_blocks = num_blocks;
  a.out = (char*)out;
  a.out_row_bytes = out_row_stride * 2;
  a.block_tables = block_tables;
  a.max_nb = max_blocks_per_seq;
  a.context_lens = context_lens;
  a.plan = plan;
  a.pieces = (char*)workspace;
  a.pieces_bytes = (uint32_t)((size_t)max_pieces * piece);
  a.piece_bytes = (int32_t)piece;
  a.arrivals = arrivals;
  a.violations = violations;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.rep = rep;
  a.log2_bs = log2_bs;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.k_new = (const char*)k_new;
  a.k_new_row_bytes = k_row_stride * 2;
  a.v_new = (const char*)v_new;
  a.v_new_row_bytes = v_row_stride * 2;
  a.rope = rope_tables{rope_cos, rope_sin, rope_max_position};
  a.merge_in_kernel = merge_in_kernel;
  const int units = max_units;
  if (dtype == TB_DTYPE_F16) {
    head_dim == 64 ? launch_decode<f16_t, 64>(a, plan_workgroups, units, stream)
                   : launch_decode<f16_t, 128>(a, plan_workgroups, units, stream);
  } else {
    head_dim == 64 ? launch_decode<bf16_t, 64>(a, plan_workgroups, units, stream)
                   : launch_decode<bf16_t, 128>(a, plan_workgroups, units, stream);
  }
  TB_RETURN_LAUNCH_STATUS();
}
