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
// tile count; each XCD's tiles are split evenly over the waves (workers) of the
// persistent workgroups that run on it (workgroup g on XCD g % num_xcds), and
// a worker's range is cut at unit boundaries into segments. Every wave
// therefore streams the same number of bytes, which keeps every CU's memory
// pipeline busy until the end of the launch, and the waves of a workgroup never
// wait for each other: a workgroup is only the container that gives its four
// waves (one per SIMD) a quarter of the CU's LDS each.
//
// The plan carries each worker's segments (with their context lengths) and the
// pool block of every tile it streams, so a wave issues its first tile loads
// after two dependent reads (its worker record, then its segments and blocks).
// Its q rows (and RoPE rows) are loaded into registers before the tile loads
// and written to LDS after them: the wait for them leaves the tiles in flight.
//
// A wave streams its tiles through a ring of RING tile slots in its LDS area,
// filled by direct global->LDS loads issued RING tiles ahead of their use. A
// pair of tiles (32 positions) is one step:
//   S^T[pos][head] = K[pos][:] . Q[head][:]  v_mfma_f32_16x16x32, A = K rows (LDS),
//                                            B = q (registers, per segment)
//   O[head][d]   += P[head][pos] . V[pos][d] A = P (the S^T registers, repacked),
//                                            B = V rows (LDS transpose reads)
// with the online softmax state (max, sum, O) of every head kept in registers.
// The ring is the only target of direct loads and every read of it is an asm
// block, so the compiler inserts no wait for direct loads anywhere; the waits
// for ring slots are explicit and exact: the wave counts every vector memory
// instruction it issues (tile loads and stores alike, which complete in issue
// order) and waits until at most the number issued after a step's last tile
// are outstanding.
//
// A unit held whole by one segment writes its output (staged in LDS for
// 16-byte stores). A unit cut into several segments leaves one partial
// (unnormalised O, max, sum) per segment; after its last tile each wave waits
// for its stores, counts its partials in the units' arrival words, and the
// wave whose partial arrives last merges them all (log-sum-exp) and writes the
// output. All of a unit's partials are written and read inside one XCD, whose
// L2 every CU of the XCD shares: plain stores (acknowledged by the L2 before the
// arrival is counted) and L1-bypassing loads suffice, with no cache write-back.
// The arrival word of a unit counts pieces per XCD (8-bit fields), so a piece
// that ran on another XCD is detected and reported in `violations`. Without the
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
  // waves (workers) per workgroup: two per SIMD where their rings fit (one wave's
  // step computes while the other's tiles land), else one
  static constexpr int NW = D == 64 ? 8 : 4;
  static constexpr int RING = 3;               // tile slots per wave (a step takes 2)
  static constexpr int SLOT = 2 * TB;          // K tile then V tile
  static constexpr int SEGW = D == 64 ? 3 : 8;            // segments per worker
  static constexpr int TMAXW = D == 64 ? 256 : 512;       // tiles per worker (their blocks in LDS)
  static constexpr int QW = D == 64 ? 4096 : 8192;        // q rows of a worker's segments (and output staging)
  static constexpr int HMAX = 8;               // query heads per kv head
  static constexpr int QI = QW / 1024;         // 16-byte q loads per lane
  // cos | sin rows (fp32) per segment, in whole 1 KiB direct loads (64 lanes x 16 bytes)
  static constexpr int ROPE_W = (SEGW * D * 4 + 1023) / 1024 * 1024;
  static constexpr int OUTI = HMAX * RB / 1024;    // 16-byte output stores per lane and unit
  static constexpr int RING_BYTES = NW * RING * SLOT;
  static constexpr int LDS = RING_BYTES + NW * (QW + ROPE_W + SEGW * 32 + TMAXW * 4);
  static_assert(QW % 1024 == 0, "q area in whole direct loads");
  static_assert(LDS <= 160 * 1024, "LDS budget of a workgroup");
  static_assert(LPT * RING <= 63, "vmcnt range");
  // K row r keeps its 16-byte chunk c in slot c ^ (r & 7): the A-operand reads
  // (16 rows x 16 bytes per 16 lanes) then cover every bank. V row r keeps c in
  // slot c ^ 2 (r & 3): the transpose reads (4 rows x 32 bytes per 16 lanes) too.
  static __device__ __forceinline__ int kswz(int r) { return r & 7; }
  static __device__ __forceinline__ int vswz(int r) { return 2 * (r & 3); }
};

typedef unsigned int u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned int u32x4_t_ __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// The reads of one step's two ring slots, one asm block complete when it ends
// (lgkmcnt(0) inside, early-clobber outputs): the A-operand reads of the K rows
// (both tiles, every k-slice) and the transpose reads of the V operand (both
// tiles, every 16-dim slice). As compiler-visible LDS reads each would wait for
// every direct global->LDS load of the wave in flight (the compiler cannot tell
// which ring slot a read depends on), which would drain the prefetch ring; the
// ring's own waits (vmcnt) already cover the slots read here. Once the block
// ends, the slots can be refilled.
template <int KS, int NSL>
struct step_reads;
template <>
struct step_reads<2, 4> {
  static __device__ __forceinline__ void run(const uint32_t (&ad)[4], const uint32_t (&lo)[4], const uint32_t (&hi)[4],
                                             u32x4_t_ (&k)[4], u32x2_t (&a)[4], u32x2_t (&b)[4]) {
    asm volatile(
        "ds_read_b128 %0, %12\n\tds_read_b128 %1, %13\n\tds_read_b128 %2, %14\n\tds_read_b128 %3, %15\n\t"
        "ds_read_b64_tr_b16 %4, %16\n\tds_read_b64_tr_b16 %5, %17\n\t"
        "ds_read_b64_tr_b16 %6, %18\n\tds_read_b64_tr_b16 %7, %19\n\t"
        "ds_read_b64_tr_b16 %8, %20\n\tds_read_b64_tr_b16 %9, %21\n\t"
        "ds_read_b64_tr_b16 %10, %22\n\tds_read_b64_tr_b16 %11, %23\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]),
          "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3])
        : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]),
          "v"(hi[0]), "v"(hi[1]), "v"(hi[2]), "v"(hi[3])
        : "memory");
  }
};
template <>
struct step_reads<4, 8> {
  static __device__ __forceinline__ void run(const uint32_t (&ad)[8], const uint32_t (&lo)[8], const uint32_t (&hi)[8],
                                             u32x4_t_ (&k)[8], u32x2_t (&a)[8], u32x2_t (&b)[8]) {
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
          "=&v"(a[0]), "=&v"(a[1]), "=&v"(a[2]), "=&v"(a[3]), "=&v"(a[4]), "=&v"(a[5]), "=&v"(a[6]), "=&v"(a[7]),
          "=&v"(b[0]), "=&v"(b[1]), "=&v"(b[2]), "=&v"(b[3]), "=&v"(b[4]), "=&v"(b[5]), "=&v"(b[6]), "=&v"(b[7])
        : "v"(ad[0]), "v"(ad[1]), "v"(ad[2]), "v"(ad[3]), "v"(ad[4]), "v"(ad[5]), "v"(ad[6]), "v"(ad[7]),
          "v"(lo[0]), "v"(lo[1]), "v"(lo[2]), "v"(lo[3]), "v"(lo[4]), "v"(lo[5]), "v"(lo[6]), "v"(lo[7]),
          "v"(hi[0]), "v"(hi[1]), "v"(hi[2]), "v"(hi[3]), "v"(hi[4]), "v"(hi[5]), "v"(hi[6]), "v"(hi[7])
        : "memory");
  }
};

// One 16-byte ring read and one 16-byte ring write (the newest row of a unit).
__device__ __forceinline__ u32x4_t_ ring_read16(const void* p) {
  u32x4_t_ r;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=&v"(r) : "v"(lds_addr(p)) : "memory");
  return r;
}
__device__ __forceinline__ void ring_write16(void* p, u32x4_t_ x) {
  asm volatile("ds_write_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(lds_addr(p)), "v"(x) : "memory");
}

// One direct global->LDS load of a wave: lane l's 16 bytes at src go to lds_dst + 16 l
// (lds_dst wave-uniform; M0 holds it). Issued as asm so that the compiler, which
// cannot tell which LDS a direct load writes, sees none and never makes an LDS
// access wait for one; every wait for these loads is explicit (vm_wait_le). The
// s_nop is the wait state an M0 write needs before a direct load.
__device__ __forceinline__ void dma16(const void* src, const void* lds_dst) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off nt" ::"v"(src), "{m0}"(lds_addr(lds_dst)) : "memory");
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t raw_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
// A lane's offset that the buffer range check drops (every resource here covers < 2^31 bytes).
constexpr uint32_t OOB = 0x80000000u;

// Wait until at most n vector memory instructions of this wave are outstanding
// (they complete in issue order); n is wave-uniform, the immediate is chosen by
// a scalar binary search.
template <int LO, int HI>
__device__ __forceinline__ void vm_wait_range(int n) {
  if constexpr (LO == HI) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LO) : "memory");
  } else {
    constexpr int MID = (LO + HI) / 2;
    if (n <= MID)
      vm_wait_range<LO, MID>(n);
    else
      vm_wait_range<MID + 1, HI>(n);
  }
}
__device__ __forceinline__ void vm_wait_le(int n) { vm_wait_range<0, 63>(n < 0 ? 0 : (n > 63 ? 63 : n)); }

// LDS written by some lanes of a wave and read by others: the wave's LDS
// operations run in order; this keeps the compiler from reordering them.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// A unit's partials merged (log-sum-exp) by one wave and written as its output:
//   out = sum_k 2^(m_k - M) acc_k / sum_k 2^(m_k - M) l_k,  M = max_k m_k
// Piece layout: acc [rep][D] fp32, then (m, l) [rep] float2. Every lane owns up
// to CPL float4 columns; pieces are read in batches whose loads are all in
// flight (a unit of up to BATCH pieces costs one round trip to the L2). AUX is
// the load cache policy (1: L1 bypass, for partials that other CUs of this XCD
// wrote during this launch).
template <typename Tag, int D, int AUX>
__device__ __forceinline__ void merge_unit(const decode_args& a, int unit, int np, int base, int lane) {
  typedef typename dmath<Tag>::scalar_t scalar_t;
  constexpr int CPL = (dshape<D>::HMAX * D / 4 + 63) / 64;
  constexpr int BATCH = 24 / CPL;
  const int b = unit / a.num_kv_heads, h = unit - b * a.num_kv_heads;
  const auto rs = raw_rsrc(a.pieces, a.pieces_bytes);
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
  constexpr int NSL = S::NSL, NW = S::NW, RING = S::RING, SLOT = S::SLOT;
  // the ring (the only target of direct loads) and the other areas are separate
  // arrays, so the compiler sees that reads of the latter never wait for the ring
  __shared__ __align__(16) char ring_all[S::RING_BYTES];
  __shared__ __align__(16) char q_all[NW * S::QW];                  // q rows per segment; output staging
  __shared__ __align__(16) float rope_all[NW * S::ROPE_W / 4];       // cos | sin rows per segment
  __shared__ __align__(16) int32_t seg_all[NW * S::SEGW * 8];
  __shared__ __align__(16) int32_t blk_all[NW * S::TMAXW];

  // wave-uniform values (the wave index, the plan records and everything derived
  // from them) are made scalar, so the loop control and the waits stay scalar
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int32_t* const P = a.plan;
  const int W = P[0], nS = P[1], nU = P[2];
  const bool grouped = P[7] != 0;                // pieces merged per workgroup in LDS first
  const int worker = blockIdx.x * NW + wave;
  if (worker >= W) return;                       // a grid larger than the plan's
  const int4 wr = reinterpret_cast<const int4*>(P + 8)[worker];
  const int sf = __builtin_amdgcn_readfirstlane(wr.x), nseg = __builtin_amdgcn_readfirstlane(wr.y);
  const int tf = __builtin_amdgcn_readfirstlane(wr.z), ntiles = __builtin_amdgcn_readfirstlane(wr.w);
  const int rep = a.rep;
  // the plan builder keeps every worker within its LDS areas; a plan that does not
  // is not served (nothing is read or written). Waves without work still reach the
  // workgroup's barrier below.
  const bool live = !(ntiles <= 0 || nseg <= 0 || nseg > S::SEGW || ntiles > S::TMAXW || nseg * rep * RB > S::QW);
  const int32_t* const units_g = P + 8 + 4 * W + 8 * nS;
  char* const ring = ring_all + wave * RING * SLOT;
  char* const qw = q_all + wave * S::QW;
  float* const rw = rope_all + wave * S::ROPE_W / 4;
  int32_t* const sw = seg_all + wave * S::SEGW * 8;
  int32_t* const bw = blk_all + wave * S::TMAXW;

  // the online-softmax state of the current segment: O[head 4 lg + j][16 nn + lc], the max
  // of head lc (base-2 domain) and its sum; and that of the first segment, kept to the
  // end when it is a piece
  float4_t acc[NSL], acc0[NSL];
  float m_run = -INFINITY, l_w = 0.f, m0 = -INFINITY, lw0 = 0.f;
#pragma unroll
  for (int nn = 0; nn < NSL; ++nn) acc[nn] = acc0[nn] = float4_t{0.f, 0.f, 0.f, 0.f};
  if (live) {
    // ---- the worker's segments and tile blocks into LDS ----
    {
      const int32_t* const segs_g = P + 8 + 4 * W + 8 * sf;
      const int32_t* const tiles_g = units_g + 2 * nU + tf;
      for (int f = lane; f < nseg * 8; f += 64) sw[f] = segs_g[f];
      for (int f = lane; f < ntiles; f += 64) {
        int blk = tiles_g[f];
        if (blk < 0 || blk >= a.num_blocks) blk = 0;   // the plan builder validates blocks; stay inside the pool
        bw[f] = blk;
      }
    }
    wave_lds_sync();
    const bool fused = a.k_new != nullptr;
    const bool roped = a.rope.cos != nullptr;

    const int per_seg = rep * RB / 16;             // 16-byte chunks of a segment's q rows
    constexpr int RC = D / 4;                      // 16-byte chunks of a segment's cos | sin rows

    const int bs = 1 << a.log2_bs;
    const int64_t tile_bytes = (int64_t)bs * RB;                 // one kv head's K (or V) rows of a block
    const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * tile_bytes;
    const int64_t v_off = (int64_t)a.num_kv_heads * tile_bytes;

    // ---- loads: the worker's tiles in order, RING slots ahead ----
    int vmi = 0;                 // vector memory instructions issued since the first tile load
    int slot_done = 0;           // lane s: vmi once the tile in ring slot s was issued
    int ls = 0, lt = 0, lk = 0, islot = 0;   // load cursor: segment, its tile, the worker's tile, slot
    int l_t0 = 0, l_len = 0, l_ctx = 1, l_b = 0, l_h = 0;
    auto load_seg = [&]() {
      const int4 v = *reinterpret_cast<const int4*>(sw + 8 * ls);
      const int u = __builtin_amdgcn_readfirstlane(v.x);
      l_t0 = __builtin_amdgcn_readfirstlane(v.y);
      l_len = __builtin_amdgcn_readfirstlane(v.z) - l_t0;
      l_ctx = __builtin_amdgcn_readfirstlane(sw[8 * ls + 4]);
      l_b = u / a.num_kv_heads;
      l_h = u - l_b * a.num_kv_heads;
    };
    load_seg();
    // one tile's K and V rows into ring slot islot; `real` false: the same count of
    // loads of a valid address whose data is never read (a ring longer than the work)
    auto issue = [&](bool real) {
      char* const dst = ring + islot * SLOT;
      if (real) {
        const int t = l_t0 + lt;
        const int blk = __builtin_amdgcn_readfirstlane(bw[lk]);
        const int p0 = 16 * t;
        const char* kbase =
            a.pool + (int64_t)blk * blk_bytes + (int64_t)l_h * tile_bytes + (int64_t)(p0 & (bs - 1)) * RB;
        const char* kn = fused ? a.k_new + l_b * a.k_new_row_bytes + (int64_t)l_h * RB : nullptr;
        const char* vn = fused ? a.v_new + l_b * a.v_new_row_bytes + (int64_t)l_h * RB : nullptr;
#pragma unroll
        for (int j = 0; j < TLD; ++j) {
          const int f = 64 * j + lane;                // 16-byte slot of the tile
          const int r = f / VCOLS, cs = f % VCOLS;
          int p = p0 + r;
          if (p >= l_ctx) p = l_ctx - 1;              // rows past the context read a valid row (masked)
          const int rr = p - p0;
          const bool newest = fused && p == l_ctx - 1;
          const int ck = cs ^ S::kswz(r), cv = cs ^ S::vswz(r);
          const char* ks = newest ? kn + 16 * ck : kbase + rr * RB + 16 * ck;
          const char* vs = newest ? vn + 16 * cv : kbase + v_off + rr * RB + 16 * cv;
          dma16(ks, dst + 1024 * j);
          dma16(vs, dst + TB + 1024 * j);
        }
        ++lt;
        ++lk;
        if (lt == l_len && lk < ntiles) {
          ++ls;
          lt = 0;
          load_seg();
        }
      } else {
#pragma unroll
        for (int j = 0; j < TLD; ++j) {
          const char* src = a.pool + 16 * lane;      // the pool holds at least one block (>= 2 KiB)
          dma16(src, dst + 1024 * j);
          dma16(src, dst + TB + 1024 * j);
        }
      }
      vmi += LPT;
      slot_done = lane == islot ? vmi : slot_done;
      islot = islot + 1 == RING ? 0 : islot + 1;
    };
    // The first step's two tiles, then the q rows and RoPE rows of every segment (direct
    // loads into the wave's q and RoPE areas; lanes past the rows load a valid address into
    // the unused rest of the area), then the rest of the ring.
    issue(lk < ntiles);
    issue(lk < ntiles);
    {
      const int nq = (nseg * per_seg + 63) / 64;   // <= QW / 1024 (the plan keeps nseg * rep * RB <= QW)
      for (int j = 0; j < nq; ++j) {
        const int f = 64 * j + lane;
        const char* src = a.q;
        if (f < nseg * per_seg) {
          const int i = f / per_seg, w = f - i * per_seg;
          const int u = sw[8 * i];
          const int b = u / a.num_kv_heads, h = u - b * a.num_kv_heads;
          src = a.q + b * a.q_row_bytes + (int64_t)h * rep * RB + 16 * w;
        }
        dma16(src, qw + 1024 * j);
      }
      vmi += nq;
      if (roped) {
        const int nr = (nseg * RC + 63) / 64;      // <= ROPE_W / 1024
        for (int j = 0; j < nr; ++j) {
          const int f = 64 * j + lane;
          const float* src = a.rope.cos;
          if (f < nseg * RC) {
            const int i = f / RC, w = f - i * RC;
            const int64_t row = a.rope.row(sw[8 * i + 4] - 1, D / 2);   // the row's own position
            src = w < RC / 2 ? a.rope.cos + row + 4 * w : a.rope.sin + row + 4 * (w - RC / 2);
          }
          dma16(src, reinterpret_cast<char*>(rw) + 1024 * j);
        }
        vmi += nr;
      }
    }
    const int q_done = vmi;
#pragma unroll
    for (int r = 2; r < RING; ++r) issue(lk < ntiles);
    vm_wait_le(vmi - q_done);                      // q and RoPE rows have landed

    // ---- consume ----
    int cslot = 0;                                 // the slot of the next tile
    int cbase = 0;                                 // the worker's tiles before segment i
    for (int i = 0; i < nseg; ++i) {
      if (i == 1) {                                // the first segment's state, kept when it is a piece
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) acc0[nn] = acc[nn];
        m0 = m_run;
        lw0 = l_w;
      }
      const int4 sgv = *reinterpret_cast<const int4*>(sw + 8 * i);
      const int u = __builtin_amdgcn_readfirstlane(sgv.x);
      const int t0 = __builtin_amdgcn_readfirstlane(sgv.y);
      const int n = __builtin_amdgcn_readfirstlane(sgv.z) - t0;
      const int slot = __builtin_amdgcn_readfirstlane(sgv.w);
      const int ctx = __builtin_amdgcn_readfirstlane(sw[8 * i + 4]);
      const int b = u / a.num_kv_heads, h = u - b * a.num_kv_heads;
      const int head0 = h * rep;
      const int newest = ctx - 1;
      const float* const cosr = rw + i * D;       // this segment's RoPE rows (position ctx - 1)
      const float* const sinr = cosr + D / 2;
      // q (B operand): lane (lc, lg) holds q[b][head0 + lc][32 s + 8 lg .. + 8]; heads past rep are 0
      vec16 qb[KS];
#pragma unroll
      for (int s = 0; s < KS; ++s) qb[s] = zero16();
      if (lc < rep) {
        const char* qrow = qw + (i * rep + lc) * RB + 16 * lg;
#pragma unroll
        for (int s = 0; s < KS; ++s) qb[s] = *reinterpret_cast<const vec16*>(qrow + 64 * s);
        if (roped) {   // slice s (dims 32 s + 8 lg ..) pairs with slice s + KS/2
#pragma unroll
          for (int s = 0; s < KS / 2; ++s)
            rope_pair<scalar_t>(qb[s], qb[s + KS / 2], cosr + 32 * s + 8 * lg, sinr + 32 * s + 8 * lg);
        }
      }
      m_run = -INFINITY;
      float l_part = 0.f;          // this lane's share of head lc's sum
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) acc[nn] = float4_t{0.f, 0.f, 0.f, 0.f};

      for (int k = 0; k < n; k += 2) {
        const bool two = k + 1 < n;
        const int cslot2 = cslot + 1 == RING ? 0 : cslot + 1;
        // this step's tiles have landed: at most the instructions issued after its last tile are outstanding
        vm_wait_le(vmi - __builtin_amdgcn_readlane(slot_done, two ? cslot2 : cslot));
        const char* ta = ring + cslot * SLOT;
        const char* tb2 = two ? ring + cslot2 * SLOT : ta;
        const int pa0 = 16 * (t0 + k), pb0 = pa0 + 16;
        // fused append: the unit's newest row was loaded from k_new / v_new; with RoPE its K
        // is rotated in place before the scores read it; either way it goes to its pool slot
        if (fused) {
#pragma unroll
          for (int tt = 0; tt < 2; ++tt) {
            const int pt0 = tt == 0 ? pa0 : pb0;
            if ((tt == 0 || two) && newest >= pt0 && newest < pt0 + 16) {   // wave-uniform
              char* kt = const_cast<char*>(tt == 0 ? ta : tb2);
              const int r = newest - pt0;
              if (roped && lane < VCOLS / 2) {
                char* c1 = kt + r * RB + 16 * (lane ^ S::kswz(r));
                char* c2 = kt + r * RB + 16 * ((lane + VCOLS / 2) ^ S::kswz(r));
                vec16 x1 = __builtin_bit_cast(vec16, ring_read16(c1));
                vec16 x2 = __builtin_bit_cast(vec16, ring_read16(c2));
                rope_pair<scalar_t>(x1, x2, cosr + 8 * lane, sinr + 8 * lane);
                ring_write16(c1, __builtin_bit_cast(u32x4_t_, x1));
                ring_write16(c2, __builtin_bit_cast(u32x4_t_, x2));
              }
              // lanes 0 .. VCOLS-1 store the K row, VCOLS .. 2 VCOLS-1 the V row, the others
              // nothing (their offset is dropped): one store instruction, counted
              const bool act = lane < 2 * VCOLS;
              const bool is_v = lane >= VCOLS;
              const int c = lane % VCOLS;
              u32x4_t_ x = u32x4_t_{0u, 0u, 0u, 0u};
              if (act)
                x = ring_read16(kt + (is_v ? TB : 0) + r * RB + 16 * (c ^ (is_v ? S::vswz(r) : S::kswz(r))));
              const int nblk = __builtin_amdgcn_readfirstlane(bw[cbase + k + tt]);   // a tile lies in one block
              const char* row = a.pool + (int64_t)nblk * blk_bytes + (int64_t)h * tile_bytes +
                                (int64_t)(newest & (bs - 1)) * RB;
              const auto rs = raw_rsrc(row, (uint32_t)(v_off + RB));
              const uint32_t off = act ? (uint32_t)((is_v ? v_off : 0) + 16 * c) : OOB;
              __builtin_amdgcn_raw_buffer_store_b128(x, rs, off, 0, 0);
              vmi += 1;
            }
          }
        }
        // the step's K rows (A operand) and V rows (transposed reads) out of the ring; then
        // the two slots are refilled at once, so their loads fly while the step computes
        uint32_t kad[2 * KS], alo[NSL], ahi[NSL];
        u32x4_t_ kv[2 * KS];
        u32x2_t vlo[NSL], vhi[NSL];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt)
#pragma unroll
          for (int s = 0; s < KS; ++s)
            kad[tt * KS + s] = lds_addr((tt == 0 ? ta : tb2) + lc * RB + 16 * ((4 * s + lg) ^ S::kswz(lc)));
        // O += P.V: k index 8 lg + j <-> row 4 lg + j of tile a (j < 4) or of tile b (j >= 4)
        const int rv_ = 4 * lg + (lc >> 2);
        const int half8 = 8 * (lc & 1);
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) {
          const int c = ((lc & 3) >> 1) + 2 * nn;
          const int off = TB + rv_ * RB + 16 * (c ^ S::vswz(rv_)) + half8;
          alo[nn] = lds_addr(ta + off);
          ahi[nn] = lds_addr(tb2 + off);
        }
        step_reads<KS, NSL>::run(kad, alo, ahi, kv, vlo, vhi);
        cslot = two ? (cslot2 + 1 == RING ? 0 : cslot2 + 1) : cslot2;
        if (lk < ntiles) issue(true);
        if (two && lk < ntiles) issue(true);
        // S^T for both tiles
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
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) {
          vec16 vb;
          vb.w[0] = vlo[nn].x; vb.w[1] = vlo[nn].y; vb.w[2] = vhi[nn].x; vb.w[3] = vhi[nn].y;
          acc[nn] = M::mfma(pa, __builtin_bit_cast(vec8_t, vb), acc[nn]);
        }
      }
      cbase += n;

      // ---- the segment's end: the output of a unit it holds whole; a piece's state stays in
      // registers until the end of the stream ----
      l_w = sum_xor32(sum_xor16(l_part));        // head lc's sum over the segment
      if (__builtin_amdgcn_readfirstlane(sw[8 * i + 5]) < 0) {
        // O / l through this segment's q rows in LDS (read into registers above), then
        // 16-byte stores of the rep output rows
        char* const stage = qw + i * rep * RB;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float inv = 1.f / __shfl(l_w, 4 * lg + j);
          const int hh = 4 * lg + j;
          if (hh < rep) {
#pragma unroll
            for (int nn = 0; nn < NSL; ++nn)
              reinterpret_cast<scalar_t*>(stage + hh * RB)[16 * nn + lc] = (scalar_t)(acc[nn][j] * inv);
          }
        }
        wave_lds_sync();
        const auto rs = raw_rsrc(a.out + b * a.out_row_bytes + (int64_t)head0 * RB, (uint32_t)(rep * RB));
#pragma unroll
        for (int j = 0; j < S::OUTI; ++j) {
          const int c = 64 * j + lane;
          const bool act = c < per_seg;
          const vec16 x = act ? *reinterpret_cast<const vec16*>(stage + 16 * c) : zero16();
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t_, x), rs, act ? 16u * c : OOB, 0, 0);
        }
        vmi += S::OUTI;
      } else if (!grouped) {
        // the piece's partial: acc [rep][D] fp32 (unnormalised), then (m, l) [rep]; lanes
        // of heads past rep address nothing (one store instruction each, counted)
        const auto rs = raw_rsrc(a.pieces, a.pieces_bytes);
        const uint32_t p = (uint32_t)__builtin_amdgcn_readfirstlane(sw[8 * i + 3]) * a.piece_bytes;
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int hh = 4 * lg + j;
            const uint32_t off = hh < rep ? p + 4u * (hh * D + 16 * nn + lc) : OOB;
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(acc[nn][j]), rs, off, 0, 0);
          }
        const uint32_t moff = (lg == 0 && lc < rep) ? p + 4u * rep * D + 8u * lc : OOB;
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, make_float2(m_run, l_w)), rs, moff, 0, 0);
        vmi += NSL * 4 + 1;
      }
    }
  }
  // every load has landed and every store is acknowledged (nothing is in flight when
  // the wave ends, and the ring is idle)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  // ---- pieces: merged per workgroup in LDS, then per unit through the L2 ----
  // After the barrier the four waves have streamed their last tiles and the ring area
  // holds the pieces' states (acc [rep][D] fp32, then (m, l) [rep]); the first member
  // of each group of a unit's consecutive pieces merges them. (Loads issued while the
  // other waves of the CU still had tiles in flight would also queue behind those.)
  if (grouped) __syncthreads();                  // uniform: one plan for the workgroup
  constexpr int STATE = (S::HMAX * D * 4 + S::HMAX * 8 + 15) / 16 * 16;
  static_assert(2 * NW * STATE <= S::RING_BYTES, "piece states in the ring area");
  auto piece_seg = [&](int e) {                  // the wave's first (e = 0) or last segment if a piece, else -1
    if (!live || (e == 1 && nseg < 2)) return -1;
    const int i = e == 0 ? 0 : nseg - 1;
    return __builtin_amdgcn_readfirstlane(sw[8 * i + 5]) >= 0 ? i : -1;
  };
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int i = grouped ? piece_seg(e) : -1;
    if (i < 0) continue;
    const bool last = i == nseg - 1;             // the live state, else the kept first one
    float* const st = reinterpret_cast<float*>(ring_all + __builtin_amdgcn_readfirstlane(sw[8 * i + 5]) * STATE);
#pragma unroll
    for (int nn = 0; nn < NSL; ++nn)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int hh = 4 * lg + j;
        if (hh < rep) st[hh * D + 16 * nn + lc] = last ? acc[nn][j] : acc0[nn][j];
      }
    if (lg == 0 && lc < rep)
      reinterpret_cast<float2*>(st + rep * D)[lc] = last ? make_float2(m_run, l_w) : make_float2(m0, lw0);
  }
  if (grouped) __syncthreads();
  // the leaders: a group's states merged (log-sum-exp); the output when the group holds
  // the whole unit, else the group's partial for the unit-level merge
  constexpr int CPL = (S::HMAX * D / 4 + 63) / 64;
  const int n4 = rep * D / 4;
  int lead_u[2] = {-1, -1}, lead_np[2] = {0, 0}, lead_base[2] = {0, 0};
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int i = piece_seg(e);
    if (i < 0) continue;
    const int role = __builtin_amdgcn_readfirstlane(sw[8 * i + 6]);
    if (role == 0) continue;                     // a member: its leader merges it
    if (!grouped) {                              // the piece was stored at its segment's end
      lead_u[e] = __builtin_amdgcn_readfirstlane(sw[8 * i]);
      lead_np[e] = role >> 8;
      lead_base[e] = __builtin_amdgcn_readfirstlane(sw[8 * i + 7]);
      continue;
    }
    const int u = __builtin_amdgcn_readfirstlane(sw[8 * i]);
    const int slot = __builtin_amdgcn_readfirstlane(sw[8 * i + 3]);
    const int k0 = __builtin_amdgcn_readfirstlane(sw[8 * i + 5]);
    const int members = role & 0xFF;
    const int b = u / a.num_kv_heads, h = u - b * a.num_kv_heads;
    // every member's (m, l) and acc columns read at once (the loop runs over the most
    // members a group can have, 2 NW, so that the reads are not serialised)
    float Mx[CPL], L[CPL];
    float4_t o[CPL];
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const int c = lane + 64 * q;
      const int head = (4 * c) / D;
      const bool act = c < n4;
      float2 ml[2 * NW];
      float4_t v[2 * NW];
#pragma unroll
      for (int k = 0; k < 2 * NW; ++k) {
        ml[k] = make_float2(-INFINITY, 0.f);
        v[k] = float4_t{0.f, 0.f, 0.f, 0.f};
        if (act && k < members) {
          const float* st = reinterpret_cast<const float*>(ring_all + (k0 + k) * STATE);
          ml[k] = reinterpret_cast<const float2*>(st + rep * D)[head];
          v[k] = *reinterpret_cast<const float4_t*>(st + 4 * c);
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int k = 0; k < 2 * NW; ++k) mx = fmaxf(mx, ml[k].x);
      float l = 0.f;
      float4_t acc_o = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 2 * NW; ++k) {
        const float w = ml[k].y > 0.f ? fast_exp2(ml[k].x - mx) : 0.f;
        l = fmaf(ml[k].y, w, l);
        acc_o += v[k] * w;
      }
      Mx[q] = mx;
      L[q] = l;
      o[q] = acc_o;
    }
    if (slot < 0) {
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int c = lane + 64 * q;
        if (c >= n4) continue;
        const float inv = 1.f / L[q];
        typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
        s4_t r;
#pragma unroll
        for (int j = 0; j < 4; ++j) r[j] = (scalar_t)(o[q][j] * inv);
        *reinterpret_cast<s4_t*>(a.out + b * a.out_row_bytes + ((int64_t)h * rep * D + 4 * c) * 2) = r;
      }
    } else {
      const auto rs = raw_rsrc(a.pieces, a.pieces_bytes);
      const uint32_t p = (uint32_t)slot * a.piece_bytes;
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int c = lane + 64 * q;
        const bool act = c < n4;
        const int head = (4 * c) / D;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t_, o[q]), rs, act ? p + 16u * c : OOB, 0, 0);
        const bool first_col = act && (4 * c) % D == 0;   // one (M, L) per head
        __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2_t, make_float2(Mx[q], L[q])), rs,
                                              first_col ? p + 4u * rep * D + 8u * head : OOB, 0, 0);
      }
      lead_u[e] = u;
      lead_np[e] = role >> 8;
      lead_base[e] = __builtin_amdgcn_readfirstlane(sw[8 * i + 7]);
    }
  }
  if (a.merge_in_kernel && (lead_u[0] >= 0 || lead_u[1] >= 0)) {
    // the group partials are in this XCD's L2 (their stores acknowledged) before their
    // arrivals count them; both arrivals in flight together
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7;                                    // arrival fields: 8 XCDs of 8 bits
    const unsigned long long mine = 1ull << (8 * xcc);
    unsigned long long prev[2] = {0, 0};
#pragma unroll
    for (int e = 0; e < 2; ++e)
      if (lead_u[e] >= 0 && lane == 0)
        prev[e] = __hip_atomic_fetch_add(a.arrivals + 16 * (int64_t)lead_u[e], mine, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      if (lead_u[e] < 0) continue;
      const int u = lead_u[e], np = lead_np[e];
      const unsigned long long now = __shfl(prev[e], 0) + mine;
      int arrived = 0;
#pragma unroll
      for (int x = 0; x < 8; ++x) arrived += (int)((now >> (8 * x)) & 0xFF);
      if (arrived == np) {                       // the last partial: merge them all
        if (now != ((unsigned long long)np << (8 * xcc)) && lane == 0)
          __hip_atomic_fetch_add(a.violations, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        merge_unit<Tag, D, 1>(a, u, np, lead_base[e], lane);
        if (lane == 0)
          __hip_atomic_store(a.arrivals + 16 * (int64_t)u, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

// Partials merged after the launch (merge_in_kernel = 0): one wave per split unit.
template <typename Tag, int D>
__global__ __launch_bounds__(64) void decode_combine_kernel(const decode_args a) {
  const int u = blockIdx.x;
  const int32_t* const P = a.plan;
  if (u >= P[2]) return;                          // grids may be sized for a capacity
  const int32_t* const unit_rec = P + 8 + 4 * P[0] + 8 * P[1];
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
                                    int32_t* max_tiles_per_worker, int32_t* max_segments_per_worker,
                                    int32_t* waves_per_wg) {
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads) return TB_ERR_INVALID_ARG;
  if (head_dim != 64 && head_dim != 128) return TB_ERR_UNSUPPORTED;
  const int rep = num_heads / num_kv_heads;
  if (rep > tb::dshape<64>::HMAX) return TB_ERR_UNSUPPORTED;
  const bool d64 = head_dim == 64;
  const int tmax = d64 ? tb::dshape<64>::TMAXW : tb::dshape<128>::TMAXW;
  const int segw = d64 ? tb::dshape<64>::SEGW : tb::dshape<128>::SEGW;
  const int qw = d64 ? tb::dshape<64>::QW : tb::dshape<128>::QW;
  const int by_q = qw / (rep * 2 * head_dim);
  if (max_tiles_per_worker) *max_tiles_per_worker = tmax;
  if (max_segments_per_worker) *max_segments_per_worker = by_q < segw ? by_q : segw;
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
                                   int64_t out_row_stride, int32_t num_seqs, const int32_t* plan,
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
  TB_CHECK_ARG(q && pool && out && plan && num_blocks > 0);
  TB_CHECK_ARG((((uintptr_t)q | (uintptr_t)pool | (uintptr_t)out) & 15u) == 0);
  TB_CHECK_ARG(q_row_stride >= (int64_t)num_heads * head_dim && out_row_stride >= (int64_t)num_heads * head_dim);
  TB_CHECK_ARG((q_row_stride * 2) % 16 == 0 && (out_row_stride * 2) % 16 == 0);
  // a block's K and V rows of one position are addressed through one buffer resource
  TB_CHECK_ARG((int64_t)num_kv_heads * block_size * head_dim * 2 + head_dim * 2 < ((int64_t)1 << 31));
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
