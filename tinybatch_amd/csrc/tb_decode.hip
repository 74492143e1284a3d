// K2 for decode steps, streaming form (one query row per sequence), fp16 / bf16.
//
// Replaces, for the decode rows of Qwen2Paged.forward (reference
// src/tinybatch/model.py:130-147), the per-sequence gather (kv_cache.py:40-45),
// repeat_interleave (model.py:135-137) and SDPA over the whole context (a decode
// row sees every position, model.py:142-146), with the fused append of the row's
// new K/V (kv_cache.py:25-38) when k_new is given.
//
// Work: a unit is one sequence's K/V rows of one kv head (u = b * Hkv + h), cut
// into 16-position tiles (a tile lies in one pool block: block_size >= 16).
// The host plan (tb_stream_build_plan) packs whole units onto the XCDs, longest
// first, and splits each XCD's tile list evenly over the waves of the
// workgroups that run there (workgroup g on XCD g % num_xcds; a workgroup fills
// one CU). Every wave is an independent worker that streams its own range of
// tiles: the plan gives each worker a record of per-tile entries
//   (byte offset of the tile's K rows >> 8, sequence | kv head << 20 | valid
//    rows - 1 << 24 | the unit's last tile << 28 | padding tile << 29,
//    context | piece index << 24, first partial slot | pieces - 1 << 20 |
//    wave of piece 0 << 28, or -1 for a unit one worker holds whole)
// so its first tile loads wait on one read (its entries).
//
// Loads. Every K and V tile moves by direct global->LDS loads of 1 KiB of
// consecutive pool bytes per instruction, non-temporal (a 16-row x 64-byte
// operand-shaped load is markedly slower from HBM), into a ring of R tile slots
// per wave; the loads of tile j + R are issued once tile j's rows are read out
// of its slot. Two cursors walk the worker's tiles: the issuing one, R tiles
// ahead, also starts each new unit's q rows (and RoPE rows) on their way into
// one of R + 1 q slots, ahead of that unit's first tile, so a wave never waits
// on a dependent read inside its stream. The waits are explicit vmcnt counts
// (the direct loads are asm the compiler does not see; the loads of a wave
// complete in issue order).
//
// Math per tile (16 positions), with the GQA group of the kv head as the 16
// MFMA columns (heads past rep are zero):
//   S^T[pos][head] = K[pos][:] . q[head][:]     v_mfma_f32_16x16x32, A = K rows (LDS)
//   O^T[d][head]  += V^T[d][pos] . P^T[pos][head]  v_mfma_f32_16x16x16, A = V^T (LDS
//                                                 transpose reads), B = the S^T registers
// so the online-softmax state of head lc (max, sum, its O^T column) lives in the
// lanes of column lc, and rescaling needs no lane exchange.
//
// A unit whose tiles one worker streams whole writes its output. A unit spread
// over several workers leaves one partial (unnormalised O, max, sum) per worker
// (a worker holds at most two: its range's first and last units); after its last
// tile each wave counts its partials in the units' arrival words and the wave
// whose partial arrives last merges them (log-sum-exp) and writes the output.
// All of a unit's partials are written and read inside one XCD, whose L2 every
// CU of the XCD shares: plain stores (acknowledged before the arrival is
// counted) and L1-bypassing loads suffice. The arrival word keeps a count per
// XCD (8-bit fields), so a partial that ran on another XCD is detected and
// counted in `violations`.
#include "tb_stream.h"

namespace tb {

struct stream_args {
  const char* q;            // [B][Hq][D]
  int64_t q_row_bytes;
  char* pool;               // [NB][2][Hkv][BS][D]
  int64_t num_blocks;
  char* out;                // [B][Hq*D]
  int64_t out_row_bytes;
  const int32_t* counts;    // [workers] tiles of each worker
  const int4* entries;      // [workers][stride] (+ 64 entries of padding)
  int32_t stride;
  int32_t workers;
  char* pieces;             // partials: piece_bytes each
  uint32_t pieces_bytes;    // bytes addressable through the buffer resource
  int32_t piece_bytes;
  unsigned long long* arrivals;   // per unit, 128 bytes apart, zero between launches
  uint32_t* violations;     // incremented when a unit's partials ran on more than one XCD
  int32_t num_heads, num_kv_heads, rep;
  int32_t log2_sub;         // log2(block_size / 16): 16-position tiles per block
  float scale_log2e;
  const char* k_new;        // fused append (may be null)
  int64_t k_new_row_bytes;
  const char* v_new;
  int64_t v_new_row_bytes;
  rope_tables rope;
};

template <int D, int W, int R>
struct sshape {
  static constexpr int RB = 2 * D;             // bytes per K or V row
  static constexpr int TB = 16 * RB;           // bytes of a 16-position K (or V) tile
  static constexpr int VCOLS = RB / 16;        // 16-byte chunks per row
  static constexpr int TLD = TB / 1024;        // direct loads per tile, of K and of V each
  static constexpr int KS = D / 32;            // k-slices of q.k
  static constexpr int NSL = D / 16;           // 16-dim slices of O
  static constexpr int HMAX = 8;               // query heads per kv head
  // q slot of a unit: q rows [HMAX][D], then cos [D/2] | sin [D/2] fp32 at the row's
  // position, then the fused append's new K row and V row
  static constexpr int QROPE = HMAX * RB;
  static constexpr int QNEW = QROPE + 4 * D;
  static constexpr int QSLOT = (QNEW + 2 * RB + 1023) / 1024 * 1024;
  static constexpr int QLD = QSLOT / 1024;     // direct loads per q slot
  static constexpr int QS = R + 1;             // q slots: the consumed unit's and R ahead
  static constexpr int ENT = 2 * 1024;         // two chunks of 64 entries
  static constexpr int STATE = 8 * D * 4 + 8 * 8;   // a partial's state: acc [8][D] fp32, (m, l) [8]
  static constexpr int WAVE_LDS = R * 2 * TB + QS * QSLOT + ENT + (STATE + 15) / 16 * 16;
  static constexpr int LDS = W * WAVE_LDS;
  static constexpr int CW = (R - 1) * 2 * TLD; // loads in flight after a tile, in a steady stream
  static_assert(LDS <= 160 * 1024, "LDS budget of a workgroup");
  static_assert(2 * TLD * R + QLD * R + 2 <= 63, "vmcnt range");
  static_assert(STATE <= R * 2 * TB, "a partial's state fits in the ring");
  // the swizzled tile layout of tb_stream.h
  static __device__ __forceinline__ int kswz(int r) { return stream_kswz(r); }
  static __device__ __forceinline__ int vswz(int r) { return stream_vswz(r); }
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t s_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
constexpr uint32_t S_OOB = 0x80000000u;   // an offset the buffer range check drops

// A unit's group partials merged (log-sum-exp) by one wave, on top of the running state
// (Mx, L, o) it is given (group `skip`, if any, is not read), and written as its output:
//   out = sum_g 2^(m_g - M) acc_g / sum_g 2^(m_g - M) l_g,  M = max_g m_g
// The pieces of a unit that one workgroup holds were merged in LDS into one group
// partial, stored in the slot of the group's first piece: piece 0 and every piece
// i with (w0 + i) % W == 0 (w0: the wave index of piece 0's worker). Partial
// layout: acc [rep][D] fp32 (unnormalised), then (m, l) [rep] float2. Lane l owns
// float4 columns c = l + 64 q of the rep * D / 4 and keeps its own running (M, L,
// o), so no lane exchange is needed; all groups' loads are in flight at once
// (up to 8 groups per batch). Loads are device scope (they miss in L1): other CUs of this XCD wrote them.
template <typename Tag, int D, int W>
__device__ __forceinline__ void stream_merge(const stream_args& a, int b, int h, int np, int base, int w0,
                                             int lane, int skip, float (&Mx)[(8 * D / 4 + 63) / 64],
                                             float (&L)[(8 * D / 4 + 63) / 64],
                                             float4_t (&o)[(8 * D / 4 + 63) / 64]) {
  typedef typename smath<Tag>::scalar_t scalar_t;
  constexpr int CPL = (8 * D / 4 + 63) / 64;     // float4 columns per lane (up to 8 heads)
  constexpr int BATCH = 8;
  const auto rs = s_rsrc(a.pieces, a.pieces_bytes);
  const int n4 = a.rep * D / 4;
  const uint32_t ml_off = (uint32_t)(a.rep * D * 4);
  const int groups = 1 + (w0 + np - 1) / W;
  for (int g0 = 0; g0 < groups; g0 += BATCH) {
    float2 ml[BATCH][CPL];
    float4_t v[BATCH][CPL];
#pragma unroll
    for (int kk = 0; kk < BATCH; ++kk) {
      const int g = g0 + kk;
      if (g >= groups) break;
      const uint32_t p = (uint32_t)(base + (g == 0 ? 0 : W * g - w0)) * a.piece_bytes;
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int c = lane + 64 * q;
        const bool act = c < n4 && g != skip;     // the caller's own group is already in (Mx, L, o)
        ml[kk][q] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, act ? p + ml_off + 8 * ((4 * c) / D) : S_OOB, 0, LOAD_DEVICE_SCOPE));
        v[kk][q] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, act ? p + 16 * c : S_OOB, 0, LOAD_DEVICE_SCOPE));
      }
    }
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      float mb = Mx[q];
#pragma unroll
      for (int kk = 0; kk < BATCH; ++kk)
        if (g0 + kk < groups && g0 + kk != skip) mb = fmaxf(mb, ml[kk][q].x);
      const float keep = fast_exp2(Mx[q] - mb);   // 0 while Mx = -inf
      L[q] *= keep;
      o[q] *= keep;
#pragma unroll
      for (int kk = 0; kk < BATCH; ++kk) {
        if (g0 + kk >= groups) break;
        const float w = (g0 + kk != skip && ml[kk][q].y > 0.f) ? fast_exp2(ml[kk][q].x - mb) : 0.f;
        L[q] = fmaf(ml[kk][q].y, w, L[q]);
        o[q] += v[kk][q] * w;
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
    st8_through(a.out + b * a.out_row_bytes + ((int64_t)h * a.rep * D + 4 * c) * 2, r);
  }
}

constexpr int E_LAST_D = 1 << 28;   // entry flags (device side)
constexpr int E_NULL_D = 1 << 29;

template <typename Tag, int D, int W, int R>
__global__ __launch_bounds__(64 * W) void paged_stream_kernel(const stream_args a) {
  using S = sshape<D, W, R>;
  using M = smath<Tag>;
  typedef typename M::scalar_t scalar_t;
  constexpr int RB = S::RB, TB = S::TB, VCOLS = S::VCOLS, TLD = S::TLD, KS = S::KS, NSL = S::NSL;
  constexpr int QS = S::QS, QSLOT = S::QSLOT, QLD = S::QLD, QROPE = S::QROPE, QNEW = S::QNEW;
  constexpr int STEPS = R / 2;                   // steps (tile pairs) in flight
  constexpr int CW2 = (R - 2) * 2 * TLD;         // loads issued after a step's pair, in a steady stream
  constexpr int STATE = S::STATE;
  static_assert(R % 2 == 0, "a step is a pair of ring slots");
  __shared__ __align__(1024) char lds_all[S::LDS];
  __shared__ __align__(16) int pend_sh[W][2][4];   // per wave: its partials (unit, np | w0 << 8 | idx << 16, base,
                                                 // sequence | kv head << 20)

  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int k = blockIdx.x * W + wave;
  char* const ring = lds_all + wave * S::WAVE_LDS;
  char* const qsl = ring + R * 2 * TB;
  char* const ents = qsl + QS * QSLOT;
  char* const pst = ents + S::ENT;               // the state of a partial finished mid-stream
  const int rep = a.rep;
  const int4* const ent_g = a.entries + (int64_t)(k < a.workers ? k : 0) * a.stride;

  // ---- the worker's entry count and its first 64 entries (one round trip) ----
  int4 ev = ent_g[lane];                         // the issuing cursor's entries, lane = tile (the
                                                 // entry array is padded by 64 entries)
  int n = k < a.workers ? __builtin_amdgcn_readfirstlane(a.counts[k]) : 0;
  asm volatile("" : "+v"(ev.x), "+v"(ev.y), "+v"(ev.z), "+v"(ev.w));   // complete here, for the compiler too
  {
    // count word: tiles | newest slots shared by two sequences << 30. A malformed count
    // (the plan builder never makes one) and a fused append the plan cannot serve are
    // refused: nothing is streamed or written, and the call's error count says so
    const bool shared_newest = (n >> 30) & 1;
    const int cnt = n & 0x3FFFFFFF;
    const bool bad = n < 0 || cnt > a.stride || (cnt & 1);
    const bool refused = shared_newest && a.k_new != nullptr;
    if ((bad || (refused && k == 0)) && lane == 0)
      __hip_atomic_fetch_add(a.violations, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    n = (bad || refused) ? 0 : cnt;
  }

  const bool fused = a.k_new != nullptr;
  const bool roped = a.rope.cos != nullptr;
  const uint32_t v_off = (uint32_t)(a.num_kv_heads * ((int64_t)TB << a.log2_sub));
  const char* const dummy = a.q;                 // finite bytes for q-slot lanes with nothing to load

  // per-lane byte offsets of a tile's direct loads (16-byte chunks, swizzled per row)
  uint32_t koff[TLD], voff[TLD];
#pragma unroll
  for (int i = 0; i < TLD; ++i) {
    const int f = 64 * i + lane;
    const int r = f / VCOLS, cs = f % VCOLS;
    koff[i] = (uint32_t)(r * RB + 16 * (cs ^ S::kswz(r)));
    voff[i] = v_off + (uint32_t)(r * RB + 16 * (cs ^ S::vswz(r)));
  }

  int issued = 0;           // vector memory instructions counted since the entries landed
  int chunk_mark = 0;       // `issued` once the next chunk of entries was issued
  int iseg = -1, icur = -1; // issuing cursor: its unit ordinal and unit key

  // Issue tiles j, j + 1 (j even) into ring slots j % R, j % R + 1 (at a new unit, that
  // unit's q slot first). Returns their entries.
  auto issue = [&](int j, int4& eA, int4& eB) {
    if ((j & 63) == 0 && j > 0) {                // the chunk's entries have landed: into registers
      s_vm_wait_le(issued - chunk_mark);
      ev = *reinterpret_cast<const int4*>(ents + 1024 * ((j >> 6) & 1) + 16 * lane);
    }
    if ((j & 63) == 32 && j + 32 < n) {          // the next chunk of entries
      s_dma16(ent_g + (j + 32) + lane, ents + 1024 * (((j + 32) >> 6) & 1));
      issued += 1;
      chunk_mark = issued;
    }
    const int jl = j & 63;
    eA = int4{__builtin_amdgcn_readlane(ev.x, jl), __builtin_amdgcn_readlane(ev.y, jl),
              __builtin_amdgcn_readlane(ev.z, jl), __builtin_amdgcn_readlane(ev.w, jl)};
    eB = int4{__builtin_amdgcn_readlane(ev.x, jl + 1), __builtin_amdgcn_readlane(ev.y, jl + 1),
              __builtin_amdgcn_readlane(ev.z, jl + 1), __builtin_amdgcn_readlane(ev.w, jl + 1)};
    const int key = eA.y & 0xFFFFFF;
    if (key != icur) {                           // a new unit: q, RoPE and new K/V rows into its q slot
      icur = key;
      ++iseg;
      const int b = eA.y & 0xFFFFF, h = (eA.y >> 20) & 15;
      char* const qd = qsl + (iseg % QS) * QSLOT;
      const char* const qrow = a.q + b * a.q_row_bytes + (int64_t)h * rep * RB;
      const int64_t rrow = roped ? a.rope.row((eA.z & 0xFFFFFF) - 1, D / 2) : 0;
      const char* const kn = fused ? a.k_new + b * a.k_new_row_bytes + (int64_t)h * RB : dummy;
      const char* const vn = fused ? a.v_new + b * a.v_new_row_bytes + (int64_t)h * RB : dummy;
#pragma unroll
      for (int i = 0; i < QLD; ++i) {
        const int f = 64 * i + lane;             // 16-byte chunk of the slot
        const char* src = dummy;
        if (f < rep * VCOLS) {
          src = qrow + 16 * f;
        } else if (f >= QROPE / 16 && f < QROPE / 16 + D / 4) {
          const int g = f - QROPE / 16;          // cos chunks 0 .. D/8-1, then sin
          if (roped)
            src = reinterpret_cast<const char*>(g < D / 8 ? a.rope.cos + rrow + 4 * g
                                                          : a.rope.sin + rrow + 4 * (g - D / 8));
        } else if (f >= QNEW / 16 && f < QNEW / 16 + 2 * VCOLS) {
          const int g = f - QNEW / 16;
          src = g < VCOLS ? kn + 16 * g : vn + 16 * (g - VCOLS);
        }
        s_dma16(src, qd + 1024 * i);
      }
      issued += QLD;
    }
    const char* const baseA = a.pool + ((uint64_t)(uint32_t)eA.x << 8);
    const char* const baseB = a.pool + ((uint64_t)(uint32_t)eB.x << 8);
    char* const dst = ring + (j % R) * 2 * TB;
#pragma unroll
    for (int i = 0; i < TLD; ++i) {
      s_dma16_s(koff[i], baseA, dst + 1024 * i);
      s_dma16_s(voff[i], baseA, dst + TB + 1024 * i);
    }
    // a pad loads nothing: its scores are masked and its V operand is tile A's, so its
    // slot's stale bytes are never used
    if (!(eB.y & E_NULL_D)) {
#pragma unroll
      for (int i = 0; i < TLD; ++i) {
        s_dma16_s(koff[i], baseB, dst + 2 * TB + 1024 * i);
        s_dma16_s(voff[i], baseB, dst + 3 * TB + 1024 * i);
      }
      issued += 2 * TLD;
    }
    issued += 2 * TLD;
  };

  int4 esA[STEPS], esB[STEPS];                   // the entries of each step slot's pair
  int mark[STEPS];                               // `issued` once the pair was issued
#pragma unroll
  for (int t = 0; t < STEPS; ++t)
    if (2 * t < n) {
      issue(2 * t, esA[t], esB[t]);
      mark[t] = issued;
    }

  int cseg = -1, ccur = -1;
  su32x4_t qb[KS];
  float4_t acc[NSL];
  float m_run = -INFINITY, l_part = 0.f;
  bool pend0 = false, pend1 = false;            // partials: finished mid-stream (in pst), at the end
  int pinfo1[4] = {0, 0, 0, 0};
  int pbh1 = 0;                                 // the end partial's sequence | kv head << 20
  const auto prs = s_rsrc(a.pieces, a.pieces_bytes);
#pragma unroll
  for (int s = 0; s < KS; ++s) qb[s] = su32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
  for (int nn = 0; nn < NSL; ++nn) acc[nn] = float4_t{0.f, 0.f, 0.f, 0.f};

  // the partial state (unnormalised O^T of head lc, its max and sum) into LDS:
  // acc [8][D] fp32, then (m, l) [8] float2
  auto save_state = [&](char* dst, float l_tot) {
    if (lc < rep) {
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn)
        *reinterpret_cast<float4_t*>(dst + 4 * (lc * D + 16 * nn + 4 * lg)) = acc[nn];
      if (lg == 0) *reinterpret_cast<float2*>(dst + 4 * 8 * D + 8 * lc) = make_float2(m_run, l_tot);
    }
  };

  for (int j0 = 0; j0 < n; j0 += R) {
#pragma unroll
    for (int t = 0; t < STEPS; ++t) {
      const int j = j0 + 2 * t;
      if (j >= n) break;
      {                                          // the pair (and everything issued before it) has landed
        const int after = issued - mark[t];
        if (after >= CW2)
          asm volatile("s_waitcnt vmcnt(%0)" ::"n"(CW2) : "memory");
        else
          s_vm_wait_le(after);
      }
      const int4 eA = esA[t], eB = esB[t];
      const int key = eA.y & 0xFFFFFF;
      const int b = eA.y & 0xFFFFF, h = (eA.y >> 20) & 15;
      const bool bnull = eB.y & E_NULL_D;
      const bool lastA = eA.y & E_LAST_D;      // then tile B is a pad
      const bool lastB = eB.y & E_LAST_D;
      const int rows_a = lastA ? (eA.y >> 24) & 15 : 15;
      const int rows_b = lastB ? (eB.y >> 24) & 15 : 15;
      char* const slotA = ring + (2 * t) * 2 * TB;
      char* const slotB = slotA + 2 * TB;
      char* const qd = qsl + ((cseg + (key != ccur ? 1 : 0)) % QS) * QSLOT;
      const float* const cosr = reinterpret_cast<const float*>(qd + QROPE);
      const float* const sinr = cosr + D / 2;
      if (key != ccur) {                         // a new unit: q (B operand) from its slot, rotated
        ccur = key;
        ++cseg;
#pragma unroll
        for (int s = 0; s < KS; ++s) qb[s] = su32x4_t{0u, 0u, 0u, 0u};
        if (lc < rep) {
#pragma unroll
          for (int s = 0; s < KS; ++s) qb[s] = *reinterpret_cast<const su32x4_t*>(qd + lc * RB + 64 * s + 16 * lg);
          if (roped) {                           // slice s pairs with slice s + KS/2 (dims + D/2)
#pragma unroll
            for (int s = 0; s < KS / 2; ++s) {
              vec16 x1 = __builtin_bit_cast(vec16, qb[s]), x2 = __builtin_bit_cast(vec16, qb[s + KS / 2]);
              rope_pair<scalar_t>(x1, x2, cosr + 32 * s + 8 * lg, sinr + 32 * s + 8 * lg);
              qb[s] = __builtin_bit_cast(su32x4_t, x1);
              qb[s + KS / 2] = __builtin_bit_cast(su32x4_t, x2);
            }
          }
        }
        m_run = -INFINITY;
        l_part = 0.f;
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) acc[nn] = float4_t{0.f, 0.f, 0.f, 0.f};
      }
      if (lastA || lastB) {
        // the unit's last tile: V rows past the context become zeros (a stale slot may hold
        // any bits; their p is 0); with the fused append its newest row comes from the q
        // slot (K rotated with RoPE) into the ring and goes to its pool slot
        char* const sl = lastA ? slotA : slotB;
        const int rn = lastA ? rows_a : rows_b;
        if (rn < 15) {
#pragma unroll
          for (int i = 0; i < TLD; ++i) {
            const int f = 64 * i + lane;
            if (f / VCOLS > rn) *reinterpret_cast<su32x4_t*>(sl + TB + 16 * f) = su32x4_t{0u, 0u, 0u, 0u};
          }
        }
        if (fused) {
          char* const prow = a.pool + ((uint64_t)(uint32_t)(lastA ? eA.x : eB.x) << 8) + (int64_t)rn * RB;
          if (lane < VCOLS / 2) {                // K chunks lane and lane + VCOLS/2 (dims + D/2)
            vec16 x1 = *reinterpret_cast<const vec16*>(qd + QNEW + 16 * lane);
            vec16 x2 = *reinterpret_cast<const vec16*>(qd + QNEW + 16 * (lane + VCOLS / 2));
            if (roped) rope_pair<scalar_t>(x1, x2, cosr + 8 * lane, sinr + 8 * lane);
            *reinterpret_cast<vec16*>(sl + rn * RB + 16 * (lane ^ S::kswz(rn))) = x1;
            *reinterpret_cast<vec16*>(sl + rn * RB + 16 * ((lane + VCOLS / 2) ^ S::kswz(rn))) = x2;
            st16_through(prow + 16 * lane, x1);
            st16_through(prow + 16 * (lane + VCOLS / 2), x2);
          } else if (lane >= 32 && lane < 32 + VCOLS) {   // V chunk lane - 32
            const int c = lane - 32;
            const vec16 x = *reinterpret_cast<const vec16*>(qd + QNEW + RB + 16 * c);
            *reinterpret_cast<vec16*>(sl + TB + rn * RB + 16 * (c ^ S::vswz(rn))) = x;
            st16_through(prow + v_off + 16 * c, x);
          }
        }
      }
      // both slots' K rows (A operand) and V rows (transposed; a pad's are tile A's), then
      // the refill of the pair
      char* const vslotB = bnull ? slotA : slotB;
      uint32_t ka[2 * KS], va[NSL], vb[NSL];
      su32x4_t kv[2 * KS];
      su32x2_t vlo[NSL], vhi[NSL];
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        ka[s] = s_lds_addr(slotA + lc * RB + 16 * ((4 * s + lg) ^ S::kswz(lc)));
        ka[KS + s] = s_lds_addr(slotB + lc * RB + 16 * ((4 * s + lg) ^ S::kswz(lc)));
      }
      {
        const int rv = 4 * lg + (lc >> 2);
        const int half8 = 8 * (lc & 1);
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) {
          const int c = ((lc & 3) >> 1) + 2 * nn;
          const int off = TB + rv * RB + 16 * (c ^ S::vswz(rv)) + half8;
          va[nn] = s_lds_addr(slotA + off);
          vb[nn] = s_lds_addr(vslotB + off);
        }
      }
      step_reads2<KS, NSL>::run(ka, va, vb, kv, vlo, vhi);
      if (j + R < n) {
        issue(j + R, esA[t], esB[t]);
        mark[t] = issued;
      }
      // S^T of both tiles: lane holds positions 4 lg + jj of head lc
      float4_t sa = float4_t{0.f, 0.f, 0.f, 0.f}, sb = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        sa = M::mfma32(kv[s], qb[s], sa);
        sb = M::mfma32(kv[KS + s], qb[s], sb);
      }
      if (rows_a < 15 || rows_b < 15 || bnull) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          if (4 * lg + jj > rows_a) sa[jj] = -INFINITY;
          if (bnull || 4 * lg + jj > rows_b) sb[jj] = -INFINITY;
        }
      }
      float mx = max3_f32(max_f32(sa[0], sa[1]), sa[2], sa[3]);
      mx = max3_f32(mx, max_f32(sb[0], sb[1]), max_f32(sb[2], sb[3]));
      mx = max_xor32(max_xor16(mx)) * a.scale_log2e;   // finite: tile A holds >= 1 row
      const float m_new = fmaxf(m_run, mx);
      const float alpha = fast_exp2(m_run - m_new);     // 0 while m_run = -inf
      m_run = m_new;
      float pv[8];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        pv[jj] = fast_exp2(fmaf(sa[jj], a.scale_log2e, -m_new));
        pv[4 + jj] = fast_exp2(fmaf(sb[jj], a.scale_log2e, -m_new));
      }
      l_part = fmaf(l_part, alpha, ((pv[0] + pv[1]) + (pv[2] + pv[3])) + ((pv[4] + pv[5]) + (pv[6] + pv[7])));
      const su32x4_t pb = M::pack8(pv);
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn)
        acc[nn] = M::mfma32(su32x4_t{vlo[nn].x, vlo[nn].y, vhi[nn].x, vhi[nn].y}, pb, acc[nn] * alpha);

      if (lastA || lastB || bnull || j + 2 == n) {
        // ---- the unit's end in this worker: its output, or its partial ----
        const float l_tot = sum_xor32(sum_xor16(l_part));   // head lc's sum
        if (eA.w < 0) {
          // lane (lg, lc) holds O^T[16 nn + 4 lg + jj][head lc]
          if (lc < rep) {
            const float inv = 1.f / l_tot;
            char* const orow = a.out + b * a.out_row_bytes + (int64_t)(h * rep + lc) * RB;
            typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
#pragma unroll
            for (int nn = 0; nn < NSL; ++nn) {
              s4_t o;
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) o[jj] = (scalar_t)(acc[nn][jj] * inv);
              st8_through(orow + 2 * (16 * nn + 4 * lg), o);
            }
          }
        } else {
          // a partial: the first one of the range (mid-stream) waits in pst, the one at the
          // range's end in registers, until the workgroup merges its partials
          const int info1 = (((eA.w >> 20) & 0xFF) + 1) | (((eA.w >> 28) & 15) << 8) | (((eA.z >> 24) & 0xFF) << 16);
          const int u = b * a.num_kv_heads + h;
          if (j + 2 < n) {
            save_state(pst, l_tot);
            if (lane == 0) {
              pend_sh[wave][0][0] = u;
              pend_sh[wave][0][1] = info1;
              pend_sh[wave][0][2] = eA.w & 0xFFFFF;
              pend_sh[wave][0][3] = b | (h << 20);
            }
            pend0 = true;
          } else {
            pinfo1[0] = u;
            pinfo1[1] = info1;
            pinfo1[2] = eA.w & 0xFFFFF;
            pinfo1[3] = __float_as_int(l_tot);
            pbh1 = b | (h << 20);
            pend1 = true;
          }
        }
      }
    }
  }

  // ---- partials: merged per workgroup (LDS), then per unit through the L2 ----
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the ring is idle (and the partial loads done)
  if (pend1) save_state(ring, __int_as_float(pinfo1[3]));
  if (lane == 0) {
    if (!pend0) pend_sh[wave][0][0] = -1;
    pend_sh[wave][1][0] = pend1 ? pinfo1[0] : -1;
    pend_sh[wave][1][1] = pinfo1[1];
    pend_sh[wave][1][2] = pinfo1[2];
    pend_sh[wave][1][3] = pbh1;
  }
  __syncthreads();
  constexpr int CPL = (8 * D / 4 + 63) / 64;
  const int n4 = rep * D / 4;
  // this wave's partials and the first-partial unit of each later wave of the
  // workgroup, read together (one LDS round trip)
  const int4 own[2] = {*reinterpret_cast<const int4*>(&pend_sh[wave][0][0]),
                       *reinterpret_cast<const int4*>(&pend_sh[wave][1][0])};
  int mfirst[W];
  mfirst[0] = own[0].x;
#pragma unroll
  for (int m = 1; m < W; ++m) mfirst[m] = pend_sh[min(wave + m, W - 1)][0][0];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int u = __builtin_amdgcn_readfirstlane(own[e].x);
    if (u < 0) continue;
    const int info = __builtin_amdgcn_readfirstlane(own[e].y);
    const int np = info & 0xFF, w0 = (info >> 8) & 0xFF, idx = info >> 16;   // np <= 255
    const int pbase = __builtin_amdgcn_readfirstlane(own[e].z);
    if (idx != 0 && (w0 + idx) % W != 0) continue;   // a member: its group's leader merges it
    // the group: this wave's piece and the next waves' pieces of the unit in this workgroup
    int cnt = 1;
    while (idx + cnt < np && (w0 + idx + cnt) % W != 0) ++cnt;
    const int bh = __builtin_amdgcn_readfirstlane(own[e].w);
    const int b = bh & 0xFFFFF, h = bh >> 20;
    // the members' states (LDS; a member's piece of the unit is its first partial, in pst,
    // or its last, in its ring): the reads of all members in flight at once, then one
    // log-sum-exp per column
    float Mx[CPL], L[CPL];
    float4_t o[CPL];
    {
      const char* stp[W];
#pragma unroll
      for (int m = 0; m < W; ++m) {
        const int w = m < cnt ? wave + m : wave;   // members are the next waves of this workgroup
        const bool first = __builtin_amdgcn_readfirstlane(mfirst[m < cnt ? m : 0]) == u;
        stp[m] = lds_all + w * S::WAVE_LDS + (first ? (int)(pst - ring) : 0);
      }
      float2 ml[CPL][W];
      float4_t v[CPL][W];
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int c = lane + 64 * q;
        const int cc = c < n4 ? c : 0;
        const int head = (4 * cc) / D;
#pragma unroll
        for (int m = 0; m < W; ++m) {
          if (m >= cnt) break;
          ml[q][m] = *reinterpret_cast<const float2*>(stp[m] + 4 * 8 * D + 8 * head);
          v[q][m] = *reinterpret_cast<const float4_t*>(stp[m] + 4 * (head * D + (4 * cc) % D));
        }
      }
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        float mb = -INFINITY;
#pragma unroll
        for (int m = 0; m < W; ++m)
          if (m < cnt) mb = fmaxf(mb, ml[q][m].x);
        float l = 0.f;
        float4_t acc_o = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int m = 0; m < W; ++m) {
          if (m >= cnt) break;
          const float wgt = ml[q][m].y > 0.f ? fast_exp2(ml[q][m].x - mb) : 0.f;
          l = fmaf(ml[q][m].y, wgt, l);
          acc_o += v[q][m] * wgt;
        }
        Mx[q] = mb;
        L[q] = l;
        o[q] = acc_o;
      }
    }
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7;                                    // arrival fields: 8 XCDs of 8 bits (pieces)
    if (cnt == np) {                             // the workgroup held the whole unit
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        const int c = lane + 64 * q;
        if (c >= n4) continue;
        const float inv = 1.f / L[q];
        typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
        s4_t r;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) r[jj] = (scalar_t)(o[q][jj] * inv);
        st8_through(a.out + b * a.out_row_bytes + ((int64_t)h * rep * D + 4 * c) * 2, r);
      }
      continue;
    }
    // the group partial into the slot of its first piece, then counted (cnt pieces)
    const uint32_t p0 = (uint32_t)(pbase + idx) * a.piece_bytes;
#pragma unroll
    for (int q = 0; q < CPL; ++q) {
      const int c = lane + 64 * q;
      const bool act = c < n4;
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(su32x4_t, o[q]), prs, act ? p0 + 16u * c : S_OOB, 0, 0);
      const bool first_col = act && (4 * c) % D == 0;   // one (M, L) per head
      __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(su32x2_t, make_float2(Mx[q], L[q])), prs,
                                            first_col ? p0 + 4u * rep * D + 8u * ((4 * c) / D) : S_OOB, 0, 0);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the group partial is in this XCD's L2
    const unsigned long long mine = (unsigned long long)cnt << (8 * xcc);
    unsigned long long prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(a.arrivals + 16 * (int64_t)u, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const unsigned long long now = __shfl(prev, 0) + mine;
    int arrived = 0;
#pragma unroll
    for (int x = 0; x < 8; ++x) arrived += (int)((now >> (8 * x)) & 0xFF);
    if (arrived == np) {                         // the last group: merge the unit's group partials
      if (now != ((unsigned long long)np << (8 * xcc)) && lane == 0)
        __hip_atomic_fetch_add(a.violations, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      // every group's partial (this one's too, stored above) in group order, whichever
      // group arrived last: the same bits on every call
#pragma unroll
      for (int q = 0; q < CPL; ++q) {
        Mx[q] = -INFINITY;
        L[q] = 0.f;
        o[q] = float4_t{0.f, 0.f, 0.f, 0.f};
      }
      stream_merge<Tag, D, W>(a, b, h, np, pbase, w0, lane, -1, Mx, L, o);
      if (lane == 0)
        __hip_atomic_store(a.arrivals + 16 * (int64_t)u, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

}  // namespace tb

// ---------------------------------------------------------------------------
// Host side: the plan (no device call, nothing allocated) and the launch.

#include <algorithm>
#include <vector>

namespace {

struct stream_layout {
  int workers = 0, max_entries = 0, pieces = 0;
};

constexpr int E_LAST = 1 << 28;   // the unit's last tile
constexpr int SEG_LAST = 1 << 30; // a segment descriptor holds its unit's last tile
constexpr int E_NULL = 1 << 29;   // a padding tile (no positions)

// The assignment of a step's tiles to workers, and (with `entries`) their entries.
// Worker kk of XCD x (kk = gi * waves + w, workgroup g = gi * num_xcds + x, global
// worker g * waves + w) streams tiles [T kk / n, T (k + 1) / n) of the XCD's list;
// each unit segment of its range is padded to an even number of tiles.
int32_t stream_assign(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads, int32_t head_dim,
                      const int32_t* block_tables, int32_t max_blocks_per_seq, int32_t block_size,
                      int64_t num_blocks, int32_t workgroups, int32_t waves, int32_t num_xcds, int32_t unit_cost,
                      int32_t stride, int32_t* counts, int32_t* entries, stream_layout& lay,
                      int32_t* segs = nullptr, int64_t seg_capacity = 0, int64_t* nsegs = nullptr) {
  if (!context_lens || num_seqs < 0 || num_kv_heads <= 0 || workgroups <= 0 || waves <= 0 || waves > 16 ||
      num_xcds <= 0 || num_xcds > 8 || workgroups < num_xcds || (head_dim != 64 && head_dim != 128) ||
      unit_cost < 0 || unit_cost > 64)
    return TB_ERR_INVALID_ARG;
  const int64_t U = (int64_t)num_seqs * num_kv_heads;
  if (num_seqs >= (1 << 20) || num_kv_heads > 16) return TB_ERR_UNSUPPORTED;
  std::vector<int32_t> nt(U);
  for (int b = 0; b < num_seqs; ++b) {
    const int c = context_lens[b];
    if (c <= 0 || c >= (1 << 24)) return TB_ERR_INVALID_ARG;
    for (int h = 0; h < num_kv_heads; ++h) nt[(int64_t)b * num_kv_heads + h] = (c + 15) / 16;
  }
  // units onto XCDs, longest first, to the XCD with the least cost so far
  std::vector<int32_t> order(U);
  for (int64_t u = 0; u < U; ++u) order[u] = (int32_t)u;
  std::stable_sort(order.begin(), order.end(), [&](int32_t x, int32_t y) { return nt[x] > nt[y]; });
  std::vector<int64_t> load(num_xcds, 0);
  std::vector<std::vector<int32_t>> xu(num_xcds);
  for (int32_t u : order) {
    int best = 0;
    for (int x = 1; x < num_xcds; ++x)
      if (load[x] < load[best]) best = x;
    load[best] += nt[u] + unit_cost;
    xu[best].push_back(u);
  }
  const int64_t tb = 16 * 2 * (int64_t)head_dim;                  // bytes of a 16-row K (or V) tile
  const int64_t tile_bytes = tb * (block_size / 16);               // one kv head's K rows of a block
  const int64_t blk_bytes = 2 * (int64_t)num_kv_heads * tile_bytes;
  lay.workers = workgroups * waves;
  lay.max_entries = 0;
  lay.pieces = 0;
  if (counts)
    for (int k = 0; k < lay.workers; ++k) counts[k] = 0;
  // A unit costs its tiles plus unit_cost tile-equivalents (its q rows, padding, output):
  // the XCDs' and the workers' shares are cut on that cost, so workers whose range
  // crosses many short units get fewer tiles. A worker's range is cut in whole tiles
  // and holds at least one while tiles remain, so the workers holding a unit are
  // consecutive (its pieces are workers kk0, kk0 + 1, ...) and idle ones come last.
  for (int x = 0; x < num_xcds; ++x) {
    const int nwg = (workgroups - x + num_xcds - 1) / num_xcds;
    const int64_t nx = (int64_t)nwg * waves;
    int64_t T = 0, Wt = 0;                                          // real tiles, weight
    for (int32_t u : xu[x]) {
      T += nt[u];
      Wt += nt[u] + unit_cost;
    }
    // end[kk]: tiles of the XCD's list (real tiles, in order) that workers 0 .. kk hold
    std::vector<int64_t> end(nx, 0);
    {
      int64_t r = 0, wpos = 0;                                      // real tiles and weight before the unit
      size_t ui = 0;
      std::vector<int32_t>& lst = xu[x];
      for (int64_t kk = 0; kk < nx; ++kk) {
        const int64_t target = Wt * (kk + 1) / nx;                  // the worker's end on the weight axis
        // real tiles whose weighted position (unit's weight offset + tile index) is below target
        while (ui < lst.size()) {
          const int64_t n = nt[lst[ui]];
          if (wpos + n <= target) {
            r += n;
            wpos += n + unit_cost;
            ++ui;
            continue;
          }
          break;
        }
        int64_t e = r + (ui < lst.size() ? std::max<int64_t>(0, std::min<int64_t>(nt[lst[ui]], target - wpos)) : 0);
        const int64_t prev = kk > 0 ? end[kk - 1] : 0;
        if (e <= prev && prev < T) e = prev + 1;                    // at least one tile while tiles remain
        end[kk] = std::min(std::max(e, prev), T);
      }
      end[nx - 1] = T;
    }
    auto start = [&](int64_t kk) { return kk == 0 ? (int64_t)0 : end[kk - 1]; };
    auto worker_of = [&](int64_t t) {                              // the worker whose range holds tile t
      return (int64_t)(std::upper_bound(end.begin(), end.end(), t) - end.begin());
    };
    std::vector<int32_t> cnt(nx, 0);                               // entries per worker, padding included
    int64_t t0 = 0;
    for (int32_t u : xu[x]) {
      const int64_t t1 = t0 + nt[u];
      const int64_t k0 = worker_of(t0), k1 = worker_of(t1 - 1);
      const int np = (int)(k1 - k0 + 1);
      if (np > 255) return TB_ERR_UNSUPPORTED;      // arrival words count pieces in 8-bit fields
      const int base = np > 1 ? lay.pieces : -1;
      if (np > 1) lay.pieces += np;
      if (lay.pieces >= (1 << 20)) return TB_ERR_UNSUPPORTED;
      const int b = u / num_kv_heads, h = u - b * num_kv_heads;
      const int ctx = context_lens[b];
      for (int64_t kk = k0; kk <= k1; ++kk) {
        const int64_t s0 = std::max(t0, start(kk)), s1 = std::min(t1, end[kk]);   // the segment
        const int g = (int)(kk / waves) * num_xcds + x;            // the workgroup, and its wave
        const int k = g * waves + (int)(kk % waves);
        if (segs) {                                                // one descriptor per segment
          if (*nsegs >= seg_capacity) return TB_ERR_INVALID_ARG;
          int32_t* d = segs + 8 * (*nsegs)++;
          d[0] = k;
          d[1] = cnt[kk];                                          // its first entry in the worker's list
          d[2] = b | (h << 20);
          d[3] = (int32_t)(s0 - t0);                               // its first tile of the unit
          d[4] = (int32_t)(s1 - s0) | (s1 == t1 ? SEG_LAST : 0);
          d[5] = ctx;
          d[6] = (int32_t)(kk - k0);                               // piece index
          d[7] = np > 1 ? (base | ((np - 1) << 20) | ((int)(k0 % waves) << 28)) : -1;
        }
        if (!entries) {                                            // counts only
          cnt[kk] += (int32_t)((s1 - s0) + ((s1 - s0) & 1));
          continue;
        }
        for (int64_t t = s0; t < s1 + ((s1 - s0) & 1); ++t) {      // the segment, then a pad if odd
          const bool pad = t >= s1;
          const int64_t tt = pad ? s1 - 1 : t;
          int32_t e[4];
          if (entries) {
            const int tu = (int)(tt - t0);                        // tile of the unit
            const int pos0 = 16 * tu;
            const int bi = pos0 / block_size;
            if (bi >= max_blocks_per_seq) return TB_ERR_INDEX;
            const int32_t blk = block_tables[(int64_t)b * max_blocks_per_seq + bi];
            if (blk < 0 || blk >= num_blocks) return TB_ERR_INDEX;
            const int64_t off = (int64_t)blk * blk_bytes + h * tile_bytes + (int64_t)((pos0 % block_size) / 16) * tb;
            if ((off >> 8) >= ((int64_t)1 << 32)) return TB_ERR_UNSUPPORTED;
            const int rows = std::min(16, ctx - pos0);
            e[0] = (int32_t)(uint32_t)(off >> 8);   // a pad: the segment's last tile (never loaded)
            e[1] = b | (h << 20) | ((rows - 1) << 24) | (!pad && t == t1 - 1 ? E_LAST : 0) | (pad ? E_NULL : 0);
            e[2] = ctx | ((int)(kk - k0) << 24);
            e[3] = np > 1 ? (base | ((np - 1) << 20) | ((int)(k0 % waves) << 28)) : -1;
          }
          const int64_t pos = cnt[kk]++;
          if (entries) {
            if (pos >= stride) return TB_ERR_INVALID_ARG;
            int32_t* d = entries + 4 * ((int64_t)k * stride + pos);
            d[0] = e[0];
            d[1] = e[1];
            d[2] = e[2];
            d[3] = e[3];
          }
        }
      }
      t0 = t1;
    }
    for (int64_t kk = 0; kk < nx; ++kk) {
      if (cnt[kk] > lay.max_entries) lay.max_entries = cnt[kk];
      if (counts) {
        const int g = (int)(kk / waves) * num_xcds + x;
        counts[g * waves + (int)(kk % waves)] = cnt[kk];
      }
    }
  }
  return TB_OK;
}

}  // namespace


namespace tb {

// The tile entries of a decode plan from its segment descriptors (tb_build_decode_segments)
// and the step's block tables on the device: one workgroup per descriptor, a thread per
// entry (the segment's tiles, then a pad that repeats its last tile when the count is
// odd). The same entries tb_build_decode_plan writes on the host. A block id outside
// [0, num_blocks) or past its table is counted in `errors` and replaced by block 0,
// so the decode kernel never reads outside the pool.
__global__ void expand_plan_kernel(const int32_t* segs, const int32_t* tables, int32_t max_blocks_per_seq,
                                   int32_t log2_bs, int64_t num_blocks, int32_t num_kv_heads, int32_t head_dim,
                                   int4* entries, int32_t stride, uint32_t* errors) {
  const int32_t* d = segs + 8 * (int64_t)blockIdx.x;
  const int k = d[0], pos_first = d[1], bh = d[2], tu0 = d[3];
  const int n = d[4] & 0x3FFFFFFF;
  const bool unit_end = d[4] & (1 << 30);
  const int ctx = d[5], piece = d[6], e3 = d[7];
  const int b = bh & 0xFFFFF, h = bh >> 20;
  const int bs = 1 << log2_bs;
  const int64_t tb = 16 * 2 * (int64_t)head_dim;            // bytes of a 16-row K (or V) tile
  const int64_t tile_bytes = tb << (log2_bs - 4);           // one kv head's K rows of a block
  const int64_t blk_bytes = 2 * (int64_t)num_kv_heads * tile_bytes;
  const int nent = n + (n & 1);
  for (int i = threadIdx.x; i < nent; i += blockDim.x) {
    const bool pad = i >= n;
    const int tu = tu0 + (pad ? n - 1 : i);                  // tile of the unit
    const int pos0 = 16 * tu;
    const int bi = pos0 >> log2_bs;
    int32_t blk = bi < max_blocks_per_seq ? tables[(int64_t)b * max_blocks_per_seq + bi] : -1;
    if (blk < 0 || blk >= num_blocks) {
      __hip_atomic_fetch_add(errors, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      blk = 0;
    }
    const int64_t off = (int64_t)blk * blk_bytes + h * tile_bytes + (int64_t)((pos0 & (bs - 1)) >> 4) * tb;
    const int rows = ctx - pos0 < 16 ? ctx - pos0 : 16;
    int4 e;
    e.x = (int32_t)(uint32_t)(off >> 8);
    e.y = b | (h << 20) | ((rows - 1) << 24) | (!pad && unit_end && i == n - 1 ? E_LAST_D : 0) | (pad ? E_NULL_D : 0);
    e.z = ctx | (piece << 24);
    e.w = e3;
    entries[(int64_t)k * stride + pos_first + i] = e;
  }
}

__global__ void xcc_probe_kernel(int32_t* out) {
  unsigned x;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  if (threadIdx.x == 0) out[blockIdx.x] = (int32_t)(x & 0xF);
}

// The compiled (head dim, waves per workgroup) variants and their ring depths; the
// first of each head dim is the default. A workgroup fills one CU (its LDS), so the
// waves are that CU's workers: more waves hide each other's per-step latency, a
// deeper ring keeps more tiles in flight per wave. Head dim 64: four waves with two
// tile pairs in flight each beat eight waves with one (same-box, Qwen layer, fp16,
// 24 pools: 12.1 against 12.9 us per call at 32 sequences, 17.9 against 18.0 at 64).
struct decode_variant {
  int head_dim, waves, ring, unit_cost;
};
constexpr decode_variant DECODE_VARIANTS[] = {
    {64, 4, 4, 8}, {64, 8, 2, 8}, {64, 6, 2, 4}, {128, 4, 2, 4}, {128, 3, 4, 4},
};

template <typename Tag, int D, int W, int R>
static void launch_stream(const stream_args& a, int wgs, hipStream_t stream) {
  hipLaunchKernelGGL((paged_stream_kernel<Tag, D, W, R>), dim3(wgs), dim3(64 * W), 0, stream, a);
}

template <typename Tag>
static bool launch_variant(const stream_args& a, int head_dim, int waves, int wgs, hipStream_t stream) {
  if (head_dim == 64 && waves == 8) launch_stream<Tag, 64, 8, 2>(a, wgs, stream);
  else if (head_dim == 64 && waves == 6) launch_stream<Tag, 64, 6, 2>(a, wgs, stream);
  else if (head_dim == 64 && waves == 4) launch_stream<Tag, 64, 4, 4>(a, wgs, stream);
  else if (head_dim == 128 && waves == 4) launch_stream<Tag, 128, 4, 2>(a, wgs, stream);
  else if (head_dim == 128 && waves == 3) launch_stream<Tag, 128, 3, 4>(a, wgs, stream);
  else return false;
  return true;
}

}  // namespace tb

extern "C" int32_t tb_decode_defaults(int32_t head_dim, int32_t* waves, int32_t* unit_cost) {
  for (const auto& v : tb::DECODE_VARIANTS)
    if (v.head_dim == head_dim) {
      if (waves) *waves = v.waves;
      if (unit_cost) *unit_cost = v.unit_cost;
      return TB_OK;
    }
  return TB_ERR_UNSUPPORTED;
}

extern "C" int32_t tb_decode_variant_supported(int32_t head_dim, int32_t waves) {
  for (const auto& v : tb::DECODE_VARIANTS)
    if (v.head_dim == head_dim && v.waves == waves) return 1;
  return 0;
}

extern "C" int32_t tb_decode_plan_shape(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                                        int32_t head_dim, int32_t workgroups, int32_t waves, int32_t num_xcds,
                                        int32_t unit_cost, int32_t* max_entries, int32_t* pieces) {
  stream_layout lay;
  const int32_t rc = stream_assign(context_lens, num_seqs, num_kv_heads, head_dim, nullptr, 0, 16, 0, workgroups,
                                   waves, num_xcds, unit_cost, 0, nullptr, nullptr, lay);
  if (rc != TB_OK) return rc;
  if (max_entries) *max_entries = lay.max_entries;
  if (pieces) *pieces = lay.pieces;
  return TB_OK;
}

// The plan balances weights (tiles + unit cost per unit), but a worker's time goes by
// its entries, in pairs: when the weight shares round the busiest workers up to an
// extra pair, a unit cost 2 lower that saves >= 5% of the busiest worker's entries is
// used instead. Measured at head dim 64, four waves, 64 / 128 sequences of 513..4096
// positions: 20 -> 18 and 38 -> 36 entries, +1.3..3.7% and +1.2% per call; where the
// entries tie (56 decode rows of a mixed step) the lower cost was 2..6% slower.
extern "C" int32_t tb_decode_unit_cost(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                                       int32_t head_dim, int32_t workgroups, int32_t waves, int32_t num_xcds,
                                       int32_t* unit_cost) {
  if (!unit_cost) return TB_ERR_INVALID_ARG;
  int32_t dw = 0, uc = 0;
  int32_t rc = tb_decode_defaults(head_dim, &dw, &uc);
  if (rc != TB_OK) return rc;
  int32_t me = 0, me_lower = 0;
  rc = tb_decode_plan_shape(context_lens, num_seqs, num_kv_heads, head_dim, workgroups, waves, num_xcds, uc, &me,
                            nullptr);
  if (rc != TB_OK) return rc;
  if (uc >= 2 &&
      tb_decode_plan_shape(context_lens, num_seqs, num_kv_heads, head_dim, workgroups, waves, num_xcds, uc - 2,
                           &me_lower, nullptr) == TB_OK &&
      (int64_t)me_lower * 20 <= (int64_t)me * 19)
    uc -= 2;
  *unit_cost = uc;
  return TB_OK;
}

extern "C" size_t tb_decode_plan_words(int32_t workers, int32_t stride) {
  if (workers <= 0 || stride <= 0) return 0;
  return (size_t)(workers + 3) / 4 * 4 + ((size_t)workers * stride + 64) * 4;
}

extern "C" int32_t tb_build_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                                        int32_t head_dim, const int32_t* block_tables, int32_t max_blocks_per_seq,
                                        int32_t block_size, int64_t num_blocks, int32_t workgroups, int32_t waves,
                                        int32_t num_xcds, int32_t unit_cost, int32_t stride, int32_t* plan,
                                        size_t plan_words) {
  if (!plan || (num_seqs > 0 && !block_tables) || block_size < 16 || (block_size & (block_size - 1)) ||
      stride <= 0 || (stride & 1) || max_blocks_per_seq <= 0 || num_blocks <= 0)
    return TB_ERR_INVALID_ARG;
  if (workgroups <= 0 || waves <= 0) return TB_ERR_INVALID_ARG;
  const int workers = workgroups * waves;
  const size_t need = tb_decode_plan_words(workers, stride);
  if (need == 0 || plan_words < need) return TB_ERR_INVALID_ARG;
  std::fill(plan, plan + need, 0);
  int32_t* const counts = plan;
  int32_t* const entries = plan + (size_t)(workers + 3) / 4 * 4;
  stream_layout lay;
  const int32_t rc = stream_assign(context_lens, num_seqs, num_kv_heads, head_dim, block_tables, max_blocks_per_seq,
                                   block_size, num_blocks, workgroups, waves, num_xcds, unit_cost, stride, counts,
                                   entries, lay);
  if (rc != TB_OK) return rc;
  // Two sequences whose newest positions share a pool slot: the fused append would
  // let each attend to its own new K/V, where the reference's sequential write lets
  // the last one win (kv_cache.py:33-38). Every count word carries the mark (bit
  // 30); the kernel refuses a fused call on such a plan.
  std::vector<int64_t> newest(num_seqs);
  for (int b = 0; b < num_seqs; ++b) {
    const int p = context_lens[b] - 1;
    newest[b] = (int64_t)block_tables[(int64_t)b * max_blocks_per_seq + p / block_size] * block_size + p % block_size;
  }
  std::sort(newest.begin(), newest.end());
  if (std::adjacent_find(newest.begin(), newest.end()) != newest.end())
    for (int k = 0; k < workers; ++k) counts[k] |= TB_DECODE_SHARED_NEWEST;
  return TB_OK;
}

extern "C" int32_t tb_build_decode_segments(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                                            int32_t head_dim, const int32_t* block_tables,
                                            int32_t max_blocks_per_seq, int32_t block_size, int32_t workgroups,
                                            int32_t waves, int32_t num_xcds, int32_t unit_cost, int32_t* counts,
                                            int32_t* segments, int32_t segment_capacity, int32_t* num_segments,
                                            int32_t* max_entries, int32_t* pieces) {
  if (!counts || !segments || !num_segments || segment_capacity <= 0 || workgroups <= 0 || waves <= 0)
    return TB_ERR_INVALID_ARG;
  if (block_tables && (max_blocks_per_seq <= 0 || block_size < 16 || (block_size & (block_size - 1))))
    return TB_ERR_INVALID_ARG;
  const int workers = workgroups * waves;
  stream_layout lay;
  int64_t ns = 0;
  for (int k = 0; k < workers; ++k) counts[k] = 0;
  const int32_t rc = stream_assign(context_lens, num_seqs, num_kv_heads, head_dim, nullptr, 0, 16, 0, workgroups,
                                   waves, num_xcds, unit_cost, 0, counts, nullptr, lay, segments,
                                   segment_capacity, &ns);
  if (rc != TB_OK) return rc;
  *num_segments = (int32_t)ns;
  if (max_entries) *max_entries = lay.max_entries;
  if (pieces) *pieces = lay.pieces;
  if (block_tables) {   // the shared-newest-slot mark, as tb_build_decode_plan
    std::vector<int64_t> newest(num_seqs);
    for (int b = 0; b < num_seqs; ++b) {
      const int p = context_lens[b] - 1;
      if (p / block_size >= max_blocks_per_seq) return TB_ERR_INDEX;
      newest[b] = (int64_t)block_tables[(int64_t)b * max_blocks_per_seq + p / block_size] * block_size + p % block_size;
    }
    std::sort(newest.begin(), newest.end());
    if (std::adjacent_find(newest.begin(), newest.end()) != newest.end())
      for (int k = 0; k < workers; ++k) counts[k] |= TB_DECODE_SHARED_NEWEST;
  }
  return TB_OK;
}

extern "C" int32_t tb_expand_decode_plan(const int32_t* segments, int32_t num_segments, const int32_t* block_tables,
                                         int32_t max_blocks_per_seq, int32_t block_size, int64_t num_blocks,
                                         int32_t num_kv_heads, int32_t head_dim, int32_t workers, int32_t stride,
                                         int32_t* plan, uint32_t* errors, hipStream_t stream) {
  if (num_segments < 0 || workers <= 0 || stride <= 0 || (stride & 1) || num_kv_heads <= 0 || num_kv_heads > 16 ||
      (head_dim != 64 && head_dim != 128) || block_size < 16 || (block_size & (block_size - 1)) ||
      max_blocks_per_seq <= 0 || num_blocks <= 0)
    return TB_ERR_INVALID_ARG;
  if (num_segments == 0) return TB_OK;
  if (!segments || !block_tables || !plan || !errors || (((uintptr_t)plan) & 15u)) return TB_ERR_INVALID_ARG;
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  // every tile offset >> 8 fits the entry's 32 bits
  const int64_t blk_bytes = 2 * (int64_t)num_kv_heads * block_size * 2 * head_dim;
  if (num_blocks > (((int64_t)1 << 40) / blk_bytes)) return TB_ERR_UNSUPPORTED;
  int4* entries = reinterpret_cast<int4*>(plan + (size_t)(workers + 3) / 4 * 4);
  hipLaunchKernelGGL(tb::expand_plan_kernel, dim3(num_segments), dim3(128), 0, stream, segments, block_tables,
                     max_blocks_per_seq, log2_bs, num_blocks, num_kv_heads, head_dim, entries, stride, errors);
  TB_RETURN_LAUNCH_STATUS();
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
                                   int32_t plan_workgroups, int32_t plan_waves, int32_t plan_stride,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                   float scale, int32_t dtype, const void* k_new, int64_t k_row_stride,
                                   const void* v_new, int64_t v_row_stride, void* workspace, size_t workspace_bytes,
                                   int32_t max_pieces, unsigned long long* arrivals, int32_t arrival_units,
                                   uint32_t* violations, const float* rope_cos, const float* rope_sin,
                                   int32_t rope_max_position, hipStream_t stream) {
  using namespace tb;
  if (dtype != TB_DTYPE_F16 && dtype != TB_DTYPE_BF16) return TB_ERR_UNSUPPORTED;
  if (head_dim != 64 && head_dim != 128) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0);
  const int rep = num_heads / num_kv_heads;
  if (rep > 8 || num_kv_heads > 16) return TB_ERR_UNSUPPORTED;
  if (block_size < 16 || (block_size & (block_size - 1))) return TB_ERR_UNSUPPORTED;
  if (!tb_decode_variant_supported(head_dim, plan_waves)) return TB_ERR_UNSUPPORTED;
  int log2_sub = 0;
  while ((16 << log2_sub) < block_size) ++log2_sub;
  TB_CHECK_ARG(num_seqs >= 0 && num_seqs < (1 << 20) && plan_workgroups > 0 && plan_stride > 0 &&
               (plan_stride & 1) == 0 && max_pieces >= 0);
  if (num_seqs == 0) return TB_OK;
  TB_CHECK_ARG(q && pool && out && plan && num_blocks > 0 && violations && arrivals);
  TB_CHECK_ARG((((uintptr_t)q | (uintptr_t)pool | (uintptr_t)out | (uintptr_t)plan) & 15u) == 0);
  TB_CHECK_ARG(q_row_stride >= (int64_t)num_heads * head_dim && out_row_stride >= (int64_t)num_heads * head_dim);
  TB_CHECK_ARG((q_row_stride * 2) % 16 == 0 && (out_row_stride * 2) % 16 == 0);
  // the V rows of a tile lie num_kv_heads tiles past its K rows (a 32-bit offset)
  TB_CHECK_ARG((int64_t)num_kv_heads * block_size * head_dim * 2 < ((int64_t)1 << 31));
  const size_t piece = tb_paged_decode_piece_bytes(num_heads, num_kv_heads, head_dim);
  const size_t need = tb_paged_decode_workspace_bytes(max_pieces, num_heads, num_kv_heads, head_dim);
  TB_CHECK_ARG(max_pieces == 0 || (workspace != nullptr && workspace_bytes >= need));
  TB_CHECK_ARG((((uintptr_t)workspace) & 127u) == 0);
  TB_CHECK_ARG((size_t)max_pieces * piece < ((size_t)1 << 31));
  TB_CHECK_ARG(arrival_units >= num_seqs * num_kv_heads && (((uintptr_t)arrivals) & 127u) == 0);
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
  const int workers = plan_workgroups * plan_waves;
  stream_args a;
  a.q = (const char*)q;
  a.q_row_bytes = q_row_stride * 2;
  a.pool = (char*)pool;
  a.num_blocks = num_blocks;
  a.out = (char*)out;
  a.out_row_bytes = out_row_stride * 2;
  a.counts = plan;
  a.entries = reinterpret_cast<const int4*>(plan + (size_t)(workers + 3) / 4 * 4);
  a.stride = plan_stride;
  a.workers = workers;
  a.pieces = (char*)workspace;
  a.pieces_bytes = (uint32_t)((size_t)max_pieces * piece);
  a.piece_bytes = (int32_t)piece;
  a.arrivals = arrivals;
  a.violations = violations;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.rep = rep;
  a.log2_sub = log2_sub;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.k_new = (const char*)k_new;
  a.k_new_row_bytes = k_row_stride * 2;
  a.v_new = (const char*)v_new;
  a.v_new_row_bytes = v_row_stride * 2;
  a.rope = rope_tables{rope_cos, rope_sin, rope_max_position};
  const bool ok = dtype == TB_DTYPE_F16 ? launch_variant<f16_t>(a, head_dim, plan_waves, plan_workgroups, stream)
                                        : launch_variant<bf16_t>(a, head_dim, plan_waves, plan_workgroups, stream);
  if (!ok) return TB_ERR_UNSUPPORTED;
  TB_RETURN_LAUNCH_STATUS();
}
