// K2 — fused paged attention (decode rows and any other query row).
//
// Replaces the per-sequence loop of Qwen2Paged.forward
// (reference src/tinybatch/model.py:130-147): gather of the sequence's blocks
// (kv_cache.py:40-45), GQA repeat_interleave (model.py:135-137), the
// offset-causal mask j <= ctx - q_len + i (model.py:139-145) and
// scaled_dot_product_attention with scale 1/sqrt(D) (model.py:140,146).
//
// Work decomposition: one workgroup = one work item = (query rows of one
// sequence, kv head, head group, partition of P positions). Each K/V row of the
// partition is read once, in place through the block table, and serves every
// query head of the GQA group (no repeat_interleave, no gathered copy). A row
// longer than P is split over several workgroups that store (max, sum,
// unnormalised acc) partials; combine_partials_kernel merges them with a
// log-sum-exp (the kernel boundary makes the partials visible across XCDs).
//
// fp16 / bf16 (the hot path): paged_attn_mfma_kernel, P/CT waves of CT
// positions each, every wave issuing all of its loads at once. The GQA group
// (up to 16 heads, padded) is one MFMA operand, so q.K^T and p.V are
// v_mfma_f32_16x16x32_{f16,bf16} over 16-position tiles:
//   S^T[pos][head] = K[pos][:] . Q[head][:]   A = K rows straight from the pool
//                                              B = q (registers, loaded once)
//   O[head][dv]   += P[head][pos] . V[pos][dv] A = p (the S^T tile registers,
//                                              repacked in place), B = V rows
//                                              loaded into LDS directly, read
//                                              transposed
// and the waves' softmax states merge in LDS.
// Prefill tiles (fp16 / bf16): paged_prefill_mfma_kernel, a flash-style
// workgroup per (64 query rows of one sequence, query head) that walks the
// causal range in 64-position chunks staged in LDS (see the kernel).
// fp32: paged_attn_valu_kernel, fp32 FMAs on the VALU (no fp32 MFMA of the
// needed precision on CDNA4), same decomposition.
// Positions >= the row's context are never loaded from the pool (stale slots
// may hold any bits, NaN included): their scores are -inf, so p = 0, and what
// stands in for their V rows is finite.
#include <atomic>
#include <mutex>

#include "tb_common.h"

namespace tb {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf168_t __attribute__((ext_vector_type(8)));

template <typename Tag>
struct math;

template <>
struct math<f16_t> {
  typedef _Float16 scalar_t;
  typedef half8_t vec8_t;
  static __device__ __forceinline__ float4_t mfma(vec8_t a, vec8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct math<bf16_t> {
  typedef __bf16 scalar_t;
  typedef bf168_t vec8_t;
  static __device__ __forceinline__ float4_t mfma(vec8_t a, vec8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};

constexpr int PART16 = 256;   // partition length of the 16-bit kernel (positions)

struct attn_args {
  const char* q;          // [rows][Hq][D]
  int64_t q_row_bytes;
  char* pool;             // [NB][2][Hkv][BS][D]
  int64_t num_blocks;
  char* out;              // [rows][Hq*D]
  int64_t out_row_bytes;
  const int32_t* block_tables;
  int32_t max_nb;
  const int4* work;       // (row, seq, part, row_ctx)
  const int32_t* row_part_off;
  const int4* tiles;      // prefill tiles (row0, seq, rows, pos0)
  const int4* split_rows;  // (row, first partial slot, partial count, 0)
  const int32_t* counts;  // optional: work items, split rows, tiles present (grids are capacities)
  float* ws_acc;          // [parts][Hq][D]
  float* ws_ml;           // [parts][Hq][2]
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t rep;            // num_heads / num_kv_heads
  int32_t group;          // heads per wave (grid z = rep / group)
  int32_t log2_bs;
  int32_t part_tokens;
  float scale_log2e;
  const char* k_new;      // fused decode append (may be null)
  int64_t k_new_row_bytes;
  const char* v_new;
  int64_t v_new_row_bytes;
  rope_tables rope;       // rope.cos != null: q (and a fused append's K) rotated at position row_ctx - 1
  // split rows merged inside the launch (tb_paged_attention_merged; null otherwise):
  const int32_t* slot_map;          // grid slot -> item * num_kv_heads + kv head, or -1
  unsigned long long* arrivals;     // per (first row of an item, kv head), 128 bytes apart, zero between launches
  uint32_t* violations;             // incremented when a row group's partials ran on more than one XCD
  uint32_t ws_bytes;                // the workspace bytes addressable through a buffer resource
  int32_t num_work;                 // work items (bounds the slot map's values)
};


// ---------------------------------------------------------------------------
// fp32 path: single pass, online softmax per chunk, fp32 FMAs.
template <typename Tag, int D>
struct valu_shape {
  static constexpr int EB = elem<Tag>::bytes;
  static constexpr int EPL = 16 / EB;     // elements per lane per load
  static constexpr int LPT = D / EPL;     // lanes per token row
  static constexpr int TPL = 64 / LPT;    // tokens per wave load
  static constexpr int CH_LOADS = 8;      // wave loads of K (and of V) per chunk
  static constexpr int CH = CH_LOADS * TPL;  // tokens per chunk
  static_assert(LPT >= 1 && LPT <= 64 && (64 % LPT) == 0, "lane split");
};

// End of a VALU work item. acc[h][e] holds, in lanes 0..LPT-1 (column j = lane),
// the unnormalised output of head h over the partition for dims j*EPL..;
// m[h] / l[h] (wave-uniform) are its max (base-2 domain) and sum. One
// partition: write the output. Several: write the partial for the combine.
template <typename Tag, int D, int REP, int EPL, int LPT>
__device__ __forceinline__ void finish_valu(const attn_args& a, int row, int part, int head0, int lane,
                                            float (&acc)[REP][EPL], const float (&m)[REP],
                                            const float (&l)[REP]) {
  const int j = lane % LPT;
  if (lane >= LPT) return;
  const int pbeg = a.row_part_off[row];
  const int nparts = a.row_part_off[row + 1] - pbeg;
  if (nparts == 1) {
    char* orow = a.out + row * a.out_row_bytes + j * 16;
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      const float inv = 1.f / l[h];
      vec16 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o.w[e] = __float_as_uint(acc[h][e] * inv);
      st16_through(orow + (int64_t)(head0 + h) * D * 4, o);
    }
    return;
  }
  const int64_t pidx = pbeg + part;
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float* dst = a.ws_acc + (pidx * a.num_heads + head0 + h) * D + j * EPL;
#pragma unroll
    for (int e = 0; e < EPL; e += 4)
      *reinterpret_cast<float4*>(dst + e) = make_float4(acc[h][e], acc[h][e + 1], acc[h][e + 2], acc[h][e + 3]);
  }
  if (lane == 0) {
#pragma unroll
    for (int h = 0; h < REP; ++h)
      *reinterpret_cast<float2*>(a.ws_ml + (pidx * a.num_heads + head0 + h) * 2) = make_float2(m[h], l[h]);
  }
}

template <typename Tag, int D, int REP>
__global__ __launch_bounds__(64) void paged_attn_valu_kernel(const attn_args a) {
  using S = valu_shape<Tag, D>;
  constexpr int EB = S::EB, EPL = S::EPL, LPT = S::LPT, TPL = S::TPL;
  constexpr int CH_LOADS = S::CH_LOADS, CH = S::CH;
  static_assert(EB == 4, "the 16-bit types use paged_attn_mfma_kernel");

  const int lane = threadIdx.x;
  const int j = lane % LPT;  // 16-byte column of the token row
  const int g = lane / LPT;  // token slot inside one wave load

  const int4 wi = a.work[blockIdx.x];   // one row per item on this path; the array holds the grid's capacity
  if (a.counts && (int)blockIdx.x >= a.counts[0]) return;   // beyond this step's work items
  const int row = wi.x, seq = wi.y, part = wi.z & 0xFFFFFF, ctx = wi.w;
  const int kvh = blockIdx.y;
  const int head0 = kvh * a.rep + blockIdx.z * REP;

  const int p0 = part * a.part_tokens;
  const int p1 = min(p0 + a.part_tokens, ctx);
  const int bs = 1 << a.log2_bs;

  // Block-table entries of this partition: lane l holds entry p0/BS + l.
  const int blk_first = p0 >> a.log2_bs;
  const int blk_count = ((p1 - 1) >> a.log2_bs) - blk_first + 1;  // <= 64 (host-checked)
  int my_blk = 0;
  if (lane < blk_count) {
    my_blk = a.block_tables[(int64_t)seq * a.max_nb + blk_first + lane];
    if (my_blk < 0 || my_blk >= a.num_blocks) my_blk = 0;  // host validates; stay inside the pool
  }

  const int64_t tile_bytes = (int64_t)bs * D * EB;
  const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * tile_bytes;
  const int64_t v_off = (int64_t)a.num_kv_heads * tile_bytes;
  const char* pool_kvh = a.pool + kvh * tile_bytes + j * 16;
  const int new_pos = ctx - 1;
  const bool fused = (a.k_new != nullptr);
  const char* k_new_row = fused ? a.k_new + row * a.k_new_row_bytes + (int64_t)kvh * D * EB + j * 16 : nullptr;
  const char* v_new_row = fused ? a.v_new + row * a.v_new_row_bytes + (int64_t)kvh * D * EB + j * 16 : nullptr;

  vec16 qv[REP];
  {
    const char* qrow = a.q + row * a.q_row_bytes + j * 16;
#pragma unroll
    for (int h = 0; h < REP; ++h) qv[h] = ld16(qrow + (int64_t)(head0 + h) * D * EB);
  }
  // RoPE: chunk j of the first half pairs with chunk j + LPT/2 of the second,
  // held by lane ^ LPT/2 of the same token slot (every lane holds its chunk)
  vec16 k_new_rot = zero16();
  if (a.rope.cos) {
    const bool first = j < LPT / 2;
    const int64_t r = a.rope.row(ctx - 1, D / 2) + (first ? j : j - LPT / 2) * 4;
    auto rotate = [&](vec16& x) {
      vec16 y;
#pragma unroll
      for (int e = 0; e < 4; ++e) y.w[e] = (uint32_t)__shfl_xor((int)x.w[e], LPT / 2);
      if (first) rope_pair<float>(x, y, a.rope.cos + r, a.rope.sin + r);
      else rope_pair<float>(y, x, a.rope.cos + r, a.rope.sin + r);
    };
#pragma unroll
    for (int h = 0; h < REP; ++h) rotate(qv[h]);
    if (fused) {
      k_new_rot = ld16(k_new_row);
      rotate(k_new_rot);
    }
  }

  float m_run[REP], l_run[REP], acc[REP][EPL];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }

  int64_t new_off = 0;
  if (fused) {
    const int nb = __shfl(my_blk, ((new_pos - p0) >> a.log2_bs) & 63);
    new_off = (int64_t)nb * blk_bytes + (int64_t)(new_pos & (bs - 1)) * (D * EB);
  }

  for (int c0 = p0; c0 < p1; c0 += CH) {
    vec16 kbuf[CH_LOADS], vbuf[CH_LOADS];
#pragma unroll
    for (int i = 0; i < CH_LOADS; ++i) {
      const int tau = c0 + i * TPL + g;
      const int blk = __shfl(my_blk, ((tau - p0) >> a.log2_bs) & 63);
      const int64_t off = (int64_t)blk * blk_bytes + (int64_t)(tau & (bs - 1)) * (D * EB);
      const char* kp = pool_kvh + off;
      const char* vp = kp + v_off;
      if (fused && tau == new_pos) { kp = k_new_row; vp = v_new_row; }
      if (tau < p1) { kbuf[i] = ld16(kp); vbuf[i] = ld16(vp); }
      else { kbuf[i] = zero16(); vbuf[i] = zero16(); }
      if (fused && a.rope.cos && tau == new_pos) kbuf[i] = k_new_rot;
    }
    if (fused) {
#pragma unroll
      for (int i = 0; i < CH_LOADS; ++i) {
        if (c0 + i * TPL + g == new_pos) {
          char* kp = const_cast<char*>(pool_kvh) + new_off;
          st16_through(kp, kbuf[i]);
          st16_through(kp + v_off, vbuf[i]);
        }
      }
    }
    float s[CH_LOADS][REP];
#pragma unroll
    for (int i = 0; i < CH_LOADS; ++i) {
      const bool valid = (c0 + i * TPL + g) < p1;
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) d = fmaf(bits_to_f32(qv[h].w[e]), bits_to_f32(kbuf[i].w[e]), d);
        d = group_sum<LPT>(d);
        s[i][h] = valid ? d * a.scale_log2e : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float cm = s[0][h];
#pragma unroll
      for (int i = 1; i < CH_LOADS; ++i) cm = fmaxf(cm, s[i][h]);
      cm = cross_group_max<LPT>(cm);
      const float m_new = fmaxf(m_run[h], cm);
      const float alpha = fast_exp2(m_run[h] - m_new);
      m_run[h] = m_new;
      l_run[h] *= alpha;
#pragma unroll
      for (int e = 0; e < EPL; ++e) acc[h][e] *= alpha;
    }
#pragma unroll
    for (int i = 0; i < CH_LOADS; ++i) {
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        const float p = fast_exp2(s[i][h] - m_run[h]);
        l_run[h] += p;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[h][e] = fmaf(p, bits_to_f32(vbuf[i].w[e]), acc[h][e]);
      }
    }
  }

  // l was accumulated per token slot; sum over the slots like acc
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    l_run[h] = cross_group_sum<LPT>(l_run[h]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = cross_group_sum<LPT>(acc[h][e]);
  }
  finish_valu<Tag, D, REP, EPL, LPT>(a, row, part, head0, lane, acc, m_run, l_run);
}

// ---------------------------------------------------------------------------
// 16-bit kernel (see the file header). A workgroup of NW waves owns one
// partition of P positions; wave w takes positions [w*CT, (w+1)*CT) and issues
// all of its K and V loads at once, so a whole partition is in flight. The
// waves' (max, sum, acc) are merged in LDS; one partial (or the output) leaves
// the workgroup. Lane l = 16*lg + lc.
// MFMA 16x16x32 operand layouts (gfx950): A lane l holds A[l%16][8*(l/16)+j],
// B lane l holds B[8*(l/16)+j][l%16], C/D lane l holds D[4*(l/16)+j][l%16].
template <int D>
struct mfma_shape {
  static constexpr int RB = D * 2;           // bytes per K or V row
  static constexpr int KS = D / 32;          // q.k k-slices (32 dims each)
  static constexpr int NSL = D / 16;         // p.V output slices (16 dims each)
  static constexpr int P = PART16;
  static constexpr int CT = 8192 / RB;       // positions per wave (8 KB of K, 8 KB of V)
  static constexpr int NW = P / CT;          // waves per workgroup
  static constexpr int TILES = CT / 16;      // 16-position tiles per wave
  static constexpr int VCOLS = RB / 16;      // 16-byte columns of a row
  static constexpr int VT = 64 / VCOLS;      // rows per V load instruction
  static constexpr int VLD = CT / VT;        // V loads per lane
  // V rows of a wave pass through LDS in VPH phases of CT / VPH rows. With
  // two phases (D = 64) the first half is loaded straight into LDS and the
  // second half into registers, written over the first once that is consumed:
  // 16 KB of LDS per workgroup instead of 32, so five workgroups fit on a CU
  // instead of four.
  static constexpr int VPH = (TILES % 4 == 0) ? 2 : 1;
  static constexpr int VDMA = VLD / VPH;     // V loads per lane that go straight to LDS
  static constexpr int VST = CT * RB / VPH;  // LDS bytes of V per wave
  static constexpr int MERGE = 16 * D * 4;   // per-wave acc bytes in the merge
  static constexpr int ML = NW * 16 * 8;     // per-column (max, sum) of every wave, after the acc area
  static constexpr int LDS = (NW * VST > NW * MERGE + ML) ? NW * VST : NW * MERGE + ML;
  static_assert(TILES % 2 == 0 && P % CT == 0 && VT * RB == 1024 && VLD % VPH == 0, "chunk shape");
  // V row r of a wave keeps its 16-byte chunk c in slot c ^ swz(r): the transpose
  // reads of P.V (4 rows x 32 bytes per 16 lanes) then hit distinct banks.
  static __device__ __forceinline__ int swz(int r) { return 2 * (r & 3); }
};

// Loads of one kv head's K/V rows. UT ("uniform tiles", block_size >= 16):
// every 16-position K tile and every V row group of a wave lies inside one
// block, so the block id and the tile base are wave-uniform (a scalar table
// read and scalar address arithmetic per tile); otherwise each lane looks its
// block up in a per-lane copy of the partition's table entries.
// Split rows merged inside the launch (tb_paged_attention_merged). All partitions
// of a row group and kv head ran on one XCD (the slot map places them so), whose
// L2 every CU of the XCD shares: once a workgroup's partials are acknowledged by
// the L2 it counts itself in the group's arrival word (8-bit fields per XCD, so a
// partition that ran elsewhere is detected and reported), and the workgroup whose
// partition arrives last merges the nparts partials of every (row, head) of the
// item with L1-bypassing loads, as combine_partials_kernel does, and writes the
// output. It leaves the arrival word zero for the next launch.
template <typename Tag, int D>
__device__ __forceinline__ void merge_in_launch(const attn_args& a, int row0, int kvh, int head0, int R, int ncols,
                                                int pbeg0, int nparts) {
  typedef typename math<Tag>::scalar_t scalar_t;
  constexpr int NT = 64 * mfma_shape<D>::NW;
  constexpr int BATCH = 8;                       // as combine_partials_kernel: the same bits
  __shared__ int last;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this thread's partial stores are in the L2
  __syncthreads();
  unsigned long long* const word = a.arrivals + 16 * ((int64_t)row0 * a.num_kv_heads + kvh);
  if (threadIdx.x == 0) {
    unsigned xcc;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    xcc &= 7;
    const unsigned long long mine = 1ull << (8 * xcc);
    const unsigned long long now = __hip_atomic_fetch_add(word, mine, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + mine;
    int arrived = 0;
#pragma unroll
    for (int x = 0; x < 8; ++x) arrived += (int)((now >> (8 * x)) & 0xFF);
    const bool is_last = arrived == nparts;
    if (is_last && now != ((unsigned long long)nparts << (8 * xcc)))
      __hip_atomic_fetch_add(a.violations, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = is_last;
  }
  __syncthreads();
  if (!last) return;
  const auto rs = __builtin_amdgcn_make_buffer_rsrc(a.ws_acc, 0, a.ws_bytes, 0x00020000);
  const uint32_t ml_base = (uint32_t)((const char*)a.ws_ml - (const char*)a.ws_acc);
  for (int idx = threadIdx.x; idx < ncols * (D / 4); idx += NT) {
    const int h = idx / (D / 4), d4 = idx - h * (D / 4);
    const int row = row0 + h / R, head = head0 + h - (h / R) * R;
    const int pfirst = pbeg0 + (h / R) * nparts;
    float M = -INFINITY, L = 0.f;
    float4_t o = float4_t{0.f, 0.f, 0.f, 0.f};
    for (int p0 = 0; p0 < nparts; p0 += BATCH) {
      float2 ml[BATCH];
      float4_t av[BATCH];
#pragma unroll
      for (int k = 0; k < BATCH; ++k) {
        ml[k] = make_float2(-INFINITY, 0.f);
        av[k] = float4_t{0.f, 0.f, 0.f, 0.f};
        if (p0 + k < nparts) {
          const uint32_t slot = (uint32_t)(pfirst + p0 + k) * a.num_heads + head;
          ml[k] = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(rs, ml_base + 8u * slot, 0, LOAD_DEVICE_SCOPE));
          av[k] = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, 4u * (slot * D + 4 * d4), 0, LOAD_DEVICE_SCOPE));
        }
      }
      float mb = M;
#pragma unroll
      for (int k = 0; k < BATCH; ++k) mb = fmaxf(mb, ml[k].x);
      const float keep = fast_exp2(M - mb);   // 0 while M = -inf
      L *= keep;
      o *= keep;
#pragma unroll
      for (int k = 0; k < BATCH; ++k) {
        const float w = ml[k].y > 0.f ? fast_exp2(ml[k].x - mb) : 0.f;
        L = fmaf(ml[k].y, w, L);
        o += av[k] * w;
      }
      M = mb;
    }
    const float inv = 1.f / L;
    typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
    s4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = (scalar_t)(o[j] * inv);
    st_through(a.out + row * a.out_row_bytes + ((int64_t)head * D + 4 * d4) * 2, r);
  }
  if (threadIdx.x == 0) __hip_atomic_store(word, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename Tag, int D, bool UT>
__device__ __forceinline__ void decode_items_body(const attn_args& a, char* const lds, const int bx, const int bz) {
  using S = mfma_shape<D>;
  using M = math<Tag>;
  typedef typename M::vec8_t vec8_t;
  typedef typename M::scalar_t scalar_t;
  constexpr int RB = S::RB, KS = S::KS, NSL = S::NSL, P = S::P, CT = S::CT, NW = S::NW;
  constexpr int TILES = S::TILES, VCOLS = S::VCOLS, VT = S::VT, VLD = S::VLD;

  float2 (*const ml_lds)[16] = reinterpret_cast<float2 (*)[16]>(lds + NW * S::MERGE);

  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int lc = lane & 15, lg = lane >> 4;
  // Work item: rows row0 .. row0+nrows-1 of one sequence (consecutive query
  // rows, row_ctx ctx0, ctx0+1, ...), one partition. The 16 MFMA columns are
  // (row, head) pairs: column c = qi*R + h. Decode rows come one per item.
  // The kv head varies fastest across the grid: the workgroups reading the K
  // and V tiles of the same blocks for the two (or more) kv heads run side by
  // side, so each block's bytes are fetched close together in time.
  // the grid slot's item and kv head (a slot map places every partition of a split row
  // group on one XCD, for the merge inside the launch; slots past the work hold -1)
  const int slot_v = a.slot_map ? a.slot_map[bx] : bx;
  if (slot_v < 0 || (a.slot_map && slot_v >= a.num_work * a.num_kv_heads)) return;   // whole workgroup
  const int item = slot_v / a.num_kv_heads;
  const int kvh = slot_v - item * a.num_kv_heads;
  const int4 wi = a.work[item];                  // the array holds the grid's capacity
  if (a.counts && item >= a.counts[0]) return;   // whole workgroup: beyond this step's items
  const int row0 = wi.x, seq = wi.y, part = wi.z & 0xFFFFFF, nrows = (wi.z >> 24) + 1, ctx0 = wi.w;
  const int R = a.group;                    // heads of this workgroup; nrows * R <= 16
  const int head0 = kvh * a.rep + bz * R;
  const int p0 = part * P;
  const int n = min(P, ctx0 + nrows - 1 - p0);   // positions visible to the last row (>= 1)
  const int ctx = ctx0;                     // the single decode row's context (fused append)
  const int ncols = nrows * R;
  const int qi = lc / R;                    // this lane's column: row qi, head lc - qi*R
  const int n_col = lc < ncols ? min(P, ctx0 + qi - p0) : n;   // positions visible to the column
  const int wb = wave * CT;                // this wave's first position (partition-relative)
  const bool busy = wb < n;                // wave 0 always is
  const int bs = 1 << a.log2_bs;

  const int64_t tile_bytes = (int64_t)bs * RB;
  const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * tile_bytes;
  const int64_t v_off = (int64_t)a.num_kv_heads * tile_bytes;
  char* const pool_kvh = a.pool + kvh * tile_bytes;
  const bool fused = (a.k_new != nullptr);
  const int new_tau = ctx - 1 - p0;         // partition-relative index of the newest position
  const char* k_new_row = fused ? a.k_new + row0 * a.k_new_row_bytes + (int64_t)kvh * RB : nullptr;
  const char* v_new_row = fused ? a.v_new + row0 * a.v_new_row_bytes + (int64_t)kvh * RB : nullptr;

  // Pool addresses: K tile t (A operand: lane holds position wb+16t+lc, bytes
  // 64s+16lg) and V row group i (16-byte column lane%VCOLS of row VT*i + lane/VCOLS),
  // recomputed where used so that no per-lane 64-bit pointer stays live.
  char* tile_base[TILES];   // UT: wave-uniform start of tile t in the pool
  int my_blk = 0;           // otherwise: lane l holds the partition's table entry p0/BS + l
  if constexpr (UT) {
    const int32_t* tbl = a.block_tables + (int64_t)seq * a.max_nb;
    const int wbu = __builtin_amdgcn_readfirstlane(wb);
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int pt = p0 + wbu + 16 * t;     // the tile's first position (wave-uniform)
      int blk = 0;
      if (wbu + 16 * t < n) {               // entries past the context are never read
        blk = tbl[pt >> a.log2_bs];
        if (blk < 0 || blk >= a.num_blocks) blk = 0;   // host validates; stay inside the pool
      }
      tile_base[t] = pool_kvh + (int64_t)blk * blk_bytes + (int64_t)(pt & (bs - 1)) * RB;
    }
  } else {
    const int blk_count = ((n - 1) >> a.log2_bs) + 1;   // <= 64: BS >= 4
    if (lane < blk_count) {
      my_blk = a.block_tables[(int64_t)seq * a.max_nb + (p0 >> a.log2_bs) + lane];
      if (my_blk < 0 || my_blk >= a.num_blocks) my_blk = 0;
    }
  }
  auto pos_off = [&](int tau) -> int64_t {   // generic path; shuffles: every lane runs it
    const int blk = __shfl(my_blk, (tau >> a.log2_bs) & 63);
    return (int64_t)blk * blk_bytes + (int64_t)(tau & (bs - 1)) * RB;
  };
  auto k_at = [&](int t) -> char* {
    if constexpr (UT) return tile_base[t] + (lc * RB + 16 * lg);
    else return pool_kvh + pos_off(wb + 16 * t + lc) + 16 * lg;
  };
  auto v_row = [&](int i) -> char* {   // pool address of V row VT*i + lane/VCOLS of the wave
    if constexpr (UT) return tile_base[(VT * i) / 16] + (v_off + ((VT * i) % 16 + lane / VCOLS) * RB);
    else return pool_kvh + v_off + pos_off(wb + VT * i + lane / VCOLS);
  };

  // q first (vector loads retire in order: S^T = K.Q^T can start while V is
  // still in flight); the B operand of S^T: lane holds q[row0+qi][head0+h][32s + 8lg .. +8].
  vec16 qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qb[s] = zero16();
  if (lc < ncols) {
    const char* qrow = a.q + (row0 + qi) * a.q_row_bytes + (int64_t)(head0 + lc - qi * R) * RB + 16 * lg;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = ld16(qrow + 64 * s);
  }
  // All of the wave's K and V loads are issued now, unconditionally: a lane
  // whose position lies past the context reads 16 bytes of q instead (a cache
  // hit, finite values that meet p = 0). A predicated load would put a branch
  // and a copy of the loaded value in between, and that copy waits for the
  // load. K goes to registers (the A operand of S^T = K.Q^T); V goes straight
  // to this wave's LDS rows (global_load_lds: lane l of load i fills bytes
  // 16 l .. 16 l + 15 of the i-th KiB), swizzled per row. The fused append's
  // newest position is read from k_new/v_new.
  char* const vl = lds + wave * S::VST;
  vec16 kd[TILES][KS];
  vec16 vr[VLD > S::VDMA ? VLD - S::VDMA : 1];   // second-phase V rows (registers)
  if (busy) {
    const char* const dummy = a.q;
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      const int tau = wb + 16 * t + lc;
      const char* const kp = k_at(t);   // on every lane: the generic lookup is a shuffle
      const char* src = tau >= n ? dummy : (fused && tau == new_tau) ? k_new_row + 16 * lg : kp;
#pragma unroll
      for (int s = 0; s < KS; ++s) kd[t][s] = ld16_stream(src + 64 * s);
    }
#pragma unroll
    for (int i = 0; i < VLD; ++i) {
      const int r = VT * i + lane / VCOLS;                  // wave-relative row
      const int c = (lane % VCOLS) ^ S::swz(r);             // the row's chunk this lane's slot holds
      const int tau = wb + r;
      const char* const vp = v_row(i);
      const char* src = tau >= n ? dummy + 16 * c : (fused && tau == new_tau) ? v_new_row + 16 * c : vp + 16 * c;
      if (i < S::VDMA)
        __builtin_amdgcn_global_load_lds((const __attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(vl + 1024 * i), 16, 0, 2);
      else
        vr[i - S::VDMA] = ld16_stream(src);
    }
  }
  // Read now what the tail needs, so that no workgroup ends on a memory round
  // trip: the item's first partial slot and partition count (the item's rows
  // are consecutive with equal counts, so row row0 + i starts at pbeg0 + i *
  // nparts) and, for the wave holding the fused append's newest position, its
  // block id.
  const int pbeg0 = a.row_part_off[row0];
  const int nparts = a.row_part_off[row0 + 1] - pbeg0;
  const bool stores_new = fused && bz == 0 && new_tau >= wb && new_tau < wb + CT;   // wave-uniform
  int new_blk = 0;
  if (stores_new) {
    new_blk = a.block_tables[(int64_t)seq * a.max_nb + ((ctx - 1) >> a.log2_bs)];
    if (new_blk < 0 || new_blk >= a.num_blocks) new_blk = 0;   // host validates; stay inside the pool
  }
  // every load is issued before the first use of K (the scheduler would
  // otherwise sink direct loads below the wait for K, serialising V behind it)
  __builtin_amdgcn_sched_barrier(0);

  // RoPE: slice s (dims 32s + 8lg ..) of the first half pairs with slice
  // s + KS/2 of the second in the same lane, for q and for the K row of the
  // fused append's newest position
  if (a.rope.cos) {
    if (lc < ncols) {
      const int64_t r = a.rope.row(ctx0 + qi - 1, D / 2) + 8 * lg;
#pragma unroll
      for (int s = 0; s < KS / 2; ++s)
        rope_pair<scalar_t>(qb[s], qb[s + KS / 2], a.rope.cos + r + 32 * s, a.rope.sin + r + 32 * s);
    }
    if (fused && busy) {
      const int64_t r = a.rope.row(ctx - 1, D / 2) + 8 * lg;
#pragma unroll
      for (int t = 0; t < TILES; ++t)
        if (wb + 16 * t + lc == new_tau) {
#pragma unroll
          for (int s = 0; s < KS / 2; ++s)
            rope_pair<scalar_t>(kd[t][s], kd[t][s + KS / 2], a.rope.cos + r + 32 * s, a.rope.sin + r + 32 * s);
        }
    }
  }

  float m_w = -INFINITY;     // max of head lc over this wave's positions (base-2 domain)
  float l_part = 0.f;        // this lane's share of head lc's sum
  float4_t acc[NSL];         // O[head 4lg+j][16n + lc]
#pragma unroll
  for (int nn = 0; nn < NSL; ++nn) acc[nn] = float4_t{0.f, 0.f, 0.f, 0.f};
  float4_t sc[TILES];        // S^T, then P: lane holds positions 16t + 4lg + j of head lc

  if (busy) {
#pragma unroll
    for (int t = 0; t < TILES; ++t) {
      sc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sc[t] = M::mfma(__builtin_bit_cast(vec8_t, kd[t][s]), __builtin_bit_cast(vec8_t, qb[s]), sc[t]);
    }
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        sc[t][j] = (wb + 16 * t + 4 * lg + j) < n_col ? sc[t][j] * a.scale_log2e : -INFINITY;
    float cm = max_f32(sc[0][0], sc[0][1]);
#pragma unroll
    for (int e = 2; e < TILES * 4; e += 2) cm = max3_f32(cm, sc[e >> 2][e & 3], sc[e >> 2][(e & 3) + 1]);
    m_w = max_xor32(max_xor16(cm));
    // a column whose visible positions all lie before this wave's range gets p = 0
    const float m_safe = m_w == -INFINITY ? 0.f : m_w;
#pragma unroll
    for (int t = 0; t < TILES; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[t][j] = fast_exp2(sc[t][j] - m_safe);
        l_part += sc[t][j];
      }
  }
  // O += P.V over 32-position blocks: k index 8lg+j <-> position 32u + 4lg + j (j<4)
  // or 32u + 16 + 4lg + (j-4): exactly the S^T values this lane holds. The B
  // operand comes from the wave's V rows by transpose reads once its direct
  // loads have landed (the wait is explicit: the compiler does not see that
  // these LDS reads depend on them).
  if (busy) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int u = 0; u < TILES / 2; ++u) {
      if (S::VPH == 2 && u == TILES / 4) {
        // the first half's rows are consumed (LDS accesses of a wave run in
        // order): the second half takes their place, in the same slot layout
#pragma unroll
        for (int j = 0; j < VLD - S::VDMA; ++j) st16(vl + 1024 * j + 16 * lane, vr[j]);
      }
      vec8_t pa;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pa[j] = (scalar_t)sc[2 * u][j];
        pa[4 + j] = (scalar_t)sc[2 * u + 1][j];
      }
      // lane (lg, lc) points at elements 4 (lc & 3) .. +3 of dims 16nn.. of row
      // 32u + 4lg + (lc >> 2) (and the row 16 further): chunk (lc & 3) / 2 + 2nn
      // (rows of the second phase sit CT/2 rows lower; swz has period 4, so their slots match)
      const int rlo = 32 * u - (S::VPH == 2 && u >= TILES / 4 ? CT / 2 : 0) + 4 * lg + (lc >> 2), rhi = rlo + 16;
      const int half8 = 8 * (lc & 1);
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) {
        const int c = ((lc & 3) >> 1) + 2 * nn;
        const uint2 lo = lds_read_tr16(vl + rlo * RB + 16 * (c ^ S::swz(rlo)) + half8);
        const uint2 hi = lds_read_tr16(vl + rhi * RB + 16 * (c ^ S::swz(rhi)) + half8);
        vec16 vb;
        vb.w[0] = lo.x; vb.w[1] = lo.y; vb.w[2] = hi.x; vb.w[3] = hi.y;
        acc[nn] = M::mfma(pa, __builtin_bit_cast(vec8_t, vb), acc[nn]);
      }
    }
    // Fused append: the wave holding the newest position (wave-uniform test)
    // writes its K and V rows to their pool slot, lanes 0..VCOLS-1 the K row
    // and the next VCOLS lanes the V row; one head group does it for the kv head.
    if (stores_new && lane < 2 * VCOLS) {
      const int c = lane % VCOLS;
      const bool is_v = lane >= VCOLS;
      char* const dst = pool_kvh + (int64_t)new_blk * blk_bytes + (int64_t)((ctx - 1) & (bs - 1)) * RB;
      vec16 x = ld16((is_v ? v_new_row : k_new_row) + 16 * c);
      if (!is_v && a.rope.cos) {   // K chunk c pairs with chunk c +- VCOLS/2
        const bool first = c < VCOLS / 2;
        const int c1 = first ? c : c - VCOLS / 2;
        vec16 y = ld16(k_new_row + 16 * (first ? c + VCOLS / 2 : c1));
        const int64_t r = a.rope.row(ctx - 1, D / 2) + 8 * c1;
        if (first) rope_pair<scalar_t>(x, y, a.rope.cos + r, a.rope.sin + r);
        else rope_pair<scalar_t>(y, x, a.rope.cos + r, a.rope.sin + r);
      }
      st16_through(dst + (is_v ? v_off : 0) + 16 * c, x);
    }
  }
  __syncthreads();   // every wave is done with its V rows: the area takes the merge
  float l_w = l_part + __shfl_xor(l_part, 16);
  l_w += __shfl_xor(l_w, 32);
  if (lg == 0) ml_lds[wave][lc] = make_float2(m_w, l_w);
  __syncthreads();   // stats visible

  // ---- merge the waves: acc rows (columns 4lg+j) scaled to the workgroup max ----
  float* const acc_lds = reinterpret_cast<float*>(lds);   // [wave][16 columns][D]
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = 4 * lg + j;
    float Mh = ml_lds[0][h].x;
#pragma unroll
    for (int w = 1; w < NW; ++w) Mh = fmaxf(Mh, ml_lds[w][h].x);
    const float mw = ml_lds[wave][h].x;
    const float f = (busy && mw != -INFINITY) ? fast_exp2(mw - Mh) : 0.f;
    float* dst = acc_lds + ((wave * 16) + h) * D + lc;
#pragma unroll
    for (int nn = 0; nn < NSL; ++nn) dst[16 * nn] = acc[nn][j] * f;
  }
  __syncthreads();

  for (int idx = threadIdx.x; idx < ncols * D; idx += 64 * NW) {
    const int h = idx / D, d = idx - h * D;          // h: column
    const int row = row0 + h / R, head = head0 + h - (h / R) * R;
    const int64_t pidx = pbeg0 + (h / R) * nparts + part;
    float Mh = ml_lds[0][h].x;
#pragma unroll
    for (int w = 1; w < NW; ++w) Mh = fmaxf(Mh, ml_lds[w][h].x);
    float L = 0.f, o = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float2 ml = ml_lds[w][h];
      if (ml.y > 0.f) L = fmaf(ml.y, fast_exp2(ml.x - Mh), L);   // idle waves hold (-inf, 0)
      o += acc_lds[(w * 16 + h) * D + d];
    }
    if (nparts == 1) {
      reinterpret_cast<scalar_t*>(a.out + row * a.out_row_bytes)[(int64_t)head * D + d] = (scalar_t)(o / L);
    } else {
      a.ws_acc[(pidx * a.num_heads + head) * D + d] = o;
      if (d == 0) *reinterpret_cast<float2*>(a.ws_ml + (pidx * a.num_heads + head) * 2) = make_float2(Mh, L);
    }
  }
  if (nparts > 1 && a.arrivals) merge_in_launch<Tag, D>(a, row0, kvh, head0, R, ncols, pbeg0, nparts);
}

template <typename Tag, int D, bool UT>
__global__ __launch_bounds__(64 * mfma_shape<D>::NW) __attribute__((amdgpu_waves_per_eu(5)))
void paged_attn_mfma_kernel(const attn_args a) {
  __shared__ __align__(16) char lds[mfma_shape<D>::LDS];
  decode_items_body<Tag, D, UT>(a, lds, blockIdx.x, blockIdx.z);
}

// ---------------------------------------------------------------------------
// Prefill tiles (16-bit). A workgroup of 4 waves owns up to 64 consecutive
// query rows of one sequence (wave w: rows 16w .. 16w+15; lane column lc is
// the row), one query head and one tile partition of PART_TILE positions (a
// row longer than that leaves partials for the combine kernel, like a split
// decode row). It walks its partition in chunks of 64 positions: each chunk's
// K and V rows are loaded once per workgroup (coalesced 16-byte loads through
// the block table) and staged in LDS for the four waves, K as rows and V
// transposed (one LDS row per head dim); the next chunk's loads are in flight
// while a chunk is computed.
//   S^T[pos][row] = K[pos][:] . Q[row][:]         A = K rows (LDS), B = q (registers)
//   O^T[dv][row] += V^T[dv][pos] . P^T[pos][row]  A = V^T rows (LDS, 8-byte reads),
//                                                 B = P (the S^T registers, repacked)
// Every operand a lane holds belongs to its own row, so the softmax state
// stays in the lane; row max / sum reduce across the four 16-lane groups with
// permlane swaps. The softmax is VALU-bound on CDNA (16-lane SIMDs), so per
// score it costs one max, one FMA (scale and max folded) and one exp2; the
// reference max m moves only when a row's max grows past m + 8, so p <= 2^8
// and the accumulator rescale is rare (m, l and the accumulator always refer
// to the same m, which is what the partials record). Only chunks that cross a
// row's diagonal are masked. Row i (position pos0 + i) sees positions
// 0 .. pos0 + i: the mask of model.py:139-146 for both the causal prefill and
// a prefill tail.
constexpr int PART_TILE = TB_PREFILL_TILE_PARTITION;   // positions per tile partition
static_assert(TB_PREFILL_TILE_ROWS == 64, "four waves of 16 rows");

template <int D>
struct prefill_shape {
  static constexpr int RB = 2 * D;             // bytes per K or V row
  static constexpr int KS = D / 32;            // q.k k-slices
  static constexpr int NSL = D / 16;           // O^T slices of 16 dims
  static constexpr int RS = RB + 16;           // K row stride in LDS: the 16-byte row reads of 16 lanes hit distinct banks
  static constexpr int RSV = RB + 32;          // V row stride: the 4 rows of a transpose read start 8 banks apart
  static constexpr int CK = 64;                // positions per chunk
  static constexpr int NCH = PART_TILE / CK;   // chunks per partition
  static constexpr int VCOLS = RB / 16;        // 16-byte pieces of a row
  static constexpr int LPT = CK * VCOLS / 256; // 16-byte loads per thread per chunk, of K and of V each
  static constexpr int BLKS = PART_TILE / 4;   // block ids of a partition (block size >= 4)
  static constexpr int LDS = CK * RS + CK * RSV + BLKS * 4;
  static constexpr int PF = LPT <= 2 ? 2 : 1;  // chunks loaded ahead (register sets; D = 128 has room for one)
  static_assert(LPT >= 1 && (CK * VCOLS) % 256 == 0 && PART_TILE % CK == 0, "chunk split");
};

template <typename Tag, int D>
__device__ __forceinline__ void prefill_tiles_body(const attn_args& a, char* const lds, const int bx) {
  using S = prefill_shape<D>;
  using M = math<Tag>;
  typedef typename M::vec8_t vec8_t;
  typedef typename M::scalar_t scalar_t;
  constexpr int RB = S::RB, KS = S::KS, NSL = S::NSL, RS = S::RS, CK = S::CK, NCH = S::NCH;
  constexpr int VCOLS = S::VCOLS, LPT = S::LPT, RSV = S::RSV, EB = 2;
  char* const k_lds = lds;
  char* const v_lds = lds + CK * RS;
  int32_t* const blk_lds = reinterpret_cast<int32_t*>(lds + CK * RS + CK * RSV);

  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int item = bx / a.num_heads;
  const int head = bx - item * a.num_heads;
  const int4 ti = a.tiles[item];                 // the array holds the grid's capacity
  if (a.counts && item >= a.counts[2]) return;   // whole workgroup: beyond this step's tiles
  const int row0 = ti.x, seq = ti.y, nrows = ti.z & 0xFF, part = ti.z >> 8, pos0 = ti.w;
  const int kvh = head / a.rep;
  const int limit = pos0 + nrows;                  // positions the tile's last row sees
  const int c0 = part * NCH;                       // first chunk of the partition
  const int c_end = min(c0 + NCH, (limit + CK - 1) / CK);
  const int my_row = 16 * wave + lc;               // tile-relative row of this lane
  const int my_pos = pos0 + my_row;                // sees positions 0 .. my_pos
  const int wave_first = pos0 + 16 * wave;         // smallest position a row of this wave has
  const int wave_last = pos0 + min(nrows, 16 * wave + 16) - 1;
  const bool wave_busy = 16 * wave < nrows;

  const int bs = 1 << a.log2_bs;
  const int64_t tile_bytes = (int64_t)bs * RB;
  const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * tile_bytes;
  const int64_t v_off = (int64_t)a.num_kv_heads * tile_bytes;
  const char* const pool_kvh = a.pool + kvh * tile_bytes;
  const int32_t* const table = a.block_tables + (int64_t)seq * a.max_nb;

  // the row's partition count decides between final output and a partial slot
  int pbeg = 0, nparts = 0;
  if (my_row < nrows) {
    pbeg = a.row_part_off[row0 + my_row];
    nparts = a.row_part_off[row0 + my_row + 1] - pbeg;
  }

  // The block ids of the partition's positions, read once into LDS: a table read
  // inside the chunk loop would be a load whose result the next chunk's addresses
  // wait for, and since loads complete in issue order that wait would also take
  // every K/V load issued before it, leaving one chunk in flight instead of PF.
  const int blk0 = (c0 * CK) >> a.log2_bs;                    // first block of the partition
  const int nblk = c_end > c0 ? (((c_end * CK < limit ? c_end * CK : limit) - 1) >> a.log2_bs) - blk0 + 1 : 0;
  for (int i = threadIdx.x; i < nblk; i += 256) {           // nblk <= PART_TILE / block_size <= BLKS
    int b = table[blk0 + i];
    if (b < 0 || b >= a.num_blocks) b = 0;   // host validates; stay inside the pool
    blk_lds[i] = b;
  }
  __syncthreads();
  // Thread t, load i: row (t + 256 i) / VCOLS of the chunk, 16-byte piece (t + 256 i) % VCOLS.
  auto load_ids = [&](int c, int (&ids)[LPT]) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int p = c * CK + (threadIdx.x + 256 * i) / VCOLS;
      ids[i] = (c < c_end && p < limit) ? blk_lds[(p >> a.log2_bs) - blk0] : -1;
    }
  };
  auto load_kv = [&](int c, const int (&ids)[LPT], vec16 (&kr)[LPT], vec16 (&vr)[LPT]) {
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int f = threadIdx.x + 256 * i;
      const int p = c * CK + f / VCOLS;
      if (ids[i] >= 0) {
        const int64_t off = (int64_t)ids[i] * blk_bytes + (int64_t)(p & (bs - 1)) * RB + 16 * (f % VCOLS);
        kr[i] = ld16(pool_kvh + off);
        vr[i] = ld16(pool_kvh + v_off + off);
      } else {
        kr[i] = zero16();   // positions past the tile's range: zero K and V
        vr[i] = zero16();
      }
    }
  };

  vec16 qb[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) qb[s] = zero16();
  if (my_row < nrows) {
    const char* qrow = a.q + (row0 + my_row) * a.q_row_bytes + (int64_t)head * RB + 16 * lg;
#pragma unroll
    for (int s = 0; s < KS; ++s) qb[s] = ld16(qrow + 64 * s);
  }

  float m = -INFINITY;       // reference max of row lc (scaled, base-2 domain)
  float4_t acc[NSL];         // O^T[16n + 4lg + j][row lc], relative to m
#pragma unroll
  for (int nn = 0; nn < NSL; ++nn) acc[nn] = float4_t{0.f, 0.f, 0.f, 0.f};
  // The row sums ride on the matrix unit: an A operand whose first row is all
  // ones turns P into sum_k P[k][row] in element 0 of lanes 0..15 (D[0][row]),
  // one MFMA per 32 positions instead of 16 adds per lane per chunk. The sum
  // is of the rounded P that multiplies V.
  float4_t acc_l = float4_t{0.f, 0.f, 0.f, 0.f};
  vec8_t ones;
#pragma unroll
  for (int j = 0; j < 8; ++j) ones[j] = (scalar_t)(lc == 0 ? 1.f : 0.f);

  // stage one chunk (already in registers) in LDS
  auto stage = [&](const vec16 (&kr)[LPT], const vec16 (&vr)[LPT]) {
    __syncthreads();   // the previous chunk's LDS reads are done
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
      const int f = threadIdx.x + 256 * i;
      const int r = f / VCOLS, d0 = 8 * (f % VCOLS);
      st16(k_lds + r * RS + 2 * d0, kr[i]);
      st16(v_lds + r * RSV + 2 * d0, vr[i]);
    }
    __syncthreads();   // chunk staged
  };
  // fold the staged chunk c into the row state
  auto compute = [&](int c) {
    const int cb = c * CK;
    if (!(wave_busy && cb <= wave_last)) return;
    float4_t sc[4];   // S^T (raw): lane holds positions cb + 16t + 4lg + j of row lc
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      sc[t] = float4_t{0.f, 0.f, 0.f, 0.f};
      const char* krow = k_lds + (16 * t + lc) * RS + 16 * lg;
#pragma unroll
      for (int s = 0; s < KS; ++s)
        sc[t] = M::mfma(__builtin_bit_cast(vec8_t, ld16(krow + 64 * s)), __builtin_bit_cast(vec8_t, qb[s]), sc[t]);
    }
    if (cb + CK - 1 > wave_first) {   // the chunk crosses the diagonal of some row of this wave
#pragma unroll
      for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (cb + 16 * t + 4 * lg + j > my_pos) sc[t][j] = -INFINITY;
    }
    float cm = max_f32(sc[0][0], sc[0][1]);
#pragma unroll
    for (int e = 2; e < 16; e += 2) cm = max3_f32(cm, sc[e >> 2][e & 3], sc[e >> 2][(e & 3) + 1]);
    cm = max_xor32(max_xor16(cm)) * a.scale_log2e;   // the row's chunk max, scaled (-inf if all masked)
    if (__any(cm > m + 8.f)) {   // some row outgrew its reference: move every row's reference up
      const float m_new = fmaxf(m, cm);
      const float alpha = fast_exp2(m - (m_new == -INFINITY ? 0.f : m_new));   // 0 while m = -inf
      m = m_new;
      acc_l *= alpha;
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) acc[nn] *= alpha;
    }
    const float neg_m = m == -INFINITY ? 0.f : -m;   // a row that has seen nothing keeps p = 0
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) sc[t][j] = fast_exp2(fmaf(sc[t][j], a.scale_log2e, neg_m));
    // k index 8lg+j <-> position 32u + 4lg + j (j < 4) or 32u + 16 + 4lg + (j-4)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      vec8_t pb;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        pb[j] = (scalar_t)sc[2 * u][j];
        pb[4 + j] = (scalar_t)sc[2 * u + 1][j];
      }
      // A operand lane (lg, lc): V[position of k = 8lg + j][16nn + lc], by transpose
      // reads of rows 32u + 4lg + 0..3 (and 16 further), elements 4 (lc & 3) ..
      const char* vrow = v_lds + (32 * u + 4 * lg + (lc >> 2)) * RSV + 8 * (lc & 3);
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) {
        const uint2 lo = lds_read_tr16(vrow + 32 * nn);
        const uint2 hi = lds_read_tr16(vrow + 16 * RSV + 32 * nn);
        vec16 va;
        va.w[0] = lo.x; va.w[1] = lo.y; va.w[2] = hi.x; va.w[3] = hi.y;
        acc[nn] = M::mfma(__builtin_bit_cast(vec8_t, va), pb, acc[nn]);
      }
      acc_l = M::mfma(ones, pb, acc_l);
    }
  };

  // K/V of chunk c + PF are loaded into registers while chunk c is computed
  // (PF register sets; LDS holds the chunk being computed)
  int ids[LPT];
  vec16 kr0[LPT], vr0[LPT], kr1[LPT], vr1[LPT];
  load_ids(c0, ids);
  load_kv(c0, ids, kr0, vr0);
  load_ids(c0 + 1, ids);
  if constexpr (S::PF == 2) {
    load_kv(c0 + 1, ids, kr1, vr1);
    load_ids(c0 + 2, ids);
  }
  if (a.rope.cos && my_row < nrows) {   // RoPE of q at the row's position (slices s and s + KS/2 pair)
    const int64_t r = a.rope.row(pos0 + my_row, D / 2) + 8 * lg;
#pragma unroll
    for (int s = 0; s < KS / 2; ++s)
      rope_pair<scalar_t>(qb[s], qb[s + KS / 2], a.rope.cos + r + 32 * s, a.rope.sin + r + 32 * s);
  }
  auto iter = [&](int c, vec16 (&kr)[LPT], vec16 (&vr)[LPT]) {
    stage(kr, vr);
    if (c + S::PF < c_end) {
      load_kv(c + S::PF, ids, kr, vr);
      load_ids(c + S::PF + 1, ids);
    }
    compute(c);
  };
  if constexpr (S::PF == 2) {
    for (int c = c0; c < c_end; c += 2) {   // workgroup-uniform trip count
      iter(c, kr0, vr0);
      if (c + 1 < c_end) iter(c + 1, kr1, vr1);
    }
  } else {
    for (int c = c0; c < c_end; ++c) iter(c, kr0, vr0);
  }

  const float l = __shfl(acc_l[0], lc);   // row lc's sum sits in lane lc
  if (my_row < nrows && part < nparts) {   // rows that end before this partition own no slot here
    const int row = row0 + my_row;
    if (nparts == 1) {           // the whole row: final output
      const float inv = 1.f / l;
      char* orow = a.out + row * a.out_row_bytes + (int64_t)head * D * EB;
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) {
        typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
        s4_t o;
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = (scalar_t)(acc[nn][j] * inv);
        st_through(orow + (16 * nn + 4 * lg) * EB, o);
      }
    } else {                     // partial of a split row
      const int64_t pidx = pbeg + part;
      float* dst = a.ws_acc + (pidx * a.num_heads + head) * D;
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) *reinterpret_cast<float4_t*>(dst + 16 * nn + 4 * lg) = acc[nn];
      if (lg == 0) *reinterpret_cast<float2*>(a.ws_ml + (pidx * a.num_heads + head) * 2) = make_float2(m, l);
    }
  }
}

template <typename Tag, int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void paged_prefill_mfma_kernel(const attn_args a) {
  __shared__ __align__(16) char lds[prefill_shape<D>::LDS];
  prefill_tiles_body<Tag, D>(a, lds, blockIdx.x);
}

// One launch for a step that has both prefill tiles and decode work items
// (head dim 64: both are workgroups of four waves): workgroups below
// tile_wgs are prefill tiles (issued first, the longest work), the rest are
// the decode items. The decode items are latency-bound and the tiles
// VALU/latency-bound, so sharing the machine lets one hide the other instead
// of running back to back.
template <typename Tag, int D, bool UT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4)))
void paged_step_mfma_kernel(const attn_args a, const int tile_wgs) {
  constexpr int L1 = mfma_shape<D>::LDS, L2 = prefill_shape<D>::LDS;
  static_assert(mfma_shape<D>::NW == 4, "one workgroup shape for both");
  __shared__ __align__(16) char lds[L1 > L2 ? L1 : L2];
  if ((int)blockIdx.x < tile_wgs) prefill_tiles_body<Tag, D>(a, lds, blockIdx.x);
  else decode_items_body<Tag, D, UT>(a, lds, blockIdx.x - tile_wgs, 0);
}

// ---------------------------------------------------------------------------
// Log-sum-exp merge of the partials of one split row: workgroup (r, c) owns
// COMBINE_THREADS float4 columns (4 consecutive output dims each, head =
// column / (D/4)) of split row r, starting at column COMBINE_THREADS * c. One
// wave per workgroup: a row's partials are read by several CUs at once instead
// of streaming through one.
constexpr int COMBINE_THREADS = 64;
//
//   out = sum_p 2^(m_p - M) acc_p / sum_p 2^(m_p - M) l_p.
// The row's record (row, first partial, count) is one 16-byte load, issued
// together with the device count; the partials follow in batches of 16 whose
// loads are all in flight (one batch for a row of up to 16 partitions).
template <typename Tag, int D>
__global__ __launch_bounds__(COMBINE_THREADS) void combine_partials_kernel(const attn_args a) {
  constexpr int EB = elem<Tag>::bytes;
  constexpr int QPH = D / 4;                       // float4 columns per head
  constexpr int BATCH = 8;                       // as merge_in_launch: the same bits
  const int col = threadIdx.x + COMBINE_THREADS * blockIdx.y;
  if (col >= a.num_heads * QPH) return;
  const int4 rec = a.split_rows[blockIdx.x];       // the array holds the grid's capacity
  if (a.counts && (int)blockIdx.x >= a.counts[1]) return;   // beyond this step's split rows
  const int row = rec.x, pbeg = rec.y, n = rec.z;
  const int head = col / QPH, d4 = col - head * QPH;
  float M = -INFINITY, L = 0.f;
  float4_t o = float4_t{0.f, 0.f, 0.f, 0.f};
  for (int p0 = 0; p0 < n; p0 += BATCH) {
    float2 ml[BATCH];
    float4_t av[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      if (p0 + k < n) {
        const int64_t slot = (int64_t)(pbeg + p0 + k) * a.num_heads + head;
        ml[k] = *reinterpret_cast<const float2*>(a.ws_ml + slot * 2);
        av[k] = *reinterpret_cast<const float4_t*>(a.ws_acc + slot * D + 4 * d4);
      } else {
        ml[k] = make_float2(-INFINITY, 0.f);
        av[k] = float4_t{0.f, 0.f, 0.f, 0.f};
      }
    }
    float mb = M;
#pragma unroll
    for (int k = 0; k < BATCH; ++k) mb = fmaxf(mb, ml[k].x);   // finite: every partial saw a position
    const float keep = fast_exp2(M - mb);                        // 0 while M = -inf
    L *= keep;
    o *= keep;
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const float w = ml[k].y > 0.f ? fast_exp2(ml[k].x - mb) : 0.f;
      L = fmaf(ml[k].y, w, L);
      o += av[k] * w;
    }
    M = mb;
  }
  const float inv = 1.f / L;
  char* const dst = a.out + row * a.out_row_bytes + ((int64_t)head * D + 4 * d4) * EB;
  if constexpr (EB == 4) {
    *reinterpret_cast<float4_t*>(dst) = o * inv;
  } else {
    typedef typename elem<Tag>::type s_t;
    typedef s_t s4_t __attribute__((ext_vector_type(4)));
    s4_t r;
#pragma unroll
    for (int j = 0; j < 4; ++j) r[j] = (s_t)(o[j] * inv);
    st_through(dst, r);
  }
}

// ---- dispatch ---------------------------------------------------------------
template <typename Tag, int D, int REP>
static void launch_valu(const attn_args& a, int num_work, hipStream_t stream) {
  hipLaunchKernelGGL((paged_attn_valu_kernel<Tag, D, REP>), dim3(num_work, a.num_kv_heads, a.rep / a.group),
                     dim3(64), 0, stream, a);
}

template <int D>
static int dispatch_valu_rep(const attn_args& a, int num_work, hipStream_t s) {
  switch (a.group) {
    case 1: launch_valu<f32_t, D, 1>(a, num_work, s); return TB_OK;
    case 2: launch_valu<f32_t, D, 2>(a, num_work, s); return TB_OK;
    case 3: launch_valu<f32_t, D, 3>(a, num_work, s); return TB_OK;
    case 4: launch_valu<f32_t, D, 4>(a, num_work, s); return TB_OK;
    case 5: launch_valu<f32_t, D, 5>(a, num_work, s); return TB_OK;
    case 6: launch_valu<f32_t, D, 6>(a, num_work, s); return TB_OK;
    case 7: launch_valu<f32_t, D, 7>(a, num_work, s); return TB_OK;
    case 8: launch_valu<f32_t, D, 8>(a, num_work, s); return TB_OK;
    default: return TB_ERR_UNSUPPORTED;
  }
}

template <typename Tag, int D>
static void launch_mfma(const attn_args& a, int num_work, hipStream_t stream) {
  const dim3 grid(num_work * a.num_kv_heads, 1, a.rep / a.group), block(64 * mfma_shape<D>::NW);
  if (a.log2_bs >= 4)   // 16-position tiles never cross a block
    hipLaunchKernelGGL((paged_attn_mfma_kernel<Tag, D, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((paged_attn_mfma_kernel<Tag, D, false>), grid, block, 0, stream, a);
}

template <typename Tag, int D>
static void launch_mfma_grid(const attn_args& a, dim3 grid, dim3 block, hipStream_t stream) {
  if (a.log2_bs >= 4)   // 16-position tiles never cross a block
    hipLaunchKernelGGL((paged_attn_mfma_kernel<Tag, D, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((paged_attn_mfma_kernel<Tag, D, false>), grid, block, 0, stream, a);
}

template <typename Tag, int D>
static void launch_combine(const attn_args& a, int num_split_rows, hipStream_t stream) {
  if (num_split_rows > 0)
    hipLaunchKernelGGL((combine_partials_kernel<Tag, D>),
                       dim3(num_split_rows, (a.num_heads * (D / 4) + COMBINE_THREADS - 1) / COMBINE_THREADS),
                       dim3(COMBINE_THREADS), 0, stream, a);
}

template <typename Tag, int D>
static void launch_prefill(const attn_args& a, int num_tiles, hipStream_t stream) {
  if (num_tiles > 0)
    hipLaunchKernelGGL((paged_prefill_mfma_kernel<Tag, D>), dim3(num_tiles * a.num_heads), dim3(256), 0, stream, a);
}

template <typename Tag, int D>
static void launch_step(const attn_args& a, int num_work, int num_tiles, hipStream_t stream) {
  const int tile_wgs = num_tiles * a.num_heads;
  const dim3 grid(tile_wgs + num_work * a.num_kv_heads);
  if (a.log2_bs >= 4)
    hipLaunchKernelGGL((paged_step_mfma_kernel<Tag, D, true>), grid, dim3(256), 0, stream, a, tile_wgs);
  else
    hipLaunchKernelGGL((paged_step_mfma_kernel<Tag, D, false>), grid, dim3(256), 0, stream, a, tile_wgs);
}

template <typename Tag>
static void launch_16bit(const attn_args& a, bool d64, int num_work, int num_tiles, int num_split_rows,
                         hipStream_t stream) {
  if (d64) {
    if (num_work > 0 && num_tiles > 0 && a.rep == a.group) {
      launch_step<Tag, 64>(a, num_work, num_tiles, stream);
    } else {
      if (num_work > 0) launch_mfma<Tag, 64>(a, num_work, stream);
      launch_prefill<Tag, 64>(a, num_tiles, stream);
    }
    launch_combine<Tag, 64>(a, num_split_rows, stream);
  } else {
    if (num_work > 0) launch_mfma<Tag, 128>(a, num_work, stream);
    launch_prefill<Tag, 128>(a, num_tiles, stream);
    launch_combine<Tag, 128>(a, num_split_rows, stream);
  }
}

static int largest_divisor_upto(int rep, int cap) {
  for (int t = cap; t >= 1; --t)
    if (rep % t == 0) return t;
  return 1;
}

static int elem_bytes(int32_t dtype) {
  return dtype == TB_DTYPE_F32 ? 4 : (dtype == TB_DTYPE_F16 || dtype == TB_DTYPE_BF16) ? 2 : 0;
}

// Partition lengths each kernel accepts.
static bool partition_ok(int32_t dtype, int head_dim, int block_size, int part) {
  if (part <= 0 || part % block_size != 0 || part / block_size > 64) return false;
  if (elem_bytes(dtype) == 2) return part == PART16;
  const int lpt = head_dim * 4 / 16;
  const int chunk = 8 * (64 / lpt);
  return part % chunk == 0;
}

}  // namespace tb

extern "C" int32_t tb_attention_partition_tokens(int32_t dtype, int32_t head_dim) {
  if (tb::elem_bytes(dtype) == 2) return tb::PART16;
  return 256;
}

extern "C" size_t tb_paged_attention_workspace_bytes(int32_t total_partitions, int32_t num_heads,
                                                     int32_t head_dim) {
  if (total_partitions <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return (size_t)total_partitions * num_heads * ((size_t)head_dim + 2) * sizeof(float);
}

namespace tb {

static int32_t paged_attention_impl(const void* q, int64_t q_row_stride, void* pool,
                                    int64_t num_blocks, void* out, int64_t out_row_stride,
                                    const int32_t* block_tables, int32_t max_blocks_per_seq,
                                    const int32_t* work_items, int32_t num_work_items,
                                    const int32_t* prefill_tiles, int32_t num_prefill_tiles,
                                    const int32_t* row_part_offsets, int32_t num_rows,
                                    const int32_t* split_rows, int32_t num_split_rows,
                                    int32_t max_parts_per_row, int32_t partition_tokens,
                                    int32_t total_partitions, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                    float scale, int32_t dtype, const void* k_new,
                                    int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                                    void* workspace, size_t workspace_bytes,
                                    const int32_t* device_counts, const float* rope_cos,
                                    const float* rope_sin, int32_t rope_max_position,
                                    hipStream_t stream, const int32_t* slot_map = nullptr,
                                    int32_t slot_count = 0, unsigned long long* arrivals = nullptr,
                                    int32_t arrival_units = 0, uint32_t* violations = nullptr) {
  const int eb = elem_bytes(dtype);
  TB_CHECK_ARG(eb > 0);
  TB_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0);
  if (head_dim != 64 && head_dim != 128) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(block_size >= 4 && (block_size & (block_size - 1)) == 0);
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  TB_CHECK_ARG(num_rows >= 0 && num_work_items >= 0 && num_prefill_tiles >= 0 && num_split_rows >= 0);
  TB_CHECK_ARG(max_blocks_per_seq > 0 && num_blocks > 0);
  TB_CHECK_ARG(partition_ok(dtype, head_dim, block_size, partition_tokens));
  TB_CHECK_ARG(q_row_stride >= (int64_t)num_heads * head_dim);
  TB_CHECK_ARG(out_row_stride >= (int64_t)num_heads * head_dim);
  if (num_prefill_tiles > 0 && eb != 2) return TB_ERR_UNSUPPORTED;   // fp32 rows go to work items
  if (num_work_items == 0 && num_prefill_tiles == 0) return TB_OK;
  TB_CHECK_ARG(q && pool && out && block_tables && num_rows > 0);
  TB_CHECK_ARG(num_work_items == 0 || (work_items && row_part_offsets));
  TB_CHECK_ARG(num_prefill_tiles == 0 || prefill_tiles);
  TB_CHECK_ARG((((uintptr_t)q | (uintptr_t)pool | (uintptr_t)out) & 15u) == 0);
  TB_CHECK_ARG((q_row_stride * eb) % 16 == 0 && (out_row_stride * eb) % 16 == 0);
  TB_CHECK_ARG(max_parts_per_row >= (num_work_items > 0 ? 1 : 0) && total_partitions >= num_work_items);
  TB_CHECK_ARG(num_split_rows <= num_rows && (num_split_rows == 0 || (split_rows && max_parts_per_row > 1)));
  TB_CHECK_ARG(((uintptr_t)split_rows & 15u) == 0);
  if (max_parts_per_row > 1) {
    TB_CHECK_ARG(workspace != nullptr);
    TB_CHECK_ARG(workspace_bytes >= tb_paged_attention_workspace_bytes(total_partitions, num_heads, head_dim));
    TB_CHECK_ARG(((uintptr_t)workspace & 15u) == 0);
  }
  if (rope_cos || rope_sin) {
    TB_CHECK_ARG(rope_cos && rope_sin && rope_max_position > 0);
    TB_CHECK_ARG((((uintptr_t)rope_cos | (uintptr_t)rope_sin) & 15u) == 0);
  }
  if (k_new || v_new) {
    TB_CHECK_ARG(k_new && v_new && num_prefill_tiles == 0);
    TB_CHECK_ARG(k_row_stride >= (int64_t)num_kv_heads * head_dim && v_row_stride >= (int64_t)num_kv_heads * head_dim);
    TB_CHECK_ARG((((uintptr_t)k_new | (uintptr_t)v_new) & 15u) == 0);
    TB_CHECK_ARG((k_row_stride * eb) % 16 == 0 && (v_row_stride * eb) % 16 == 0);
  }

  const int rep = num_heads / num_kv_heads;
  // heads per wave: the MFMA operand holds 16; the fp32 kernel keeps 8 in registers
  const int group = largest_divisor_upto(rep, eb == 2 ? 16 : 8);
  const bool merged = slot_map != nullptr;
  if (merged) {   // split rows merged inside the launch of the 16-bit work-item kernel
    if (eb != 2 || num_prefill_tiles > 0 || group != rep || device_counts) return TB_ERR_UNSUPPORTED;
    // a row's partitions are counted in 8-bit per-XCD fields of its arrival word
    if (max_parts_per_row > TB_MERGED_MAX_PARTS) return TB_ERR_UNSUPPORTED;
    TB_CHECK_ARG(slot_count >= num_work_items * num_kv_heads && arrivals && violations);
    TB_CHECK_ARG(((uintptr_t)arrivals & 127u) == 0 && (int64_t)arrival_units >= (int64_t)num_rows * num_kv_heads);
    TB_CHECK_ARG(max_parts_per_row <= 1 ||
                 tb_paged_attention_workspace_bytes(total_partitions, num_heads, head_dim) < ((size_t)1 << 31));
  }
  TB_CHECK_ARG(num_kv_heads <= 65535 && rep / group <= 65535);
  TB_CHECK_ARG((int64_t)num_work_items * num_kv_heads < ((int64_t)1 << 31));

  attn_args a;
  a.q = (const char*)q;
  a.q_row_bytes = q_row_stride * eb;
  a.pool = (char*)pool;
  a.num_blocks = num_blocks;
  a.out = (char*)out;
  a.out_row_bytes = out_row_stride * eb;
  a.block_tables = block_tables;
  a.max_nb = max_blocks_per_seq;
  a.work = reinterpret_cast<const int4*>(work_items);
  a.row_part_off = row_part_offsets;
  a.tiles = reinterpret_cast<const int4*>(prefill_tiles);
  a.split_rows = reinterpret_cast<const int4*>(split_rows);
  a.rope = rope_tables{rope_cos, rope_sin, rope_max_position};
  a.counts = device_counts;
  // workspace: [acc partials: parts x Hq x D][max/sum partials: parts x Hq x 2]
  a.ws_acc = (float*)workspace;
  a.ws_ml = workspace ? a.ws_acc + (size_t)total_partitions * num_heads * head_dim : nullptr;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.rep = rep;
  a.group = group;
  a.log2_bs = log2_bs;
  a.part_tokens = partition_tokens;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.k_new = (const char*)k_new;
  a.k_new_row_bytes = k_row_stride * eb;
  a.v_new = (const char*)v_new;
  a.v_new_row_bytes = v_row_stride * eb;
  a.slot_map = slot_map;
  a.num_work = num_work_items;
  a.arrivals = merged ? arrivals : nullptr;
  a.violations = violations;
  a.ws_bytes = workspace ? (uint32_t)tb_paged_attention_workspace_bytes(total_partitions, num_heads, head_dim) : 0u;

  const bool d64 = head_dim == 64;
  if (merged) {
    if (num_work_items > 0) {
      const dim3 grid(slot_count), block(64 * (d64 ? mfma_shape<64>::NW : mfma_shape<128>::NW));
      if (dtype == TB_DTYPE_F16) {
        if (d64) launch_mfma_grid<f16_t, 64>(a, grid, block, stream);
        else launch_mfma_grid<f16_t, 128>(a, grid, block, stream);
      } else {
        if (d64) launch_mfma_grid<bf16_t, 64>(a, grid, block, stream);
        else launch_mfma_grid<bf16_t, 128>(a, grid, block, stream);
      }
    }
    TB_RETURN_LAUNCH_STATUS();
  }
  int st = TB_OK;
  switch (dtype) {
    case TB_DTYPE_F32:
      st = d64 ? dispatch_valu_rep<64>(a, num_work_items, stream) : dispatch_valu_rep<128>(a, num_work_items, stream);
      if (st == TB_OK)
        d64 ? launch_combine<f32_t, 64>(a, num_split_rows, stream) : launch_combine<f32_t, 128>(a, num_split_rows, stream);
      break;
    case TB_DTYPE_F16:
      launch_16bit<f16_t>(a, d64, num_work_items, num_prefill_tiles, num_split_rows, stream);
      break;
    case TB_DTYPE_BF16:
      launch_16bit<bf16_t>(a, d64, num_work_items, num_prefill_tiles, num_split_rows, stream);
      break;
    default: return TB_ERR_INVALID_ARG;
  }
  if (st != TB_OK) return st;
  TB_RETURN_LAUNCH_STATUS();
}

// ---- scratch of the allocation-free entry point ------------------------------
// The split-row partials of tb_paged_attention_noalloc live in this array: one
// copy per GPU, resident from the code object's load until the process ends.
// Its device address is looked up once per device (hipGetSymbolAddress with
// that device current) and only that address reaches a kernel or a copy.
static __device__ __align__(256) char scratch[TB_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
static std::atomic<void*> scratch_ptr[MAX_DEVICES];
static std::mutex scratch_mu;

static int32_t scratch_address(hipStream_t stream, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES) return TB_ERR_LAUNCH;
  if (stream != nullptr) {   // the stream must belong to the current device, whose copy is used
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return TB_ERR_INVALID_ARG;
    if ((int)sdev != dev) return TB_ERR_INVALID_ARG;
  }
  void* p = scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lock(scratch_mu);
    p = scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return TB_ERR_LAUNCH;
      scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return TB_OK;
}

}  // namespace tb

extern "C" int32_t tb_paged_attention(const void* q, int64_t q_row_stride, void* pool,
                                      int64_t num_blocks, void* out, int64_t out_row_stride,
                                      const int32_t* block_tables, int32_t max_blocks_per_seq,
                                      const int32_t* work_items, int32_t num_work_items,
                                      const int32_t* prefill_tiles, int32_t num_prefill_tiles,
                                      const int32_t* row_part_offsets, int32_t num_rows,
                                      const int32_t* split_rows, int32_t num_split_rows,
                                      int32_t max_parts_per_row, int32_t partition_tokens,
                                      int32_t total_partitions, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                      float scale, int32_t dtype, const void* k_new,
                                      int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                                      void* workspace, size_t workspace_bytes,
                                      const int32_t* device_counts, const float* rope_cos,
                                      const float* rope_sin, int32_t rope_max_position,
                                      hipStream_t stream) {
  return tb::paged_attention_impl(q, q_row_stride, pool, num_blocks, out, out_row_stride, block_tables,
                                  max_blocks_per_seq, work_items, num_work_items, prefill_tiles,
                                  num_prefill_tiles, row_part_offsets, num_rows, split_rows, num_split_rows,
                                  max_parts_per_row, partition_tokens, total_partitions, num_heads,
                                  num_kv_heads, head_dim, block_size, scale, dtype, k_new, k_row_stride, v_new,
                                  v_row_stride, workspace, workspace_bytes, device_counts, rope_cos, rope_sin,
                                  rope_max_position, stream);
}

extern "C" int32_t tb_paged_attention_noalloc(const void* q, int64_t q_row_stride, void* pool,
                                              int64_t num_blocks, void* out, int64_t out_row_stride,
                                              const int32_t* block_tables, int32_t max_blocks_per_seq,
                                              const int32_t* work_items, int32_t num_work_items,
                                              const int32_t* prefill_tiles, int32_t num_prefill_tiles,
                                              const int32_t* row_part_offsets, int32_t num_rows,
                                              const int32_t* split_rows, int32_t num_split_rows,
                                              int32_t max_parts_per_row, int32_t partition_tokens,
                                              int32_t total_partitions, int32_t num_heads,
                                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                              float scale, int32_t dtype, const void* k_new,
                                              int64_t k_row_stride, const void* v_new,
                                              int64_t v_row_stride, const int32_t* device_counts,
                                              const float* rope_cos, const float* rope_sin,
                                              int32_t rope_max_position, hipStream_t stream) {
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (max_parts_per_row > 1) {   // partials are only written for rows of more than one partition
    const size_t need = tb_paged_attention_workspace_bytes(total_partitions, num_heads, head_dim);
    if (need > (size_t)TB_NOALLOC_SCRATCH_BYTES) return TB_ERR_SCRATCH;
    const int32_t st = tb::scratch_address(stream, &ws);
    if (st != TB_OK) return st;
    ws_bytes = TB_NOALLOC_SCRATCH_BYTES;
  }
  return tb::paged_attention_impl(q, q_row_stride, pool, num_blocks, out, out_row_stride, block_tables,
                                  max_blocks_per_seq, work_items, num_work_items, prefill_tiles,
                                  num_prefill_tiles, row_part_offsets, num_rows, split_rows, num_split_rows,
                                  max_parts_per_row, partition_tokens, total_partitions, num_heads,
                                  num_kv_heads, head_dim, block_size, scale, dtype, k_new, k_row_stride, v_new,
                                  v_row_stride, ws, ws_bytes, device_counts, rope_cos, rope_sin,
                                  rope_max_position, stream);
}

extern "C" int32_t tb_paged_attention_merged(const void* q, int64_t q_row_stride, void* pool,
                                             int64_t num_blocks, void* out, int64_t out_row_stride,
                                             const int32_t* block_tables, int32_t max_blocks_per_seq,
                                             const int32_t* work_items, int32_t num_work_items,
                                             const int32_t* row_part_offsets, int32_t num_rows,
                                             int32_t max_parts_per_row, int32_t partition_tokens,
                                             int32_t total_partitions, int32_t num_heads,
                                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                             float scale, int32_t dtype, const void* k_new,
                                             int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                                             void* workspace, size_t workspace_bytes,
                                             const int32_t* slot_map, int32_t slot_count,
                                             unsigned long long* arrivals, int32_t arrival_units,
                                             uint32_t* violations, const float* rope_cos,
                                             const float* rope_sin, int32_t rope_max_position,
                                             hipStream_t stream) {
  if (!slot_map || slot_count <= 0) return TB_ERR_INVALID_ARG;
  return tb::paged_attention_impl(q, q_row_stride, pool, num_blocks, out, out_row_stride, block_tables,
                                  max_blocks_per_seq, work_items, num_work_items, nullptr, 0, row_part_offsets,
                                  num_rows, nullptr, 0, max_parts_per_row, partition_tokens, total_partitions,
                                  num_heads, num_kv_heads, head_dim, block_size, scale, dtype, k_new, k_row_stride,
                                  v_new, v_row_stride, workspace, workspace_bytes, nullptr, rope_cos, rope_sin,
                                  rope_max_position, stream, slot_map, slot_count, arrivals, arrival_units,
                                  violations);
}
