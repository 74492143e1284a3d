// K2 for prefill sequences, streaming form (fp16 / bf16): the causal attention
// of a sequence's new rows over its whole context (reference
// src/tinybatch/model.py:130-147: gather, repeat_interleave, the mask of
// model.py:139-146 and SDPA), for sequences whose context fits in one
// workgroup's LDS.
//
// Work: one workgroup per (sequence, kv head, pair of 16-row blocks). The new
// rows are cut into blocks of 16; pair p holds blocks p and nb - 1 - p, so every
// pair of a sequence sees the same number of (row, position) scores. The
// workgroup has two waves per query head of the kv head (2 * rep waves), A and
// B: B takes the earlier block (and writes it), then the later block's steps
// past those A takes, so that A and B do equal work; at the end A merges B's
// part of the later block (log-sum-exp, through LDS) and writes it. Nothing
// goes through global memory but q, K/V and the output rows.
//
// Loads. The workgroup's K/V range (positions 0 .. the later block's last row)
// moves into LDS once, as 16-position tiles in the swizzled layout of
// tb_stream.h, by direct global->LDS loads of 1 KiB of consecutive pool bytes per
// instruction, all issued at the start (tile t by wave t % (2 rep)), so the
// range costs one memory round trip; the query heads of
// the kv head share it. V rows past the context are zeroed in LDS (a stale slot
// may hold any bits; their p is 0). One barrier, then every wave streams its
// tiles from LDS without further synchronisation.
//
// Math per pair of tiles (32 positions), the 16 rows of a wave as the 16 MFMA
// columns:
//   S^T[pos][row] = K[pos][:] . q[row][:]         v_mfma_f32_16x16x32, A = K rows (LDS)
//   O^T[d][row]  += V^T[d][pos] . P^T[pos][row]    v_mfma_f32_16x16x32, A = V^T (LDS
//                                                   transpose reads), B = the S^T registers
// so the online-softmax state of row lc (max, sum, its O^T column) lives in the
// lanes of column lc. Row i of the sequence's new rows is position pos0 + i and
// sees positions 0 .. pos0 + i; only tiles that cross a row's position are
// masked.
#include <type_traits>


#include "tb_stream.h"

namespace tb {

struct prefill_args {
  const char* q;               // [T][Hq][D] rows of the step
  int64_t q_row_bytes;
  char* pool;                  // [NB][2][Hkv][BS][D]
  int64_t num_blocks;
  char* out;                   // [T][Hq*D]
  int64_t out_row_bytes;
  const int32_t* block_tables; // [B][max_nb]
  int32_t max_nb;
  const int4* work;            // [num_work] (row0, seq, pos0, nrows | pair << 16 | kv head << 24)
  int32_t num_kv_heads, rep;
  int32_t log2_bs;             // block size: a power of two >= 16
  float scale_log2e;
  rope_tables rope;
  // fused append (may be null): the step's new K / V rows [T][Hkv][D] (K before
  // RoPE when rope tables are given); a sequence's new rows (positions pos0 ..) are
  // read from here, K rotated in LDS, and stored to their pool slots by the
  // workgroup of block pair 0
  const char* k_new;
  int64_t k_new_row_bytes;
  const char* v_new;
  int64_t v_new_row_bytes;
};

template <int D>
struct pshape {
  static constexpr int RB = 2 * D;              // bytes per K or V row
  static constexpr int TB = 16 * RB;            // bytes of a 16-position K (or V) tile
  static constexpr int TILE = 2 * TB;           // K then V
  static constexpr int VCOLS = RB / 16;         // 16-byte chunks per row
  static constexpr int TLD = TB / 1024;         // direct loads per tile, of K and of V each
  static constexpr int KS = D / 32;             // k-slices of q.k
  static constexpr int NSL = D / 16;            // 16-dim slices of O
  static constexpr int MAXT = TB_PREFILL_STREAM_LDS / TILE;   // tiles a workgroup holds
  static constexpr int HPW = 1;                // query heads per wave
  static constexpr int MAXREP = D == 64 ? 8 : 4;   // two waves per query head: 16 waves at head dim 64, 8 at 128
  // tiles per chunk (a barrier per chunk, the chunk's steps shared evenly by A and
  // B): one chunk holds every range; per-chunk barriers measured slower, also with
  // each chunk's loads issued only two or three chunks ahead so that the first
  // chunks land first (8 x 512 bf16: chunks of 8 tiles 15.2, of 16 13.7, one chunk
  // 12.7 us per layer)
  static constexpr int CH = 64;
  static_assert(MAXT * TILE <= 160 * 1024, "LDS budget of a workgroup");
  static_assert(MAXT <= CH, "one chunk: the tile loads may go out in any order");
};

// The reads of a step's two tiles (A at the given addresses, B one tile further,
// through the instructions' immediate offsets) as MFMA operands, in one asm
// block that ends complete: K rows of both (A operand of S^T) and the transposed
// V rows of both (lo: tile A, hi: tile B). Compiler-visible, each read would
// wait for every direct load of the wave in flight; the chunk's barrier
// already covers them.
template <int KS, int NSL, int OFF>
struct pair_reads;
template <int OFF>
struct pair_reads<2, 4, OFF> {
  static __device__ __forceinline__ void run(const uint32_t (&ka)[2], const uint32_t (&va)[4], su32x4_t (&k)[4],
                                             su32x2_t (&lo)[4], su32x2_t (&hi)[4]) {
    asm volatile(
        "ds_read_b128 %0, %12\n\tds_read_b128 %1, %13\n\t"
        "ds_read_b128 %2, %12 offset:%18\n\tds_read_b128 %3, %13 offset:%18\n\t"
        "ds_read_b64_tr_b16 %4, %14\n\tds_read_b64_tr_b16 %5, %15\n\t"
        "ds_read_b64_tr_b16 %6, %16\n\tds_read_b64_tr_b16 %7, %17\n\t"
        "ds_read_b64_tr_b16 %8, %14 offset:%18\n\tds_read_b64_tr_b16 %9, %15 offset:%18\n\t"
        "ds_read_b64_tr_b16 %10, %16 offset:%18\n\tds_read_b64_tr_b16 %11, %17 offset:%18\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(lo[0]), "=&v"(lo[1]), "=&v"(lo[2]), "=&v"(lo[3]),
          "=&v"(hi[0]), "=&v"(hi[1]), "=&v"(hi[2]), "=&v"(hi[3])
        : "v"(ka[0]), "v"(ka[1]), "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]), "n"(OFF)
        : "memory");
  }
};
template <int OFF>
struct pair_reads<4, 8, OFF> {
  static __device__ __forceinline__ void run(const uint32_t (&ka)[4], const uint32_t (&va)[8], su32x4_t (&k)[8],
                                             su32x2_t (&lo)[8], su32x2_t (&hi)[8]) {
    asm volatile(
        "ds_read_b128 %0, %24\n\tds_read_b128 %1, %25\n\tds_read_b128 %2, %26\n\tds_read_b128 %3, %27\n\t"
        "ds_read_b128 %4, %24 offset:%36\n\tds_read_b128 %5, %25 offset:%36\n\t"
        "ds_read_b128 %6, %26 offset:%36\n\tds_read_b128 %7, %27 offset:%36\n\t"
        "ds_read_b64_tr_b16 %8, %28\n\tds_read_b64_tr_b16 %9, %29\n\t"
        "ds_read_b64_tr_b16 %10, %30\n\tds_read_b64_tr_b16 %11, %31\n\t"
        "ds_read_b64_tr_b16 %12, %32\n\tds_read_b64_tr_b16 %13, %33\n\t"
        "ds_read_b64_tr_b16 %14, %34\n\tds_read_b64_tr_b16 %15, %35\n\t"
        "ds_read_b64_tr_b16 %16, %28 offset:%36\n\tds_read_b64_tr_b16 %17, %29 offset:%36\n\t"
        "ds_read_b64_tr_b16 %18, %30 offset:%36\n\tds_read_b64_tr_b16 %19, %31 offset:%36\n\t"
        "ds_read_b64_tr_b16 %20, %32 offset:%36\n\tds_read_b64_tr_b16 %21, %33 offset:%36\n\t"
        "ds_read_b64_tr_b16 %22, %34 offset:%36\n\tds_read_b64_tr_b16 %23, %35 offset:%36\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(k[0]), "=&v"(k[1]), "=&v"(k[2]), "=&v"(k[3]), "=&v"(k[4]), "=&v"(k[5]), "=&v"(k[6]), "=&v"(k[7]),
          "=&v"(lo[0]), "=&v"(lo[1]), "=&v"(lo[2]), "=&v"(lo[3]), "=&v"(lo[4]), "=&v"(lo[5]), "=&v"(lo[6]), "=&v"(lo[7]),
          "=&v"(hi[0]), "=&v"(hi[1]), "=&v"(hi[2]), "=&v"(hi[3]), "=&v"(hi[4]), "=&v"(hi[5]), "=&v"(hi[6]), "=&v"(hi[7])
        : "v"(ka[0]), "v"(ka[1]), "v"(ka[2]), "v"(ka[3]), "v"(va[0]), "v"(va[1]), "v"(va[2]), "v"(va[3]),
          "v"(va[4]), "v"(va[5]), "v"(va[6]), "v"(va[7]), "n"(OFF)
        : "memory");
  }
};

// The ones of the row-sum product (an all-ones A operand turns P into its column sums).
template <typename Tag>
__device__ __forceinline__ su32x4_t ones_operand() {
  const uint32_t one2 = std::is_same<Tag, f16_t>::value ? 0x3C003C00u : 0x3F803F80u;
  return su32x4_t{one2, one2, one2, one2};
}

// The online-softmax state of HPW heads x 16 rows (lane (lg, lc) holds row lc):
// the row's reference max m (p <= 2^8 against it; -inf until the row has seen a
// position, with -m taken as 0 then, so that masked scores give p = 0), the raw
// score above which m must move (thr = (m + 8) / (scale log2 e)), its O^T column
// (acc[h][nn] = O^T[16 nn + 4 lg + jj][row lc]) and its sum (every element of l[h]).
template <int NSL, int HPW>
struct pstate {
  float m[HPW], negm[HPW], thr[HPW];
  float4_t acc[HPW][NSL];
  float4_t l[HPW];
  __device__ __forceinline__ void reset() {
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      m[h] = -INFINITY;
      negm[h] = 0.f;
      thr[h] = -INFINITY;
      l[h] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int nn = 0; nn < NSL; ++nn) acc[h][nn] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
  }
};

// One step: tiles t and t + 1 of the workgroup's LDS range (t + 1 stands for
// nothing when bnull) folded into the state of HPW heads of 16 rows; row lc sees
// positions 0 .. prow.
template <typename Tag, int D, int HPW>
__device__ __forceinline__ void pstep(pstate<D / 16, HPW>& st, const su32x4_t (&q)[HPW][D / 32], uint32_t lds_tile,
                                      const uint32_t (&ka0)[D / 32], const uint32_t (&va0)[D / 16], int t, bool bnull,
                                      int prow, int first_pos, float sl2e, float inv_sl2e, su32x4_t ones) {
  using S = pshape<D>;
  using M = smath<Tag>;
  constexpr int KS = S::KS, NSL = S::NSL, TILE = S::TILE;
  const int lane = threadIdx.x & 63, lg = lane >> 4;
  uint32_t ka[KS], va[NSL];
#pragma unroll
  for (int s = 0; s < KS; ++s) ka[s] = lds_tile + ka0[s];
#pragma unroll
  for (int nn = 0; nn < NSL; ++nn) va[nn] = lds_tile + va0[nn];
  su32x4_t kv[2 * KS];
  su32x2_t vlo[NSL], vhi[NSL];
  pair_reads<KS, NSL, TILE>::run(ka, va, kv, vlo, vhi);
  float4_t sa[HPW], sb[HPW];
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    sa[h] = float4_t{0.f, 0.f, 0.f, 0.f};
    sb[h] = float4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      sa[h] = M::mfma32(kv[s], q[h][s], sa[h]);
      sb[h] = M::mfma32(kv[KS + s], q[h][s], sb[h]);
    }
  }
  if (16 * t + 31 > first_pos || bnull) {          // the step crosses the diagonal of some row
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const bool ma = 16 * t + 4 * lg + jj > prow;
      const bool mb = bnull || 16 * t + 16 + 4 * lg + jj > prow;
#pragma unroll
      for (int h = 0; h < HPW; ++h) {
        if (ma) sa[h][jj] = -INFINITY;
        if (mb) sb[h][jj] = -INFINITY;
      }
    }
  }
  // the reference max moves only when some row outgrows it by 8 (rare after a
  // row's first steps): then the exact row maxima, and that head's state rescaled
  float lm[HPW];
  bool grow = false;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    lm[h] = max3_f32(max3_f32(sa[h][0], sa[h][1], sa[h][2]), max3_f32(sa[h][3], sb[h][0], sb[h][1]),
                     max_f32(sb[h][2], sb[h][3]));
    grow = grow || lm[h] > st.thr[h];
  }
  if (__any(grow)) {
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const float rm = max_xor32(max_xor16(lm[h])) * sl2e;
      const float m_new = fmaxf(st.m[h], rm);
      if (m_new != -INFINITY) {                    // the row has seen a position
        const float alpha = fast_exp2(st.m[h] - m_new);   // 0 while m = -inf
        st.m[h] = m_new;
        st.negm[h] = -m_new;
        st.thr[h] = (m_new + 8.f) * inv_sl2e;
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) st.acc[h][nn] *= alpha;
        st.l[h] *= alpha;
      }
    }
  }
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    float pv[8];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      pv[jj] = fast_exp2(fmaf(sa[h][jj], sl2e, st.negm[h]));
      pv[4 + jj] = fast_exp2(fmaf(sb[h][jj], sl2e, st.negm[h]));
    }
    const su32x4_t pb = M::pack8(pv);
#pragma unroll
    for (int nn = 0; nn < NSL; ++nn)
      st.acc[h][nn] = M::mfma32(su32x4_t{vlo[nn].x, vlo[nn].y, vhi[nn].x, vhi[nn].y}, pb, st.acc[h][nn]);
    st.l[h] = M::mfma32(ones, pb, st.l[h]);
  }
}

// The output rows of a state: rows 16 blk .. of the sequence's new rows, heads hd0 .. hd0 + nh - 1.
template <typename Tag, int D, int HPW>
__device__ __forceinline__ void pwrite(const prefill_args& a, const pstate<D / 16, HPW>& st, int row0, int nrows,
                                       int blk, int hd0, int nh) {
  typedef typename smath<Tag>::scalar_t scalar_t;
  constexpr int RB = 2 * D, NSL = D / 16;
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int my_row = 16 * blk + lc;
  if (my_row >= nrows) return;
  typedef scalar_t s4_t __attribute__((ext_vector_type(4)));
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    if (h >= nh) break;
    const float inv = 1.f / st.l[h][0];
    char* const orow = a.out + (int64_t)(row0 + my_row) * a.out_row_bytes + (int64_t)(hd0 + h) * RB;
#pragma unroll
    for (int nn = 0; nn < NSL; ++nn) {
      s4_t o;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) o[jj] = (scalar_t)(st.acc[h][nn][jj] * inv);
      st8_through(orow + 2 * (16 * nn + 4 * lg), o);
    }
  }
}

// q rows 16 blk .. (heads hd0 ..) as loaded; rows past the step's last row are zero.
// The loads are left in flight (nothing here uses them).
template <int D, int HPW>
__device__ __forceinline__ void pload_q(const prefill_args& a, vec16 (&qv)[HPW][D / 32], int row0, int nrows, int blk,
                                       int hd0, int nh) {
  constexpr int RB = 2 * D, KS = D / 32;
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int my_row = 16 * blk + lc;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
#pragma unroll
    for (int s = 0; s < KS; ++s) qv[h][s] = zero16();
    if (my_row < nrows && h < nh) {
      const char* qrow = a.q + (int64_t)(row0 + my_row) * a.q_row_bytes + (int64_t)(hd0 + h) * RB + 16 * lg;
#pragma unroll
      for (int s = 0; s < KS; ++s) qv[h][s] = ld16(qrow + 64 * s);
    }
  }
}

// The loaded q rows rotated at the rows' positions (with RoPE) as B operands.
template <typename Tag, int D, int HPW>
__device__ __forceinline__ void prot_q(const prefill_args& a, vec16 (&qv)[HPW][D / 32], su32x4_t (&q)[HPW][D / 32],
                                      int pos0, int nrows, int blk, int nh) {
  typedef typename smath<Tag>::scalar_t scalar_t;
  constexpr int KS = D / 32;
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int my_row = 16 * blk + lc;
#pragma unroll
  for (int h = 0; h < HPW; ++h) {
    if (a.rope.cos && my_row < nrows && h < nh) {   // slices s and s + KS/2 pair (dims i and i + D/2)
      const int64_t r = a.rope.row(pos0 + my_row, D / 2) + 8 * lg;
#pragma unroll
      for (int s = 0; s < KS / 2; ++s)
        rope_pair<scalar_t>(qv[h][s], qv[h][s + KS / 2], a.rope.cos + r + 32 * s, a.rope.sin + r + 32 * s);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) q[h][s] = __builtin_bit_cast(su32x4_t, qv[h][s]);
  }
}

template <typename Tag, int D>
__global__ __launch_bounds__(pshape<D>::MAXREP / pshape<D>::HPW * 128, 1) void paged_prefill_stream_kernel(
    const prefill_args a) {
  using S = pshape<D>;
  constexpr int RB = S::RB, TB = S::TB, TILE = S::TILE, VCOLS = S::VCOLS, TLD = S::TLD, KS = S::KS, NSL = S::NSL;
  constexpr int CH = S::CH, HPW = S::HPW;
  __shared__ __align__(1024) char lds[S::MAXT * TILE];

  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
  const int lane = threadIdx.x & 63, lc = lane & 15, lg = lane >> 4;
  const int4 wi = a.work[blockIdx.x];
  const int row0 = wi.x, seq = wi.y, pos0 = wi.z;
  const int nrows = wi.w & 0xFFFF, pair = (wi.w >> 16) & 0xFF, kvh = (wi.w >> 24) & 0x7F;
  const int rep = a.rep;
  const int G = (rep + HPW - 1) / HPW;            // head groups, two waves (A, B) each
  const int NW = 2 * G;
  // Waves onto (head group g, role). Waves w and w + 4 of a workgroup share a SIMD
  // (measured: the first SIMD rotates between workgroups, the grouping by w % 4 does
  // not), so with an odd number of groups (2 G waves, G > 1) waves w % 4 = 0, 1 share
  // their SIMD with one wave more than waves w % 4 = 2, 3. Groups 0 .. G - 2 then put A
  // on such a busier SIMD (w % 4 = 0, 1) and B on a quieter one (w % 4 = 2, 3), B taking
  // G / (2 (G - 1)) of the group's steps (sb24 in 24ths); the last group takes waves
  // 2 G - 2 (A) and 2 G - 1 (B), evenly: every SIMD then carries G / 4 groups of steps.
  // B's share never falls below the earlier block it must take (<= half the steps).
  // An even number of groups is balanced as it is: A = wave g, B = wave G + g, evenly.
  int g, sb24 = 12;
  bool role_b;
  if ((G & 1) && G > 1) {
    const int K = G - 1;
    if (wave < 2 * K) {
      g = 2 * (wave >> 2) + (wave & 1);
      role_b = (wave & 3) >= 2;
      sb24 = 12 * G / K;
    } else {
      g = K;
      role_b = wave == 2 * K + 1;
    }
  } else {
    g = wave % G;
    role_b = wave >= G;
  }
  const int hd0 = kvh * rep + g * HPW;
  const int nh = min(HPW, rep - g * HPW);
  const int nb = (nrows + 15) >> 4;
  const int blk_l = nb - 1 - pair;                // the later block
  const bool has_e = pair < blk_l;                // the earlier block (none for a lone middle block)
  const int ctx = pos0 + nrows;                   // context of the sequence after this step
  const int TL = (pos0 + min(nrows, 16 * (blk_l + 1)) + 15) >> 4;   // tiles of the later block = the range
  const int TE = has_e ? (pos0 + 16 * (pair + 1) + 15) >> 4 : 0;
  const int T = TL;                                // (host-checked: T < MAXT)
  // Wave A and wave B of a head group share the later block (B hands its partial
  // state to A at the end); B also takes the earlier block.
  const int sl = (TL + 1) >> 1, se = (TE + 1) >> 1;   // steps (tile pairs) of the two blocks

  // q rows, then the block ids of this wave's tiles (tile t by wave t % NW; lane j: the
  // wave's j-th tile). A tile load waits for the block ids (and with them q) only when the
  // wave has tiles with pool rows (rows before pos0): a fresh prefill's tiles go out right
  // after the work item; q is needed only once the range has landed
  const int blk_a = role_b && has_e ? pair : blk_l;   // the current task's block; B's second task: blk_l
  vec16 qra[HPW][KS], qrb[HPW][KS];
  pload_q<D, HPW>(a, qra, row0, nrows, blk_a, hd0, nh);
  if (role_b && has_e) pload_q<D, HPW>(a, qrb, row0, nrows, blk_l, hd0, nh);
  int myb = 0;
  {
    const int32_t* table = a.block_tables + (int64_t)seq * a.max_nb;
    const int tl = wave + NW * lane;
    if (tl < T) myb = table[(tl << 4) >> a.log2_bs];   // checked where it is used
  }

  // ---- the workgroup's K/V range into LDS: tile t by wave t % NW ----
  const int64_t head_bytes = ((int64_t)1 << a.log2_bs) * RB;     // one kv head's K (or V) rows of a block
  const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * head_bytes;
  const uint32_t v_off = (uint32_t)(a.num_kv_heads * head_bytes);
  const int sub_mask = (1 << (a.log2_bs - 4)) - 1;                // 16-position tiles per block - 1
  {
    uint32_t koff[TLD], voff[TLD];
#pragma unroll
    for (int i = 0; i < TLD; ++i) {
      const int f = 64 * i + lane;
      const int r = f / VCOLS, cs = f % VCOLS;
      koff[i] = (uint32_t)(r * RB + 16 * (cs ^ stream_kswz(r)));
      voff[i] = v_off + (uint32_t)(r * RB + 16 * (cs ^ stream_vswz(r)));
    }
    // the tiles that hold pool rows (rows before pos0) first, behind one wait for the
    // block ids while nothing else is in flight; then those holding only new rows, which
    // need no block id, so that a fresh prefill's tiles go out right after the work item
    // (the range is one chunk, so the order is free)
    auto issue = [&](auto pool_pass) {
      constexpr bool POOL = decltype(pool_pass)::value;
      for (int j = 0; wave + NW * j < T; ++j) {
        const int t = wave + NW * j;
        char* const dst = lds + t * TILE;
        const bool new_rows = a.k_new != nullptr && 16 * t + 15 >= pos0;
        const bool pool_rows = !new_rows || 16 * t < pos0;
        if (pool_rows != POOL) continue;
        const char* base = a.pool;                   // the tile's rows in the pool (when it holds any)
        if (POOL) {
          int b = __builtin_amdgcn_readlane(myb, j);
          b = (b < 0 || b >= a.num_blocks) ? 0 : b;   // host validates; stay inside the pool
          base = a.pool + (int64_t)b * blk_bytes + kvh * head_bytes + (int64_t)(t & sub_mask) * TB;
        }
        if (new_rows) {
          // a tile holding new rows: those from the step's k / v rows (rows past the
          // sequence's last one repeat it: their scores are masked and their V rows
          // zeroed below), the tile's rows before pos0 from the pool
          const char* kb = a.k_new + (int64_t)row0 * a.k_new_row_bytes + (int64_t)kvh * RB;
          const char* vb = a.v_new + (int64_t)row0 * a.v_new_row_bytes + (int64_t)kvh * RB;
#pragma unroll
          for (int i = 0; i < TLD; ++i) {
            const int f = 64 * i + lane;
            const int r = f / VCOLS, cs = f % VCOLS;
            const int nr = 16 * t + r - pos0;            // the row's index among the new rows
            const int rr = nr < nrows - 1 ? nr : nrows - 1;
            const uint32_t kc = 16u * (uint32_t)(cs ^ stream_kswz(r)), vc = 16u * (uint32_t)(cs ^ stream_vswz(r));
            const char* ks = nr >= 0 ? kb + (int64_t)rr * a.k_new_row_bytes + kc : base + (int64_t)r * RB + kc;
            const char* vs = nr >= 0 ? vb + (int64_t)rr * a.v_new_row_bytes + vc : base + v_off + (int64_t)r * RB + vc;
            s_dma16_l2p(ks, dst + 1024 * i);
            s_dma16_l2p(vs, dst + TB + 1024 * i);
          }
          continue;
        }
#pragma unroll
        for (int i = 0; i < TLD; ++i) {
          s_dma16_l2(koff[i], base, dst + 1024 * i);
          s_dma16_l2(voff[i], base, dst + TB + 1024 * i);
        }
      }
    };
    if (a.k_new == nullptr || 16 * wave < pos0) {   // this wave has pool rows (its first tile is its lowest)
      asm volatile("" : "+v"(myb));
      issue(std::integral_constant<bool, true>());
    }
    issue(std::integral_constant<bool, false>());
    if (wave == 0) {   // the tile after the range stands in for a missing second tile of a step: finite V
      char* const vt = lds + T * TILE + TB;
      for (int f = lane; f < 16 * VCOLS; f += 64) *reinterpret_cast<su32x4_t*>(vt + 16 * f) = su32x4_t{0u, 0u, 0u, 0u};
    }
  }
  // q rotated (RoPE rows loaded now, behind the tiles) and complete here, for the compiler
  // too (no wait inside the loops)
  su32x4_t qa[HPW][KS], qb2[HPW][KS];              // the current task's q; B's second task (the later block)
  prot_q<Tag, D, HPW>(a, qra, qa, pos0, nrows, blk_a, nh);
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int s = 0; s < KS; ++s) qb2[h][s] = su32x4_t{0u, 0u, 0u, 0u};
  if (role_b && has_e) prot_q<Tag, D, HPW>(a, qrb, qb2, pos0, nrows, blk_l, nh);
#pragma unroll
  for (int h = 0; h < HPW; ++h)
#pragma unroll
    for (int s = 0; s < KS; ++s) asm volatile("" : "+v"(qa[h][s]), "+v"(qb2[h][s]));

  // ---- the wave's tasks over their tiles, chunk by chunk as the chunks land ----
  const float sl2e = a.scale_log2e, inv_sl2e = 1.f / a.scale_log2e;
  const su32x4_t ones = ones_operand<Tag>();
  uint32_t ka0[KS], va0[NSL];                       // tile 0's addresses of this lane
  {
    const uint32_t lds0 = s_lds_addr(lds);
#pragma unroll
    for (int s = 0; s < KS; ++s) ka0[s] = lds0 + (uint32_t)(lc * RB + 16 * ((4 * s + lg) ^ stream_kswz(lc)));
    const int rv = 4 * lg + (lc >> 2);
    const int half8 = 8 * (lc & 1);
#pragma unroll
    for (int nn = 0; nn < NSL; ++nn) {
      const int c = ((lc & 3) >> 1) + 2 * nn;
      va0[nn] = lds0 + (uint32_t)(TB + rv * RB + 16 * (c ^ stream_vswz(rv)) + half8);
    }
  }
  // Chunk c holds steps CH/2 c .. CH/2 (c + 1) - 1 (tiles CH c ..). Its steps of the
  // earlier block go to B; its steps of the later block are shared so that A and
  // B have equal work in every chunk (A the first ones, B the rest), so both
  // waves of a head group stream together while the next chunks land. B finishes
  // the earlier block (and writes it) before its first step of the later one.
  pstate<NSL, HPW> st;
  st.reset();
  bool in_e = role_b && has_e;                    // B is still on the earlier block
  const int nch = (T + CH - 1) / CH;
  for (int c = 0; c < nch; ++c) {
    {   // this wave's tiles of chunk c have landed (its later tiles may still be in flight)
      int after = 0;
      for (int tt = wave; tt < T; tt += NW) after += tt >= CH * (c + 1);
      s_vm_wait_le(2 * TLD * after);
      if (a.k_new != nullptr && a.rope.cos != nullptr) {
        // RoPE of the new K rows this wave loaded (the reference rotates k before the
        // write, model.py:125,128): chunk cs of a row pairs with chunk cs + VCOLS/2
        // (dims i and i + D/2), at the row's position; the bits of tb_kv_append_rope
        for (int tt = wave; tt < min(T, CH * (c + 1)); tt += NW) {
          if (tt < CH * c || 16 * tt + 15 < pos0) continue;
          char* const kt = lds + tt * TILE;
          for (int f = lane; f < 16 * (VCOLS / 2); f += 64) {
            const int r = f / (VCOLS / 2), cs = f % (VCOLS / 2);
            const int p = 16 * tt + r;
            if (p < pos0 || p >= ctx) continue;
            vec16* const x1 = reinterpret_cast<vec16*>(kt + r * RB + 16 * (cs ^ stream_kswz(r)));
            vec16* const x2 = reinterpret_cast<vec16*>(kt + r * RB + 16 * ((cs + VCOLS / 2) ^ stream_kswz(r)));
            vec16 v1 = *x1, v2 = *x2;
            const int64_t rr = a.rope.row(p, D / 2) + 8 * cs;
            rope_pair<typename smath<Tag>::scalar_t>(v1, v2, a.rope.cos + rr, a.rope.sin + rr);
            *x1 = v1;
            *x2 = v2;
          }
        }
      }
      if ((T - 1) / CH == c && (T - 1) % NW == wave && 16 * T > ctx) {   // V rows past the context: zeros
        char* const vt = lds + (T - 1) * TILE + TB;
        const int r0 = ctx - 16 * (T - 1);
        for (int f = lane; f < 16 * VCOLS; f += 64)
          if (f / VCOLS >= r0) *reinterpret_cast<su32x4_t*>(vt + 16 * f) = su32x4_t{0u, 0u, 0u, 0u};
      }
    }
    __syncthreads();
    if (c == 0 && pair == 0 && a.k_new != nullptr) {
      // the fused append: the workgroup of block pair 0 holds every new row of the
      // sequence for this kv head; each wave stores the new-row tiles it loaded,
      // from LDS (chunk f of a tile holds row f / VCOLS, chunk (f % VCOLS) ^ swizzle)
      for (int j = 0; wave + NW * j < T; ++j) {
        const int t = wave + NW * j;
        if (16 * t + 15 < pos0) continue;
        const int first = max(0, pos0 - 16 * t);           // the tile's rows first .. valid - 1 are new
        const int valid = min(16, pos0 + nrows - 16 * t);
        int b = __builtin_amdgcn_readlane(myb, j);
        b = (b < 0 || b >= a.num_blocks) ? 0 : b;   // host validates; stay inside the pool
        char* const pk = a.pool + (int64_t)b * blk_bytes + kvh * head_bytes +
                         (int64_t)(t & sub_mask) * TB;
        const char* const src = lds + t * TILE;
#pragma unroll
        for (int i = 0; i < TLD; ++i) {
          const int f = 64 * i + lane;
          const int r = f / VCOLS, cs = f % VCOLS;
          if (r >= first && r < valid) {
            st16_through(pk + r * RB + 16 * (cs ^ stream_kswz(r)), *reinterpret_cast<const vec16*>(src + 16 * f));
            st16_through(pk + v_off + r * RB + 16 * (cs ^ stream_vswz(r)),
                         *reinterpret_cast<const vec16*>(src + TB + 16 * f));
          }
        }
      }
    }
    const int s0 = (CH / 2) * c;
    const int nl = max(0, min(s0 + CH / 2, sl) - s0);    // later-block steps in the chunk
    const int ne = max(0, min(s0 + CH / 2, se) - s0);    // earlier-block steps in the chunk
    const int nbl = min(nl, max(0, sb24 * (nl + ne) / 24 - ne));   // B's share of the later block's steps
    const int na = nl - nbl;
    // this wave's steps of the chunk: B's earlier-block ones first, then its share
    // of the later block; one call site keeps the registers of one step live
    const int ne_me = role_b && in_e ? ne : 0;
    const int nl_me = role_b ? nl - na : na;
    const int l_first = role_b ? s0 + na : s0;
    const uint32_t lds0 = s_lds_addr(lds);
    for (int i = 0; i < ne_me + nl_me; ++i) {
      const bool e_step = i < ne_me;
      const int k = e_step ? s0 + i : l_first + (i - ne_me);
      const int bk = e_step ? pair : blk_l;
      const int tk = e_step ? TE : TL;
      pstep<Tag, D, HPW>(st, qa, lds0 + 2 * k * TILE, ka0, va0, 2 * k, 2 * k + 1 >= tk,
                         pos0 + min(16 * bk + lc, nrows - 1), pos0 + 16 * bk, sl2e, inv_sl2e, ones);
      if (e_step && i == ne_me - 1 && k + 1 >= se) {   // the earlier block is done: written whole
        pwrite<Tag, D, HPW>(a, st, row0, nrows, pair, hd0, nh);
        st.reset();
#pragma unroll
        for (int h = 0; h < HPW; ++h)
#pragma unroll
          for (int s2 = 0; s2 < KS; ++s2) qa[h][s2] = qb2[h][s2];
        in_e = false;
      }
    }
  }
  // B took later-block steps in some chunk (the same rule decides it for every wave)
  bool b_has_l = false;
  for (int c = 0; c < nch; ++c) {
    const int s0 = (CH / 2) * c;
    const int nl = max(0, min(s0 + CH / 2, sl) - s0), ne = max(0, min(s0 + CH / 2, se) - s0);
    b_has_l = b_has_l || min(nl, max(0, sb24 * (nl + ne) / 24 - ne)) > 0;
  }
  const bool has_l2 = b_has_l;

  // ---- the later block: A's part and B's part merged (log-sum-exp), by A ----
  constexpr int SACC = HPW * NSL * 64 * 16, SGRP = SACC + HPW * 64 * 8;
  if (has_l2) {
    __syncthreads();                                // every wave is done with the tiles
    char* const slot = lds + g * SGRP;
    if (role_b) {
#pragma unroll
      for (int h = 0; h < HPW; ++h) {
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn)
          *reinterpret_cast<float4_t*>(slot + ((h * NSL + nn) * 64 + lane) * 16) = st.acc[h][nn];
        *reinterpret_cast<float2*>(slot + SACC + (h * 64 + lane) * 8) = make_float2(st.m[h], st.l[h][0]);
      }
    }
    __syncthreads();
    if (!role_b) {
#pragma unroll
      for (int h = 0; h < HPW; ++h) {
        const float2 mlb = *reinterpret_cast<const float2*>(slot + SACC + (h * 64 + lane) * 8);
        const float m = fmaxf(st.m[h], mlb.x);    // finite: A's part holds position 0
        const float wa = fast_exp2(st.m[h] - m), wb = fast_exp2(mlb.x - m);   // 0 for a part with m = -inf
#pragma unroll
        for (int nn = 0; nn < NSL; ++nn) {
          const float4_t vb = *reinterpret_cast<const float4_t*>(slot + ((h * NSL + nn) * 64 + lane) * 16);
          st.acc[h][nn] = st.acc[h][nn] * wa + vb * wb;
        }
        st.l[h] = float4_t{1.f, 1.f, 1.f, 1.f} * (st.l[h][0] * wa + mlb.y * wb);
      }
    }
  }
  if (!role_b) pwrite<Tag, D, HPW>(a, st, row0, nrows, blk_l, hd0, nh);
}

}  // namespace tb

// ---------------------------------------------------------------------------
// Host side: the work list (no device call, nothing allocated) and the launch.

#include <algorithm>
#include <vector>

namespace {

int prefill_max_tiles(int head_dim) {
  return head_dim == 64 ? tb::pshape<64>::MAXT : head_dim == 128 ? tb::pshape<128>::MAXT : 0;
}

}  // namespace

// the tile after a workgroup's range must lie in its LDS too
extern "C" int32_t tb_prefill_stream_max_context(int32_t head_dim) {
  return head_dim == 64 || head_dim == 128 ? 16 * (prefill_max_tiles(head_dim) - 1) : 0;
}

extern "C" int32_t tb_prefill_stream_max_group(int32_t head_dim) {
  return head_dim == 64 ? tb::pshape<64>::MAXREP : head_dim == 128 ? tb::pshape<128>::MAXREP : 0;
}

extern "C" int32_t tb_prefill_work_count(const int32_t* new_rows, int32_t num_seqs, int32_t num_kv_heads) {
  if (num_seqs < 0 || num_kv_heads <= 0 || (num_seqs > 0 && !new_rows)) return -1;
  int64_t n = 0;
  for (int i = 0; i < num_seqs; ++i) {
    if (new_rows[i] <= 0) return -1;
    const int nb = (new_rows[i] + 15) / 16;
    n += (int64_t)((nb + 1) / 2) * num_kv_heads;
  }
  return n > INT32_MAX ? -1 : (int32_t)n;
}

extern "C" int32_t tb_build_prefill_work(const int32_t* first_row, const int32_t* seq_index, const int32_t* pos0,
                                         const int32_t* new_rows, int32_t num_seqs, int32_t num_kv_heads,
                                         int32_t head_dim, int32_t num_xcds, int32_t* work, int32_t capacity,
                                         int32_t* max_tiles) {
  const int mt = prefill_max_tiles(head_dim);
  if (mt == 0 || num_kv_heads <= 0 || num_kv_heads > 127 || num_seqs < 0 || num_xcds <= 0 || !max_tiles)
    return TB_ERR_INVALID_ARG;
  if (num_seqs > 0 && (!first_row || !seq_index || !pos0 || !new_rows)) return TB_ERR_INVALID_ARG;
  const int32_t need = tb_prefill_work_count(new_rows, num_seqs, num_kv_heads);
  if (need < 0) return TB_ERR_INVALID_ARG;
  if (need > capacity || (need > 0 && !work)) return TB_ERR_INVALID_ARG;
  for (int i = 0; i < num_seqs; ++i) {
    if (pos0[i] < 0 || first_row[i] < 0 || seq_index[i] < 0 || new_rows[i] > 0xFFFF) return TB_ERR_INVALID_ARG;
    if ((int64_t)pos0[i] + new_rows[i] > 16 * (int64_t)(mt - 1)) return TB_ERR_UNSUPPORTED;   // context past the LDS
  }
  // Groups = (sequence, kv head): every pair of a group reads the same K/V, so a
  // group's entries go to one XCD (entry g runs on XCD g % num_xcds), whose L2
  // then serves the group's re-reads. Groups are placed longest first on the
  // least loaded XCD; the list takes one entry of each XCD in turn (an XCD whose
  // list ran out lends the slot to the longest remaining list).
  struct group { int seq, kvh, pairs; int64_t weight; };
  std::vector<group> groups;
  for (int i = 0; i < num_seqs; ++i) {
    const int nb = (new_rows[i] + 15) / 16;
    for (int h = 0; h < num_kv_heads; ++h)
      groups.push_back({i, h, (nb + 1) / 2, (int64_t)((nb + 1) / 2) * (pos0[i] + new_rows[i])});
  }
  std::stable_sort(groups.begin(), groups.end(), [](const group& x, const group& y) { return x.weight > y.weight; });
  const int X = num_xcds;
  std::vector<std::vector<int>> bins(X);   // per XCD: entries as (group << 8 | pair)
  std::vector<int64_t> load(X, 0);
  for (int gi = 0; gi < (int)groups.size(); ++gi) {
    const int x = (int)(std::min_element(load.begin(), load.end()) - load.begin());
    load[x] += groups[gi].weight;
    for (int p = 0; p < groups[gi].pairs; ++p) bins[x].push_back(gi << 8 | p);
  }
  std::vector<size_t> next(X, 0);
  int n = 0, tiles = 0;
  while (n < need) {
    for (int x = 0; x < X && n < need; ++x) {
      int src = x;
      if (next[x] >= bins[x].size()) {   // lend the slot
        size_t best = 0;
        for (int y = 0; y < X; ++y)
          if (bins[y].size() - next[y] > best) best = bins[y].size() - next[y], src = y;
      }
      const int e = bins[src][next[src]++];
      const group& g = groups[e >> 8];
      const int p = e & 0xFF, i = g.seq;
      const int nb = (new_rows[i] + 15) / 16;
      const int range = pos0[i] + std::min(new_rows[i], 16 * (nb - p));
      tiles = std::max(tiles, (range + 15) / 16);
      int32_t* w = work + 4 * (int64_t)n++;
      w[0] = first_row[i];
      w[1] = seq_index[i];
      w[2] = pos0[i];
      w[3] = new_rows[i] | (p << 16) | (g.kvh << 24);
    }
  }
  *max_tiles = tiles;
  return TB_OK;
}

namespace {

template <typename Tag, int D>
void launch_prefill_stream(const tb::prefill_args& a, int num_work, hipStream_t stream) {
  constexpr int HPW = tb::pshape<D>::HPW;
  const int waves = 2 * ((a.rep + HPW - 1) / HPW);
  hipLaunchKernelGGL((tb::paged_prefill_stream_kernel<Tag, D>), dim3(num_work), dim3(64 * waves), 0, stream, a);
}

}  // namespace

extern "C" int32_t tb_paged_prefill(const void* q, int64_t q_row_stride, void* pool, int64_t num_blocks,
                                    void* out, int64_t out_row_stride, const int32_t* block_tables,
                                    int32_t max_blocks_per_seq, const int32_t* work, int32_t num_work,
                                    int32_t max_tiles, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                    int32_t block_size, float scale, int32_t dtype, const void* k_new,
                                    int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                                    const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                                    hipStream_t stream) {
  TB_CHECK_ARG(num_work >= 0 && num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0);
  if (num_work == 0) return TB_OK;
  TB_CHECK_ARG(q && pool && out && block_tables && work && num_blocks > 0 && max_blocks_per_seq > 0);
  TB_CHECK_ARG(q_row_stride > 0 && out_row_stride > 0 && scale > 0.f);
  const int rep = num_heads / num_kv_heads;
  if (dtype != TB_DTYPE_F16 && dtype != TB_DTYPE_BF16) return TB_ERR_UNSUPPORTED;
  if ((head_dim != 64 && head_dim != 128) || num_kv_heads > 127) return TB_ERR_UNSUPPORTED;
  if (rep > (head_dim == 64 ? tb::pshape<64>::MAXREP : tb::pshape<128>::MAXREP)) return TB_ERR_UNSUPPORTED;
  if (block_size < 16 || (block_size & (block_size - 1))) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(max_tiles >= 0);
  if (max_tiles >= prefill_max_tiles(head_dim)) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(!rope_cos == !rope_sin && (!rope_cos || rope_max_position > 0));
  TB_CHECK_ARG(!k_new == !v_new);
  if (k_new) {
    TB_CHECK_ARG(k_row_stride >= (int64_t)num_kv_heads * head_dim && v_row_stride >= (int64_t)num_kv_heads * head_dim);
    TB_CHECK_ARG((((uintptr_t)k_new | (uintptr_t)v_new) & 15u) == 0 && (k_row_stride * 2) % 16 == 0 &&
                 (v_row_stride * 2) % 16 == 0);
    TB_CHECK_ARG(16 * 2 * k_row_stride < ((int64_t)1 << 31) && 16 * 2 * v_row_stride < ((int64_t)1 << 31));
  }
  tb::prefill_args a{};
  a.q = static_cast<const char*>(q);
  a.q_row_bytes = q_row_stride * 2;
  a.pool = static_cast<char*>(pool);
  a.num_blocks = num_blocks;
  a.out = static_cast<char*>(out);
  a.out_row_bytes = out_row_stride * 2;
  a.block_tables = block_tables;
  a.max_nb = max_blocks_per_seq;
  a.work = reinterpret_cast<const int4*>(work);
  a.num_kv_heads = num_kv_heads;
  a.rep = rep;
  int lb = 0;
  while ((1 << lb) < block_size) ++lb;
  a.log2_bs = lb;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.rope = tb::rope_tables{rope_cos, rope_sin, rope_max_position};
  a.k_new = static_cast<const char*>(k_new);
  a.k_new_row_bytes = k_row_stride * 2;
  a.v_new = static_cast<const char*>(v_new);
  a.v_new_row_bytes = v_row_stride * 2;
  if (dtype == TB_DTYPE_F16)
    head_dim == 64 ? launch_prefill_stream<tb::f16_t, 64>(a, num_work, stream)
                   : launch_prefill_stream<tb::f16_t, 128>(a, num_work, stream);
  else
    head_dim == 64 ? launch_prefill_stream<tb::bf16_t, 64>(a, num_work, stream)
                   : launch_prefill_stream<tb::bf16_t, 128>(a, num_work, stream);
  TB_RETURN_LAUNCH_STATUS();
}
