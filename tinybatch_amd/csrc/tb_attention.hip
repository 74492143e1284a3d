// K2 — fused paged attention on the VALU path (decode rows; any query row).
//
// Replaces the per-sequence loop of Qwen2Paged.forward
// (reference src/tinybatch/model.py:130-147): gather of the sequence's blocks
// (kv_cache.py:40-45), GQA repeat_interleave (model.py:135-137), the
// offset-causal mask j <= ctx - q_len + i (model.py:139-145) and
// scaled_dot_product_attention with scale 1/sqrt(D) (model.py:140,146).
//
// Mapping onto CDNA4 (wave64):
// * One wave = one work item = (query row, kv head, head group, partition of
//   P tokens). The wave reads each K/V token row once, through the block table
//   in place, and serves all REP query heads of the GQA group from registers
//   (no repeat_interleave, no gather copy).
// * A K or V tile [BS][D] of one (block, kv head) is contiguous. The wave
//   splits a token row into LPT lanes of 16 bytes (D=64 fp16: 8 lanes), so one
//   wave load instruction moves 1 KiB of consecutive bytes (TPL = 64/LPT
//   tokens).
// * q.k: v_dot2_f32_{f16,bf16} over the lane's 8 elements, then a DPP
//   butterfly over the LPT lanes of the token (fp32 accumulation).
// * p.V: tokens are paired across two consecutive loads and packed with
//   v_perm so that one v_dot2 applies (p_a, p_b) to (v_a[d], v_b[d]); the
//   softmax denominator uses the same rounded p, so numerator and denominator
//   agree.
// * Online softmax over chunks in the base-2 domain (scores pre-scaled by
//   scale*log2(e)), wave-wide max by DPP/ds_bpermute.
// * Split-K: a row longer than P tokens is cut into partitions whose
//   (max, sum, unnormalised acc) partials are merged by a log-sum-exp combine
//   kernel. Rows of one partition write the output directly.
// * Positions >= the row's context are never loaded (stale slots may hold
//   anything, including NaN): their V registers are zero and their scores -inf.
#include "tb_common.h"

namespace tb {

template <typename Tag>
struct math;

template <>
struct math<f16_t> {
  typedef half2_t pair_t;
  static __device__ __forceinline__ pair_t as_pair(uint32_t w) { return __builtin_bit_cast(pair_t, w); }
  static __device__ __forceinline__ float dot2(pair_t a, pair_t b, float c) {
    return __builtin_amdgcn_fdot2(a, b, c, false);
  }
  static __device__ __forceinline__ pair_t pack(float a, float b) {
    pair_t r = {(_Float16)a, (_Float16)b};
    return r;
  }
  static __device__ __forceinline__ uint32_t pack_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, pack(a, b));
  }
};

template <>
struct math<bf16_t> {
  typedef bf162_t pair_t;
  static __device__ __forceinline__ pair_t as_pair(uint32_t w) { return __builtin_bit_cast(pair_t, w); }
  static __device__ __forceinline__ float dot2(pair_t a, pair_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(a, b, c, false);
  }
  static __device__ __forceinline__ pair_t pack(float a, float b) {
    pair_t r = {(__bf16)a, (__bf16)b};
    return r;
  }
  static __device__ __forceinline__ uint32_t pack_bits(float a, float b) {
    return __builtin_bit_cast(uint32_t, pack(a, b));
  }
};

// Shape constants of the VALU kernel for element type Tag and head_dim D.
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
  float* ws_acc;          // [parts][Hq][D]
  float* ws_ml;           // [parts][Hq][2]
  int32_t num_heads;
  int32_t num_kv_heads;
  int32_t rep;            // num_heads / num_kv_heads
  int32_t log2_bs;
  int32_t part_tokens;
  float scale_log2e;
  const char* k_new;      // fused decode append (may be null)
  int64_t k_new_row_bytes;
  const char* v_new;
  int64_t v_new_row_bytes;
};

template <typename Tag, int D, int REP>
__global__ __launch_bounds__(64) void paged_attn_valu_kernel(const attn_args a) {
  using S = valu_shape<Tag, D>;
  constexpr int EB = S::EB, EPL = S::EPL, LPT = S::LPT, TPL = S::TPL;
  constexpr int CH_LOADS = S::CH_LOADS, CH = S::CH;
  constexpr bool F32 = (EB == 4);

  const int lane = threadIdx.x;
  const int j = lane % LPT;  // 16-byte column of the token row
  const int g = lane / LPT;  // token slot inside one wave load

  const int4 wi = a.work[blockIdx.x];
  const int row = wi.x, seq = wi.y, part = wi.z, ctx = wi.w;
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

  const int64_t tile_bytes = (int64_t)bs * D * EB;              // one [BS][D] tile
  const int64_t blk_bytes = 2 * (int64_t)a.num_kv_heads * tile_bytes;
  const int64_t v_off = (int64_t)a.num_kv_heads * tile_bytes;
  const char* pool_kvh = a.pool + kvh * tile_bytes + j * 16;
  const int new_pos = ctx - 1;
  const bool fused = (a.k_new != nullptr);
  const char* k_new_row = fused ? a.k_new + row * a.k_new_row_bytes + (int64_t)kvh * D * EB + j * 16 : nullptr;
  const char* v_new_row = fused ? a.v_new + row * a.v_new_row_bytes + (int64_t)kvh * D * EB + j * 16 : nullptr;

  // Query registers: REP heads x this lane's EPL elements.
  vec16 qv[REP];
  {
    const char* qrow = a.q + row * a.q_row_bytes + j * 16;
#pragma unroll
    for (int h = 0; h < REP; ++h) qv[h] = ld16(qrow + (int64_t)(head0 + h) * D * EB);
  }

  float m_run[REP], l_run[REP], acc[REP][EPL];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m_run[h] = -INFINITY;
    l_run[h] = 0.f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = 0.f;
  }

  // Pool offset of the row's newest position (fused append only). Every lane
  // runs the shuffle; the partition may not contain new_pos, then it is unused.
  int64_t new_off = 0;
  if (fused) {
    const int nb = __shfl(my_blk, ((new_pos - p0) >> a.log2_bs) & 63);
    new_off = (int64_t)nb * blk_bytes + (int64_t)(new_pos & (bs - 1)) * (D * EB);
  }

  vec16 kbuf[CH_LOADS], vbuf[CH_LOADS];

  auto issue = [&](int c0, vec16* kd, vec16* vd) {
#pragma unroll
    for (int i = 0; i < CH_LOADS; ++i) {
      const int tau = c0 + i * TPL + g;
      const int bidx = (tau - p0) >> a.log2_bs;
      const int blk = __shfl(my_blk, bidx & 63);
      const int64_t off = (int64_t)blk * blk_bytes + (int64_t)(tau & (bs - 1)) * (D * EB);
      const char* kp = pool_kvh + off;
      const char* vp = kp + v_off;
      if (fused && tau == new_pos) {
        kp = k_new_row;
        vp = v_new_row;
      }
      if (tau < p1) {
        kd[i] = ld16(kp);
        vd[i] = ld16(vp);
      } else {
        kd[i] = zero16();
        vd[i] = zero16();
      }
    }
  };

  for (int c0 = p0; c0 < p1; c0 += CH) {
    issue(c0, kbuf, vbuf);
    if (fused) {
#pragma unroll
      for (int i = 0; i < CH_LOADS; ++i) {
        const int tau = c0 + i * TPL + g;
        if (tau == new_pos) {
          char* kp = const_cast<char*>(pool_kvh) + new_off;
          st16(kp, kbuf[i]);
          st16(kp + v_off, vbuf[i]);
        }
      }
    }

    // ---- scores (base-2 domain) ----
    float s[CH_LOADS][REP];
#pragma unroll
    for (int i = 0; i < CH_LOADS; ++i) {
      const bool valid = (c0 + i * TPL + g) < p1;
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        float d = 0.f;
        if constexpr (F32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) d = fmaf(bits_to_f32(qv[h].w[e]), bits_to_f32(kbuf[i].w[e]), d);
        } else {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            d = math<Tag>::dot2(math<Tag>::as_pair(qv[h].w[e]), math<Tag>::as_pair(kbuf[i].w[e]), d);
        }
        d = group_sum<LPT>(d);
        s[i][h] = valid ? d * a.scale_log2e : -INFINITY;
      }
    }

    // ---- online-softmax rescale ----
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

    // ---- p.V over token pairs (i, i+1) ----
#pragma unroll
    for (int i = 0; i < CH_LOADS; i += 2) {
      if constexpr (F32) {
#pragma unroll
        for (int h = 0; h < REP; ++h) {
          const float pa = fast_exp2(s[i][h] - m_run[h]);
          const float pb = fast_exp2(s[i + 1][h] - m_run[h]);
          l_run[h] += pa + pb;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[h][e] = fmaf(pb, bits_to_f32(vbuf[i + 1].w[e]), fmaf(pa, bits_to_f32(vbuf[i].w[e]), acc[h][e]));
        }
      } else {
        typedef typename math<Tag>::pair_t pair_t;
        pair_t lo[4], hi[4];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          lo[c] = math<Tag>::as_pair(__builtin_amdgcn_perm(vbuf[i + 1].w[c], vbuf[i].w[c], 0x05040100u));
          hi[c] = math<Tag>::as_pair(__builtin_amdgcn_perm(vbuf[i + 1].w[c], vbuf[i].w[c], 0x07060302u));
        }
        const pair_t ones = math<Tag>::pack(1.f, 1.f);
#pragma unroll
        for (int h = 0; h < REP; ++h) {
          const pair_t p2 = math<Tag>::pack(fast_exp2(s[i][h] - m_run[h]), fast_exp2(s[i + 1][h] - m_run[h]));
          l_run[h] = math<Tag>::dot2(p2, ones, l_run[h]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            acc[h][2 * c] = math<Tag>::dot2(p2, lo[c], acc[h][2 * c]);
            acc[h][2 * c + 1] = math<Tag>::dot2(p2, hi[c], acc[h][2 * c + 1]);
          }
        }
      }
    }
  }

  // ---- reduce over the token slots g of the wave ----
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    l_run[h] = cross_group_sum<LPT>(l_run[h]);
#pragma unroll
    for (int e = 0; e < EPL; ++e) acc[h][e] = cross_group_sum<LPT>(acc[h][e]);
  }

  const int pbeg = a.row_part_off[row];
  const int nparts = a.row_part_off[row + 1] - pbeg;
  if (nparts == 1) {
    if (g == 0) {
      char* orow = a.out + row * a.out_row_bytes + j * 16;
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        const float inv = 1.f / l_run[h];
        vec16 o;
        if constexpr (F32) {
#pragma unroll
          for (int e = 0; e < 4; ++e) o.w[e] = __float_as_uint(acc[h][e] * inv);
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c) o.w[c] = math<Tag>::pack_bits(acc[h][2 * c] * inv, acc[h][2 * c + 1] * inv);
        }
        st16(orow + (int64_t)(head0 + h) * D * EB, o);
      }
    }
  } else {
    const int64_t pidx = pbeg + part;
    if (g == 0) {
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        float* dst = a.ws_acc + (pidx * a.num_heads + head0 + h) * D + j * EPL;
#pragma unroll
        for (int e = 0; e < EPL; e += 4) {
          float4 v4 = make_float4(acc[h][e], acc[h][e + 1], acc[h][e + 2], acc[h][e + 3]);
          *reinterpret_cast<float4*>(dst + e) = v4;
        }
      }
    }
    if (lane < REP) {
      // lane h publishes head h's running max and sum (uniform across the wave)
      float mh = m_run[0], lh = l_run[0];
#pragma unroll
      for (int h = 1; h < REP; ++h) {
        if (lane == h) { mh = m_run[h]; lh = l_run[h]; }
      }
      float* ml = a.ws_ml + (pidx * a.num_heads + head0 + lane) * 2;
      ml[0] = mh;
      ml[1] = lh;
    }
  }
}

// Log-sum-exp merge of the partition partials of one (row, head).
// Grid: (rows, heads); block: D threads, thread d owns output column d.
template <typename Tag, int D>
__global__ __launch_bounds__(128) void combine_partials_kernel(const attn_args a) {
  constexpr int EB = elem<Tag>::bytes;
  const int row = blockIdx.x, head = blockIdx.y, d = threadIdx.x;
  const int pbeg = a.row_part_off[row];
  const int n = a.row_part_off[row + 1] - pbeg;
  if (n <= 1) return;
  float M = -INFINITY;
  for (int p = 0; p < n; ++p) M = fmaxf(M, a.ws_ml[((int64_t)(pbeg + p) * a.num_heads + head) * 2]);
  float L = 0.f, o = 0.f;
  for (int p = 0; p < n; ++p) {
    const int64_t idx = (int64_t)(pbeg + p) * a.num_heads + head;
    const float w = fast_exp2(a.ws_ml[idx * 2] - M);
    L = fmaf(a.ws_ml[idx * 2 + 1], w, L);
    o = fmaf(a.ws_acc[idx * D + d], w, o);
  }
  o = o / L;
  char* dst = a.out + row * a.out_row_bytes + ((int64_t)head * D + d) * EB;
  if constexpr (EB == 4) *reinterpret_cast<float*>(dst) = o;
  else *reinterpret_cast<typename elem<Tag>::type*>(dst) = (typename elem<Tag>::type)o;
}

// ---- dispatch ---------------------------------------------------------------
template <typename Tag, int D, int REP>
static void launch_valu(const attn_args& a, int num_work, int head_groups, hipStream_t stream) {
  hipLaunchKernelGGL((paged_attn_valu_kernel<Tag, D, REP>), dim3(num_work, a.num_kv_heads, head_groups),
                     dim3(64), 0, stream, a);
}

template <typename Tag, int D>
static int dispatch_rep(const attn_args& a, int rep_tile, int num_work, int head_groups, hipStream_t s) {
  switch (rep_tile) {
    case 1: launch_valu<Tag, D, 1>(a, num_work, head_groups, s); return TB_OK;
    case 2: launch_valu<Tag, D, 2>(a, num_work, head_groups, s); return TB_OK;
    case 3: launch_valu<Tag, D, 3>(a, num_work, head_groups, s); return TB_OK;
    case 4: launch_valu<Tag, D, 4>(a, num_work, head_groups, s); return TB_OK;
    case 5: launch_valu<Tag, D, 5>(a, num_work, head_groups, s); return TB_OK;
    case 6: launch_valu<Tag, D, 6>(a, num_work, head_groups, s); return TB_OK;
    case 7: launch_valu<Tag, D, 7>(a, num_work, head_groups, s); return TB_OK;
    case 8: launch_valu<Tag, D, 8>(a, num_work, head_groups, s); return TB_OK;
    default: return TB_ERR_UNSUPPORTED;
  }
}

template <typename Tag>
static int dispatch_dim(const attn_args& a, int D, int rep_tile, int num_work, int head_groups,
                        int num_rows, int max_parts, hipStream_t s) {
  int st;
  if (D == 64) st = dispatch_rep<Tag, 64>(a, rep_tile, num_work, head_groups, s);
  else if (D == 128) st = dispatch_rep<Tag, 128>(a, rep_tile, num_work, head_groups, s);
  else return TB_ERR_UNSUPPORTED;
  if (st != TB_OK) return st;
  if (max_parts > 1) {
    if (D == 64)
      hipLaunchKernelGGL((combine_partials_kernel<Tag, 64>), dim3(num_rows, a.num_heads), dim3(64), 0, s, a);
    else
      hipLaunchKernelGGL((combine_partials_kernel<Tag, 128>), dim3(num_rows, a.num_heads), dim3(128), 0, s, a);
  }
  return TB_OK;
}

static int largest_rep_tile(int rep) {
  for (int t = 8; t >= 1; --t)
    if (rep % t == 0) return t;
  return 1;
}

static int elem_bytes(int32_t dtype) {
  return dtype == TB_DTYPE_F32 ? 4 : (dtype == TB_DTYPE_F16 || dtype == TB_DTYPE_BF16) ? 2 : 0;
}

static int chunk_tokens(int32_t dtype, int head_dim) {
  const int eb = elem_bytes(dtype);
  const int lpt = head_dim * eb / 16;
  return 8 * (64 / lpt);
}

}  // namespace tb

extern "C" int32_t tb_attention_partition_tokens(void) { return 256; }

extern "C" size_t tb_paged_attention_workspace_bytes(int32_t total_partitions, int32_t num_heads,
                                                     int32_t head_dim) {
  if (total_partitions <= 0 || num_heads <= 0 || head_dim <= 0) return 0;
  return (size_t)total_partitions * num_heads * ((size_t)head_dim + 2) * sizeof(float);
}

extern "C" int32_t tb_paged_attention(const void* q, int64_t q_row_stride, void* pool,
                                      int64_t num_blocks, void* out, int64_t out_row_stride,
                                      const int32_t* block_tables, int32_t max_blocks_per_seq,
                                      const int32_t* work_items, int32_t num_work_items,
                                      const int32_t* row_part_offsets, int32_t num_rows,
                                      int32_t max_parts_per_row, int32_t partition_tokens,
                                      int32_t total_partitions, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                      float scale, int32_t dtype, const void* k_new,
                                      int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                                      void* workspace, size_t workspace_bytes, hipStream_t stream) {
  using namespace tb;
  const int eb = elem_bytes(dtype);
  TB_CHECK_ARG(eb > 0);
  TB_CHECK_ARG(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0);
  if (head_dim != 64 && head_dim != 128) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(block_size >= 4 && (block_size & (block_size - 1)) == 0);
  int log2_bs = 0;
  while ((1 << log2_bs) < block_size) ++log2_bs;
  TB_CHECK_ARG(num_rows >= 0 && num_work_items >= 0 && max_blocks_per_seq > 0 && num_blocks > 0);
  // A partition is a whole number of chunks and spans at most 64 blocks.
  TB_CHECK_ARG(partition_tokens > 0 && partition_tokens % chunk_tokens(dtype, head_dim) == 0);
  TB_CHECK_ARG(partition_tokens % block_size == 0 && partition_tokens / block_size <= 64);
  TB_CHECK_ARG(q_row_stride >= (int64_t)num_heads * head_dim);
  TB_CHECK_ARG(out_row_stride >= (int64_t)num_heads * head_dim);
  if (num_work_items == 0) return TB_OK;
  TB_CHECK_ARG(q && pool && out && block_tables && work_items && row_part_offsets);
  TB_CHECK_ARG((((uintptr_t)q | (uintptr_t)pool | (uintptr_t)out) & 15u) == 0);
  TB_CHECK_ARG((q_row_stride * eb) % 16 == 0 && (out_row_stride * eb) % 16 == 0);
  TB_CHECK_ARG(max_parts_per_row >= 1);
  if (max_parts_per_row > 1) {
    TB_CHECK_ARG(workspace != nullptr);
    TB_CHECK_ARG(workspace_bytes >= tb_paged_attention_workspace_bytes(total_partitions, num_heads, head_dim));
    TB_CHECK_ARG(((uintptr_t)workspace & 15u) == 0);
  }
  if (k_new || v_new) {
    TB_CHECK_ARG(k_new && v_new);
    TB_CHECK_ARG(k_row_stride >= (int64_t)num_kv_heads * head_dim && v_row_stride >= (int64_t)num_kv_heads * head_dim);
    TB_CHECK_ARG((((uintptr_t)k_new | (uintptr_t)v_new) & 15u) == 0);
    TB_CHECK_ARG((k_row_stride * eb) % 16 == 0 && (v_row_stride * eb) % 16 == 0);
  }

  const int rep = num_heads / num_kv_heads;
  const int rep_tile = largest_rep_tile(rep);
  const int head_groups = rep / rep_tile;
  TB_CHECK_ARG(num_kv_heads <= 65535 && head_groups <= 65535);

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
  a.ws_acc = (float*)workspace;
  a.ws_ml = workspace ? (float*)workspace + (size_t)total_partitions * num_heads * head_dim : nullptr;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.rep = rep;
  a.log2_bs = log2_bs;
  a.part_tokens = partition_tokens;
  a.scale_log2e = scale * 1.4426950408889634f;
  a.k_new = (const char*)k_new;
  a.k_new_row_bytes = k_row_stride * eb;
  a.v_new = (const char*)v_new;
  a.v_new_row_bytes = v_row_stride * eb;

  int st;
  switch (dtype) {
    case TB_DTYPE_F32: st = dispatch_dim<f32_t>(a, head_dim, rep_tile, num_work_items, head_groups, num_rows, max_parts_per_row, stream); break;
    case TB_DTYPE_F16: st = dispatch_dim<f16_t>(a, head_dim, rep_tile, num_work_items, head_groups, num_rows, max_parts_per_row, stream); break;
    case TB_DTYPE_BF16: st = dispatch_dim<bf16_t>(a, head_dim, rep_tile, num_work_items, head_groups, num_rows, max_parts_per_row, stream); break;
    default: return TB_ERR_INVALID_ARG;
  }
  if (st != TB_OK) return st;
  TB_RETURN_LAUNCH_STATUS();
}
