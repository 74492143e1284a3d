// Host-side builder of a step's metadata for tb_kv_append and tb_paged_attention.
//
// The reference hands its forward pass host lists (src/tinybatch/model.py:101-109:
// positions, seq_slices, block_tables, context_lens, built by LLMEngine.step,
// engine.py:99-126) and turns them into device tensors inside every layer
// (kv_cache.py:35,43; the mask loop of model.py:142-145). These functions take
// the same step as plain arrays - query_start_loc (the slices), padded block
// tables and context lengths - and write the int32 arrays the kernels read
// into caller buffers, once per step. They allocate nothing.
//
// Row i of sequence b (flat row query_start_loc[b] + i) sits at position
// context_lens[b] - q_len[b] + i and sees positions 0 .. that position
// (engine.py:110,117; the mask j <= ctx - q_len + i of model.py:139-145).
#include <stdint.h>
#include <string.h>

#include "../../include/tinybatch_amd.h"

namespace {

constexpr int TILE_MIN_ROWS = 16;       // a sequence needs this many new rows for tiles
constexpr int TILE_MAX_CTX = 4096;      // ... and a context this short (or <= 16 x its new rows)
constexpr int MAX_PARTITION = 8192;     // longest partition_tokens accepted (histogram on the stack)
constexpr int64_t INDEX_LIMIT = (1 << 24) - 1;   // row / item / partition indices share 24 bits

struct Step {
  const int32_t* qsl;
  const int32_t* ctx;
  int32_t B, T, bs, P, rows_per_item;
  bool tile;

  int q(int b) const { return qsl[b + 1] - qsl[b]; }
  int base(int b) const { return ctx[b] - q(b); }   // position of the sequence's first new row
  bool tiled(int b) const {
    const int n = q(b), c = ctx[b];
    return tile && n >= TILE_MIN_ROWS && (c <= TILE_MAX_CTX || c <= 16 * n);
  }
  // partitions of row i of sequence b
  int64_t nparts(int b, int i) const {
    const int64_t row_ctx = (int64_t)base(b) + i + 1;
    const int64_t len = tiled(b) ? TB_PREFILL_TILE_PARTITION : P;
    return (row_ctx + len - 1) / len;
  }
};

int32_t check_step(const Step& s, const int64_t* positions) {
  if (s.B < 0 || s.T < 0 || !s.qsl || (s.B > 0 && !s.ctx)) return TB_ERR_INVALID_ARG;
  if (s.bs <= 0 || (s.bs & (s.bs - 1)) || s.P <= 0 || s.P > MAX_PARTITION) return TB_ERR_INVALID_ARG;
  if (s.rows_per_item < 1 || s.rows_per_item > 16) return TB_ERR_INVALID_ARG;
  if (s.qsl[0] < 0) return TB_ERR_INVALID_ARG;
  for (int b = 0; b < s.B; ++b) {
    if (s.qsl[b + 1] < s.qsl[b]) return TB_ERR_INVALID_ARG;
    if (s.ctx[b] < s.q(b)) return TB_ERR_INVALID_ARG;             // fewer positions than new rows
  }
  if (s.B > 0 && s.qsl[s.B] > s.T) return TB_ERR_INVALID_ARG;
  if (s.T >= INDEX_LIMIT) return TB_ERR_INVALID_ARG;
  if (positions) {
    for (int b = 0; b < s.B; ++b)
      for (int i = 0; i < s.q(b); ++i)
        if (positions[s.qsl[b] + i] != (int64_t)s.base(b) + i) return TB_ERR_INVALID_ARG;
  }
  return TB_OK;
}

// Work items are issued shortest partition first (stable), tiles longest first
// (stable): a counting sort over the lengths, whose histogram lives on the stack.
struct Counts {
  int64_t work = 0, tiles = 0, split = 0, parts = 0, max_parts = 0;
};

template <typename WorkFn, typename TileFn, typename RowFn>
void walk(const Step& s, WorkFn&& on_work, TileFn&& on_tile, RowFn&& on_row) {
  for (int b = 0; b < s.B; ++b) {
    const int n = s.q(b), r0 = s.qsl[b];
    for (int i = 0; i < n; ++i) on_row(r0 + i, s.nparts(b, i));
    if (n == 0) continue;
    if (s.tiled(b)) {
      for (int r = 0; r < n; r += TB_PREFILL_TILE_ROWS) {
        const int rows = n - r < TB_PREFILL_TILE_ROWS ? n - r : TB_PREFILL_TILE_ROWS;
        const int pos0 = s.base(b) + r;
        const int end = pos0 + rows;                      // positions the tile's last row sees
        const int np = (end + TB_PREFILL_TILE_PARTITION - 1) / TB_PREFILL_TILE_PARTITION;
        for (int part = 0; part < np; ++part) {
          const int rest = end - part * TB_PREFILL_TILE_PARTITION;
          on_tile(r0 + r, b, rows | (part << 8), pos0,
                  rest < TB_PREFILL_TILE_PARTITION ? rest : TB_PREFILL_TILE_PARTITION);
        }
      }
      continue;
    }
    // groups of up to rows_per_item consecutive rows with equal partition counts
    for (int i = 0; i < n;) {
      const int j = i + s.rows_per_item < n ? i + s.rows_per_item : n;
      const int64_t np = s.nparts(b, i);
      int k = i + 1;
      while (k < j && s.nparts(b, k) == np) ++k;
      const int row_ctx = s.base(b) + i + 1;
      for (int64_t part = 0; part < np; ++part) {
        const int64_t rest = row_ctx - part * s.P;
        on_work(r0 + i, b, (int32_t)part | ((k - i - 1) << 24), row_ctx, rest < s.P ? rest : s.P);
      }
      i = k;
    }
  }
}

Counts count(const Step& s) {
  Counts c;
  walk(
      s, [&](int, int, int32_t, int, int64_t) { ++c.work; },
      [&](int, int, int32_t, int, int) { ++c.tiles; },
      [&](int, int64_t np) {
        c.parts += np;
        if (np > 1) ++c.split;
        if (np > c.max_parts) c.max_parts = np;
      });
  return c;
}

}  // namespace

extern "C" int32_t tb_step_metadata_counts(const int32_t* query_start_loc, int32_t num_seqs,
                                           const int32_t* context_lens, int32_t num_tokens,
                                           int32_t block_size, int32_t partition_tokens,
                                           int32_t rows_per_item, int32_t tile_prefill, int64_t* counts) {
  const Step s{query_start_loc, context_lens, num_seqs, num_tokens, block_size, partition_tokens,
               rows_per_item, tile_prefill != 0};
  if (!counts) return TB_ERR_INVALID_ARG;
  const int32_t st = check_step(s, nullptr);
  if (st != TB_OK) return st;
  const Counts c = count(s);
  counts[0] = c.work;
  counts[1] = c.tiles;
  counts[2] = c.split;
  counts[3] = c.parts;
  counts[4] = c.max_parts;
  return TB_OK;
}

extern "C" int32_t tb_build_step_metadata(const int32_t* query_start_loc, int32_t num_seqs,
                                          const int32_t* context_lens, const int64_t* positions,
                                          int32_t num_tokens, const int32_t* block_tables,
                                          int32_t max_blocks_per_seq, int64_t num_blocks, int32_t block_size,
                                          int32_t partition_tokens, int32_t rows_per_item, int32_t tile_prefill,
                                          int32_t* slot_mapping, int32_t* row_part_offsets,
                                          int32_t* work_items, int32_t work_capacity, int32_t* prefill_tiles,
                                          int32_t tile_capacity, int32_t* split_rows, int32_t split_capacity,
                                          int64_t* counts) {
  const Step s{query_start_loc, context_lens, num_seqs, num_tokens, block_size, partition_tokens,
               rows_per_item, tile_prefill != 0};
  int32_t st = check_step(s, positions);
  if (st != TB_OK) return st;
  if (!counts || !slot_mapping || !row_part_offsets) return TB_ERR_INVALID_ARG;
  if (num_seqs > 0 && (!block_tables || max_blocks_per_seq <= 0 || num_blocks <= 0)) return TB_ERR_INVALID_ARG;
  const Counts c = count(s);
  counts[0] = c.work;
  counts[1] = c.tiles;
  counts[2] = c.split;
  counts[3] = c.parts;
  counts[4] = c.max_parts;
  if (c.work > work_capacity || c.tiles > tile_capacity || c.split > split_capacity) return TB_ERR_INVALID_ARG;
  if ((c.work && !work_items) || (c.tiles && !prefill_tiles) || (c.split && !split_rows)) return TB_ERR_INVALID_ARG;
  if (c.work >= INDEX_LIMIT || c.parts >= INDEX_LIMIT || max_blocks_per_seq >= INDEX_LIMIT) return TB_ERR_INVALID_ARG;

  // tables: every entry a sequence's context reaches is a block of the pool
  // (the reference's tensor indexing raises IndexError, kv_cache.py:35,43)
  for (int b = 0; b < num_seqs; ++b) {
    if (s.q(b) == 0) continue;
    const int64_t need = ((int64_t)context_lens[b] + block_size - 1) / block_size;
    if (need > max_blocks_per_seq) return TB_ERR_INDEX;
    const int32_t* t = block_tables + (int64_t)b * max_blocks_per_seq;
    for (int64_t j = 0; j < need; ++j)
      if (t[j] < 0 || t[j] >= num_blocks) return TB_ERR_INDEX;
  }

  // slot mapping (kv_cache.py:34-38), -1 outside every slice
  for (int r = 0; r < num_tokens; ++r) slot_mapping[r] = -1;
  for (int b = 0; b < num_seqs; ++b) {
    const int32_t* t = block_tables + (int64_t)b * max_blocks_per_seq;
    for (int i = 0; i < s.q(b); ++i) {
      const int p = s.base(b) + i;
      slot_mapping[s.qsl[b] + i] = t[p / block_size] * block_size + (p & (block_size - 1));
    }
  }
  // Last writer wins (the reference writes sequence after sequence): a row whose
  // slot a later row also writes gets -1. Two rows can only share a slot inside a
  // block both write to, so the blocks each sequence writes are compared pairwise.
  for (int a = 0; a < num_seqs; ++a) {
    if (s.q(a) == 0) continue;
    const int32_t* ta = block_tables + (int64_t)a * max_blocks_per_seq;
    const int a_first = s.base(a), a_last = context_lens[a] - 1;
    for (int i = a_first / block_size; i <= a_last / block_size; ++i) {
      const int lo_a = (a_first > i * block_size ? a_first : i * block_size) - i * block_size;
      const int hi_a = (a_last < i * block_size + block_size - 1 ? a_last : i * block_size + block_size - 1) -
                       i * block_size;
      for (int b = a; b < num_seqs; ++b) {
        if (s.q(b) == 0) continue;
        const int32_t* tb_ = block_tables + (int64_t)b * max_blocks_per_seq;
        const int b_first = s.base(b), b_last = context_lens[b] - 1;
        for (int j = (b == a ? i + 1 : b_first / block_size); j <= b_last / block_size; ++j) {
          if (tb_[j] != ta[i]) continue;
          const int lo_b = (b_first > j * block_size ? b_first : j * block_size) - j * block_size;
          const int hi_b = (b_last < j * block_size + block_size - 1 ? b_last : j * block_size + block_size - 1) -
                           j * block_size;
          for (int o = (lo_a > lo_b ? lo_a : lo_b); o <= (hi_a < hi_b ? hi_a : hi_b); ++o)
            slot_mapping[s.qsl[a] + i * block_size + o - a_first] = -1;   // a row of b (later) writes it too
        }
      }
    }
  }

  // partition offsets per row, split-row records
  for (int r = 0; r <= num_tokens; ++r) row_part_offsets[r] = 0;
  walk(
      s, [](int, int, int32_t, int, int64_t) {}, [](int, int, int32_t, int, int) {},
      [&](int row, int64_t np) { row_part_offsets[row + 1] = (int32_t)np; });
  for (int r = 0; r < num_tokens; ++r) row_part_offsets[r + 1] += row_part_offsets[r];
  int64_t ns = 0;
  for (int r = 0; r < num_tokens; ++r) {
    const int32_t np = row_part_offsets[r + 1] - row_part_offsets[r];
    if (np > 1) {
      int32_t* rec = split_rows + 4 * ns++;
      rec[0] = r;
      rec[1] = row_part_offsets[r];
      rec[2] = np;
      rec[3] = 0;
    }
  }

  // work items by partition length, shortest first; tiles by covered positions,
  // most first; both stable (generation order among equals)
  static_assert(TB_PREFILL_TILE_PARTITION <= MAX_PARTITION, "histogram size");
  int32_t hist[MAX_PARTITION + 2];
  memset(hist, 0, sizeof(int32_t) * (partition_tokens + 2));
  walk(
      s, [&](int, int, int32_t, int, int64_t len) { ++hist[len + 1]; }, [](int, int, int32_t, int, int) {},
      [](int, int64_t) {});
  for (int l = 1; l <= partition_tokens + 1; ++l) hist[l] += hist[l - 1];   // hist[len] = first slot of len
  walk(
      s,
      [&](int row, int b, int32_t part, int row_ctx, int64_t len) {
        int32_t* w = work_items + 4 * (int64_t)hist[len]++;
        w[0] = row;
        w[1] = b;
        w[2] = part;
        w[3] = row_ctx;
      },
      [](int, int, int32_t, int, int) {}, [](int, int64_t) {});
  if (c.tiles) {
    int32_t th[TB_PREFILL_TILE_PARTITION + 2];
    memset(th, 0, sizeof(th));
    // descending: bucket key TILE_PARTITION - covered
    walk(
        s, [](int, int, int32_t, int, int64_t) {},
        [&](int, int, int32_t, int, int cov) { ++th[TB_PREFILL_TILE_PARTITION - cov + 1]; }, [](int, int64_t) {});
    for (int l = 1; l <= TB_PREFILL_TILE_PARTITION + 1; ++l) th[l] += th[l - 1];
    walk(
        s, [](int, int, int32_t, int, int64_t) {},
        [&](int row0, int b, int32_t rows_part, int pos0, int cov) {
          int32_t* t = prefill_tiles + 4 * (int64_t)th[TB_PREFILL_TILE_PARTITION - cov]++;
          t[0] = row0;
          t[1] = b;
          t[2] = rows_part;
          t[3] = pos0;
        },
        [](int, int64_t) {});
  }
  return TB_OK;
}

// ---------------------------------------------------------------------------
// Decode plan of tb_paged_decode (decode-only steps: row b = sequence b, one new
// token each). Units are (sequence, kv head) pairs; a unit's positions are cut
// into tiles of 16. Units are assigned to XCDs by longest-first bin packing on
// their tile counts; each XCD's tiles (its units back to back) are split evenly
// over the workgroups that run on it (workgroup g runs on XCD g % num_xcds), and
// each workgroup's range is cut at unit boundaries into segments. A unit spread
// over several workgroups leaves one partial per segment, all on one XCD.
//
// Layout (int32): [0] workgroups G, [1] segments S, [2] units U, [3] pieces,
// [4] num_xcds, [5..7] 0; then wg_first [G + 1] (segment index of each
// workgroup's first segment), padded to 4; segments [S][4] = (unit, first tile,
// end tile, piece slot or -1 for a unit held whole by one segment); units [U][2]
// = (pieces, first slot).
namespace {
constexpr int DECODE_TILE = 16;

int64_t plan_ints(int64_t G, int64_t S, int64_t U) {
  const int64_t wg = (G + 1 + 3) / 4 * 4;
  return 8 + wg + 4 * S + 2 * U;
}
}  // namespace

extern "C" size_t tb_decode_plan_bytes(int32_t num_seqs, int32_t num_kv_heads, int32_t workgroups) {
  if (num_seqs < 0 || num_kv_heads <= 0 || workgroups <= 0) return 0;
  const int64_t U = (int64_t)num_seqs * num_kv_heads;
  return (size_t)plan_ints(workgroups, U + workgroups, U) * sizeof(int32_t);
}

extern "C" int32_t tb_build_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                                        int32_t workgroups, int32_t num_xcds, int32_t max_tiles_per_wg,
                                        int32_t max_segments_per_wg, int32_t* plan, size_t plan_bytes) {
  if (num_seqs < 0 || num_kv_heads <= 0 || workgroups <= 0 || num_xcds <= 0 || num_xcds > 64 || !plan)
    return TB_ERR_INVALID_ARG;
  if (workgroups % num_xcds || max_tiles_per_wg <= 0 || max_segments_per_wg <= 0) return TB_ERR_INVALID_ARG;
  if (num_seqs > 0 && !context_lens) return TB_ERR_INVALID_ARG;
  if (plan_bytes < tb_decode_plan_bytes(num_seqs, num_kv_heads, workgroups)) return TB_ERR_INVALID_ARG;
  if ((int64_t)num_seqs * num_kv_heads >= INDEX_LIMIT) return TB_ERR_INVALID_ARG;
  const int32_t U = num_seqs * num_kv_heads, G = workgroups, NX = num_xcds, per = G / NX;
  for (int b = 0; b < num_seqs; ++b)
    if (context_lens[b] < 1) return TB_ERR_INVALID_ARG;
  auto tiles = [&](int u) { return (context_lens[u / num_kv_heads] + DECODE_TILE - 1) / DECODE_TILE; };
  int32_t* const wg_first = plan + 8;
  int32_t* const segs = wg_first + (G + 1 + 3) / 4 * 4;
  int32_t* const units = segs + 4 * ((int64_t)U + G);   // each unit's XCD, past every segment the plan can hold

  // 1. XCDs: longest unit first (stable), onto the least loaded XCD (lowest index among equals)
  int64_t load[64];
  for (int x = 0; x < NX; ++x) load[x] = 0;
  int32_t max_t = 0;
  for (int u = 0; u < U; ++u) max_t = tiles(u) > max_t ? tiles(u) : max_t;
  for (int t = max_t; t >= 1; --t)
    for (int u = 0; u < U; ++u) {
      if (tiles(u) != t) continue;
      int best = 0;
      for (int x = 1; x < NX; ++x)
        if (load[x] < load[best]) best = x;
      units[2 * u] = best;
      load[best] += t;
    }

  // 2. segments in workgroup order: workgroup g = j * NX + x takes the j-th of XCD x's
  // `per` even ranges of its tiles (its units in unit order, back to back)
  int32_t cur_u[64], cur_t[64];
  auto next_unit = [&](int x, int from) {
    for (int v = from; v < U; ++v)
      if (units[2 * v] == x) return v;
    return U;
  };
  for (int x = 0; x < NX; ++x) {
    cur_u[x] = next_unit(x, 0);
    cur_t[x] = 0;
  }
  int64_t S = 0;
  for (int g = 0; g < G; ++g) {
    const int x = g % NX, j = g / NX;
    const int64_t a = load[x] * j / per, b = load[x] * (j + 1) / per;
    if (b - a > max_tiles_per_wg) return TB_ERR_UNSUPPORTED;
    wg_first[g] = (int32_t)S;
    int64_t left = b - a;
    int nseg = 0;
    while (left > 0) {
      const int u = cur_u[x];
      const int take = (int)(tiles(u) - cur_t[x] < left ? tiles(u) - cur_t[x] : left);
      int32_t* sg = segs + 4 * S++;
      sg[0] = u;
      sg[1] = cur_t[x];
      sg[2] = cur_t[x] + take;
      sg[3] = 0;
      ++nseg;
      cur_t[x] += take;
      left -= take;
      if (cur_t[x] == tiles(u)) {
        cur_u[x] = next_unit(x, u + 1);
        cur_t[x] = 0;
      }
    }
    if (nseg > max_segments_per_wg) return TB_ERR_UNSUPPORTED;
  }
  wg_first[G] = (int32_t)S;
  for (int i = G + 1; i < (G + 1 + 3) / 4 * 4; ++i) wg_first[i] = 0;

  // 3. pieces: a unit cut into several segments leaves one partial per segment. The
  // unit records follow the S segments (the XCD assignment above is no longer needed).
  int32_t* const rec = segs + 4 * S;
  for (int u = 0; u < U; ++u) rec[2 * u] = rec[2 * u + 1] = 0;
  for (int64_t i = 0; i < S; ++i) ++rec[2 * segs[4 * i]];
  int32_t pieces = 0;
  for (int u = 0; u < U; ++u) {
    if (rec[2 * u] > 255) return TB_ERR_UNSUPPORTED;   // arrival counts are 8-bit fields
    rec[2 * u + 1] = rec[2 * u] > 1 ? pieces : -1;
    if (rec[2 * u] > 1) pieces += rec[2 * u];
  }
  for (int64_t i = 0; i < S; ++i) {
    const int u = segs[4 * i];
    segs[4 * i + 3] = rec[2 * u] > 1 ? rec[2 * u + 1]++ : -1;
  }
  for (int u = 0; u < U; ++u)
    if (rec[2 * u] > 1) rec[2 * u + 1] -= rec[2 * u];
  plan[0] = G;
  plan[1] = (int32_t)S;
  plan[2] = U;
  plan[3] = pieces;
  plan[4] = NX;
  plan[5] = plan[6] = plan[7] = 0;
  return TB_OK;
}
