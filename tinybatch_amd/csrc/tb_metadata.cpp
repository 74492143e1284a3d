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

#include <algorithm>
#include <vector>

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
  counts[5] = 0;
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
  // superseded rows: inside a sequence, slot -1 (a fused append cannot serve the step)
  int64_t superseded = 0;
  for (int b = 0; b < num_seqs; ++b)
    for (int i = 0; i < s.q(b); ++i) superseded += slot_mapping[s.qsl[b] + i] < 0;
  counts[5] = superseded;

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
// Slot map of tb_paged_attention_merged: a unit is (row group, kv head), a row
// group being the work items that share their first row (the partitions of
// that row, or of a run of decode rows of one sequence). Units are packed onto
// the XCDs by item count, longest first onto the least loaded XCD (lowest index
// among equals); XCD x's slot values (item * num_kv_heads + kv head, ascending)
// fill slots x, x + num_xcds, ...; the rest hold -1.
namespace {
int32_t xcd_slot_lists(const int32_t* work_items, int32_t num_work_items, int32_t num_kv_heads, int32_t num_xcds,
                       std::vector<std::vector<int32_t>>& lists) {
  if (num_work_items < 0 || num_kv_heads <= 0 || num_xcds <= 0 || num_xcds > 64) return TB_ERR_INVALID_ARG;
  if (num_work_items > 0 && !work_items) return TB_ERR_INVALID_ARG;
  if ((int64_t)num_work_items * num_kv_heads >= ((int64_t)1 << 31)) return TB_ERR_INVALID_ARG;
  // row groups in order of first appearance
  std::vector<std::pair<int32_t, int32_t>> by_row(num_work_items);   // (first row, item)
  for (int i = 0; i < num_work_items; ++i) by_row[i] = {work_items[4 * (int64_t)i], i};
  std::stable_sort(by_row.begin(), by_row.end(),
                   [](const std::pair<int32_t, int32_t>& x, const std::pair<int32_t, int32_t>& y) {
                     return x.first < y.first;
                   });
  std::vector<std::pair<int32_t, int32_t>> groups;   // (first index in by_row, items)
  for (int i = 0; i < num_work_items;) {
    int j = i;
    while (j < num_work_items && by_row[j].first == by_row[i].first) ++j;
    if (j - i > TB_MERGED_MAX_PARTS) return TB_ERR_UNSUPPORTED;   // 8-bit arrival fields
    groups.push_back({i, j - i});
    i = j;
  }
  // units (group, kv head), longest first (stable: group order, then kv head)
  std::vector<int64_t> units(groups.size() * (size_t)num_kv_heads);
  for (size_t u = 0; u < units.size(); ++u) units[u] = (int64_t)u;
  std::stable_sort(units.begin(), units.end(), [&](int64_t x, int64_t y) {
    return groups[x / num_kv_heads].second > groups[y / num_kv_heads].second;
  });
  std::vector<int64_t> load(num_xcds, 0);
  lists.assign(num_xcds, {});
  for (const int64_t u : units) {
    int best = 0;
    for (int x = 1; x < num_xcds; ++x)
      if (load[x] < load[best]) best = x;
    const auto& g = groups[u / num_kv_heads];
    const int32_t kvh = (int32_t)(u % num_kv_heads);
    for (int k = 0; k < g.second; ++k) lists[best].push_back(by_row[g.first + k].second * num_kv_heads + kvh);
    load[best] += g.second;
  }
  for (auto& l : lists) std::sort(l.begin(), l.end());
  return TB_OK;
}
}  // namespace

extern "C" int32_t tb_xcd_slot_map_slots(const int32_t* work_items, int32_t num_work_items, int32_t num_kv_heads,
                                         int32_t num_xcds) {
  std::vector<std::vector<int32_t>> lists;
  const int32_t st = xcd_slot_lists(work_items, num_work_items, num_kv_heads, num_xcds, lists);
  if (st != TB_OK) return st;
  size_t most = 0;
  for (const auto& l : lists) most = l.size() > most ? l.size() : most;
  if (most * (size_t)num_xcds >= ((size_t)1 << 31)) return TB_ERR_INVALID_ARG;
  return (int32_t)(most * num_xcds);
}

extern "C" int32_t tb_build_xcd_slot_map(const int32_t* work_items, int32_t num_work_items, int32_t num_kv_heads,
                                         int32_t num_xcds, int32_t* slot_map, int32_t slots) {
  if (!slot_map || slots < 0) return TB_ERR_INVALID_ARG;
  std::vector<std::vector<int32_t>> lists;
  const int32_t st = xcd_slot_lists(work_items, num_work_items, num_kv_heads, num_xcds, lists);
  if (st != TB_OK) return st;
  size_t most = 0;
  for (const auto& l : lists) most = l.size() > most ? l.size() : most;
  if ((int64_t)slots < (int64_t)(most * num_xcds)) return TB_ERR_INVALID_ARG;
  for (int32_t s = 0; s < slots; ++s) slot_map[s] = -1;
  for (int x = 0; x < num_xcds; ++x)
    for (size_t j = 0; j < lists[x].size(); ++j) slot_map[j * num_xcds + x] = lists[x][j];
  return TB_OK;
}
