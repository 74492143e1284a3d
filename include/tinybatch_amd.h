/*
 * tinybatch_amd — C ABI of the MI355X (gfx950) paged KV-cache data path.
 *
 * Every entry point takes plain device pointers, integer sizes, a dtype code and
 * the HIP stream to launch on. Nothing here allocates, synchronises or throws:
 * each call enqueues kernels on `stream` and returns a status code
 * (TB_OK = 0, negative on a rejected argument or a failed launch).
 * All kernels are stateless, so calls are reentrant; calls on one stream run
 * in issue order, which is how the "all K/V appended before any attention
 * read" ordering of the reference forward pass is kept
 * (reference: src/tinybatch/model.py:127-132).
 *
 * Pool layout, unchanged from the reference (src/tinybatch/kv_cache.py:1-7,17-20):
 *   pool[num_blocks][2][num_kv_heads][block_size][head_dim]   (axis 1: 0 = K, 1 = V)
 * Slot contract (src/tinybatch/block_manager.py, kv_cache.py:35-36):
 *   slot(pos) = table[pos / block_size] * block_size + pos % block_size
 */
#ifndef TINYBATCH_AMD_H
#define TINYBATCH_AMD_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define TB_OK 0
#define TB_ERR_INVALID_ARG (-1)  /* null pointer, bad size, inconsistent shape */
#define TB_ERR_UNSUPPORTED (-2)  /* shape/dtype combination with no compiled kernel */
#define TB_ERR_LAUNCH (-3)       /* hipLaunchKernel reported an error */
#define TB_ERR_SCRATCH (-4)      /* tb_paged_attention_noalloc: partials exceed its scratch */
#define TB_ERR_INDEX (-5)        /* a block table too short for a context, or a block id outside the pool */

/* element type of q / k / v / pool / out */
#define TB_DTYPE_F32 0
#define TB_DTYPE_F16 1
#define TB_DTYPE_BF16 2

/* Human-readable text for a status code (static storage). */
const char* tb_status_string(int32_t status);

/* ---------------------------------------------------------------------------
 * K1 — KV append.
 * Replaces PagedKVCache.write (src/tinybatch/kv_cache.py:25-38): for every
 * token t with slot_mapping[t] >= 0,
 *   pool[slot/BS][0][h][slot%BS][:] = k[t][h][:]
 *   pool[slot/BS][1][h][slot%BS][:] = v[t][h][:]      for all kv heads h.
 * Tokens with a negative slot are skipped (the host marks all but the last
 * writer of a duplicated slot this way, so the result equals the reference's
 * sequential "last sequence in batch order wins").
 * k, v: [num_tokens][num_kv_heads][head_dim], token row stride in elements.
 * Bytes are copied verbatim (bit-exact for every dtype).
 */
int32_t tb_kv_append(const void* k, int64_t k_row_stride,
                     const void* v, int64_t v_row_stride,
                     void* pool, int64_t num_blocks,
                     const int32_t* slot_mapping, int32_t num_tokens,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int32_t dtype, hipStream_t stream);

/* K1 with the K rotation folded in: the engine's rotate-half RoPE of k
 * (src/tinybatch/model.py:72-80, applied at :125) followed by write
 * (kv_cache.py:25-38). K rows are rotated at positions[t] (int64) on their way
 * to the pool, V rows are copied:
 *   k1' = k1 cos - k2 sin,  k2' = k2 cos + k1 sin   (k1 / k2 the two halves of a head row)
 * with rope_cos / rope_sin fp32 [rope_max_position][head_dim / 2] (16-byte
 * aligned; positions are clamped into the table), each product rounded on its
 * own and the result rounded to the element type: the bits of rotating with
 * the separate tensor ops, then tb_kv_append. head_dim * element size must be
 * a multiple of 32 bytes.
 */
int32_t tb_kv_append_rope(const void* k, int64_t k_row_stride,
                          const void* v, int64_t v_row_stride,
                          void* pool, int64_t num_blocks,
                          const int32_t* slot_mapping, const int64_t* positions,
                          const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                          int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                          int32_t block_size, int32_t dtype, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Paged gather of one sequence into contiguous K and V.
 * Replaces PagedKVCache.gather (src/tinybatch/kv_cache.py:40-45):
 *   k_out[t][h][:] = pool[table[t/BS]][0][h][t%BS][:],  v_out likewise with 1,
 * for t < context_len. k_out, v_out: [context_len][num_kv_heads][head_dim].
 */
int32_t tb_kv_gather(const void* pool, int64_t num_blocks,
                     const int32_t* table, int32_t context_len,
                     void* k_out, void* v_out,
                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int32_t dtype, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * K2 — fused paged attention (any query rows: decode, prefill, cached-prefix tail).
 * Replaces the per-sequence loop of Qwen2Paged.forward
 * (src/tinybatch/model.py:130-147: gather, GQA repeat_interleave, offset-causal
 * mask, scaled_dot_product_attention, attn_out assembly).
 *
 * Query row r (a token of the flat batch) of sequence b attends to positions
 * j < row_ctx[r] = context_len[b] - q_len[b] + i + 1 of its sequence, i being
 * the row's index inside the sequence (the mask j <= ctx - q_len + i of
 * model.py:142-145, which is also is_causal when q_len == ctx). Query head h
 * reads kv head h / (num_heads / num_kv_heads) (repeat_interleave, model.py:136-137).
 *   q:   [num_rows][num_heads][head_dim], row stride q_row_stride (elements)
 *   out: [num_rows][num_heads * head_dim], row stride out_row_stride
 *   block_tables: [num_seqs][max_blocks_per_seq] int32 physical block ids
 *   work_items: [num_work_items][4] int32 = (row, seq, partition | (rows-1) << 24,
 *     row_ctx): rows row .. row+rows-1 of sequence seq (fp16/bf16 only: up to
 *     16 / heads-per-group consecutive query rows whose partition counts are
 *     equal; the later rows see one more position each; fp32: rows = 1);
 *     partition p covers positions [p*P, min((p+1)*P, row_ctx)) with
 *     P = partition_tokens (a multiple of block_size spanning at most 64
 *     blocks; fp16/bf16 require tb_attention_partition_tokens(dtype, D),
 *     fp32 accepts any multiple of its 8-load chunk). Every row served by
 *     work items lists partitions 0 .. ceil(row_ctx/P)-1,
 *     row_part_offsets[num_rows+1] is their running count (row r owns
 *     partial slots row_part_offsets[r] ..; rows served by tiles count 0),
 *     total_partitions = row_part_offsets[num_rows] and max_parts_per_row is
 *     the largest per-row count.
 *   prefill_tiles: [num_prefill_tiles][4] int32 = (row0, seq,
 *     rows | part << 8, pos0), fp16/bf16 only: query rows row0 .. row0+rows-1
 *     (rows <= TB_PREFILL_TILE_ROWS) of sequence seq at positions
 *     pos0 .. pos0+rows-1, positions [part*T, (part+1)*T) of their range with
 *     T = TB_PREFILL_TILE_PARTITION (one workgroup per item and query head).
 *     A tile row counts ceil(row_ctx/T) partitions in row_part_offsets; one
 *     item per partition its tile's last row reaches. Rows in tiles must not
 *     also appear in work items.
 *   split_rows: [num_split_rows][4] int32 (16-byte aligned) = (row,
 *     row_part_offsets[row], partition count, 0) of every row with more than
 *     one partition; their partials are merged by a combine kernel.
 *   workspace: >= tb_paged_attention_workspace_bytes(total_partitions, ...)
 *     bytes of device memory (16-byte aligned) for the split-row partials;
 *     only used when a row has > 1 partition (max_parts_per_row > 1), which
 *     also launches a second (combine) kernel. Calls that may overlap in time
 *     need their own workspace.
 * device_counts (may be NULL): device array {work items, split rows, prefill
 *   tiles} read by the kernels when they run; num_work_items, num_split_rows
 *   and num_prefill_tiles are then capacities that size the grids and the
 *   workgroups past the counts exit at once. One launch recorded in a HIP
 *   graph thus serves every step whose metadata fits the capacities (the
 *   metadata arrays are refreshed in place before each replay).
 * Fused decode append (k_new != NULL): each row's own newest position
 * row_ctx-1 is read from k_new/v_new ([num_rows][num_kv_heads][head_dim]) and
 * written to its slot in the pool by the same kernel, replacing a separate
 * tb_kv_append. Valid only for decode rows (one new token per sequence) whose
 * newest positions map to distinct pool slots: each row stores and attends to
 * its own new K/V, where the reference's sequential write would let the last
 * row in batch order win a shared slot for every row that reads it
 * (src/tinybatch/kv_cache.py:33-38). A step with a shared slot must use
 * tb_kv_append (its slot_mapping marks the superseded rows -1) and then this
 * call without k_new. The kernels do not read slot_mapping and cannot detect it.
 * RoPE in the prologue (rope_cos != NULL, the tables of tb_kv_append_rope):
 * q holds the projections before rotation; every query row is rotated at its
 * position row_ctx - 1 as it is loaded (the engine's _rope of q,
 * src/tinybatch/model.py:72-80,125), and with the fused append so is the K row
 * of k_new. NULL: q (and k_new) are already rotated.
 */
int32_t tb_attention_partition_tokens(int32_t dtype, int32_t head_dim);

/* ---------------------------------------------------------------------------
 * Host-side builder of a step's metadata (no device call, nothing allocated).
 * Takes the step as the reference's forward pass receives it
 * (src/tinybatch/model.py:101-109, built by LLMEngine.step, engine.py:99-126):
 *   query_start_loc [num_seqs + 1]: sequence b's new rows are the flat rows
 *     query_start_loc[b] .. query_start_loc[b+1]-1 (its seq_slices entry),
 *     non-decreasing, query_start_loc[num_seqs] <= num_tokens;
 *   context_lens [num_seqs]: positions each sequence has after the step;
 *   positions [num_tokens] (int64, may be NULL): row i of sequence b must be
 *     at context_lens[b] - q_len[b] + i (engine.py:110,117), which the mask
 *     of model.py:139-145 assumes; checked when given;
 *   block_tables [num_seqs][max_blocks_per_seq]: physical block ids, padded;
 *     the first ceil(context_lens[b] / block_size) entries are read.
 * Writes, for tb_kv_append and tb_paged_attention:
 *   slot_mapping [num_tokens]: slot of every new row (kv_cache.py:34-38), -1
 *     outside every sequence and for every row whose slot a later row also
 *     writes (the reference's sequential write lets the last one win);
 *   row_part_offsets [num_tokens + 1], work_items [W][4], prefill_tiles [N][4]
 *     (rows of sequences with >= 16 new rows and a context <= 4096 or <= 16x
 *     those rows, when tile_prefill != 0), split_rows [S][4]: the arrays
 *     tb_paged_attention documents, work items ordered by partition length
 *     (shortest first) and tiles by positions covered (most first), both
 *     stable, rows_per_item (1..16) consecutive rows grouped per item;
 *   counts [6] (int64): W, N, S, total_partitions, max_parts_per_row, and the
 *     superseded rows (rows inside a sequence whose slot_mapping is -1
 *     because a later row writes the same slot). A fused append (k_new given
 *     to tb_paged_attention, tb_paged_decode or tb_paged_prefill) needs
 *     counts[5] == 0: each of those rows would attend to its own new K/V,
 *     where the reference's sequential write lets the last writer win
 *     (kv_cache.py:33-38); append with tb_kv_append and call without k_new.
 * tb_step_metadata_counts gives the first five counts alone (the sizes to
 * provide; it sees no block tables, so counts [5] suffice there).
 * Capacities below the counts: TB_ERR_INVALID_ARG (counts still written).
 * A table shorter than a context or a block id outside [0, num_blocks):
 * TB_ERR_INDEX (the reference's IndexError, kv_cache.py:35,43). partition_tokens
 * <= 8192. Replaces the per-layer host-to-device table copies and the mask
 * loop of the reference (kv_cache.py:35,43; model.py:142-145). */
int32_t tb_step_metadata_counts(const int32_t* query_start_loc, int32_t num_seqs,
                                const int32_t* context_lens, int32_t num_tokens,
                                int32_t block_size, int32_t partition_tokens,
                                int32_t rows_per_item, int32_t tile_prefill, int64_t* counts);

int32_t tb_build_step_metadata(const int32_t* query_start_loc, int32_t num_seqs,
                               const int32_t* context_lens, const int64_t* positions,
                               int32_t num_tokens, const int32_t* block_tables,
                               int32_t max_blocks_per_seq, int64_t num_blocks, int32_t block_size,
                               int32_t partition_tokens, int32_t rows_per_item, int32_t tile_prefill,
                               int32_t* slot_mapping, int32_t* row_part_offsets,
                               int32_t* work_items, int32_t work_capacity,
                               int32_t* prefill_tiles, int32_t tile_capacity,
                               int32_t* split_rows, int32_t split_capacity, int64_t* counts);

/* Prefill tile shape: rows per tile, positions per tile partition. */
#define TB_PREFILL_TILE_ROWS 64
#define TB_PREFILL_TILE_PARTITION 1024

/* K2 for whole prefill sequences whose context fits in one workgroup's LDS
 * (reference src/tinybatch/model.py:130-147 for the rows of those sequences:
 * gather, repeat_interleave, the causal mask of model.py:139-146 and SDPA).
 * fp16 / bf16, head_dim 64 or 128, num_heads / num_kv_heads <=
 * tb_prefill_stream_max_group (8 at head dim 64, 4 at 128), block_size a
 * power of two >= 16, context (pos0 + new rows) <= tb_prefill_stream_max_context
 * (TB_ERR_UNSUPPORTED otherwise: use tb_paged_attention's tiles). Each sequence's
 * K/V range moves into LDS once per (kv head, pair of 16-row blocks p and
 * nb-1-p) and the kv head's query heads share it; every row's output is written
 * whole (no workspace). The rows it serves must not also be given to
 * tb_paged_attention. The K/V of the step's new rows must already be in the pool
 * (append first), unless k_new / v_new are given:
 *   k_new, v_new (may be NULL, both or neither): the step's new K / V rows
 *     [num_rows][num_kv_heads][head_dim] (row strides in elements, 16-byte
 *     aligned); the kernel then reads each sequence's new rows from them (the
 *     cached rows of a 16-position tile that holds the first new position from
 *     the pool) and stores them to their pool slots (the append of
 *     kv_cache.py:25-38 fused: the pool afterwards equals tb_kv_append's, bit
 *     for bit). With rope tables the K rows are rotated at their positions
 *     first, as tb_kv_append_rope does (model.py:125,128). The new rows' slots
 *     must not be written by another row of the step (slot_mapping's superseded
 *     rows, tb_build_step_metadata's counts[5], must be 0).
 *   work: tb_build_prefill_work's list (device memory), num_work entries;
 *     max_tiles: the value the builder returned.
 * q, out, strides, scale, dtype, rope: as tb_paged_attention. */
#define TB_PREFILL_STREAM_LDS (144 * 1024)
int32_t tb_paged_prefill(const void* q, int64_t q_row_stride, void* pool, int64_t num_blocks,
                         void* out, int64_t out_row_stride, const int32_t* block_tables,
                         int32_t max_blocks_per_seq, const int32_t* work, int32_t num_work,
                         int32_t max_tiles, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                         int32_t block_size, float scale, int32_t dtype,
                         const void* k_new, int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                         const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                         hipStream_t stream);
/* The longest context (positions) and the most query heads per kv head
 * tb_paged_prefill serves at a head dim (0: none). */
int32_t tb_prefill_stream_max_context(int32_t head_dim);
int32_t tb_prefill_stream_max_group(int32_t head_dim);
/* Work entries for num_seqs prefill sequences (host arrays: first row of the
 * sequence in q / out, its index into block_tables, position of its first new
 * row, new rows >= 1): sum over sequences of ceil(ceil(new_rows / 16) / 2) *
 * num_kv_heads, or -1 for bad arguments. */
int32_t tb_prefill_work_count(const int32_t* new_rows, int32_t num_seqs, int32_t num_kv_heads);
/* The work list (host memory, int32 x4 per entry: first row, sequence, pos0,
 * new rows | pair << 16 | kv head << 24) and the most 16-position tiles one
 * entry holds (*max_tiles). The entries of one (sequence, kv head), which read
 * the same K/V, are placed where entry g runs on XCD g % num_xcds (1: no
 * placement), longest contexts first. Nothing is allocated. */
int32_t tb_build_prefill_work(const int32_t* first_row, const int32_t* seq_index, const int32_t* pos0,
                              const int32_t* new_rows, int32_t num_seqs, int32_t num_kv_heads,
                              int32_t head_dim, int32_t num_xcds, int32_t* work, int32_t capacity,
                              int32_t* max_tiles);

size_t tb_paged_attention_workspace_bytes(int32_t total_partitions, int32_t num_heads,
                                          int32_t head_dim);

int32_t tb_paged_attention(const void* q, int64_t q_row_stride,
                           void* pool, int64_t num_blocks,
                           void* out, int64_t out_row_stride,
                           const int32_t* block_tables, int32_t max_blocks_per_seq,
                           const int32_t* work_items, int32_t num_work_items,
                           const int32_t* prefill_tiles, int32_t num_prefill_tiles,
                           const int32_t* row_part_offsets, int32_t num_rows,
                           const int32_t* split_rows, int32_t num_split_rows,
                           int32_t max_parts_per_row, int32_t partition_tokens,
                           int32_t total_partitions,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                           int32_t block_size, float scale, int32_t dtype,
                           const void* k_new, int64_t k_row_stride,
                           const void* v_new, int64_t v_row_stride,
                           void* workspace, size_t workspace_bytes,
                           const int32_t* device_counts,
                           const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                           hipStream_t stream);

/* tb_paged_attention without a workspace: the split-row partials go to a
 * static device array of TB_NOALLOC_SCRATCH_BYTES that the library holds on
 * every GPU it runs on, until the process ends. No counterpart in the
 * reference (which allocates per call): this entry point is for callers that
 * cannot allocate device memory, such as code under HIP graph capture, tight
 * serving loops or harnesses that forbid hipMalloc; it calls no hipMalloc,
 * hipFree or allocating library routine. Arguments and results are those of
 * tb_paged_attention (the same kernels). A call whose partials need more than
 * TB_NOALLOC_SCRATCH_BYTES (tb_paged_attention_workspace_bytes of its
 * total_partitions) returns TB_ERR_SCRATCH and launches nothing. `stream` must
 * belong to the current device. Every call on a GPU shares that GPU's array,
 * so calls that may overlap in time on one GPU race (issue them on one
 * stream); nothing in it needs to start at zero, each partial a call reads
 * being written by that call first. */
#define TB_NOALLOC_SCRATCH_BYTES (32u << 20)

int32_t tb_paged_attention_noalloc(const void* q, int64_t q_row_stride,
                                   void* pool, int64_t num_blocks,
                                   void* out, int64_t out_row_stride,
                                   const int32_t* block_tables, int32_t max_blocks_per_seq,
                                   const int32_t* work_items, int32_t num_work_items,
                                   const int32_t* prefill_tiles, int32_t num_prefill_tiles,
                                   const int32_t* row_part_offsets, int32_t num_rows,
                                   const int32_t* split_rows, int32_t num_split_rows,
                                   int32_t max_parts_per_row, int32_t partition_tokens,
                                   int32_t total_partitions,
                                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t block_size, float scale, int32_t dtype,
                                   const void* k_new, int64_t k_row_stride,
                                   const void* v_new, int64_t v_row_stride,
                                   const int32_t* device_counts,
                                   const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                                   hipStream_t stream);

/* K2 with the split rows merged inside the launch (no combine kernel), for a
 * 16-bit step of work items only (no prefill tiles; num_heads / num_kv_heads
 * <= 16; TB_ERR_UNSUPPORTED otherwise). Arguments as tb_paged_attention, plus:
 *   slot_map: device int32 [slot_count], the grid: slot s runs item
 *     slot_map[s] / num_kv_heads for kv head slot_map[s] % num_kv_heads, or
 *     nothing for -1. Every item of a row group (the partitions of split rows)
 *     and kv head must sit in slots s with one s % num_xcds, the XCD that slot
 *     runs on (slot s on XCD s % num_xcds: verify with tb_decode_xcc_probe);
 *     tb_build_xcd_slot_map builds such a map.
 *   arrivals: device memory of arrival_units * 128 bytes (arrival_units >=
 *     num_rows * num_kv_heads, 128-byte aligned), zero before the first call
 *     and left zero by every call; `violations` (device uint32) is incremented
 *     for every row group whose partitions ran on more than one XCD (its
 *     output may then be wrong). Calls that may overlap in time need their own
 *     workspace and arrival counters.
 * The workspace holds the split rows' partials as for tb_paged_attention
 * (< 2 GiB). The outputs equal tb_paged_attention's bit for bit.
 * A row's partitions are counted in 8-bit per-XCD fields of its arrival word:
 * max_parts_per_row above TB_MERGED_MAX_PARTS returns TB_ERR_UNSUPPORTED and
 * launches nothing (use tb_paged_attention, whose combine kernel has no such
 * limit); tb_xcd_slot_map_slots / tb_build_xcd_slot_map refuse such steps the
 * same way.
 */
#define TB_MERGED_MAX_PARTS 255
int32_t tb_paged_attention_merged(const void* q, int64_t q_row_stride, void* pool, int64_t num_blocks,
                                  void* out, int64_t out_row_stride,
                                  const int32_t* block_tables, int32_t max_blocks_per_seq,
                                  const int32_t* work_items, int32_t num_work_items,
                                  const int32_t* row_part_offsets, int32_t num_rows,
                                  int32_t max_parts_per_row, int32_t partition_tokens, int32_t total_partitions,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                  float scale, int32_t dtype,
                                  const void* k_new, int64_t k_row_stride, const void* v_new, int64_t v_row_stride,
                                  void* workspace, size_t workspace_bytes,
                                  const int32_t* slot_map, int32_t slot_count,
                                  unsigned long long* arrivals, int32_t arrival_units, uint32_t* violations,
                                  const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                                  hipStream_t stream);

/* Host-side slot map of tb_paged_attention_merged (nothing allocated): the
 * row groups (work items sharing their first row, all of one row's
 * partitions) of each kv head are packed onto num_xcds XCDs by item count
 * (longest first, least loaded XCD), and XCD x's items, in item order, fill
 * slots x, x + num_xcds, ...; the map is padded with -1 to
 * tb_xcd_slot_map_slots(...) slots (a multiple of num_xcds). work_items is
 * the host copy of the step's work items (int32 [num_work_items][4]). */
int32_t tb_xcd_slot_map_slots(const int32_t* work_items, int32_t num_work_items, int32_t num_kv_heads,
                              int32_t num_xcds);
int32_t tb_build_xcd_slot_map(const int32_t* work_items, int32_t num_work_items, int32_t num_kv_heads,
                              int32_t num_xcds, int32_t* slot_map, int32_t slots);

/* ---------------------------------------------------------------------------
 * K2 for decode steps: row b of q / out / k_new / v_new is sequence b's one new
 * token, at position context_lens[b] - 1, attending to positions
 * 0 .. context_lens[b] - 1 (reference src/tinybatch/model.py:130-147 for
 * decode rows, with the append of kv_cache.py:25-38 fused when k_new != NULL).
 * fp16 / bf16, head_dim 64 or 128, num_heads / num_kv_heads <= 8,
 * num_kv_heads <= 16, block_size a power of two >= 16 (TB_ERR_UNSUPPORTED
 * otherwise: use tb_paged_attention).
 *
 * The work is a plan (tb_build_decode_plan) for plan_workgroups workgroups of
 * plan_waves waves, one workgroup per CU: every wave streams its own share of
 * the step's 16-position tiles (sequence, kv head, 16 positions) through a ring
 * in LDS; a (sequence, kv head) unit cut over several waves is merged first per
 * workgroup, by the wave whose piece arrives last there, then by the workgroup
 * whose partial completes the unit.
 *   workspace: >= tb_paged_decode_workspace_bytes(max_pieces, ...) bytes of
 *     device memory, 128-byte aligned, for the partials (max_pieces >= the
 *     plan's pieces).
 *   arrivals: arrival_units * 128 bytes of device memory (arrival_units >=
 *     num_seqs * num_kv_heads, 128-byte aligned), zero before the first call
 *     (allocate it zeroed) and left zero by every call, so one buffer serves
 *     every later call. The partials of a unit are written and merged inside one
 *     XCD: the plan assumes that workgroup g runs on XCD g % num_xcds (verify
 *     with tb_decode_xcc_probe). Calls that may overlap in time need their own
 *     workspace and arrival counters.
 *   violations (device uint32): the call's error count, incremented for every
 *     unit whose partials ran on more than one XCD (its output may then be
 *     wrong), for every worker whose plan count is malformed (its tiles are
 *     not streamed), and once when k_new is given with a plan marked
 *     TB_DECODE_SHARED_NEWEST (then nothing is appended or written). Zero
 *     before a call and still zero after it means every output row is right;
 *     after a nonzero count the outputs are unusable and the arrival counters
 *     must be zeroed again.
 * RoPE (rope_cos != NULL) and the fused append: as tb_paged_attention. With
 * k_new the newest positions of the rows must map to distinct pool slots
 * (the reference's sequential write lets the last writer win a shared slot,
 * kv_cache.py:33-38): tb_build_decode_plan marks a plan where they do not,
 * and such a fused call is refused as above; append with tb_kv_append and
 * call without k_new instead.
 */
#define TB_DECODE_SHARED_NEWEST (1 << 30)
int32_t tb_paged_decode(const void* q, int64_t q_row_stride, void* pool, int64_t num_blocks,
                        void* out, int64_t out_row_stride, int32_t num_seqs,
                        const int32_t* plan, int32_t plan_workgroups, int32_t plan_waves, int32_t plan_stride,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                        float scale, int32_t dtype, const void* k_new, int64_t k_row_stride,
                        const void* v_new, int64_t v_row_stride, void* workspace, size_t workspace_bytes,
                        int32_t max_pieces, unsigned long long* arrivals, int32_t arrival_units,
                        uint32_t* violations, const float* rope_cos, const float* rope_sin,
                        int32_t rope_max_position, hipStream_t stream);
size_t tb_paged_decode_piece_bytes(int32_t num_heads, int32_t num_kv_heads, int32_t head_dim);
size_t tb_paged_decode_workspace_bytes(int32_t max_pieces, int32_t num_heads, int32_t num_kv_heads,
                                       int32_t head_dim);

/* The default waves per workgroup and per-unit cost (below) of tb_paged_decode
 * for a head dim (TB_ERR_UNSUPPORTED for head dims it does not serve), and
 * whether a (head dim, waves) pair is compiled. */
int32_t tb_decode_defaults(int32_t head_dim, int32_t* waves, int32_t* unit_cost);
int32_t tb_decode_variant_supported(int32_t head_dim, int32_t waves);

/* The per-unit cost to build this step's decode plan with (the plan builders
 * below take it): tb_decode_defaults' cost, or that cost - 2 when the lower one
 * gives the busiest worker >= 5% fewer entries (tb_decode_plan_shape), since a
 * worker's time goes by its entries. context_lens is host memory; returns the
 * errors of tb_decode_plan_shape. No counterpart in the reference (part of the
 * decode plan that replaces its per-sequence gather, src/tinybatch/kv_cache.py:40-45). */
int32_t tb_decode_unit_cost(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                            int32_t head_dim, int32_t workgroups, int32_t waves, int32_t num_xcds,
                            int32_t* unit_cost);

/* Host-side plan of a decode step (no device call, nothing allocated): units
 * (sequence b, kv head h), each cut into ceil(context_lens[b] / 16) tiles, are
 * packed onto num_xcds XCDs (longest first, least loaded XCD; a unit weighs
 * its tiles + unit_cost). XCD x's list is split evenly on that weight over
 * its workers (worker kk = wave kk % waves of workgroup
 * (kk / waves) * num_xcds + x); each unit segment of a worker is padded to an
 * even number of tiles. Layout (int32): counts [workers] (padded to a multiple
 * of 4), then entries [workers][stride] + 64 of padding, each int32 x4 =
 *   (byte offset of the tile's K rows in the pool >> 8,
 *    b | h << 20 | (valid rows - 1) << 24 | unit's last tile << 28 | pad << 29,
 *    context_lens[b] | piece index << 24,
 *    -1 for a unit one worker holds whole, else first partial slot |
 *      (pieces - 1) << 20 | (wave of piece 0) << 28).
 * Each count word is the worker's entry count, with TB_DECODE_SHARED_NEWEST
 * set in every word when two sequences' newest positions (context_lens[b] - 1)
 * map to one pool slot (a plan tb_paged_decode serves only without k_new).
 * tb_decode_plan_shape gives the entries of the busiest worker (stride must be
 * at least that, and even) and the partial slots (max_pieces); both return
 * TB_ERR_UNSUPPORTED when a unit would be cut over more than 255 workers (use
 * fewer waves or tb_paged_attention), TB_ERR_INDEX when a block id lies
 * outside [0, num_blocks) or a table is too short. context_lens and
 * block_tables (int32 [num_seqs][max_blocks_per_seq]) are host memory. */
int32_t tb_decode_plan_shape(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                             int32_t head_dim, int32_t workgroups, int32_t waves, int32_t num_xcds,
                             int32_t unit_cost, int32_t* max_entries, int32_t* pieces);
size_t tb_decode_plan_words(int32_t workers, int32_t stride);
int32_t tb_build_decode_plan(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                             int32_t head_dim, const int32_t* block_tables, int32_t max_blocks_per_seq,
                             int32_t block_size, int64_t num_blocks, int32_t workgroups, int32_t waves,
                             int32_t num_xcds, int32_t unit_cost, int32_t stride, int32_t* plan,
                             size_t plan_words);

/* The same plan built on the device (replaces tb_build_decode_plan's per-tile
 * host work and the upload of its entries; the reference builds its step
 * metadata as host lists, src/tinybatch/engine.py:99-126). Host part,
 * tb_build_decode_segments (nothing allocated, no device call): the assignment
 * of tb_build_decode_plan, written as the count words (counts [workers],
 * TB_DECODE_SHARED_NEWEST included when block_tables is given; may be NULL to
 * skip that mark) and one descriptor per (worker, unit) segment, int32 x 8 =
 *   (worker, first entry in the worker's list, b | h << 20, first tile of the
 *    unit, tiles | unit's last tile << 30, context_lens[b], piece index,
 *    the entries' fourth word),
 * at most num_seqs * num_kv_heads + workgroups * waves of them
 * (segment_capacity); *max_entries and *pieces as tb_decode_plan_shape.
 * Device part, tb_expand_decode_plan: writes every tile entry of the plan at
 * `plan` (device memory of tb_decode_plan_words(workers, stride) int32, the
 * count words copied to its start by the caller) from the descriptors and the
 * step's device block tables (int32 [num_seqs][max_blocks_per_seq]), one
 * workgroup per descriptor, on `stream`; the entries equal tb_build_decode_plan's.
 * A block id outside [0, num_blocks) or past its table is counted in `errors`
 * (device uint32) and replaced by block 0 (validate the tables on the host, as
 * tb_build_step_metadata does, to raise instead). */
int32_t tb_build_decode_segments(const int32_t* context_lens, int32_t num_seqs, int32_t num_kv_heads,
                                 int32_t head_dim, const int32_t* block_tables, int32_t max_blocks_per_seq,
                                 int32_t block_size, int32_t workgroups, int32_t waves, int32_t num_xcds,
                                 int32_t unit_cost, int32_t* counts, int32_t* segments,
                                 int32_t segment_capacity, int32_t* num_segments, int32_t* max_entries,
                                 int32_t* pieces);
int32_t tb_expand_decode_plan(const int32_t* segments, int32_t num_segments, const int32_t* block_tables,
                              int32_t max_blocks_per_seq, int32_t block_size, int64_t num_blocks,
                              int32_t num_kv_heads, int32_t head_dim, int32_t workers, int32_t stride,
                              int32_t* plan, uint32_t* errors, hipStream_t stream);

/* Records, for each of `workgroups` workgroups of one launch, the XCD it ran on
 * (device int32 [workgroups]): the check behind the in-launch merges. */
int32_t tb_decode_xcc_probe(int32_t workgroups, int32_t* out, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * K3 — block copy across every layer pool in one launch.
 * No reference counterpart: the reference shares blocks copy-free
 * (README.md:22) and evicts by metadata only (src/tinybatch/block_manager.py:68-80).
 * This is the data movement behind eviction compaction and copy-on-write:
 *   for every layer l and pair i: pool_l[dst[i]] = pool_l[src[i]]   (block_bytes each)
 * layer_pools: device array of num_layers pool base addresses.
 * dst ids must be distinct and disjoint from the src ids (checked by the host
 * wrapper), so the result does not depend on execution order.
 */
int32_t tb_block_copy(const uint64_t* layer_pools, int32_t num_layers, int64_t num_blocks,
                      const int32_t* src_blocks, const int32_t* dst_blocks, int32_t num_pairs,
                      int64_t block_bytes, hipStream_t stream);

/* Swap-out / swap-in halves of K3 for one pool: staging[i] <-> pool[blocks[i]]
 * (block_bytes each); staging may be device or pinned host memory.
 * Reference counterpart: none (preemption recomputes instead of swapping,
 * src/tinybatch/scheduler.py:141-149). */
int32_t tb_block_gather(const void* pool, int64_t num_blocks, const int32_t* blocks,
                        int32_t num_blocks_to_move, void* staging, int64_t block_bytes,
                        hipStream_t stream);
int32_t tb_block_scatter(const void* staging, void* pool, int64_t num_blocks,
                         const int32_t* blocks, int32_t num_blocks_to_move,
                         int64_t block_bytes, hipStream_t stream);

/* ---------------------------------------------------------------------------
 * Model-side fused elementwise ops of the engine's Qwen2 layer (one launch
 * each instead of chains of tensor ops). Row strides are in elements.
 *
 * RMSNorm, src/tinybatch/model.py:65-69 (with the residual add of
 * model.py:149/154 when residual != NULL):
 *   if residual: residual[r] = x[r] + residual[r]  (rounded), h = residual[r]
 *   else h = x[r];  out[r] = (h * rsqrt(mean(h^2) + eps)) * weight, in fp32.
 *   dim <= 4096.
 */
int32_t tb_rms_norm(const void* x, int64_t x_row_stride, void* residual, int64_t residual_row_stride,
                    const void* weight, void* out, int64_t out_row_stride, int32_t rows, int32_t dim,
                    float eps, int32_t dtype, hipStream_t stream);

/* Rotate-half RoPE of q and k, src/tinybatch/model.py:72-80,125: qkv rows hold
 * num_heads q heads then num_kv_heads k heads of head_dim each; with
 * c, s = cos_table / sin_table [max_position][head_dim/2] (fp32) at the row's
 * position, x1 = x[i], x2 = x[i + D/2]:
 *   out[i] = x1*c - x2*s,  out[i + D/2] = x2*c + x1*s,
 * written to q_out [rows][num_heads][D] and k_out [rows][num_kv_heads][D]. */
int32_t tb_rope_qk(const void* qkv, int64_t row_stride, const int64_t* positions, const float* cos_table,
                   const float* sin_table, int32_t max_position, void* q_out, void* k_out, int32_t rows,
                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                   hipStream_t stream);

/* SwiGLU gate, src/tinybatch/model.py:152-154: gate_up rows hold gate [d_ff]
 * then up [d_ff]; out = silu(gate) (rounded) * up. */
int32_t tb_silu_mul(const void* gate_up, int64_t row_stride, void* out, int64_t out_row_stride,
                    int32_t rows, int32_t d_ff, int32_t dtype, hipStream_t stream);

/* Skinny linear layer (engine layer, not the KV path): the projections of the
 * reference's layer (src/tinybatch/model.py:121-124,149-154, F.linear with a
 * [out_features][in_features] weight) at decode batch sizes:
 *   y[r][n] = sum_k x[r][k] * w[n][k] (+ bias[n])   for rows <= 64,
 * fp16 / bf16, fp32 accumulation, rounded once to the element type.
 * out_features % 16 == 0 and in_features % 32 == 0 (TB_ERR_UNSUPPORTED
 * otherwise, and for more than 64 rows); x, w 16-byte aligned, rows strided.
 */
int32_t tb_linear(const void* x, int64_t x_row_stride, const void* w, const void* bias,
                  void* y, int64_t y_row_stride, int32_t rows, int32_t out_features,
                  int32_t in_features, int32_t dtype, hipStream_t stream);

/* Split-K pieces of tb_linear (no bias) for a projection whose output goes
 * straight into tb_rms_norm_partials (o_proj and down_proj, model.py:149,154):
 * with S = in_features / 32 k-slices of 32, range s of the `splits` ranges
 * (1 <= splits <= min(64, S)) holds slices [s*S/splits, (s+1)*S/splits) and
 *   partials[s][r][n] = sum over range s of x[r][k] * w[n][k]   (fp32, unrounded).
 * partials is float [splits][rows][out_features], contiguous. */
int32_t tb_linear_partials(const void* x, int64_t x_row_stride, const void* w, float* partials,
                           int32_t splits, int32_t rows, int32_t out_features, int32_t in_features,
                           int32_t dtype, hipStream_t stream);

/* gate/up projection fused with the SwiGLU gate (model.py:151-154):
 * w_gate_up = [2 d_ff][in_features] (gate rows, then up rows);
 *   y[r][c] = silu(T(g)) * T(u),  g = x[r] . w[c],  u = x[r] . w[d_ff + c],
 * with the roundings of tb_linear followed by tb_silu_mul (the same bits for
 * the same launch shape). d_ff % 16 == 0; other limits as tb_linear. */
int32_t tb_linear_silu_mul(const void* x, int64_t x_row_stride, const void* w_gate_up, void* y,
                           int64_t y_row_stride, int32_t rows, int32_t d_ff, int32_t in_features,
                           int32_t dtype, hipStream_t stream);

/* LM head followed by greedy sampling (model.py:157-158, engine.py:145-151):
 *   ids[r] = argmax_n T(x[r] . w[n])  (the rounded logits, as torch.argmax over
 * F.linear's output: NaN above every number, -0 equal to +0, the first index
 * among equal values), without writing the logits. `workspace` holds one
 * 8-byte candidate per (row, 16 columns): tb_linear_argmax_workspace_bytes;
 * 8-byte aligned. ids is int64 [rows]. Limits as tb_linear. */
size_t tb_linear_argmax_workspace_bytes(int32_t rows, int32_t out_features);
int32_t tb_linear_argmax(const void* x, int64_t x_row_stride, const void* w, int32_t rows,
                         int32_t out_features, int32_t in_features, void* workspace,
                         size_t workspace_bytes, int64_t* ids, int32_t dtype, hipStream_t stream);

/* tb_rms_norm whose input is the projection output held as split-K partials
 * (tb_linear_partials): x[r] = T(partials[0][r] + ... + partials[splits-1][r])
 * (fp32 adds in split order, one rounding), then the residual add and RMSNorm
 * of tb_rms_norm. fp16 / bf16; splits in {1, 2, 4, 8}; dim % 8 == 0,
 * dim <= 4096; partials, residual, weight, out 16-byte aligned with row
 * strides that are multiples of 8 elements. */
int32_t tb_rms_norm_partials(const float* partials, int32_t splits, void* residual,
                             int64_t residual_row_stride, const void* weight, void* out,
                             int64_t out_row_stride, int32_t rows, int32_t dim, float eps,
                             int32_t dtype, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TINYBATCH_AMD_H */
