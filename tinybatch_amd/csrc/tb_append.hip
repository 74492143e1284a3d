// K1 (KV append through a slot mapping) and the paged gather of one sequence.
//
// Both are pure data movement: 16-byte vector copies of K/V rows, bit-exact for
// every dtype. One thread moves one 16-byte chunk; a token's [Hkv][D] row of K
// (or V) is Hkv*D*b bytes, so consecutive threads write consecutive chunks of
// one contiguous [D] pool row and the wave's stores coalesce per row.
#include "tb_common.h"

namespace tb {

// K1. Reference: PagedKVCache.write, src/tinybatch/kv_cache.py:25-38
// (block = table[pos // BS], slot = pos % BS, pool[block, 0/1, :, slot] = k/v).
// Grid: one thread per (token, kv in {K,V}, kv head, 16-byte chunk of head_dim).
__global__ __launch_bounds__(256) void kv_append_kernel(
    const char* __restrict__ k, int64_t k_row_bytes, const char* __restrict__ v,
    int64_t v_row_bytes, char* __restrict__ pool, const int32_t* __restrict__ slot_mapping,
    int32_t num_tokens, int64_t num_blocks, int32_t num_kv_heads, int32_t chunks_per_head,
    int32_t head_bytes, int32_t log2_bs) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_token = 2LL * num_kv_heads * chunks_per_head;
  if (gid >= (int64_t)num_tokens * per_token) return;
  const int32_t t = (int32_t)(gid / per_token);
  int32_t rem = (int32_t)(gid - (int64_t)t * per_token);
  const int32_t kv = rem / (num_kv_heads * chunks_per_head);
  rem -= kv * num_kv_heads * chunks_per_head;
  const int32_t h = rem / chunks_per_head;
  const int32_t c = rem - h * chunks_per_head;

  const int32_t slot = slot_mapping[t];
  if (slot < 0) return;  // padding / superseded duplicate
  const int64_t blk = slot >> log2_bs;
  if (blk >= num_blocks) return;  // host validates; never write outside the pool
  const int32_t off = slot & ((1 << log2_bs) - 1);
  const int32_t bs = 1 << log2_bs;

  const char* src = (kv == 0 ? k + t * k_row_bytes : v + t * v_row_bytes) +
                    (int64_t)h * head_bytes + (int64_t)c * 16;
  char* dst = pool + (((blk * 2 + kv) * num_kv_heads + h) * bs + off) * (int64_t)head_bytes +
              (int64_t)c * 16;
  st16_through(dst, ld16(src));
}

// K1 with the K rotation folded in (the engine's _rope, model.py:72-80,125,
// followed by write, kv_cache.py:25-38): K rows are rotated at positions[t] on
// their way to the pool, V rows are copied. A thread owns one 16-byte chunk of
// a row and reads the chunk it pairs with in the other half of the head.
template <typename T>
__global__ __launch_bounds__(256) void kv_append_rope_kernel(
    const char* __restrict__ k, int64_t k_row_bytes, const char* __restrict__ v,
    int64_t v_row_bytes, char* __restrict__ pool, const int32_t* __restrict__ slot_mapping,
    const int64_t* __restrict__ positions, rope_tables rope, int32_t num_tokens, int64_t num_blocks,
    int32_t num_kv_heads, int32_t chunks_per_head, int32_t head_bytes, int32_t log2_bs) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_token = 2LL * num_kv_heads * chunks_per_head;
  if (gid >= (int64_t)num_tokens * per_token) return;
  const int32_t t = (int32_t)(gid / per_token);
  int32_t rem = (int32_t)(gid - (int64_t)t * per_token);
  const int32_t kv = rem / (num_kv_heads * chunks_per_head);
  rem -= kv * num_kv_heads * chunks_per_head;
  const int32_t h = rem / chunks_per_head;
  const int32_t c = rem - h * chunks_per_head;

  const int32_t slot = slot_mapping[t];
  if (slot < 0) return;  // padding / superseded duplicate
  const int64_t blk = slot >> log2_bs;
  if (blk >= num_blocks) return;  // host validates; never write outside the pool
  const int32_t off = slot & ((1 << log2_bs) - 1);
  const int32_t bs = 1 << log2_bs;

  const char* row = (kv == 0 ? k + t * k_row_bytes : v + t * v_row_bytes) + (int64_t)h * head_bytes;
  vec16 x = ld16(row + (int64_t)c * 16);
  if (kv == 0) {
    const int half_chunks = chunks_per_head / 2;
    const bool first = c < half_chunks;
    const int c1 = first ? c : c - half_chunks;            // chunk index within a half
    vec16 y = ld16(row + (int64_t)(first ? c + half_chunks : c1) * 16);
    constexpr int N = 16 / sizeof(T);
    const int half = chunks_per_head * N / 2;               // head_dim / 2
    const int64_t r = rope.row(positions[t], half) + c1 * N;
    if (first) {
      rope_pair<T>(x, y, rope.cos + r, rope.sin + r);       // x is the first-half chunk
    } else {
      rope_pair<T>(y, x, rope.cos + r, rope.sin + r);       // x is the second-half chunk
    }
  }
  char* dst = pool + (((blk * 2 + kv) * num_kv_heads + h) * bs + off) * (int64_t)head_bytes + (int64_t)c * 16;
  st16_through(dst, x);
}

// Reference: PagedKVCache.gather, src/tinybatch/kv_cache.py:40-45
// (pool[table] -> permute(1,0,3,2,4) -> reshape -> [:context_len]).
// Grid: one thread per (position t, kv, head, 16-byte chunk).
__global__ __launch_bounds__(256) void kv_gather_kernel(
    const char* __restrict__ pool, const int32_t* __restrict__ table, int32_t context_len,
    char* __restrict__ k_out, char* __restrict__ v_out, int64_t num_blocks, int32_t num_kv_heads,
    int32_t chunks_per_head, int32_t head_bytes, int32_t log2_bs) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_token = 2LL * num_kv_heads * chunks_per_head;
  if (gid >= (int64_t)context_len * per_token) return;
  const int32_t t = (int32_t)(gid / per_token);
  int32_t rem = (int32_t)(gid - (int64_t)t * per_token);
  const int32_t kv = rem / (num_kv_heads * chunks_per_head);
  rem -= kv * num_kv_heads * chunks_per_head;
  const int32_t h = rem / chunks_per_head;
  const int32_t c = rem - h * chunks_per_head;

  const int32_t bs = 1 << log2_bs;
  const int64_t blk = table[t >> log2_bs];
  if (blk < 0 || blk >= num_blocks) return;  // host validates; never read outside the pool
  const int32_t off = t & (bs - 1);
  const char* src = pool + (((blk * 2 + kv) * num_kv_heads + h) * bs + off) * (int64_t)head_bytes +
                    (int64_t)c * 16;
  char* dst = (kv == 0 ? k_out : v_out) + ((int64_t)t * num_kv_heads + h) * head_bytes +
              (int64_t)c * 16;
  st16(dst, ld16(src));
}

static int dtype_bytes(int32_t dtype) {
  switch (dtype) {
    case TB_DTYPE_F32: return 4;
    case TB_DTYPE_F16: return 2;
    case TB_DTYPE_BF16: return 2;
    default: return 0;
  }
}

static int log2_exact(int32_t x) {
  if (x <= 0 || (x & (x - 1)) != 0) return -1;
  int l = 0;
  while ((1 << l) < x) ++l;
  return l;
}

}  // namespace tb

extern "C" int32_t tb_kv_append(const void* k, int64_t k_row_stride, const void* v,
                                int64_t v_row_stride, void* pool, int64_t num_blocks,
                                const int32_t* slot_mapping, int32_t num_tokens,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t dtype, hipStream_t stream) {
  using namespace tb;
  const int eb = dtype_bytes(dtype);
  TB_CHECK_ARG(eb > 0);
  TB_CHECK_ARG(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0);
  const int log2_bs = log2_exact(block_size);
  TB_CHECK_ARG(log2_bs >= 0);
  const int head_bytes = head_dim * eb;
  if (head_bytes % 16 != 0) return TB_ERR_UNSUPPORTED;
  TB_CHECK_ARG(k_row_stride >= (int64_t)num_kv_heads * head_dim);
  TB_CHECK_ARG(v_row_stride >= (int64_t)num_kv_heads * head_dim);
  TB_CHECK_ARG((k_row_stride * eb) % 16 == 0 && (v_row_stride * eb) % 16 == 0);
  if (num_tokens == 0) return TB_OK;
  TB_CHECK_ARG(k && v && pool && slot_mapping);
  TB_CHECK_ARG((((uintptr_t)k | (uintptr_t)v | (uintptr_t)pool) & 15u) == 0);
  const int chunks = head_bytes / 16;
  const int64_t threads = (int64_t)num_tokens * 2 * num_kv_heads * chunks;
  const int64_t grid = (threads + 255) / 256;
  TB_CHECK_ARG(grid <= 0x7fffffffLL);
  hipLaunchKernelGGL(kv_append_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                     (const char*)k, k_row_stride * eb, (const char*)v, v_row_stride * eb,
                     (char*)pool, slot_mapping, num_tokens, num_blocks, num_kv_heads, chunks,
                     head_bytes, log2_bs);
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_kv_append_rope(const void* k, int64_t k_row_stride, const void* v,
                                     int64_t v_row_stride, void* pool, int64_t num_blocks,
                                     const int32_t* slot_mapping, const int64_t* positions,
                                     const float* rope_cos, const float* rope_sin, int32_t rope_max_position,
                                     int32_t num_tokens, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t block_size, int32_t dtype, hipStream_t stream) {
  using namespace tb;
  const int eb = dtype_bytes(dtype);
  TB_CHECK_ARG(eb > 0);
  TB_CHECK_ARG(num_tokens >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0);
  const int log2_bs = log2_exact(block_size);
  TB_CHECK_ARG(log2_bs >= 0);
  const int head_bytes = head_dim * eb;
  if (head_bytes % 32 != 0) return TB_ERR_UNSUPPORTED;   // each half a whole number of 16-byte chunks
  TB_CHECK_ARG(k_row_stride >= (int64_t)num_kv_heads * head_dim);
  TB_CHECK_ARG(v_row_stride >= (int64_t)num_kv_heads * head_dim);
  TB_CHECK_ARG((k_row_stride * eb) % 16 == 0 && (v_row_stride * eb) % 16 == 0);
  if (num_tokens == 0) return TB_OK;
  TB_CHECK_ARG(k && v && pool && slot_mapping && positions && rope_cos && rope_sin && rope_max_position > 0);
  TB_CHECK_ARG((((uintptr_t)k | (uintptr_t)v | (uintptr_t)pool | (uintptr_t)rope_cos | (uintptr_t)rope_sin) & 15u) == 0);
  const int chunks = head_bytes / 16;
  const int64_t threads = (int64_t)num_tokens * 2 * num_kv_heads * chunks;
  const int64_t grid = (threads + 255) / 256;
  TB_CHECK_ARG(grid <= 0x7fffffffLL);
  const rope_tables rope{rope_cos, rope_sin, rope_max_position};
#define TB_APPEND_ROPE(T)                                                                              \
  hipLaunchKernelGGL(kv_append_rope_kernel<T>, dim3((unsigned)grid), dim3(256), 0, stream, (const char*)k, \
                     k_row_stride * eb, (const char*)v, v_row_stride * eb, (char*)pool, slot_mapping,   \
                     positions, rope, num_tokens, num_blocks, num_kv_heads, chunks, head_bytes, log2_bs)
  switch (dtype) {
    case TB_DTYPE_F32: TB_APPEND_ROPE(float); break;
    case TB_DTYPE_F16: TB_APPEND_ROPE(_Float16); break;
    default: TB_APPEND_ROPE(__bf16); break;
  }
#undef TB_APPEND_ROPE
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_kv_gather(const void* pool, int64_t num_blocks, const int32_t* table,
                                int32_t context_len, void* k_out, void* v_out,
                                int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                int32_t dtype, hipStream_t stream) {
  using namespace tb;
  const int eb = dtype_bytes(dtype);
  TB_CHECK_ARG(eb > 0);
  TB_CHECK_ARG(context_len >= 0 && num_kv_heads > 0 && head_dim > 0 && num_blocks > 0);
  const int log2_bs = log2_exact(block_size);
  TB_CHECK_ARG(log2_bs >= 0);
  const int head_bytes = head_dim * eb;
  if (head_bytes % 16 != 0) return TB_ERR_UNSUPPORTED;
  if (context_len == 0) return TB_OK;
  TB_CHECK_ARG(pool && table && k_out && v_out);
  TB_CHECK_ARG((((uintptr_t)pool | (uintptr_t)k_out | (uintptr_t)v_out) & 15u) == 0);
  const int chunks = head_bytes / 16;
  const int64_t threads = (int64_t)context_len * 2 * num_kv_heads * chunks;
  const int64_t grid = (threads + 255) / 256;
  TB_CHECK_ARG(grid <= 0x7fffffffLL);
  hipLaunchKernelGGL(kv_gather_kernel, dim3((unsigned)grid), dim3(256), 0, stream,
                     (const char*)pool, table, context_len, (char*)k_out, (char*)v_out,
                     num_blocks, num_kv_heads, chunks, head_bytes, log2_bs);
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" const char* tb_status_string(int32_t status) {
  switch (status) {
    case TB_OK: return "ok";
    case TB_ERR_INVALID_ARG: return "invalid argument";
    case TB_ERR_UNSUPPORTED: return "unsupported shape or dtype (no compiled kernel)";
    case TB_ERR_LAUNCH: return "kernel launch failed";
    case TB_ERR_INDEX: return "block table too short for a context, or a block id outside the pool";
    case TB_ERR_SCRATCH: return "the call needs more scratch than the allocation-free entry point holds";
    default: return "unknown status";
  }
}
