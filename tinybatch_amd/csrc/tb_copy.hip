// K3 — whole-block copies: across every layer pool in one launch (eviction
// compaction / copy-on-write), and between a pool and a contiguous staging
// buffer (swap out / swap in).
//
// The reference moves no KV data for sharing or eviction (README.md:22,
// src/tinybatch/block_manager.py:68-80); these kernels define that movement
// for the same block layout: a block is the [2][Hkv][BS][D] slab
// pool[blk], block_bytes long and contiguous, so a copy is a 16-byte-vector
// memcpy of the slab. Bit-exact by construction.
#include "tb_common.h"

namespace tb {

// Grid: (pairs, layers, slices). Each workgroup copies a 1/slices share of one
// block of one layer; 256 threads x 16 bytes per step.
__global__ __launch_bounds__(256) void block_copy_kernel(const uint64_t* __restrict__ layer_pools,
                                                         const int32_t* __restrict__ src,
                                                         const int32_t* __restrict__ dst,
                                                         int64_t num_blocks, int64_t block_vecs,
                                                         int64_t slice_vecs) {
  const int pair = blockIdx.x;
  const int layer = blockIdx.y;
  char* base = reinterpret_cast<char*>(layer_pools[layer]);
  const int64_t s = src[pair], d = dst[pair];
  if (s < 0 || s >= num_blocks || d < 0 || d >= num_blocks) return;  // host validates
  const char* from = base + s * block_vecs * 16;
  char* to = base + d * block_vecs * 16;
  const int64_t begin = (int64_t)blockIdx.z * slice_vecs;
  const int64_t end = min(begin + slice_vecs, block_vecs);
  for (int64_t v = begin + threadIdx.x; v < end; v += blockDim.x) st16(to + v * 16, ld16(from + v * 16));
}

// staging[i] <- pool[blocks[i]]  (to_staging = 1)   or   pool[blocks[i]] <- staging[i]  (0)
__global__ __launch_bounds__(256) void block_stage_kernel(char* __restrict__ pool,
                                                          char* __restrict__ staging,
                                                          const int32_t* __restrict__ blocks,
                                                          int64_t num_blocks, int64_t block_vecs,
                                                          int64_t slice_vecs, int to_staging) {
  const int i = blockIdx.x;
  const int64_t b = blocks[i];
  if (b < 0 || b >= num_blocks) return;  // host validates
  char* p = pool + b * block_vecs * 16;
  char* s = staging + (int64_t)i * block_vecs * 16;
  const int64_t begin = (int64_t)blockIdx.y * slice_vecs;
  const int64_t end = min(begin + slice_vecs, block_vecs);
  for (int64_t v = begin + threadIdx.x; v < end; v += blockDim.x) {
    if (to_staging) st16(s + v * 16, ld16(p + v * 16));
    else st16(p + v * 16, ld16(s + v * 16));
  }
}

// 4096 16-byte vectors (64 KiB) per workgroup at most.
static int64_t slices_for(int64_t block_vecs, int64_t* slice_vecs) {
  const int64_t per = 4096;
  const int64_t n = (block_vecs + per - 1) / per;
  *slice_vecs = (block_vecs + n - 1) / n;
  return n;
}

}  // namespace tb

extern "C" int32_t tb_block_copy(const uint64_t* layer_pools, int32_t num_layers, int64_t num_blocks,
                                 const int32_t* src_blocks, const int32_t* dst_blocks,
                                 int32_t num_pairs, int64_t block_bytes, hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(num_layers >= 0 && num_pairs >= 0 && num_blocks > 0 && block_bytes > 0 && block_bytes % 16 == 0);
  if (num_layers == 0 || num_pairs == 0) return TB_OK;
  TB_CHECK_ARG(layer_pools && src_blocks && dst_blocks);
  TB_CHECK_ARG(num_layers <= 65535);
  int64_t slice_vecs = 0;
  const int64_t slices = slices_for(block_bytes / 16, &slice_vecs);
  TB_CHECK_ARG(slices <= 65535);
  hipLaunchKernelGGL(block_copy_kernel, dim3(num_pairs, num_layers, (unsigned)slices), dim3(256), 0, stream,
                     layer_pools, src_blocks, dst_blocks, num_blocks, block_bytes / 16, slice_vecs);
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_block_gather(const void* pool, int64_t num_blocks, const int32_t* blocks,
                                   int32_t num_blocks_to_move, void* staging, int64_t block_bytes,
                                   hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(num_blocks_to_move >= 0 && num_blocks > 0 && block_bytes > 0 && block_bytes % 16 == 0);
  if (num_blocks_to_move == 0) return TB_OK;
  TB_CHECK_ARG(pool && blocks && staging);
  TB_CHECK_ARG((((uintptr_t)pool | (uintptr_t)staging) & 15u) == 0);
  int64_t slice_vecs = 0;
  const int64_t slices = slices_for(block_bytes / 16, &slice_vecs);
  TB_CHECK_ARG(slices <= 65535);
  hipLaunchKernelGGL(block_stage_kernel, dim3(num_blocks_to_move, (unsigned)slices), dim3(256), 0, stream,
                     (char*)pool, (char*)staging, blocks, num_blocks, block_bytes / 16, slice_vecs, 1);
  TB_RETURN_LAUNCH_STATUS();
}

extern "C" int32_t tb_block_scatter(const void* staging, void* pool, int64_t num_blocks,
                                    const int32_t* blocks, int32_t num_blocks_to_move,
                                    int64_t block_bytes, hipStream_t stream) {
  using namespace tb;
  TB_CHECK_ARG(num_blocks_to_move >= 0 && num_blocks > 0 && block_bytes > 0 && block_bytes % 16 == 0);
  if (num_blocks_to_move == 0) return TB_OK;
  TB_CHECK_ARG(pool && blocks && staging);
  TB_CHECK_ARG((((uintptr_t)pool | (uintptr_t)staging) & 15u) == 0);
  int64_t slice_vecs = 0;
  const int64_t slices = slices_for(block_bytes / 16, &slice_vecs);
  TB_CHECK_ARG(slices <= 65535);
  hipLaunchKernelGGL(block_stage_kernel, dim3(num_blocks_to_move, (unsigned)slices), dim3(256), 0, stream,
                     (char*)pool, (char*)staging, blocks, num_blocks, block_bytes / 16, slice_vecs, 0);
  TB_RETURN_LAUNCH_STATUS();
}
