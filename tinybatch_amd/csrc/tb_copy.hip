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

// The copy is viewed as one run of 16-byte vectors: vector v of the round is
// vector v % V of pair v / V (V = vectors per block). A workgroup moves
// 256 x CU consecutive vectors of one layer; every thread issues its CU loads
// before its first store. The host guarantees that no dst block is a src block
// (and that dst blocks are distinct), so the loads may run ahead of the stores.
// Measured on 24 pools x 1024 pairs of 8 KiB blocks (403 MB moved), with CU = 2,
// non-temporal loads and the stores written through the L2 (st16_through):
// 73.0 us (5.52 TB/s). With non-temporal stores it was 83.8-87 us: the copy's
// last dirty L2 lines were written back only at the kernel's end. CU = 1 / 4 / 8
// measure 78.9 / 73.2-73.4 / 76.3-76.8 us (CU = 2: 72.7-73.7, same box); plain
// loads in place of the non-temporal ones 83.8-85.3 us.
// A plain contiguous device copy of the same bytes (torch) takes 80.2 us.
constexpr int COPY_CU = 2;

template <int CU, bool NT>
__global__ __launch_bounds__(256) void block_copy_kernel(const uint64_t* __restrict__ layer_pools,
                                                         const int32_t* __restrict__ src,
                                                         const int32_t* __restrict__ dst,
                                                         int64_t num_blocks, uint32_t block_vecs,
                                                         uint32_t total_vecs) {
  char* base = reinterpret_cast<char*>(layer_pools[blockIdx.y]);
  const uint32_t first = blockIdx.x * (256u * CU) + threadIdx.x;
  vec16 r[CU];
  char* to[CU];
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    const uint32_t v = first + 256u * u;
    to[u] = nullptr;
    if (v < total_vecs) {
      const uint32_t pair = v / block_vecs, off = v - pair * block_vecs;
      const int64_t s = src[pair], d = dst[pair];
      if (s >= 0 && s < num_blocks && d >= 0 && d < num_blocks) {   // host validates
        const char* from = base + (s * block_vecs + off) * 16;
        to[u] = base + (d * block_vecs + off) * 16;
        r[u] = NT ? ld16_stream(from) : ld16(from);
      }
    }
  }
#pragma unroll
  for (int u = 0; u < CU; ++u) {
    if (to[u]) {
      if (NT) st16_through(to[u], r[u]);
      else st16(to[u], r[u]);
    }
  }
}

// staging[i] <- pool[blocks[i]]  (to_staging = 1)   or   pool[blocks[i]] <- staging[i]  (0)
__global__ __launch_bounds__(256) void block_stage_kernel(char* __restrict__ pool,
                                                          char* __restrict__ staging,
                                                          const int32_t* __restrict__ blocks,
                                                          int64_t num_blocks, uint32_t block_vecs,
                                                          uint32_t total_vecs, int to_staging) {
  const uint32_t first = blockIdx.x * (256u * COPY_CU) + threadIdx.x;
  vec16 r[COPY_CU];
  char* to[COPY_CU];
#pragma unroll
  for (int u = 0; u < COPY_CU; ++u) {
    const uint32_t v = first + 256u * u;
    to[u] = nullptr;
    if (v < total_vecs) {
      const uint32_t i = v / block_vecs, off = v - i * block_vecs;
      const int64_t b = blocks[i];
      if (b >= 0 && b < num_blocks) {   // host validates
        char* p = pool + (b * block_vecs + off) * 16;
        char* st = staging + ((int64_t)i * block_vecs + off) * 16;
        r[u] = ld16(to_staging ? p : st);
        to[u] = to_staging ? st : p;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < COPY_CU; ++u)
    if (to[u]) st16(to[u], r[u]);
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
  const int64_t total = (int64_t)num_pairs * (block_bytes / 16);
  TB_CHECK_ARG(total < (int64_t)1 << 31);
  const unsigned wgs = (unsigned)((total + 256 * COPY_CU - 1) / (256 * COPY_CU));
  hipLaunchKernelGGL((block_copy_kernel<COPY_CU, true>), dim3(wgs, num_layers), dim3(256), 0, stream, layer_pools,
                     src_blocks, dst_blocks, num_blocks, (uint32_t)(block_bytes / 16), (uint32_t)total);
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
  const int64_t total = (int64_t)num_blocks_to_move * (block_bytes / 16);
  TB_CHECK_ARG(total < (int64_t)1 << 31);
  const unsigned wgs = (unsigned)((total + 256 * COPY_CU - 1) / (256 * COPY_CU));
  hipLaunchKernelGGL(block_stage_kernel, dim3(wgs), dim3(256), 0, stream, (char*)pool, (char*)staging, blocks,
                     num_blocks, (uint32_t)(block_bytes / 16), (uint32_t)total, 1);
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
  const int64_t total = (int64_t)num_blocks_to_move * (block_bytes / 16);
  TB_CHECK_ARG(total < (int64_t)1 << 31);
  const unsigned wgs = (unsigned)((total + 256 * COPY_CU - 1) / (256 * COPY_CU));
  hipLaunchKernelGGL(block_stage_kernel, dim3(wgs), dim3(256), 0, stream, (char*)pool, (char*)staging, blocks,
                     num_blocks, (uint32_t)(block_bytes / 16), (uint32_t)total, 0);
  TB_RETURN_LAUNCH_STATUS();
}
