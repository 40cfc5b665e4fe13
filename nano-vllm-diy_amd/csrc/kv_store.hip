// store_kvcache scatter and block-table gather for gfx950.
//
// Reference: store_kvcache_kernel (src/layers/attention.py:10-34) runs one Triton
// program per token and copies the token's K row and V row (num_kv_heads * head_dim
// elements each) into slot slot_mapping[i], skipping slot -1.
//
// Here a work-group moves the rows of a few consecutive tokens (4 tokens of a 2 KiB
// row): a thread moves two 16-byte chunks of K rows and the matching chunks of the V
// rows, so a wavefront stores 1 KiB of contiguous cache row per operand and
// instruction, with dwordx4 stores. The copy is a bit copy: results are identical to
// the reference for any 16-bit dtype.
#include "common.h"

namespace pk {
namespace {

constexpr int kStoreThreads = 256;
// 16-byte chunks per thread and round, loads issued together. Measured (cold caches, K and V
// rows of 2 KiB, µs for 16384 / 2048 / 256 tokens): 2 chunks 26.2 / 7.4 / 6.2, 4 chunks
// 26.9 / 8.6 / 7.0, 8 chunks 26.4 / 10.6 / 9.5; non-temporal loads of the new rows no faster;
// non-temporal cache stores 26.5 -> 29.8 at 16384 tokens; two or four rounds per work-group
// (fewer, longer work-groups) 28.0 and 26.8 at 16384 tokens, slower at 2048 and 256.
#ifndef PK_STORE_UNROLL
#define PK_STORE_UNROLL 2
#endif
constexpr int kStoreUnroll = PK_STORE_UNROLL;
constexpr int kStoreChunks = kStoreThreads * kStoreUnroll;  // chunks a work-group moves per round

// Work-group x moves tokens [x * tokens_per_group, ...): its chunks are numbered i = token
// offset * row_vec + chunk, and a round gives thread j chunks j, j + 256, ....
// The token of chunk i is i >> row_shift when the row is a power of two of chunks (every
// head geometry with a power-of-two kv head count and head_dim 128), else a 32-bit
// division. All slot loads of a round go out first, then all K and V loads (from a valid
// row even where the slot is -1, so no load waits behind a branch), then the stores.
__global__ __launch_bounds__(kStoreThreads) void store_kvcache_kernel(
    const uint4* __restrict__ key, int64_t key_row_vec, const uint4* __restrict__ value,
    int64_t value_row_vec, uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int32_t num_tokens, int32_t row_vec, int32_t row_shift,
    int32_t tokens_per_group, int64_t num_slots) {
  const int32_t t0 = blockIdx.x * tokens_per_group;
  const int32_t n = min(tokens_per_group, num_tokens - t0) * row_vec;  // chunks of this work-group
  for (int32_t base = 0; base < n; base += kStoreChunks) {
    int32_t tok[kStoreUnroll], chunk[kStoreUnroll], slot[kStoreUnroll];
#pragma unroll
    for (int j = 0; j < kStoreUnroll; ++j) {
      const int32_t i = min(base + j * kStoreThreads + (int32_t)threadIdx.x, n - 1);
      const int32_t t = row_shift >= 0 ? i >> row_shift : i / row_vec;
      tok[j] = t0 + t;
      chunk[j] = i - t * row_vec;
      slot[j] = slot_mapping[tok[j]];
    }
    uint4 kv[kStoreUnroll], vv[kStoreUnroll];
#pragma unroll
    for (int j = 0; j < kStoreUnroll; ++j) {
      kv[j] = key[(int64_t)tok[j] * key_row_vec + chunk[j]];
      vv[j] = value[(int64_t)tok[j] * value_row_vec + chunk[j]];
    }
#pragma unroll
    for (int j = 0; j < kStoreUnroll; ++j) {
      const int32_t s = slot[j];
      const bool live = base + j * kStoreThreads + (int32_t)threadIdx.x < n && s != -1 &&  // attention.py:23
                        (num_slots <= 0 || (s >= 0 && (int64_t)s < num_slots));          // opt-in bound check
      if (live) {
        const int64_t dst = (int64_t)s * row_vec + chunk[j];
        k_cache[dst] = kv[j];
        v_cache[dst] = vv[j];
      }
    }
  }
}

// dst[(cu_k[b] + t) * row + e] = cache[block_table[b][t / bs] * block_stride + (t % bs) * row + e]
__global__ __launch_bounds__(kStoreThreads) void gather_kv_kernel(
    const uint4* __restrict__ cache, int64_t block_stride_vec, int32_t block_size,
    const int32_t* __restrict__ block_table, int32_t bt_stride, const int32_t* __restrict__ cu_k,
    int32_t row_vec, uint4* __restrict__ dst) {
  const int32_t b = blockIdx.y;
  const int32_t k0 = cu_k[b];
  const int32_t len = cu_k[b + 1] - k0;
  if (len <= 0) return;
  const int64_t total = (int64_t)len * row_vec;
  const int64_t step = (int64_t)gridDim.x * kStoreThreads;
  for (int64_t idx = (int64_t)blockIdx.x * kStoreThreads + threadIdx.x; idx < total; idx += step) {
    const int32_t t = (int32_t)(idx / row_vec);
    const int32_t chunk = (int32_t)(idx - (int64_t)t * row_vec);
    const int32_t blk = block_table[(int64_t)b * bt_stride + t / block_size];
    const int32_t off = t % block_size;
    dst[(int64_t)(k0 + t) * row_vec + chunk] =
        cache[(int64_t)blk * block_stride_vec + (int64_t)off * row_vec + chunk];
  }
}

}  // namespace

hipError_t launch_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                int64_t value_row_stride, void* k_cache, void* v_cache,
                                const int32_t* slot_mapping, int32_t num_tokens,
                                int32_t row_elems, int64_t num_slots, hipStream_t stream) {
  if (num_tokens <= 0) return hipSuccess;
  const int32_t row_vec = row_elems / 8;
  int32_t row_shift = -1;
  if ((row_vec & (row_vec - 1)) == 0) row_shift = __builtin_ctz((unsigned)row_vec);
  // one round of kStoreChunks chunks per work-group (4 tokens of a 2 KiB row), at least one token
  const int32_t per_group = row_vec >= kStoreChunks ? 1 : kStoreChunks / row_vec;
  const int64_t groups = ((int64_t)num_tokens + per_group - 1) / per_group;
  hipLaunchKernelGGL(store_kvcache_kernel, dim3((unsigned)groups), dim3(kStoreThreads), 0, stream,
                     static_cast<const uint4*>(key), key_row_stride / 8,
                     static_cast<const uint4*>(value), value_row_stride / 8,
                     static_cast<uint4*>(k_cache), static_cast<uint4*>(v_cache), slot_mapping,
                     num_tokens, row_vec, row_shift, per_group, num_slots);
  return hipGetLastError();
}

hipError_t launch_gather_kv(const void* cache, int64_t block_stride, int32_t block_size,
                            const int32_t* block_table, int32_t bt_stride, const int32_t* cu_k,
                            int32_t num_seqs, int32_t max_seqlen_k, int32_t row_elems, void* dst,
                            hipStream_t stream) {
  if (num_seqs <= 0 || max_seqlen_k <= 0) return hipSuccess;
  const int32_t row_vec = row_elems / 8;
  const int64_t per_seq = (int64_t)max_seqlen_k * row_vec;
  int64_t bx = (per_seq + kStoreThreads - 1) / kStoreThreads;
  if (bx > 4096) bx = 4096;
  hipLaunchKernelGGL(gather_kv_kernel, dim3((unsigned)bx, (unsigned)num_seqs), dim3(kStoreThreads),
                     0, stream, static_cast<const uint4*>(cache), block_stride / 8, block_size,
                     block_table, bt_stride, cu_k, row_vec, static_cast<uint4*>(dst));
  return hipGetLastError();
}

}  // namespace pk
