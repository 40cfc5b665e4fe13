// store_kvcache scatter and block-table gather for gfx950.
//
// Reference: store_kvcache_kernel (src/layers/attention.py:10-34) runs one Triton
// program per token and copies the token's K row and V row (num_kv_heads * head_dim
// elements each) into slot slot_mapping[i], skipping slot -1.
//
// Here a thread moves one 16-byte chunk of a K row and the matching chunk of the V
// row, so a wavefront stores 1 KiB of contiguous cache row per operand with
// dwordx4 stores and many tokens are in flight per work-group. The copy is a bit
// copy: results are identical to the reference for any 16-bit dtype.
#include "common.h"

namespace pk {
namespace {

constexpr int kStoreThreads = 256;

__global__ __launch_bounds__(kStoreThreads) void store_kvcache_kernel(
    const uint4* __restrict__ key, int64_t key_row_vec, const uint4* __restrict__ value,
    int64_t value_row_vec, uint4* __restrict__ k_cache, uint4* __restrict__ v_cache,
    const int32_t* __restrict__ slot_mapping, int32_t num_tokens, int32_t row_vec,
    int64_t num_slots) {
  const int64_t total = (int64_t)num_tokens * row_vec;
  const int64_t step = (int64_t)gridDim.x * kStoreThreads;
  for (int64_t idx = (int64_t)blockIdx.x * kStoreThreads + threadIdx.x; idx < total; idx += step) {
    const int32_t token = (int32_t)(idx / row_vec);
    const int32_t chunk = (int32_t)(idx - (int64_t)token * row_vec);
    const int32_t slot = slot_mapping[token];
    if (slot == -1) continue;                                        // attention.py:23
    if (num_slots > 0 && (slot < 0 || (int64_t)slot >= num_slots)) continue;  // opt-in bound check
    const uint4 kv = key[(int64_t)token * key_row_vec + chunk];
    const uint4 vv = value[(int64_t)token * value_row_vec + chunk];
    const int64_t dst = (int64_t)slot * row_vec + chunk;
    k_cache[dst] = kv;
    v_cache[dst] = vv;
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
  const int64_t total = (int64_t)num_tokens * row_vec;
  int64_t blocks = (total + kStoreThreads - 1) / kStoreThreads;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(store_kvcache_kernel, dim3((unsigned)blocks), dim3(kStoreThreads), 0, stream,
                     static_cast<const uint4*>(key), key_row_stride / 8,
                     static_cast<const uint4*>(value), value_row_stride / 8,
                     static_cast<uint4*>(k_cache), static_cast<uint4*>(v_cache), slot_mapping,
                     num_tokens, row_vec, num_slots);
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
