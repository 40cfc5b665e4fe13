// Shared definitions for the gfx950 paged-KV kernels (libpagedkv.so).
//
// Layout facts every kernel relies on (reference: src/engine/model_runner.py:159-165,
// src/layers/attention.py:51-53):
//   * a KV cache is (num_blocks, block_size, num_kv_heads, head_dim), 16-bit elements;
//     slot s = block * block_size + offset addresses one contiguous token row of
//     num_kv_heads * head_dim elements;
//   * q and out are (tokens, num_heads, head_dim) with heads contiguous inside a row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pk {

constexpr int kHeadDim = 128;   // the only head_dim built (Qwen3 family)
constexpr int kWave = 64;       // CDNA wavefront width

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

// Everything the attention kernels need; passed by value as the kernel argument.
struct AttnArgs {
  const uint16_t* q;
  int64_t q_row_stride;
  const uint16_t* k;
  const uint16_t* v;
  int64_t k_row_stride, v_row_stride;
  int64_t k_block_stride, v_block_stride;
  const int32_t* block_table;   // nullptr in flat mode
  int32_t bt_stride;
  int32_t block_size;
  const int32_t* cu_q;
  const int32_t* cu_k;
  int32_t num_seqs;
  int32_t max_seqlen_k;         // keys past this bound are ignored (keeps every access in bounds)
  int32_t num_heads;
  int32_t num_kv_heads;
  float scale_log2;             // softmax_scale * log2(e): scores live in the exp2 domain
  uint16_t* out;
  int64_t out_row_stride;
  // split-K decode scratch (workspace)
  uint16_t* part_o;             // [unit][num_heads][head_dim] bf16: the unit's normalised output o / l
  float* part_ml;               // [unit][num_heads][2] = (max in the exp2 domain, sum)
  int32_t stream_from;           // decode splits starting at key >= this use non-temporal loads (< 0: none)
  int32_t store_through;         // decode partials written through L2 (set by the decode launch)
  int32_t combine_in_merge;      // the decode combines run in the prefill merge kernel
  int32_t split_tokens;
  int32_t max_splits;           // partial slots per sequence (stride of part_o / part_ml)
  int32_t grid_splits;          // splits the decode grid covers per sequence
  // Flat decode grid (flat_groups > 0): the decode keys of the batch -- per decode sequence
  // b its keys after the shared prefix, c_b = Lk - min(prefix_keys, Lk) of them -- laid end
  // to end in sequence order (the key line: sequence b from position pos_b = c_0 + ... +
  // c_{b-1}) and cut into flat_groups runs of `chunk` keys; the piece of sequence b in run w
  // is work-group b + w and partial unit flat_unit0 + b + w. chunk >= flat_min_chunk is set
  // on the device; flat_meta holds chunk, then pos_b, for the combine. flat_step = keys per
  // pipeline step (set by the decode launch).
  int32_t flat_groups;
  int32_t flat_min_chunk;
  int32_t flat_step;
  int32_t flat_unit0;
  int32_t* flat_meta;
  // Shared-prefix decode: keys [0, min(prefix_keys, Lk)) of a decode sequence are computed by
  // the shared-prefix kernel, one partial per chunk of prefix_chunk keys in slots
  // [0, prefix_slots); the decode kernel covers the keys after them (split grid: its split s
  // in slot prefix_slots + s; flat grid: its pieces). prefix_keys == 0 (prefix_chunk 1,
  // prefix_slots 0): off.
  int32_t prefix_keys;
  int32_t prefix_chunk;
  int32_t prefix_slots;
  int32_t prefix_stride;        // partial units per sequence of the prefix chunk partials (chunk j of
                                // sequence b at unit b * prefix_stride + j)
  int32_t sp_replicas;          // shared-prefix kernel: work-groups per window of sequences (set by its launch)
  // One launch for the shared-prefix work and the flat decode grid (set by that launch):
  // work-groups [0, sp_groups) take the (chunk, kv head, window) prefix work and then
  // sp_tail flat groups each, the sp_decode work-groups after them sp_per flat groups each;
  // a flat group is sp_quads wavefronts (4 kv heads each, or 4 / R with key rows).
  int32_t sp_groups;
  int32_t sp_decode;
  int32_t sp_per;
  int32_t sp_tail;
  int32_t sp_quads;
  // chunked-prefill work plan (workspace): a work item is (sequence, kv head, query tile,
  // key-tile range); items of one query tile that was split over several key ranges write
  // fp32 partials that a merge pass combines.
  int32_t* pf_queue;            // kPrefillQueueInts header: 8 claim counters, item / merge counts, split size
  int4* pf_items;               // [pf_item_cap] groups (b, qt, tile_begin | tile_end << 16, partial group);
                                // item i = kv head i % Hkv of group i / Hkv
  int4* pf_merges;              // [pf_merge_cap] split units (b, qt, first partial group, splits)
  uint16_t* pf_part_o;          // [part][32 chunks of 4 dims][kPrefillRows][4] the split's output (bf16)
  float* pf_part_ml;            // [part][kPrefillRows][2] = (running max in the exp2 domain, sum)
  int32_t pf_item_cap;
  int32_t pf_merge_cap;
  int32_t pf_part_cap;
  int32_t pf_slots;             // persistent work-groups of the prefill kernel
  int32_t prefill_qtiles;       // upper bound on query tiles per sequence (from max_seqlen_q)
  // Fused decode step (qkv != nullptr): q is the per-head RMSNorm + RoPE of the q part of
  // the fused qkv row of the sequence's token, and the split holding the sequence's last key
  // first stores that token's normalised + rotated K row and raw V row at slot_mapping.
  const uint16_t* qkv;
  int64_t qkv_row_stride;
  const int64_t* positions;
  const float* cos_sin;         // (max_position, D): cos in [0, D/2), sin in [D/2, D)
  int64_t max_position;
  const uint16_t* q_norm;       // (D,) bf16 or nullptr
  const uint16_t* k_norm;
  float norm_eps;
  const int32_t* slot_mapping;
  int64_t num_slots;            // > 0: slots outside [0, num_slots) are not written
  // Fused store + decode (new_k != nullptr, qkv == nullptr): q comes from `q`, and the
  // token's K and V rows from new_k / new_v (row = the token's index) go to slot_mapping
  // unchanged, as store_kvcache writes them.
  const uint16_t* new_k;
  int64_t new_k_stride;
  const uint16_t* new_v;
  int64_t new_v_stride;
};

// Shared-prefix decode limits: batches of up to this many sequences, chunks of at most two
// cache blocks (a group's key compares two block ids).
constexpr int kSharedPrefixMaxSeqs = 1024;
constexpr int kSharedPrefixMaxChunkBlocks = 2;

// Prefill plan sizes. The kernel runs kPrefillSlotsMax persistent work-groups at most (one
// per CU on a 256-CU part). The split size T is at least 2/3 x total work / slots, and
// every split unit has more than T tiles, so its n splits satisfy n < 2 t / T: fewer than
// 3 x slots partials (all kv heads) ever exist, in fewer than 1.5 x slots split units.
constexpr int kPrefillSlotsMax = 256;
constexpr int kPrefillQueueStride = 32;  // claim counter q at pf_queue[32 q]: one 128-byte line each
constexpr int kPrefillQueueMeta = 8 * kPrefillQueueStride;  // then item count, merge count, split size
constexpr int kPrefillQueueInts = kPrefillQueueMeta + 64;   // header ints (1280 bytes)
constexpr int kPrefillRows = 256;       // query rows per work item (query tokens x GQA heads)
constexpr int kPrefillPartCap = 3 * kPrefillSlotsMax;
constexpr int kPrefillMergeCap = 3 * kPrefillSlotsMax / 2;
// Groups: one per (sequence, query tile) plus the extra splits (fewer than partials).
// Query tiles per sequence are at most ceil(Lq * G / 256) <= ceil(Lq * Hq / 256).
inline int64_t prefill_item_cap(int num_seqs, int num_heads, int max_seqlen_q) {
  return (int64_t)num_seqs * (((int64_t)max_seqlen_q * num_heads + kPrefillRows - 1) / kPrefillRows) +
         kPrefillPartCap;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// fp32 -> bf16, round to nearest even (gfx950 converts in hardware).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}

// DPP lane moves inside a 16-lane row (bound_ctrl: out-of-row sources read 0).
template <int kCtrl>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4e;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <- lane 7-i inside each half-row
constexpr int kDppMirror = 0x140;     // lane i <- lane 15-i inside each row

// Sum over the 16 lanes of a DPP row; every lane of the row receives the total.
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return v;
}

// Maximum over the 16 lanes of a DPP row; every lane of the row receives it.
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return v;
}

// Lane `l`'s value (l a compile-time constant), in a scalar register for the wavefront.
__device__ __forceinline__ float lane_value(float v, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ float xor_shfl(float v, int mask) { return __shfl_xor(v, mask, kWave); }

}  // namespace pk

// Host-side launchers (one per kernel file); each returns a hipError_t.
namespace pk {
hipError_t launch_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                                int64_t value_row_stride, void* k_cache, void* v_cache,
                                const int32_t* slot_mapping, int32_t num_tokens,
                                int32_t row_elems, int64_t num_slots, hipStream_t stream);
hipError_t launch_gather_kv(const void* cache, int64_t block_stride, int32_t block_size,
                            const int32_t* block_table, int32_t bt_stride,
                            const int32_t* cu_k, int32_t num_seqs, int32_t max_seqlen_k,
                            int32_t row_elems, void* dst, hipStream_t stream);
// Split-K decode over sequences with exactly one query row, plus the combine pass.
hipError_t launch_decode(const AttnArgs& a, int group, bool paged, int max_seqlen_k,
                         hipStream_t stream);
// Decode rows over their shared-prefix keys (a.prefix_keys > 0): MFMA tiles of the query rows
// of every sequence whose block table names the same blocks, one partial per chunk.
hipError_t launch_shared_prefix(const AttnArgs& a, int group, hipStream_t stream);
// The shared-prefix work and the flat decode grid over the keys after the prefix in one launch
// (when the flat grid is on and the kv heads divide into the work-group's wavefronts);
// returns false (nothing launched) when the separate launches apply.
bool launch_shared_prefix_flat(AttnArgs& a, int group, hipStream_t stream, hipError_t* err);
// The decode launch's combine pass alone (after launch_shared_prefix_flat).
hipError_t launch_decode_combine(const AttnArgs& a, int group, hipStream_t stream);
// bf16-MFMA attention over sequences with more than one query row.
hipError_t launch_prefill(const AttnArgs& a, int group, bool paged, bool causal,
                          int max_seqlen_q, hipStream_t stream);
// Split size (keys per work-group) the decode kernel uses for these launch bounds.
int decode_split_tokens(int num_seqs, int max_seqlen_k);
// Flat decode grid for these launch bounds: groups == 0 when the split grid is used.
struct FlatDecodePlan {
  int groups;
  int min_chunk;
};
FlatDecodePlan decode_flat_plan(int num_seqs, int max_seqlen_k);
// Per-head RMSNorm + RoPE of q and k from the fused qkv row, K/V rows into their slots.
hipError_t launch_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride,
                                     const int64_t* positions, const float* cos_sin,
                                     int64_t max_position, const void* q_norm_weight,
                                     const void* k_norm_weight, float eps, int32_t num_tokens,
                                     int32_t num_heads, int32_t num_kv_heads, void* q_out,
                                     int64_t q_out_row_stride, void* k_out,
                                     int64_t k_out_row_stride, void* k_cache, void* v_cache,
                                     const int32_t* slot_mapping, int64_t num_slots,
                                     hipStream_t stream);
// Residual add + RMSNorm, SiLU * mul and the greedy LM head of the serving loop.
hipError_t launch_add_rmsnorm(const void* x, int64_t x_stride, const void* residual,
                              int64_t res_stride, const void* weight, float eps, int32_t rows,
                              int32_t hidden, void* out, int64_t out_stride, void* residual_out,
                              int64_t res_out_stride, hipStream_t stream);
hipError_t launch_silu_and_mul(const void* x, int64_t x_stride, int32_t rows, int32_t inter,
                               void* out, int64_t out_stride, hipStream_t stream);
// Decode-step linear layers (at most 128 rows) with fused epilogues.
constexpr int kLinearStore = 0;       // y = bf16(x W^T)
constexpr int kLinearSiluMul = 1;     // y = bf16(silu(g) * u) of the merged gate / up weight
constexpr int kLinearAddRmsNorm = 2;  // residual add + RMSNorm of bf16(x W^T)
constexpr int kLinearMaxRows = 128;
size_t linear_workspace_bytes(int32_t rows, int32_t n_out, int32_t k, int32_t epilogue);
hipError_t launch_linear(const void* x, int64_t x_stride, const void* w, int64_t w_stride, int32_t rows,
                         int32_t n_out, int32_t k, int32_t epilogue, void* y, int64_t y_stride, void* ws,
                         hipStream_t stream);
hipError_t launch_linear_add_rmsnorm(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                                     int32_t rows, int32_t n_out, int32_t k, const void* residual,
                                     int64_t res_stride, const void* norm_weight, float eps, void* out,
                                     int64_t out_stride, void* residual_out, int64_t res_out_stride, void* ws,
                                     hipStream_t stream);
hipError_t launch_lm_head_greedy(const void* x, int64_t x_stride, const int32_t* cu_rows,
                                 const void* w, int64_t w_stride, int32_t rows, int32_t vocab,
                                 int32_t k_dim, unsigned long long* keys, int32_t* ids,
                                 hipStream_t stream);
}  // namespace pk
