// Fused producer of the attention inputs for gfx950: per-head RMSNorm of q and k, rotary
// embedding of q and k, and the store of the new K and V rows into the paged cache.
//
// Reference (src/models/qwen3.py:80-89): after the fused qkv projection the layer runs
//   q = q_norm(q); k = k_norm(k)            RMSNorm over head_dim (src/layers/layernorm.py:11-16)
//   q, k = rotary_emb(q, k, positions)      rotate-half RoPE      (src/layers/pos_embedding.py:30-48)
//   attn(q, k, v, ctx) -> store_kvcache      K and V rows to slot  (src/layers/attention.py:10-34,87-88)
// as four passes over q/k (two norms, one RoPE, one store) plus the V copy. Here one pass
// reads the fused qkv row once and writes q, the cache rows and, when the attention reads
// fresh keys (no block table), k.
//
// Arithmetic follows the reference's rounding points: the norm is computed in fp32 and
// rounded to bf16 after the weight multiply (layernorm.py:16); RoPE upcasts that bf16 value,
// rotates in fp32 with the fp32 cos/sin table row of the token's position and rounds to bf16
// again (pos_embedding.py:40-46).
//
// Lane layout: a 16-lane DPP row owns one head row of D = 128 elements at a time, lane c
// holding elements [8c, 8c + 8); the four DPP rows of a wavefront share one token. The
// rotate-half partner of element d is d + 64 (d < 64) or d - 64, i.e. the same slot of
// lane c ^ 8, one DPP row rotation by 8 away. The sum of squares of the norm is a 16-lane
// DPP reduction. In the fused row [q heads | k heads | v heads] head row r starts at
// element r * D, so every row is addressed the same way.
#include "norm_rope.h"

namespace pk {
namespace {

constexpr int kProdThreads = 256;
struct ProducerArgs {
  const uint16_t* qkv;          // (N, (Hq + 2 Hkv) * D), row stride qkv_row_stride
  int64_t qkv_row_stride;
  const int64_t* positions;     // (N,)
  const float* cos_sin;         // (max_position, D): cos in [0, D/2), sin in [D/2, D)
  int64_t max_position;
  const uint16_t* q_weight;     // (D,) bf16 or nullptr (no norm)
  const uint16_t* k_weight;
  float eps;
  int32_t num_tokens;
  int32_t num_heads, num_kv_heads;
  uint16_t* q_out;              // (N, Hq, D), row stride q_out_row_stride
  int64_t q_out_row_stride;
  uint16_t* k_out;              // (N, Hkv, D) or nullptr
  int64_t k_out_row_stride;
  uint16_t* k_cache;            // slot rows of Hkv * D, or nullptr (no store)
  uint16_t* v_cache;
  const int32_t* slot_mapping;
  int64_t num_slots;            // > 0: slots outside [0, num_slots) are not written
};

// Rows a DPP row (16 lanes) keeps in flight: its loads for one token are issued together.
#ifndef PK_PROD_ROWS_IN_FLIGHT
#define PK_PROD_ROWS_IN_FLIGHT 8
#endif
constexpr int kRowsInFlight = PK_PROD_ROWS_IN_FLIGHT;
// Batches below this many tokens spread each token over several wavefronts (more
// wavefronts in flight for a latency-bound launch).
#ifndef PK_PROD_SPREAD_BELOW
#define PK_PROD_SPREAD_BELOW 1024
#endif

// One work item = one token's share `part` of `parts` (grid-stride, one wavefront per
// item): the token's position and slot are wave-uniform loads, the cos/sin row is read once
// per lane, and DPP row j of the wave walks head rows r = 4 (part + parts i) + j with up to
// kRowsInFlight row loads issued before any is used.
__global__ __launch_bounds__(kProdThreads) void qk_norm_rope_store_kernel(const ProducerArgs a,
                                                                          int parts) {
  constexpr int D = kHeadDim;
  constexpr int kWavesPerBlock = kProdThreads / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int c = lane & (kLanesPerRow - 1);
  const int row0 = lane / kLanesPerRow;                          // this DPP row's first head row
  const bool lower = c < kLanesPerRow / 2;
  const int rows = a.num_heads + 2 * a.num_kv_heads;            // head rows per token
  const int64_t row_elems = (int64_t)a.num_kv_heads * D;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t items = (int64_t)a.num_tokens * parts;
  for (int64_t item = (int64_t)blockIdx.x * kWavesPerBlock + wave; item < items;
       item += (int64_t)gridDim.x * kWavesPerBlock) {
    const int32_t token = (int32_t)(item / parts);
    const int part = (int)(item - (int64_t)token * parts);
    const uint16_t* src = a.qkv + (int64_t)token * a.qkv_row_stride + c * 8;
    int32_t slot = -1;
    if (a.k_cache != nullptr) {
      slot = a.slot_mapping[token];
      if (slot < 0 || (a.num_slots > 0 && (int64_t)slot >= a.num_slots)) slot = -1;
    }
    float cv[8], sv[8];
    rope_cos_sin_row(a.cos_sin, a.max_position, a.positions[token], c, cv, sv);

    const int stride = 4 * parts;                                // between this row's head rows
    for (int base = 4 * part + row0; base < rows; base += stride * kRowsInFlight) {
      uint4 w[kRowsInFlight];
#pragma unroll
      for (int i = 0; i < kRowsInFlight; ++i) {
        const int r = base + stride * i;
        w[i] = *reinterpret_cast<const uint4*>(src + (r < rows ? r : base) * D);
      }
#pragma unroll
      for (int i = 0; i < kRowsInFlight; ++i) {
        const int r = base + stride * i;
        if (r >= rows) break;
        if (r >= a.num_heads + a.num_kv_heads) {  // attention.py:28,34: raw V row into its slot
          if (slot != -1) {
            const int g = r - a.num_heads - a.num_kv_heads;
            *reinterpret_cast<uint4*>(a.v_cache + (int64_t)slot * row_elems + g * D + c * 8) = w[i];
          }
        } else if (r < a.num_heads) {
          const uint4 ow = norm_rope_row(w[i], a.q_weight, a.eps, cv, sv, lower, c);
          *reinterpret_cast<uint4*>(a.q_out + (int64_t)token * a.q_out_row_stride + r * D + c * 8) = ow;
        } else {
          const uint4 ow = norm_rope_row(w[i], a.k_weight, a.eps, cv, sv, lower, c);
          const int g = r - a.num_heads;
          if (a.k_out != nullptr)
            *reinterpret_cast<uint4*>(a.k_out + (int64_t)token * a.k_out_row_stride + g * D + c * 8) = ow;
          if (slot != -1)  // attention.py:27,33
            *reinterpret_cast<uint4*>(a.k_cache + (int64_t)slot * row_elems + g * D + c * 8) = ow;
        }
      }
    }
  }
}

}  // namespace

hipError_t launch_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride,
                                     const int64_t* positions, const float* cos_sin,
                                     int64_t max_position, const void* q_norm_weight,
                                     const void* k_norm_weight, float eps, int32_t num_tokens,
                                     int32_t num_heads, int32_t num_kv_heads, void* q_out,
                                     int64_t q_out_row_stride, void* k_out,
                                     int64_t k_out_row_stride, void* k_cache, void* v_cache,
                                     const int32_t* slot_mapping, int64_t num_slots,
                                     hipStream_t stream) {
  if (num_tokens <= 0) return hipSuccess;
  ProducerArgs a;
  a.qkv = static_cast<const uint16_t*>(qkv);
  a.qkv_row_stride = qkv_row_stride;
  a.positions = positions;
  a.cos_sin = cos_sin;
  a.max_position = max_position;
  a.q_weight = static_cast<const uint16_t*>(q_norm_weight);
  a.k_weight = static_cast<const uint16_t*>(k_norm_weight);
  a.eps = eps;
  a.num_tokens = num_tokens;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.q_out_row_stride = q_out_row_stride;
  a.k_out = static_cast<uint16_t*>(k_out);
  a.k_out_row_stride = k_out_row_stride;
  a.k_cache = static_cast<uint16_t*>(k_cache);
  a.v_cache = static_cast<uint16_t*>(v_cache);
  a.slot_mapping = slot_mapping;
  a.num_slots = num_slots;
  const int quads = (num_heads + 2 * num_kv_heads + 3) / 4;  // 4 head rows per wavefront step
  int parts = num_tokens < PK_PROD_SPREAD_BELOW ? 4 : 1;
  if (parts > quads) parts = quads;
  const int64_t per_block = kProdThreads / kWave;             // one wavefront per work item
  int64_t blocks = ((int64_t)num_tokens * parts + per_block - 1) / per_block;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(qk_norm_rope_store_kernel, dim3((unsigned)blocks), dim3(kProdThreads), 0,
                     stream, a, parts);
  return hipGetLastError();
}

}  // namespace pk
