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
#include "common.h"

namespace pk {
namespace {

constexpr int kProdThreads = 256;
constexpr int kLanesPerRow = kHeadDim / 8;   // 16: one DPP row per head row
constexpr int kDppRowRor8 = 0x128;           // row_ror:8 -> lane (c + 8) mod 16 = c ^ 8

__device__ __forceinline__ float dpp_ror8(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kDppRowRor8, 0xf, 0xf, false));
}

__device__ __forceinline__ float round_bf16(float f) {
  return __uint_as_float((uint32_t)f32_to_bf16(f) << 16);
}

__device__ __forceinline__ void unpack8(const uint4 w, float f[8]) {
  f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
}

__device__ __forceinline__ uint4 pack8(const float f[8]) {
  uint4 w;
  w.x = pack_bf16x2(f[0], f[1]);
  w.y = pack_bf16x2(f[2], f[3]);
  w.z = pack_bf16x2(f[4], f[5]);
  w.w = pack_bf16x2(f[6], f[7]);
  return w;
}

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

// Normalise + rotate one head row held as 8 elements per lane; returns the packed bf16 row.
__device__ __forceinline__ uint4 norm_rope_row(const uint4 w, const uint16_t* wt, float eps,
                                               const float cv[8], const float sv[8], bool lower,
                                               int c) {
  constexpr int D = kHeadDim;
  float f[8];
  unpack8(w, f);
  // RMSNorm (layernorm.py:11-16): fp32, weight multiply, round to bf16.
  if (wt != nullptr) {
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf(f[e], f[e], ss);
    ss = row16_sum(ss);
    const float rs = 1.0f / __builtin_sqrtf(ss * (1.0f / D) + eps);
    float wf[8];
    unpack8(*reinterpret_cast<const uint4*>(wt + c * 8), wf);
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = round_bf16(wf[e] * (f[e] * rs));
  }
  // RoPE (pos_embedding.py:37-46): t1 = x[:64], t2 = x[64:];
  //   out[:64] = t1 cos - t2 sin, out[64:] = t1 sin + t2 cos, cos/sin of column d mod 64.
  float o[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float p = dpp_ror8(f[e]);                  // element d +- 64
    const float t1 = lower ? f[e] : p;
    const float t2 = lower ? p : f[e];
    o[e] = lower ? t1 * cv[e] - t2 * sv[e] : t1 * sv[e] + t2 * cv[e];
  }
  return pack8(o);
}

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
    int64_t pos = a.positions[token];
    pos = pos < 0 ? 0 : (pos >= a.max_position ? a.max_position - 1 : pos);
    int32_t slot = -1;
    if (a.k_cache != nullptr) {
      slot = a.slot_mapping[token];
      if (slot < 0 || (a.num_slots > 0 && (int64_t)slot >= a.num_slots)) slot = -1;
    }
    const float* cs = a.cos_sin + pos * D + (c & 7) * 8;
    const float4 c0 = *reinterpret_cast<const float4*>(cs);
    const float4 c1 = *reinterpret_cast<const float4*>(cs + 4);
    const float4 s0 = *reinterpret_cast<const float4*>(cs + D / 2);
    const float4 s1 = *reinterpret_cast<const float4*>(cs + D / 2 + 4);
    const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
    const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};

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
