// Per-head RMSNorm + rotate-half RoPE of one head row held by a 16-lane DPP row, shared by
// the fused producer kernel (qk_norm_rope.hip) and the fused decode step (paged_decode.hip),
// so both produce bit-identical q / k rows.
//
// Reference: src/layers/layernorm.py:11-16 (RMSNorm in fp32, weight multiply, round to
// bf16) and src/layers/pos_embedding.py:30-48 (RoPE on the bf16 value in fp32 with the fp32
// cos/sin row of the position, rounded to bf16). Lane c of the row holds elements
// [8c, 8c + 8); the rotate-half partner of element d is d +- 64, the same slot of lane c ^ 8.
#pragma once

#include "common.h"

namespace pk {

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

// cos and sin of this lane's 8 elements (columns d mod 64) at position pos, clamped into the
// (max_position, D) table: cos in [0, D/2), sin in [D/2, D).
__device__ __forceinline__ void rope_cos_sin_row(const float* cos_sin, int64_t max_position, int64_t pos, int c,
                                                 float cv[8], float sv[8]) {
  constexpr int D = kHeadDim;
  pos = pos < 0 ? 0 : (pos >= max_position ? max_position - 1 : pos);
  const float* cs = cos_sin + pos * D + (c & 7) * 8;
  const float4 c0 = *reinterpret_cast<const float4*>(cs);
  const float4 c1 = *reinterpret_cast<const float4*>(cs + 4);
  const float4 s0 = *reinterpret_cast<const float4*>(cs + D / 2);
  const float4 s1 = *reinterpret_cast<const float4*>(cs + D / 2 + 4);
  cv[0] = c0.x; cv[1] = c0.y; cv[2] = c0.z; cv[3] = c0.w; cv[4] = c1.x; cv[5] = c1.y; cv[6] = c1.z; cv[7] = c1.w;
  sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w; sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
}

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

}  // namespace pk
