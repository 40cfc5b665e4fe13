// Split-K paged decode attention for gfx950 (one query row per sequence).
//
// Reference semantics: flash_attn_varlen_func with max_seqlen_q == 1 and a block
// table (src/layers/attention.py:95-104, replayed inside the decode graph,
// src/engine/model_runner.py:245-259). For sequence b and query head h:
//     o = softmax(scale * q . K_b^T) V_b,   K_b[t] = k_cache[bt[b][t / BS], t % BS, h / G]
// over all Lk keys (a single bottom-right-aligned causal row sees every key).
//
// Work decomposition
//   grid = (split, sequence, kv-head group of up to 8); one work-group per (sequence,
//   split of `split_tokens` keys); wavefront w of the group owns kv head g and both
//   (all G) query heads that read it, so every K/V row fetched from HBM serves the
//   whole GQA group. The 8 wavefronts of a group together read whole 2 KiB token rows.
//
// Lane layout inside a wavefront: lane = 16 * r + c. Lanes of DPP row r hold key
// row (t + 4u + r) for unrolled step u; lane c holds head_dim elements [8c, 8c+8).
//   * q.k: 8 FMAs per head per lane, then a 4-step DPP sum across the 16-lane row;
//     every lane of the row ends with the full score of its key, so the softmax
//     weight p needed for P.V is already in the lane that holds that key's V chunk.
//   * running max: one xor-16/xor-32 exchange per step of 4U keys.
//   * acc[h][8 elements] += p * v is lane-local; the 4 rows are summed once per split.
// Partial (max, sum, acc) per (sequence, split, head) go to the workspace and a small
// combine kernel merges them; a sequence with one split writes its output directly.
#include "common.h"

namespace pk {
namespace {

constexpr int kDecodeMaxWaves = 8;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

template <int G, int U, bool PAGED>
__global__ __launch_bounds__(kWave* kDecodeMaxWaves) void decode_split_kernel(const AttnArgs a) {
  constexpr int D = kHeadDim;
  constexpr int STEP = 4 * U;  // keys per inner step of one wavefront
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int waves = blockDim.x / kWave;
  const int g = blockIdx.z * waves + wave;
  const int b = blockIdx.y;
  const int split = blockIdx.x;
  if (g >= a.num_kv_heads) return;
  const int q0 = a.cu_q[b];
  if (a.cu_q[b + 1] - q0 != 1) return;  // rows with Lq != 1 belong to the prefill kernel
  const int k0 = a.cu_k[b];
  const int Lk = min(a.cu_k[b + 1] - k0, a.max_seqlen_k);
  const int t_begin = split * a.split_tokens;
  if (t_begin >= Lk) return;            // also skips Lk <= 0 (graph padding)
  const int t_end = min(Lk, t_begin + a.split_tokens);
  const int nsplit = (Lk + a.split_tokens - 1) / a.split_tokens;

  const int r = lane >> 4;  // key sub-row 0..3
  const int c = lane & 15;  // head_dim chunk
  const int H = a.num_heads;

  float qf[G][8];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int h = g * G + i;
    const uint4 w = *reinterpret_cast<const uint4*>(a.q + (int64_t)q0 * a.q_row_stride + h * D + c * 8);
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      qf[i][2 * e] = bf16_lo(ww[e]) * a.scale_log2;
      qf[i][2 * e + 1] = bf16_hi(ww[e]) * a.scale_log2;
    }
  }

  float m[G], l[G], acc[G][8];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    m[i] = -INFINITY;
    l[i] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[i][e] = 0.f;
  }

  for (int t = t_begin; t < t_end; t += STEP) {
    // [t, t + STEP) lies inside one cache block: STEP divides block_size and split_tokens.
    const uint16_t* kp;
    const uint16_t* vp;
    if constexpr (PAGED) {
      const int blk = a.block_table[(int64_t)b * a.bt_stride + t / a.block_size];
      const int off = t % a.block_size;
      kp = a.k + (int64_t)blk * a.k_block_stride + (int64_t)off * a.k_row_stride;
      vp = a.v + (int64_t)blk * a.v_block_stride + (int64_t)off * a.v_row_stride;
    } else {
      kp = a.k + (int64_t)(k0 + t) * a.k_row_stride;
      vp = a.v + (int64_t)(k0 + t) * a.v_row_stride;
    }
    kp += g * D + c * 8;
    vp += g * D + c * 8;

    uint4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int j = 4 * u + r;
      if (t + j < t_end) {
        kr[u] = *reinterpret_cast<const uint4*>(kp + (int64_t)j * a.k_row_stride);
        vr[u] = *reinterpret_cast<const uint4*>(vp + (int64_t)j * a.v_row_stride);
      } else {
        kr[u] = make_uint4(0, 0, 0, 0);  // keys past Lk: score masked, value zero (no NaN * 0)
        vr[u] = make_uint4(0, 0, 0, 0);
      }
    }

    float s[U][G];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t kw[4] = {kr[u].x, kr[u].y, kr[u].z, kr[u].w};
#pragma unroll
      for (int i = 0; i < G; ++i) {
        float d0 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          d0 = fmaf(qf[i][2 * e], bf16_lo(kw[e]), d0);
          d0 = fmaf(qf[i][2 * e + 1], bf16_hi(kw[e]), d0);
        }
        s[u][i] = row16_sum(d0);
      }
      if (t + 4 * u + r >= t_end) {
#pragma unroll
        for (int i = 0; i < G; ++i) s[u][i] = -INFINITY;
      }
    }

#pragma unroll
    for (int i = 0; i < G; ++i) {
      float mx = s[0][i];
#pragma unroll
      for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[u][i]);
      mx = fmaxf(mx, xor_shfl(mx, 16));
      mx = fmaxf(mx, xor_shfl(mx, 32));
      const float m_new = fmaxf(m[i], mx);  // finite: the step holds >= 1 valid key
      const float alpha = exp2_fast(m[i] - m_new);
      m[i] = m_new;
      l[i] *= alpha;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[i][e] *= alpha;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const float p = exp2_fast(s[u][i] - m_new);
        l[i] += p;
        const uint32_t vw[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          acc[i][2 * e] = fmaf(p, bf16_lo(vw[e]), acc[i][2 * e]);
          acc[i][2 * e + 1] = fmaf(p, bf16_hi(vw[e]), acc[i][2 * e + 1]);
        }
      }
    }
  }

  // Sum the four key sub-rows (lanes c, c+16, c+32, c+48).
#pragma unroll
  for (int i = 0; i < G; ++i) {
    l[i] += xor_shfl(l[i], 16);
    l[i] += xor_shfl(l[i], 32);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[i][e] += xor_shfl(acc[i][e], 16);
      acc[i][e] += xor_shfl(acc[i][e], 32);
    }
  }

  if (r != 0) return;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int h = g * G + i;
    if (nsplit == 1) {
      const float inv = 1.f / l[i];
      uint4 w;
      w.x = pack_bf16x2(acc[i][0] * inv, acc[i][1] * inv);
      w.y = pack_bf16x2(acc[i][2] * inv, acc[i][3] * inv);
      w.z = pack_bf16x2(acc[i][4] * inv, acc[i][5] * inv);
      w.w = pack_bf16x2(acc[i][6] * inv, acc[i][7] * inv);
      *reinterpret_cast<uint4*>(a.out + (int64_t)q0 * a.out_row_stride + h * D + c * 8) = w;
    } else {
      const int64_t unit = ((int64_t)b * a.max_splits + split) * H + h;
      float4* po = reinterpret_cast<float4*>(a.part_o + unit * D + c * 8);
      po[0] = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
      po[1] = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
      if (c == 0) *reinterpret_cast<float2*>(a.part_ml + unit * 2) = make_float2(m[i], l[i]);
    }
  }
}

// Merge the per-split partials of one (sequence, head): thread d owns element d.
__global__ __launch_bounds__(kHeadDim) void decode_combine_kernel(const AttnArgs a) {
  constexpr int D = kHeadDim;
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int d = threadIdx.x;
  const int q0 = a.cu_q[b];
  if (a.cu_q[b + 1] - q0 != 1) return;
  const int Lk = min(a.cu_k[b + 1] - a.cu_k[b], a.max_seqlen_k);
  if (Lk <= 0) return;
  const int nsplit = (Lk + a.split_tokens - 1) / a.split_tokens;
  if (nsplit <= 1) return;  // written directly by the split kernel
  const int H = a.num_heads;
  const int64_t unit0 = (int64_t)b * a.max_splits * H + h;
  float mx = -INFINITY;
  for (int j = 0; j < nsplit; ++j) mx = fmaxf(mx, a.part_ml[(unit0 + (int64_t)j * H) * 2]);
  float lsum = 0.f, o = 0.f;
  for (int j = 0; j < nsplit; ++j) {
    const int64_t unit = unit0 + (int64_t)j * H;
    const float w = exp2_fast(a.part_ml[unit * 2] - mx);
    lsum = fmaf(w, a.part_ml[unit * 2 + 1], lsum);
    o = fmaf(w, a.part_o[unit * D + d], o);
  }
  a.out[(int64_t)q0 * a.out_row_stride + h * D + d] = f32_to_bf16(o / lsum);
}

template <int G, int U>
hipError_t launch_decode_g(const AttnArgs& a, bool paged, dim3 grid, dim3 block, hipStream_t stream) {
  if (paged)
    hipLaunchKernelGGL((decode_split_kernel<G, U, true>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((decode_split_kernel<G, U, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

}  // namespace

int decode_split_tokens(int num_seqs, int max_seqlen_k) {
  // One 256-key cache block per work-group when the batch yields enough work-groups
  // to cover the 256 CUs several times; shorter splits for small batches.
  int split = 256;
  while (split > 64 && (int64_t)num_seqs * ((max_seqlen_k + split - 1) / split) < 2048) split /= 2;
  return split;
}

hipError_t launch_decode(const AttnArgs& a, int group, bool paged, int max_seqlen_k,
                         hipStream_t stream) {
  if (a.num_seqs <= 0 || max_seqlen_k <= 0) return hipSuccess;
  const int waves = a.num_kv_heads < kDecodeMaxWaves ? a.num_kv_heads : kDecodeMaxWaves;
  const int zgroups = (a.num_kv_heads + waves - 1) / waves;
  const dim3 grid((unsigned)a.max_splits, (unsigned)a.num_seqs, (unsigned)zgroups);
  const dim3 block((unsigned)(waves * kWave));
  hipError_t err;
  switch (group) {
    case 1: err = launch_decode_g<1, 8>(a, paged, grid, block, stream); break;
    case 2: err = launch_decode_g<2, 8>(a, paged, grid, block, stream); break;
    case 4: err = launch_decode_g<4, 4>(a, paged, grid, block, stream); break;
    case 8: err = launch_decode_g<8, 2>(a, paged, grid, block, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (err != hipSuccess) return err;
  if (a.max_splits > 1) {
    hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)a.num_heads, (unsigned)a.num_seqs),
                       dim3(kHeadDim), 0, stream, a);
    err = hipGetLastError();
  }
  return err;
}

}  // namespace pk
