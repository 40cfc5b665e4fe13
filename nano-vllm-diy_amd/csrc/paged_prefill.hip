// Chunked-prefill / dense varlen attention on bf16 MFMA for gfx950.
//
// Reference semantics: flash_attn_varlen_func(..., causal=True, block_table) at
// src/layers/attention.py:95-104 for sequences with Lq > 1 query rows. Row i of a
// sequence with Lq rows and Lk keys sees keys t <= i + (Lk - Lq) (bottom-right
// alignment, the cached prefix P = Lk - Lq precedes the chunk; model_runner.py:186-190).
// Keys come through the block table (paged, chunked prefill / prefix-cache hits) or
// from fresh rows at cu_seqlens_k (flat, all-fresh prompts).
//
// Work decomposition: grid = (query tile, kv head g, sequence). A work-group of four
// wavefronts owns 128 query rows = TM = 128 / G query tokens x the G query heads of kv
// head g, so each K/V tile staged in LDS serves the whole GQA group. Wavefront w owns
// 32 rows (one head, 32 consecutive tokens, or 2 heads x 16 tokens when G = 8).
//
// Per 64-key tile:
//   S^T (64 keys x 32 rows)  = K (64 x 128) . Q^T (128 x 32)   2 x 8 v_mfma_f32_32x32x16_bf16
//   online softmax down each column (a lane owns one query row: 32 scores in registers,
//   one xor-32 exchange for the column max)
//   O^T (128 x 32)          += V^T (128 x 64) . P^T (64 x 32)   4 x 4 v_mfma_f32_32x32x16_bf16
// K is staged row-major in LDS; V is staged transposed (d-major) so that the MFMA A
// operand (8 keys of one d) is two 8-byte LDS reads. P^T never leaves registers: the
// S^T accumulator layout already holds, per lane, the keys the P.V B operand needs
// once the k-order of the instruction is permuted (same permutation on the V^T side).
#include "common.h"

namespace pk {
namespace {

constexpr int kTileKeys = 64;
constexpr int kPrefillThreads = 256;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ uint32_t dword_of(const uint4& w, int i) {
  return i == 0 ? w.x : (i == 1 ? w.y : (i == 2 ? w.z : w.w));
}

template <int G, bool PAGED, bool CAUSAL>
__global__ __launch_bounds__(kPrefillThreads) void prefill_kernel(const AttnArgs a) {
  constexpr int D = kHeadDim;
  constexpr int TN = kTileKeys;
  constexpr int TM = 128 / G;  // query tokens per work-group
  constexpr int KS = D + 8;    // LDS row stride of the K tile (elements)
  constexpr int VS = TN + 4;   // LDS row stride of the transposed V tile (elements)
  __shared__ __attribute__((aligned(16))) uint16_t sK[TN * KS];
  __shared__ __attribute__((aligned(16))) uint16_t sVt[D * VS];

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int qt = blockIdx.x;
  const int g = blockIdx.y;
  const int b = blockIdx.z;

  const int q0 = a.cu_q[b];
  const int Lq = a.cu_q[b + 1] - q0;
  if (Lq <= 1) return;  // Lq == 1 rows belong to the decode kernel; Lq <= 0 is padding
  const int k0 = a.cu_k[b];
  const int Lk = min(a.cu_k[b + 1] - k0, a.max_seqlen_k);
  if (Lk <= 0) return;
  const int tok_begin = qt * TM;
  if (tok_begin >= Lq) return;
  const int P = Lk - Lq;  // cached prefix length
  int kv_end = Lk;
  if (CAUSAL) kv_end = min(Lk, tok_begin + TM + P);  // keys any row of this tile can see

  const int col = lane & 31;   // MFMA column = this lane's query row
  const int half = lane >> 5;
  const int row = wave * 32 + col;
  const int h = g * G + row / TM;
  const int tok = tok_begin + row % TM;
  const bool row_valid = tok < Lq;
  const int lim = CAUSAL ? min(Lk - 1, tok + P) : Lk - 1;  // last key this row sees

  // Q^T B operand: k-block kb covers d in [16 kb, 16 kb + 16); lane holds 8 of them.
  bf16x8 qb[D / 16];
  {
    const uint16_t* qp = a.q + (int64_t)(q0 + (row_valid ? tok : 0)) * a.q_row_stride + h * D + 8 * half;
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb) {
      uint4 w = make_uint4(0, 0, 0, 0);
      if (row_valid) w = *reinterpret_cast<const uint4*>(qp + kb * 16);
      qb[kb] = __builtin_bit_cast(bf16x8, w);
    }
  }

  f32x16 o[4];
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) o[md][rr] = 0.f;
  float m_i = -INFINITY;
  float l_i = 0.f;

  for (int t0 = 0; t0 < kv_end; t0 += TN) {
    const uint16_t* kbase;
    const uint16_t* vbase;
    if constexpr (PAGED) {
      // block_size % 64 == 0, so the 64-key tile sits inside one cache block.
      const int blk = a.block_table[(int64_t)b * a.bt_stride + t0 / a.block_size];
      const int off = t0 % a.block_size;
      kbase = a.k + (int64_t)blk * a.k_block_stride + (int64_t)off * a.k_row_stride;
      vbase = a.v + (int64_t)blk * a.v_block_stride + (int64_t)off * a.v_row_stride;
    } else {
      kbase = a.k + (int64_t)(k0 + t0) * a.k_row_stride;
      vbase = a.v + (int64_t)(k0 + t0) * a.v_row_stride;
    }
    kbase += g * D;
    vbase += g * D;

    __syncthreads();  // the previous tile is no longer read
    // K tile: 64 keys x 16 chunks of 16 B; keys past Lk are zero (masked below).
#pragma unroll
    for (int i = 0; i < (TN * D / 8) / kPrefillThreads; ++i) {
      const int idx = tid + kPrefillThreads * i;
      const int tk = idx >> 4;
      const int ch = idx & 15;
      uint4 w = make_uint4(0, 0, 0, 0);
      if (t0 + tk < Lk) w = *reinterpret_cast<const uint4*>(kbase + (int64_t)tk * a.k_row_stride + ch * 8);
      *reinterpret_cast<uint4*>(&sK[tk * KS + ch * 8]) = w;
    }
    // V tile, transposed: thread (ch, tq) loads keys 4tq..4tq+3 of chunk ch and writes
    // 8 rows of V^T, 4 keys (8 bytes) each. Keys past Lk are zero so P.V stays finite.
    {
      const int ch = tid & 15;
      const int tq = tid >> 4;
      uint4 w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int tk = 4 * tq + j;
        w[j] = make_uint4(0, 0, 0, 0);
        if (t0 + tk < Lk) w[j] = *reinterpret_cast<const uint4*>(vbase + (int64_t)tk * a.v_row_stride + ch * 8);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t x0 = dword_of(w[0], e >> 1), x1 = dword_of(w[1], e >> 1);
        const uint32_t x2 = dword_of(w[2], e >> 1), x3 = dword_of(w[3], e >> 1);
        uint2 pr;
        if (e & 1) {
          pr.x = (x0 >> 16) | (x1 & 0xffff0000u);
          pr.y = (x2 >> 16) | (x3 & 0xffff0000u);
        } else {
          pr.x = (x0 & 0xffffu) | (x1 << 16);
          pr.y = (x2 & 0xffffu) | (x3 << 16);
        }
        *reinterpret_cast<uint2*>(&sVt[(ch * 8 + e) * VS + 4 * tq]) = pr;
      }
    }
    __syncthreads();

    // S^T = K . Q^T. Accumulator element rr of half-tile mb is key
    // t0 + 32 mb + 8 (rr >> 2) + 4 half + (rr & 3), column = this lane's row.
    f32x16 s[2];
#pragma unroll
    for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) s[mb][rr] = 0.f;
#pragma unroll
      for (int kb = 0; kb < D / 16; ++kb) {
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(&sK[(mb * 32 + col) * KS + kb * 16 + 8 * half]);
        s[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, qb[kb], s[mb], 0, 0, 0);
      }
    }

    float tmax = -INFINITY;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const int t = t0 + mb * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3);
        float v = s[mb][rr] * a.scale_log2;
        if (t > lim) v = -INFINITY;
        s[mb][rr] = v;
        tmax = fmaxf(tmax, v);
      }
    tmax = fmaxf(tmax, xor_shfl(tmax, 32));
    const float m_new = fmaxf(m_i, tmax);
    const float m_use = (m_new == -INFINITY) ? 0.f : m_new;  // row saw no key yet
    const float alpha = exp2_fast(m_i - m_use);
    m_i = m_new;
    float psum = 0.f;
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) {
        const float p = exp2_fast(s[mb][rr] - m_use);
        s[mb][rr] = p;
        psum += p;
      }
    l_i = l_i * alpha + psum;
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) o[md][rr] *= alpha;

    // O^T += V^T . P^T over four 16-key k-blocks. The instruction pairs A and B by
    // (lane half, element e); element e of half `half` stands for key
    // 16 kb2 + 8 (e >> 2) + 4 half + (e & 3), which is accumulator element
    // 8 (kb2 & 1) + e of S^T half-tile kb2 >> 1.
#pragma unroll
    for (int kb2 = 0; kb2 < TN / 16; ++kb2) {
      bf16x8 pb;
#pragma unroll
      for (int e = 0; e < 8; ++e) pb[e] = static_cast<__bf16>(s[kb2 >> 1][8 * (kb2 & 1) + e]);
      const int base = 16 * kb2 + 4 * half;
#pragma unroll
      for (int md = 0; md < 4; ++md) {
        const uint16_t* vrow = &sVt[(md * 32 + col) * VS + base];
        const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
        const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
        const bf16x8 av = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
        o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb, o[md], 0, 0, 0);
      }
    }
  }

  // Epilogue: O^T element rr of d-block md is d = 32 md + 8 (rr >> 2) + 4 half + (rr & 3).
  const float l_tot = l_i + xor_shfl(l_i, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;  // a row that saw no key is written as 0
  if (!row_valid) return;
  uint16_t* op = a.out + (int64_t)(q0 + tok) * a.out_row_stride + h * D + 4 * half;
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int grp = 0; grp < 4; ++grp) {
      uint2 w;
      w.x = pack_bf16x2(o[md][4 * grp] * inv, o[md][4 * grp + 1] * inv);
      w.y = pack_bf16x2(o[md][4 * grp + 2] * inv, o[md][4 * grp + 3] * inv);
      *reinterpret_cast<uint2*>(op + md * 32 + 8 * grp) = w;
    }
}

template <int G>
hipError_t launch_prefill_g(const AttnArgs& a, bool paged, bool causal, int max_seqlen_q,
                            hipStream_t stream) {
  constexpr int TM = 128 / G;
  const dim3 grid((unsigned)((max_seqlen_q + TM - 1) / TM), (unsigned)a.num_kv_heads,
                  (unsigned)a.num_seqs);
  const dim3 block(kPrefillThreads);
  if (paged) {
    if (causal)
      hipLaunchKernelGGL((prefill_kernel<G, true, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_kernel<G, true, false>), grid, block, 0, stream, a);
  } else {
    if (causal)
      hipLaunchKernelGGL((prefill_kernel<G, false, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((prefill_kernel<G, false, false>), grid, block, 0, stream, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill(const AttnArgs& a, int group, bool paged, bool causal, int max_seqlen_q,
                          hipStream_t stream) {
  if (a.num_seqs <= 0 || max_seqlen_q <= 1) return hipSuccess;
  switch (group) {
    case 1: return launch_prefill_g<1>(a, paged, causal, max_seqlen_q, stream);
    case 2: return launch_prefill_g<2>(a, paged, causal, max_seqlen_q, stream);
    case 4: return launch_prefill_g<4>(a, paged, causal, max_seqlen_q, stream);
    case 8: return launch_prefill_g<8>(a, paged, causal, max_seqlen_q, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pk
