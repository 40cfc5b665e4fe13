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
// Per tile of TN = 32 keys (per wavefront):
//   S^T (32 keys x 32 rows)  = K (32 x 128) . Q^T (128 x 32)   8 v_mfma_f32_32x32x16_bf16
//   online softmax down each column (a lane owns one query row: 16 scores in registers,
//   one xor-32 exchange for the column max)
//   O^T (128 x 32)          += V^T (128 x 32) . P^T (32 x 32)  4 x 2 v_mfma_f32_32x32x16_bf16
// K is staged row-major in LDS; V is staged transposed (d-major) so that the MFMA A
// operand (8 keys of one d) is two 8-byte LDS reads. P^T never leaves registers: the
// S^T accumulator layout already holds, per lane, the keys the P.V B operand needs
// once the k-order of the instruction is permuted (same permutation on the V^T side).
#include "common.h"

namespace pk {
namespace {

constexpr int kTileKeys = 64;        // keys per K/V tile
constexpr int kPrefillThreads = 256;  // four wavefronts
constexpr int kRowBytes = kHeadDim * 2;                  // one head's row of a K or V tile (256 B)
constexpr int kTileBytes = kTileKeys * kRowBytes;        // 16 KiB per operand per buffer

#ifndef PK_PREFILL_WAVES_PER_SIMD
#define PK_PREFILL_WAVES_PER_SIMD 2  // register budget: 512 / this per lane (VGPR + AGPR)
#endif

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// LDS tiles are stored unpadded, one 256-byte row per key, with the row's sixteen 16-byte
// chunks XOR-swizzled so that the MFMA operand reads hit distinct banks:
//   K: chunk c of row r lives in slot c ^ (r & 15)      (32 consecutive rows read chunk c)
//   V: chunk c of row r lives in slot c ^ ((2 r) & 15)  (4 consecutive rows x 2 chunks read)
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((2 * r) & 15); }

// Global -> LDS for keys [t0, t0 + 64) of kv head g straight into `kdst` / `vdst` with
// global_load_lds_dwordx4: wavefront w moves rows 16 w .. 16 w + 15, four rows (1 KiB) per
// instruction, lane l writing slot (l & 15) of row (l >> 4) and therefore reading the
// swizzled source chunk. No registers hold tile data. Keys past Lk re-read the last key's
// row (same cache block, finite data); their scores are masked and their p is 0.
template <bool PAGED>
__device__ __forceinline__ void load_tile_lds(const AttnArgs& a, int b, int k0, int Lk, int g, int bt_lane, int wave,
                                              int lane, int t0, lds_char* kdst, lds_char* vdst) {
  const uint16_t* kbase;
  const uint16_t* vbase;
  if constexpr (PAGED) {
    const int j = t0 / a.block_size;  // block_size % 64 == 0: the tile sits inside one block
    const int blk = j < kWave ? __builtin_amdgcn_readlane(bt_lane, j)
                              : a.block_table[(int64_t)b * a.bt_stride + j];
    const int off = t0 % a.block_size;
    kbase = a.k + (int64_t)blk * a.k_block_stride + (int64_t)off * a.k_row_stride;
    vbase = a.v + (int64_t)blk * a.v_block_stride + (int64_t)off * a.v_row_stride;
  } else {
    kbase = a.k + (int64_t)(k0 + t0) * a.k_row_stride;
    vbase = a.v + (int64_t)(k0 + t0) * a.v_row_stride;
  }
  kbase += g * kHeadDim;
  vbase += g * kHeadDim;
  const int last = Lk - 1 - t0;
  const int slot = lane & 15;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = 16 * wave + 4 * i + (lane >> 4);  // tile row this lane fills
    const int rs = min(r, last);                    // source row
    const uint16_t* ksrc = kbase + (int64_t)rs * a.k_row_stride + (slot ^ (r & 15)) * 8;
    const uint16_t* vsrc = vbase + (int64_t)rs * a.v_row_stride + (slot ^ ((2 * r) & 15)) * 8;
    __builtin_amdgcn_global_load_lds(ksrc, kdst + (16 * wave + 4 * i) * kRowBytes, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(vsrc, vdst + (16 * wave + 4 * i) * kRowBytes, 16, 0, 0);
  }
}

// One key tile for this wavefront's 32 query rows:
//   S^T = K Q^T, online softmax down the columns, O^T += V^T P^T.
// full: no key of the tile is masked for any row of the wavefront (wave-uniform).
__device__ __forceinline__ void compute_tile(const lds_char* sK, const lds_char* sV, const bf16x8 (&qb)[kHeadDim / 16],
                                             f32x16 (&o)[4], float& m_i, float& l_i, int t0, int lim, bool full,
                                             float scale_log2, int lane) {
  const int col = lane & 31;
  const int half = lane >> 5;
  // S^T accumulator element rr of half-tile mb is key t0 + 32 mb + 8 (rr >> 2) + 4 half + (rr & 3).
  // A operand: lane (col, half) needs chunk 2 kb + half of K row 32 mb + col.
  f32x16 s[2];
#pragma unroll
  for (int mb = 0; mb < 2; ++mb) {
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) s[mb][rr] = 0.f;
    const int r = mb * 32 + col;
#pragma unroll
    for (int kb = 0; kb < kHeadDim / 16; ++kb) {
      const bf16x8 av = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(
          sK + r * kRowBytes + k_slot(r, 2 * kb + half) * 16);
      s[mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, qb[kb], s[mb], 0, 0, 0);
    }
  }
  float tmax = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < 2; ++mb)
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      float v = s[mb][rr] * scale_log2;
      if (!full && t0 + mb * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3) > lim) v = -INFINITY;
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
  // rescale the numerator only when some row of the wavefront raised its max (rare once
  // the running max has settled)
  if (__builtin_amdgcn_ballot_w64(alpha != 1.f) != 0) {
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) o[md][rr] *= alpha;
  }
  // O^T += V^T . P^T over 16-key k-blocks. The instruction pairs A and B by (lane half,
  // element e); element e of half `half` stands for key 16 kb2 + 8 (e >> 2) + 4 half +
  // (e & 3), which is accumulator element 8 (kb2 & 1) + e of S^T half-tile kb2 >> 1.
  // The A operand (4 consecutive keys of one head_dim element, twice) comes from the
  // row-major V tile through the LDS transpose read: in each 16-lane group, source lane
  // s addresses 4 elements of key row key0 + (s >> 2) at head_dim d0 + 4 (s & 3), and
  // lane i receives element d0 + i of keys key0 .. key0 + 3.
  const int grp = lane >> 4;
  const int src = lane & 15;
#pragma unroll
  for (int kb2 = 0; kb2 < 4; ++kb2) {
    bf16x8 pb;
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[e] = static_cast<__bf16>(s[kb2 >> 1][8 * (kb2 & 1) + e]);
#pragma unroll
    for (int md = 0; md < 4; ++md) {
      const int d = md * 32 + 16 * (grp & 1) + 4 * (src & 3);
      const int r_lo = 16 * kb2 + 4 * half + (src >> 2);
      const int r_hi = r_lo + 8;
      const lds_v4i16* p_lo = reinterpret_cast<const lds_v4i16*>(sV + r_lo * kRowBytes + v_slot(r_lo, d >> 3) * 16 + (d & 7) * 2);
      const lds_v4i16* p_hi = reinterpret_cast<const lds_v4i16*>(sV + r_hi * kRowBytes + v_slot(r_hi, d >> 3) * 16 + (d & 7) * 2);
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_v4i16*>(p_lo));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_v4i16*>(p_hi));
      const bf16x8 av = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      o[md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb, o[md], 0, 0, 0);
    }
  }
}

template <int G, bool PAGED, bool CAUSAL>
__global__ __launch_bounds__(kPrefillThreads, PK_PREFILL_WAVES_PER_SIMD) void prefill_kernel(const AttnArgs a) {
  constexpr int D = kHeadDim;
  constexpr int TN = kTileKeys;
  constexpr int TM = 128 / G;  // query tokens per work-group
  // two buffers per operand, as distinct objects so the compiler can tell the tile being
  // filled by the DMA apart from the tile being read
  __shared__ __attribute__((aligned(1024))) char sK0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV0[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sK1[kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV1[kTileBytes];
  lds_char* const K0 = (lds_char*)sK0;  // address-space cast to LDS
  lds_char* const V0 = (lds_char*)sV0;
  lds_char* const K1 = (lds_char*)sK1;
  lds_char* const V1 = (lds_char*)sV1;

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
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
  // the wavefront's rows are tokens [w_lo, w_lo + min(32, TM)) of one or two heads
  const int w_lo = tok_begin + (wave * 32) % TM;
  const int w_hi = w_lo + (TM < 32 ? TM : 32) - 1;
  const int lim_lo = CAUSAL ? min(Lk - 1, w_lo + P) : Lk - 1;  // keys <= lim_lo: seen by all rows
  const int lim_hi = CAUSAL ? min(Lk - 1, w_hi + P) : Lk - 1;  // keys >  lim_hi: seen by none

  // Q^T B operand: k-block kb covers d in [16 kb, 16 kb + 16); lane holds 8 of them.
  // Rows past Lq read the last row (finite) and are never stored.
  bf16x8 qb[D / 16];
  {
    const uint16_t* qp = a.q + (int64_t)(q0 + min(tok, Lq - 1)) * a.q_row_stride + h * D + 8 * half;
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb) qb[kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp + kb * 16));
  }
  // The sequence's first 64 block-table entries sit one per lane in a register, so a tile's
  // block id is a readlane instead of a dependent global load.
  int bt_lane = 0;
  if constexpr (PAGED) {
    const int nblk = (Lk + a.block_size - 1) / a.block_size;
    if (lane < nblk) bt_lane = a.block_table[(int64_t)b * a.bt_stride + lane];
  }

  f32x16 o[4];
#pragma unroll
  for (int md = 0; md < 4; ++md)
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) o[md][rr] = 0.f;
  float m_i = -INFINITY;
  float l_i = 0.f;

  // Pipeline (one barrier per tile): after the barrier, tile n is complete in LDS and no
  // wavefront still reads the other buffer, so tile n+1 is sent there by DMA while tile n
  // is computed; the wavefront then waits for its own DMA, and the next barrier publishes
  // it. Tiles entirely above a wavefront's causal limit are skipped by that wavefront.
  const int ntiles = (kv_end + TN - 1) / TN;
  if (ntiles > 0) load_tile_lds<PAGED>(a, b, k0, Lk, g, bt_lane, wave, lane, 0, K0, V0);
  __builtin_amdgcn_s_waitcnt(0);  // Q operand, block table and tile 0 have landed
  __syncthreads();
  for (int n = 0; n < ntiles; n += 2) {
    const int t0 = n * TN;
    if (n + 1 < ntiles) load_tile_lds<PAGED>(a, b, k0, Lk, g, bt_lane, wave, lane, t0 + TN, K1, V1);
    if (t0 <= lim_hi) compute_tile(K0, V0, qb, o, m_i, l_i, t0, lim, t0 + TN - 1 <= lim_lo, a.scale_log2, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (n + 1 >= ntiles) break;
    const int t1 = t0 + TN;
    if (n + 2 < ntiles) load_tile_lds<PAGED>(a, b, k0, Lk, g, bt_lane, wave, lane, t1 + TN, K0, V0);
    if (t1 <= lim_hi) compute_tile(K1, V1, qb, o, m_i, l_i, t1, lim, t1 + TN - 1 <= lim_lo, a.scale_log2, lane);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
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
