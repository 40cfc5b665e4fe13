// Kernels around the attention path of the serving loop, for gfx950:
//   * add_rmsnorm       -- RMSNorm with the residual add fused (src/layers/layernorm.py:11-28)
//   * silu_and_mul      -- SiluAndMul (src/layers/activation.py:6-10)
//   * lm_head_greedy    -- logits = x W^T (src/layers/llm_head.py:60-64) followed by a greedy
//                          argmax, without writing the logits
//
// Rounding points follow the reference. The norms compute in fp32 and round the output
// (and the new residual) to bf16. SiluAndMul runs under torch.compile, which upcasts both
// halves, computes silu(x) * y in fp32 and rounds once. The LM head's logits are bf16 in
// the reference (F.linear on bf16 operands); the greedy choice here compares the fp32 dot
// products after rounding them to bf16 and keeps the lowest vocabulary index among equal
// maxima, which is what argmax over the bf16 logits returns.
#include "common.h"

namespace pk {
namespace {

__device__ __forceinline__ float round_to_bf16(float f) {
  return __uint_as_float((uint32_t)f32_to_bf16(f) << 16);
}

// ---------------------------------------------------------------- add + RMSNorm ---------

constexpr int kNormThreads = 128;

// One work-group per row; each thread owns 8 consecutive elements (hidden <= 8 * 128 * 4).
// out = bf16(w * (s * rsqrt(mean(s^2) + eps))) with s = x (+ residual) in fp32;
// residual_out = bf16(s) when a residual is given (layernorm.py:24-28), else untouched.
template <int kVecs>
__global__ __launch_bounds__(kNormThreads) void add_rmsnorm_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, const uint16_t* residual, int64_t res_stride,
    const uint16_t* __restrict__ weight, float eps, int32_t hidden, uint16_t* out, int64_t out_stride,
    uint16_t* residual_out, int64_t res_out_stride) {
  const int64_t row = blockIdx.x;
  // x, residual and weight loads all go out before any of them is used (one round of loads)
  uint4 xv[kVecs], rv[kVecs], wv[kVecs];
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
      xv[j] = *reinterpret_cast<const uint4*>(x + row * x_stride + col);
      rv[j] = residual != nullptr ? *reinterpret_cast<const uint4*>(residual + row * res_stride + col)
                                  : make_uint4(0, 0, 0, 0);
      wv[j] = *reinterpret_cast<const uint4*>(weight + col);
    }
  }
  float v[kVecs][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
      const uint32_t ww[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[j][2 * e] = bf16_lo(ww[e]);
        v[j][2 * e + 1] = bf16_hi(ww[e]);
      }
      if (residual != nullptr) {
        const uint32_t rr[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          v[j][2 * e] += bf16_lo(rr[e]);
          v[j][2 * e + 1] += bf16_hi(rr[e]);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);
    }
  }
  for (int m = kWave / 2; m >= 1; m >>= 1) ss += xor_shfl(ss, m);
  __shared__ float part[kNormThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kNormThreads / kWave; ++i) tot += part[i];
  const float rs = 1.0f / __builtin_sqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
      const uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
      uint32_t o[4], ro[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = pack_bf16x2(bf16_lo(ww[e]) * (v[j][2 * e] * rs), bf16_hi(ww[e]) * (v[j][2 * e + 1] * rs));
        ro[e] = pack_bf16x2(v[j][2 * e], v[j][2 * e + 1]);
      }
      *reinterpret_cast<uint4*>(out + row * out_stride + col) = make_uint4(o[0], o[1], o[2], o[3]);
      if (residual != nullptr && residual_out != nullptr)
        *reinterpret_cast<uint4*>(residual_out + row * res_out_stride + col) = make_uint4(ro[0], ro[1], ro[2], ro[3]);
    }
  }
}

// ---------------------------------------------------------------- SiLU * mul ------------

constexpr int kActThreads = 256;

// out[r, c] = bf16(silu(x[r, c]) * x[r, inter + c]) in fp32, c < inter; 8 columns per thread.
__global__ __launch_bounds__(kActThreads) void silu_and_mul_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, int32_t rows, int32_t inter,
    uint16_t* __restrict__ out, int64_t out_stride) {
  const int32_t vecs = inter / 8;
  const int64_t total = (int64_t)rows * vecs;
  for (int64_t i = (int64_t)blockIdx.x * kActThreads + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * kActThreads) {
    const int64_t r = i / vecs;
    const int32_t c = (int32_t)(i - r * vecs) * 8;
    const uint4 g = *reinterpret_cast<const uint4*>(x + r * x_stride + c);
    const uint4 u = *reinterpret_cast<const uint4*>(x + r * x_stride + inter + c);
    const uint32_t gg[4] = {g.x, g.y, g.z, g.w}, uu[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g0 = bf16_lo(gg[e]), g1 = bf16_hi(gg[e]);
      const float s0 = g0 / (1.0f + expf(-g0)), s1 = g1 / (1.0f + expf(-g1));
      o[e] = pack_bf16x2(s0 * bf16_lo(uu[e]), s1 * bf16_hi(uu[e]));
    }
    *reinterpret_cast<uint4*>(out + r * out_stride + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---------------------------------------------------------------- greedy LM head --------
//
// D = W_tile (vocab x K) . X^T (K x rows) on v_mfma_f32_32x32x16_bf16. A work-group owns 128
// vocabulary rows (32 per wavefront) and 32 * RT hidden rows; K is walked in chunks of 128.
// Each lane streams its vocabulary row from HBM with contiguous 16-byte loads: in k-step s of
// a chunk, MFMA k-slot (half h, element e) carries k = chunk + 64 h + 8 s + e. The B operand
// (the hidden rows, shared by every work-group and so L2-resident) is staged per chunk in LDS
// with the same k order, rows padded by 16 bytes so the 16-byte reads are conflict-free.
// The per-row best (bf16-rounded logit, lowest index on ties) is packed into one 64-bit key
// -- orderable logit bits above the complemented index -- and merged with a global atomic
// max; a finishing kernel turns keys into token ids.

constexpr int kLmThreads = 256;
constexpr int kLmVocabTile = 128;       // 4 wavefronts x 32 vocabulary rows
constexpr int kLmKChunk = 128;
constexpr int kLmLdsRow = kLmKChunk + 8;  // bf16 elements per staged row (16-byte pad)

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;

__device__ __forceinline__ uint64_t logit_key(float v, uint32_t idx) {
  const uint32_t b = __float_as_uint(v);
  const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
  return ((uint64_t)ord << 32) | (uint64_t)(~idx);
}

template <int RT>
__global__ __launch_bounds__(kLmThreads, 2) void lm_head_greedy_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ cu_rows,
    const uint16_t* __restrict__ w, int64_t w_stride, int32_t rows, int32_t vocab, int32_t k_dim,
    unsigned long long* __restrict__ keys) {
  constexpr int MT = 32 * RT;
  __shared__ __attribute__((aligned(16))) uint16_t xs[MT * kLmLdsRow];
  __shared__ unsigned long long best_s[4][MT];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane & 31, h = lane >> 5;
  const int m0 = blockIdx.y * MT;
  const int v_row = blockIdx.x * kLmVocabTile + wave * 32 + r;
  const uint16_t* wrow = w + (int64_t)(v_row < vocab ? v_row : vocab - 1) * w_stride + 64 * h;

  f32x16 acc[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.f;

  uint4 a_cur[8], a_nxt[8];
#pragma unroll
  for (int s = 0; s < 8; ++s) a_cur[s] = *reinterpret_cast<const uint4*>(wrow + 8 * s);

  for (int kc = 0; kc < k_dim; kc += kLmKChunk) {
    const bool more = kc + kLmKChunk < k_dim;
    if (more) {
#pragma unroll
      for (int s = 0; s < 8; ++s)
        a_nxt[s] = *reinterpret_cast<const uint4*>(wrow + kc + kLmKChunk + 8 * s);
    }
    // stage the chunk of the hidden rows: MT rows x 16 pieces of 16 bytes
    __syncthreads();  // the previous chunk's reads are done
#pragma unroll
    for (int p = threadIdx.x; p < MT * 16; p += kLmThreads) {
      const int row = p >> 4, piece = p & 15;
      const int m = m0 + row;
      uint4 val = make_uint4(0, 0, 0, 0);
      if (m < rows) {
        // last row of sequence m when selecting (llm_head.py:61-63); a padded sequence
        // (zeroed cu_seqlens tail) has no row and contributes zeros
        const int src = cu_rows != nullptr ? cu_rows[m + 1] - 1 : m;
        if (src >= 0)
          val = *reinterpret_cast<const uint4*>(x + (int64_t)src * x_stride + kc + piece * 8);
      }
      *reinterpret_cast<uint4*>(xs + row * kLmLdsRow + piece * 8) = val;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a_cur[s]);
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const uint4 bw = *reinterpret_cast<const uint4*>(xs + (32 * t + r) * kLmLdsRow + 64 * h + 8 * s);
        acc[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8_t, bw), acc[t], 0, 0, 0);
      }
    }
    if (more) {
#pragma unroll
      for (int s = 0; s < 8; ++s) a_cur[s] = a_nxt[s];
    }
  }

  // D layout: lane holds column (hidden row) 32 t + r and vocab rows 8 (i >> 2) + 4 h + (i & 3)
  const int v_base = blockIdx.x * kLmVocabTile + wave * 32;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    unsigned long long best = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int v = v_base + 8 * (i >> 2) + 4 * h + (i & 3);
      if (v < vocab) {
        const unsigned long long key = logit_key(round_to_bf16(acc[t][i]), (uint32_t)v);
        best = key > best ? key : best;
      }
    }
    const unsigned long long other = __shfl_xor(best, 32, kWave);
    best = other > best ? other : best;
    if (h == 0) best_s[wave][32 * t + r] = best;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < MT; j += kLmThreads) {
    unsigned long long b = best_s[0][j];
#pragma unroll
    for (int q = 1; q < 4; ++q) b = best_s[q][j] > b ? best_s[q][j] : b;
    if (m0 + j < rows) atomicMax(keys + m0 + j, b);
  }
}

// Resident variant for hidden <= kLmResidentMaxK: a persistent work-group (one per CU) keeps
// its group of up to 64 hidden rows in LDS for the whole call and walks vocabulary tiles,
// so the hidden rows cross from L2 once per work-group instead of once per tile. The
// `groups` work-groups that cover the row groups of one vocabulary sequence have linear
// ids l, l + 8, ... and so sit on one XCD: each weight tile comes from HBM once and is
// shared through that XCD's L2.
constexpr int kLmResidentMaxK = 1024;
constexpr int kLmResidentRows = 64;
constexpr int kLmResidentWaves = 8;
constexpr int kLmResidentThreads = kLmResidentWaves * 64;
constexpr int kLmResidentTile = kLmResidentWaves * 32;  // vocabulary rows per tile

template <int RT>
__global__ __launch_bounds__(kLmResidentThreads, 1) void lm_head_resident_kernel(
    const uint16_t* __restrict__ x, int64_t x_stride, const int32_t* __restrict__ cu_rows,
    const uint16_t* __restrict__ w, int64_t w_stride, int32_t rows, int32_t vocab, int32_t k_dim,
    int32_t groups, unsigned long long* __restrict__ keys) {
  constexpr int MT = 32 * RT;
  constexpr int kRowElems = kLmResidentMaxK + 8;  // staged row with a 16-byte pad
  __shared__ __attribute__((aligned(16))) uint16_t xs[MT * kRowElems];
  __shared__ unsigned long long best_s[kLmResidentWaves][MT];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane & 31, h = lane >> 5;
  const int j = blockIdx.x >> 3;
  const int rg = j % groups;                          // row group
  const int rank = (j / groups) * 8 + (blockIdx.x & 7);  // position in the vocabulary walk
  const int nrank = gridDim.x / groups;
  const int m0 = rg * MT;

  // stage the group's hidden rows (the last row of sequence m when selecting,
  // llm_head.py:61-63; padded sequences and rows past `rows` stage zeros)
  const int pieces = k_dim / 8;
  for (int p = threadIdx.x; p < MT * pieces; p += kLmResidentThreads) {
    const int row = p / pieces, piece = p - row * pieces;
    const int m = m0 + row;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (m < rows) {
      const int src = cu_rows != nullptr ? cu_rows[m + 1] - 1 : m;
      if (src >= 0) val = *reinterpret_cast<const uint4*>(x + (int64_t)src * x_stride + piece * 8);
    }
    *reinterpret_cast<uint4*>(xs + row * kRowElems + piece * 8) = val;
  }
  __syncthreads();

  unsigned long long best[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) best[t] = 0;
  // One stream of (tile, chunk) steps: the weight chunk of step n + 2 is in flight while
  // step n runs, across tile boundaries too.
  const int ntiles = (vocab + kLmResidentTile - 1) / kLmResidentTile;
  const int nchunks = k_dim / kLmKChunk;
  const int my_tiles = rank < ntiles ? (ntiles - rank + nrank - 1) / nrank : 0;
  const int steps = my_tiles * nchunks;
  auto wchunk = [&](int step) {
    const int t = step / nchunks;
    const int c = step - t * nchunks;
    const int v_row = (rank + t * nrank) * kLmResidentTile + wave * 32 + r;
    return w + (int64_t)(v_row < vocab ? v_row : vocab - 1) * w_stride + 64 * h + c * kLmKChunk;
  };
  f32x16 acc[RT];
  auto run_step = [&](const uint4 (&a)[8], int step) {
    const int t = step / nchunks;
    const int c = step - t * nchunks;
    if (c == 0) {
#pragma unroll
      for (int q = 0; q < RT; ++q)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[q][i] = 0.f;
    }
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) {
      const bf16x8_t av = __builtin_bit_cast(bf16x8_t, a[s8]);
#pragma unroll
      for (int q = 0; q < RT; ++q) {
        const uint4 bw = *reinterpret_cast<const uint4*>(xs + (32 * q + r) * kRowElems + c * kLmKChunk + 64 * h + 8 * s8);
        acc[q] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, __builtin_bit_cast(bf16x8_t, bw), acc[q], 0, 0, 0);
      }
    }
    if (c == nchunks - 1) {
      // D layout: lane holds column (hidden row) 32 q + r and vocab rows 8 (i >> 2) + 4 h + (i & 3)
      const int v_base = (rank + t * nrank) * kLmResidentTile + wave * 32;
#pragma unroll
      for (int q = 0; q < RT; ++q)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int v = v_base + 8 * (i >> 2) + 4 * h + (i & 3);
          if (v < vocab) {
            const unsigned long long key = logit_key(round_to_bf16(acc[q][i]), (uint32_t)v);
            best[q] = key > best[q] ? key : best[q];
          }
        }
    }
  };
  uint4 a0[8], a1[8];
  if (steps > 0) {
    const uint16_t* p0 = wchunk(0);
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) a0[s8] = *reinterpret_cast<const uint4*>(p0 + 8 * s8);
  }
  if (steps > 1) {
    const uint16_t* p1 = wchunk(1);
#pragma unroll
    for (int s8 = 0; s8 < 8; ++s8) a1[s8] = *reinterpret_cast<const uint4*>(p1 + 8 * s8);
  }
  for (int step = 0; step < steps; step += 2) {
    run_step(a0, step);
    if (step + 2 < steps) {
      const uint16_t* pn = wchunk(step + 2);
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) a0[s8] = *reinterpret_cast<const uint4*>(pn + 8 * s8);
    }
    if (step + 1 >= steps) break;
    run_step(a1, step + 1);
    if (step + 3 < steps) {
      const uint16_t* pn = wchunk(step + 3);
#pragma unroll
      for (int s8 = 0; s8 < 8; ++s8) a1[s8] = *reinterpret_cast<const uint4*>(pn + 8 * s8);
    }
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const unsigned long long other = __shfl_xor(best[t], 32, kWave);
    const unsigned long long b = other > best[t] ? other : best[t];
    if (h == 0) best_s[wave][32 * t + r] = b;
  }
  __syncthreads();
  for (int q = threadIdx.x; q < MT; q += kLmResidentThreads) {
    unsigned long long b = best_s[0][q];
#pragma unroll
    for (int wv = 1; wv < kLmResidentWaves; ++wv) b = best_s[wv][q] > b ? best_s[wv][q] : b;
    if (m0 + q < rows) atomicMax(keys + m0 + q, b);
  }
}

__global__ void lm_keys_clear_kernel(unsigned long long* keys, int32_t rows) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows) keys[i] = 0ull;
}

__global__ void lm_keys_to_ids_kernel(const unsigned long long* keys, int32_t rows, int32_t* ids) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < rows) ids[i] = (int32_t)(~(uint32_t)(keys[i] & 0xffffffffull));
}

}  // namespace

hipError_t launch_add_rmsnorm(const void* x, int64_t x_stride, const void* residual,
                              int64_t res_stride, const void* weight, float eps, int32_t rows,
                              int32_t hidden, void* out, int64_t out_stride, void* residual_out,
                              int64_t res_out_stride, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int vecs = (hidden / 8 + kNormThreads - 1) / kNormThreads;
  auto* xp = static_cast<const uint16_t*>(x);
  auto* rp = static_cast<const uint16_t*>(residual);
  auto* wp = static_cast<const uint16_t*>(weight);
  auto* op = static_cast<uint16_t*>(out);
  auto* rop = static_cast<uint16_t*>(residual_out);
  switch (vecs) {
    case 1: hipLaunchKernelGGL(add_rmsnorm_kernel<1>, dim3(rows), dim3(kNormThreads), 0, stream, xp, x_stride, rp, res_stride, wp, eps, hidden, op, out_stride, rop, res_out_stride); break;
    case 2: hipLaunchKernelGGL(add_rmsnorm_kernel<2>, dim3(rows), dim3(kNormThreads), 0, stream, xp, x_stride, rp, res_stride, wp, eps, hidden, op, out_stride, rop, res_out_stride); break;
    case 3: hipLaunchKernelGGL(add_rmsnorm_kernel<3>, dim3(rows), dim3(kNormThreads), 0, stream, xp, x_stride, rp, res_stride, wp, eps, hidden, op, out_stride, rop, res_out_stride); break;
    case 4: hipLaunchKernelGGL(add_rmsnorm_kernel<4>, dim3(rows), dim3(kNormThreads), 0, stream, xp, x_stride, rp, res_stride, wp, eps, hidden, op, out_stride, rop, res_out_stride); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_silu_and_mul(const void* x, int64_t x_stride, int32_t rows, int32_t inter,
                               void* out, int64_t out_stride, hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const int64_t total = (int64_t)rows * (inter / 8);
  int64_t blocks = (total + kActThreads - 1) / kActThreads;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(silu_and_mul_kernel, dim3((unsigned)blocks), dim3(kActThreads), 0, stream,
                     static_cast<const uint16_t*>(x), x_stride, rows, inter,
                     static_cast<uint16_t*>(out), out_stride);
  return hipGetLastError();
}

hipError_t launch_lm_head_greedy(const void* x, int64_t x_stride, const int32_t* cu_rows,
                                 const void* w, int64_t w_stride, int32_t rows, int32_t vocab,
                                 int32_t k_dim, unsigned long long* keys, int32_t* ids,
                                 hipStream_t stream) {
  if (rows <= 0) return hipSuccess;
  const unsigned small = (unsigned)((rows + 255) / 256);
  hipLaunchKernelGGL(lm_keys_clear_kernel, dim3(small), dim3(256), 0, stream, keys, rows);
  const unsigned vt = (unsigned)((vocab + kLmVocabTile - 1) / kLmVocabTile);
  auto* xp = static_cast<const uint16_t*>(x);
  auto* wp = static_cast<const uint16_t*>(w);
  if (k_dim <= kLmResidentMaxK) {
    static int cus_cached = 0;
    if (cus_cached == 0) {
      int dev = 0, cus = 0;
      if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
        cus = 256;
      cus_cached = cus;
    }
    const int groups = (rows + kLmResidentRows - 1) / kLmResidentRows;
    const int per = 8 * groups;                      // one XCD round of every row group
    int grid = (cus_cached / per) * per;
    if (grid == 0) grid = per;
    if (rows <= 32)
      hipLaunchKernelGGL(lm_head_resident_kernel<1>, dim3(grid), dim3(kLmResidentThreads), 0, stream, xp, x_stride, cu_rows, wp, w_stride, rows, vocab, k_dim, groups, keys);
    else
      hipLaunchKernelGGL(lm_head_resident_kernel<2>, dim3(grid), dim3(kLmResidentThreads), 0, stream, xp, x_stride, cu_rows, wp, w_stride, rows, vocab, k_dim, groups, keys);
  } else if (rows <= 32) {
    hipLaunchKernelGGL(lm_head_greedy_kernel<1>, dim3(vt, 1), dim3(kLmThreads), 0, stream, xp, x_stride, cu_rows, wp, w_stride, rows, vocab, k_dim, keys);
  } else if (rows <= 64) {
    hipLaunchKernelGGL(lm_head_greedy_kernel<2>, dim3(vt, 1), dim3(kLmThreads), 0, stream, xp, x_stride, cu_rows, wp, w_stride, rows, vocab, k_dim, keys);
  } else {
    hipLaunchKernelGGL(lm_head_greedy_kernel<4>, dim3(vt, (unsigned)((rows + 127) / 128)), dim3(kLmThreads), 0, stream, xp, x_stride, cu_rows, wp, w_stride, rows, vocab, k_dim, keys);
  }
  hipError_t err = hipGetLastError();
  if (err != hipSuccess) return err;
  hipLaunchKernelGGL(lm_keys_to_ids_kernel, dim3(small), dim3(256), 0, stream, keys, rows, ids);
  return hipGetLastError();
}

}  // namespace pk
