// Linear layers of the serving loop's decode steps (at most 128 token rows) on gfx950,
// with the operations that follow them fused where the data allows:
//   * linear           -- y = bf16(x W^T): F.linear of ColumnParallelLinear / RowParallelLinear
//                         (src/layers/linear.py:74-75, :169-170) as qkv_proj (qwen3.py:80)
//   * linear_silu_mul  -- y = bf16(silu(g) * u), g, u = bf16(x Wg^T), bf16(x Wu^T): the merged
//                         gate/up projection and SiluAndMul (qwen3.py:120-121, activation.py:6-10)
//   * linear_add_rmsnorm -- h = bf16(x W^T); s = h + residual (fp32);
//                         out = bf16(w * s * rsqrt(mean(s^2) + eps)), residual_out = bf16(s):
//                         o_proj / down_proj (qwen3.py:90, :122) and the RMSNorm after them
//                         (qwen3.py:165, :167; layernorm.py:18-28)
// Rounding points are the reference's: the linear output is bf16 before anything uses it.
//
// At these row counts the work is reading the weight once: 4-12 MB per projection for
// Qwen3-0.6B against at most 0.8 MB of x. The weight is cut into 32-row tiles (one MFMA
// tile; 32 gate + 32 up rows for SiLU * mul) and the token rows into 32-row tiles; a
// work-group owns one weight tile, MT row tiles and a K range. Row groups of one weight
// tile are consecutive multiples of the tile count apart in the grid, so they run on one
// XCD and read the weight tile from HBM once, through that XCD's L2. The K range is split
// (KS > 1) only when the (weight tile x row group) grid is too small to keep the CUs
// streaming. A work-group's four wavefronts take interleaved 64-wide K blocks of its range,
// issue the loads of up to four blocks before the first MFMA, and add their accumulators
// through LDS. With KS = 1 the epilogue runs in the work-group; otherwise fp32 partial sums
// go to the workspace and a second kernel adds them and applies it (the residual-add +
// RMSNorm epilogue needs whole rows and always takes that path).
//
// MFMA: v_mfma_f32_32x32x16_bf16 with D = W_tile (32 x 16) . x^T (16 x 32 rows). In K
// block kb, step q, lane (r, h) supplies weight row r and x row c = r at K positions
// kb + 32 h + 8 q + e (e < 8), so each lane reads 64 contiguous bytes of a row per block
// and A and B agree on the (permuted) k order. D element i of lane (c, h) of x-row tile t
// is y[32 t + c][n0 + 8 (i >> 2) + 4 h + (i & 3)].
#include "common.h"

namespace pk {
namespace {

constexpr int kLinThreads = 256;   // four wavefronts
constexpr int kLinTile = 32;       // weight rows (output columns) per tile
constexpr int kLinKBlock = 64;     // K elements per wavefront block (4 MFMA steps)
constexpr int kLinChunk = 4 * kLinKBlock;  // K elements per LDS stage (one block per wavefront)
#ifndef PK_LINEAR_TARGET_GROUPS
#define PK_LINEAR_TARGET_GROUPS 256
#endif
#ifndef PK_LINEAR_MIN_GROUPS
#define PK_LINEAR_MIN_GROUPS 64
#endif
#ifndef PK_LINEAR_MT2_ROWS
#define PK_LINEAR_MT2_ROWS 64
#endif
constexpr int kLinTargetGroups = PK_LINEAR_TARGET_GROUPS;  // work-groups a split launch aims for
constexpr int kLinMinGroups = PK_LINEAR_MIN_GROUPS;        // smallest grid left unsplit
constexpr int kLinMaxChunks = 4;                           // longest unsplit K walk (chunks)
constexpr int kLinMt2Rows = PK_LINEAR_MT2_ROWS;            // more rows: two row tiles per group

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;
// 16-byte register value for the staged loads (a native vector: HIP's uint4 struct is
// copied through private memory by the staging loops)
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float silu_mul(float g, float u) {
  const float gb = bf16_lo(pack_bf16x2(g, 0.f));  // g and u rounded to bf16 (the GEMM output)
  const float ub = bf16_lo(pack_bf16x2(u, 0.f));
  return gb / (1.0f + expf(-gb)) * ub;
}

enum Epi { kEpiStore = 0, kEpiSiluMul = 1, kEpiPartial = 2 };

struct LinArgs {
  const uint16_t* x;
  int64_t x_stride;
  const uint16_t* w;
  int64_t w_stride;
  int32_t rows;
  int32_t n_out;     // output columns (inter for SiLU * mul)
  int32_t k;
  int32_t ks;        // K splits
  uint16_t* y;       // bf16 output (store / SiLU epilogue)
  int64_t y_stride;
  float* part;       // [ks][rows][np * n_out] fp32 partial sums
};

// Waits for this wavefront's LDS operations, then for every wavefront of the work-group.
// s_waitcnt lgkmcnt(0) on its own: __syncthreads() would also wait for vmcnt(0), i.e. for
// the global loads of later K chunks that are still in flight.
__device__ __forceinline__ void lin_lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0) only
  asm volatile("s_barrier" ::: "memory");
}

// NP = weight tiles per work-group (2: gate rows n0.., up rows n_out + n0..); MT = 32-row x
// tiles per work-group; NB = 256-wide K chunks whose global loads are issued together.
//
// Loads: a 32-row x 256-column operand tile (16 KB) is read by the 256 threads as four
// instructions of 8 rows x 512 contiguous bytes (thread t: row 8 i + t / 32, 16-byte
// column t % 32), so every 4-lane quad reads 64 bytes of one row. (Loading the MFMA layout
// straight from memory puts 32 different rows in one instruction and 4 in every quad,
// which costs four L1 tag lookups per quad.) The tile goes to LDS with 16-byte column c of
// row r at r * 512 + ((c ^ r) & 31) * 16, so the stores and the MFMA operand reads
// (16 lanes = 16 rows of one column) are free of bank conflicts. Two LDS stages: chunk c
// is stored in stage c & 1 while the other stage may still be read for chunk c - 1.
// Wavefront w multiplies the 64 columns [64 w, 64 w + 64) of every chunk.
template <int NP, int MT, int NB, int EPI>
__global__ __launch_bounds__(kLinThreads) void linear_kernel(const LinArgs a) {
  constexpr int kOps = NP + MT;               // operand tiles per chunk
  constexpr int kTileBytes = 32 * kLinChunk * 2;
  constexpr int kStage = kOps * kTileBytes;
  constexpr int kRedBytes = 4 * NP * 4 * kWave * 16;
  constexpr int kSmem = 2 * kStage > kRedBytes ? 2 * kStage : kRedBytes;
  __shared__ __attribute__((aligned(16))) char smem[kSmem];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane & 31, h = lane >> 5;
  const int ntiles = a.n_out / kLinTile;
  const int per_group = ntiles * a.ks;  // work-groups of one row group
  const int mgroup = blockIdx.x / per_group;
  const int rem = blockIdx.x - mgroup * per_group;
  const int split = rem / ntiles;
  const int n0 = (rem - split * ntiles) * kLinTile;
  const int row0 = mgroup * MT * 32;
  const int kc = a.k / a.ks;
  const int kbeg = split * kc;

  // loader: thread row lr (+ 8 i), 16-byte column lc
  const int lr = threadIdx.x >> 5, lc = threadIdx.x & 31;
  const uint16_t* src[kOps][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
      src[p][i] = a.w + (int64_t)(p * a.n_out + n0 + 8 * i + lr) * a.w_stride + kbeg + 8 * lc;
#pragma unroll
    for (int t = 0; t < MT; ++t)
      src[NP + t][i] =
          a.x + (int64_t)min(row0 + 32 * t + 8 * i + lr, a.rows - 1) * a.x_stride + kbeg + 8 * lc;
  }
  int wofs[4], rofs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 8 * i + lr;
    wofs[i] = row * (2 * kLinChunk) + ((lc ^ row) & 31) * 16;
    const int cc = 8 * wave + 4 * h + i;  // MFMA step i reads 16-byte column cc of row r
    rofs[i] = r * (2 * kLinChunk) + ((cc ^ r) & 31) * 16;
  }

  f32x16 acc[NP][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[p][t][i] = 0.f;

  const int nch = kc / kLinChunk;
  for (int j0 = 0; j0 < nch; j0 += NB) {
    u32x4_t st[NB][kOps][4];
#pragma unroll
    for (int j = 0; j < NB; ++j)
#pragma unroll
      for (int o = 0; o < kOps; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          st[j][o][i] = *reinterpret_cast<const u32x4_t*>(src[o][i] + (j0 + j) * kLinChunk);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      char* stage = smem + ((j0 + j) & 1) * kStage;
#pragma unroll
      for (int o = 0; o < kOps; ++o)
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4_t*>(stage + o * kTileBytes + wofs[i]) = st[j][o][i];
      lin_lds_barrier();
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        u32x4_t xv[MT];
#pragma unroll
        for (int t = 0; t < MT; ++t) xv[t] = *reinterpret_cast<const u32x4_t*>(stage + (NP + t) * kTileBytes + rofs[q]);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(stage + p * kTileBytes + rofs[q]);
#pragma unroll
          for (int t = 0; t < MT; ++t)
            acc[p][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, wv),
                                                                __builtin_bit_cast(bf16x8_t, xv[t]),
                                                                acc[p][t], 0, 0, 0);
        }
      }
    }
  }
  __syncthreads();  // every wavefront is done with the stages before they hold the sums
  auto red = reinterpret_cast<float4 (*)[NP][4][kWave]>(smem);

  // Add the four wavefronts' accumulators one x-row tile at a time. Thread (c, q) then owns
  // x row 32 t + c and the 4 output columns n0 + 4 q .. + 3: D elements 4 (q >> 1) .. + 3 of
  // lane c + 32 (q & 1), stored as one float4 per lane and element quad.
  const int c = threadIdx.x >> 3, q = threadIdx.x & 7;
  const int n = n0 + 4 * q;
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    if (t) __syncthreads();
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        red[wave][p][j][lane] = make_float4(acc[p][t][4 * j], acc[p][t][4 * j + 1], acc[p][t][4 * j + 2],
                                            acc[p][t][4 * j + 3]);
    __syncthreads();
    const int m = row0 + 32 * t + c;
    float4 v[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float4 a0 = red[0][p][q >> 1][c + 32 * (q & 1)], a1 = red[1][p][q >> 1][c + 32 * (q & 1)];
      const float4 a2 = red[2][p][q >> 1][c + 32 * (q & 1)], a3 = red[3][p][q >> 1][c + 32 * (q & 1)];
      v[p] = make_float4(a0.x + a1.x + a2.x + a3.x, a0.y + a1.y + a2.y + a3.y, a0.z + a1.z + a2.z + a3.z,
                         a0.w + a1.w + a2.w + a3.w);
    }
    if (m < a.rows) {
      if constexpr (EPI == kEpiStore) {
        *reinterpret_cast<uint2*>(a.y + (int64_t)m * a.y_stride + n) =
            make_uint2(pack_bf16x2(v[0].x, v[0].y), pack_bf16x2(v[0].z, v[0].w));
      } else if constexpr (EPI == kEpiSiluMul) {
        *reinterpret_cast<uint2*>(a.y + (int64_t)m * a.y_stride + n) =
            make_uint2(pack_bf16x2(silu_mul(v[0].x, v[NP - 1].x), silu_mul(v[0].y, v[NP - 1].y)),
                       pack_bf16x2(silu_mul(v[0].z, v[NP - 1].z), silu_mul(v[0].w, v[NP - 1].w)));
      } else {
        float* pp = a.part + ((int64_t)split * a.rows + m) * (NP * a.n_out) + n;
#pragma unroll
        for (int p = 0; p < NP; ++p) *reinterpret_cast<float4*>(pp + p * a.n_out) = v[p];
      }
    }
  }
}

// Sum of the KS partials, then the store or SiLU * mul epilogue; 8 output columns per thread.
template <int NP>
__global__ __launch_bounds__(256) void linear_reduce_kernel(const LinArgs a) {
  const int cols8 = a.n_out / 8;
  const int64_t total = (int64_t)a.rows * cols8;
  const int64_t row_w = (int64_t)NP * a.n_out;
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < total; e += (int64_t)gridDim.x * blockDim.x) {
    const int m = (int)(e / cols8);
    const int c = (int)(e - (int64_t)m * cols8) * 8;
    float v[NP][8];
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int j = 0; j < 8; ++j) v[p][j] = 0.f;
    for (int s = 0; s < a.ks; ++s) {
      const float* pp = a.part + ((int64_t)s * a.rows + m) * row_w + c;
#pragma unroll
      for (int p = 0; p < NP; ++p) {
        const float4 lo = *reinterpret_cast<const float4*>(pp + p * a.n_out);
        const float4 hi = *reinterpret_cast<const float4*>(pp + p * a.n_out + 4);
        v[p][0] += lo.x; v[p][1] += lo.y; v[p][2] += lo.z; v[p][3] += lo.w;
        v[p][4] += hi.x; v[p][5] += hi.y; v[p][6] += hi.z; v[p][7] += hi.w;
      }
    }
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (NP == 1)
        o[j] = pack_bf16x2(v[0][2 * j], v[0][2 * j + 1]);
      else
        o[j] = pack_bf16x2(silu_mul(v[0][2 * j], v[1][2 * j]), silu_mul(v[0][2 * j + 1], v[1][2 * j + 1]));
    }
    *reinterpret_cast<uint4*>(a.y + (int64_t)m * a.y_stride + c) = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// Sum of the KS partials rounded to bf16 (the linear output), then the residual add and
// RMSNorm of layernorm.py:18-28. One 128-thread work-group per row, 8 columns per thread.
constexpr int kLinNormThreads = 128;

template <int kVecs>
__global__ __launch_bounds__(kLinNormThreads) void linear_add_rmsnorm_kernel(
    const LinArgs a, const uint16_t* residual, int64_t res_stride, const uint16_t* __restrict__ weight,
    float eps, uint16_t* out, int64_t out_stride, uint16_t* residual_out, int64_t res_out_stride) {
  const int64_t row = blockIdx.x;
  const int hidden = a.n_out;
  // The residual and weight rows do not depend on the partial sums: their loads go out
  // first, and the partials of kNormBatch splits at a time after them, so the kernel waits
  // for one round of loads per batch instead of one per split plus two more. The splits are
  // still added in order 0, 1, 2, ... (the fp32 sum is unchanged).
  constexpr int kNormBatch = 8;
  uint4 rv[kVecs], wv[kVecs];
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kLinNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
      rv[j] = *reinterpret_cast<const uint4*>(residual + row * res_stride + col);
      wv[j] = *reinterpret_cast<const uint4*>(weight + col);
    }
  }
  float v[kVecs][8];
#pragma unroll
  for (int j = 0; j < kVecs; ++j)
#pragma unroll
    for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
  for (int s0 = 0; s0 < a.ks; s0 += kNormBatch) {
    float4 lo[kNormBatch][kVecs], hi[kNormBatch][kVecs];
#pragma unroll
    for (int u = 0; u < kNormBatch; ++u) {
      const int s = min(s0 + u, a.ks - 1);  // past the last split: re-read it, not added
#pragma unroll
      for (int j = 0; j < kVecs; ++j) {
        const int col = (j * kLinNormThreads + threadIdx.x) * 8;
        if (col < hidden) {
          const float* pp = a.part + ((int64_t)s * a.rows + row) * hidden + col;
          lo[u][j] = *reinterpret_cast<const float4*>(pp);
          hi[u][j] = *reinterpret_cast<const float4*>(pp + 4);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < kNormBatch; ++u) {
      if (s0 + u >= a.ks) break;
#pragma unroll
      for (int j = 0; j < kVecs; ++j) {
        v[j][0] += lo[u][j].x; v[j][1] += lo[u][j].y; v[j][2] += lo[u][j].z; v[j][3] += lo[u][j].w;
        v[j][4] += hi[u][j].x; v[j][5] += hi[u][j].y; v[j][6] += hi[u][j].z; v[j][7] += hi[u][j].w;
      }
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kLinNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
      const uint32_t rr[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // the linear output is bf16 before the residual add
        const uint32_t hb = pack_bf16x2(v[j][2 * e], v[j][2 * e + 1]);
        v[j][2 * e] = bf16_lo(hb) + bf16_lo(rr[e]);
        v[j][2 * e + 1] = bf16_hi(hb) + bf16_hi(rr[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = fmaf(v[j][e], v[j][e], ss);
    }
  }
  for (int m = kWave / 2; m >= 1; m >>= 1) ss += xor_shfl(ss, m);
  __shared__ float part[kLinNormThreads / kWave];
  if ((threadIdx.x & (kWave - 1)) == 0) part[threadIdx.x / kWave] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int i = 0; i < kLinNormThreads / kWave; ++i) tot += part[i];
  const float rs = 1.0f / __builtin_sqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kLinNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
      const uint32_t ww[4] = {wv[j].x, wv[j].y, wv[j].z, wv[j].w};
      uint32_t o[4], ro[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = pack_bf16x2(bf16_lo(ww[e]) * (v[j][2 * e] * rs), bf16_hi(ww[e]) * (v[j][2 * e + 1] * rs));
        ro[e] = pack_bf16x2(v[j][2 * e], v[j][2 * e + 1]);
      }
      *reinterpret_cast<uint4*>(out + row * out_stride + col) = make_uint4(o[0], o[1], o[2], o[3]);
      *reinterpret_cast<uint4*>(residual_out + row * res_out_stride + col) = make_uint4(ro[0], ro[1], ro[2], ro[3]);
    }
  }
}

// Launch shape: MT row tiles per work-group, row groups, K splits, blocks per load batch.
struct LinCfg {
  int mt, mgroups, ks, nb;
};

// K is left unsplit when the grid of (weight tile x 32-row tile) work-groups has at least
// kLinMinGroups entries and a work-group then walks at most kLinMaxChunks 256-wide
// chunks; otherwise KS is the smallest divisor of K / 256 whose grid reaches
// kLinTargetGroups (K / 256 at most). KS does not depend on the epilogue, so every
// epilogue sums the same products in the same order and the fused entry points equal
// linear + the standalone epilogue kernels bit for bit. The merged gate / up weight
// (np = 2) takes two row tiles per work-group above kLinMt2Rows rows, which keeps its
// grid within one work-group per CU (its stages take 128 KB of LDS); row tiles do not
// change any sum. Wavefronts batch the loads of up to four chunks.
LinCfg choose_config(int rows, int tiles, int k, int np) {
  LinCfg c{};
  const int64_t base = (int64_t)tiles * ((rows + 31) / 32);
  const int blocks = k / kLinChunk;
  c.ks = blocks;
  if (base >= kLinMinGroups && blocks <= kLinMaxChunks) {
    c.ks = 1;
  } else {
    for (int s = 1; s < blocks; ++s)
      if (blocks % s == 0 && base * s >= kLinTargetGroups) {
        c.ks = s;
        break;
      }
  }
  c.mt = np == 2 && rows > kLinMt2Rows ? 2 : 1;
  c.mgroups = (rows + 32 * c.mt - 1) / (32 * c.mt);
  const int chunks = blocks / c.ks;  // 256-wide K chunks per work-group
  c.nb = chunks % 4 == 0 ? 4 : chunks % 2 == 0 ? 2 : 1;
  return c;
}

template <int NP, int MT, int EPI>
hipError_t launch_nb(const LinArgs& a, const LinCfg& c, hipStream_t stream) {
  const dim3 grid((unsigned)((a.n_out / kLinTile) * a.ks * c.mgroups));
  // at most 128 staging registers per lane: 16 per operand tile and chunk
  const int nb = (NP + MT) * 16 * c.nb > 128 ? c.nb / 2 : c.nb;
  switch (nb) {
    case 1: hipLaunchKernelGGL((linear_kernel<NP, MT, 1, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((linear_kernel<NP, MT, 2, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((linear_kernel<NP, MT, 4, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int NP, int EPI>
hipError_t launch_main(const LinArgs& a, const LinCfg& c, hipStream_t stream) {
  switch (c.mt) {
    case 1: return launch_nb<NP, 1, EPI>(a, c, stream);
    case 2: return launch_nb<NP, 2, EPI>(a, c, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

size_t linear_workspace_bytes(int32_t rows, int32_t n_out, int32_t k, int32_t epilogue) {
  if (rows <= 0 || n_out <= 0 || k <= 0) return 0;
  const bool partial = epilogue == kLinearAddRmsNorm;
  const LinCfg c = choose_config(rows, n_out / kLinTile, k, epilogue == kLinearSiluMul ? 2 : 1);
  if (c.ks == 1 && !partial) return 0;
  return (size_t)c.ks * rows * (epilogue == kLinearSiluMul ? 2 : 1) * n_out * sizeof(float);
}

hipError_t launch_linear(const void* x, int64_t x_stride, const void* w, int64_t w_stride, int32_t rows,
                         int32_t n_out, int32_t k, int32_t epilogue, void* y, int64_t y_stride, void* ws,
                         hipStream_t stream) {
  LinArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_stride = x_stride;
  a.w = static_cast<const uint16_t*>(w);
  a.w_stride = w_stride;
  a.rows = rows;
  a.n_out = n_out;
  a.k = k;
  const LinCfg c = choose_config(rows, n_out / kLinTile, k, epilogue == kLinearSiluMul ? 2 : 1);
  a.ks = c.ks;
  a.y = static_cast<uint16_t*>(y);
  a.y_stride = y_stride;
  a.part = static_cast<float*>(ws);
  const bool pair = epilogue == kLinearSiluMul;
  if (a.ks == 1) return pair ? launch_main<2, kEpiSiluMul>(a, c, stream) : launch_main<1, kEpiStore>(a, c, stream);
  hipError_t err = pair ? launch_main<2, kEpiPartial>(a, c, stream) : launch_main<1, kEpiPartial>(a, c, stream);
  if (err != hipSuccess) return err;
  const int64_t total = (int64_t)rows * (n_out / 8);
  const unsigned blocks = (unsigned)std::min<int64_t>((total + 255) / 256, 1024);
  if (pair)
    hipLaunchKernelGGL(linear_reduce_kernel<2>, dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(linear_reduce_kernel<1>, dim3(blocks), dim3(256), 0, stream, a);
  return hipGetLastError();
}

hipError_t launch_linear_add_rmsnorm(const void* x, int64_t x_stride, const void* w, int64_t w_stride,
                                     int32_t rows, int32_t n_out, int32_t k, const void* residual,
                                     int64_t res_stride, const void* norm_weight, float eps, void* out,
                                     int64_t out_stride, void* residual_out, int64_t res_out_stride, void* ws,
                                     hipStream_t stream) {
  LinArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.x_stride = x_stride;
  a.w = static_cast<const uint16_t*>(w);
  a.w_stride = w_stride;
  a.rows = rows;
  a.n_out = n_out;
  a.k = k;
  const LinCfg c = choose_config(rows, n_out / kLinTile, k, 1);
  a.ks = c.ks;
  a.part = static_cast<float*>(ws);
  hipError_t err = launch_main<1, kEpiPartial>(a, c, stream);
  if (err != hipSuccess) return err;
  const int vecs = (n_out / 8 + kLinNormThreads - 1) / kLinNormThreads;
  auto* rp = static_cast<const uint16_t*>(residual);
  auto* nw = static_cast<const uint16_t*>(norm_weight);
  auto* op = static_cast<uint16_t*>(out);
  auto* rop = static_cast<uint16_t*>(residual_out);
  switch (vecs) {
    case 1: hipLaunchKernelGGL(linear_add_rmsnorm_kernel<1>, dim3(rows), dim3(kLinNormThreads), 0, stream, a, rp, res_stride, nw, eps, op, out_stride, rop, res_out_stride); break;
    case 2: hipLaunchKernelGGL(linear_add_rmsnorm_kernel<2>, dim3(rows), dim3(kLinNormThreads), 0, stream, a, rp, res_stride, nw, eps, op, out_stride, rop, res_out_stride); break;
    case 3: hipLaunchKernelGGL(linear_add_rmsnorm_kernel<3>, dim3(rows), dim3(kLinNormThreads), 0, stream, a, rp, res_stride, nw, eps, op, out_stride, rop, res_out_stride); break;
    case 4: hipLaunchKernelGGL(linear_add_rmsnorm_kernel<4>, dim3(rows), dim3(kLinNormThreads), 0, stream, a, rp, res_stride, nw, eps, op, out_stride, rop, res_out_stride); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace pk
