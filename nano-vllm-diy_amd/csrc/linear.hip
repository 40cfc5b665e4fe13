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
// tile; 32 gate + 32 up rows for SiLU * mul) and, when there are fewer tiles than CUs, its
// K range into KS equal splits, so enough work-groups stream it at once. A work-group's
// four wavefronts take interleaved 64-wide K blocks of its range and add their
// accumulators through LDS. With KS = 1 the epilogue runs in the work-group; otherwise
// fp32 partial sums go to the workspace and a second kernel adds them and applies it
// (the residual-add + RMSNorm epilogue needs whole rows and always takes that path).
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
#ifndef PK_LINEAR_TARGET_GROUPS
#define PK_LINEAR_TARGET_GROUPS 256
#endif
constexpr int kLinTargetGroups = PK_LINEAR_TARGET_GROUPS;  // work-groups a launch aims for

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8_t;

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

// NP = weight tiles per work-group (2: gate rows n0.., up rows n_out + n0..); MT = 32-row x tiles.
template <int NP, int MT, int EPI>
__global__ __launch_bounds__(kLinThreads) void linear_kernel(const LinArgs a) {
  __shared__ float4 red[4][NP][4][kWave];  // one x-row tile of every wavefront's accumulators
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int r = lane & 31, h = lane >> 5;
  const int ntile = blockIdx.x % (a.n_out / kLinTile);
  const int split = blockIdx.x / (a.n_out / kLinTile);
  const int n0 = ntile * kLinTile;
  const int kc = a.k / a.ks;
  const int kbeg = split * kc;

  const uint16_t* wrow[NP];
#pragma unroll
  for (int p = 0; p < NP; ++p) wrow[p] = a.w + (int64_t)(p * a.n_out + n0 + r) * a.w_stride + 32 * h;
  const uint16_t* xrow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) xrow[t] = a.x + (int64_t)min(32 * t + r, a.rows - 1) * a.x_stride + 32 * h;

  f32x16 acc[NP][MT];
#pragma unroll
  for (int p = 0; p < NP; ++p)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[p][t][i] = 0.f;

  // blocks kbeg + 64 (wave + 4 j): the next block's weight is in flight during this one
  const int nblk = kc / kLinKBlock;
  uint4 wa[NP][4], wn[NP][4];
  int b = wave;
  if (b < nblk) {
#pragma unroll
    for (int p = 0; p < NP; ++p)
#pragma unroll
      for (int q = 0; q < 4; ++q) wa[p][q] = *reinterpret_cast<const uint4*>(wrow[p] + kbeg + b * kLinKBlock + 8 * q);
  }
  for (; b < nblk; b += 4) {
    const int kb = kbeg + b * kLinKBlock;
    const bool more = b + 4 < nblk;
    if (more) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) wn[p][q] = *reinterpret_cast<const uint4*>(wrow[p] + kb + 4 * kLinKBlock + 8 * q);
    }
    uint4 xb[MT][4];
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int q = 0; q < 4; ++q) xb[t][q] = *reinterpret_cast<const uint4*>(xrow[t] + kb + 8 * q);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int t = 0; t < MT; ++t)
          acc[p][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, wa[p][q]),
                                                              __builtin_bit_cast(bf16x8_t, xb[t][q]), acc[p][t], 0, 0, 0);
    if (more) {
#pragma unroll
      for (int p = 0; p < NP; ++p)
#pragma unroll
        for (int q = 0; q < 4; ++q) wa[p][q] = wn[p][q];
    }
  }

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
    const int m = 32 * t + c;
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
  float v[kVecs][8];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kVecs; ++j) {
    const int col = (j * kLinNormThreads + threadIdx.x) * 8;
    if (col < hidden) {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[j][e] = 0.f;
      for (int s = 0; s < a.ks; ++s) {
        const float* pp = a.part + ((int64_t)s * a.rows + row) * hidden + col;
        const float4 lo = *reinterpret_cast<const float4*>(pp);
        const float4 hi = *reinterpret_cast<const float4*>(pp + 4);
        v[j][0] += lo.x; v[j][1] += lo.y; v[j][2] += lo.z; v[j][3] += lo.w;
        v[j][4] += hi.x; v[j][5] += hi.y; v[j][6] += hi.z; v[j][7] += hi.w;
      }
      const uint4 rv = *reinterpret_cast<const uint4*>(residual + row * res_stride + col);
      const uint32_t rr[4] = {rv.x, rv.y, rv.z, rv.w};
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
      const uint4 w = *reinterpret_cast<const uint4*>(weight + col);
      const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
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

// K splits: the smallest divisor KS of K / 256 whose tiles x KS reach kLinTargetGroups
// work-groups (every wavefront gets at least one 64-wide block per split), else K / 256.
int choose_splits(int tiles, int k) {
  const int blocks = k / (4 * kLinKBlock);
  for (int s = 1; s < blocks; ++s)
    if (blocks % s == 0 && (int64_t)tiles * s >= kLinTargetGroups) return s;
  return blocks;
}

template <int NP, int EPI>
hipError_t launch_main(const LinArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)((a.n_out / kLinTile) * a.ks));
  const int mt = (a.rows + 31) / 32;
  switch (mt) {
    case 1: hipLaunchKernelGGL((linear_kernel<NP, 1, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    case 2: hipLaunchKernelGGL((linear_kernel<NP, 2, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    case 3: hipLaunchKernelGGL((linear_kernel<NP, 3, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    case 4: hipLaunchKernelGGL((linear_kernel<NP, 4, EPI>), grid, dim3(kLinThreads), 0, stream, a); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

size_t linear_workspace_bytes(int32_t rows, int32_t n_out, int32_t k, int32_t epilogue) {
  if (rows <= 0 || n_out <= 0 || k <= 0) return 0;
  const int ks = choose_splits(n_out / kLinTile, k);
  if (ks == 1 && epilogue != kLinearAddRmsNorm) return 0;
  return (size_t)ks * rows * (epilogue == kLinearSiluMul ? 2 : 1) * n_out * sizeof(float);
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
  a.ks = choose_splits(n_out / kLinTile, k);
  a.y = static_cast<uint16_t*>(y);
  a.y_stride = y_stride;
  a.part = static_cast<float*>(ws);
  const bool pair = epilogue == kLinearSiluMul;
  if (a.ks == 1) return pair ? launch_main<2, kEpiSiluMul>(a, stream) : launch_main<1, kEpiStore>(a, stream);
  hipError_t err = pair ? launch_main<2, kEpiPartial>(a, stream) : launch_main<1, kEpiPartial>(a, stream);
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
  a.ks = choose_splits(n_out / kLinTile, k);
  a.part = static_cast<float*>(ws);
  hipError_t err = launch_main<1, kEpiPartial>(a, stream);
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
