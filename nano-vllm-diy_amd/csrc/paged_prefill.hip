// Chunked-prefill / dense varlen attention on bf16 MFMA for gfx950.
//
// Reference semantics: flash_attn_varlen_func(..., causal=True, block_table) at
// src/layers/attention.py:95-104 for sequences with Lq > 1 query rows. Row i of a
// sequence with Lq rows and Lk keys sees keys t <= i + (Lk - Lq) (bottom-right
// alignment, the cached prefix P = Lk - Lq precedes the chunk; model_runner.py:186-190).
// Keys come through the block table (paged, chunked prefill / prefix-cache hits) or
// from fresh rows at cu_seqlens_k (flat, all-fresh prompts).
//
// Work unit: 256 query rows = TM = 256 / G query tokens x the G query heads of one kv
// head g, so each K/V tile staged in LDS serves the whole GQA group. A work-group of eight
// wavefronts (two per SIMD, one work-group per CU) owns the unit; wavefront w owns rows
// 32 w .. 32 w + 31, which are 32 consecutive tokens of one head (TM >= 32 for every GQA
// group built). All eight wavefronts pass one barrier per K/V tile, so the two wavefronts
// of a SIMD run the loop in step; what overlaps one's softmax with the other's MFMAs is
// only the hardware's interleaving of their instructions.
//
// Three launches, all sized on the host without reading device memory:
//   1. plan (one work-group): reads cu_seqlens_q/k, counts each unit's key tiles under
//      its causal limit, picks a split size T = max(8, kSplitNum / kSplitDen x total tiles
//      / pool) tiles and writes the work list: every unit longer than T is cut into equal
//      key ranges. Long items come first (four length buckets, longest first).
//   2. prefill (a persistent pool of one work-group per CU): each work-group claims items
//      from the sub-queue of its XCD (item i belongs to sub-queue i mod 8, which for 8 kv
//      heads is kv head i mod 8, so a head's K/V stays in one XCD's L2), then steals from
//      the other sub-queues. An unsplit item writes bf16 rows; a split item writes its
//      fp32 numerators and (max, sum) per row.
//   3. merge: combines the partials of every split unit, then the decode rows' partials
//      left by the call's decode launch (paged_decode.hip), which needs no combine launch.
// The split bounds the longest chain of dependent tiles (a long cached prefix would
// otherwise keep one work-group busy long after the rest of the GPU has finished).
//
// Per 64-key tile, per wavefront and 32-row block:
//   S^T (64 keys x 32 rows) = K (64 x 128) . Q^T (128 x 32)    16 v_mfma_f32_32x32x16_bf16
//   online softmax down each column (a lane owns one query row; the two lane halves
//   exchange through v_permlane32_swap)
//   O^T (128 x 32)         += V^T (128 x 64) . P^T (64 x 32)   16 v_mfma_f32_32x32x16_bf16
// K and V tiles move global -> registers -> LDS: two LDS stages of 16 KiB per operand
// (sK[2], sV[2]); at step n the loads of tile n + 2 are issued, tile n is computed and
// tile n + 1 is written from registers into the other stage. The P.V A operand comes
// from the LDS transpose read. P^T never leaves registers: the
// S^T accumulator layout already holds, per lane, the keys the P.V B operand needs once
// the k-order of the instruction is permuted (same permutation on the V side).
#include <algorithm>

#include "decode_core.h"

namespace pk {
namespace {

constexpr int kTileKeys = 64;          // keys per K/V tile
#ifndef PK_PREFILL_ROW_BLOCKS
#define PK_PREFILL_ROW_BLOCKS 1
#endif
// A wavefront owns kRowBlocks blocks of 32 query rows; every K and V operand it reads from
// LDS serves all of its blocks, so LDS read traffic per flop falls as 1 / kRowBlocks.
constexpr int kRowBlocks = PK_PREFILL_ROW_BLOCKS;
static_assert(kRowBlocks == 1 || kRowBlocks == 2, "row blocks per wavefront");
constexpr int kPrefillWaves = 8 / kRowBlocks;           // 256 rows per work-group
constexpr int kPrefillThreads = kPrefillWaves * 64;
constexpr int kWavesPerSimd = 2 / kRowBlocks;           // register file: 512 / this per lane
constexpr int kRowBytes = kHeadDim * 2;                  // one head's row of a K or V tile (256 B)
constexpr int kTileBytes = kTileKeys * kRowBytes;        // 16 KiB per operand per stage
constexpr int kPlanThreads = 1024;     // plan work-group
constexpr int kPlanCache = 2048;       // sequences whose lengths the plan keeps in LDS
constexpr int kMinSplitTiles = 8;      // never split a unit's keys below 512 per item
#ifndef PK_PREFILL_SPLIT_NUM
#define PK_PREFILL_SPLIT_NUM 2
#define PK_PREFILL_SPLIT_DEN 3
#endif
constexpr int kSplitNum = PK_PREFILL_SPLIT_NUM;  // split size = kSplitNum / kSplitDen x work per slot
constexpr int kSplitDen = PK_PREFILL_SPLIT_DEN;
constexpr int kMergeThreads = 256;     // merge: thread = row of the unit
constexpr int kMergeGroups = 1024;
constexpr int kMergeBatch = 8;         // merge: splits whose (max, sum) load in one batch
#ifndef PK_MERGE_LOADS
#define PK_MERGE_LOADS 4
#endif
constexpr int kMergeLoads = PK_MERGE_LOADS;  // merge: splits whose outputs load in one batch
#ifndef PK_PREFILL_BUCKETS
#define PK_PREFILL_BUCKETS 4
#endif
constexpr int kBuckets = PK_PREFILL_BUCKETS;  // length buckets of the work list (longest first)
constexpr float kLazyLog2 = 8.f;       // reference max moves only when exceeded by 2^8
constexpr int kStages = 2;             // K and V LDS stages of the prefill kernel

typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) char lds_char;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;


// Value of lane l ^ 32 (the other half of the wavefront), one VALU swap.
__device__ __forceinline__ float swap_halves_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}
__device__ __forceinline__ float swap_halves_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// Work-group barrier for the LDS tiles: wait until this wavefront's LDS instructions have
// completed, then s_barrier. It is issued as an instruction of its own because
// __syncthreads() would also wait for every global load in flight (its fence waits for
// vmcnt(0)), including the next tile's loads that are meant to overlap the compute.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt((15 & 15) | ((63 >> 4) << 14) | (7 << 4) | (0 << 8));  // lgkmcnt(0) only
  asm volatile("s_barrier" ::: "memory");
}

// LDS tiles are stored unpadded, one 256-byte row per key, with the row's sixteen 16-byte
// chunks XOR-swizzled so that the MFMA operand reads hit distinct banks:
//   K: chunk c of row r lives in slot c ^ (r & 15)      (32 consecutive rows read chunk c)
//   V: chunk c of row r lives in slot c ^ ((2 r) & 15) ^ 8 (c & 2)
// A V transpose read serves 32 lanes per cycle: two 16-lane groups, each reading 4
// consecutive rows x 2 chunks, the second group the next two chunks. The XOR with 2 r
// spreads a group over 8 slots; the extra 8 (c & 2) puts the second group's chunks in the
// other 8 slots, so the 32 lanes hit all 64 banks once.
__device__ __forceinline__ int k_slot(int r, int c) { return c ^ (r & 15); }
__device__ __forceinline__ int v_slot(int r, int c) { return c ^ ((2 * r) & 15) ^ ((c & 2) << 2); }
// Inverse of v_slot: the chunk stored in slot s of row r (bit 1 of the chunk survives the
// first XOR, so it names the second one).
__device__ __forceinline__ int v_chunk(int r, int s) {
  const int y = s ^ ((2 * r) & 15);
  return y ^ ((y & 2) << 2);
}

// Keys [t0, t0 + 64) of kv head g move global -> registers -> LDS: wavefront w owns tile
// rows kRowsPerWave w .. kRowsPerWave (w + 1) - 1, four rows (1 KiB) per 16-byte load
// instruction, lane l carrying slot (l & 15) of row (l >> 4) and therefore the swizzled
// source chunk. The loads for tile n + 2 are issued before tile n is computed and written
// to LDS after tile n + 1 has been (register staging keeps them off the LDS while it
// serves the MFMA operands). Keys past Lk re-read the last key's row (same cache block,
// finite data); their scores are masked and their p is 0.
constexpr int kRowsPerWave = kTileKeys / kPrefillWaves;
constexpr int kLoadsPerOperand = kRowsPerWave / 4;


// Per-lane source byte offsets of the rows this lane moves.
struct LoadLanes {
  int k[kLoadsPerOperand];
  int v[kLoadsPerOperand];
};

__device__ __forceinline__ LoadLanes load_lanes(const AttnArgs& a, int wave, int lane, int last) {
  LoadLanes l;
  const int slot = lane & 15;
#pragma unroll
  for (int i = 0; i < kLoadsPerOperand; ++i) {
    const int r = kRowsPerWave * wave + 4 * i + (lane >> 4);  // tile row this lane fills
    const int rs = min(r, last);                              // source row (clamped on the last tile)
    l.k[i] = (rs * (int)a.k_row_stride + (slot ^ (r & 15)) * 8) * 2;
    l.v[i] = (rs * (int)a.v_row_stride + v_chunk(r, slot) * 8) * 2;
  }
  return l;
}

struct KvRegs {
  u32x4 k[kLoadsPerOperand];
  u32x4 v[kLoadsPerOperand];
};

// The lane's 16-byte loads of one tile from K and V rows starting at kbase / vbase. (Buffer
// loads over the tile's rows, which keep no 64-bit lane address, measured 2-4% slower on
// the prefill batches.)
__device__ __forceinline__ void load_rows(const uint16_t* kbase, const uint16_t* vbase, const LoadLanes& l,
                                          KvRegs& R) {
#pragma unroll
  for (int i = 0; i < kLoadsPerOperand; ++i) {
    R.k[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kbase) + l.k[i]);
    R.v[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vbase) + l.v[i]);
  }
}

template <bool PAGED>
__device__ __forceinline__ void load_tile_regs(const AttnArgs& a, int b, int k0, int Lk, int g, int bt_lane, int wave,
                                               int lane, int t0, const LoadLanes& full_lanes, KvRegs& R) {
  const uint16_t* kbase;
  const uint16_t* vbase;
  if constexpr (PAGED) {
    const int j = t0 / a.block_size;  // block_size % 64 == 0: the tile sits inside one block
    const int blk = j < kWave ? __builtin_amdgcn_readlane(bt_lane, j)
                              : __builtin_amdgcn_readfirstlane(a.block_table[(int64_t)b * a.bt_stride + j]);
    const int off = t0 % a.block_size;
    kbase = a.k + (int64_t)blk * a.k_block_stride + (int64_t)off * a.k_row_stride;
    vbase = a.v + (int64_t)blk * a.v_block_stride + (int64_t)off * a.v_row_stride;
  } else {
    kbase = a.k + (int64_t)(k0 + t0) * a.k_row_stride;
    vbase = a.v + (int64_t)(k0 + t0) * a.v_row_stride;
  }
  kbase += g * kHeadDim;
  vbase += g * kHeadDim;
  load_rows(kbase, vbase, (t0 + kTileKeys <= Lk) ? full_lanes : load_lanes(a, wave, lane, Lk - 1 - t0), R);
}

__device__ __forceinline__ void store_tile_lds(const KvRegs& R, lds_char* kdst, lds_char* vdst, int wave, int lane) {
#pragma unroll
  for (int i = 0; i < kLoadsPerOperand; ++i) {
    const int off = (kRowsPerWave * wave + 4 * i) * kRowBytes + lane * 16;
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(kdst + off) = R.k[i];
    *reinterpret_cast<__attribute__((address_space(3))) u32x4*>(vdst + off) = R.v[i];
  }
}

// Online softmax of one 32-row block's S^T tile (64 keys) in place: scores become p, the
// row sums move on, and p is packed to bf16 as the P.V B operand. S^T element rr of
// half-tile mb is key t0 + 32 mb + 8 (rr >> 2) + 4 half + (rr & 3). Raw scores are
// compared (the scale is positive) and scaled inside the exponent's FMA.
// Lazy rescaling: exponentials are taken against a reference max m_i (exp2 domain) that
// moves only when some row's tile max exceeds it by more than kLazyLog2; then every row
// moves to its running max and the numerator and sum are rescaled. p <= 2^kLazyLog2, and
// numerator and sum share the reference, so o / l is unchanged.
// The parts of softmax_block over NB half-tiles of 32 keys (element rr of half-tile mb is
// key t0 + 32 mb + 8 (rr >> 2) + 4 half + (rr & 3)): the mask (diagonal tiles) and the
// row's max in the exp2 domain ...
template <int NB>
__device__ __forceinline__ void softmax_mask(f32x16 (&s)[NB], int t0, int lim, int half) {
#pragma unroll
  for (int mb = 0; mb < NB; ++mb)
#pragma unroll
    for (int rr = 0; rr < 16; ++rr)
      if (t0 + mb * 32 + 8 * (rr >> 2) + 4 * half + (rr & 3) > lim) s[mb][rr] = -INFINITY;
}

template <int NB, bool MASK>
__device__ __forceinline__ float softmax_max(f32x16 (&s)[NB], int t0, int lim, float scale_log2, int half) {
  if constexpr (MASK) softmax_mask<NB>(s, t0, lim, half);
  float tmax = -INFINITY;
#pragma unroll
  for (int mb = 0; mb < NB; ++mb)
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) tmax = fmaxf(tmax, s[mb][rr]);
  return swap_halves_max(tmax) * scale_log2;
}

// ... the lazy move of the reference max (with the rescale of numerator and sum) ...
__device__ __forceinline__ void softmax_rescale(f32x16 (&o)[4], float& m_i, float& l_i, float tm) {
  if (__builtin_amdgcn_ballot_w64(tm > m_i + kLazyLog2) != 0) {
    const float m_new = fmaxf(m_i, tm);
    const float alpha = m_new == -INFINITY ? 1.f : exp2_fast(m_i - m_new);  // 0 when m_i = -inf
    m_i = m_new;
    l_i *= alpha;
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) o[md][rr] *= alpha;
  }
}

// The row sum l from the bf16 p that the P.V product uses (16 v_dot2 per row block and tile
// instead of 32 fp32 adds): numerator and denominator then weigh every key alike. Measured
// interleaved: steady batch 693.6 -> 680.2 us, cfg3 prefill 95.9 -> 95.4 us.
#ifndef PK_PREFILL_DOT_SUM
#define PK_PREFILL_DOT_SUM 1
#endif
// ... and the exponentials against the reference max, packed to bf16 as the P.V B operand.
template <int NB>
__device__ __forceinline__ void softmax_exp(f32x16 (&s)[NB], bf16x8 (&pb)[2 * NB], float m_i, float& l_i,
                                            float scale_log2) {
  const float m_use = (m_i == -INFINITY) ? 0.f : m_i;  // row saw no key yet: every p is 0
  float psum = 0.f;
#pragma unroll
  for (int mb = 0; mb < NB; ++mb)
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const float p = exp2_fast(__builtin_fmaf(s[mb][rr], scale_log2, -m_use));
      s[mb][rr] = p;
      if (!PK_PREFILL_DOT_SUM) psum += p;
    }
  // B operand of k-block kb2: element e of lane half `half` stands for key
  // 16 kb2 + 8 (e >> 2) + 4 half + (e & 3) = accumulator element 8 (kb2 & 1) + e of
  // half-tile kb2 >> 1.
#pragma unroll
  for (int kb2 = 0; kb2 < 2 * NB; ++kb2)
#pragma unroll
    for (int e = 0; e < 8; ++e) pb[kb2][e] = static_cast<__bf16>(s[kb2 >> 1][8 * (kb2 & 1) + e]);
  if (PK_PREFILL_DOT_SUM) {
    // the row sum from the bf16 p the P.V product uses: one v_dot2 per pair of keys
    const bf16x2 one = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
#pragma unroll
    for (int kb2 = 0; kb2 < 2 * NB; ++kb2)
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        const bf16x2 pr = {pb[kb2][e], pb[kb2][e + 1]};
        psum = __builtin_amdgcn_fdot2_f32_bf16(pr, one, psum, false);
      }
  }
  l_i += psum;
}

__device__ __forceinline__ void softmax_block(f32x16 (&s)[2], f32x16 (&o)[4], bf16x8 (&pb)[4], float& m_i, float& l_i,
                                              int t0, int lim, bool full, float scale_log2, int half) {
  const float tm = full ? softmax_max<2, false>(s, t0, lim, scale_log2, half)
                        : softmax_max<2, true>(s, t0, lim, scale_log2, half);
  softmax_rescale(o, m_i, l_i, tm);
  softmax_exp<2>(s, pb, m_i, l_i, scale_log2);
}

// Per-lane LDS byte offsets of the MFMA operand reads inside a stage.
//   K, k-block kb: row col (+ 32 for the second half-tile: + 8 KiB), chunk 2 kb + half,
//     swizzled with col & 15 (32 mb + col has the same low bits);
//   V, d-block md: row 4 half + (src >> 2) (+ 16 kb2 rows: + 4 KiB, + 8 rows: + 2 KiB), the
//     swizzle (2 r) & 15 does not see those row steps.
struct TileLanes {
  int k0, v0;
  // Offsets of k-block kb and d-block md: the k-block moves the chunk by 2 kb and the d-block
  // by 4 md, bits the swizzles only XOR with lane bits, so the offsets are k0 ^ 32 kb and
  // v0 ^ 64 md (one VALU op per read instead of twelve live registers).
  __device__ __forceinline__ int k(int kb) const { return k0 ^ (32 * kb); }
  __device__ __forceinline__ int v(int md) const { return v0 ^ (64 * md); }
};

__device__ __forceinline__ TileLanes tile_lanes(int lane) {
  TileLanes t;
  const int col = lane & 31;
  const int half = lane >> 5;
  const int grp = lane >> 4;
  const int src = lane & 15;
  t.k0 = col * kRowBytes + k_slot(col, half) * 16;
  const int d = 16 * (grp & 1) + 4 * (src & 3);
  const int r = 4 * half + (src >> 2);
  t.v0 = r * kRowBytes + v_slot(r, d >> 3) * 16 + (d & 7) * 2;
  return t;
}

// One 64-key tile for the wavefront's kRowBlocks blocks of 32 query rows.
__device__ __forceinline__ void compute_tile(const lds_char* sK, const lds_char* sV, const TileLanes& tl,
                                             const bf16x8 (&qb)[kRowBlocks][kHeadDim / 16],
                                             f32x16 (&o)[kRowBlocks][4], float (&m_i)[kRowBlocks],
                                             float (&l_i)[kRowBlocks], int t0, const int (&lim)[kRowBlocks],
                                             const bool (&full)[kRowBlocks], float scale_log2, int lane) {
  const int half = lane >> 5;
  f32x16 s[kRowBlocks][2];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) s[rb][mb][rr] = 0.f;
  // K A operand of half-tile mb, k-block kb: read kKDepth k-blocks ahead of the MFMAs that
  // use it, the order pinned by scheduling groups (the compiler's own schedule read each
  // k-block right before its two MFMAs and waited for it: no read was in flight while an
  // MFMA ran).
#ifndef PK_PREFILL_KDEPTH
#define PK_PREFILL_KDEPTH 2
#endif
  constexpr int kKDepth = PK_PREFILL_KDEPTH;
  constexpr int kKBlocks = kHeadDim / 16;
  bf16x8 ka[kKBlocks][2];
  const auto read_k = [&](int kb) {
#pragma unroll
    for (int mb = 0; mb < 2; ++mb)
      ka[kb][mb] = *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(sK + tl.k(kb) +
                                                                                   mb * 32 * kRowBytes);
  };
#pragma unroll
  for (int kb = 0; kb < kKDepth; ++kb) read_k(kb);
#pragma unroll
  for (int kb = 0; kb < kKBlocks; ++kb) {
    if (kb + kKDepth < kKBlocks) read_k(kb + kKDepth);
#pragma unroll
    for (int rb = 0; rb < kRowBlocks; ++rb)
#pragma unroll
      for (int mb = 0; mb < 2; ++mb)
        s[rb][mb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ka[kb][mb], qb[rb][kb], s[rb][mb], 0, 0, 0);
  }
#pragma unroll
  for (int kb = 0; kb < kKDepth; ++kb) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);  // DS reads
#pragma unroll
  for (int kb = 0; kb < kKBlocks; ++kb) {
    if (kb + kKDepth < kKBlocks) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    __builtin_amdgcn_sched_group_barrier(0x008, 2 * kRowBlocks, 0);  // MFMAs
  }

  bf16x8 pb[kRowBlocks][4];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb)
    softmax_block(s[rb], o[rb], pb[rb], m_i[rb], l_i[rb], t0, lim[rb], full[rb], scale_log2, half);

  // O^T += V^T . P^T over 16-key k-blocks. The A operand (4 consecutive keys of one
  // head_dim element, twice) comes from the row-major V tile through the LDS transpose
  // read: in each 16-lane group, source lane s addresses 4 elements of key row
  // key0 + (s >> 2) at head_dim d0 + 4 (s & 3), and lane i receives element d0 + i of keys
  // key0 .. key0 + 3. Each A operand serves every row block.
#pragma unroll
  for (int kb2 = 0; kb2 < 4; ++kb2) {
#pragma unroll
    for (int md = 0; md < 4; ++md) {
      const lds_char* p_lo = sV + tl.v(md) + kb2 * 16 * kRowBytes;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          const_cast<lds_v4i16*>(reinterpret_cast<const lds_v4i16*>(p_lo)));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
          const_cast<lds_v4i16*>(reinterpret_cast<const lds_v4i16*>(p_lo + 8 * kRowBytes)));
      const bf16x8 av = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
      for (int rb = 0; rb < kRowBlocks; ++rb)
        o[rb][md] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, pb[rb][kb2], o[rb][md], 0, 0, 0);
    }
  }
}

// Sequence geometry shared by the plan, prefill and merge kernels.
struct SeqDims {
  int q0, Lq, k0, Lk, P, nq;  // nq: query tiles of the sequence (0: not a prefill sequence)
};

template <int TM>
__device__ __forceinline__ SeqDims seq_dims(const AttnArgs& a, int b) {
  SeqDims d;
  d.q0 = a.cu_q[b];
  d.Lq = a.cu_q[b + 1] - d.q0;
  d.k0 = a.cu_k[b];
  d.Lk = min(a.cu_k[b + 1] - d.k0, a.max_seqlen_k);
  d.P = d.Lk - d.Lq;
  // Lq == 1 rows belong to the decode kernel; Lq <= 0 or Lk <= 0 is graph padding
  d.nq = (d.Lq <= 1 || d.Lk <= 0) ? 0 : min((d.Lq + TM - 1) / TM, a.prefill_qtiles);
  return d;
}

// Key tiles query tile qt needs: keys below its last row's causal limit.
template <int TM, bool CAUSAL>
__device__ __forceinline__ int unit_tiles(const SeqDims& d, int qt) {
  const int kv_end = CAUSAL ? min(d.Lk, (qt + 1) * TM + d.P) : d.Lk;
  return kv_end > 0 ? (kv_end + kTileKeys - 1) / kTileKeys : 0;
}

// Splits of a unit of t tiles for split size T, and the start tile of split s.
__device__ __forceinline__ int unit_splits(int t, int T) { return t > T ? (t + T - 1) / T : 1; }
__device__ __forceinline__ int split_begin(int t, int n, int s) { return (int)((unsigned)(t * s) / (unsigned)n); }

// Length bucket of a group of t tiles (0 = longest) for split size T.
__device__ __forceinline__ int length_bucket(int t, int T) {
  int j = 0;  // the largest j < kBuckets with t kBuckets > j T (compares, no division)
#pragma unroll
  for (int i = 1; i < kBuckets; ++i) j = t * kBuckets > i * T ? i : j;
  return kBuckets - 1 - j;
}

// Work list. Waves take sequences in turn and lanes take a sequence's query tiles, so a
// long prompt's tiles are planned in parallel. Groups land in their length bucket through
// LDS cursors: the order inside a bucket depends on timing, but a group's work and the
// merge order of its splits do not, so results are bit-identical from run to run.
template <int G, bool CAUSAL>
__global__ __launch_bounds__(kPlanThreads) void prefill_plan_kernel(const AttnArgs a) {
  constexpr int TM = kPrefillRows / G;
  constexpr int W = kPlanThreads / kWave;
  __shared__ long long red[W];
  __shared__ int cur[kBuckets + 2];  // bucket cursors, partial-group cursor, merge cursor
  // (Lq, Lk) of up to kPlanCache sequences, so passes 2 and 3 skip the global round trip
  __shared__ int2 dims[kPlanCache];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int S = a.num_seqs;
  const int hkv = a.num_kv_heads;

  for (int b = tid; b < min(S, kPlanCache); b += kPlanThreads) {
    const SeqDims d = seq_dims<TM>(a, b);
    dims[b] = make_int2(d.Lq, d.Lk);
  }
  __syncthreads();
  auto dims_of = [&](int b) {
    if (b >= kPlanCache) return seq_dims<TM>(a, b);
    SeqDims d;
    d.q0 = d.k0 = 0;  // not used by the plan
    d.Lq = dims[b].x;
    d.Lk = dims[b].y;
    d.P = d.Lk - d.Lq;
    d.nq = (d.Lq <= 1 || d.Lk <= 0) ? 0 : min((d.Lq + TM - 1) / TM, a.prefill_qtiles);
    return d;
  };

  // pass 1: total key tiles over all units
  long long tiles = 0;
  for (int b = wave; b < S; b += W) {
    const SeqDims d = dims_of(b);
    for (int qt = lane; qt < d.nq; qt += kWave) tiles += unit_tiles<TM, CAUSAL>(d, qt);
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) tiles += __shfl_xor(tiles, o, kWave);
  if (lane == 0) red[wave] = tiles;
  if (tid < kBuckets + 2) cur[tid] = 0;
  __syncthreads();
  long long work = 0;
#pragma unroll
  for (int w = 0; w < W; ++w) work += red[w];
  work *= hkv;
  // split size: kSplitNum / kSplitDen of the work per slot, at least kMinSplitTiles (no unit
  // has 2^20 tiles)
  const int T = (int)min((long long)(1 << 20),
                         max((long long)kMinSplitTiles,
                             (kSplitNum * (work / kSplitDen) + a.pf_slots - 1) / a.pf_slots + 1));

  // pass 2: groups per length bucket
  for (int b = wave; b < S; b += W) {
    const SeqDims d = dims_of(b);
    for (int qt = lane; qt < d.nq; qt += kWave) {
      const int t = unit_tiles<TM, CAUSAL>(d, qt);
      const int n = unit_splits(t, T);
      for (int sp = 0; sp < n; ++sp)
        atomicAdd(&cur[length_bucket(split_begin(t, n, sp + 1) - split_begin(t, n, sp), T)], 1);
    }
  }
  __syncthreads();
  int tot = 0, start[kBuckets];
#pragma unroll
  for (int k = 0; k < kBuckets; ++k) {
    start[k] = tot;
    tot += cur[k];
  }
  __syncthreads();
  if (tid < kBuckets) cur[tid] = 0;
  __syncthreads();

  // pass 3: emit one entry per group; kv heads are expanded by index (item i = head i % hkv
  // of group i / hkv)
  for (int b = wave; b < S; b += W) {
    const SeqDims d = dims_of(b);
    for (int qt = lane; qt < d.nq; qt += kWave) {
      const int t = unit_tiles<TM, CAUSAL>(d, qt);
      const int n = unit_splits(t, T);
      // partial groups stay below 3 x slots / hkv (each split unit has more than T tiles)
      const int pg = n > 1 ? atomicAdd(&cur[kBuckets], n) : -1;
      for (int sp = 0; sp < n; ++sp) {
        const int tb = split_begin(t, n, sp);
        const int te = split_begin(t, n, sp + 1);
        const int k = length_bucket(te - tb, T);
        const int grp = start[k] + atomicAdd(&cur[k], 1);
        if (grp < a.pf_item_cap) a.pf_items[grp] = make_int4(b, qt, tb | (te << 16), n > 1 ? pg + sp : -1);
      }
      if (n > 1) {
        const int m = atomicAdd(&cur[kBuckets + 1], 1);
        if (m < a.pf_merge_cap) a.pf_merges[m] = make_int4(b, qt, pg, n);
      }
    }
  }
  // LDS-only: the counts in cur are final; the work-list stores need not complete before the
  // queue header's (the prefill kernel, a later launch, reads both)
  lds_barrier();
  if (tid < 8) a.pf_queue[tid * kPrefillQueueStride] = 0;
  if (tid == 0) {
    a.pf_queue[kPrefillQueueMeta] = (int)(min((int64_t)tot, (int64_t)a.pf_item_cap) * hkv);
    a.pf_queue[kPrefillQueueMeta + 1] = (int)(min((int64_t)cur[kBuckets + 1], (int64_t)a.pf_merge_cap) * hkv);
    a.pf_queue[kPrefillQueueMeta + 2] = T;
  }
}

// One work item: kv head g of group `it` = (sequence b, query tile qt, key tiles [tb, te),
// partial group or -1). The caller's hooks run at three points, which the kernel uses to
// claim and prefetch the next item: last_step when the last key tile starts, after_tiles
// after the last tile's barrier (before the epilogue), after_epilogue after its stores.
template <int G, bool PAGED, bool CAUSAL, class LastStep, class AfterTiles, class AfterEpilogue>
__device__ __forceinline__ void prefill_item(const AttnArgs& a, const int4 it, const int g, const int cuv,
                                             const int bt_lane, lds_char* const (&KS)[kStages],
                                             lds_char* const (&VS)[kStages],
                                             int wave, int lane,
                                             LastStep&& last_step, AfterTiles&& after_tiles,
                                             AfterEpilogue&& after_epilogue) {
  constexpr int D = kHeadDim;
  constexpr int TN = kTileKeys;
  constexpr int TM = kPrefillRows / G;
  static_assert(TM >= 32, "a 32-row block is one head");
  const int b = it.x;
  const int qt = it.y;
  const int tb = it.z & 0xffff;
  const int te = it.z >> 16;
  const int part = it.w < 0 ? -1 : it.w * a.num_kv_heads + g;
  // The work list is trusted only as far as the buffers reach: an entry naming a sequence or
  // key tiles outside this call (a workspace overwritten by an overlapping call) is skipped.
  // The hooks run in every case, so the work-group's barriers and claims stay in step.
  // cuv (lanes 0..3) holds the sequence's bounds, loaded by the caller.
  const int q0 = __builtin_amdgcn_readlane(cuv, 0);
  const int Lq = __builtin_amdgcn_readlane(cuv, 1) - q0;
  const int k0 = __builtin_amdgcn_readlane(cuv, 2);
  const int Lk = min(__builtin_amdgcn_readlane(cuv, 3) - k0, a.max_seqlen_k);
  const int P = Lk - Lq;
  if (b < 0 || b >= a.num_seqs || Lq <= 0 || tb > te || te > (Lk + TN - 1) / TN) {
    lds_barrier();
    after_tiles();
    after_epilogue();
    return;
  }
  const int tok_begin = qt * TM;

  const int col = lane & 31;   // MFMA column = this lane's query row inside a block
  const int half = lane >> 5;
  int row[kRowBlocks], h[kRowBlocks], tok[kRowBlocks], lim[kRowBlocks], lim_lo[kRowBlocks], lim_hi[kRowBlocks];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb) {
    const int r0 = (wave * kRowBlocks + rb) * 32;  // first row of the block: 32 tokens of one head
    row[rb] = r0 + col;
    h[rb] = g * G + row[rb] / TM;
    tok[rb] = tok_begin + row[rb] % TM;
    lim[rb] = CAUSAL ? min(Lk - 1, tok[rb] + P) : Lk - 1;  // last key this row sees
    const int blo = tok_begin + r0 % TM;
    lim_lo[rb] = CAUSAL ? min(Lk - 1, blo + P) : Lk - 1;       // keys <= lim_lo: seen by all rows
    lim_hi[rb] = CAUSAL ? min(Lk - 1, blo + 31 + P) : Lk - 1;  // keys >  lim_hi: seen by none
  }

  // Q^T B operands: k-block kb covers d in [16 kb, 16 kb + 16); lane holds 8 of them.
  // Rows past Lq read the last row (finite) and are never stored.
  bf16x8 qb[kRowBlocks][D / 16];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb) {
    const uint16_t* qp = a.q + (int64_t)(q0 + min(tok[rb], Lq - 1)) * a.q_row_stride + h[rb] * D + 8 * half;
#pragma unroll
    for (int kb = 0; kb < D / 16; ++kb)
      qb[rb][kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp + kb * 16));
  }
  f32x16 o[kRowBlocks][4];
  float m_i[kRowBlocks], l_i[kRowBlocks];
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb) {
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) o[rb][md][rr] = 0.f;
    m_i[rb] = -INFINITY;
    l_i[rb] = 0.f;
  }

  // Pipeline, one barrier per tile: at step n, tile n + 1 (registers) is written to stage
  // (n + 1) & 1 and the loads of tile n + 2 go out into the same registers, tile n is computed
  // from stage n & 1, and the barrier publishes tile n + 1.
  const int ntiles = te - tb;
  const int tbase = tb * TN;
  const LoadLanes ll = load_lanes(a, wave, lane, kTileKeys);
  const TileLanes tl = tile_lanes(lane);
  KvRegs R;
  // The tile loop is entered only from the path that stored tile 0, whose register wait also
  // covers the Q loads issued before it. (With a path around that store into the loop, the
  // compiler's wait counting assumed the Q loads could still be in flight in every iteration
  // and made each k-block's QK MFMA wait for the global loads issued before it -- tile n + 2's
  // staging loads -- exposing their latency in every tile.)
  if (ntiles <= 0) lds_barrier();
  else {
  load_tile_regs<PAGED>(a, b, k0, Lk, g, bt_lane, wave, lane, tbase, ll, R);
  store_tile_lds(R, KS[0], VS[0], wave, lane);
  if (ntiles > 1) load_tile_regs<PAGED>(a, b, k0, Lk, g, bt_lane, wave, lane, tbase + TN, ll, R);
  lds_barrier();
  for (int n0 = 0; n0 < ntiles; n0 += 2) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int n = n0 + s;
      if (n >= ntiles) break;
      if (n == ntiles - 1) last_step();
      const int t0 = tbase + n * TN;
      // tile n + 1 (loaded during tile n - 1) goes to the other stage -- last read at step
      // n - 1, before the previous barrier -- and its registers take tile n + 2's loads: one
      // set of staging registers (a second set, holding tile n + 2 while tile n + 1 waited to
      // be stored after tile n, took the kernel to 256 VGPRs with spills; 2.4% slower)
      if (n + 1 < ntiles) {
        store_tile_lds(R, KS[s ^ 1], VS[s ^ 1], wave, lane);
        if (n + 2 < ntiles) load_tile_regs<PAGED>(a, b, k0, Lk, g, bt_lane, wave, lane, t0 + 2 * TN, ll, R);
      }
      bool any = false, full[kRowBlocks];
#pragma unroll
      for (int rb = 0; rb < kRowBlocks; ++rb) {
        any |= t0 <= lim_hi[rb];
        full[rb] = t0 + TN - 1 <= lim_lo[rb];
      }
      if (any) compute_tile(KS[s], VS[s], tl, qb, o, m_i, l_i, t0, lim, full, a.scale_log2, lane);
      lds_barrier();
    }
  }
  }

  after_tiles();
  // Epilogue: O^T element rr of d-block md is d = 32 md + 8 (rr >> 2) + 4 half + (rr & 3).
#pragma unroll
  for (int rb = 0; rb < kRowBlocks; ++rb) {
    const float l_tot = swap_halves_sum(l_i[rb]);
    if (tok[rb] >= Lq) continue;
    if (part < 0) {
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;  // a row that saw no key is written as 0
      uint16_t* op = a.out + (int64_t)(q0 + tok[rb]) * a.out_row_stride + h[rb] * D + 4 * half;
#pragma unroll
      for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          uint2 w;
          w.x = pack_bf16x2(o[rb][md][4 * gq] * inv, o[rb][md][4 * gq + 1] * inv);
          w.y = pack_bf16x2(o[rb][md][4 * gq + 2] * inv, o[rb][md][4 * gq + 3] * inv);
          *reinterpret_cast<uint2*>(op + md * 32 + 8 * gq) = w;
        }
    } else if (part < a.pf_part_cap) {
      // The split's own output o / l in bf16 -- as precise as an unsplit row's output -- with
      // (max, sum) in fp32 for the merge. Chunk-major (chunk = 4 dims = d / 4): one store
      // instruction writes two contiguous 256-byte runs (32 rows x 8 bytes per lane half).
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
      uint16_t* po = a.pf_part_o + (int64_t)part * (32 * kPrefillRows * 4);
#pragma unroll
      for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
          const int chunk = 8 * md + 2 * gq + half;
          uint2 w;
          w.x = pack_bf16x2(o[rb][md][4 * gq] * inv, o[rb][md][4 * gq + 1] * inv);
          w.y = pack_bf16x2(o[rb][md][4 * gq + 2] * inv, o[rb][md][4 * gq + 3] * inv);
          *reinterpret_cast<uint2*>(po + ((int64_t)chunk * kPrefillRows + row[rb]) * 4) = w;
        }
      if (half == 0)
        *reinterpret_cast<float2*>(a.pf_part_ml + ((int64_t)part * kPrefillRows + row[rb]) * 2) =
            make_float2(m_i[rb], l_tot);
    }
  }
  after_epilogue();
}

template <int G, bool PAGED, bool CAUSAL>
__global__ __launch_bounds__(kPrefillThreads, kWavesPerSimd) void prefill_kernel(const AttnArgs a) {
  // two stages per operand (constant stage indices put the stage offset in immediates)
  __shared__ __attribute__((aligned(1024))) char sK[kStages][kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV[kStages][kTileBytes];
  __shared__ int s_item;  // the claimed item index
  lds_char* KS[kStages];
  lds_char* VS[kStages];
#pragma unroll
  for (int st = 0; st < kStages; ++st) {
    KS[st] = (lds_char*)sK[st];
    VS[st] = (lds_char*)sV[st];
  }

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  // Work-groups are dealt to the 8 XCDs round-robin by linear id: this one claims items of
  // sub-queue x = blockIdx mod 8 (items i = 8 j + x, counter x) while it has any, then steals
  // from the others. Wavefront 0 claims; lane 0 owns the atomics.
  const int xcd = blockIdx.x & 7;
  const int num_items = (int)min((int64_t)a.pf_queue[kPrefillQueueMeta], (int64_t)a.pf_item_cap * a.num_kv_heads);
  // The claim on the own sub-queue goes out when the current item starts its last key tile,
  // so the atomic overlaps that tile and the work-group holds no item it cannot start yet
  // (items are long: a claim made earlier would hold one back from idle work-groups at the
  // end). `pend` is that atomic's result (lane 0).
  bool own = true;
  int pend = 0;
  const auto claim_issue = [&]() {
    if (wave == 0 && own && lane == 0) pend = atomicAdd(&a.pf_queue[xcd * kPrefillQueueStride], 1);
  };
  // Wavefront 0: the claimed index, or -1 once every sub-queue is exhausted. Stealing reads
  // the other seven counters at once (lanes 0..6) and takes from the first sub-queue after
  // this one that has items left; a claim that lost the race reads again. Counters only
  // grow, so a stale read never shows a sub-queue exhausted too early.
  const auto claim_finish = [&]() {
    if (own) {
      const int64_t cand = (int64_t)__builtin_amdgcn_readfirstlane(pend) * 8 + xcd;
      if (cand < num_items) return (int)cand;
      own = false;
    }
    for (;;) {
      const int q = (xcd + 1 + lane) & 7;
      const int c = lane < 7 ? __hip_atomic_load(&a.pf_queue[q * kPrefillQueueStride], __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT)
                             : 0;
      const uint64_t left = __builtin_amdgcn_ballot_w64(lane < 7 && (int64_t)c * 8 + q < num_items);
      if (left == 0) return -1;
      const int qs = (xcd + 1 + __builtin_ctzll(left)) & 7;
      int r = 0;
      if (lane == 0) r = atomicAdd(&a.pf_queue[qs * kPrefillQueueStride], 1);
      const int64_t cand = (int64_t)__builtin_amdgcn_readfirstlane(r) * 8 + qs;
      if (cand < num_items) return (int)cand;
    }
  };
  if (wave == 0) {
    claim_issue();
    const int c = claim_finish();
    if (lane == 0) s_item = c;
  }
  lds_barrier();
  // The next item's inputs load in two dependent steps around the current item's epilogue:
  // its work-list group (lanes 0..3) before the epilogue's stores, then the sequence's
  // bounds (lanes 0..3: cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]) and first 64
  // block-table entries (one per lane: a tile's block id is a readlane, not a dependent
  // global load) after them.
  const auto load_group = [&](int i) {
    return lane < 4 ? reinterpret_cast<const int*>(a.pf_items)[(int64_t)(i / a.num_kv_heads) * 4 + lane] : 0;
  };
  // The work list is trusted only as far as the buffers reach: a group naming a sequence
  // outside this call (a workspace overwritten by an overlapping call) reads sequence 0's
  // bounds and is skipped by prefill_item.
  const auto seq_of = [&](int grpv) {
    const int b = __builtin_amdgcn_readlane(grpv, 0);
    return b >= 0 && b < a.num_seqs ? b : 0;
  };
  const auto load_bounds = [&](int b) {
    const int32_t* p = lane < 2 ? a.cu_q + b + lane : a.cu_k + b + (lane - 2);
    return lane < 4 ? *p : 0;
  };
  const auto load_bt = [&](int b) {
    if constexpr (!PAGED) return 0;
    return lane < min(a.bt_stride, kWave) ? a.block_table[(int64_t)b * a.bt_stride + lane] : 0;
  };
  int idx = __builtin_amdgcn_readfirstlane(s_item);
  int grpv = 0, cuv = 0, btv = 0;
  if (idx >= 0) {
    grpv = load_group(idx);
    cuv = load_bounds(seq_of(grpv));
    btv = load_bt(seq_of(grpv));
  }
  while (idx >= 0) {
    int next = -1, next_grpv = 0, next_cuv = 0, next_btv = 0;
    bool claimed = false;
    const int grp = idx / a.num_kv_heads;
    const int4 it = make_int4(__builtin_amdgcn_readlane(grpv, 0), __builtin_amdgcn_readlane(grpv, 1),
                              __builtin_amdgcn_readlane(grpv, 2), __builtin_amdgcn_readlane(grpv, 3));
    prefill_item<G, PAGED, CAUSAL>(
        a, it, idx - grp * a.num_kv_heads, cuv, btv, KS, VS, wave, lane,
        [&]() {
          claim_issue();
          claimed = true;
        },
        [&]() {
          // s_item was last read before this item's first barrier
          if (wave == 0) {
            if (!claimed) claim_issue();
            const int c = claim_finish();
            if (lane == 0) s_item = c;
          }
          lds_barrier();
          next = __builtin_amdgcn_readfirstlane(s_item);
          if (next >= 0) next_grpv = load_group(next);
        },
        [&]() {
          if (next >= 0) {
            next_cuv = load_bounds(seq_of(next_grpv));
            next_btv = load_bt(seq_of(next_grpv));
          }
        });
    idx = next;
    grpv = next_grpv;
    cuv = next_cuv;
    btv = next_btv;
  }
}

// Merge the partials of every split unit: out = sum_s w_s o_s / sum_s w_s with
// w_s = exp2(m_s - max_s m_s) l_s, o_s the split's normalised output (bf16). Work item =
// (split unit, quarter of head_dim, kv head); thread t owns row t of the unit and 8 chunks
// of 4 dims. At most 4 wavefronts per SIMD: the register budget lets the loads of
// kMergeLoads splits be in flight at once. Two rounds of loads reach the first store: the
// work-list entry (the first one read together with the work count, from a list slot that
// always exists), then the sequence's bounds with the partials (which do not depend on
// them; rows past the sequence are dropped at the store).
template <int G>
__global__ __launch_bounds__(kMergeThreads) __attribute__((amdgpu_waves_per_eu(1, 4))) void prefill_merge_kernel(
    const AttnArgs a) {
  constexpr int D = kHeadDim;
  constexpr int TM = kPrefillRows / G;
  constexpr int CQ = 8;  // chunks per quarter
  const int r = threadIdx.x;
  const int hkv = a.num_kv_heads;
  // w = (unit, quarter) * hkv + g: with 8 kv heads, head g's merges run on XCD g (work-groups
  // go to XCDs round-robin and the grid is a multiple of 8), where the prefill kernel's
  // sub-queue g wrote its partials, so the reads mostly hit that XCD's L2
  const auto entry = [&](int w) { return a.pf_merges[min((w / hkv) >> 2, a.pf_merge_cap - 1)]; };
  int w = blockIdx.x;
  int4 e = entry(w);
  const int merges = a.pf_queue[kPrefillQueueMeta + 1];
  // the entry is consumed here, so its load goes out with the count's, not after the loop test
  asm volatile("" ::"v"(e.x), "v"(e.y), "v"(e.z), "v"(e.w));
  const int nw = (int)min((int64_t)merges, (int64_t)a.pf_merge_cap * hkv) * 4;
  for (; w < nw; w += gridDim.x, e = entry(w)) {
    const int rest = w / hkv;
    const int g = w - rest * hkv;
    const int c0 = (rest & 3) * CQ;
    const int b = __builtin_amdgcn_readfirstlane(e.x);  // one entry per work-group
    const int qt = __builtin_amdgcn_readfirstlane(e.y);
    const int pg = __builtin_amdgcn_readfirstlane(e.z);
    const int n = __builtin_amdgcn_readfirstlane(e.w);
    if (b < 0 || b >= a.num_seqs || pg < 0 || n <= 0) continue;  // see prefill_item
    if ((int64_t)(pg + n) * hkv > a.pf_part_cap) continue;       // the plan bounds partial ids
    const int q0 = a.cu_q[b];
    const int q1 = a.cu_q[b + 1];
    const int tok = qt * TM + r % TM;
    const int h = g * G + r / TM;
    // Every load below reads a valid split (index clamped to the last one) and a split past
    // the end gets weight 0 by arithmetic on the loaded values (max - inf, sum x 0), which
    // keeps every load unconditional: no load sits behind a branch, so the compiler's wait
    // counts see a whole batch in flight instead of waiting out each load in turn.
    const int last = n - 1;
    const float* ml_base = a.pf_part_ml + ((int64_t)(pg * hkv + g) * kPrefillRows + r) * 2;
    const int64_t ml_step = (int64_t)hkv * kPrefillRows * 2;  // next split of the unit
    const auto load_ml = [&](int s2) {
      const float2 v = *reinterpret_cast<const float2*>(ml_base + min(s2, last) * ml_step);
      return make_float2(v.x + (s2 < n ? 0.f : -INFINITY), v.y * (s2 < n ? 1.f : 0.f));
    };
    const int64_t po_step = (int64_t)hkv * (32 * kPrefillRows * 4);
    const uint16_t* po_base = a.pf_part_o + (int64_t)(pg * hkv + g) * (32 * kPrefillRows * 4) +
                              ((int64_t)c0 * kPrefillRows + r) * 4;
    const auto load = [&](int s2, uint2 (&v)[CQ]) {
#pragma unroll
      for (int c = 0; c < CQ; ++c)
        v[c] = *reinterpret_cast<const uint2*>(po_base + min(s2, last) * po_step + (int64_t)c * kPrefillRows * 4);
    };
    float2 ml[kMergeBatch];
#pragma unroll
    for (int s2 = 0; s2 < kMergeBatch; ++s2) ml[s2] = load_ml(s2);
    uint2 v[kMergeLoads][CQ];
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j) load(j, v[j]);
    float M = -INFINITY;
#pragma unroll
    for (int s2 = 0; s2 < kMergeBatch; ++s2) M = fmaxf(M, ml[s2].x);
    for (int s2 = kMergeBatch; s2 < n; ++s2) M = fmaxf(M, ml_base[s2 * ml_step]);
    float4 acc[CQ];
#pragma unroll
    for (int c = 0; c < CQ; ++c) acc[c] = make_float4(0.f, 0.f, 0.f, 0.f);
    float L = 0.f;
    // weight 0 for a split past the end or that saw no key (and for every split of a row that
    // saw none: M = -inf)
    const auto add = [&](float2 m, const uint2 (&vv)[CQ]) {
      const float wgt = M == -INFINITY ? 0.f : exp2_fast(m.x - M) * m.y;
      L += wgt;
#pragma unroll
      for (int c = 0; c < CQ; ++c) {
        acc[c].x += wgt * bf16_lo(vv[c].x);
        acc[c].y += wgt * bf16_hi(vv[c].x);
        acc[c].z += wgt * bf16_lo(vv[c].y);
        acc[c].w += wgt * bf16_hi(vv[c].y);
      }
    };
#pragma unroll
    for (int j = 0; j < kMergeLoads; ++j) add(ml[j], v[j]);
    for (int s0 = kMergeLoads; s0 < n; s0 += kMergeLoads) {  // units of many splits
#pragma unroll
      for (int j = 0; j < kMergeLoads; ++j) load(s0 + j, v[j]);
#pragma unroll
      for (int j = 0; j < kMergeLoads; ++j) add(load_ml(s0 + j), v[j]);
    }
    if (tok >= q1 - q0) continue;  // row past the sequence
    const float inv = L > 0.f ? 1.f / L : 0.f;
    uint16_t* op = a.out + (int64_t)(q0 + tok) * a.out_row_stride + h * D + 4 * c0;
#pragma unroll
    for (int c = 0; c < CQ; ++c) {
      uint2 wv;
      wv.x = pack_bf16x2(acc[c].x * inv, acc[c].y * inv);
      wv.y = pack_bf16x2(acc[c].z * inv, acc[c].w * inv);
      *reinterpret_cast<uint2*>(op + 4 * c) = wv;
    }
  }
  // The decode rows' combines (their partials were left by this call's decode launch, which
  // runs first): one (sequence, head) per 128 threads, continuing the work-group order after
  // the split-unit merges so the groups with fewer of those start on these.
  if (a.combine_in_merge) {
    const int pairs = a.num_seqs * a.num_heads;
    const int half = (int)(threadIdx.x >> 7);
    const int grid = (int)gridDim.x;
    const int first = (int)((blockIdx.x + grid - nw % grid) % grid);
    for (int pr = 2 * first + half; pr < pairs; pr += 2 * grid) {
      const int b = pr / a.num_heads;
      combine_row(a, b, pr - b * a.num_heads, threadIdx.x & (kCombineThreads - 1));
    }
  }
}

// ---- Shared-prefix decode ------------------------------------------------------------------
// Decode rows (one query row per sequence) over keys [0, Pb), Pb = min(prefix_keys, Lk), in
// chunks of prefix_chunk keys (one or two whole cache blocks). Work-group (chunk c, kv head g,
// z) serves window z / R of MC = kPrefillRows / G consecutive sequences, as replica z % R. The
// window's sequences whose block tables name the same blocks for the chunk, and that hold the
// same number of keys in it, form a group -- with prefix caching, the sequences sharing those
// blocks; replica r takes the window's groups r, r + R, ... A group's query rows (members x
// the G heads of g) form one MFMA tile set, so each shared block is read once per window
// instead of once per sequence. Every row gets the chunk's (max, sum, numerator) partial in
// the chunk's slot of its sequence, merged with the sequence's split partials by the decode
// combine. A row's arithmetic does not depend on which other rows share its tiles, so results
// do not depend on the grouping (shared or duplicated blocks give identical bits) nor on the
// order of the members inside a group.
//
// The grouping runs in each work-group, on its own window (no plan launch, no plan in memory):
// thread t < MC holds sequence s0 + t's key (keys held in the chunk, its block ids), inserts it
// into an LDS hash table and counts itself into its entry; a group's lead is its lowest
// sequence (an atomic minimum: the same in every replica), and the groups are numbered by their
// leads in sequence order, so all replicas of a window see the same group list. Member ranks
// come from an atomic counter; they only place the rows inside the work-group's own tiles.
template <int G>
__device__ __forceinline__ void shared_prefix_work(const AttnArgs& a, const int c, const int g, const int z) {
  static_assert(kRowBlocks == 1, "one 32-row block per wavefront");
  constexpr int D = kHeadDim;
  constexpr int MC = kPrefillRows / G;  // sequences per window (and rows of one head per tile set)
  constexpr int kHash = 2 * MC;         // hash entries: more than keys, so probing ends
  static_assert(MC <= kPrefillThreads, "one thread per window sequence");
  __shared__ __attribute__((aligned(1024))) char sK[2][kTileBytes];
  __shared__ __attribute__((aligned(1024))) char sV[2][kTileBytes];
  __shared__ int4 s_key[MC];   // (keys held in the chunk, block id, second block id or -1, query row)
  __shared__ int s_owner[kHash], s_lead[kHash], s_size[kHash];
  __shared__ int2 s_group[MC];  // group k: (lead, members)
  __shared__ int s_wave_leads[kPrefillWaves];
  __shared__ int2 s_mem[MC];    // (sequence, query row) of the current group's members
  lds_char* KS[2] = {(lds_char*)sK[0], (lds_char*)sK[1]};
  lds_char* VS[2] = {(lds_char*)sV[0], (lds_char*)sV[1]};

  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int BS = a.block_size;
  const int CK = a.prefix_chunk;
  const int Cb = CK / BS;
  const int S = a.num_seqs;
  // work-group (chunk c, kv head g, z = window x replicas + replica)
  const int nrep = a.sp_replicas;
  const int win = z / nrep;
  const int rep = z - win * nrep;
  const int s0 = win * MC;
  const int nwin = min(MC, S - s0);

  // the window's bounds and block-table entries for the chunk in one round of loads (the
  // entries, clamped into the table row, are used only for a sequence holding keys in the
  // chunk, whose entries are valid)
  int4 key = make_int4(0, -1, -1, 0);
  if (tid < nwin) {
    const int b = s0 + tid;
    const int32_t* bt = a.block_table + (int64_t)b * a.bt_stride;
    const int q0 = a.cu_q[b], q1 = a.cu_q[b + 1];
    const int k_lo = a.cu_k[b], k_hi = a.cu_k[b + 1];
    const int id0 = bt[min(c * Cb, a.bt_stride - 1)];
    const int id1 = Cb > 1 ? bt[min(c * Cb + 1, a.bt_stride - 1)] : -1;
    const int Lk = min(k_hi - k_lo, a.max_seqlen_k);
    const int cnt = q1 - q0 == 1 ? max(0, min(CK, min(a.prefix_keys, Lk) - c * CK)) : 0;  // decode rows only
    if (cnt > 0) key = make_int4(cnt, id0, cnt > BS ? id1 : -1, q0);
  }
  if (tid < MC) s_key[tid] = key;
  for (int e = tid; e < kHash; e += kPrefillThreads) {
    s_owner[e] = -1;
    s_lead[e] = MC;
    s_size[e] = 0;
  }
  __syncthreads();
  int slot = -1, rank = 0;
  if (key.x > 0) {
    int h = (int)(((uint32_t)key.y * 2654435761u + (uint32_t)key.z * 40503u) >> 16) & (kHash - 1);
    for (int probe = 0; probe < kHash; ++probe, h = (h + 1) & (kHash - 1)) {
      const int e = atomicCAS(&s_owner[h], -1, tid);
      const int4 k2 = e == -1 ? key : s_key[e];
      if (k2.x == key.x && k2.y == key.y && k2.z == key.z) {
        slot = h;
        break;
      }
    }
    if (slot >= 0) {
      atomicMin(&s_lead[slot], tid);
      rank = atomicAdd(&s_size[slot], 1);
    }
  }
  __syncthreads();
  const int my_lead = slot >= 0 ? s_lead[slot] : -1;
  // group number of a lead: leads below it, in sequence order (ballots per wavefront)
  const bool is_lead = my_lead == tid;
  const uint64_t lead_bits = __builtin_amdgcn_ballot_w64(is_lead);
  if (lane == 0) s_wave_leads[wave] = __builtin_popcountll(lead_bits);
  __syncthreads();
  int before = __builtin_popcountll(lead_bits & ((1ull << lane) - 1ull)), ngroups = 0;
#pragma unroll
  for (int w = 0; w < kPrefillWaves; ++w) {
    const int n = s_wave_leads[w];
    before += w < wave ? n : 0;
    ngroups += n;
  }
  if (is_lead) s_group[before] = make_int2(tid, s_size[slot]);
  __syncthreads();

  const TileLanes tl = tile_lanes(lane);
  const int col = lane & 31;
  const int half = lane >> 5;

  for (int k = rep; k < ngroups; k += nrep) {
    const int2 grp = s_group[k];
    const int4 gkey = s_key[grp.x];
    const int nmem = grp.y;
    const int cnt = gkey.x;
    const int id0 = gkey.y, id1 = gkey.z >= 0 ? gkey.z : gkey.y;
    // tile n: keys 64 n .. of the chunk, in its block (64 n) / BS; rows past cnt re-read the
    // chunk's last key (same block) and are masked
    const auto load = [&](int n, KvRegs& R) {
      const int t0 = n * kTileKeys;
      const int id = t0 < BS ? id0 : id1;
      const int off = t0 % BS;
      const uint16_t* kbase = a.k + (int64_t)id * a.k_block_stride + (int64_t)off * a.k_row_stride + g * D;
      const uint16_t* vbase = a.v + (int64_t)id * a.v_block_stride + (int64_t)off * a.v_row_stride + g * D;
      load_rows(kbase, vbase, load_lanes(a, wave, lane, min(kTileKeys, cnt - 1 - t0)), R);
    };
    // the first two tiles are requested before the members and their q rows (which depend
    // on the member list), so the three rounds of loads overlap
    const int ntiles = (cnt + kTileKeys - 1) / kTileKeys;
    KvRegs R0, R;
    load(0, R0);
    if (ntiles > 1) load(1, R);
    // LDS-only barriers: __syncthreads() would also wait for the tile loads just issued
    lds_barrier();  // s_mem of the previous group has been read
    if (my_lead == grp.x) s_mem[rank] = make_int2(s0 + tid, key.w);
    lds_barrier();

    // rows: 32 per wavefront; TMd = members rounded up to 32 rows per head, head i = row / TMd
    const int TMd = (nmem + 31) & ~31;
    const bool active = wave * 32 < G * TMd;
    const int r0 = wave * 32;
    const int hi = active ? r0 / TMd : 0;
    const int mem = active ? r0 % TMd + col : 0;
    const int2 sm = s_mem[min(mem, nmem - 1)];  // rows past the members read the last one's q
    const int seq = min(max(sm.x, 0), a.num_seqs - 1);
    const int h = g * G + hi;
    bf16x8 qb[kRowBlocks][D / 16];
    {
      const uint16_t* qp = a.q + (int64_t)max(sm.y, 0) * a.q_row_stride + h * D + 8 * half;
#pragma unroll
      for (int kb = 0; kb < D / 16; ++kb)
        qb[0][kb] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(qp + kb * 16));
    }
    f32x16 o[kRowBlocks][4];
    float m_i[kRowBlocks] = {-INFINITY}, l_i[kRowBlocks] = {0.f};
    const int lim[kRowBlocks] = {cnt - 1};  // every member holds the chunk's cnt keys
#pragma unroll
    for (int md = 0; md < 4; ++md)
#pragma unroll
      for (int rr = 0; rr < 16; ++rr) o[0][md][rr] = 0.f;

    store_tile_lds(R0, KS[0], VS[0], wave, lane);
    lds_barrier();
    for (int n0 = 0; n0 < ntiles; n0 += 2) {
#pragma unroll
      for (int st = 0; st < 2; ++st) {
        const int n = n0 + st;
        if (n >= ntiles) break;
        const int t0 = n * kTileKeys;
        KvRegs Rn;
        if (n + 2 < ntiles) load(n + 2, Rn);
        const bool full[kRowBlocks] = {t0 + kTileKeys - 1 <= lim[0]};
        if (active) compute_tile(KS[st], VS[st], tl, qb, o, m_i, l_i, t0, lim, full, a.scale_log2, lane);
        if (n + 1 < ntiles) store_tile_lds(R, KS[st ^ 1], VS[st ^ 1], wave, lane);
        lds_barrier();
        R = Rn;
      }
    }

    // partial of (member, head h) for chunk c, in the decode kernel's layout: the normalised
    // output o / l in bf16 and (max, sum); O^T element rr of d-block md is
    // d = 32 md + 8 (rr >> 2) + 4 half + (rr & 3), i.e. four consecutive elements
    const float l_tot = swap_halves_sum(l_i[0]);
    if (active && mem < nmem) {
      const int64_t unit = ((int64_t)seq * a.prefix_stride + c) * a.num_heads + h;
      uint16_t* po = a.part_o + unit * D + 4 * half;
      const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
#pragma unroll
      for (int md = 0; md < 4; ++md)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          uint2 w;
          w.x = pack_bf16x2(o[0][md][4 * q] * inv, o[0][md][4 * q + 1] * inv);
          w.y = pack_bf16x2(o[0][md][4 * q + 2] * inv, o[0][md][4 * q + 3] * inv);
          *reinterpret_cast<uint2*>(po + 32 * md + 8 * q) = w;
        }
      if (half == 0) *reinterpret_cast<float2*>(a.part_ml + unit * 2) = make_float2(m_i[0], l_tot);
    }
  }
}

// grid (chunk, kv head, window x replicas): work-groups go to the XCDs round-robin by linear
// id, so with z slowest the first replica of every (chunk, head) spreads over all of them
template <int G>
__global__ __launch_bounds__(kPrefillThreads, kWavesPerSimd) void shared_prefix_kernel(const AttnArgs a) {
  shared_prefix_work<G>(a, blockIdx.x, blockIdx.y, blockIdx.z);
}

// The shared-prefix work and the flat decode grid over the keys after the prefix in one
// launch. Run back to back, the prefix kernel -- a chain of dependent steps in a few dozen
// work-groups (bounds, grouping, member list, q rows, tiles, partials), most of the GPU idle
// -- and the flat grid, which streams the suffixes on every CU, add up; here the first
// sp_groups work-groups take the prefix work (one replica per window) and then sp_tail flat
// groups each, and the sp_decode work-groups after them sp_per flat groups each, as many as
// the CUs left beside the prefix work hold at once. The two kinds write disjoint partial slots
// (prefix chunks, then the flat pieces), merged by the combine pass as before. A work-group's
// eight wavefronts take its flat groups sp_quads at a time (one flat group = the kv heads of
// sp_quads wavefronts); the flat grid's groups are numbered across the work-groups.
template <int G, int U, int R>
__global__ __launch_bounds__(kPrefillThreads, kWavesPerSimd) void shared_prefix_flat_kernel(const AttnArgs a) {
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int blk = blockIdx.x;
  int first, count;  // this work-group's flat groups
  if (blk < a.sp_groups) {
    const int c = blk % a.prefix_slots;
    const int rest = blk / a.prefix_slots;
    shared_prefix_work<G>(a, c, rest % a.num_kv_heads, rest / a.num_kv_heads);
    first = a.sp_decode * a.sp_per + blk * a.sp_tail;
    count = a.sp_tail;
  } else {
    first = (blk - a.sp_groups) * a.sp_per;
    count = a.sp_per;
  }
  const int j = wave / a.sp_quads;  // this wavefront's flat group, and its kv-head quad in it
  const int qd = wave - j * a.sp_quads;
  const int u = first + j;
  if (j < count && u <= a.flat_groups + a.num_seqs)
    flat_decode_piece<G, U, R, true, false, true>(a, u, qd * (4 / R), lane, qd == 0);
}


int device_prefill_slots() {
  static int cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return kPrefillSlotsMax;
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = kPrefillSlotsMax;
    cached[dev] = std::min(cus, kPrefillSlotsMax);  // one work-group per CU
  }
  return cached[dev];
}

template <int G, bool PAGED, bool CAUSAL>
hipError_t launch_prefill_gpc(const AttnArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((prefill_plan_kernel<G, CAUSAL>), dim3(1), dim3(kPlanThreads), 0, stream, a);
  hipLaunchKernelGGL((prefill_kernel<G, PAGED, CAUSAL>), dim3(a.pf_slots), dim3(kPrefillThreads), 0, stream, a);
  hipLaunchKernelGGL((prefill_merge_kernel<G>), dim3(kMergeGroups), dim3(kMergeThreads), 0, stream, a);
  return hipGetLastError();
}

template <int G>
hipError_t launch_prefill_g(const AttnArgs& a, bool paged, bool causal, int max_seqlen_q, hipStream_t stream) {
  constexpr int TM = kPrefillRows / G;
  AttnArgs pa = a;
  pa.prefill_qtiles = (max_seqlen_q + TM - 1) / TM;
  pa.pf_slots = device_prefill_slots();
  pa.flat_step = decode_flat_step(G, a.num_kv_heads);  // the decode pieces' step, for the merge kernel's combines
  if (paged)
    return causal ? launch_prefill_gpc<G, true, true>(pa, stream) : launch_prefill_gpc<G, true, false>(pa, stream);
  return causal ? launch_prefill_gpc<G, false, true>(pa, stream) : launch_prefill_gpc<G, false, false>(pa, stream);
}

}  // namespace

template <int G>
void launch_shared_prefix_g(AttnArgs a, hipStream_t stream) {
  // grid (chunk, kv head, window x replicas): windows of kPrefillRows / G sequences, and
  // replicas taking a window's groups in turn, as many as keep the grid near two work-groups
  // per CU (a window usually holds one group per chunk; the spare replicas exit after the
  // grouping)
  constexpr int MC = kPrefillRows / G;
  const int windows = (a.num_seqs + MC - 1) / MC;
  const int pool = 2 * device_prefill_slots();
  a.sp_replicas = std::max(1, std::min(MC, pool / std::max(1, a.prefix_slots * a.num_kv_heads * windows)));
  hipLaunchKernelGGL(shared_prefix_kernel<G>,
                     dim3((unsigned)a.prefix_slots, (unsigned)a.num_kv_heads, (unsigned)(windows * a.sp_replicas)),
                     dim3(kPrefillThreads), 0, stream, a);
}

template <int G, int U, int R>
void launch_shared_prefix_flat_g(const AttnArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((shared_prefix_flat_kernel<G, U, R>), dim3((unsigned)(a.sp_groups + a.sp_decode)),
                     dim3(kPrefillThreads), 0, stream, a);
}

template <int G>
void launch_shared_prefix_flat_gr(const AttnArgs& a, hipStream_t stream) {
  constexpr int U = decode_step_keys(G);
  switch (decode_key_rows(a.num_kv_heads)) {
    case 4: launch_shared_prefix_flat_g<G, U, 4>(a, stream); break;
    case 2: launch_shared_prefix_flat_g<G, U, 2>(a, stream); break;
    default: launch_shared_prefix_flat_g<G, U, 1>(a, stream); break;
  }
}

bool launch_shared_prefix_flat(AttnArgs& a, int group, hipStream_t stream, hipError_t* err) {
  *err = hipSuccess;
  if (a.num_seqs <= 0 || a.prefix_keys <= 0 || a.prefix_slots <= 0 || a.flat_groups <= 0) return false;
  if (!a.block_table || !a.part_o || !a.part_ml || a.num_seqs > kSharedPrefixMaxSeqs ||
      a.prefix_chunk % a.block_size != 0 || a.prefix_chunk / a.block_size > kSharedPrefixMaxChunkBlocks ||
      a.prefix_slots > kCombineMaxSplits)
    return false;
  const int nh = 4 / decode_key_rows(a.num_kv_heads);           // kv heads per wavefront
  const int quads = (a.num_kv_heads + nh - 1) / nh;              // wavefronts per flat group
  if (kPrefillWaves % quads != 0) return false;
  const int per = kPrefillWaves / quads;                         // flat groups per work-group
  const int MC = kPrefillRows / group;
  const int windows = (a.num_seqs + MC - 1) / MC;
  const int64_t P = (int64_t)a.prefix_slots * a.num_kv_heads * windows;
  const int cus = device_prefill_slots();                        // one work-group per CU
  if (P >= cus / 2) return false;                                // little room left for the suffixes
  // decode work-groups fill the CUs beside the prefix ones; those take half a share after
  // their prefix work. The flat grid shrinks to the groups these hold (never grows: the
  // workspace's partial slots are sized for the flat plan's grid).
#ifndef PK_SP_TAIL_DIV
#define PK_SP_TAIL_DIV 2
#endif
  const int tail = PK_SP_TAIL_DIV > 0 ? per / PK_SP_TAIL_DIV : 0;
  const int D = cus - (int)P;
  const int64_t total = (int64_t)D * per + P * tail;             // flat groups, recorder included
  const int W = (int)std::min<int64_t>(a.flat_groups, total - a.num_seqs - 1);
  if (W < 2) return false;
  a.flat_groups = W;
  a.sp_replicas = 1;
  a.sp_groups = (int)P;
  a.sp_decode = D;
  a.sp_per = per;
  a.sp_tail = tail;
  a.sp_quads = quads;
  a.flat_step = decode_flat_step(group, a.num_kv_heads);
  // the decode launch's partial-store policy (kStoreThroughBytes), on this grid's units
  a.store_through = ((int64_t)a.num_seqs + a.flat_groups) * a.num_heads * kHeadDim * 4 > kStoreThroughBytes;
  switch (group) {
    case 1: launch_shared_prefix_flat_gr<1>(a, stream); break;
    case 2: launch_shared_prefix_flat_gr<2>(a, stream); break;
    case 4: launch_shared_prefix_flat_gr<4>(a, stream); break;
    case 8: launch_shared_prefix_flat_gr<8>(a, stream); break;
    default: *err = hipErrorInvalidValue; return true;
  }
  *err = hipGetLastError();
  return true;
}

hipError_t launch_shared_prefix(const AttnArgs& a, int group, hipStream_t stream) {
  if (a.num_seqs <= 0 || a.prefix_keys <= 0 || a.prefix_slots <= 0) return hipSuccess;
  if (!a.block_table || !a.part_o || !a.part_ml || a.num_seqs > kSharedPrefixMaxSeqs ||
      a.prefix_chunk % a.block_size != 0 || a.prefix_chunk / a.block_size > kSharedPrefixMaxChunkBlocks ||
      a.prefix_slots > kCombineMaxSplits)
    return hipErrorInvalidValue;
  switch (group) {
    case 1: launch_shared_prefix_g<1>(a, stream); break;
    case 2: launch_shared_prefix_g<2>(a, stream); break;
    case 4: launch_shared_prefix_g<4>(a, stream); break;
    case 8: launch_shared_prefix_g<8>(a, stream); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_prefill(const AttnArgs& a, int group, bool paged, bool causal, int max_seqlen_q,
                          hipStream_t stream) {
  if (a.num_seqs <= 0 || max_seqlen_q <= 1) return hipSuccess;
  if (!a.pf_queue || !a.pf_items || !a.pf_merges || !a.pf_part_o || !a.pf_part_ml) return hipErrorInvalidValue;
  switch (group) {
    case 1: return launch_prefill_g<1>(a, paged, causal, max_seqlen_q, stream);
    case 2: return launch_prefill_g<2>(a, paged, causal, max_seqlen_q, stream);
    case 4: return launch_prefill_g<4>(a, paged, causal, max_seqlen_q, stream);
    case 8: return launch_prefill_g<8>(a, paged, causal, max_seqlen_q, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pk
