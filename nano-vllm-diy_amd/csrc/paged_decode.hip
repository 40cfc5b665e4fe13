// Split-K paged decode attention for gfx950 (one query row per sequence).
//
// Reference semantics: flash_attn_varlen_func with max_seqlen_q == 1 and a block
// table (src/layers/attention.py:95-104, replayed inside the decode graph,
// src/engine/model_runner.py:245-259). For sequence b and query head h:
//     o = softmax(scale * q . K_b^T) V_b,   K_b[t] = k_cache[bt[b][t / BS], t % BS, h / G]
// over all Lk keys (a single bottom-right-aligned causal row sees every key).
//
// Work decomposition
//   grid = (split, sequence, group of kv heads); a work-group handles one split of
//   `split_tokens` keys of one sequence for up to 16 kv heads (4 per wavefront), and every
//   K/V row it reads serves all G query heads of its kv head (GQA reuse in registers).
//   Sequences with one split write their output directly; longer ones leave per-split
//   (max, sum, numerator) partials in the workspace that a small combine kernel merges.
//
// Lane layout: lane = 16 hr + c. DPP row hr holds kv head 4 w + hr of wavefront w and
// lane c holds head_dim elements [8c, 8c + 8). One dwordx4 load instruction therefore
// reads one key's 4 heads = 1 KiB of a contiguous cache row (the two wavefronts of an
// 8-kv-head group read the whole 2 KiB row), the friendliest pattern for HBM.
//   * q.k: 4 v_dot2_f32_bf16 per (key, query head) on bf16 pairs, then a 4-step DPP sum
//     across the 16-lane row; every lane of the row ends with the key's full score.
//   * softmax: keys of a step are lane-local, so the running max needs no shuffles.
//   * P.V: p rounded to bf16 and paired across two keys, one dot2 per (head, element).
// Loads are software-pipelined two steps deep and all issued before the step's math.
#include <algorithm>
#include <type_traits>

#include "norm_rope.h"

namespace pk {
namespace {

// Build-time tunables (defaults are the measured best on MI355X).
#ifndef PK_DECODE_WAVES
#define PK_DECODE_WAVES 4       // max wavefronts (4 kv heads each) per work-group
#endif
#ifndef PK_DECODE_STEP_G2
#define PK_DECODE_STEP_G2 8     // keys per pipeline step for GQA groups <= 2
#endif
#ifndef PK_DECODE_SPLIT_MAX
#define PK_DECODE_SPLIT_MAX 512 // keys per work unit (split) when the batch is large
#endif
#ifndef PK_DECODE_MIN_GROUPS
#define PK_DECODE_MIN_GROUPS 2048  // work-groups a batch's grid aims for before splits stop shrinking
#endif
#ifndef PK_DECODE_MIN_SPLIT
#define PK_DECODE_MIN_SPLIT 64     // shortest split (keys) the sizing goes down to
#endif
// Flat decode grid (below): used for batches of at most PK_DECODE_FLAT_MAX_SEQS sequences
// whose launch bound (num_seqs x max_seqlen_k) holds at least PK_DECODE_FLAT_MIN_KEYS keys.
// Measured (us, split grid vs flat grid of 1024 work-groups, cold caches): 128 sequences of
// 100-1024 keys 69.5 vs 64.7, of 100-2048 108.7 vs 98.2; 64 of 100-2048 68.0 vs 60.2; 32 of
// 100-4096 66.8 vs 59.0; 16 of 1024-8192 80.5 vs 73.3; the 128 decodes of the mixed
// chunked-prefill batch 222 vs 209. The split grid stays ahead for 256 sequences (100-2048
// keys 213 vs 218; 1024-8192 keys 781 vs 789 with 1536 work-groups) and for 8 sequences of
// 256-2048 keys (18.8 vs 21.8: too few keys to pay for the flat prologue's extra round trip).
// Flat grids of 512, 768 and 1280 work-groups were each slower on most of these batches.
#ifndef PK_DECODE_FLAT_MAX_SEQS
#define PK_DECODE_FLAT_MAX_SEQS 192
#endif
#ifndef PK_DECODE_FLAT_MIN_KEYS
#define PK_DECODE_FLAT_MIN_KEYS 32768
#endif
#ifndef PK_DECODE_FLAT_GROUPS
#define PK_DECODE_FLAT_GROUPS 1024   // work-groups (runs + sequences) a flat decode launch aims for
#endif
#ifndef PK_DECODE_FLAT_MIN_CHUNK
#define PK_DECODE_FLAT_MIN_CHUNK 32  // shortest run of keys per flat work-group
#endif

constexpr int kDecodeMaxWaves = PK_DECODE_WAVES;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
constexpr int kStoreThrough = 16;  // buffer cache policy bit sc1: write through L2
// Partial footprint (launch bound: sequences x splits x heads x D x 4 bytes) above which the
// partials are written through L2. The eight XCD L2s hold 32 MB together: smaller partial
// sets stay there, dirty, until the kernel ends; larger ones get evicted in the middle of the
// K/V read stream, where write-back traffic is the costlier (measured: 256 sequences of
// 1k-8k keys, 33.5 MB bound, 0.800 -> 0.778 ms with write-through; 128 sequences, 16.8 MB
// bound, 114 -> 117 us; 128 sequences of 512-4096 keys, 221 -> 226 us).
constexpr int64_t kStoreThroughBytes = 24ll << 20;

// A unit's partial: its normalised output o / l in bf16 (as precise as an unsplit row's
// output, and half the bytes of fp32 numerators: writes that land in the middle of the K/V
// read stream cost far more than reads) and (max in the exp2 domain, sum) in fp32.
template <int AUX>
__device__ __forceinline__ void store_partial(const __amdgpu_buffer_rsrc_t& po_rs, const __amdgpu_buffer_rsrc_t& pml_rs,
                                              int o, int ml_off, const uint4& w, const f32x2& ml, bool with_ml) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, w), po_rs, o, 0, AUX);
  if (with_ml) __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, ml), pml_rs, ml_off, 0, AUX);
}

// Buffer resource over [base, base + bytes): raw addressing (stride 0), 32-bit dword format.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 16 bytes at base + row_off + lane_off: row_off is wave-uniform (scalar offset operand),
// lane_off is the lane's column (one VGPR shared by every load of the step). STREAM sets the
// non-temporal policy.
template <bool STREAM>
__device__ __forceinline__ u32x4 load16(__amdgpu_buffer_rsrc_t r, uint32_t lane_off, uint32_t row_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, (int)lane_off, (int)row_off, STREAM ? 2 : 0);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

// a.x * b.x + a.y * b.y + c on packed bf16 pairs, fp32 accumulate (v_dot2_f32_bf16).
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

// Per-lane softmax state of one work unit.
template <int G>
struct DecodeState {
  uint32_t qp[G][4];  // q in bf16 pairs (this lane's 8 elements of each query head)
  float m[G];         // running max of the unscaled scores
  float l[G];         // running softmax denominator
  float acc[G][8];    // running P.V numerator (this lane's 8 elements)
};

// Issue the K then V loads of keys [t, t + U) of this lane's kv head. lane_bytes is the
// lane's byte offset inside a token row. Keys past t_end re-read the step's last valid
// row (same cache block, finite data) and consume() masks them to p = 0, so no load
// needs a branch. The loads are buffer loads over the step's U rows: the row offsets are
// wave-uniform scalar operands and every load shares the lane-offset VGPR. (With
// global loads each load needs its own vector address register, and at this kernel's
// register pressure the compiler took those from the destinations of the previous step's
// in-flight loads: the write-after-write wait then drained the pipeline every other step.)
// STREAM selects non-temporal loads; it is a template parameter (not a runtime branch)
// so the pipelined loop stays straight-line and its wait counts stay exact.
// Block id of entry j of a (wave-uniform) block-table row, as a scalar load. The fused
// decode step stores K/V rows before its loop, after which the compiler can no longer prove
// the table unchanged: a plain load would become a vector load whose value the compiler
// treats as divergent, and every buffer load built on it would run in a waterfall loop.
__device__ __forceinline__ int scalar_block_id(const int32_t* row, int j) {
  int v;
  asm volatile("s_load_dword %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(row), "s"(j * 4));
  return v;
}

template <int U, bool PAGED, bool STREAM, bool FUSED>
__device__ __forceinline__ void issue_loads(const AttnArgs& a, uint32_t lane_bytes, int b, int k0, int t,
                                            int t_end, u32x4 (&kr)[U], u32x4 (&vr)[U]) {
  const uint16_t* kp;
  const uint16_t* vp;
  if constexpr (PAGED) {
    // [t, t + U) lies inside one cache block: U divides block_size and split_tokens.
    const int blk = FUSED ? scalar_block_id(a.block_table + (int64_t)b * a.bt_stride, t / a.block_size)
                          : a.block_table[(int64_t)b * a.bt_stride + t / a.block_size];
    const int off = t % a.block_size;
    kp = a.k + (int64_t)blk * a.k_block_stride + (int64_t)off * a.k_row_stride;
    vp = a.v + (int64_t)blk * a.v_block_stride + (int64_t)off * a.v_row_stride;
  } else {
    kp = a.k + (int64_t)(k0 + t) * a.k_row_stride;
    vp = a.v + (int64_t)(k0 + t) * a.v_row_stride;
  }
  // row strides are < 2^22 elements (checked on the host), so U rows span < 2^27 bytes
  const uint32_t k_row_bytes = (uint32_t)a.k_row_stride * 2u;
  const uint32_t v_row_bytes = (uint32_t)a.v_row_stride * 2u;
  const __amdgpu_buffer_rsrc_t kr_rs = row_rsrc(kp, (uint32_t)U * k_row_bytes);
  const __amdgpu_buffer_rsrc_t vr_rs = row_rsrc(vp, (uint32_t)U * v_row_bytes);
  const int last = t_end - 1 - t;
#pragma unroll
  for (int u = 0; u < U; ++u) kr[u] = load16<STREAM>(kr_rs, lane_bytes, __umul24((uint32_t)min(u, last), k_row_bytes));
#pragma unroll
  for (int u = 0; u < U; ++u) vr[u] = load16<STREAM>(vr_rs, lane_bytes, __umul24((uint32_t)min(u, last), v_row_bytes));
}

// Keys [t_begin, t_end) of one split through a two-stage software pipeline: the loads of
// step n+1 are in flight while step n is consumed. The prefetch is unconditional (past
// t_end it re-reads the current step, which hits in cache) so the code is straight-line
// and the wait counts stay exact. The scheduling barriers keep each step's loads together
// ahead of its math: otherwise the scheduler sinks every load next to its first use to
// save registers, which serialises their latency.
template <int G, int U, bool PAGED, bool STREAM, bool FUSED, class Pre>
__device__ __forceinline__ void decode_range(DecodeState<G>& st, const AttnArgs& a, uint32_t lane_bytes, int b,
                                             int k0, int t_begin, int t_end, Pre&& pre);

// Fold keys [t, t + U) (already loaded) into the running softmax state.
template <int G, int U>
__device__ __forceinline__ void consume(DecodeState<G>& st, float c2, int t, int t_end, const u32x4 (&kr)[U],
                                        const u32x4 (&vr)[U]) {
  // unscaled scores: 4 dot2 per (key, head) over this lane's 8 elements, then the
  // 16-lane DPP sum gives every lane of the row the full q.k of its key.
  float s[U][G];
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int i = 0; i < G; ++i) {
      float d0 = dot2(st.qp[i][0], kr[u].x, 0.f);
      d0 = dot2(st.qp[i][1], kr[u].y, d0);
      d0 = dot2(st.qp[i][2], kr[u].z, d0);
      d0 = dot2(st.qp[i][3], kr[u].w, d0);
      s[u][i] = row16_sum(d0);
    }
    if (t + u >= t_end) {
#pragma unroll
      for (int i = 0; i < G; ++i) s[u][i] = -INFINITY;
    }
  }

  // online softmax in the exp2 domain; p is rounded to bf16 for the P.V dot2 (the
  // same rounding a bf16 P.V matrix product applies), l sums the fp32 p.
  uint32_t pk[U / 2][G];
#pragma unroll
  for (int i = 0; i < G; ++i) {
    float mx = s[0][i];
#pragma unroll
    for (int u = 1; u < U; ++u) mx = fmaxf(mx, s[u][i]);
    const float m_new = fmaxf(st.m[i], mx);  // finite: the step holds >= 1 valid key
    const float alpha = exp2_fast((st.m[i] - m_new) * c2);
    st.m[i] = m_new;
    const float ms = m_new * c2;
    st.l[i] *= alpha;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[i][e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; u += 2) {
      const float p0 = exp2_fast(fmaf(s[u][i], c2, -ms));
      const float p1 = exp2_fast(fmaf(s[u + 1][i], c2, -ms));
      st.l[i] += p0 + p1;
      pk[u / 2][i] = pack_bf16x2(p0, p1);
    }
  }

  // P.V on key pairs (u, u+1): v_perm builds (v_u[e], v_u+1[e]) bf16 pairs shared by
  // the G heads, one dot2 per (head, element) adds both keys.
#pragma unroll
  for (int u = 0; u < U; u += 2) {
    const uint32_t va[4] = {vr[u].x, vr[u].y, vr[u].z, vr[u].w};
    const uint32_t vb[4] = {vr[u + 1].x, vr[u + 1].y, vr[u + 1].z, vr[u + 1].w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t lo = __builtin_amdgcn_perm(vb[j], va[j], 0x05040100u);  // elements 2j
      const uint32_t hi = __builtin_amdgcn_perm(vb[j], va[j], 0x07060302u);  // elements 2j+1
#pragma unroll
      for (int i = 0; i < G; ++i) {
        st.acc[i][2 * j] = dot2(pk[u / 2][i], lo, st.acc[i][2 * j]);
        st.acc[i][2 * j + 1] = dot2(pk[u / 2][i], hi, st.acc[i][2 * j + 1]);
      }
    }
  }
}

template <int G, int U, bool PAGED, bool STREAM, bool FUSED, class Pre>
__device__ __forceinline__ void decode_range(DecodeState<G>& st, const AttnArgs& a, uint32_t lane_bytes, int b,
                                             int k0, int t_begin, int t_end, Pre&& pre) {
  const float c2 = a.scale_log2;
  u32x4 kA[U], vA[U], kB[U], vB[U];
  issue_loads<U, PAGED, STREAM, FUSED>(a, lane_bytes, b, k0, t_begin, t_end, kA, vA);
  pre();  // q (loaded or computed) while the first K/V loads are in flight
  for (int t = t_begin; t < t_end; t += 2 * U) {
    const int t1 = t + U;
    issue_loads<U, PAGED, STREAM, FUSED>(a, lane_bytes, b, k0, t1 < t_end ? t1 : t, t_end, kB, vB);
    __builtin_amdgcn_sched_barrier(0);
    consume<G, U>(st, c2, t, t_end, kA, vA);
    if (t1 >= t_end) break;
    const int t2 = t1 + U;
    issue_loads<U, PAGED, STREAM, FUSED>(a, lane_bytes, b, k0, t2 < t_end ? t2 : t1, t_end, kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    consume<G, U>(st, c2, t1, t_end, kB, vB);
  }
}

// Fused decode step: q of this DPP row's kv head g (its G query heads) is the RMSNorm +
// RoPE of the token's fused qkv row, computed here exactly as the producer kernel computes
// it (norm_rope.h) -- or, for the fused store + decode, q as given. The split holding the
// sequence's last key -- the token itself, which attends to its own key (attention.py:87-88
// stores before attending) -- first writes the token's K row (normalised + rotated from qkv,
// or as given) and V row of kv head g into the cache slot, and
// waits for those stores before any K/V load: the same wavefront reads that row back in
// its last pipeline step, and no other work-group reads it. The slot must be the cache
// position of the sequence's last key (as the runner builds slot_mapping, model_runner.py:
// 200-210).
template <int G>
__device__ __forceinline__ void fused_producer(const AttnArgs& a, DecodeState<G>& st, int q0, int g, int c,
                                               bool row_live, bool stores_token) {
  constexpr int D = kHeadDim;
  int32_t slot = -1;
  uint4 wk, wv;
  if (stores_token) {
    slot = a.slot_mapping[q0];
    if (slot < 0 || (a.num_slots > 0 && (int64_t)slot >= a.num_slots)) slot = -1;
  }
  if (a.qkv != nullptr) {
    const bool lower = c < kLanesPerRow / 2;
    float cv[8], sv[8];
    rope_cos_sin_row(a.cos_sin, a.max_position, a.positions[q0], c, cv, sv);
    const uint16_t* row = a.qkv + (int64_t)q0 * a.qkv_row_stride + c * 8;
    uint4 w[G];
#pragma unroll
    for (int i = 0; i < G; ++i) w[i] = *reinterpret_cast<const uint4*>(row + (g * G + i) * D);
    if (stores_token) {
      wk = *reinterpret_cast<const uint4*>(row + (a.num_heads + g) * D);
      wv = *reinterpret_cast<const uint4*>(row + (a.num_heads + a.num_kv_heads + g) * D);
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const uint4 o = norm_rope_row(w[i], a.q_norm, a.norm_eps, cv, sv, lower, c);
      st.qp[i][0] = o.x;
      st.qp[i][1] = o.y;
      st.qp[i][2] = o.z;
      st.qp[i][3] = o.w;
    }
    if (slot >= 0) wk = norm_rope_row(wk, a.k_norm, a.norm_eps, cv, sv, lower, c);
  } else {  // store + decode: q as given, the raw K / V rows of the token (attention.py:27-34)
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const uint4 w = *reinterpret_cast<const uint4*>(a.q + (int64_t)q0 * a.q_row_stride + (g * G + i) * D + c * 8);
      st.qp[i][0] = w.x;
      st.qp[i][1] = w.y;
      st.qp[i][2] = w.z;
      st.qp[i][3] = w.w;
    }
    if (slot >= 0) {
      wk = *reinterpret_cast<const uint4*>(a.new_k + (int64_t)q0 * a.new_k_stride + g * D + c * 8);
      wv = *reinterpret_cast<const uint4*>(a.new_v + (int64_t)q0 * a.new_v_stride + g * D + c * 8);
    }
  }
  if (slot >= 0) {  // uniform over the work-group: one token per sequence
    if (row_live) {
      const int64_t blk = slot / a.block_size, off = slot - blk * a.block_size;
      uint16_t* kd = const_cast<uint16_t*>(a.k) + blk * a.k_block_stride + off * a.k_row_stride + g * D + c * 8;
      uint16_t* vd = const_cast<uint16_t*>(a.v) + blk * a.v_block_stride + off * a.v_row_stride + g * D + c * 8;
      *reinterpret_cast<uint4*>(kd) = wk;
      *reinterpret_cast<uint4*>(vd) = wv;
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the stores are done; no load moves above
  }
}

// One work unit: keys [t_begin, t_end) of decode sequence b (query row q0, keys from k0 in
// flat mode, Lk keys in all) for the kv heads of this wavefront. direct: the unit holds every
// key of the sequence, so it normalises and writes the output row itself; otherwise it
// leaves its (max, sum, numerator) partial at partial unit unit0 (x num_heads) for the combine.
template <int G, int U, bool PAGED, bool FUSED>
__device__ __forceinline__ void decode_unit(const AttnArgs& a, int lane, int g_first, int b, int q0, int k0, int Lk,
                                            int t_begin, int t_end, bool direct, int64_t unit0) {
  static_assert(U % 2 == 0, "P.V pairs keys");
  constexpr int D = kHeadDim;
  const int c = lane & 15;
  const int g_lane = g_first + (lane >> 4);               // this DPP row's kv head
  const bool row_live = g_lane < a.num_kv_heads;
  const int g = row_live ? g_lane : a.num_kv_heads - 1;   // idle rows read a valid head
  const int H = a.num_heads;
  const float c2 = a.scale_log2;
  const uint32_t lane_bytes = (uint32_t)(g * D + c * 8) * 2u;

  // q stays in bf16 pairs: q.k runs on v_dot2_f32_bf16 and the scale is applied to the
  // fp32 dot product (scores are kept unscaled; c2 enters the exponent). q is loaded (or,
  // in the fused decode step, computed) after the first K/V loads are issued, so its
  // latency overlaps theirs -- except in the fused split that stores the token's K/V row,
  // which must finish that store before any of its loads.
  DecodeState<G> st;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    st.m[i] = -INFINITY;
    st.l[i] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) st.acc[i][e] = 0.f;
  }
  const auto load_q = [&]() {
    if constexpr (FUSED) {
      fused_producer<G>(a, st, q0, g, c, row_live, false);
    } else {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const uint4 w = *reinterpret_cast<const uint4*>(a.q + (int64_t)q0 * a.q_row_stride + (g * G + i) * D + c * 8);
        st.qp[i][0] = w.x;
        st.qp[i][1] = w.y;
        st.qp[i][2] = w.z;
        st.qp[i][3] = w.w;
      }
    }
  };
  const auto nothing = []() {};

  // Keys at positions >= a.stream_from are read with non-temporal (streaming) loads, earlier
  // ones with normal loads: prefix caching can only share a sequence's leading blocks, so
  // those are the reads worth keeping in L2 / Infinity Cache; everything past them is read
  // once per step and only displaces useful lines. Decided per split (by its first key).
  const bool stream = a.stream_from >= 0 && t_begin >= a.stream_from;
  if (FUSED && t_end == Lk) {  // the split holding the token: store its K/V row first
    fused_producer<G>(a, st, q0, g, c, row_live, true);
    if (stream)
      decode_range<G, U, PAGED, true, FUSED>(st, a, lane_bytes, b, k0, t_begin, t_end, nothing);
    else
      decode_range<G, U, PAGED, false, FUSED>(st, a, lane_bytes, b, k0, t_begin, t_end, nothing);
  } else if (stream) {
    decode_range<G, U, PAGED, true, FUSED>(st, a, lane_bytes, b, k0, t_begin, t_end, load_q);
  } else {
    decode_range<G, U, PAGED, false, FUSED>(st, a, lane_bytes, b, k0, t_begin, t_end, load_q);
  }

  if (!row_live) return;
  // Partials of this unit: H heads x (D outputs in bf16, (max, sum)), contiguous, written
  // through L2 or left in it by the launch's choice (kStoreThroughBytes). A unit holds >= 1
  // key, so l >= 1 (its largest score contributes exp2(0)).
  const __amdgpu_buffer_rsrc_t po_rs = row_rsrc(a.part_o + unit0 * D, (uint32_t)(H * D * 2));
  const __amdgpu_buffer_rsrc_t pml_rs = row_rsrc(a.part_ml + unit0 * 2, (uint32_t)(H * 8));
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const int h = g * G + i;
    const float inv = 1.f / st.l[i];
    uint4 w;
    w.x = pack_bf16x2(st.acc[i][0] * inv, st.acc[i][1] * inv);
    w.y = pack_bf16x2(st.acc[i][2] * inv, st.acc[i][3] * inv);
    w.z = pack_bf16x2(st.acc[i][4] * inv, st.acc[i][5] * inv);
    w.w = pack_bf16x2(st.acc[i][6] * inv, st.acc[i][7] * inv);
    if (direct) {  // the only unit of this sequence: its output row
      *reinterpret_cast<uint4*>(a.out + (int64_t)q0 * a.out_row_stride + h * D + c * 8) = w;
    } else {
      const int o = (h * D + c * 8) * 2;  // 16 lanes store one 256-byte head row
      const f32x2 ml = {st.m[i] * c2, st.l[i]};  // merged in the exp2 domain: the scaled max
      if (a.store_through)
        store_partial<kStoreThrough>(po_rs, pml_rs, o, h * 8, w, ml, c == 0);
      else
        store_partial<0>(po_rs, pml_rs, o, h * 8, w, ml, c == 0);
    }
  }
}

// Split mode: grid (splits x sequences, kv-head groups); a work-group takes split `split` of
// one sequence (split_tokens keys after the shared prefix, if any).
template <int G, int U, bool PAGED, bool FUSED>
__global__ __launch_bounds__(kWave* kDecodeMaxWaves) void decode_split_kernel(const AttnArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
  // The launch divides the kv heads evenly over the waves: every wave has >= 1 live row.
  const int g_first = (blockIdx.y * (blockDim.x / kWave) + wave) * 4;   // first kv head of the wave
  // Work-groups are dispatched round-robin over the 8 XCDs in linear id order. Split-major
  // order with the sequence rotated by the split index sends consecutive splits of one
  // sequence to consecutive XCDs, so every XCD gets about 1/8 of each sequence whatever the
  // lengths (a (split, sequence) grid with 16 splits would give XCD k splits k and k+8 of
  // every sequence: split 0 always exists, split 15 only for the longest contexts).
  const int split = blockIdx.x / a.num_seqs;
  const int b = (blockIdx.x - split * a.num_seqs + split) % a.num_seqs;
  // Both length pairs are read before the first branch, in one round of scalar loads: the
  // two early exits are one test, so neither pair waits behind the other's branch.
  const int q0 = a.cu_q[b], q1 = a.cu_q[b + 1];
  const int k0 = a.cu_k[b], k1 = a.cu_k[b + 1];
  const int Lk = min(k1 - k0, a.max_seqlen_k);
  // keys below Pb belong to the shared-prefix kernel (Pb = 0 when it is off)
  const int Pb = max(0, min(a.prefix_keys, Lk));
  const int t_begin = Pb + split * a.split_tokens;
  // rows with Lq != 1 belong to the prefill kernel; t_begin >= Lk also skips Lk <= 0 (graph padding)
  if ((q1 - q0 != 1) | (t_begin >= Lk)) return;
  const int t_end = min(Lk, t_begin + a.split_tokens);
  // partials of the sequence: its prefix chunks, then its splits
  const int nsplit = (Pb + a.prefix_chunk - 1) / a.prefix_chunk + (Lk - Pb + a.split_tokens - 1) / a.split_tokens;
  const int slot = a.prefix_slots + split;
  decode_unit<G, U, PAGED, FUSED>(a, lane, g_first, b, q0, k0, Lk, t_begin, t_end, nsplit == 1,
                                  ((int64_t)b * a.max_splits + slot) * a.num_heads);
}

// Inclusive sum over the wavefront: lane i gets x_0 + ... + x_i. DPP row shifts scan each
// 16-lane row, then the totals of the rows below are added (three readlanes).
__device__ __forceinline__ int wave_inclusive_sum(int v, int lane) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1 (row lane 0 adds 0)
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  const int r0 = __builtin_amdgcn_readlane(v, 15), r1 = __builtin_amdgcn_readlane(v, 31),
            r2 = __builtin_amdgcn_readlane(v, 47);
  const int row = lane >> 4;
  return v + (row >= 1 ? r0 : 0) + (row >= 2 ? r1 : 0) + (row >= 3 ? r2 : 0);
}

// Flat mode: the decode keys of the batch -- per decode sequence b the c_b keys after its
// shared prefix (all of them without one) -- are laid end to end in sequence order (the key
// line: sequence b from position pos_b = c_0 + ... + c_{b-1}) and cut into W = flat_groups
// runs of `chunk` keys, so that every work-group streams the same number of K/V rows
// whatever the length mix (the split grid gives each sequence whole splits: its last split
// is ragged, short sequences leave many work-groups empty, and prefill rows of a mixed batch
// or keys past max_seqlen_k take no place on the line). A pipeline step (U keys at a multiple
// of U after the prefix) belongs to the run holding its first key, so sequence b has a piece
// in runs w0(b) .. w1(b) (the runs of its first and last steps). Piece (b, w) is work-group
// u = b + w and partial unit flat_unit0 + u: the index is unique because the runs and the
// sequences both tile the line in order, so b + w1(b) < b' + w0(b') for b < b'. The grid has
// W + num_seqs + 1 work-groups: those whose index falls between two sequences' ranges exit at
// once, and the last one records chunk and every pos_b for the combine. (174 VGPRs for G = 2,
// two wavefronts per SIMD: the 1024-work-group grid of two-wavefront groups fits 4 per CU.)
// chunk = max(flat_min_chunk, ceil(T / W) rounded up to U), T = the line's length. One
// wavefront holds every sequence's bounds (num_seqs < 64 * kFlatSlots), forms the line with a
// wavefront prefix sum and finds the work-group's sequence with one ballot per slot.
constexpr int kFlatSlots = 8;

template <int G, int U, bool PAGED, bool FUSED>
__global__ __launch_bounds__(kWave* kDecodeMaxWaves) void decode_flat_kernel(const AttnArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g_first = (blockIdx.y * (blockDim.x / kWave) + wave) * 4;
  const int n = a.num_seqs;
  // lane l, slot s: sequence e = l + 64 s
  int kb[kFlatSlots], qb[kFlatSlots], lk[kFlatSlots], cnt[kFlatSlots], pos[kFlatSlots];
  int T = 0;
#pragma unroll
  for (int s = 0; s < kFlatSlots; ++s) {
    kb[s] = qb[s] = lk[s] = cnt[s] = pos[s] = 0;
    if (64 * s < n) {
      const int e = lane + 64 * s;
      if (e < n) {
        kb[s] = a.cu_k[e];
        qb[s] = a.cu_q[e];
        const int k1 = a.cu_k[e + 1], q1 = a.cu_q[e + 1];
        lk[s] = min(k1 - kb[s], a.max_seqlen_k);
        const int pb = max(0, min(a.prefix_keys, lk[s]));
        cnt[s] = (q1 - qb[s] == 1 && lk[s] > 0) ? lk[s] - pb : 0;  // decode keys after the prefix
      }
      const int incl = wave_inclusive_sum(cnt[s], lane);
      pos[s] = T + incl - cnt[s];
      T += __builtin_amdgcn_readlane(incl, kWave - 1);
    }
  }
  const int per = (T + a.flat_groups - 1) / a.flat_groups;
  const int chunk = max(a.flat_min_chunk, (per + U - 1) / U * U);
  const int u = blockIdx.x;
  // the decode sequence with b + w0(b) <= u <= b + w1(b), if any
  int b = -1, q0 = 0, k0 = 0, Lk = 0, p0 = 0, cb = 0;
#pragma unroll
  for (int s = 0; s < kFlatSlots; ++s) {
    if (64 * s < n) {
      const int e = lane + 64 * s;
      const int w0 = pos[s] / chunk;
      const int w1 = (pos[s] + (cnt[s] - 1) / U * U) / chunk;
      const uint64_t m = __builtin_amdgcn_ballot_w64(cnt[s] > 0 && e + w0 <= u && u <= e + w1);
      if (m) {
        const int j = __builtin_ctzll(m);
        b = 64 * s + j;
        q0 = __builtin_amdgcn_readlane(qb[s], j);
        k0 = __builtin_amdgcn_readlane(kb[s], j);
        Lk = __builtin_amdgcn_readlane(lk[s], j);
        p0 = __builtin_amdgcn_readlane(pos[s], j);
        cb = __builtin_amdgcn_readlane(cnt[s], j);
      }
    }
  }
  if (b < 0) {
    // The last work-group holds no piece (b + w1(b) <= num_seqs - 1 + W - 1): it records the
    // line for the combine. (Recorded here, after the search, so that its stores precede no
    // block-table read on any path: the compiler then reads the table with scalar loads.)
    if (u == a.flat_groups + n && blockIdx.y == 0 && wave == 0) {
      if (lane == 0) a.flat_meta[0] = chunk;
#pragma unroll
      for (int s = 0; s < kFlatSlots; ++s)
        if (lane + 64 * s < n) a.flat_meta[1 + lane + 64 * s] = pos[s];
    }
    return;
  }
  const int Pb = Lk - cb;                                // keys of the shared prefix
  const int F0 = (u - b) * chunk, F1 = F0 + chunk;       // this run, on the line
  const int t_begin = Pb + (F0 > p0 ? (F0 - p0 + U - 1) / U * U : 0);
  const int t_end = min(Lk, Pb + (F1 - p0 + U - 1) / U * U);
  // the sequence's first and last steps in one run and no prefix partial: this piece is all of it
  const bool direct = Pb == 0 && p0 / chunk == (p0 + (cb - 1) / U * U) / chunk;
  decode_unit<G, U, PAGED, FUSED>(a, lane, g_first, b, q0, k0, Lk, t_begin, t_end, direct,
                                  ((int64_t)a.flat_unit0 + u) * a.num_heads);
}

// Merge the per-split partials of one (sequence, head). A separate launch (rather than a
// "last work-group merges" tail in the split kernel) because the XCD L2 caches are not
// coherent with each other: a device-scope fence per work-group would write back and
// invalidate a whole L2, while the kernel boundary makes every partial visible for free.
// Up to kCombineFast splits are merged from registers in two dependent memory round trips
// (the sequence's lengths, then all partials at once); longer contexts take the LDS path.
constexpr int kCombineThreads = kHeadDim;  // thread d owns output element d
constexpr int kCombineMaxSplits = 256;     // splits per sequence the weight table holds

__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  for (int m = kWave / 2; m >= 1; m >>= 1) {
    const float o = xor_shfl(v, m);
    v = is_max ? fmaxf(v, o) : v + o;
  }
  const int wave = threadIdx.x / kWave;
  __syncthreads();  // red may still be read by a previous reduction
  if ((threadIdx.x & (kWave - 1)) == 0) red[wave] = v;
  __syncthreads();
  v = red[0];
  for (int w = 1; w < kCombineThreads / kWave; ++w) v = is_max ? fmaxf(v, red[w]) : v + red[w];
  return v;
}

#ifndef PK_COMBINE_FAST
#define PK_COMBINE_FAST 64
#endif
// Splits merged from registers, without LDS: lane j of each wavefront holds split j's
// (max, sum), so at most one wavefront's width. Measured on 8 sequences of 256-2048 keys
// (29 splits of 64 keys): 4.9 us against 5.6 us on the LDS path (16-split register path).
constexpr int kCombineFast = PK_COMBINE_FAST;
static_assert(kCombineFast <= kWave && (kCombineFast & (kCombineFast - 1)) == 0, "one lane per split");

__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const AttnArgs a) {
  constexpr int D = kHeadDim;
  __shared__ float w_s[kCombineMaxSplits];
  __shared__ float red[kCombineThreads / kWave];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  const int q0 = a.cu_q[b];
  const int q1 = a.cu_q[b + 1];
  const int k_lo = a.cu_k[b];
  const int k_hi = a.cu_k[b + 1];
  // the flat grid's record is read in the same round of loads as the bounds
  const bool flat = a.flat_groups > 0;
  const int f_chunk = flat ? a.flat_meta[0] : 1;
  const int f_pos = flat ? a.flat_meta[1 + b] : 0;
  if (q1 - q0 != 1) return;
  const int Lk = min(k_hi - k_lo, a.max_seqlen_k);
  if (Lk <= 0) return;
  const int H = a.num_heads;
  // partial j of the sequence: its prefix chunks j < npre (units pre0 + j), then the decode
  // kernel's splits or pieces (units post0 + j)
  const int Pb = min(a.prefix_keys, Lk);
  const int npre = (Pb + a.prefix_chunk - 1) / a.prefix_chunk;
  int nsplit;
  int64_t pre0 = (int64_t)b * a.prefix_stride, post0;
  if (flat) {
    // flat grid: the pieces of runs w0 .. w1 (those holding the first and the last step of the
    // sequence's keys after the prefix, on the key line), piece of run w at unit flat_unit0 + b + w
    const int cb = Lk - Pb;
    int w0 = 0, w1 = -1;
    if (cb > 0) {
      w0 = f_pos / f_chunk;
      w1 = (f_pos + (cb - 1) / a.flat_step * a.flat_step) / f_chunk;
    }
    nsplit = npre + (int)(w1 - w0 + 1);
    post0 = a.flat_unit0 + b + w0 - npre;
  } else {
    nsplit = npre + (Lk - Pb + a.split_tokens - 1) / a.split_tokens;
    post0 = (int64_t)b * a.max_splits + a.prefix_slots - npre;
  }
  if (nsplit <= 1 && npre == 0) return;  // written directly by the decode kernel
  nsplit = min(nsplit, kCombineMaxSplits);  // the launch keeps it within (the weight table's size)
  const auto unit_of = [&](int j) -> int64_t { return j < npre ? pre0 + j : post0 + j; };
  const int d = threadIdx.x;
  const uint16_t* po = a.part_o + (int64_t)h * D + d;
  const int64_t stride = (int64_t)H * D;
  if (nsplit <= kCombineFast) {
    // Every load of the merge is issued at once: lane j < nsplit of each wavefront reads
    // split j's (max, sum), thread d element d of every split. The weights are formed in
    // lanes 0 .. kCombineFast - 1 and broadcast by shuffles: no LDS, no barrier.
    // Reductions are DPP row steps plus reads of the four rows' lanes, and weight j reaches
    // every lane by a readlane: no LDS permutes on the dependency chain.
    const int lane = threadIdx.x & (kWave - 1);
    float2 ml = make_float2(-INFINITY, 0.f);
    if (lane < nsplit) ml = *reinterpret_cast<const float2*>(a.part_ml + (unit_of(lane) * H + h) * 2);
    // N unconditional loads (the next power of two >= nsplit, at least 8), issued with the
    // (max, sum) loads: past nsplit the last partial is read again, and its weight there is 0.
    // (A conditional 16-bit load per split compiles to a branch and a wait per split; all 64
    // loads for every sequence cost cfg2's combine 6 -> 9.4 us.)
    const auto merge = [&](auto n_tag) {
      constexpr int N = decltype(n_tag)::value;
      float v[N];
#pragma unroll
      for (int j = 0; j < N; ++j) v[j] = bf16_to_f32(po[unit_of(min(j, nsplit - 1)) * stride]);
      const float rm = row16_max(ml.x);
      const float mx = fmaxf(fmaxf(lane_value(rm, 0), lane_value(rm, 16)), fmaxf(lane_value(rm, 32), lane_value(rm, 48)));
      const float w = lane < nsplit ? exp2_fast(ml.x - mx) * ml.y : 0.f;  // each partial's weight: its share of l
      const float rs = row16_sum(w);
      const float lsum = (lane_value(rs, 0) + lane_value(rs, 16)) + (lane_value(rs, 32) + lane_value(rs, 48));
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < N; ++j) acc = fmaf(lane_value(w, j), v[j], acc);
      a.out[(int64_t)q0 * a.out_row_stride + h * D + d] = f32_to_bf16(acc / lsum);
    };
    if (nsplit <= 8)
      merge(std::integral_constant<int, 8>{});
    else if (nsplit <= 16)
      merge(std::integral_constant<int, 16>{});
    else if (nsplit <= 32)
      merge(std::integral_constant<int, 32>{});
    else
      merge(std::integral_constant<int, kCombineFast>{});
    return;
  }
  // Long contexts: split maxima and weights by block reductions into LDS, then thread d
  // forms the weighted sum of element d with four independent accumulators.
  float mx = -INFINITY;
  for (int j = threadIdx.x; j < nsplit; j += kCombineThreads)
    mx = fmaxf(mx, a.part_ml[(unit_of(j) * H + h) * 2]);
  mx = block_reduce(mx, true, red);
  float lsum = 0.f;
  for (int j = threadIdx.x; j < nsplit; j += kCombineThreads) {
    const float2 ml = *reinterpret_cast<const float2*>(a.part_ml + (unit_of(j) * H + h) * 2);
    const float w = exp2_fast(ml.x - mx) * ml.y;
    w_s[j] = w;
    lsum += w;
  }
  lsum = block_reduce(lsum, false, red);  // its barriers also publish w_s
  float o0 = 0.f, o1 = 0.f, o2 = 0.f, o3 = 0.f;
  int j = 0;
  for (; j + 4 <= nsplit; j += 4) {
    o0 = fmaf(w_s[j], bf16_to_f32(po[unit_of(j) * stride]), o0);
    o1 = fmaf(w_s[j + 1], bf16_to_f32(po[unit_of(j + 1) * stride]), o1);
    o2 = fmaf(w_s[j + 2], bf16_to_f32(po[unit_of(j + 2) * stride]), o2);
    o3 = fmaf(w_s[j + 3], bf16_to_f32(po[unit_of(j + 3) * stride]), o3);
  }
  for (; j < nsplit; ++j) o0 = fmaf(w_s[j], bf16_to_f32(po[unit_of(j) * stride]), o0);
  a.out[(int64_t)q0 * a.out_row_stride + h * D + d] = f32_to_bf16(((o0 + o1) + (o2 + o3)) / lsum);
}

template <int G, int U>
hipError_t launch_decode_g(AttnArgs a, bool paged, hipStream_t stream) {
  const bool flat = a.flat_groups > 0;
  const int64_t units = flat ? (int64_t)a.num_seqs + a.flat_groups : (int64_t)a.num_seqs * a.max_splits;  // decode kernel's
  a.store_through = units * a.num_heads * kHeadDim * 4 > kStoreThroughBytes;
  const int quads = (a.num_kv_heads + 3) / 4;   // wavefronts needed for all kv heads
  int waves = quads < kDecodeMaxWaves ? quads : kDecodeMaxWaves;
  while (quads % waves != 0) --waves;            // no idle wavefront in any work-group
  const int zgroups = quads / waves;
  const dim3 block((unsigned)(waves * kWave));
  const bool fused = a.qkv != nullptr || a.new_k != nullptr;  // paged only (checked by their entry points)
  if (flat) {
    const dim3 grid((unsigned)(a.flat_groups + a.num_seqs + 1), (unsigned)zgroups);  // + the recorder
    if (fused)
      hipLaunchKernelGGL((decode_flat_kernel<G, U, true, true>), grid, block, 0, stream, a);
    else if (paged)
      hipLaunchKernelGGL((decode_flat_kernel<G, U, true, false>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((decode_flat_kernel<G, U, false, false>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
  if (a.grid_splits <= 0) return hipSuccess;  // every decode key lies in the shared prefix
  const dim3 grid((unsigned)(a.grid_splits * a.num_seqs), (unsigned)zgroups);
  if (fused)
    hipLaunchKernelGGL((decode_split_kernel<G, U, true, true>), grid, block, 0, stream, a);
  else if (paged)
    hipLaunchKernelGGL((decode_split_kernel<G, U, true, false>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((decode_split_kernel<G, U, false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// Keys per pipeline step of the decode kernels built for a GQA group.
constexpr int decode_step_keys(int group) { return group <= 2 ? PK_DECODE_STEP_G2 : 4; }

}  // namespace

int decode_split_tokens(int num_seqs, int max_seqlen_k) {
  // PK_DECODE_SPLIT_MAX keys per work-group when the batch yields enough work-groups to
  // cover the 256 CUs several times, shorter splits for small batches; longer ones when
  // the combine pass's weight table (kCombineMaxSplits per sequence) would overflow.
  const auto splits = [&](int split) { return (int64_t)(max_seqlen_k + split - 1) / split; };
  int split = PK_DECODE_SPLIT_MAX;
  while (split > PK_DECODE_MIN_SPLIT && (int64_t)num_seqs * splits(split) < PK_DECODE_MIN_GROUPS &&
         splits(split / 2) <= kCombineMaxSplits)
    split /= 2;
  while (splits(split) > kCombineMaxSplits) split *= 2;
  return split;
}

FlatDecodePlan decode_flat_plan(int num_seqs, int max_seqlen_k) {
  // Flat mode needs every sequence bound in one wavefront (num_seqs < 64 * kFlatSlots), key
  // positions that fit in 30 bits, and a batch the split grid would cut into several splits
  // (a batch whose sequences each fit one split needs no partials at all); it is used in the
  // measured range where it beats the split grid (PK_DECODE_FLAT_MAX_SEQS, _MIN_KEYS). Runs:
  // enough that the grid (runs + sequences) is PK_DECODE_FLAT_GROUPS work-groups, or fewer
  // when runs of PK_DECODE_FLAT_MIN_CHUNK keys cover the launch bound. The shortest run keeps
  // a sequence within the combine's kCombineMaxSplits pieces: (Lk - 1) / chunk + 2 of them.
  FlatDecodePlan p{0, 0};
  if (num_seqs <= 0 || num_seqs > PK_DECODE_FLAT_MAX_SEQS || num_seqs >= 64 * kFlatSlots || max_seqlen_k <= 0)
    return p;
  const int64_t keys = (int64_t)num_seqs * max_seqlen_k;
  if (keys < PK_DECODE_FLAT_MIN_KEYS || keys >= (1ll << 30) ||
      max_seqlen_k <= decode_split_tokens(num_seqs, max_seqlen_k))
    return p;
  int min_chunk = PK_DECODE_FLAT_MIN_CHUNK;
  const int need = (max_seqlen_k + kCombineMaxSplits - 3) / (kCombineMaxSplits - 2);
  if (min_chunk < need) min_chunk = (need + 7) / 8 * 8;
  const int64_t groups = std::min<int64_t>(std::max(PK_DECODE_FLAT_GROUPS - num_seqs, 2),
                                           (keys + min_chunk - 1) / min_chunk);
  if (groups < 2) return p;
  p.groups = (int)groups;
  p.min_chunk = min_chunk;
  return p;
}

hipError_t launch_decode(const AttnArgs& args, int group, bool paged, int max_seqlen_k,
                         hipStream_t stream) {
  if (args.num_seqs <= 0 || max_seqlen_k <= 0) return hipSuccess;
  AttnArgs a = args;
  a.flat_step = decode_step_keys(group);
  hipError_t err;
  switch (group) {
    case 1: err = launch_decode_g<1, decode_step_keys(1)>(a, paged, stream); break;
    case 2: err = launch_decode_g<2, decode_step_keys(2)>(a, paged, stream); break;
    case 4: err = launch_decode_g<4, decode_step_keys(4)>(a, paged, stream); break;
    case 8: err = launch_decode_g<8, decode_step_keys(8)>(a, paged, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (err != hipSuccess) return err;
  if (a.max_splits > 1 || a.flat_groups > 0) {
    hipLaunchKernelGGL(decode_combine_kernel, dim3((unsigned)a.num_heads, (unsigned)a.num_seqs),
                       dim3(kCombineThreads), 0, stream, a);
    err = hipGetLastError();
  }
  return err;
}

}  // namespace pk
