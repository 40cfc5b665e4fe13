// Device code of the paged decode path, kept apart from the kernels that run it
// (paged_decode.hip): the register-direct K/V pipeline, the fused producer, one decode work
// unit, and the per-(sequence, head) body of the combine pass.
#pragma once

#include "norm_rope.h"

namespace pk {
namespace {

#ifndef PK_DECODE_STEP_G2
#define PK_DECODE_STEP_G2 8     // keys per pipeline step for GQA groups <= 2
#endif
// Keys per pipeline step and DPP row of the decode units built for a GQA group.
constexpr int decode_step_keys(int group) { return group <= 2 ? PK_DECODE_STEP_G2 : 4; }
// DPP rows per kv head (key rows): a wavefront's four 16-lane rows hold four kv heads, or,
// with fewer kv heads than that (one tensor-parallel rank's share: 2 or 1), 4 / Hkv rows per
// head that take interleaved keys, so that no row re-reads another's head.
constexpr int decode_key_rows(int num_kv_heads) { return num_kv_heads == 1 ? 4 : num_kv_heads == 2 ? 2 : 1; }
// Keys a wavefront consumes per pipeline step: the flat grid's step.
inline int decode_flat_step(int group, int num_kv_heads) {
  return decode_step_keys(group) * decode_key_rows(num_kv_heads);
}

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

// Cache block ids of a unit's keys, one per lane (lane i: table entry blk0 + i), loaded once
// before its pipeline when BR is set, so that a step's block id is a readlane instead of a
// scalar load that the step waits for before its K/V loads go out. A unit spanning more than a
// wavefront's worth of blocks reads the table per step. Used where it measured faster: the
// flat groups of the shared-prefix launch (cfg4 41.9 -> 40.3 us, interleaved); in the split
// and flat decode kernels it measured slower on cfg2 (748.7 -> 757.9 us) and cfg1.
struct UnitBlocks {
  int ids;      // this lane's block id
  int blk0;     // the unit's first table entry
  bool in_regs;
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

// R key rows per kv head (decode_key_rows): DPP row j of a head takes keys t + u R + j of
// the step's U R keys, so one load instruction reads R consecutive token rows. Its lane
// offsets lane_k / lane_v include row j's key (j row strides), and the loads are bounded
// by the buffer's range instead of clamped (a row's key past t_end reads zeros, finite,
// masked to p = 0 by consume): the row offset is per lane, which a scalar offset cannot
// carry.
// live == false: a prefetch past the unit's last step, whose values are never used; its loads
// go out (the pipeline's wait counts stay exact) over an empty buffer range, so they return
// zeros without touching memory (a re-read of the last step, streamed past L2, came back from
// HBM: one extra step per unit, ~15% of the bytes of a short flat-grid piece).
template <int U, int R, bool PAGED, bool STREAM, bool FUSED, bool BR>
__device__ __forceinline__ void issue_loads(const AttnArgs& a, uint32_t lane_k, uint32_t lane_v, int b, int k0, int t,
                                            int t_end, bool live, const UnitBlocks& ub, u32x4 (&kr)[U],
                                            u32x4 (&vr)[U]) {
  const uint16_t* kp;
  const uint16_t* vp;
  if constexpr (PAGED) {
    // [t, t + U R) lies inside one cache block: U R divides block_size and split_tokens.
    const int jb = t / a.block_size;
    const int blk = (BR && ub.in_regs) ? __builtin_amdgcn_readlane(ub.ids, jb - ub.blk0)
                    : FUSED            ? scalar_block_id(a.block_table + (int64_t)b * a.bt_stride, jb)
                                       : a.block_table[(int64_t)b * a.bt_stride + jb];
    const int off = t % a.block_size;
    kp = a.k + (int64_t)blk * a.k_block_stride + (int64_t)off * a.k_row_stride;
    vp = a.v + (int64_t)blk * a.v_block_stride + (int64_t)off * a.v_row_stride;
  } else {
    kp = a.k + (int64_t)(k0 + t) * a.k_row_stride;
    vp = a.v + (int64_t)(k0 + t) * a.v_row_stride;
  }
  // row strides are < 2^22 elements (checked on the host), so U R rows span < 2^29 bytes
  const uint32_t k_row_bytes = (uint32_t)a.k_row_stride * 2u;
  const uint32_t v_row_bytes = (uint32_t)a.v_row_stride * 2u;
  if constexpr (R == 1) {
    const __amdgpu_buffer_rsrc_t kr_rs = row_rsrc(kp, live ? (uint32_t)U * k_row_bytes : 0u);
    const __amdgpu_buffer_rsrc_t vr_rs = row_rsrc(vp, live ? (uint32_t)U * v_row_bytes : 0u);
    const int last = t_end - 1 - t;
#pragma unroll
    for (int u = 0; u < U; ++u) kr[u] = load16<STREAM>(kr_rs, lane_k, __umul24((uint32_t)min(u, last), k_row_bytes));
#pragma unroll
    for (int u = 0; u < U; ++u) vr[u] = load16<STREAM>(vr_rs, lane_v, __umul24((uint32_t)min(u, last), v_row_bytes));
  } else {
    const uint32_t rows = live ? (uint32_t)min(U * R, t_end - t) : 0u;  // keys of the step that exist
    const __amdgpu_buffer_rsrc_t kr_rs = row_rsrc(kp, rows * k_row_bytes);
    const __amdgpu_buffer_rsrc_t vr_rs = row_rsrc(vp, rows * v_row_bytes);
#pragma unroll
    for (int u = 0; u < U; ++u) kr[u] = load16<STREAM>(kr_rs, lane_k + (uint32_t)(u * R) * k_row_bytes, 0);
#pragma unroll
    for (int u = 0; u < U; ++u) vr[u] = load16<STREAM>(vr_rs, lane_v + (uint32_t)(u * R) * v_row_bytes, 0);
  }
}

// Keys [t_begin, t_end) of one split through a two-stage software pipeline: the loads of
// step n+1 are in flight while step n is consumed. The prefetch is unconditional (past
// t_end it is issued over an empty range) so the code is straight-line and the wait counts
// stay exact. The scheduling barriers keep each step's loads together
// ahead of its math: otherwise the scheduler sinks every load next to its first use to
// save registers, which serialises their latency.
template <int G, int U, int R, bool PAGED, bool STREAM, bool FUSED, bool BR, class Pre>
__device__ __forceinline__ void decode_range(DecodeState<G>& st, const AttnArgs& a, uint32_t lane_k, uint32_t lane_v,
                                             int j, int b, int k0, int t_begin, int t_end, Pre&& pre);

// Fold this row's keys of the step at t (already loaded: key t + u R + j for load u) into the
// running softmax state.
template <int G, int U, int R>
__device__ __forceinline__ void consume(DecodeState<G>& st, float c2, int t, int t_end, int j, const u32x4 (&kr)[U],
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
    if (t + u * R + (R > 1 ? j : 0) >= t_end) {  // uniform over the wavefront when R == 1
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
    // R == 1: finite, the step holds >= 1 valid key. R > 1: a row may not have had a key
    // yet (-inf); its l and numerator are 0, and alpha and the exponents must stay finite.
    const float m_new = fmaxf(st.m[i], mx);
    const float alpha = (R > 1 && st.m[i] == -INFINITY) ? 0.f : exp2_fast((st.m[i] - m_new) * c2);
    st.m[i] = m_new;
    const float ms = (R > 1 && m_new == -INFINITY) ? 0.f : m_new * c2;
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

template <int G, int U, int R, bool PAGED, bool STREAM, bool FUSED, bool BR, class Pre>
__device__ __forceinline__ void decode_range(DecodeState<G>& st, const AttnArgs& a, uint32_t lane_k, uint32_t lane_v,
                                             int j, int b, int k0, int t_begin, int t_end, Pre&& pre) {
  constexpr int S = U * R;  // keys per step
  const float c2 = a.scale_log2;
  UnitBlocks ub{0, 0, false};
  if constexpr (PAGED && BR) {
    ub.blk0 = t_begin / a.block_size;
    const int nblk = (t_end - 1) / a.block_size - ub.blk0 + 1;
    ub.in_regs = nblk <= kWave;
    const int lane = __lane_id();
    if (ub.in_regs && lane < nblk) ub.ids = a.block_table[(int64_t)b * a.bt_stride + ub.blk0 + lane];
  }
  u32x4 kA[U], vA[U], kB[U], vB[U];
  issue_loads<U, R, PAGED, STREAM, FUSED, BR>(a, lane_k, lane_v, b, k0, t_begin, t_end, true, ub, kA, vA);
  pre();  // q (loaded or computed) while the first K/V loads are in flight
  for (int t = t_begin; t < t_end; t += 2 * S) {
    const int t1 = t + S;
    issue_loads<U, R, PAGED, STREAM, FUSED, BR>(a, lane_k, lane_v, b, k0, t1 < t_end ? t1 : t, t_end, t1 < t_end, ub,
                                                kB, vB);
    __builtin_amdgcn_sched_barrier(0);
    consume<G, U, R>(st, c2, t, t_end, j, kA, vA);
    if (t1 >= t_end) break;
    const int t2 = t1 + S;
    issue_loads<U, R, PAGED, STREAM, FUSED, BR>(a, lane_k, lane_v, b, k0, t2 < t_end ? t2 : t1, t_end, t2 < t_end, ub,
                                                kA, vA);
    __builtin_amdgcn_sched_barrier(0);
    consume<G, U, R>(st, c2, t1, t_end, j, kB, vB);
  }
}

// R > 1: merge the softmax states of the R rows that hold one kv head's interleaved keys
// (rows j = row / (4 / R), lanes 16 (4 / R) apart), so that every row of the head ends with
// the state over all of the unit's keys. A row that saw no key (m = -inf) adds nothing.
template <int G, int R>
__device__ __forceinline__ void merge_key_rows(DecodeState<G>& st, float c2) {
  if constexpr (R > 1) {
#pragma unroll
    for (int sh = 64 / R; sh < kWave; sh *= 2) {
#pragma unroll
      for (int i = 0; i < G; ++i) {
        const float mo = __shfl_xor(st.m[i], sh);
        const float lo = __shfl_xor(st.l[i], sh);
        const float m_new = fmaxf(st.m[i], mo);
        const float wa = st.m[i] == -INFINITY ? 0.f : exp2_fast((st.m[i] - m_new) * c2);
        const float wb = mo == -INFINITY ? 0.f : exp2_fast((mo - m_new) * c2);
        st.l[i] = st.l[i] * wa + lo * wb;
#pragma unroll
        for (int e = 0; e < 8; ++e) st.acc[i][e] = st.acc[i][e] * wa + __shfl_xor(st.acc[i][e], sh) * wb;
        st.m[i] = m_new;
      }
    }
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
// R key rows per kv head: DPP row r holds kv head g_first + r mod (4 / R) and keys
// t + u R + r / (4 / R) of every step; the rows of a head merge their states at the end.
template <int G, int U, int R, bool PAGED, bool FUSED, bool BR = false>
__device__ __forceinline__ void decode_unit(const AttnArgs& a, int lane, int g_first, int b, int q0, int k0, int Lk,
                                            int t_begin, int t_end, bool direct, int64_t unit0) {
  static_assert(U % 2 == 0, "P.V pairs keys");
  static_assert(R == 1 || R == 2 || R == 4, "key rows per kv head");
  constexpr int D = kHeadDim;
  constexpr int NH = 4 / R;                               // kv heads per wavefront
  const int c = lane & 15;
  const int row = lane >> 4;
  const int j = row / NH;                                 // this row's keys: t + u R + j
  const int g_lane = g_first + row % NH;                  // this DPP row's kv head
  const bool row_live = g_lane < a.num_kv_heads;
  const bool writer = row_live && j == 0;                 // stores the head's results
  const int g = row_live ? g_lane : a.num_kv_heads - 1;   // idle rows read a valid head
  const int H = a.num_heads;
  const float c2 = a.scale_log2;
  const uint32_t lane_bytes = (uint32_t)(g * D + c * 8) * 2u;
  const uint32_t lane_k = lane_bytes + (uint32_t)j * (uint32_t)a.k_row_stride * 2u;
  const uint32_t lane_v = lane_bytes + (uint32_t)j * (uint32_t)a.v_row_stride * 2u;

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
      fused_producer<G>(a, st, q0, g, c, writer, false);
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
    fused_producer<G>(a, st, q0, g, c, writer, true);
    if (stream)
      decode_range<G, U, R, PAGED, true, FUSED, BR>(st, a, lane_k, lane_v, j, b, k0, t_begin, t_end, nothing);
    else
      decode_range<G, U, R, PAGED, false, FUSED, BR>(st, a, lane_k, lane_v, j, b, k0, t_begin, t_end, nothing);
  } else if (stream) {
    decode_range<G, U, R, PAGED, true, FUSED, BR>(st, a, lane_k, lane_v, j, b, k0, t_begin, t_end, load_q);
  } else {
    decode_range<G, U, R, PAGED, false, FUSED, BR>(st, a, lane_k, lane_v, j, b, k0, t_begin, t_end, load_q);
  }
  merge_key_rows<G, R>(st, c2);

  if (!writer) return;
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

// Flat decode grid: the decode keys of the batch -- per decode sequence b the c_b keys after its
// shared prefix (all of them without one) -- are laid end to end in sequence order (the key
// line: sequence b from position pos_b = c_0 + ... + c_{b-1}) and cut into W = flat_groups
// runs of `chunk` keys, so that every work-group streams the same number of K/V rows
// whatever the length mix. A pipeline step (U R keys at a multiple of U R after the prefix)
// belongs to the run holding its first key, so sequence b has a piece in runs w0(b) .. w1(b).
// Piece (b, w) is work-group u = b + w and partial unit flat_unit0 + u: unique, because the
// runs and the sequences both tile the line in order (b + w1(b) < b' + w0(b') for b < b').
// Groups u = 0 .. W + num_seqs: those between two sequences' ranges hold no piece, and the
// last one records chunk and every pos_b for the combine. chunk = max(flat_min_chunk,
// ceil(T / W) rounded up to the step), T = the line's length. One wavefront holds every
// sequence's bounds (num_seqs < 64 * kFlatSlots), forms the line with a wavefront prefix sum
// and finds its group's sequence with one ballot per slot.
constexpr int kFlatSlots = 8;

// One wavefront's share of flat work-group u (its piece, for the kv heads from g_first):
// the flat decode kernel runs it with u = its work-group index, the shared-prefix launch that
// carries the flat grid with u numbered across its decode work-groups. `recorder`: this
// wavefront records the line (chunk and every pos_b) for the combine if u is the last group.
template <int G, int U, int R, bool PAGED, bool FUSED, bool BR = false>
__device__ __forceinline__ void flat_decode_piece(const AttnArgs& a, int u, int g_first, int lane, bool recorder) {
  constexpr int ST = U * R;  // keys per pipeline step: the line's step
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
  const int chunk = max(a.flat_min_chunk, (per + ST - 1) / ST * ST);
  // the decode sequence with b + w0(b) <= u <= b + w1(b), if any
  int b = -1, q0 = 0, k0 = 0, Lk = 0, p0 = 0, cb = 0;
#pragma unroll
  for (int s = 0; s < kFlatSlots; ++s) {
    if (64 * s < n) {
      const int e = lane + 64 * s;
      const int w0 = pos[s] / chunk;
      const int w1 = (pos[s] + (cnt[s] - 1) / ST * ST) / chunk;
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
    if (u == a.flat_groups + n && recorder) {
      if (lane == 0) a.flat_meta[0] = chunk;
#pragma unroll
      for (int s = 0; s < kFlatSlots; ++s)
        if (lane + 64 * s < n) a.flat_meta[1 + lane + 64 * s] = pos[s];
    }
    return;
  }
  const int Pb = Lk - cb;                                // keys of the shared prefix
  const int F0 = (u - b) * chunk, F1 = F0 + chunk;       // this run, on the line
  const int t_begin = Pb + (F0 > p0 ? (F0 - p0 + ST - 1) / ST * ST : 0);
  const int t_end = min(Lk, Pb + (F1 - p0 + ST - 1) / ST * ST);
  // the sequence's first and last steps in one run and no prefix partial: this piece is all of it
  const bool direct = Pb == 0 && p0 / chunk == (p0 + (cb - 1) / ST * ST) / chunk;
  decode_unit<G, U, R, PAGED, FUSED, BR>(a, lane, g_first, b, q0, k0, Lk, t_begin, t_end, direct,
                                         ((int64_t)a.flat_unit0 + u) * a.num_heads);
}

// Merge the per-split partials of one (sequence, head). A separate pass (rather than a "last
// work-group merges" tail in the split kernel) because the XCD L2 caches are not coherent
// with each other: a device-scope fence per work-group would write back and invalidate a
// whole L2, while a kernel boundary makes every partial visible for free. The merge runs
// from registers in 128 consecutive threads (two whole wavefronts, thread d = output element
// d) with no LDS and no barrier, so any kernel can run it on part of a work-group: the decode
// combine launch, or the prefill merge kernel of a call with prefill rows.
constexpr int kCombineThreads = kHeadDim;  // thread d owns output element d
constexpr int kCombineMaxSplits = 256;     // partials per sequence the launches are sized for

#ifndef PK_COMBINE_FAST
#define PK_COMBINE_FAST 64
#endif
// Partials merged in one round of loads: lane j of each wavefront holds partial j's (max,
// sum), so at most one wavefront's width; longer sequences take rounds of this many.
constexpr int kCombineFast = PK_COMBINE_FAST;
static_assert(kCombineFast <= kWave && (kCombineFast & (kCombineFast - 1)) == 0, "one lane per split");

// The merge of one (sequence, head) by the 128 threads whose element is d (threadIdx.x & 63
// is the lane inside each of their two wavefronts).
__device__ __forceinline__ void combine_row(const AttnArgs& a, int b, int h, int d) {
  constexpr int D = kHeadDim;
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
  nsplit = min(nsplit, kCombineMaxSplits);  // the launches keep it within
  const auto unit_of = [&](int j) -> int64_t { return j < npre ? pre0 + j : post0 + j; };
  const uint16_t* po = a.part_o + (int64_t)h * D + d;
  const int64_t stride = (int64_t)H * D;
  const int lane = threadIdx.x & (kWave - 1);
  // (max, sum, weighted sum of element d) of partials j0 .. j0 + cnt - 1. Every load of the
  // round is issued at once: lane j < cnt of each wavefront reads partial j0 + j's (max, sum),
  // thread d element d of N partials (N >= cnt a power of two, at least 8; past cnt the last
  // partial is read again and weighted 0: a conditional 16-bit load per partial compiles to a
  // branch and a wait per partial, and 64 loads for every sequence cost cfg2's combine
  // 6 -> 9.4 us). The weights are formed in lanes 0 .. kCombineFast - 1; reductions are DPP
  // row steps plus reads of the four rows' lanes, and weight j reaches every lane by a
  // readlane: no LDS permutes on the dependency chain.
  const auto round = [&](int j0, int cnt, auto n_tag) {
    constexpr int N = decltype(n_tag)::value;
    float2 ml = make_float2(-INFINITY, 0.f);
    if (lane < cnt) ml = *reinterpret_cast<const float2*>(a.part_ml + (unit_of(j0 + lane) * H + h) * 2);
    float v[N];
#pragma unroll
    for (int j = 0; j < N; ++j) v[j] = bf16_to_f32(po[unit_of(j0 + min(j, cnt - 1)) * stride]);
    const float rm = row16_max(ml.x);
    const float mx = fmaxf(fmaxf(lane_value(rm, 0), lane_value(rm, 16)), fmaxf(lane_value(rm, 32), lane_value(rm, 48)));
    const float w = lane < cnt ? exp2_fast(ml.x - mx) * ml.y : 0.f;  // each partial's share of l
    const float rs = row16_sum(w);
    const float lsum = (lane_value(rs, 0) + lane_value(rs, 16)) + (lane_value(rs, 32) + lane_value(rs, 48));
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < N; ++j) acc = fmaf(lane_value(w, j), v[j], acc);
    return make_float3(mx, lsum, acc);
  };
  float3 r;
  if (nsplit <= 8)
    r = round(0, nsplit, std::integral_constant<int, 8>{});
  else if (nsplit <= 16)
    r = round(0, nsplit, std::integral_constant<int, 16>{});
  else if (nsplit <= 32)
    r = round(0, nsplit, std::integral_constant<int, 32>{});
  else
    r = round(0, min(nsplit, kCombineFast), std::integral_constant<int, kCombineFast>{});
  // Longer sequences: further rounds of kCombineFast partials folded into the running
  // (max, sum, numerator), each rescaled to the larger max.
  for (int j0 = kCombineFast; j0 < nsplit; j0 += kCombineFast) {
    const float3 t = round(j0, min(nsplit - j0, kCombineFast), std::integral_constant<int, kCombineFast>{});
    const float m = fmaxf(r.x, t.x);
    const float sa = exp2_fast(r.x - m), sb = exp2_fast(t.x - m);
    r = make_float3(m, r.y * sa + t.y * sb, r.z * sa + t.z * sb);
  }
  a.out[(int64_t)q0 * a.out_row_stride + h * D + d] = f32_to_bf16(r.z / r.y);
}

// combine_row for a split-grid batch without a shared prefix whose sequences have at most
// max_splits <= N partials: sequence b's partials are units b * max_splits + j whatever its
// length, so every slot's (max, sum) and element d are loaded in the same round as the
// lengths (one memory round trip instead of two). Slots past the sequence's splits hold
// stale or unwritten data: they are excluded by selects, never by a multiplication by zero
// (which would let a stale NaN through).
template <int N>
__device__ __forceinline__ void combine_row_eager(const AttnArgs& a, int b, int h, int d) {
  constexpr int D = kHeadDim;
  const int H = a.num_heads;
  const int lane = threadIdx.x & (kWave - 1);
  const int ms = a.max_splits;  // <= N (checked by the launch)
  const int64_t u0 = (int64_t)b * ms;
  const uint16_t* po = a.part_o + (u0 * H + h) * D + d;
  const int64_t stride = (int64_t)H * D;
  const int q0 = a.cu_q[b];
  const int q1 = a.cu_q[b + 1];
  const int k_lo = a.cu_k[b];
  const int k_hi = a.cu_k[b + 1];
  const float2 mlr = *reinterpret_cast<const float2*>(a.part_ml + ((u0 + min(lane, ms - 1)) * H + h) * 2);
  uint16_t vr[N];
#pragma unroll
  for (int j = 0; j < N; ++j) vr[j] = po[min(j, ms - 1) * stride];
  // every value is consumed here, so the loads above go out together ahead of any branch
  // (the compiler would otherwise sink each load next to its first use, behind the lengths)
  asm volatile("" ::"v"(mlr.x), "v"(mlr.y), "s"(q0), "s"(q1), "s"(k_lo), "s"(k_hi) : "memory");
#pragma unroll
  for (int j = 0; j < N; ++j) asm volatile("" ::"v"(vr[j]));
  const float2 ml = lane < ms ? mlr : make_float2(-INFINITY, 0.f);
  float v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = bf16_to_f32(vr[j]);
  // No branch before the store (the compiler would sink the loads behind it): a row that is
  // not a decode row, or that the decode kernel wrote directly (one split), is merged anyway
  // and not stored.
  const int Lk = min(k_hi - k_lo, a.max_seqlen_k);
  const int nsplit = min((max(Lk, 0) + a.split_tokens - 1) / a.split_tokens, ms);
  const bool store = q1 - q0 == 1 && nsplit > 1;
  const float mv = lane < nsplit ? ml.x : -INFINITY;
  const float rm = row16_max(mv);
  const float mx = fmaxf(fmaxf(lane_value(rm, 0), lane_value(rm, 16)), fmaxf(lane_value(rm, 32), lane_value(rm, 48)));
  const float w = lane < nsplit ? exp2_fast(mv - mx) * ml.y : 0.f;
  const float rs = row16_sum(w);
  const float lsum = (lane_value(rs, 0) + lane_value(rs, 16)) + (lane_value(rs, 32) + lane_value(rs, 48));
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < N; ++j) acc = fmaf(lane_value(w, j), j < nsplit ? v[j] : 0.f, acc);
  if (store) a.out[(int64_t)q0 * a.out_row_stride + h * D + d] = f32_to_bf16(acc / lsum);
}

}  // namespace
}  // namespace pk
