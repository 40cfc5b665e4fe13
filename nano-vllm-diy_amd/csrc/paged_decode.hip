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

#include "decode_core.h"

namespace pk {
namespace {

// Build-time tunables (defaults are the measured best on MI355X).
#ifndef PK_DECODE_WAVES
#define PK_DECODE_WAVES 4       // max wavefronts (4 kv heads each) per work-group
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

// Split mode: grid (splits x sequences, kv-head groups); a work-group takes split `split` of
// one sequence (split_tokens keys after the shared prefix, if any).
template <int G, int U, int R, bool PAGED, bool FUSED>
__global__ __launch_bounds__(kWave* kDecodeMaxWaves) void decode_split_kernel(const AttnArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // wave-uniform (SGPR)
  // The launch divides the kv heads evenly over the waves: every wave has >= 1 live row.
  const int g_first = (blockIdx.y * (blockDim.x / kWave) + wave) * (4 / R);  // first kv head of the wave
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
  decode_unit<G, U, R, PAGED, FUSED>(a, lane, g_first, b, q0, k0, Lk, t_begin, t_end, nsplit == 1,
                                     ((int64_t)b * a.max_splits + slot) * a.num_heads);
}

// Flat mode (flat_decode_piece): the batch's decode keys laid end to end and cut into
// flat_groups runs of equal length, one work-group per (sequence, run) piece, so that every
// work-group streams the same number of K/V rows whatever the length mix (the split grid
// gives each sequence whole splits: its last split is ragged, short sequences leave many
// work-groups empty, and prefill rows of a mixed batch or keys past max_seqlen_k take no
// place on the line). (174 VGPRs for G = 2, two wavefronts per SIMD: the 1024-work-group
// grid of two-wavefront groups fits 4 per CU.)
template <int G, int U, int R, bool PAGED, bool FUSED>
__global__ __launch_bounds__(kWave* kDecodeMaxWaves) void decode_flat_kernel(const AttnArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int g_first = (blockIdx.y * (blockDim.x / kWave) + wave) * (4 / R);
  flat_decode_piece<G, U, R, PAGED, FUSED>(a, blockIdx.x, g_first, lane, blockIdx.y == 0 && wave == 0);
}

// EAGER > 0 (small split-grid batches without a shared prefix, max_splits <= EAGER): the
// partial slots' loads go out with the lengths (combine_row_eager).
template <int EAGER>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(const AttnArgs a) {
  if constexpr (EAGER > 0)
    combine_row_eager<EAGER>(a, blockIdx.y, blockIdx.x, threadIdx.x);
  else
    combine_row(a, blockIdx.y, blockIdx.x, threadIdx.x);
}

// Small split-grid batches (at most 1024 split work-groups, no shared prefix, 17 to
// kCombineFast splits per sequence, e.g. 8 rows of up to 2048 keys in 64-key splits): the
// combine is a latency-bound chain of memory round trips, and its eager form takes one of
// them off. With 16 or fewer splits it measured no faster.
bool eager_combine(const AttnArgs& a) {
  return a.flat_groups <= 0 && a.prefix_keys <= 0 && a.max_splits > 16 && a.max_splits <= kCombineFast &&
         (int64_t)a.grid_splits * a.num_seqs <= 1024;
}

template <int G, int U, int R>
hipError_t launch_decode_g(AttnArgs a, bool paged, hipStream_t stream) {
  const bool flat = a.flat_groups > 0;
  const int64_t units = flat ? (int64_t)a.num_seqs + a.flat_groups : (int64_t)a.num_seqs * a.max_splits;  // decode kernel's
  a.store_through = units * a.num_heads * kHeadDim * 4 > kStoreThroughBytes;
  constexpr int NH = 4 / R;                     // kv heads per wavefront
  const int quads = (a.num_kv_heads + NH - 1) / NH;  // wavefronts needed for all kv heads
  int waves = quads < kDecodeMaxWaves ? quads : kDecodeMaxWaves;
  while (quads % waves != 0) --waves;            // no idle wavefront in any work-group
  const int zgroups = quads / waves;
  const dim3 block((unsigned)(waves * kWave));
  const bool fused = a.qkv != nullptr || a.new_k != nullptr;  // paged only (checked by their entry points)
  if (flat) {
    const dim3 grid((unsigned)(a.flat_groups + a.num_seqs + 1), (unsigned)zgroups);  // + the recorder
    if (fused)
      hipLaunchKernelGGL((decode_flat_kernel<G, U, R, true, true>), grid, block, 0, stream, a);
    else if (paged)
      hipLaunchKernelGGL((decode_flat_kernel<G, U, R, true, false>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((decode_flat_kernel<G, U, R, false, false>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
  if (a.grid_splits <= 0) return hipSuccess;  // every decode key lies in the shared prefix
  const dim3 grid((unsigned)(a.grid_splits * a.num_seqs), (unsigned)zgroups);
  if (fused)
    hipLaunchKernelGGL((decode_split_kernel<G, U, R, true, true>), grid, block, 0, stream, a);
  else if (paged)
    hipLaunchKernelGGL((decode_split_kernel<G, U, R, true, false>), grid, block, 0, stream, a);
  else
    hipLaunchKernelGGL((decode_split_kernel<G, U, R, false, false>), grid, block, 0, stream, a);
  return hipGetLastError();
}

// One or two kv heads (a tensor-parallel rank's share) spread their keys over the
// wavefront's four DPP rows (decode_key_rows); otherwise one row per kv head.
template <int G, int U>
hipError_t launch_decode_gr(const AttnArgs& a, bool paged, hipStream_t stream) {
  switch (decode_key_rows(a.num_kv_heads)) {
    case 4: return launch_decode_g<G, U, 4>(a, paged, stream);
    case 2: return launch_decode_g<G, U, 2>(a, paged, stream);
    default: return launch_decode_g<G, U, 1>(a, paged, stream);
  }
}

}  // namespace

int decode_split_tokens(int num_seqs, int max_seqlen_k) {
  // PK_DECODE_SPLIT_MAX keys per work-group when the batch yields enough work-groups to
  // cover the 256 CUs several times, shorter splits for small batches; longer ones when
  // sequences would have more than kCombineMaxSplits partials (what the combine is sized for).
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

hipError_t launch_decode_combine(const AttnArgs& a, int group, hipStream_t stream) {
  (void)group;
  if (a.num_seqs <= 0) return hipSuccess;
  // (a call with prefill rows merges the decode partials in its prefill merge kernel)
  if ((a.max_splits > 1 || a.flat_groups > 0) && !a.combine_in_merge) {
    const dim3 grid((unsigned)a.num_heads, (unsigned)a.num_seqs), block(kCombineThreads);
    if (!eager_combine(a))
      hipLaunchKernelGGL((decode_combine_kernel<0>), grid, block, 0, stream, a);
    else if (a.max_splits <= 32)
      hipLaunchKernelGGL((decode_combine_kernel<32>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((decode_combine_kernel<kCombineFast>), grid, block, 0, stream, a);
    return hipGetLastError();
  }
  return hipSuccess;
}

hipError_t launch_decode(const AttnArgs& args, int group, bool paged, int max_seqlen_k,
                         hipStream_t stream) {
  if (args.num_seqs <= 0 || max_seqlen_k <= 0) return hipSuccess;
  AttnArgs a = args;
  a.flat_step = decode_flat_step(group, a.num_kv_heads);
  hipError_t err;
  switch (group) {
    case 1: err = launch_decode_gr<1, decode_step_keys(1)>(a, paged, stream); break;
    case 2: err = launch_decode_gr<2, decode_step_keys(2)>(a, paged, stream); break;
    case 4: err = launch_decode_gr<4, decode_step_keys(4)>(a, paged, stream); break;
    case 8: err = launch_decode_gr<8, decode_step_keys(8)>(a, paged, stream); break;
    default: return hipErrorInvalidValue;
  }
  if (err != hipSuccess) return err;
  return launch_decode_combine(a, group, stream);
}

}  // namespace pk
