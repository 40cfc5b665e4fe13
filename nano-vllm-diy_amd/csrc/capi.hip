// extern "C" entry points of libpagedkv.so (declared in include/pagedkv.h).
//
// Each entry point validates its arguments on the host (shapes, strides, 16-byte
// alignment of every vector-loaded pointer), fills the kernel argument block and
// enqueues on the caller's stream. Nothing here allocates, synchronises or reads
// device memory, so every call can be recorded into a hipGraph.
#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <numeric>
#include <string>

#include "../../include/pagedkv.h"
#include "common.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_status(hipError_t err, const char* what) {
  if (err == hipSuccess) return PK_OK;
  return fail(PK_ERR_HIP, "%s: %s", what, hipGetErrorString(err));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr size_t kWorkspaceAlign = 256;
constexpr int kMaxSeqs = 65535;
constexpr int kMaxSeqlen = 65535 * 64;  // key tiles of 64 keys fit in 16 bits

size_t round_up(size_t x, size_t a) { return (x + a - 1) / a * a; }

struct WorkspaceLayout {
  int split_tokens;
  int max_splits;
  size_t part_o_bytes;
  size_t part_ml_bytes;
  // chunked-prefill plan region (only when max_seqlen_q > 1)
  int64_t pf_item_cap;
  size_t pf_queue_off, pf_items_off, pf_merges_off, pf_part_o_off, pf_part_ml_off;
  pk::FlatDecodePlan flat;  // flat decode grid (flat.groups == 0: split grid only)
  size_t flat_meta_off;
  size_t total;
};

// [decode: partial numerators | partial (max, sum) | flat-grid record]
// (empty when no sequence can have more than one split: those write their output directly).
// Partial units: the split grid's num_seqs x max_splits (shared-prefix chunks in the first
// slots of each sequence); with the flat grid, the shared-prefix chunks (num_seqs x
// prefix_slots <= num_seqs x max_splits) followed by the grid's num_seqs + groups pieces.
// [prefill: queue header | work items | merge list | partial numerators | (max, sum)]
WorkspaceLayout workspace_layout(int num_seqs, int num_heads, int head_dim, int max_seqlen_q, int max_seqlen_k) {
  WorkspaceLayout w{};
  w.split_tokens = pk::decode_split_tokens(num_seqs, max_seqlen_k);
  w.max_splits = max_seqlen_k > 0 ? (max_seqlen_k + w.split_tokens - 1) / w.split_tokens : 0;
  w.flat = pk::decode_flat_plan(num_seqs, max_seqlen_k);  // groups > 0 only when max_splits > 1
  if (w.max_splits > 1) {  // single-split sequences write their output directly
    size_t seq_units = (size_t)num_seqs * (size_t)w.max_splits;
    if (w.flat.groups > 0) seq_units += (size_t)num_seqs + (size_t)w.flat.groups;
    const size_t units = seq_units * (size_t)num_heads;
    w.part_o_bytes = round_up(units * (size_t)head_dim * sizeof(uint16_t), kWorkspaceAlign);  // bf16
    w.part_ml_bytes = round_up(units * 2 * sizeof(float), kWorkspaceAlign);
  }
  size_t off = w.part_o_bytes + w.part_ml_bytes;
  if (w.flat.groups > 0) {  // the flat grid's run length and key-line positions, for the combine
    w.flat_meta_off = off;
    off += round_up(((size_t)num_seqs + 2) * sizeof(int32_t), kWorkspaceAlign);
  }
  if (max_seqlen_q > 1) {
    w.pf_item_cap = pk::prefill_item_cap(num_seqs, num_heads, max_seqlen_q);
    w.pf_queue_off = off;
    off += round_up(pk::kPrefillQueueInts * sizeof(int32_t), kWorkspaceAlign);
    w.pf_items_off = off;
    off += round_up((size_t)w.pf_item_cap * 16, kWorkspaceAlign);
    w.pf_merges_off = off;
    off += round_up((size_t)pk::kPrefillMergeCap * 16, kWorkspaceAlign);
    w.pf_part_o_off = off;
    off += (size_t)pk::kPrefillPartCap * 32 * pk::kPrefillRows * 4 * sizeof(uint16_t);
    w.pf_part_ml_off = off;
    off += round_up((size_t)pk::kPrefillPartCap * pk::kPrefillRows * 2 * sizeof(float), kWorkspaceAlign);
  }
  w.total = off;
  return w;
}

// The one-launch decode steps write the token's row at block * block_stride + offset *
// row_stride, where pk_store_kvcache / pk_qk_norm_rope_store write at slot * row: the two
// agree only for caches whose rows and blocks are contiguous, which both entry points
// therefore require (the reference's runner allocates the cache that way,
// model_runner.py:159-165, and asserts the row stride, attention.py:53).
int check_contiguous_cache(const char* what, int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                           int64_t v_block_stride, int32_t block_size, int32_t num_kv_heads, int32_t head_dim) {
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (k_row_stride != row || v_row_stride != row || k_block_stride != (int64_t)block_size * row ||
      v_block_stride != (int64_t)block_size * row)
    return fail(PK_ERR_INVALID_ARG,
                "%s: caches must have contiguous rows and blocks (row stride %lld, block stride %lld; got %lld/%lld, "
                "%lld/%lld)",
                what, (long long)row, (long long)block_size * row, (long long)k_row_stride, (long long)v_row_stride,
                (long long)k_block_stride, (long long)v_block_stride);
  return PK_OK;
}

// Shared argument checks of the decode-step linear entry points; 0 when valid.
int check_linear(const char* what, const void* x, int64_t x_row_stride, const void* weight,
                 int64_t weight_row_stride, int32_t rows, int32_t n_out, int32_t k,
                 const void* out, int64_t out_row_stride, void* workspace, size_t workspace_bytes,
                 size_t need) {
  if (rows < 0) return fail(PK_ERR_INVALID_ARG, "%s: rows=%d < 0", what, rows);
  if (rows > pk::kLinearMaxRows)
    return fail(PK_ERR_UNSUPPORTED, "%s: rows=%d above %d (a decode-step kernel)", what, rows, pk::kLinearMaxRows);
  if (n_out <= 0 || n_out % 32 != 0)
    return fail(PK_ERR_UNSUPPORTED, "%s: n_out=%d must be a positive multiple of 32", what, n_out);
  if (k <= 0 || k % 256 != 0) return fail(PK_ERR_UNSUPPORTED, "%s: k=%d must be a positive multiple of 256", what, k);
  if (!x || !weight || !out) return fail(PK_ERR_INVALID_ARG, "%s: null x / weight / out", what);
  if (x_row_stride < k || x_row_stride % 8 || weight_row_stride < k || weight_row_stride % 8 ||
      out_row_stride < n_out || out_row_stride % 8)
    return fail(PK_ERR_INVALID_ARG, "%s: row strides must cover their rows and be multiples of 8", what);
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out))
    return fail(PK_ERR_INVALID_ARG, "%s: x / weight / out must be 16-byte aligned", what);
  // out is written while other work-groups still read x: the two must not overlap
  const auto xb = reinterpret_cast<uintptr_t>(x), ob = reinterpret_cast<uintptr_t>(out);
  const uintptr_t x_end = xb + ((uintptr_t)(rows - 1) * x_row_stride + k) * 2;
  const uintptr_t o_end = ob + ((uintptr_t)(rows - 1) * out_row_stride + n_out) * 2;
  if (rows > 0 && xb < o_end && ob < x_end) return fail(PK_ERR_INVALID_ARG, "%s: out overlaps x", what);
  if (workspace_bytes < need)
    return fail(PK_ERR_WORKSPACE, "%s: workspace of %zu bytes needed, %zu given", what, need, workspace_bytes);
  if (need && (!workspace || !aligned16(workspace)))
    return fail(PK_ERR_WORKSPACE, "%s: workspace must be non-null and 16-byte aligned", what);
  return PK_OK;
}

}  // namespace

extern "C" {

int pk_abi_version(void) { return 9; }

const char* pk_last_error(void) { return g_last_error.c_str(); }

int pk_store_kvcache(const void* key, int64_t key_row_stride, const void* value,
                     int64_t value_row_stride, void* k_cache, void* v_cache,
                     const int32_t* slot_mapping, int32_t num_tokens, int32_t row_elems,
                     int64_t num_slots, pk_stream_t stream) {
  g_last_error.clear();
  if (num_tokens < 0) return fail(PK_ERR_INVALID_ARG, "store_kvcache: num_tokens=%d < 0", num_tokens);
  if (num_tokens == 0) return PK_OK;
  if (!key || !value || !k_cache || !v_cache || !slot_mapping)
    return fail(PK_ERR_INVALID_ARG, "store_kvcache: null pointer argument");
  if (row_elems <= 0 || row_elems % 8 != 0)
    return fail(PK_ERR_INVALID_ARG, "store_kvcache: row_elems=%d must be a positive multiple of 8", row_elems);
  if (key_row_stride < row_elems || value_row_stride < row_elems)
    return fail(PK_ERR_INVALID_ARG, "store_kvcache: row strides (%lld, %lld) smaller than row_elems=%d",
                (long long)key_row_stride, (long long)value_row_stride, row_elems);
  if (key_row_stride % 8 != 0 || value_row_stride % 8 != 0)
    return fail(PK_ERR_INVALID_ARG, "store_kvcache: row strides (%lld, %lld) must be multiples of 8 elements",
                (long long)key_row_stride, (long long)value_row_stride);
  if (!aligned16(key) || !aligned16(value) || !aligned16(k_cache) || !aligned16(v_cache))
    return fail(PK_ERR_INVALID_ARG, "store_kvcache: key/value/cache pointers must be 16-byte aligned");
  if (num_slots < 0) return fail(PK_ERR_INVALID_ARG, "store_kvcache: num_slots < 0");
  return hip_status(pk::launch_store_kvcache(key, key_row_stride, value, value_row_stride, k_cache,
                                             v_cache, slot_mapping, num_tokens, row_elems,
                                             num_slots, reinterpret_cast<hipStream_t>(stream)),
                    "store_kvcache launch");
}

int pk_gather_kv(const void* cache, int64_t block_stride, int32_t block_size,
                 const int32_t* block_table, int32_t block_table_stride,
                 const int32_t* cu_seqlens_k, int32_t num_seqs, int32_t max_seqlen_k,
                 int32_t row_elems, void* dst, pk_stream_t stream) {
  g_last_error.clear();
  if (num_seqs < 0 || max_seqlen_k < 0)
    return fail(PK_ERR_INVALID_ARG, "gather_kv: negative num_seqs or max_seqlen_k");
  if (num_seqs == 0 || max_seqlen_k == 0) return PK_OK;
  if (num_seqs > 65535) return fail(PK_ERR_INVALID_ARG, "gather_kv: num_seqs=%d > 65535", num_seqs);
  if (!cache || !block_table || !cu_seqlens_k || !dst)
    return fail(PK_ERR_INVALID_ARG, "gather_kv: null pointer argument");
  if (row_elems <= 0 || row_elems % 8 != 0 || block_stride % 8 != 0 || block_size <= 0 ||
      block_stride < (int64_t)block_size * row_elems)
    return fail(PK_ERR_INVALID_ARG, "gather_kv: bad row_elems=%d / block_size=%d / block_stride=%lld",
                row_elems, block_size, (long long)block_stride);
  if (!aligned16(cache) || !aligned16(dst))
    return fail(PK_ERR_INVALID_ARG, "gather_kv: cache and dst must be 16-byte aligned");
  return hip_status(pk::launch_gather_kv(cache, block_stride, block_size, block_table,
                                         block_table_stride, cu_seqlens_k, num_seqs, max_seqlen_k,
                                         row_elems, dst, reinterpret_cast<hipStream_t>(stream)),
                    "gather_kv launch");
}

size_t pk_varlen_attention_workspace_bytes(int32_t num_seqs, int32_t num_heads, int32_t head_dim,
                                           int32_t max_seqlen_q, int32_t max_seqlen_k) {
  if (num_seqs <= 0 || num_heads <= 0 || head_dim <= 0 || max_seqlen_k <= 0 || max_seqlen_q < 0) return 0;
  return workspace_layout(num_seqs, num_heads, head_dim, max_seqlen_q, max_seqlen_k).total;
}

int pk_varlen_attention(const void* q, int64_t q_row_stride, const void* k, const void* v,
                        int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                        int64_t v_block_stride, const int32_t* block_table,
                        int32_t block_table_stride, int32_t block_size,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                        int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                        int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
                        int32_t causal, void* out, int64_t out_row_stride, void* workspace,
                        size_t workspace_bytes, pk_stream_t stream) {
  return pk_varlen_attention_ex(q, q_row_stride, k, v, k_row_stride, v_row_stride, k_block_stride,
                                v_block_stride, block_table, block_table_stride, block_size, cu_seqlens_q,
                                cu_seqlens_k, num_seqs, max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads,
                                head_dim, softmax_scale, causal, out, out_row_stride, workspace,
                                workspace_bytes, PK_CACHED_PREFIX_KEYS_DEFAULT, stream);
}

namespace {

// Inputs of the fused decode step's producer (pk_qkv_decode_attention).
struct FusedProducer {
  const void* qkv;
  int64_t qkv_row_stride;
  const int64_t* positions;
  const float* cos_sin;
  int64_t max_position;
  const void* q_norm;
  const void* k_norm;
  float eps;
  const int32_t* slot_mapping;
  int64_t num_slots;
  const void* new_k;            // store + decode: the tokens' K / V rows (qkv == nullptr)
  int64_t new_k_stride;
  const void* new_v;
  int64_t new_v_stride;
};

// Shared body of pk_varlen_attention_ex and pk_qkv_decode_attention (fp != nullptr: q comes
// from the fused producer, q itself is unused).
int attention_impl(const void* q, int64_t q_row_stride, const void* k, const void* v, int64_t k_row_stride,
                   int64_t v_row_stride, int64_t k_block_stride, int64_t v_block_stride,
                   const int32_t* block_table, int32_t block_table_stride, int32_t block_size,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                   int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads,
                   int32_t head_dim, float softmax_scale, int32_t causal, void* out, int64_t out_row_stride,
                   void* workspace, size_t workspace_bytes, int32_t cached_prefix_keys, const FusedProducer* fp,
                   int32_t shared_prefix_keys, pk_stream_t stream) {
  if (head_dim != pk::kHeadDim)
    return fail(PK_ERR_UNSUPPORTED, "varlen_attention: head_dim=%d not built (only %d)", head_dim, pk::kHeadDim);
  if (num_seqs < 0 || max_seqlen_q < 0 || max_seqlen_k < 0)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: negative num_seqs / max_seqlen");
  if (num_seqs > kMaxSeqs) return fail(PK_ERR_INVALID_ARG, "varlen_attention: num_seqs=%d > %d", num_seqs, kMaxSeqs);
  if (num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads != 0)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: num_heads=%d not a multiple of num_kv_heads=%d",
                num_heads, num_kv_heads);
  const int group = num_heads / num_kv_heads;
  if (group != 1 && group != 2 && group != 4 && group != 8)
    return fail(PK_ERR_UNSUPPORTED, "varlen_attention: GQA group %d not built (1, 2, 4, 8)", group);
  if (num_seqs == 0 || max_seqlen_q == 0 || max_seqlen_k == 0) return PK_OK;
  if ((!q && !(fp && fp->qkv)) || !k || !v || !out || !cu_seqlens_q || !cu_seqlens_k)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: null pointer argument");
  // the prefill work list packs key-tile indices in 16 bits and the kv head in 8
  if (max_seqlen_k > kMaxSeqlen || max_seqlen_q > kMaxSeqlen)
    return fail(PK_ERR_UNSUPPORTED, "varlen_attention: max_seqlen_q=%d / max_seqlen_k=%d above %d",
                max_seqlen_q, max_seqlen_k, kMaxSeqlen);
  if (num_kv_heads > 255)
    return fail(PK_ERR_UNSUPPORTED, "varlen_attention: num_kv_heads=%d above 255", num_kv_heads);
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(out))
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: q/k/v/out must be 16-byte aligned");
  if (fp && fp->qkv) q_row_stride = (int64_t)num_heads * head_dim;  // unused: q comes from qkv
  const int64_t kv_row = (int64_t)num_kv_heads * head_dim;
  if (q_row_stride < (int64_t)num_heads * head_dim || out_row_stride < (int64_t)num_heads * head_dim ||
      k_row_stride < kv_row || v_row_stride < kv_row)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: a row stride is smaller than its row");
  if (q_row_stride % 8 || out_row_stride % 8 || k_row_stride % 8 || v_row_stride % 8)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: row strides must be multiples of 8 elements");
  if (k_row_stride >= (1 << 22) || v_row_stride >= (1 << 22))
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: K/V row strides must be below 2^22 elements");
  const bool paged = block_table != nullptr;
  if (paged) {
    if (block_size <= 0 || block_size % 64 != 0)
      return fail(PK_ERR_INVALID_ARG, "varlen_attention: block_size=%d must be a positive multiple of 64",
                  block_size);
    if (block_table_stride < (max_seqlen_k + block_size - 1) / block_size)
      return fail(PK_ERR_INVALID_ARG,
                  "varlen_attention: block_table_stride=%d < ceil(max_seqlen_k=%d / block_size=%d)",
                  block_table_stride, max_seqlen_k, block_size);
    if (k_block_stride % 8 || v_block_stride % 8 || k_block_stride < (int64_t)block_size * k_row_stride ||
        v_block_stride < (int64_t)block_size * v_row_stride)
      return fail(PK_ERR_INVALID_ARG, "varlen_attention: bad cache block strides (%lld, %lld)",
                  (long long)k_block_stride, (long long)v_block_stride);
  }
  if (!(softmax_scale > 0.f) || !std::isfinite(softmax_scale))
    return fail(PK_ERR_INVALID_ARG, "varlen_attention: softmax_scale must be positive and finite");
  if (fp) {  // a one-launch decode step stores into the cache it reads
    if (int rc = check_contiguous_cache(fp->qkv ? "qkv_decode_attention" : "store_decode_attention", k_row_stride,
                                        v_row_stride, k_block_stride, v_block_stride, block_size, num_kv_heads,
                                        head_dim))
      return rc;
  }

  const WorkspaceLayout ws = workspace_layout(num_seqs, num_heads, head_dim, max_seqlen_q, max_seqlen_k);
  if (ws.total > 0) {
    if (!workspace || workspace_bytes < ws.total)
      return fail(PK_ERR_WORKSPACE, "varlen_attention: workspace of %zu bytes needed, %zu given",
                  ws.total, workspace ? workspace_bytes : (size_t)0);
    if ((reinterpret_cast<uintptr_t>(workspace) % kWorkspaceAlign) != 0)
      return fail(PK_ERR_WORKSPACE, "varlen_attention: workspace must be %zu-byte aligned", kWorkspaceAlign);
  }

  if (max_seqlen_q > 1 && ws.pf_item_cap > INT32_MAX)
    return fail(PK_ERR_UNSUPPORTED, "varlen_attention: prefill work list of %lld items too large",
                (long long)ws.pf_item_cap);

  pk::AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.q_row_stride = q_row_stride;
  a.k = static_cast<const uint16_t*>(k);
  a.v = static_cast<const uint16_t*>(v);
  a.k_row_stride = k_row_stride;
  a.v_row_stride = v_row_stride;
  a.k_block_stride = paged ? k_block_stride : 0;
  a.v_block_stride = paged ? v_block_stride : 0;
  a.block_table = block_table;
  a.bt_stride = paged ? block_table_stride : 0;
  a.block_size = paged ? block_size : 0;
  a.cu_q = cu_seqlens_q;
  a.cu_k = cu_seqlens_k;
  a.num_seqs = num_seqs;
  a.max_seqlen_k = max_seqlen_k;
  a.num_heads = num_heads;
  a.num_kv_heads = num_kv_heads;
  a.scale_log2 = softmax_scale * 1.4426950408889634f;
  a.out = static_cast<uint16_t*>(out);
  a.out_row_stride = out_row_stride;
  a.stream_from = cached_prefix_keys;
  if (fp) {
    a.qkv = static_cast<const uint16_t*>(fp->qkv);
    a.qkv_row_stride = fp->qkv_row_stride;
    a.positions = fp->positions;
    a.cos_sin = fp->cos_sin;
    a.max_position = fp->max_position;
    a.q_norm = static_cast<const uint16_t*>(fp->q_norm);
    a.k_norm = static_cast<const uint16_t*>(fp->k_norm);
    a.norm_eps = fp->eps;
    a.slot_mapping = fp->slot_mapping;
    a.num_slots = fp->num_slots;
    a.new_k = static_cast<const uint16_t*>(fp->new_k);
    a.new_k_stride = fp->new_k_stride;
    a.new_v = static_cast<const uint16_t*>(fp->new_v);
    a.new_v_stride = fp->new_v_stride;
  }
  a.split_tokens = ws.split_tokens;
  a.max_splits = ws.max_splits > 0 ? ws.max_splits : 1;
  a.grid_splits = a.max_splits;
  a.prefix_chunk = 1;
  a.prefix_stride = a.max_splits;
  if (shared_prefix_keys > 0 && paged && !fp && ws.max_splits > 1 && num_seqs <= pk::kSharedPrefixMaxSeqs) {
    // Shared-prefix decode. Chunks of CK = lcm(block_size, split) keys and a prefix of a
    // whole number of chunks keep the partial slots within the workspace's: P / CK prefix
    // slots + ceil((max_k - P) / split) split slots <= ceil(max_k / split).
    const int s = ws.split_tokens;
    const int ck = block_size / std::gcd(block_size, s) * s;
    const int P = std::min(shared_prefix_keys, max_seqlen_k) / ck * ck;
    if (P > 0 && ck / block_size <= pk::kSharedPrefixMaxChunkBlocks) {
      a.prefix_keys = P;
      a.prefix_chunk = ck;
      a.prefix_slots = P / ck;
      a.grid_splits = (max_seqlen_k - P + s - 1) / s;
      if (a.prefix_slots + a.grid_splits > a.max_splits)
        return fail(PK_ERR_HIP, "varlen_attention: shared-prefix slots %d + %d exceed %d", a.prefix_slots,
                    a.grid_splits, a.max_splits);
    }
  }
  char* const wsb = static_cast<char*>(workspace);
  if (ws.part_o_bytes > 0) {
    a.part_o = reinterpret_cast<uint16_t*>(wsb);
    a.part_ml = reinterpret_cast<float*>(wsb + ws.part_o_bytes);
  }
  if (ws.flat.groups > 0) {  // the flat decode grid: pieces after the shared-prefix chunks, if any
    a.flat_groups = ws.flat.groups;
    a.flat_min_chunk = ws.flat.min_chunk;
    a.flat_meta = reinterpret_cast<int32_t*>(wsb + ws.flat_meta_off);
    if (a.prefix_keys > 0) {
      a.prefix_stride = a.prefix_slots;
      a.flat_unit0 = num_seqs * a.prefix_slots;
    }
  }
  if (max_seqlen_q > 1) {
    a.pf_queue = reinterpret_cast<int32_t*>(wsb + ws.pf_queue_off);
    a.pf_items = reinterpret_cast<int4*>(wsb + ws.pf_items_off);
    a.pf_merges = reinterpret_cast<int4*>(wsb + ws.pf_merges_off);
    a.pf_part_o = reinterpret_cast<uint16_t*>(wsb + ws.pf_part_o_off);
    a.pf_part_ml = reinterpret_cast<float*>(wsb + ws.pf_part_ml_off);
    a.pf_item_cap = (int32_t)std::min<int64_t>(ws.pf_item_cap, INT32_MAX);
    a.pf_merge_cap = pk::kPrefillMergeCap;
    a.pf_part_cap = pk::kPrefillPartCap;
  }

  const hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // with prefill rows the decode partials are merged by the prefill merge kernel, which the
  // call launches anyway (one launch fewer)
  a.combine_in_merge = max_seqlen_q > 1;
  int rc = PK_OK;
  hipError_t e = hipSuccess;
  if (a.prefix_keys > 0 && pk::launch_shared_prefix_flat(a, group, s, &e)) {
    // the shared-prefix work and the flat decode grid in one launch, then the combine
    rc = hip_status(e, "shared-prefix + flat decode launch");
    if (rc != PK_OK) return rc;
    rc = hip_status(pk::launch_decode_combine(a, group, s), "decode combine launch");
  } else {
    if (a.prefix_keys > 0) {
      rc = hip_status(pk::launch_shared_prefix(a, group, s), "shared-prefix launch");
      if (rc != PK_OK) return rc;
    }
    rc = hip_status(pk::launch_decode(a, group, paged, max_seqlen_k, s), "decode launch");
  }
  if (rc != PK_OK) return rc;
  if (max_seqlen_q > 1)
    rc = hip_status(pk::launch_prefill(a, group, paged, causal != 0, max_seqlen_q, s), "prefill launch");
  return rc;
}

}  // namespace

int pk_varlen_attention_ex(const void* q, int64_t q_row_stride, const void* k, const void* v,
                           int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                           int64_t v_block_stride, const int32_t* block_table,
                           int32_t block_table_stride, int32_t block_size,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                           int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, float softmax_scale,
                           int32_t causal, void* out, int64_t out_row_stride, void* workspace,
                           size_t workspace_bytes, int32_t cached_prefix_keys, pk_stream_t stream) {
  g_last_error.clear();
  return attention_impl(q, q_row_stride, k, v, k_row_stride, v_row_stride, k_block_stride, v_block_stride,
                        block_table, block_table_stride, block_size, cu_seqlens_q, cu_seqlens_k, num_seqs,
                        max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, causal, out,
                        out_row_stride, workspace, workspace_bytes, cached_prefix_keys, nullptr, 0, stream);
}

int pk_varlen_attention_shared_prefix(const void* q, int64_t q_row_stride, const void* k, const void* v,
                                      int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                                      int64_t v_block_stride, const int32_t* block_table,
                                      int32_t block_table_stride, int32_t block_size,
                                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                                      int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                                      int32_t num_kv_heads, int32_t head_dim, float softmax_scale, int32_t causal,
                                      void* out, int64_t out_row_stride, void* workspace, size_t workspace_bytes,
                                      int32_t cached_prefix_keys, int32_t shared_prefix_keys, pk_stream_t stream) {
  g_last_error.clear();
  if (shared_prefix_keys < 0)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention_shared_prefix: shared_prefix_keys=%d < 0", shared_prefix_keys);
  if (block_table == nullptr && shared_prefix_keys > 0)
    return fail(PK_ERR_INVALID_ARG, "varlen_attention_shared_prefix: a shared prefix needs paged K/V (block_table)");
  return attention_impl(q, q_row_stride, k, v, k_row_stride, v_row_stride, k_block_stride, v_block_stride,
                        block_table, block_table_stride, block_size, cu_seqlens_q, cu_seqlens_k, num_seqs,
                        max_seqlen_q, max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, causal, out,
                        out_row_stride, workspace, workspace_bytes, cached_prefix_keys, nullptr, shared_prefix_keys,
                        stream);
}

int pk_qkv_decode_attention(const void* qkv, int64_t qkv_row_stride, const int64_t* positions,
                            const float* cos_sin, int64_t max_position, const void* q_norm_weight,
                            const void* k_norm_weight, float eps, void* k_cache, void* v_cache,
                            int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                            int64_t v_block_stride, const int32_t* slot_mapping, int64_t num_slots,
                            const int32_t* block_table, int32_t block_table_stride, int32_t block_size,
                            const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                            int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                            float softmax_scale, void* out, int64_t out_row_stride, void* workspace,
                            size_t workspace_bytes, int32_t cached_prefix_keys, pk_stream_t stream) {
  g_last_error.clear();
  if (num_seqs <= 0 || max_seqlen_k <= 0) return num_seqs < 0 || max_seqlen_k < 0 ?
      fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: negative num_seqs / max_seqlen_k") : PK_OK;
  if (!qkv || !positions || !cos_sin || !slot_mapping || !block_table)
    return fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: null qkv / positions / cos_sin / slot_mapping / block_table");
  if (max_position <= 0) return fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: max_position must be positive");
  if (!(eps >= 0.f)) return fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: eps must be >= 0");
  if (num_slots < 0) return fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: num_slots < 0");
  const int64_t row = (int64_t)(num_heads + 2 * num_kv_heads) * head_dim;
  if (qkv_row_stride < row || qkv_row_stride % 8 != 0)
    return fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: qkv_row_stride=%lld must be >= %lld and a multiple of 8",
                (long long)qkv_row_stride, (long long)row);
  if (!aligned16(qkv) || !aligned16(cos_sin) || (q_norm_weight && !aligned16(q_norm_weight)) ||
      (k_norm_weight && !aligned16(k_norm_weight)))
    return fail(PK_ERR_INVALID_ARG, "qkv_decode_attention: qkv / cos_sin / norm weights must be 16-byte aligned");
  const FusedProducer fp{qkv, qkv_row_stride, positions, cos_sin, max_position, q_norm_weight, k_norm_weight,
                         eps, slot_mapping, num_slots, nullptr, 0, nullptr, 0};
  return attention_impl(nullptr, 0, k_cache, v_cache, k_row_stride, v_row_stride, k_block_stride, v_block_stride,
                        block_table, block_table_stride, block_size, cu_seqlens_q, cu_seqlens_k, num_seqs, 1,
                        max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, 1, out, out_row_stride,
                        workspace, workspace_bytes, cached_prefix_keys, &fp, 0, stream);
}

int pk_store_decode_attention(const void* q, int64_t q_row_stride, const void* key, int64_t key_row_stride,
                              const void* value, int64_t value_row_stride, void* k_cache, void* v_cache,
                              int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                              int64_t v_block_stride, const int32_t* slot_mapping, int64_t num_slots,
                              const int32_t* block_table, int32_t block_table_stride, int32_t block_size,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t num_seqs,
                              int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              float softmax_scale, void* out, int64_t out_row_stride, void* workspace,
                              size_t workspace_bytes, int32_t cached_prefix_keys, pk_stream_t stream) {
  g_last_error.clear();
  if (num_seqs <= 0 || max_seqlen_k <= 0) return num_seqs < 0 || max_seqlen_k < 0 ?
      fail(PK_ERR_INVALID_ARG, "store_decode_attention: negative num_seqs / max_seqlen_k") : PK_OK;
  if (!key || !value || !slot_mapping || !block_table)
    return fail(PK_ERR_INVALID_ARG, "store_decode_attention: null key / value / slot_mapping / block_table");
  if (num_slots < 0) return fail(PK_ERR_INVALID_ARG, "store_decode_attention: num_slots < 0");
  const int64_t row = (int64_t)num_kv_heads * head_dim;
  if (key_row_stride < row || value_row_stride < row || key_row_stride % 8 || value_row_stride % 8)
    return fail(PK_ERR_INVALID_ARG, "store_decode_attention: key/value row strides must be >= %lld and multiples of 8",
                (long long)row);
  if (!aligned16(key) || !aligned16(value))
    return fail(PK_ERR_INVALID_ARG, "store_decode_attention: key / value must be 16-byte aligned");
  const FusedProducer fp{nullptr, 0, nullptr, nullptr, 0, nullptr, nullptr, 0.f, slot_mapping, num_slots,
                         key, key_row_stride, value, value_row_stride};
  return attention_impl(q, q_row_stride, k_cache, v_cache, k_row_stride, v_row_stride, k_block_stride,
                        v_block_stride, block_table, block_table_stride, block_size, cu_seqlens_q, cu_seqlens_k,
                        num_seqs, 1, max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, 1, out,
                        out_row_stride, workspace, workspace_bytes, cached_prefix_keys, &fp, 0, stream);
}

int pk_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride, const int64_t* positions,
                          const float* cos_sin, int64_t max_position, const void* q_norm_weight,
                          const void* k_norm_weight, float eps, int32_t num_tokens,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, void* q_out,
                          int64_t q_out_row_stride, void* k_out, int64_t k_out_row_stride,
                          void* k_cache, void* v_cache, const int32_t* slot_mapping,
                          int64_t num_slots, pk_stream_t stream) {
  g_last_error.clear();
  if (head_dim != pk::kHeadDim)
    return fail(PK_ERR_UNSUPPORTED, "qk_norm_rope_store: head_dim=%d not built (only %d)", head_dim, pk::kHeadDim);
  if (num_tokens < 0) return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: num_tokens=%d < 0", num_tokens);
  if (num_heads <= 0 || num_kv_heads <= 0)
    return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: num_heads=%d, num_kv_heads=%d must be positive",
                num_heads, num_kv_heads);
  if (num_tokens == 0) return PK_OK;
  if (!qkv || !positions || !cos_sin || !q_out)
    return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: null qkv / positions / cos_sin / q_out");
  if ((k_cache == nullptr) != (v_cache == nullptr))
    return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: pass both caches or neither");
  if (k_cache && !slot_mapping) return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: null slot_mapping");
  if (max_position <= 0) return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: max_position must be positive");
  if (!(eps >= 0.f)) return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: eps must be >= 0");
  if (num_slots < 0) return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: num_slots < 0");
  const int64_t row = (int64_t)(num_heads + 2 * num_kv_heads) * head_dim;
  if (qkv_row_stride < row || qkv_row_stride % 8 != 0)
    return fail(PK_ERR_INVALID_ARG, "qkv_row_stride=%lld must be >= %lld and a multiple of 8",
                (long long)qkv_row_stride, (long long)row);
  if (q_out_row_stride < (int64_t)num_heads * head_dim || q_out_row_stride % 8 != 0)
    return fail(PK_ERR_INVALID_ARG, "q_out_row_stride=%lld must be >= %d and a multiple of 8",
                (long long)q_out_row_stride, num_heads * head_dim);
  if (k_out && (k_out_row_stride < (int64_t)num_kv_heads * head_dim || k_out_row_stride % 8 != 0))
    return fail(PK_ERR_INVALID_ARG, "k_out_row_stride=%lld must be >= %d and a multiple of 8",
                (long long)k_out_row_stride, num_kv_heads * head_dim);
  if (!aligned16(qkv) || !aligned16(q_out) || (k_out && !aligned16(k_out)) ||
      (k_cache && (!aligned16(k_cache) || !aligned16(v_cache))) || !aligned16(cos_sin) ||
      (q_norm_weight && !aligned16(q_norm_weight)) || (k_norm_weight && !aligned16(k_norm_weight)))
    return fail(PK_ERR_INVALID_ARG, "qk_norm_rope_store: tensors must be 16-byte aligned");
  return hip_status(pk::launch_qk_norm_rope_store(qkv, qkv_row_stride, positions, cos_sin, max_position,
                                                  q_norm_weight, k_norm_weight, eps, num_tokens,
                                                  num_heads, num_kv_heads, q_out, q_out_row_stride,
                                                  k_out, k_out_row_stride, k_cache, v_cache,
                                                  slot_mapping, num_slots,
                                                  reinterpret_cast<hipStream_t>(stream)),
                    "qk_norm_rope_store launch");
}

int pk_add_rmsnorm(const void* x, int64_t x_row_stride, const void* residual,
                   int64_t residual_row_stride, const void* weight, float eps, int32_t rows,
                   int32_t hidden, void* out, int64_t out_row_stride, void* residual_out,
                   int64_t residual_out_row_stride, pk_stream_t stream) {
  g_last_error.clear();
  if (rows < 0) return fail(PK_ERR_INVALID_ARG, "add_rmsnorm: rows=%d < 0", rows);
  if (rows == 0) return PK_OK;
  if (hidden <= 0 || hidden % 8 != 0 || hidden > 4096)
    return fail(PK_ERR_UNSUPPORTED, "add_rmsnorm: hidden=%d must be a multiple of 8 and <= 4096", hidden);
  if (!x || !weight || !out || (residual && !residual_out))
    return fail(PK_ERR_INVALID_ARG, "add_rmsnorm: null x / weight / out, or residual without residual_out");
  if (x_row_stride < hidden || out_row_stride < hidden || x_row_stride % 8 || out_row_stride % 8 ||
      (residual && (residual_row_stride < hidden || residual_row_stride % 8 ||
                    residual_out_row_stride < hidden || residual_out_row_stride % 8)))
    return fail(PK_ERR_INVALID_ARG, "add_rmsnorm: row strides must be >= hidden and multiples of 8");
  if (!aligned16(x) || !aligned16(weight) || !aligned16(out) ||
      (residual && (!aligned16(residual) || !aligned16(residual_out))))
    return fail(PK_ERR_INVALID_ARG, "add_rmsnorm: tensors must be 16-byte aligned");
  return hip_status(pk::launch_add_rmsnorm(x, x_row_stride, residual, residual_row_stride, weight, eps,
                                           rows, hidden, out, out_row_stride, residual_out,
                                           residual_out_row_stride, reinterpret_cast<hipStream_t>(stream)),
                    "add_rmsnorm launch");
}

int pk_silu_and_mul(const void* x, int64_t x_row_stride, int32_t rows, int32_t inter, void* out,
                    int64_t out_row_stride, pk_stream_t stream) {
  g_last_error.clear();
  if (rows < 0) return fail(PK_ERR_INVALID_ARG, "silu_and_mul: rows=%d < 0", rows);
  if (rows == 0) return PK_OK;
  if (inter <= 0 || inter % 8 != 0)
    return fail(PK_ERR_UNSUPPORTED, "silu_and_mul: width %d must be a positive multiple of 8", inter);
  if (!x || !out) return fail(PK_ERR_INVALID_ARG, "silu_and_mul: null pointer argument");
  if (x_row_stride < 2 * (int64_t)inter || x_row_stride % 8 || out_row_stride < inter || out_row_stride % 8)
    return fail(PK_ERR_INVALID_ARG, "silu_and_mul: bad row strides");
  if (!aligned16(x) || !aligned16(out)) return fail(PK_ERR_INVALID_ARG, "silu_and_mul: tensors must be 16-byte aligned");
  return hip_status(pk::launch_silu_and_mul(x, x_row_stride, rows, inter, out, out_row_stride,
                                            reinterpret_cast<hipStream_t>(stream)),
                    "silu_and_mul launch");
}

int pk_lm_head_greedy(const void* hidden_states, int64_t row_stride, const int32_t* cu_seqlens_q,
                      const void* weight, int64_t weight_row_stride, int32_t rows, int32_t vocab,
                      int32_t hidden, uint64_t* keys, int32_t* token_ids, pk_stream_t stream) {
  g_last_error.clear();
  if (rows < 0 || vocab <= 0) return fail(PK_ERR_INVALID_ARG, "lm_head_greedy: rows=%d, vocab=%d", rows, vocab);
  if (rows == 0) return PK_OK;
  if (hidden <= 0 || hidden % 128 != 0)
    return fail(PK_ERR_UNSUPPORTED, "lm_head_greedy: hidden=%d must be a positive multiple of 128", hidden);
  if (!hidden_states || !weight || !keys || !token_ids)
    return fail(PK_ERR_INVALID_ARG, "lm_head_greedy: null pointer argument");
  if (row_stride < hidden || row_stride % 8 || weight_row_stride < hidden || weight_row_stride % 8)
    return fail(PK_ERR_INVALID_ARG, "lm_head_greedy: row strides must be >= hidden and multiples of 8");
  if (!aligned16(hidden_states) || !aligned16(weight) || (reinterpret_cast<uintptr_t>(keys) & 7u))
    return fail(PK_ERR_INVALID_ARG, "lm_head_greedy: hidden_states / weight 16-byte, keys 8-byte aligned");
  return hip_status(pk::launch_lm_head_greedy(hidden_states, row_stride, cu_seqlens_q, weight,
                                              weight_row_stride, rows, vocab, hidden,
                                              reinterpret_cast<unsigned long long*>(keys), token_ids,
                                              reinterpret_cast<hipStream_t>(stream)),
                    "lm_head_greedy launch");
}

size_t pk_linear_workspace_bytes(int32_t rows, int32_t n_out, int32_t k, int32_t epilogue) {
  if (rows <= 0 || rows > pk::kLinearMaxRows || n_out <= 0 || n_out % 32 || k <= 0 || k % 256) return 0;
  return pk::linear_workspace_bytes(rows, n_out, k, epilogue);
}

int pk_linear(const void* x, int64_t x_row_stride, const void* weight, int64_t weight_row_stride,
              int32_t rows, int32_t n_out, int32_t k, int32_t epilogue, void* out, int64_t out_row_stride,
              void* workspace, size_t workspace_bytes, pk_stream_t stream) {
  g_last_error.clear();
  if (epilogue != PK_LINEAR_STORE && epilogue != PK_LINEAR_SILU_MUL)
    return fail(PK_ERR_INVALID_ARG, "linear: epilogue=%d is not PK_LINEAR_STORE or PK_LINEAR_SILU_MUL", epilogue);
  const size_t need = pk_linear_workspace_bytes(rows, n_out, k, epilogue);
  if (int rc = check_linear("linear", x, x_row_stride, weight, weight_row_stride, rows, n_out, k, out,
                            out_row_stride, workspace, workspace_bytes, need))
    return rc;
  if (rows == 0) return PK_OK;
  return hip_status(pk::launch_linear(x, x_row_stride, weight, weight_row_stride, rows, n_out, k, epilogue, out,
                                      out_row_stride, workspace, reinterpret_cast<hipStream_t>(stream)),
                    "linear launch");
}

int pk_linear_add_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, int64_t weight_row_stride,
                          int32_t rows, int32_t hidden, int32_t k, const void* residual,
                          int64_t residual_row_stride, const void* norm_weight, float eps, void* out,
                          int64_t out_row_stride, void* residual_out, int64_t residual_out_row_stride,
                          void* workspace, size_t workspace_bytes, pk_stream_t stream) {
  g_last_error.clear();
  if (hidden > 4096) return fail(PK_ERR_UNSUPPORTED, "linear_add_rmsnorm: hidden=%d above 4096", hidden);
  const size_t need = pk_linear_workspace_bytes(rows, hidden, k, PK_LINEAR_ADD_RMSNORM);
  if (int rc = check_linear("linear_add_rmsnorm", x, x_row_stride, weight, weight_row_stride, rows, hidden, k, out,
                            out_row_stride, workspace, workspace_bytes, need))
    return rc;
  if (!residual || !residual_out || !norm_weight)
    return fail(PK_ERR_INVALID_ARG, "linear_add_rmsnorm: null residual / residual_out / norm_weight");
  if (residual_row_stride < hidden || residual_row_stride % 8 || residual_out_row_stride < hidden ||
      residual_out_row_stride % 8)
    return fail(PK_ERR_INVALID_ARG, "linear_add_rmsnorm: residual row strides must be >= hidden and multiples of 8");
  if (!aligned16(residual) || !aligned16(residual_out) || !aligned16(norm_weight))
    return fail(PK_ERR_INVALID_ARG, "linear_add_rmsnorm: residual / residual_out / norm_weight must be 16-byte aligned");
  if (!(eps >= 0.f)) return fail(PK_ERR_INVALID_ARG, "linear_add_rmsnorm: eps must be >= 0");
  if (rows == 0) return PK_OK;
  return hip_status(pk::launch_linear_add_rmsnorm(x, x_row_stride, weight, weight_row_stride, rows, hidden, k,
                                                  residual, residual_row_stride, norm_weight, eps, out,
                                                  out_row_stride, residual_out, residual_out_row_stride,
                                                  workspace, reinterpret_cast<hipStream_t>(stream)),
                    "linear_add_rmsnorm launch");
}

}  // extern "C"

// ---- allocation-free entry point --------------------------------------------------------
// pk_varlen_attention_noalloc runs the kernels of pk_varlen_attention_ex on this file-scope
// device array instead of a caller's workspace. Each GPU holds its own copy
// (PK_NOALLOC_SCRATCH_BYTES) from the first call of this entry point on it until the process
// ends: the array is the only device content of this file's code object, which loads at the
// symbol lookup below, not at the library's other launches. In host
// code `scratch` names a host-side stand-in, not device memory: its device address comes from
// hipGetSymbolAddress, once per device with that device current, and only that address is
// ever passed to a kernel.
static __device__ __align__(256) unsigned char scratch[PK_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};  // device address of `scratch` per device ordinal

// Device address of the current device's scratch, looked up on its first use (no allocation).
int device_scratch(pk_stream_t stream, void** out) {
  int dev = -1;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return hip_status(e, "varlen_attention_noalloc: hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(PK_ERR_UNSUPPORTED, "varlen_attention_noalloc: device ordinal %d above %d", dev, kMaxDevices - 1);
  if (stream != nullptr) {  // the kernels run on the stream's device: it must own this scratch
    int sdev = -1;
    if (hipError_t e = hipStreamGetDevice(reinterpret_cast<hipStream_t>(stream), &sdev); e != hipSuccess)
      return hip_status(e, "varlen_attention_noalloc: hipStreamGetDevice");
    if (sdev != dev)
      return fail(PK_ERR_INVALID_ARG, "varlen_attention_noalloc: stream belongs to device %d, current device is %d",
                  sdev, dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    if (hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); e != hipSuccess)
      return hip_status(e, "varlen_attention_noalloc: hipGetSymbolAddress(scratch)");
    if (p == nullptr || (reinterpret_cast<uintptr_t>(p) % kWorkspaceAlign) != 0)
      return fail(PK_ERR_HIP, "varlen_attention_noalloc: scratch address %p unusable", p);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PK_OK;
}

}  // namespace

extern "C" int pk_varlen_attention_noalloc(const void* q, int64_t q_row_stride, const void* k, const void* v,
                                           int64_t k_row_stride, int64_t v_row_stride, int64_t k_block_stride,
                                           int64_t v_block_stride, const int32_t* block_table,
                                           int32_t block_table_stride, int32_t block_size,
                                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                           int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                           float softmax_scale, int32_t causal, void* out, int64_t out_row_stride,
                                           int32_t cached_prefix_keys, pk_stream_t stream) {
  g_last_error.clear();
  const size_t need = pk_varlen_attention_workspace_bytes(num_seqs, num_heads, head_dim, max_seqlen_q, max_seqlen_k);
  if (need > (size_t)PK_NOALLOC_SCRATCH_BYTES)
    return fail(PK_ERR_WORKSPACE,
                "varlen_attention_noalloc: these launch bounds (num_seqs=%d, max_seqlen_q=%d, max_seqlen_k=%d) need "
                "%zu bytes of scratch; the static scratch holds %zu (use pk_varlen_attention_ex with a workspace)",
                num_seqs, max_seqlen_q, max_seqlen_k, need, (size_t)PK_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (need > 0) {
    if (int rc = device_scratch(stream, &ws)) return rc;
  }
  return attention_impl(q, q_row_stride, k, v, k_row_stride, v_row_stride, k_block_stride, v_block_stride, block_table,
                        block_table_stride, block_size, cu_seqlens_q, cu_seqlens_k, num_seqs, max_seqlen_q,
                        max_seqlen_k, num_heads, num_kv_heads, head_dim, softmax_scale, causal, out, out_row_stride,
                        ws, need > 0 ? (size_t)PK_NOALLOC_SCRATCH_BYTES : 0, cached_prefix_keys, nullptr, 0, stream);
}
