/*
 * pagedkv.h -- C-ABI of the MI355X (gfx950) paged-KV attention library
 * (libpagedkv.so).
 *
 * The library implements the device side of the reference's
 * Attention.forward (src/layers/attention.py:79-105):
 *
 *   1. the store_kvcache scatter of new K/V token rows into cache slots
 *      (src/layers/attention.py:10-34, host wrapper :36-61);
 *   2. varlen causal attention over either fresh K/V rows ("flat" mode,
 *      block_table == NULL) or a paged KV cache read through per-sequence
 *      block tables ("paged" mode) -- the flash_attn_varlen_func call at
 *      src/layers/attention.py:95-104. Sequences with one query row go to
 *      the split-K decode kernel, sequences with more go to the bf16-MFMA
 *      prefill kernel; both run in the same call.
 *
 * Conventions
 *   - Every pointer is a borrowed device pointer; the library allocates
 *     nothing. Scratch memory for split-K partial results is passed in as
 *     `workspace` (size from pk_varlen_attention_workspace_bytes; no
 *     initial contents needed). Two calls that can run at the same time
 *     (e.g. on different streams) must not share a workspace.
 *   - Strides are in ELEMENTS, not bytes.
 *   - Element type: 16-bit. The store copies bits (bf16 or fp16); the
 *     attention entry points read and write bf16.
 *   - Every entry point takes the hipStream_t to enqueue on (0 = the null
 *     stream), never synchronises, never reads device memory from the host,
 *     and is safe to record into a hipGraph: all per-sequence lengths are
 *     read on the device from cu_seqlens_q / cu_seqlens_k.
 *   - Return value: PK_OK (0) or a negative PK_ERR_* code; the message for
 *     the last failure on the calling thread is pk_last_error(). Nothing
 *     throws across the ABI.
 */
#ifndef PAGEDKV_H
#define PAGEDKV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PK_OK 0
#define PK_ERR_INVALID_ARG (-1)   /* shape / stride / alignment / null-pointer error */
#define PK_ERR_UNSUPPORTED (-2)   /* valid but not built (e.g. head_dim != 128)      */
#define PK_ERR_WORKSPACE (-3)     /* workspace too small or misaligned                 */
#define PK_ERR_HIP (-4)           /* a HIP runtime call or kernel launch failed        */

/* hipStream_t without pulling in the HIP headers. */
typedef struct ihipStream_t* pk_stream_t;

/* Version of this ABI (bumped on any signature change). */
int pk_abi_version(void);

/* Message describing the last error returned on the calling thread
 * ("" if none). The pointer stays valid until the next call on this thread. */
const char* pk_last_error(void);

/*
 * pk_store_kvcache -- replaces store_kvcache() / store_kvcache_kernel
 * (src/layers/attention.py:36-61 and :10-34).
 *
 * For every token i < num_tokens with s = slot_mapping[i] != -1:
 *     k_cache[s * row_elems + e] = key[i * key_row_stride + e]
 *     v_cache[s * row_elems + e] = value[i * value_row_stride + e]
 * for e < row_elems (row_elems = num_kv_heads * head_dim, the reference's
 * `D`). Tokens with slot -1 (graph padding, model_runner.py:250-251) are
 * skipped; their cache bits are untouched.
 *
 * num_slots > 0 enables a device-side bound check: a slot outside
 * [-1, num_slots) is not written (the reference performs no check,
 * attention.py:59). Pass 0 to mirror the reference exactly.
 *
 * Requirements: row_elems % 8 == 0; key, value, k_cache, v_cache 16-byte
 * aligned; key_row_stride and value_row_stride multiples of 8 elements.
 * The cache rows are contiguous (the reference asserts
 * k_cache.stride(1) == D, attention.py:53).
 */
int pk_store_kvcache(const void* key, int64_t key_row_stride,
                     const void* value, int64_t value_row_stride,
                     void* k_cache, void* v_cache,
                     const int32_t* slot_mapping, int32_t num_tokens,
                     int32_t row_elems, int64_t num_slots,
                     pk_stream_t stream);

/*
 * pk_varlen_attention -- replaces flash_attn_varlen_func(q, k, v,
 * cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, softmax_scale,
 * causal, block_table) as called at src/layers/attention.py:95-104.
 *
 *   q    (Nq, num_heads, head_dim) bf16, token row stride q_row_stride,
 *        head stride head_dim (heads contiguous within a row).
 *   k, v flat mode  (block_table == NULL): (Nk, num_kv_heads, head_dim),
 *          key row of sequence b, position t at k + (cu_seqlens_k[b] + t) *
 *          k_row_stride; k_block_stride / v_block_stride are ignored.
 *        paged mode (block_table != NULL): caches (num_blocks, block_size,
 *          num_kv_heads, head_dim); position t of sequence b lives at
 *          k + block_table[b * block_table_stride + t / block_size] *
 *          k_block_stride + (t % block_size) * k_row_stride.
 *   cu_seqlens_q, cu_seqlens_k  (num_seqs + 1,) int32 prefix sums.
 *        Sequence b has Lq = cu_seqlens_q[b+1] - cu_seqlens_q[b] query rows
 *        and Lk = cu_seqlens_k[b+1] - cu_seqlens_k[b] keys; sequences with
 *        Lq <= 0 or Lk <= 0 (graph padding, model_runner.py:252-255) are
 *        skipped and their output rows are not written.
 *   max_seqlen_q, max_seqlen_k  host-side upper bounds (launch sizes only).
 *   causal != 0: bottom-right aligned mask -- query row i of a sequence
 *        sees keys t <= i + Lk - Lq. A row that sees no key is written as 0.
 *   GQA: query head h reads kv head h / (num_heads / num_kv_heads).
 *   out  (Nq, num_heads, head_dim) bf16, token row stride out_row_stride.
 *
 * Built for head_dim == 128, num_heads % num_kv_heads == 0 with the group
 * size in {1, 2, 4, 8}, num_kv_heads <= 255, max_seqlen_q and max_seqlen_k up
 * to 65535 * 64; block_size a multiple of 64 in paged mode. Softmax and
 * accumulation are fp32.
 */
int pk_varlen_attention(const void* q, int64_t q_row_stride,
                        const void* k, const void* v,
                        int64_t k_row_stride, int64_t v_row_stride,
                        int64_t k_block_stride, int64_t v_block_stride,
                        const int32_t* block_table, int32_t block_table_stride,
                        int32_t block_size,
                        const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                        int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        float softmax_scale, int32_t causal,
                        void* out, int64_t out_row_stride,
                        void* workspace, size_t workspace_bytes,
                        pk_stream_t stream);

/*
 * pk_varlen_attention_ex -- pk_varlen_attention with a cache hint for the decode reads
 * (no counterpart in the reference: flash_attn_varlen_func has no such argument).
 * Decode K/V reads at key positions >= cached_prefix_keys use non-temporal (streaming)
 * loads, earlier ones normal loads, decided per split of split-K work by its first key;
 * cached_prefix_keys < 0 reads every key with normal loads. Prefix caching only ever
 * shares a sequence's leading blocks, so a caller sets this to the longest prefix its
 * block manager may share (0 when blocks are never shared between sequences).
 * pk_varlen_attention uses PK_CACHED_PREFIX_KEYS_DEFAULT. The hint never changes results.
 */
#define PK_CACHED_PREFIX_KEYS_DEFAULT 2048

int pk_varlen_attention_ex(const void* q, int64_t q_row_stride,
                           const void* k, const void* v,
                           int64_t k_row_stride, int64_t v_row_stride,
                           int64_t k_block_stride, int64_t v_block_stride,
                           const int32_t* block_table, int32_t block_table_stride,
                           int32_t block_size,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                           int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                           float softmax_scale, int32_t causal,
                           void* out, int64_t out_row_stride,
                           void* workspace, size_t workspace_bytes,
                           int32_t cached_prefix_keys, pk_stream_t stream);

/*
 * pk_varlen_attention_shared_prefix -- pk_varlen_attention_ex that computes the leading keys
 * sequences share once per shared block instead of once per sequence (no counterpart in the
 * reference, whose flash-attn call reads a shared prefix block again for every sequence that
 * holds it, attention.py:95-104; prefix blocks are shared through the block manager's
 * reference counts, block_manager.py:96-181).
 *   shared_prefix_keys: the caller's bound on the shared prefix, e.g. the longest leading
 *     run of blocks whose reference count exceeds 1 (pagedkv.shared_prefix_keys). For every
 *     decode sequence (one query row) its keys below P = shared_prefix_keys, rounded down to
 *     whole chunks of lcm(block_size, the decode split) keys, are processed in chunks: the
 *     sequences whose block tables name the same blocks for a chunk (and hold the same number
 *     of keys in it) put their query rows into one set of bf16 MFMA tiles, so each shared
 *     block is read once per kv head and window of 256 / (num_heads / num_kv_heads)
 *     consecutive sequences; the keys past P go through the split-K decode kernel, and the
 *     combine merges both. Sequences that share nothing are still correct (a group of one).
 *     0 is pk_varlen_attention_ex. Paged mode only; prefill rows (Lq > 1) are unaffected.
 *   Results: within the attention tolerance of pk_varlen_attention_ex (the prefix is summed
 *   in another order), bit-identical from run to run, and bit-identical whether the prefix
 *   blocks are shared or duplicated (a row's arithmetic does not depend on its tile mates).
 *   Workspace: pk_varlen_attention_workspace_bytes, as for pk_varlen_attention_ex.
 */
int pk_varlen_attention_shared_prefix(const void* q, int64_t q_row_stride,
                                      const void* k, const void* v,
                                      int64_t k_row_stride, int64_t v_row_stride,
                                      int64_t k_block_stride, int64_t v_block_stride,
                                      const int32_t* block_table, int32_t block_table_stride,
                                      int32_t block_size,
                                      const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                      int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                      float softmax_scale, int32_t causal,
                                      void* out, int64_t out_row_stride,
                                      void* workspace, size_t workspace_bytes,
                                      int32_t cached_prefix_keys, int32_t shared_prefix_keys,
                                      pk_stream_t stream);

/*
 * pk_varlen_attention_noalloc -- pk_varlen_attention_ex for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. Same arguments, semantics and kernels as
 * pk_varlen_attention_ex -- outputs are bit-identical -- minus the workspace: the split-K
 * partials and the prefill work plan live in a static device array of
 * PK_NOALLOC_SCRATCH_BYTES (128 MiB) that each GPU holds from the first call on it until the
 * process ends. The array is the only content of its own code object, which the HIP runtime
 * (deferred code-object loading, its default) loads at the first address lookup: a process
 * that never calls this entry point does not hold it (measured on MI355X: free device memory
 * drops by 130 MiB at the first call, by none at the library's other launches). The call
 * allocates nothing (no hipMalloc, no allocating library routine).
 *   - Launch bounds whose pk_varlen_attention_workspace_bytes exceeds the scratch return
 *     PK_ERR_WORKSPACE before any launch (every batch of the five benchmark shapes fits:
 *     256 decode sequences of up to 8192 keys need 32.5 MiB, a mixed chunked-prefill batch
 *     about 115 MiB).
 *   - The stream must belong to the current device (PK_ERR_INVALID_ARG otherwise). The first
 *     call on a device looks the array's address up (hipGetSymbolAddress): make it outside
 *     graph capture.
 *   - Every call on one GPU shares that GPU's array: calls that can overlap on one GPU
 *     (two streams, two threads, concurrently replayed graphs) race and give wrong results.
 *     Each call writes every scratch byte it reads first; no contents carry over.
 */
#define PK_NOALLOC_SCRATCH_BYTES ((size_t)128 << 20)

int pk_varlen_attention_noalloc(const void* q, int64_t q_row_stride,
                                const void* k, const void* v,
                                int64_t k_row_stride, int64_t v_row_stride,
                                int64_t k_block_stride, int64_t v_block_stride,
                                const int32_t* block_table, int32_t block_table_stride,
                                int32_t block_size,
                                const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                int32_t num_seqs, int32_t max_seqlen_q, int32_t max_seqlen_k,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                float softmax_scale, int32_t causal,
                                void* out, int64_t out_row_stride,
                                int32_t cached_prefix_keys, pk_stream_t stream);

/*
 * pk_qkv_decode_attention -- one decode step of an attention layer from the fused qkv
 * projection, in one split-K launch (no counterpart in the reference: it is
 * pk_qk_norm_rope_store(qkv, ..., k_cache, v_cache, slot_mapping) followed by
 * pk_varlen_attention_ex(q, ..., k_cache, v_cache, block_table, ...) for a batch in which
 * every sequence has one query row, i.e. src/models/qwen3.py:80-89 plus
 * src/layers/attention.py:87-104 on a decode step). Results are bit-identical to those
 * two calls. qkv is (num_seqs, (num_heads + 2 num_kv_heads) head_dim) with row stride
 * qkv_row_stride; positions (num_seqs,) int64; cos_sin, norm weights, eps and num_slots as
 * for pk_qk_norm_rope_store; caches, block table, lengths and workspace as for
 * pk_varlen_attention_ex with max_seqlen_q = 1 (workspace: pk_varlen_attention_workspace_bytes
 * with max_seqlen_q = 1). cu_seqlens_q must give every sequence one row (graph padding
 * rows: 0 or fewer keys and slot -1). slot_mapping[i] must be the cache slot of the last
 * key of sequence i (the token's own position), as the runner builds it: the key is
 * written there and read back through the block table by the same wavefront.
 * Preconditions of the one launch (checked where the host can: PK_ERR_INVALID_ARG):
 *   - the caches have contiguous rows and blocks (k_row_stride == num_kv_heads * head_dim,
 *     k_block_stride == block_size * k_row_stride, the same for v), so the row lands where
 *     pk_qk_norm_rope_store writes it (slot * row);
 *   - no other sequence of the batch reads the cache block holding slot_mapping[i]: the
 *     row is written while other work-groups of the launch read the cache, unordered with
 *     their reads. With prefix caching a fully cached prompt recomputes its last token into
 *     a shared block (src/engine/scheduler.py:77-80, model_runner.py:185-186); such a batch
 *     must use the two calls, whose store is ordered before every read.
 */
int pk_qkv_decode_attention(const void* qkv, int64_t qkv_row_stride,
                            const int64_t* positions, const float* cos_sin, int64_t max_position,
                            const void* q_norm_weight, const void* k_norm_weight, float eps,
                            void* k_cache, void* v_cache,
                            int64_t k_row_stride, int64_t v_row_stride,
                            int64_t k_block_stride, int64_t v_block_stride,
                            const int32_t* slot_mapping, int64_t num_slots,
                            const int32_t* block_table, int32_t block_table_stride,
                            int32_t block_size,
                            const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                            int32_t num_seqs, int32_t max_seqlen_k,
                            int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                            float softmax_scale,
                            void* out, int64_t out_row_stride,
                            void* workspace, size_t workspace_bytes,
                            int32_t cached_prefix_keys, pk_stream_t stream);

/*
 * pk_store_decode_attention -- Attention.forward (attention.py:79-105) on a decode step in
 * one split-K launch: store_kvcache of the tokens' key / value rows (attention.py:87-88,
 * the contract of pk_store_kvcache) followed by paged decode attention
 * (pk_varlen_attention_ex with max_seqlen_q = 1). No counterpart in the reference as one
 * call; results, output and caches, are bit-identical to the two calls. Every sequence has
 * one query row (row i of q, key and value is sequence i's token; graph padding rows: 0 or
 * fewer keys and slot -1) and slot_mapping[i] is the cache slot of sequence i's last key.
 * Same two preconditions as pk_qkv_decode_attention: contiguous cache rows and blocks
 * (the row lands where pk_store_kvcache writes it, slot * row), and no other sequence of
 * the batch reads the block holding slot_mapping[i]. pagedkv.Attention takes this path
 * only when its Context states that no block is shared (cached_prefix_keys == 0).
 */
int pk_store_decode_attention(const void* q, int64_t q_row_stride,
                              const void* key, int64_t key_row_stride,
                              const void* value, int64_t value_row_stride,
                              void* k_cache, void* v_cache,
                              int64_t k_row_stride, int64_t v_row_stride,
                              int64_t k_block_stride, int64_t v_block_stride,
                              const int32_t* slot_mapping, int64_t num_slots,
                              const int32_t* block_table, int32_t block_table_stride,
                              int32_t block_size,
                              const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                              int32_t num_seqs, int32_t max_seqlen_k,
                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              float softmax_scale,
                              void* out, int64_t out_row_stride,
                              void* workspace, size_t workspace_bytes,
                              int32_t cached_prefix_keys, pk_stream_t stream);

/*
 * Bytes of workspace pk_varlen_attention needs for these launch bounds: the
 * split-K partial outputs of the decode kernel (none when every sequence fits
 * one split) and, when max_seqlen_q > 1, the prefill work plan (work list,
 * merge list and the partial outputs of query tiles split over key ranges,
 * about 100 MB at most). 0 means workspace may be NULL. The contents need no
 * initialisation: each call writes what it reads. No counterpart in the
 * reference: flash-attn allocates its split-K buffers internally, which a
 * graph-capturable, allocation-free ABI cannot do.
 */
size_t pk_varlen_attention_workspace_bytes(int32_t num_seqs, int32_t num_heads,
                                           int32_t head_dim, int32_t max_seqlen_q,
                                           int32_t max_seqlen_k);

/*
 * pk_gather_kv -- materialise the keys (or values) of every sequence from a
 * paged cache into a flat (sum Lk, row_elems) buffer:
 *     dst[(cu_seqlens_k[b] + t) * row_elems + e] =
 *         cache[block_table[b * block_table_stride + t / block_size] *
 *               block_stride + (t % block_size) * row_elems + e]
 * This is the block-table addressing flash-attn performs internally for
 * paged K/V (attention.py:93-104 with model_runner.py:168-172); it has no
 * separate reference function and exists so the addressing can be checked
 * bit-exactly and so a paged prefix can be copied out. Same alignment
 * rules as pk_store_kvcache.
 */
int pk_gather_kv(const void* cache, int64_t block_stride, int32_t block_size,
                 const int32_t* block_table, int32_t block_table_stride,
                 const int32_t* cu_seqlens_k, int32_t num_seqs, int32_t max_seqlen_k,
                 int32_t row_elems, void* dst, pk_stream_t stream);

/*
 * pk_qk_norm_rope_store -- the producer of the attention inputs, fused: replaces
 * q_norm / k_norm (RMSNorm over head_dim, src/layers/layernorm.py:11-16),
 * rotary_emb (rotate-half RoPE, src/layers/pos_embedding.py:30-48) and the
 * store_kvcache call (src/layers/attention.py:87-88) as run by
 * Qwen3Attention.forward (src/models/qwen3.py:80-89).
 *
 *   qkv  (num_tokens, (num_heads + 2 num_kv_heads) * head_dim) bf16, the fused
 *        projection output [q heads | k heads | v heads], row stride
 *        qkv_row_stride.
 *   positions (num_tokens,) int64; cos_sin (max_position, head_dim) fp32, row p =
 *        [cos(p f_0..f_63) | sin(p f_0..f_63)] (pos_embedding.py:6-18). Positions
 *        outside [0, max_position) are clamped (the reference would index out of
 *        range).
 *   q_norm_weight, k_norm_weight (head_dim,) bf16, or NULL to skip the norm (the
 *        qkv_bias variant, qwen3.py:85).
 * For every token i and head h:
 *   x  = bf16(w * (x * rsqrt(mean(x^2) + eps)))          (fp32 inside)
 *   q_out[i, h]  = bf16(rope(x, positions[i]))            (fp32 inside)
 * and the same for k heads, written to k_out (if non-NULL, for attention over
 * fresh keys) and, when the caches are non-NULL and slot_mapping[i] != -1, to
 * k_cache[slot]; the raw v row goes to v_cache[slot]. num_slots > 0 drops slots
 * outside [0, num_slots) (no reference counterpart, as in pk_store_kvcache).
 * Built for head_dim 128; all tensors 16-byte aligned, strides multiples of 8.
 */
int pk_qk_norm_rope_store(const void* qkv, int64_t qkv_row_stride,
                          const int64_t* positions, const float* cos_sin, int64_t max_position,
                          const void* q_norm_weight, const void* k_norm_weight, float eps,
                          int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, void* q_out, int64_t q_out_row_stride,
                          void* k_out, int64_t k_out_row_stride,
                          void* k_cache, void* v_cache, const int32_t* slot_mapping,
                          int64_t num_slots, pk_stream_t stream);

/*
 * Kernels of the serving loop around the attention path (used by the end-to-end engine).
 *
 * pk_add_rmsnorm -- RMSNorm.forward (src/layers/layernorm.py:30-39): with residual == NULL,
 *   out = bf16(w * (x * rsqrt(mean(x^2) + eps))) (normal_forward, :11-16); otherwise
 *   s = x + residual in fp32, out = bf16(w * (s * rsqrt(mean(s^2) + eps))) and
 *   residual_out = bf16(s) (residual_forward, :18-28). bf16 rows of `hidden` <= 4096
 *   elements (multiple of 8); out / residual_out may alias x / residual.
 */
int pk_add_rmsnorm(const void* x, int64_t x_row_stride, const void* residual,
                   int64_t residual_row_stride, const void* weight, float eps, int32_t rows,
                   int32_t hidden, void* out, int64_t out_row_stride, void* residual_out,
                   int64_t residual_out_row_stride, pk_stream_t stream);

/*
 * pk_silu_and_mul -- SiluAndMul.forward (src/layers/activation.py:6-10):
 *   out[r, c] = bf16(silu(x[r, c]) * x[r, inter + c]), computed in fp32 (the compiled
 *   reference fuses both and rounds once). inter a multiple of 8.
 */
int pk_silu_and_mul(const void* x, int64_t x_row_stride, int32_t rows, int32_t inter, void* out,
                    int64_t out_row_stride, pk_stream_t stream);

/*
 * pk_lm_head_greedy -- ParallelLMHead.forward (src/layers/llm_head.py:60-64) followed by a
 * greedy choice (the reference samples, sampler.py:14-16; the serving benchmark runs greedy):
 *   row m = hidden_states[cu_seqlens_q[m+1] - 1] when cu_seqlens_q != NULL (prefill: the
 *   last token of each sequence, llm_head.py:61-63), else hidden_states[m];
 *   token_ids[m] = argmax_v bf16(row . weight[v]) with the lowest v among equal maxima
 *   (argmax over the reference's bf16 logits). The logits are never written.
 *   keys: scratch of `rows` 64-bit words (no initial contents needed). hidden a multiple
 *   of 128; weight (vocab, hidden) bf16 rows.
 */
int pk_lm_head_greedy(const void* hidden_states, int64_t row_stride, const int32_t* cu_seqlens_q,
                      const void* weight, int64_t weight_row_stride, int32_t rows, int32_t vocab,
                      int32_t hidden, uint64_t* keys, int32_t* token_ids, pk_stream_t stream);

/*
 * Decode-step linear layers: y = x W^T for at most 128 token rows (the serving loop's decode
 * batches), bf16 operands with fp32 accumulation, the output rounded to bf16 before the
 * operation that follows it (as F.linear's bf16 result is in the reference), and that
 * operation fused. They replace the F.linear calls of Qwen3Attention / Qwen3MLP
 * (src/models/qwen3.py:80, :90, :120, :122 through ColumnParallelLinear.forward and
 * RowParallelLinear.forward, src/layers/linear.py:74-75, :169-170) together with the op
 * after them (SiluAndMul at qwen3.py:121; the decoder layer's RMSNorms at qwen3.py:165, :167).
 * x (rows, k), weight (rows_w, k) row-major, n_out a multiple of 32, k a multiple of 256;
 * every pointer 16-byte aligned, row strides multiples of 8 elements; out must not overlap x.
 * rows > 128 returns PK_ERR_UNSUPPORTED (larger batches belong to a library GEMM).
 * workspace: pk_linear_workspace_bytes(rows, n_out, k, epilogue) bytes (may be 0), 16-byte
 * aligned; its contents are not needed before or after a call. Calls that share a
 * workspace must not overlap.
 *
 * pk_linear -- epilogue PK_LINEAR_STORE: out = bf16(x W^T), W = weight (n_out rows).
 *   epilogue PK_LINEAR_SILU_MUL: weight holds 2 n_out rows (gate rows, then up rows, the
 *   MergedColumnParallelLinear layout) and out[r, c] = bf16(silu(g) * u) with
 *   g = bf16(x . gate[c]), u = bf16(x . up[c]) (SiluAndMul, src/layers/activation.py:6-10,
 *   computed in fp32 and rounded once).
 * pk_linear_add_rmsnorm -- h = bf16(x W^T) (hidden = n_out columns, at most 4096), then
 *   RMSNorm.residual_forward (src/layers/layernorm.py:18-28): s = h + residual in fp32,
 *   out = bf16(norm_weight * (s * rsqrt(mean(s^2) + eps))), residual_out = bf16(s).
 *   out and residual_out may alias residual.
 */
#define PK_LINEAR_STORE 0
#define PK_LINEAR_SILU_MUL 1
#define PK_LINEAR_ADD_RMSNORM 2

size_t pk_linear_workspace_bytes(int32_t rows, int32_t n_out, int32_t k, int32_t epilogue);
int pk_linear(const void* x, int64_t x_row_stride, const void* weight, int64_t weight_row_stride,
              int32_t rows, int32_t n_out, int32_t k, int32_t epilogue, void* out, int64_t out_row_stride,
              void* workspace, size_t workspace_bytes, pk_stream_t stream);
int pk_linear_add_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, int64_t weight_row_stride,
                          int32_t rows, int32_t hidden, int32_t k, const void* residual,
                          int64_t residual_row_stride, const void* norm_weight, float eps, void* out,
                          int64_t out_row_stride, void* residual_out, int64_t residual_out_row_stride,
                          void* workspace, size_t workspace_bytes, pk_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* PAGEDKV_H */
