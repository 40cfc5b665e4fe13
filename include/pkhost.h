/*
 * pkhost.h -- C-ABI of the host-side serving core (libpkhost.so, plain C++, no GPU code).
 *
 * It replaces the per-step Python work of the reference engine that surrounds the
 * paged-KV attention path:
 *   - Scheduler.schedule / postprocess        (src/engine/scheduler.py:35-161)
 *   - BlockManager allocate / deallocate /
 *     can_append / may_append                  (src/engine/block_manager.py:183-246)
 *   - Sequence bookkeeping                     (src/engine/sequence.py:13-69)
 *   - ModelRunner.prepare_seqs and
 *     prepare_block_tables                     (src/engine/model_runner.py:168-233)
 * The scheduling policy is the reference's (decode first, at most 128 live sequences,
 * chunked prefill of at most one sequence per step, recompute on preemption); prefix
 * caching (block hashing and reuse) is not implemented, so scheduling matches the
 * reference whenever its prefix cache would not hit.
 *
 * Conventions: a pkh_engine is single-threaded; every call returns 0 or a negative PKH_ERR_*
 * code with pkh_last_error() describing it. The step arrays are written into caller-owned
 * buffers (typically pinned host memory) registered with pkh_set_buffers.
 */
#ifndef PKHOST_H
#define PKHOST_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKH_OK 0
#define PKH_ERR_INVALID_ARG (-1)
#define PKH_ERR_CAPACITY (-2)   /* a request or step does not fit the registered buffers / pool */
#define PKH_ERR_STATE (-3)      /* call out of order (e.g. postprocess without a schedule) */

typedef struct pkh_engine pkh_engine;

typedef struct pkh_config {
  int32_t num_blocks;              /* KV cache blocks in the pool                     */
  int32_t block_size;              /* tokens per block (runner_config.py:20)          */
  int32_t max_num_seqs;            /* sequences per step (runner_config.py:12)        */
  int32_t max_num_batched_tokens;  /* tokens per step (runner_config.py:11)           */
  int32_t chunked_prefill_size;    /* chunk of a prefill that does not fit (:14)      */
  int32_t max_live_seqs;           /* waiting -> prefill admission cap (scheduler.py:37: 128) */
  int32_t eos;                     /* eos token id (scheduler_cfg.py:10)              */
} pkh_config;

/* The arrays of one step, as ModelRunner.prepare_seqs builds them (model_runner.py:174-233).
 * Pointers are the registered buffers; counts say how much of each is valid. */
typedef struct pkh_step {
  int32_t num_seqs;          /* S: scheduled sequences, decodes first (scheduler.py:47-110) */
  int32_t num_tokens;        /* N = cu_seqlens_q[S]                                        */
  int32_t num_prefill_tokens, num_decode_tokens;
  int32_t max_seqlen_q, max_seqlen_k;
  int32_t is_prefill;        /* max_seqlen_q > 1 (model_runner.py:229-232)                 */
  int32_t block_table_width; /* W, 0 when no block table is needed (model_runner.py:211)   */
  int64_t* input_ids;        /* (N,)  */
  int64_t* positions;        /* (N,)  */
  int32_t* cu_seqlens_q;     /* (S+1,) */
  int32_t* cu_seqlens_k;     /* (S+1,) */
  int32_t* slot_mapping;     /* (N,)  */
  int32_t* context_lens;     /* (S,)  */
  int32_t* block_tables;     /* (S, W) row-major, -1 padded */
  int64_t* seq_ids;          /* (S,)  ids of the scheduled sequences, in batch order */
} pkh_step;

const char* pkh_last_error(void);

pkh_engine* pkh_create(const pkh_config* cfg);
void pkh_destroy(pkh_engine* e);

/* Register the step buffers: max_tokens rows for the per-token arrays, max_seqs rows for
 * the per-sequence arrays, max_seqs * max_width entries for the block tables. */
int pkh_set_buffers(pkh_engine* e, int64_t* input_ids, int64_t* positions, int32_t* cu_seqlens_q,
                    int32_t* cu_seqlens_k, int32_t* slot_mapping, int32_t* context_lens,
                    int32_t* block_tables, int64_t* seq_ids, int32_t max_tokens,
                    int32_t max_seqs, int32_t max_width);

/* LLMEngine.add_request (llm_engine.py:70-105): queue a prompt; returns the sequence id
 * (>= 0) or a negative error (prompt or prompt + max_tokens larger than the pool). */
int64_t pkh_add_request(pkh_engine* e, const int32_t* prompt, int32_t prompt_len,
                        int32_t max_tokens, int32_t ignore_eos);

/* Scheduler.schedule + ModelRunner.prepare_seqs: pick this step's sequences and write
 * their arrays. Returns PKH_OK with step->num_seqs == 0 when nothing is left. */
int pkh_schedule(pkh_engine* e, pkh_step* step);

/* Scheduler.postprocess (scheduler.py:134-161): one sampled token per scheduled sequence,
 * in the step's batch order. *num_finished receives how many sequences finished. */
int pkh_postprocess(pkh_engine* e, const int32_t* token_ids, int32_t n, int32_t* num_finished);

int pkh_is_finished(const pkh_engine* e);     /* no waiting, prefill or decode sequence */
int32_t pkh_num_free_blocks(const pkh_engine* e);

/* Tokens generated so far by a sequence (sequence.py:46-48); returns the count written
 * (at most cap) or a negative error. */
int32_t pkh_generated(const pkh_engine* e, int64_t seq_id, int32_t* out, int32_t cap);
int32_t pkh_num_generated(const pkh_engine* e, int64_t seq_id);

#ifdef __cplusplus
}
#endif

#endif /* PKHOST_H */
