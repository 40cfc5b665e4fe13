// Host-side serving core (libpkhost.so): scheduler, block pool and per-step context
// arrays of the reference engine, restated in C++ so a step's host work is a few
// microseconds instead of Python loops over every token and block.
//
// Reference files (paths relative to the reference repository):
//   src/engine/scheduler.py:35-161      schedule / postprocess
//   src/engine/block_manager.py:183-246 allocate / deallocate / can_append / may_append
//   src/engine/sequence.py:13-69        sequence state
//   src/engine/model_runner.py:168-233  prepare_block_tables / prepare_seqs
//   src/engine/llm_engine.py:70-105     add_request capacity checks
// Prefix caching (block hashes, block_manager.py:96-181, 248-264) is not restated: a step
// truncates a prefill sequence's cached count to a block boundary exactly as the
// reference's hit-free prefix lookup does (update_prefix_cache_block sets
// num_cached_tokens = total_hits * block_size, block_manager.py:130-158, called at
// scheduler.py:68-69), and never finds a hit.
#include <cstdarg>
#include <cstdio>
#include <deque>
#include <memory>
#include <string>
#include <vector>

#include "../../include/pkhost.h"

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

enum class Status { kWaiting, kPrefill, kDecode, kFinished };

struct Seq {
  int64_t id = 0;
  std::vector<int32_t> tokens;
  int32_t num_prompt = 0;
  int32_t max_tokens = 0;
  bool ignore_eos = false;
  int32_t num_cached = 0;
  int32_t num_scheduled = 0;
  std::vector<int32_t> block_table;
  Status status = Status::kWaiting;

  int32_t len() const { return (int32_t)tokens.size(); }
  int32_t generated() const { return len() - num_prompt; }
};

template <class T>
bool erase_one(std::deque<T>& d, const T& v) {
  for (auto it = d.begin(); it != d.end(); ++it)
    if (*it == v) {
      d.erase(it);
      return true;
    }
  return false;
}

}  // namespace

struct pkh_engine {
  pkh_config cfg{};
  std::vector<std::unique_ptr<Seq>> seqs;  // index == sequence id
  std::deque<Seq*> waiting, prefill, decode;
  std::deque<int32_t> free_blocks;          // popped at the front, freed to the back
  std::vector<int32_t> ref_count;
  std::vector<Seq*> scheduled;              // the last step's batch, awaiting postprocess
  bool step_open = false;
  int64_t live = 0;                         // sequences not finished

  // registered step buffers
  int64_t* input_ids = nullptr;
  int64_t* positions = nullptr;
  int32_t* cu_q = nullptr;
  int32_t* cu_k = nullptr;
  int32_t* slots = nullptr;
  int32_t* ctx_lens = nullptr;
  int32_t* tables = nullptr;
  int64_t* seq_ids = nullptr;
  int32_t cap_tokens = 0, cap_seqs = 0, cap_width = 0;

  // ---- block pool (block_manager.py:183-246) ----
  int32_t bs() const { return cfg.block_size; }

  void allocate(Seq* s, int32_t n) {        // :183-207, pops free_block_ids[0]
    for (int32_t i = 0; i < n; ++i) {
      const int32_t b = free_blocks.front();
      free_blocks.pop_front();
      ref_count[b] = 1;
      s->block_table.push_back(b);
    }
  }
  void free_block(int32_t b) {              // :88-94
    if (--ref_count[b] == 0) free_blocks.push_back(b);
  }
  void deallocate(Seq* s) {                 // :209-214
    for (int32_t b : s->block_table) free_block(b);
    s->num_cached = 0;
    s->block_table.clear();
  }
  bool can_append(const Seq* s) const {     // :216-218
    return (int64_t)free_blocks.size() >= (s->len() % bs() == 1 ? 1 : 0);
  }
  void may_append(Seq* s) {                 // :220-246: a new block when the token opens one
    if (s->len() % bs() == 1) allocate(s, 1);
  }

  // ---- scheduler (scheduler.py:29-132) ----
  void back_to_prefill(Seq* s) {            // :29-33
    s->status = Status::kPrefill;
    deallocate(s);
    prefill.push_front(s);
  }

  int schedule(int32_t* prefill_tokens, int32_t* decode_tokens, int depth) {
    while (!waiting.empty() && (int64_t)(prefill.size() + decode.size()) < cfg.max_live_seqs) {
      Seq* s = waiting.front();             // :37-40
      waiting.pop_front();
      s->status = Status::kPrefill;
      prefill.push_back(s);
    }
    scheduled.clear();
    int32_t pt = 0, dt = 0;
    const int max_chunked = 1;              // :44
    int chunked = 0;

    // decode (:47-61): one token per sequence, preempting from the back when the pool is dry
    while (!decode.empty() && (int32_t)scheduled.size() < cfg.max_num_seqs) {
      Seq* s = decode.front();
      decode.pop_front();
      bool preempted_self = false;
      while (!can_append(s)) {
        if (!decode.empty()) {
          Seq* victim = decode.back();
          decode.pop_back();
          back_to_prefill(victim);
        } else {
          back_to_prefill(s);
          preempted_self = true;
          break;
        }
      }
      if (preempted_self) continue;
      s->num_scheduled = 1;
      may_append(s);
      dt += 1;
      scheduled.push_back(s);
    }
    for (auto it = scheduled.rbegin(); it != scheduled.rend(); ++it) decode.push_front(*it);

    // prefill (:64-110)
    while (!prefill.empty() && (int32_t)scheduled.size() < cfg.max_num_seqs) {
      Seq* s = prefill.front();
      // hit-free prefix lookup: the cached count drops to its block boundary
      // (block_manager.py:158), restored when the sequence is not scheduled this step (the
      // undo closure, block_manager.py:160-177)
      const int32_t prev_cached = s->num_cached;
      s->num_cached = s->num_cached / bs() * bs();
      const int64_t num_free = (int64_t)free_blocks.size();
      const int32_t remaining = cfg.max_num_batched_tokens - pt - dt;
      if (remaining <= 0) {
        s->num_cached = prev_cached;
        break;
      }
      const int32_t max_avail = s->len() - s->num_cached;
      if (max_avail <= 0) {                 // :77-81 (only reachable through prefix hits)
        s->num_cached -= 1;
        prefill.pop_front();
        decode.push_back(s);
        continue;
      }
      const int32_t limit = remaining < max_avail ? remaining : max_avail;
      const int64_t bt_room = (int64_t)s->block_table.size() * bs() - s->num_cached;
      const int64_t oom_limit = num_free * bs() + bt_room;
      if (oom_limit <= 0) {
        s->num_cached = prev_cached;
        break;
      }
      const int64_t fit = limit < oom_limit ? limit : oom_limit;
      int32_t n;
      if (max_avail > fit) {                // chunked prefill (:90-98)
        if (chunked < max_chunked) {
          int64_t c = fit < cfg.chunked_prefill_size ? fit : cfg.chunked_prefill_size;
          n = (int32_t)c;
          ++chunked;
        } else {
          s->num_cached = prev_cached;
          break;
        }
      } else {
        n = max_avail;
      }
      s->num_scheduled = n;
      const int32_t need = (s->num_cached + n + bs() - 1) / bs();   // :104-106
      if (need > (int32_t)s->block_table.size()) allocate(s, need - (int32_t)s->block_table.size());
      pt += n;
      prefill.pop_front();
      scheduled.push_back(s);
    }

    if (scheduled.empty() && !(waiting.empty() && prefill.empty() && decode.empty())) {
      // :118-131: release the first partially prefilled sequence and try again
      Seq* victim = nullptr;
      for (Seq* s : prefill)
        if (s->num_cached != 0) {
          victim = s;
          break;
        }
      if (victim == nullptr || depth > 1024)
        return fail(PKH_ERR_CAPACITY, "schedule: no sequence can be scheduled (pool of %d blocks exhausted)",
                    cfg.num_blocks);
      erase_one(prefill, victim);
      deallocate(victim);
      prefill.push_back(victim);
      return schedule(prefill_tokens, decode_tokens, depth + 1);
    }
    *prefill_tokens = pt;
    *decode_tokens = dt;
    return PKH_OK;
  }

  // ---- ModelRunner.prepare_seqs / prepare_block_tables (model_runner.py:168-233) ----
  int prepare(pkh_step* st) {
    const int32_t S = (int32_t)scheduled.size();
    if (S > cap_seqs) return fail(PKH_ERR_CAPACITY, "step has %d sequences > buffer %d", S, cap_seqs);
    int64_t N = 0;
    for (Seq* s : scheduled) N += s->num_scheduled;
    if (N > cap_tokens) return fail(PKH_ERR_CAPACITY, "step has %lld tokens > buffer %d", (long long)N, cap_tokens);
    int32_t n = 0, max_q = 0, max_k = 0, width = 0;
    cu_q[0] = 0;
    cu_k[0] = 0;
    for (int32_t i = 0; i < S; ++i) {
      Seq* s = scheduled[i];
      const int32_t len = s->len();
      const int32_t start = s->num_cached < len - 1 ? s->num_cached : len - 1;   // :186
      const int32_t q = s->num_scheduled;
      const int32_t end = start + q;                                            // :188-190
      for (int32_t p = start; p < end; ++p, ++n) {
        input_ids[n] = s->tokens[p];
        positions[n] = p;
        // the block walk of :200-210 is slot(p) = table[p / bs] * bs + p % bs
        slots[n] = s->block_table[p / bs()] * bs() + p % bs();
      }
      cu_q[i + 1] = cu_q[i] + q;
      cu_k[i + 1] = cu_k[i] + end;
      ctx_lens[i] = end;
      seq_ids[i] = s->id;
      if (q > max_q) max_q = q;
      if (end > max_k) max_k = end;
      if ((int32_t)s->block_table.size() > width) width = (int32_t)s->block_table.size();
    }
    st->block_table_width = 0;
    if (cu_k[S] > cu_q[S]) {                                                      // :211-212
      if (width > cap_width) return fail(PKH_ERR_CAPACITY, "block table width %d > buffer %d", width, cap_width);
      for (int32_t i = 0; i < S; ++i) {                                           // :168-172
        const auto& bt = scheduled[i]->block_table;
        int32_t* row = tables + (int64_t)i * width;
        int32_t j = 0;
        for (; j < (int32_t)bt.size(); ++j) row[j] = bt[j];
        for (; j < width; ++j) row[j] = -1;
      }
      st->block_table_width = width;
    }
    st->num_seqs = S;
    st->num_tokens = n;
    st->max_seqlen_q = max_q;
    st->max_seqlen_k = max_k;
    st->is_prefill = max_q > 1 ? 1 : 0;                                           // :229-232
    st->input_ids = input_ids;
    st->positions = positions;
    st->cu_seqlens_q = cu_q;
    st->cu_seqlens_k = cu_k;
    st->slot_mapping = slots;
    st->context_lens = ctx_lens;
    st->block_tables = tables;
    st->seq_ids = seq_ids;
    return PKH_OK;
  }
};

extern "C" {

const char* pkh_last_error(void) { return g_err.c_str(); }

pkh_engine* pkh_create(const pkh_config* cfg) {
  g_err.clear();
  if (cfg == nullptr || cfg->num_blocks <= 0 || cfg->block_size <= 0 || cfg->max_num_seqs <= 0 ||
      cfg->max_num_batched_tokens <= 0 || cfg->chunked_prefill_size <= 0 || cfg->max_live_seqs <= 0) {
    fail(PKH_ERR_INVALID_ARG, "pkh_create: every size in the config must be positive");
    return nullptr;
  }
  auto* e = new pkh_engine();
  e->cfg = *cfg;
  e->ref_count.assign(cfg->num_blocks, 0);
  for (int32_t b = 0; b < cfg->num_blocks; ++b) e->free_blocks.push_back(b);   // deque(range(n))
  return e;
}

void pkh_destroy(pkh_engine* e) { delete e; }

int pkh_set_buffers(pkh_engine* e, int64_t* input_ids, int64_t* positions, int32_t* cu_seqlens_q,
                    int32_t* cu_seqlens_k, int32_t* slot_mapping, int32_t* context_lens,
                    int32_t* block_tables, int64_t* seq_ids, int32_t max_tokens, int32_t max_seqs,
                    int32_t max_width) {
  g_err.clear();
  if (!e || !input_ids || !positions || !cu_seqlens_q || !cu_seqlens_k || !slot_mapping ||
      !context_lens || !block_tables || !seq_ids || max_tokens <= 0 || max_seqs <= 0 || max_width <= 0)
    return fail(PKH_ERR_INVALID_ARG, "pkh_set_buffers: null buffer or non-positive capacity");
  e->input_ids = input_ids;
  e->positions = positions;
  e->cu_q = cu_seqlens_q;
  e->cu_k = cu_seqlens_k;
  e->slots = slot_mapping;
  e->ctx_lens = context_lens;
  e->tables = block_tables;
  e->seq_ids = seq_ids;
  e->cap_tokens = max_tokens;
  e->cap_seqs = max_seqs;
  e->cap_width = max_width;
  return PKH_OK;
}

int64_t pkh_add_request(pkh_engine* e, const int32_t* prompt, int32_t prompt_len, int32_t max_tokens,
                        int32_t ignore_eos) {
  g_err.clear();
  if (!e || !prompt || prompt_len <= 0 || max_tokens <= 0)
    return fail(PKH_ERR_INVALID_ARG, "pkh_add_request: empty prompt or max_tokens <= 0");
  const int64_t bs = e->cfg.block_size;
  if ((prompt_len + bs - 1) / bs > e->cfg.num_blocks)                           // llm_engine.py:79-85
    return fail(PKH_ERR_CAPACITY, "prompt of %d tokens needs more than the %d blocks of the pool",
                prompt_len, e->cfg.num_blocks);
  if (((int64_t)prompt_len + max_tokens + bs - 1) / bs > e->cfg.num_blocks)     // :88-95
    return fail(PKH_ERR_CAPACITY, "prompt %d + max_tokens %d exceeds the pool of %d blocks",
                prompt_len, max_tokens, e->cfg.num_blocks);
  auto s = std::make_unique<Seq>();
  s->id = (int64_t)e->seqs.size();
  s->tokens.assign(prompt, prompt + prompt_len);
  s->num_prompt = prompt_len;
  s->max_tokens = max_tokens;
  s->ignore_eos = ignore_eos != 0;
  e->waiting.push_back(s.get());
  e->seqs.push_back(std::move(s));
  ++e->live;
  return e->seqs.back()->id;
}

int pkh_schedule(pkh_engine* e, pkh_step* step) {
  g_err.clear();
  if (!e || !step) return fail(PKH_ERR_INVALID_ARG, "pkh_schedule: null argument");
  if (!e->input_ids) return fail(PKH_ERR_STATE, "pkh_schedule: buffers not registered");
  if (e->step_open) return fail(PKH_ERR_STATE, "pkh_schedule: previous step not postprocessed");
  *step = pkh_step{};
  int32_t pt = 0, dt = 0;
  int rc = e->schedule(&pt, &dt, 0);
  if (rc != PKH_OK) return rc;
  step->num_prefill_tokens = pt;
  step->num_decode_tokens = dt;
  if (e->scheduled.empty()) return PKH_OK;
  rc = e->prepare(step);
  if (rc != PKH_OK) return rc;
  e->step_open = true;
  return PKH_OK;
}

int pkh_postprocess(pkh_engine* e, const int32_t* token_ids, int32_t n, int32_t* num_finished) {
  g_err.clear();
  if (!e || (!token_ids && n > 0)) return fail(PKH_ERR_INVALID_ARG, "pkh_postprocess: null argument");
  if (!e->step_open) return fail(PKH_ERR_STATE, "pkh_postprocess: no open step");
  if (n != (int32_t)e->scheduled.size())
    return fail(PKH_ERR_INVALID_ARG, "pkh_postprocess: %d tokens for %d sequences", n, (int)e->scheduled.size());
  int32_t finished = 0;
  for (int32_t i = 0; i < n; ++i) {                                             // scheduler.py:134-161
    Seq* s = e->scheduled[i];
    const int32_t tok = token_ids[i];
    s->num_cached += s->num_scheduled;
    s->num_scheduled = 0;
    s->tokens.push_back(tok);
    if (s->status == Status::kPrefill) {
      if (s->num_cached == s->len() - 1) {
        s->status = Status::kDecode;
        e->decode.push_back(s);
      } else if (s->num_cached < s->len() - 1) {
        e->prefill.push_front(s);
      } else {
        return fail(PKH_ERR_STATE, "postprocess: sequence %lld cached past its length", (long long)s->id);
      }
    }
    if ((!s->ignore_eos && tok == e->cfg.eos) || s->generated() == s->max_tokens) {
      s->status = Status::kFinished;
      e->deallocate(s);
      if (!erase_one(e->decode, s)) erase_one(e->prefill, s);
      --e->live;
      ++finished;
    }
  }
  e->scheduled.clear();
  e->step_open = false;
  if (num_finished) *num_finished = finished;
  return PKH_OK;
}

int pkh_is_finished(const pkh_engine* e) {
  return e && e->waiting.empty() && e->prefill.empty() && e->decode.empty() ? 1 : 0;
}

int32_t pkh_num_free_blocks(const pkh_engine* e) { return e ? (int32_t)e->free_blocks.size() : -1; }

int32_t pkh_num_generated(const pkh_engine* e, int64_t seq_id) {
  if (!e || seq_id < 0 || seq_id >= (int64_t)e->seqs.size())
    return fail(PKH_ERR_INVALID_ARG, "pkh_num_generated: unknown sequence %lld", (long long)seq_id);
  return e->seqs[seq_id]->generated();
}

int32_t pkh_generated(const pkh_engine* e, int64_t seq_id, int32_t* out, int32_t cap) {
  if (!e || seq_id < 0 || seq_id >= (int64_t)e->seqs.size() || (!out && cap > 0))
    return fail(PKH_ERR_INVALID_ARG, "pkh_generated: unknown sequence %lld", (long long)seq_id);
  const Seq& s = *e->seqs[seq_id];
  int32_t n = s.generated() < cap ? s.generated() : cap;
  for (int32_t i = 0; i < n; ++i) out[i] = s.tokens[s.num_prompt + i];
  return n;
}

}  // extern "C"
