"""CPU restatement of the reference engine's per-step host logic -- the oracle for the
C++ host core (libpkhost.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.

Restated (paths relative to the reference repository), in plain Python:

* Sequence state              -- src/engine/sequence.py:13-69
* block pool                   -- src/engine/block_manager.py:75-94 (free list: pop the
  front, free to the back), :183-246 (allocate, deallocate, can_append, may_append)
* Scheduler.schedule           -- src/engine/scheduler.py:35-132: admission up to 128 live
  sequences, decode first with preemption from the back of the decode queue, then prefill
  under the token budget with at most one chunked sequence per step, and the fallback
  that releases a partially prefilled sequence when nothing fits
* Scheduler.postprocess        -- src/engine/scheduler.py:134-161
* ModelRunner.prepare_seqs     -- src/engine/model_runner.py:168-233 (token ids, positions,
  cu_seqlens, slot walk over the block table, -1 padded block tables when any sequence
  has cached keys)

Prefix caching is restated only as far as it acts when no block hash matches, which is
every case where the cached blocks do not repeat a previous prompt's tokens: the lookup at
the start of a prefill step sets num_cached_tokens to its block boundary
(update_prefix_cache_block, block_manager.py:130-158, called at scheduler.py:68-69) and
restores it when the sequence is not scheduled (the undo closure, :160-177).

Pinning (tests/test_host_engine.py): hand-worked schedules with closed-form arrays,
invariants checked on every step of random workloads (token budget, sequence cap, block
conservation and exclusive ownership, slots equal to the block walk, contiguous
positions per sequence, at most one chunked prefill, decodes before prefills), and
planted mistakes (LIFO free list, slot offset dropped, no preemption) that must fail.
"""
from __future__ import annotations

from collections import deque

PREFILL, DECODE, FINISHED, WAITING = "prefill", "decode", "finished", "waiting"


class _Seq:
    def __init__(self, sid, prompt, max_tokens, ignore_eos):
        self.id = sid
        self.tokens = list(prompt)
        self.num_prompt = len(self.tokens)
        self.max_tokens = max_tokens
        self.ignore_eos = ignore_eos
        self.cached = 0
        self.sched = 0
        self.table: list[int] = []
        self.status = WAITING

    def __len__(self):
        return len(self.tokens)

    @property
    def generated(self):
        return len(self.tokens) - self.num_prompt


class RefEngine:
    def __init__(self, num_blocks, block_size=256, max_num_seqs=512, max_num_batched_tokens=16384,
                 chunked_prefill_size=512, max_live_seqs=128, eos=-1):
        self.bs = block_size
        self.max_seqs = max_num_seqs
        self.budget = max_num_batched_tokens
        self.chunk = chunked_prefill_size
        self.live_cap = max_live_seqs
        self.eos = eos
        self.num_blocks = num_blocks
        self.free = deque(range(num_blocks))
        self.refs = [0] * num_blocks
        self.seqs: list[_Seq] = []
        self.waiting: deque = deque()
        self.prefill: deque = deque()
        self.decode: deque = deque()
        self.batch: list[_Seq] = []

    # ---- pool ----
    def _take(self, seq, n):
        for _ in range(n):
            b = self.free.popleft()
            self.refs[b] = 1
            seq.table.append(b)

    def _release(self, seq):
        for b in seq.table:
            self.refs[b] -= 1
            if self.refs[b] == 0:
                self.free.append(b)
        seq.table = []
        seq.cached = 0

    def _opens_block(self, seq):
        return len(seq) % self.bs == 1

    def _preempt(self, seq):
        seq.status = PREFILL
        self._release(seq)
        self.prefill.appendleft(seq)

    # ---- requests ----
    def add(self, prompt, max_tokens, ignore_eos=False):
        if -(-len(prompt) // self.bs) > self.num_blocks or \
                -(-(len(prompt) + max_tokens) // self.bs) > self.num_blocks:
            raise ValueError("request does not fit the pool")
        s = _Seq(len(self.seqs), prompt, max_tokens, ignore_eos)
        self.seqs.append(s)
        self.waiting.append(s)
        return s.id

    def finished(self):
        return not (self.waiting or self.prefill or self.decode)

    # ---- one step ----
    def _pick(self):
        while self.waiting and len(self.prefill) + len(self.decode) < self.live_cap:
            s = self.waiting.popleft()
            s.status = PREFILL
            self.prefill.append(s)
        batch, used_p, used_d, chunked = [], 0, 0, 0
        while self.decode and len(batch) < self.max_seqs:
            s = self.decode.popleft()
            ok = True
            while len(self.free) < (1 if self._opens_block(s) else 0):
                if self.decode:
                    self._preempt(self.decode.pop())
                else:
                    self._preempt(s)
                    ok = False
                    break
            if not ok:
                continue
            s.sched = 1
            if self._opens_block(s):
                self._take(s, 1)
            used_d += 1
            batch.append(s)
        for s in reversed(batch):
            self.decode.appendleft(s)
        while self.prefill and len(batch) < self.max_seqs:
            s = self.prefill[0]
            before = s.cached
            s.cached = (s.cached // self.bs) * self.bs
            left = self.budget - used_p - used_d
            if left <= 0:
                s.cached = before
                break
            want = len(s) - s.cached
            if want <= 0:
                s.cached -= 1
                self.prefill.popleft()
                self.decode.append(s)
                continue
            room = len(self.free) * self.bs + len(s.table) * self.bs - s.cached
            if room <= 0:
                s.cached = before
                break
            cap = min(left, want, room)
            if want > cap:
                if chunked >= 1:
                    s.cached = before
                    break
                n = min(cap, self.chunk)
                chunked += 1
            else:
                n = want
            s.sched = n
            blocks = -(-(s.cached + n) // self.bs)
            if blocks > len(s.table):
                self._take(s, blocks - len(s.table))
            used_p += n
            batch.append(self.prefill.popleft())
        if not batch and not self.finished():
            victim = next((s for s in self.prefill if s.cached != 0), None)
            if victim is None:
                raise RuntimeError("no sequence can be scheduled")
            self.prefill.remove(victim)
            self._release(victim)
            self.prefill.append(victim)
            return self._pick()
        return batch, used_p, used_d

    def schedule(self):
        """The step's arrays as prepare_seqs builds them, or None when done."""
        if self.finished():
            return None
        batch, used_p, used_d = self._pick()
        self.batch = batch
        ids, pos, slots, cu_q, cu_k, ctx = [], [], [], [0], [0], []
        for s in batch:
            start = min(s.cached, len(s) - 1)
            end = start + s.sched
            ids += s.tokens[start:end]
            pos += list(range(start, end))
            # walk the blocks the new tokens fall into (model_runner.py:200-210)
            first, last = start // self.bs, -(-end // self.bs)
            for i in range(first, last):
                lo = s.table[i] * self.bs + (start % self.bs if i == first else 0)
                hi = s.table[i] * self.bs + (self.bs if i != last - 1 else end - i * self.bs)
                slots += list(range(lo, hi))
            cu_q.append(cu_q[-1] + s.sched)
            cu_k.append(cu_k[-1] + end)
            ctx.append(end)
        tables = None
        if cu_k[-1] > cu_q[-1]:
            w = max(len(s.table) for s in batch)
            tables = [s.table + [-1] * (w - len(s.table)) for s in batch]
        return dict(input_ids=ids, positions=pos, slot_mapping=slots, cu_seqlens_q=cu_q,
                    cu_seqlens_k=cu_k, context_lens=ctx, block_tables=tables,
                    max_seqlen_q=max(s.sched for s in batch), max_seqlen_k=max(ctx),
                    seq_ids=[s.id for s in batch], num_prefill_tokens=used_p,
                    num_decode_tokens=used_d)

    def postprocess(self, tokens):
        done = 0
        for s, t in zip(self.batch, tokens):
            s.cached += s.sched
            s.sched = 0
            s.tokens.append(t)
            if s.status == PREFILL:
                if s.cached == len(s) - 1:
                    s.status = DECODE
                    self.decode.append(s)
                elif s.cached < len(s) - 1:
                    self.prefill.appendleft(s)
                else:
                    raise RuntimeError("cached past the sequence length")
            if (not s.ignore_eos and t == self.eos) or s.generated == s.max_tokens:
                s.status = FINISHED
                self._release(s)
                if s in self.decode:
                    self.decode.remove(s)
                elif s in self.prefill:
                    self.prefill.remove(s)
                done += 1
        self.batch = []
        return done

    def generated(self, sid):
        s = self.seqs[sid]
        return s.tokens[s.num_prompt:]
