"""The host core (libpkhost.so) against the oracle restatement of the reference's
scheduler, block pool and prepare_seqs (oracle/engine.py), on the CPU.

The oracle is pinned first: hand-worked schedules whose arrays follow in closed form,
invariants on every step of random workloads, and planted mistakes that must fail.
Then every step of random workloads (chunking, preemption, eos, tight pools) must give
identical arrays from the C++ core and the oracle.
"""
import random

import pytest
import torch

from oracle import engine as E
from pagedkv._host import HostError, HostScheduler


def cpp(**kw):
    return HostScheduler(pin_memory=False, **kw)


def step_dict(st):
    if st is None:
        return None
    return dict(input_ids=st.input_ids.tolist(), positions=st.positions.tolist(),
                slot_mapping=st.slot_mapping.tolist(), cu_seqlens_q=st.cu_seqlens_q.tolist(),
                cu_seqlens_k=st.cu_seqlens_k.tolist(), context_lens=st.context_lens.tolist(),
                block_tables=None if st.block_tables is None else st.block_tables.tolist(),
                max_seqlen_q=st.max_seqlen_q, max_seqlen_k=st.max_seqlen_k,
                seq_ids=st.seq_ids.tolist(), num_prefill_tokens=st.num_prefill_tokens,
                num_decode_tokens=st.num_decode_tokens)


# ------------------------------------------------------------- closed forms -----------

def test_single_sequence_prefill_then_decode():
    eng = E.RefEngine(num_blocks=4, block_size=16)
    sid = eng.add(list(range(100, 110)), max_tokens=3, ignore_eos=True)
    s = eng.schedule()
    assert s["input_ids"] == list(range(100, 110)) and s["positions"] == list(range(10))
    assert s["slot_mapping"] == list(range(10))          # block 0 is popped first
    assert s["cu_seqlens_q"] == [0, 10] and s["cu_seqlens_k"] == [0, 10]
    assert s["block_tables"] is None and s["max_seqlen_q"] == 10
    eng.postprocess([7])
    s = eng.schedule()
    assert s["input_ids"] == [7] and s["positions"] == [10] and s["slot_mapping"] == [10]
    assert s["cu_seqlens_k"] == [0, 11] and s["block_tables"] == [[0]]
    eng.postprocess([8])
    s = eng.schedule()
    assert s["positions"] == [11]
    eng.postprocess([9])
    assert eng.finished() and eng.generated(sid) == [7, 8, 9]
    assert sorted(eng.free) == [0, 1, 2, 3]


def test_decode_that_opens_a_block_takes_the_next_free_block():
    eng = E.RefEngine(num_blocks=4, block_size=16)
    eng.add(list(range(16)), max_tokens=2, ignore_eos=True)
    s = eng.schedule()
    assert s["slot_mapping"] == list(range(16))
    eng.postprocess([5])
    s = eng.schedule()                                    # position 16 opens block 1
    assert s["positions"] == [16] and s["slot_mapping"] == [16] and s["block_tables"] == [[0, 1]]


def test_budget_and_single_chunk():
    eng = E.RefEngine(num_blocks=16, block_size=16, max_num_batched_tokens=32, chunked_prefill_size=8)
    eng.add(list(range(20)), max_tokens=5, ignore_eos=True)
    eng.add(list(range(1000, 1030)), max_tokens=5, ignore_eos=True)
    eng.add(list(range(2000, 2004)), max_tokens=5, ignore_eos=True)
    s = eng.schedule()
    # seq0 whole (20 of 32), seq1 chunked to min(12, 8) = 8, seq2's 4 tokens fill the budget
    assert s["seq_ids"] == [0, 1, 2] and s["cu_seqlens_q"] == [0, 20, 28, 32]
    assert s["positions"] == list(range(20)) + list(range(8)) + list(range(4))
    # blocks are popped in order: seq0 -> 0, 1; seq1 -> 2; seq2 -> 3
    assert s["slot_mapping"] == list(range(20)) + list(range(32, 40)) + list(range(48, 52))
    assert s["block_tables"] is None
    eng.postprocess([1, 2, 3])
    s = eng.schedule()
    # decodes first (seq0 at 20, seq2 at 4); seq1's cached 8 tokens drop to the block
    # boundary 0 (the hit-free prefix lookup), so its next chunk is again positions 0..7
    assert s["seq_ids"] == [0, 2, 1] and s["num_decode_tokens"] == 2
    assert s["positions"] == [20, 4] + list(range(8))
    assert s["input_ids"] == [1, 3] + list(range(1000, 1008))
    assert s["cu_seqlens_k"] == [0, 21, 26, 34]
    assert s["block_tables"] == [[0, 1], [3, -1], [2, -1]]


# ------------------------------------------------------------- invariants -------------

def _check_invariants(eng, s, budget, max_seqs):
    n = len(s["input_ids"])
    assert n == s["cu_seqlens_q"][-1] <= budget
    assert len(s["seq_ids"]) <= max_seqs
    q = [b - a for a, b in zip(s["cu_seqlens_q"], s["cu_seqlens_q"][1:])]
    assert all(x == 1 for x in q[:s["num_decode_tokens"]])       # decodes come first
    owned = set()
    for i, sid in enumerate(s["seq_ids"]):
        seq = eng.seqs[sid]
        k = s["context_lens"][i]
        pos = s["positions"][s["cu_seqlens_q"][i]:s["cu_seqlens_q"][i + 1]]
        assert pos == list(range(k - q[i], k))                     # contiguous, ends at Lk
        for j, p in enumerate(pos):
            slot = s["slot_mapping"][s["cu_seqlens_q"][i] + j]
            assert slot == seq.table[p // eng.bs] * eng.bs + p % eng.bs
        assert not owned & set(seq.table)                          # blocks are exclusive
        owned |= set(seq.table)
    live = [x for x in eng.seqs if x.status != E.FINISHED]
    assert len(eng.free) + sum(len(x.table) for x in live) == eng.num_blocks


def _random_workload(seed, n_req=14):
    rng = random.Random(seed)
    reqs = [([rng.randrange(50000) for _ in range(rng.randint(1, 90))], rng.randint(1, 40),
             rng.random() < 0.7) for _ in range(n_req)]
    return rng, reqs


KW = dict(num_blocks=24, block_size=16, max_num_seqs=5, max_num_batched_tokens=64,
          chunked_prefill_size=16, max_live_seqs=6, eos=3)


def _tokens(step, ids):
    return [(step * 7 + sid * 13) % 11 for sid in ids]   # eos (3) shows up now and then


@pytest.mark.parametrize("seed", [0, 1, 2, 3])
def test_oracle_invariants_on_random_workloads(seed):
    _, reqs = _random_workload(seed)
    eng = E.RefEngine(**KW)
    for p, m, ign in reqs:
        eng.add(p, m, ign)
    step = 0
    while not eng.finished():
        s = eng.schedule()
        _check_invariants(eng, s, KW["max_num_batched_tokens"], KW["max_num_seqs"])
        eng.postprocess(_tokens(step, s["seq_ids"]))
        step += 1
        assert step < 5000
    assert len(eng.free) == KW["num_blocks"]


# ------------------------------------------------------------- planted mistakes -------

def _lifo_take(self, seq, n):
    for _ in range(n):
        b = self.free.pop()
        self.refs[b] = 1
        seq.table.append(b)


def _no_new_block(self, seq):
    return False


@pytest.mark.parametrize("attr,fake,check", [
    ("_take", _lifo_take, test_single_sequence_prefill_then_decode),
    ("_opens_block", _no_new_block, test_decode_that_opens_a_block_takes_the_next_free_block),
])
def test_planted_mistake_is_caught(monkeypatch, attr, fake, check):
    monkeypatch.setattr(E.RefEngine, attr, fake)
    with pytest.raises((AssertionError, IndexError)):
        check()


def test_planted_slot_offset_mistake_is_caught(monkeypatch):
    orig = E.RefEngine.schedule

    def bad(self):
        s = orig(self)
        if s is not None and s["slot_mapping"]:
            s["slot_mapping"] = [x - x % self.bs for x in s["slot_mapping"]]
        return s
    monkeypatch.setattr(E.RefEngine, "schedule", bad)
    with pytest.raises(AssertionError):
        test_single_sequence_prefill_then_decode()


# ------------------------------------------------------------- C++ == oracle ----------

@pytest.mark.parametrize("seed", list(range(8)))
def test_host_core_matches_oracle_step_by_step(seed):
    _, reqs = _random_workload(seed, n_req=18)
    ref = E.RefEngine(**KW)
    core = cpp(max_seq_len=512, **KW)
    for p, m, ign in reqs:
        assert ref.add(p, m, ign) == core.add_request(p, m, ign)
    step = 0
    while True:
        want = ref.schedule()
        got = step_dict(core.schedule())
        assert got == want, f"step {step}"
        if want is None:
            break
        toks = _tokens(step, want["seq_ids"])
        assert core.postprocess(toks) == ref.postprocess(toks)
        assert core.num_free_blocks() == len(ref.free)
        step += 1
    assert core.is_finished()
    for sid in range(len(reqs)):
        assert core.generated(sid) == ref.generated(sid)


def test_host_core_config5_shape_matches_oracle():
    # the serving configuration's shape: 256 requests, prompts and outputs U[100, 1024],
    # block 256, 16384-token budget, 512-token chunks, 128 live sequences, ignore_eos
    rng = random.Random(5)
    reqs = [([rng.randrange(151936) for _ in range(rng.randint(100, 1024))], rng.randint(100, 1024))
            for _ in range(256)]
    kw = dict(num_blocks=2048, block_size=256, max_num_seqs=512, max_num_batched_tokens=16384,
              chunked_prefill_size=512, max_live_seqs=128, eos=151645)
    ref, core = E.RefEngine(**kw), cpp(max_seq_len=8192, **kw)
    for p, m in reqs:
        ref.add(p, m, True)
        core.add_request(p, m, True)
    step = 0
    while True:
        want = ref.schedule()
        got = step_dict(core.schedule())
        if step % 25 == 0 or want is None:      # full comparison on a sample of steps
            assert got == want, f"step {step}"
        else:
            assert got["cu_seqlens_k"] == want["cu_seqlens_k"] and got["slot_mapping"] == want["slot_mapping"]
        if want is None:
            break
        toks = [(step + sid) % 151936 for sid in want["seq_ids"]]
        core.postprocess(toks)
        ref.postprocess(toks)
        step += 1
    assert sum(len(core.generated(i)) for i in range(256)) == sum(m for _, m in reqs)


def test_host_core_rejects_bad_calls():
    core = cpp(num_blocks=4, block_size=16, max_seq_len=64)
    with pytest.raises(HostError):
        core.add_request(list(range(100)), 4)          # prompt larger than the pool
    with pytest.raises(HostError):
        core.add_request(list(range(10)), 100)         # prompt + output larger than the pool
    with pytest.raises(HostError):
        core.postprocess([1])                          # no open step
    assert core.schedule() is None and core.is_finished()
    sid = core.add_request([1, 2, 3], 2)
    st = core.schedule()
    assert st.num_seqs == 1 and st.is_prefill
    with pytest.raises(HostError):
        core.schedule()                                # previous step still open
    with pytest.raises(HostError):
        core.postprocess([1, 2])                       # wrong count
    core.postprocess([4])
    assert core.generated(sid) == [4]
    assert torch.is_tensor(st.input_ids)


def test_kv_cache_sizing_follows_reference_formula(monkeypatch):
    """model_runner.py:149-157: blocks = (total x util - used - peak + current) // block_bytes,
    block_bytes = 2 x layers x block_size x kv_heads x head_dim x itemsize; a request above
    that raises; None or <= 0 takes the maximum."""
    import torch
    from pagedkv.runner import kv_cache_num_blocks

    gib = 1 << 30
    total, free = 288 * gib, 280 * gib
    stats = {"allocated_bytes.all.peak": 3 * gib, "allocated_bytes.all.current": 2 * gib}
    monkeypatch.setattr(torch.cuda, "mem_get_info", lambda device=None: (free, total))
    monkeypatch.setattr(torch.cuda, "memory_stats", lambda device=None: stats)
    block_bytes = 2 * 28 * 256 * 8 * 128 * 2                      # Qwen3-0.6B, block 256, bf16
    budget = int(total * 0.9 - (total - free) - 3 * gib + 2 * gib)
    want = budget // block_bytes
    assert kv_cache_num_blocks(28, 256, 8, 128, 0.9) == want
    assert kv_cache_num_blocks(28, 256, 8, 128, 0.9, requested=0) == want
    assert kv_cache_num_blocks(28, 256, 8, 128, 0.9, requested=100) == 100
    with pytest.raises(RuntimeError, match="Not enough GPU memory"):
        kv_cache_num_blocks(28, 256, 8, 128, 0.9, requested=want + 1)
    # the activation headroom counts: a higher peak leaves fewer blocks
    stats["allocated_bytes.all.peak"] = 10 * gib
    assert kv_cache_num_blocks(28, 256, 8, 128, 0.9) == (budget - 7 * gib) // block_bytes
