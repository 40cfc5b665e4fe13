"""GPU parity of chunked prefill when the work list splits query tiles over key ranges.

The prefill path plans its work on the device: query tiles whose causal key range is long
compared with the total work are cut into key splits whose partial numerators a merge
pass combines. These batches are shaped so that splits, unsplit tiles and both together
occur, for every GQA group built, paged and flat, causal and not; each result is held to
the same bar as the other attention tests (2e-2 max abs, 1e-2 mean abs of the fp32
oracle), and split results must be run-to-run bit-identical (the work list order varies,
the arithmetic of every row does not).
"""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from paged_helpers import assert_close_bf16, bits_equal
from pagedkv.workloads import BLOCK_SIZE

pytestmark = pytest.mark.gpu


def _batch(dev, seqs, hq=16, hkv=8, seed=0, paged=True):
    """seqs: list of (Lq, Lk). Returns the call arguments and the oracle inputs."""
    g = torch.Generator(device=dev).manual_seed(seed)
    nq = sum(lq for lq, _ in seqs)
    q = torch.randn(nq, hq, 128, generator=g, device=dev, dtype=torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum([s[0] for s in seqs]).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum([s[1] for s in seqs]).tolist(), dtype=torch.int32)
    if paged:
        nb_per = [math.ceil(lk / BLOCK_SIZE) for _, lk in seqs]
        nb = sum(nb_per)
        perm = torch.randperm(nb, generator=torch.Generator().manual_seed(seed + 1)).tolist()
        bt = torch.full((len(seqs), max(nb_per)), -1, dtype=torch.int32)
        pos = 0
        for i, c in enumerate(nb_per):
            bt[i, :c] = torch.tensor(perm[pos:pos + c])
            pos += c
        k = torch.randn(nb, BLOCK_SIZE, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(nb, BLOCK_SIZE, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
    else:
        bt = None
        nk = sum(lk for _, lk in seqs)
        k = torch.randn(nk, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
        v = torch.randn(nk, hkv, 128, generator=g, device=dev, dtype=torch.bfloat16)
    return q, k, v, cu_q, cu_k, bt


def _ws_bytes(args, seqs):
    q = args[0]
    return pagedkv.workspace_bytes(len(seqs), q.shape[1], q.shape[2], max(s[0] for s in seqs),
                                   max(s[1] for s in seqs))


def _run(dev, q, k, v, cu_q, cu_k, bt, seqs, causal=True, workspace=None, fresh_workspace=False):
    """fresh_workspace: a zero-filled workspace of exactly the needed size for this call."""
    if fresh_workspace:
        workspace = torch.zeros(max(1, _ws_bytes((q,), seqs)), dtype=torch.uint8, device=dev)
    return pagedkv.varlen_attention(q, k, v, cu_q.to(dev), cu_k.to(dev), max(s[0] for s in seqs),
                                    max(s[1] for s in seqs), None, causal, None if bt is None else bt.to(dev),
                                    workspace=workspace)


def _check(dev, seqs, hq=16, hkv=8, paged=True, causal=True, seed=0, what=""):
    q, k, v, cu_q, cu_k, bt = _batch(dev, seqs, hq, hkv, seed, paged)
    print(f"[prefill-split] {what} hq={hq} hkv={hkv} paged={paged} causal={causal} seqs={seqs}", flush=True)
    out = _run(dev, q, k, v, cu_q, cu_k, bt, seqs, causal)
    want = oracle.varlen_attention(q.cpu(), k.cpu(), v.cpu(), cu_q, cu_k, None, causal, bt)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, what)
    return out


# one long chunk over a long cached prefix (split into many key ranges) next to short ones
SKEWED = [(256, 256 + 12000), (300, 400), (64, 64), (2, 5000), (1, 3000), (130, 130 + 700)]


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4), (32, 4)])
def test_skewed_chunked_prefill_paged(gpu, hq, hkv):
    _check(gpu, SKEWED, hq, hkv, what="skewed paged")


def test_skewed_noncausal_paged(gpu):
    _check(gpu, SKEWED, causal=False, what="skewed non-causal")


def test_flat_prompts_like_serving_prefill(gpu):
    """All-fresh prompts of the serving workload's lengths (no split needed: many units)."""
    rng = np.random.default_rng(7)
    seqs = [(int(n), int(n)) for n in rng.integers(100, 1025, size=24)]
    _check(gpu, seqs, paged=False, what="flat prompts")


def test_single_long_flat_prompt(gpu):
    """One 6000-token fresh prompt: the last query tiles see the whole prompt and split."""
    _check(gpu, [(6000, 6000)], paged=False, what="one long prompt")


def test_rows_without_keys_are_zero(gpu):
    """Lk < Lq (not produced by the reference runner): rows before the first key see nothing
    and are written as 0, split or not, matching the oracle."""
    seqs = [(300, 200), (40, 3000)]
    out = _check(gpu, seqs, what="rows without keys")
    assert torch.count_nonzero(out[:100].float()) == 0


def test_split_results_bit_identical_across_runs(gpu):
    q, k, v, cu_q, cu_k, bt = _batch(gpu, SKEWED, seed=3)
    outs = [_run(gpu, q, k, v, cu_q, cu_k, bt, SKEWED) for _ in range(3)]
    torch.cuda.synchronize()
    assert all(bits_equal(o, outs[0]) for o in outs[1:])


def test_workspace_reuse_after_split_call(gpu):
    """A split-heavy call, then small ones, then the split call again on one shared
    workspace: every result equals the same call on a fresh zero-filled workspace (the plan
    resets its claim counters and rewrites its lists each call)."""
    batches = [SKEWED, [(70, 70), (3, 900)], [(512, 512 + 4000)], SKEWED]
    args = [_batch(gpu, s, seed=11 + i) for i, s in enumerate(batches)]
    fresh = [_run(gpu, *a, s, fresh_workspace=True) for s, a in zip(batches, args)]
    shared = torch.empty(max(_ws_bytes(a, s) for s, a in zip(batches, args)), dtype=torch.uint8, device=gpu)
    for rep in range(2):
        for s, a, want in zip(batches, args, fresh):
            got = _run(gpu, *a, s, workspace=shared)
            torch.cuda.synchronize()
            assert bits_equal(got, want), f"rep {rep} seqs {s}"


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 2), (8, 1)])
def test_many_small_items_exhaust_and_steal(gpu, hq, hkv):
    """Hundreds of short prompts over short cached prefixes: several items per work-group,
    so every work-group claims past its own sub-queue's end and steals from the others."""
    rng = np.random.default_rng(hq * 10 + hkv)
    seqs = []
    for i in range(300):
        lq = int(rng.integers(2, 41))
        seqs.append((lq, lq + int(rng.integers(0, 300))))
    _check(gpu, seqs, hq, hkv, seed=hkv, what=f"300 small prompts hkv={hkv}")


@pytest.mark.parametrize("hkv", [1, 8])
def test_fewer_items_than_work_groups(gpu, hkv):
    """One 2-token prompt (a single work item for hkv = 1): every other work-group finds all
    sub-queues empty on its first claim and leaves."""
    _check(gpu, [(2, 3)], 8 if hkv == 1 else 16, hkv, seed=3, what=f"one item hkv={hkv}")
    _check(gpu, [(2, 2), (1, 7), (3, 300)], 8 if hkv == 1 else 16, hkv, seed=4, what=f"three seqs hkv={hkv}")
