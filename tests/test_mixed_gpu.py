"""GPU parity of calls that mix decode rows (Lq == 1) with prefill rows.

One varlen_attention call runs the decode launch (split or flat grid, and the combine) for the
decode rows, then the prefill plan, persistent prefill kernel and merge for the rest. These
tests hold both kinds of rows to the oracle (attention.py:95-104) at serving size, the decode
rows also to the decode-only call of the same sequences (the call's launch bounds choose the
cut into pieces, so the two agree to within the merge rounding), and cover the edge cases of
such batches: a row long enough to be cut into many pieces, rows of one key, decode rows
between prefill chunks, graph-padded tails with raised launch bounds, GQA groups whose kv
heads fill part of a quad, and run-to-run determinism.
"""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from pagedkv import workloads as W
from paged_helpers import assert_close_bf16, bits_equal, subset_oracle

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _batch(spec, seed, dev):
    """spec: (Lq, Lk) per sequence in batch order; non-contiguous tables from a shuffled pool."""
    g = torch.Generator().manual_seed(seed)
    lks = [lk for _, lk in spec]
    nb = sum(math.ceil(lk / W.BLOCK_SIZE) for lk in lks)
    tables = W._pop_tables(lks, torch.randperm(nb, generator=g).tolist())
    return W._assemble("mixed", [(lq, lk, bt) for (lq, lk), bt in zip(spec, tables)], nb, seed, dev)


def _attend(w, cu_q=None, cu_k=None, bt=None, max_q=None, max_k=None):
    cu_q = w.cu_seqlens_q if cu_q is None else cu_q
    cu_k = w.cu_seqlens_k if cu_k is None else cu_k
    bt = w.block_tables if bt is None else bt
    return pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, cu_q, cu_k, max_q or w.max_seqlen_q,
                                    max_k or w.max_seqlen_k, SCALE, True, bt, cached_prefix_keys=0)


def _store(w):
    pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, w.slot_mapping)


def _assert_within_merge_rounding(a, b):
    """Two cuts of the same rows into pieces: each rounds its pieces' outputs to bf16 before the
    merge (an error relative to the pieces' outputs) and the merged row once more."""
    a, b = a.float(), b.float()
    bound = 2.0 ** -7 * torch.maximum(a.abs(), b.abs()) + 4e-3
    assert ((a - b).abs() <= bound).all(), f"max diff {(a - b).abs().max().item():.3e}"


def test_mixed_serving_batch_matches_oracle(gpu):
    """The mixed chunked-prefill batch at full size (128 decodes of 512-4096 keys, 8 prefill
    chunks of 512 tokens over prefixes of 0-4096): every decode row and two prefill chunks
    against the oracle."""
    w = W.make_workload("cfg3", gpu)
    ids = list(range(128)) + [128, 133]
    rows, want = subset_oracle(w, ids)
    _store(w)
    out = _attend(w)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, "mixed batch, decode rows + 2 prefill chunks")


def test_mixed_decode_rows_match_decode_only_call(gpu):
    """The decode rows of a mixed batch against the same sequences called alone (the decode
    launch): within the merge rounding, and both within tolerance of the oracle."""
    spec = [(1, lk) for lk in W._uniform(torch.Generator().manual_seed(91), 100, 3000, 96)]
    spec[10:10] = [(256, 1000), (512, 512)]
    spec.append((300, 4300))
    w = _batch(spec, 91, gpu)
    dec = [i for i, (lq, _) in enumerate(spec) if lq == 1]
    rows, want = subset_oracle(w, dec)
    _store(w)
    mixed = _attend(w)
    # the decode sequences alone: their rows of the batch, cu_seqlens of the subset
    ridx = torch.tensor(rows, dtype=torch.long, device=gpu)
    lks = [spec[i][1] for i in dec]
    cu_q = torch.arange(len(dec) + 1, dtype=torch.int32, device=gpu)
    cu_k = torch.tensor([0] + np.cumsum(lks).tolist(), dtype=torch.int32, device=gpu)
    bt = w.block_tables[torch.tensor(dec, device=gpu)]
    alone = pagedkv.varlen_attention(w.q.index_select(0, ridx), w.k_cache, w.v_cache, cu_q, cu_k, 1, max(lks),
                                     SCALE, True, bt, cached_prefix_keys=0)
    torch.cuda.synchronize()
    assert_close_bf16(mixed[rows], want, "mixed path")
    assert_close_bf16(alone, want, "decode launch")
    _assert_within_merge_rounding(mixed[rows], alone)


def test_mixed_long_tiny_and_interleaved_rows(gpu):
    """A 40000-key decode row (many pieces), rows of 1 and 7 keys, decode rows between prefill
    chunks, and a prefill chunk first: every row against the oracle."""
    spec = [(64, 5000), (1, 40000), (1, 1), (300, 300), (1, 7), (1, 2047), (1, 300), (17, 17), (1, 256)]
    w = _batch(spec, 92, gpu)
    rows, want = subset_oracle(w, list(range(len(spec))))
    _store(w)
    out = _attend(w)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, "long, tiny and interleaved rows")


def test_mixed_graph_padding_and_bound(gpu):
    """Graph-padded tail rows (zero cu_seqlens) and launch bounds above every sequence: the
    padding takes no part, prefill rows are bit-identical and decode rows agree to within the
    merge rounding (the raised bounds may cut them into different pieces)."""
    spec = [(1, lk) for lk in W._uniform(torch.Generator().manual_seed(93), 300, 3000, 60)] + [(128, 2000)]
    w = _batch(spec, 93, gpu)
    _store(w)
    base = _attend(w)
    z = torch.zeros(9, dtype=torch.int32, device=gpu)
    cu_q = torch.cat([w.cu_seqlens_q, z])
    cu_k = torch.cat([w.cu_seqlens_k, z])
    bt = torch.cat([w.block_tables, torch.full((9, w.block_tables.shape[1]), -1, dtype=torch.int32, device=gpu)])
    bt = torch.cat([bt, torch.full((bt.shape[0], 4), -1, dtype=torch.int32, device=gpu)], 1)
    pad = _attend(w, cu_q, cu_k, bt, max_q=w.max_seqlen_q + 64, max_k=w.max_seqlen_k + 1000)
    torch.cuda.synchronize()
    _assert_within_merge_rounding(base, pad)
    pre = slice(int(w.cu_seqlens_q[-2]), int(w.cu_seqlens_q[-1]))
    assert bits_equal(base[pre], pad[pre])


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 4), (8, 2), (16, 16)])
def test_mixed_gqa_groups(gpu, hq, hkv):
    """Groups of 1, 4, 4 and 1 query heads with 8, 4, 2 and 16 kv heads (decode wavefronts of
    4 kv heads with idle rows, and several per work-group), decode rows long enough to be cut
    into pieces."""
    g = torch.Generator().manual_seed(hq * 10 + hkv)
    seqs = [(1, 3000), (1, 33), (200, 700), (1, 1500), (1, 9000), (40, 40)]
    nb_per = [math.ceil(lk / W.BLOCK_SIZE) for _, lk in seqs]
    nb = sum(nb_per)
    perm = torch.randperm(nb, generator=g).tolist()
    bt = torch.full((len(seqs), max(nb_per)), -1, dtype=torch.int32)
    pos = 0
    for i, c in enumerate(nb_per):
        bt[i, :c] = torch.tensor(perm[pos:pos + c])
        pos += c
    nq = sum(s[0] for s in seqs)
    q = torch.randn(nq, hq, 128, generator=g).to(torch.bfloat16)
    kc = torch.randn(nb, W.BLOCK_SIZE, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, W.BLOCK_SIZE, hkv, 128, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum([s[0] for s in seqs]).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum([s[1] for s in seqs]).tolist(), dtype=torch.int32)
    out = pagedkv.varlen_attention(q.to(gpu), kc.to(gpu), vc.to(gpu), cu_q.to(gpu), cu_k.to(gpu), 200, 9000, SCALE,
                                   True, bt.to(gpu))
    want = oracle.varlen_attention(q, kc, vc, cu_q, cu_k, SCALE, True, bt)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, f"mixed gqa {hq}/{hkv}")


def test_mixed_deterministic(gpu):
    """Prefill items are claimed in a different order on every call; the pieces, their merge
    order and so every output bit are not."""
    w = W.make_workload("cfg3", gpu, num_seqs=64)
    _store(w)
    a = _attend(w)
    b = _attend(w)
    torch.cuda.synchronize()
    assert bits_equal(a, b)
