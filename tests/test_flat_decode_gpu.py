"""GPU parity of the flat decode grid (paged_decode.hip decode_flat_kernel).

Batches of at most 192 sequences with a launch bound (num_seqs x max_seqlen_k) of at least
32768 keys are cut into equal runs of keys over the whole batch instead of per-sequence
splits; a sequence's pieces are merged by the combine pass from partial units b + w. These
tests hold that grid to the oracle (attention.py:95-104 decode rows) on serving-sized
batches, against the split grid on the same sequences (the split grid is selected by padding
the batch past 192 sequences with zero-length rows, as graph padding does), on sequences
long enough to need more pieces than one round of the combine's loads merges, and on the two
one-launch decode steps (store + decode, norm + RoPE + store + decode), which must stay
bit-identical to their unfused sequences.
"""
import math

import pytest
import torch

import pagedkv
from pagedkv import workloads as W
from paged_helpers import assert_close_bf16, subset_oracle
from test_fused_decode_gpu import _assert_same, _batch, _both

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5


def _decode_batch(lens, seed, dev):
    g = torch.Generator().manual_seed(seed)
    nb = sum(math.ceil(lk / W.BLOCK_SIZE) for lk in lens)
    tables = W._pop_tables(lens, torch.randperm(nb, generator=g).tolist())
    return W._assemble("flat", [(1, lk, bt) for lk, bt in zip(lens, tables)], nb, seed, dev, unique_blocks=nb)


def _store(w):
    """The batch's new K/V rows into their slots, as Attention.forward stores them before
    attending (attention.py:87-88); subset_oracle computes what that store then attends."""
    pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, w.slot_mapping)


def _attend(w, cu_q=None, cu_k=None, bt=None):
    cu_q = w.cu_seqlens_q if cu_q is None else cu_q
    cu_k = w.cu_seqlens_k if cu_k is None else cu_k
    bt = w.block_tables if bt is None else bt
    return pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, cu_q, cu_k, 1, w.max_seqlen_k, SCALE, True, bt,
                                    cached_prefix_keys=0)


def _padded(w, pad):
    """cu_seqlens and block tables of w followed by `pad` zero-length rows (graph padding:
    the reference runner zero-fills the tail of cu_seqlens, model_runner.py:251-254)."""
    z = torch.zeros(pad, dtype=torch.int32, device=w.q.device)
    bt = torch.cat([w.block_tables, torch.full((pad, w.block_tables.shape[1]), -1, dtype=torch.int32,
                                               device=w.q.device)])
    return torch.cat([w.cu_seqlens_q, z]), torch.cat([w.cu_seqlens_k, z]), bt


def test_flat_serving_batch_matches_oracle(gpu):
    """128 sequences of 100-2048 keys (the flat grid), every sequence against the oracle."""
    lens = W._uniform(torch.Generator().manual_seed(81), 100, 2048, 128)
    w = _decode_batch(lens, 81, gpu)
    rows, want = subset_oracle(w, list(range(len(lens))))
    _store(w)
    out = _attend(w)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, "flat grid, 128 x U[100, 2048]")


@pytest.mark.parametrize("n,lo,hi", [(128, 100, 2048), (16, 1024, 8192), (64, 1, 600)])
def test_flat_and_split_grids_agree(gpu, n, lo, hi):
    """The same sequences through the flat grid (n <= 192) and the split grid (padded to
    200 > 192 rows): both within tolerance of the oracle and within the merge rounding of
    each other (each path rounds its pieces' outputs to bf16 before the merge, an error
    relative to the pieces' outputs rather than to the merged row, and rounds the merged row
    once more); the padding rows take no part (their cu_seqlens differences are 0 or
    negative)."""
    lens = W._uniform(torch.Generator().manual_seed(n + lo), lo, hi, n)
    w = _decode_batch(lens, n + lo, gpu)
    ids = list(range(0, n, max(1, n // 24)))
    rows, want = subset_oracle(w, ids)
    _store(w)
    flat = _attend(w)
    cu_q, cu_k, bt = _padded(w, 200 - n)
    split = _attend(w, cu_q, cu_k, bt)
    torch.cuda.synchronize()
    assert_close_bf16(flat[rows], want, "flat grid")
    assert_close_bf16(split[rows], want, "split grid")
    _assert_within_merge_rounding(flat, split)


def _assert_within_merge_rounding(a, b):
    a, b = a.float(), b.float()
    bound = 2.0 ** -7 * torch.maximum(a.abs(), b.abs()) + 4e-3
    assert ((a - b).abs() <= bound).all(), f"max diff {(a - b).abs().max().item():.3e}"


def test_flat_long_sequences_merge_many_pieces(gpu):
    """Two 40k-key sequences among short ones: their pieces (~250 each) exceed one round of
    the combine's loads (64 partials), so they merge in several rounds folded together."""
    lens = [40000, 38111, 300, 5, 1, 2047]
    w = _decode_batch(lens, 83, gpu)
    rows, want = subset_oracle(w, list(range(len(lens))))
    _store(w)
    out = _attend(w)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, "flat grid, 40k-key sequences")


def test_flat_graph_padding_and_truncation(gpu):
    """Graph-padded tail rows (zero cu_seqlens) inside the flat grid's range, and a
    max_seqlen_k larger than every sequence (a captured graph's bound): the padding takes no
    part and the results agree with the unpadded call to within the merge rounding (the two
    launch bounds give slightly different run lengths)."""
    lens = W._uniform(torch.Generator().manual_seed(84), 300, 3000, 100)
    w = _decode_batch(lens, 84, gpu)
    base = _attend(w)
    cu_q, cu_k, bt = _padded(w, 12)
    bt = torch.cat([bt, torch.full((bt.shape[0], 4), -1, dtype=torch.int32, device=gpu)], 1)
    pad = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, cu_q, cu_k, 1, w.max_seqlen_k + 1000, SCALE, True,
                                   bt, cached_prefix_keys=0)
    torch.cuda.synchronize()
    _assert_within_merge_rounding(base, pad)


@pytest.mark.parametrize("hq,hkv", [(16, 8), (16, 2), (8, 4), (2, 1)])
def test_flat_fused_decode_bit_identical(gpu, hq, hkv):
    """pk_qkv_decode_attention against pk_qk_norm_rope_store + pk_varlen_attention_ex on a
    flat-grid batch with graph padding: output and caches bit for bit."""
    lens = W._uniform(torch.Generator().manual_seed(85 + hkv), 100, 2048, 120)
    b = _batch(lens, hq, hkv, seed=85 + hkv, dev=gpu, pad=8)
    cs = pagedkv.rope_cos_sin(40960, 128, 1000000.0, gpu)
    a, f = _both(b, hq, hkv, cs)
    _assert_same(a, f, b["S"])


def test_flat_store_decode_bit_identical(gpu):
    """Attention.forward's one-launch store + decode against store_kvcache +
    varlen_attention on a flat-grid batch with graph padding rows."""
    hq, hkv, D = 16, 8, 128
    lens = W._uniform(torch.Generator().manual_seed(86), 100, 2048, 120)
    b = _batch(lens, hq, hkv, seed=86, dev=gpu, pad=8)
    S, n = b["S"], b["S"] + 8
    g = torch.Generator().manual_seed(87)
    q = torch.randn(n, hq, D, generator=g).to(torch.bfloat16).to(gpu)
    key = torch.randn(n, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    value = torch.randn(n, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    kca, vca = b["kc"].clone(), b["vc"].clone()
    pagedkv.store_kvcache(key, value, kca, vca, b["slot"])
    out_a = pagedkv.varlen_attention(q, kca, vca, b["cu_q"], b["cu_k"], 1, b["maxk"], SCALE, True, b["bt"],
                                     cached_prefix_keys=0)
    kcb, vcb = b["kc"].clone(), b["vc"].clone()
    layer = pagedkv.Attention(D, hq, hkv, SCALE)
    layer.k_cache, layer.v_cache = kcb, vcb
    ctx = pagedkv.Context(False, b["cu_q"], b["cu_k"], 1, b["maxk"], b["slot"], None, b["bt"], 0)
    out_b = layer(q, key, value, ctx)
    torch.cuda.synchronize()
    _assert_same((out_a, kca, vca), (out_b, kcb, vcb), S)
