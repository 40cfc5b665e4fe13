"""GPU parity of the shared-prefix decode path (pk_varlen_attention_shared_prefix, through the
C-ABI): decode rows whose leading blocks several sequences share are computed once per shared
block on MFMA tiles, the rest by the split-K kernel, merged by the combine.

Bars: within 2e-2 max / 1e-2 mean abs of the fp32 oracle (the reference's semantics,
attention.py:95-104 over block tables that share blocks through reference counts,
block_manager.py:96-181); bit-identical run to run; bit-identical whether the prefix blocks are
shared or duplicated per sequence (a row's arithmetic does not depend on its tile mates).
"""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from paged_helpers import assert_close_bf16, bits_equal, subset_oracle
from pagedkv.workloads import BLOCK_SIZE, make_workload

pytestmark = pytest.mark.gpu
BS = BLOCK_SIZE


def _batch(tables, lens, q_lens, hq, hkv, nb, seed, dev):
    """Caches of nb random blocks, the given (-1 padded) block tables, q rows per sequence."""
    g = torch.Generator().manual_seed(seed)
    width = max(len(t) for t in tables)
    bt = torch.full((len(tables), width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    kc = torch.randn(nb, BS, hkv, 128, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, BS, hkv, 128, generator=g).to(torch.bfloat16)
    q = torch.randn(sum(q_lens), hq, 128, generator=g).to(torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum(q_lens).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32)
    return dict(q=q.to(dev), kc=kc.to(dev), vc=vc.to(dev), bt=bt.to(dev), cu_q=cu_q.to(dev), cu_k=cu_k.to(dev),
                maxq=max(q_lens), maxk=max(lens), cpu=(q, kc, vc, cu_q, cu_k, bt))


def _run(b, shared, hint=None):
    return pagedkv.varlen_attention(b["q"], b["kc"], b["vc"], b["cu_q"], b["cu_k"], b["maxq"], b["maxk"], None, True,
                                    b["bt"], cached_prefix_keys=hint, shared_prefix_keys=shared)


def _oracle(b):
    q, kc, vc, cu_q, cu_k, bt = b["cpu"]
    return oracle.varlen_attention(q, kc, vc, cu_q, cu_k, None, True, bt)


def test_cfg4_shared_prefix_matches_oracle_and_private_copies(gpu):
    """cfg4 at full size: 64 sequences share one 2048-key prefix (8 blocks)."""
    print("[shared prefix] cfg4, 64 sequences", flush=True)
    w = make_workload("cfg4", gpu)
    assert w.shared_prefix_keys == 2048
    rows, want = subset_oracle(w, list(range(len(w.q_lens))))
    pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, w.slot_mapping)
    args = (w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k, 1, w.max_seqlen_k, None, True,
            w.block_tables)
    out = pagedkv.varlen_attention(*args, cached_prefix_keys=2048, shared_prefix_keys=2048)
    again = pagedkv.varlen_attention(*args, cached_prefix_keys=2048, shared_prefix_keys=2048)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, "cfg4 shared prefix")
    assert bits_equal(out, again)
    # the same batch with a private copy of the prefix per sequence: identical bits
    shared = w.meta["shared_blocks"]
    nb, s = w.k_cache.shape[0], len(w.q_lens)
    extra = torch.tensor(shared, device=gpu).repeat(s)
    kc = torch.cat([w.k_cache, w.k_cache[extra]])
    vc = torch.cat([w.v_cache, w.v_cache[extra]])
    bt = w.block_tables.clone()
    bt[:, :len(shared)] = (nb + torch.arange(s * len(shared), device=gpu).view(s, -1)).int()
    priv = pagedkv.varlen_attention(w.q, kc, vc, w.cu_seqlens_q, w.cu_seqlens_k, 1, w.max_seqlen_k, None, True, bt,
                                    cached_prefix_keys=2048, shared_prefix_keys=2048)
    torch.cuda.synchronize()
    assert bits_equal(out, priv)


def test_attention_forward_takes_shared_prefix_path(gpu):
    """Attention.forward with a Context that states the shared prefix (cfg4's 2048 keys)."""
    w = make_workload("cfg4", gpu, num_seqs=24)
    rows, want = subset_oracle(w, list(range(len(w.q_lens))))
    layer = pagedkv.Attention(128, 16, 8, 128 ** -0.5)
    layer.k_cache, layer.v_cache = w.k_cache, w.v_cache
    assert w.ctx.cached_prefix_keys == 2048
    out = layer(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, "forward, shared prefix")


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4), (16, 2)])
def test_irregular_sharing_matches_oracle(gpu, hq, hkv):
    """Tree-shaped sharing (a common first block, then two branches), sequences that end
    inside the shared region or exactly at its end, one sequence sharing nothing, graph
    padding rows, and a prefix bound that is not a whole number of chunks."""
    root, left, right = 0, 1, 2
    tables, lens = [], []
    nxt = 3
    for i in range(12):                      # branch left: blocks (0, 1), then private ones
        priv = list(range(nxt, nxt + 2))
        nxt += 2
        tables.append([root, left] + priv)
        lens.append(2 * BS + 17 + 37 * i)
    for i in range(9):                       # branch right: blocks (0, 2)
        priv = [nxt]
        nxt += 1
        tables.append([root, right] + priv)
        lens.append(2 * BS + 5 + 11 * i)
    tables.append([root, left])              # ends exactly at the end of the shared region
    lens.append(2 * BS)
    tables.append([root])                    # ends inside the first shared block
    lens.append(100)
    tables.append([root, left])              # ends inside the second one
    lens.append(BS + 200)
    tables.append(list(range(nxt, nxt + 4)))  # shares nothing
    nxt += 4
    lens.append(4 * BS - 3)
    tables.append([])                        # graph padding: no keys
    lens.append(0)
    q_lens = [1] * (len(tables) - 1) + [0]
    b = _batch(tables, lens, q_lens, hq, hkv, nxt, seed=hq * 10 + hkv, dev=gpu)
    want = _oracle(b)
    for shared in (2 * BS, 2 * BS + 100, 3 * BS):
        out = _run(b, shared, hint=shared)
        torch.cuda.synchronize()
        n = sum(q_lens)
        assert_close_bf16(out[:n], want[:n], f"irregular sharing, P={shared}")


def test_more_sharers_than_one_tile(gpu):
    """200 sequences share three blocks: more members than one MFMA item holds (128 for
    GQA group 2), so the prefix chunks are processed by several items."""
    tables, lens = [], []
    nxt = 3
    for i in range(200):
        tables.append([0, 1, 2, nxt])
        nxt += 1
        lens.append(3 * BS + 1 + (i * 7) % 250)
    b = _batch(tables, lens, [1] * 200, 16, 8, nxt, seed=5, dev=gpu)
    out = _run(b, 3 * BS)
    torch.cuda.synchronize()
    assert_close_bf16(out, _oracle(b), "200 sharers")


def test_mixed_batch_with_shared_prefix(gpu):
    """Decode rows over a shared prefix next to chunked-prefill rows over the same blocks:
    the prefill rows go to the prefill kernel as without the shared-prefix path."""
    tables = [[0, 1, 2 + i] for i in range(6)] + [[0, 1, 8, 9]]
    lens = [2 * BS + 30 * (i + 1) for i in range(6)] + [3 * BS + 64]
    q_lens = [1] * 6 + [300]
    b = _batch(tables, lens, q_lens, 16, 8, 10, seed=7, dev=gpu)
    out = _run(b, 2 * BS)
    plain = _run(b, None, hint=2 * BS)
    torch.cuda.synchronize()
    assert_close_bf16(out, _oracle(b), "mixed batch, shared prefix")
    # prefill rows do not depend on the decode path
    assert bits_equal(out[6:], plain[6:])


def test_shared_prefix_in_graph_replays(gpu):
    """Captured once, replayed: every replay equals the eager call bit for bit."""
    w = make_workload("cfg4", gpu, num_seqs=32)
    ws = torch.empty(pagedkv.workspace_bytes(32, 16, 128, 1, w.max_seqlen_k), dtype=torch.uint8, device=gpu)

    def run():
        return pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k, 1, w.max_seqlen_k,
                                        None, True, w.block_tables, cached_prefix_keys=2048,
                                        shared_prefix_keys=2048, workspace=ws)
    want = run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert bits_equal(out, want), f"replay {rep}"
        again = run()
        torch.cuda.synchronize()
        assert bits_equal(again, want)


def test_prefix_below_one_chunk_is_the_plain_path(gpu):
    """The prefix is rounded down to whole chunks (lcm of the block size and the decode
    split); a bound below one chunk leaves the call on the plain path, bit for bit."""
    tables = [[0, 1 + i, 9 + i] for i in range(8)]
    lens = [2 * BS + 30 * i + 3 for i in range(8)]
    b = _batch(tables, lens, [1] * 8, 16, 8, 17, seed=9, dev=gpu)
    out = _run(b, BS - 56, hint=BS - 56)
    plain = _run(b, None, hint=BS - 56)
    torch.cuda.synchronize()
    assert bits_equal(out, plain)


@pytest.mark.parametrize("grid", ["flat", "split"])
def test_long_rows_merge_prefix_chunks_and_many_pieces(gpu, grid):
    """Rows of ~40k keys after a 2048-key shared prefix: each has the prefix chunks' partials
    plus its decode pieces (about 250 on the flat grid, 79 splits of 512 keys on the split
    grid), more than one round of the combine's loads (64 partials), so the combine folds
    several rounds that mix prefix and decode units. The 4-row batch takes the flat decode
    grid; padded with zero-length rows past 192 it takes the split grid."""
    lens = [2048 + 40000, 2048 + 39111, 2048 + 1000, 2048 + 38000]
    nsh = 2048 // BS
    priv = [math.ceil(lk / BS) - nsh for lk in lens]
    nb = nsh + sum(priv)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(21)).tolist()
    shared, pos, tables = perm[:nsh], nsh, []
    for n in priv:
        tables.append(shared + perm[pos:pos + n])
        pos += n
    q_lens = [1] * len(lens)
    if grid == "split":  # graph-padding rows: zero-length sequences after the real ones
        tables += [[-1]] * 196
        lens += [0] * 196
        q_lens += [0] * 196
    b = _batch(tables, lens, q_lens, 16, 8, nb, 22, gpu)
    print(f"[shared prefix] long rows, {grid} grid", flush=True)
    out = _run(b, 2048, hint=2048)
    want = _oracle(b)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, f"long rows, {grid} grid")


@pytest.mark.parametrize("hq,hkv", [(16, 8), (16, 2)])
def test_work_groups_take_several_groups_in_turn(gpu, hq, hkv):
    """256 sequences in six prefix groups (sequence b shares the 8 prefix blocks of group
    b mod 6), one private block each: every window of sequences (128 for GQA 2, 32 for GQA 8)
    holds all six groups, and the grid has 4 work-groups per window and chunk, so some take
    two groups in turn (reusing their member list and tile stages)."""
    nsh, ngrp, n = 8, 6, 256
    tables, lens = [], []
    nxt = ngrp * nsh
    for b in range(n):
        g = b % ngrp
        tables.append(list(range(g * nsh, (g + 1) * nsh)) + [nxt])
        nxt += 1
        lens.append(nsh * BS + 1 + (b * 37) % (BS - 1))
    b = _batch(tables, lens, [1] * n, hq, hkv, nxt, seed=31 + hkv, dev=gpu)
    print(f"[shared prefix] several groups per work-group, hq={hq} hkv={hkv}", flush=True)
    out = _run(b, nsh * BS, hint=nsh * BS)
    plain = _run(b, None, hint=nsh * BS)
    want = _oracle(b)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, f"six groups per window, hkv={hkv}")
    assert_close_bf16(plain, want, f"plain path, hkv={hkv}")


@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4), (32, 4), (16, 16), (24, 12), (2, 1)])
def test_one_launch_prefix_and_flat_suffixes(gpu, hq, hkv):
    """Batches whose suffixes take the flat decode grid run the prefix work and the suffix
    grid in one launch: 150 sequences over a 1024-key shared prefix (two shapes of sharing:
    all of it, and a branch sharing only its first block) with ragged suffixes, one sequence
    ending inside the prefix, and graph padding. GQA groups 1-8; 16 kv heads (four wavefronts
    per flat group), 12 (not a divisor of the work-group's wavefronts: two launches), and one.
    Every row against the oracle; bit-identical to private copies of the prefix blocks."""
    g = torch.Generator().manual_seed(hq * 100 + hkv)
    tables, lens = [], []
    nxt = 4
    for i in range(150):
        suffix = int(torch.randint(100, 1500, (1,), generator=g))
        nb_s = math.ceil(suffix / BS)
        head = [0, 1, 2, 3] if i % 5 else [0, 50000]                 # every fifth shares one block
        if head[-1] == 50000:
            head = [0, nxt]
            nxt += 1
        tables.append(head + list(range(nxt, nxt + nb_s)))
        lens.append(len(head) * BS + suffix)
        nxt += nb_s
    tables.append([0, 1])
    lens.append(BS + 77)                                              # ends inside the prefix
    tables.append([])
    lens.append(0)                                                    # graph padding
    q_lens = [1] * (len(tables) - 1) + [0]
    b = _batch(tables, lens, q_lens, hq, hkv, nxt, seed=hq * 10 + hkv, dev=gpu)
    print(f"[shared prefix] one launch {hq}/{hkv}", flush=True)
    want = _oracle(b)
    out = _run(b, 4 * BS, hint=4 * BS)
    torch.cuda.synchronize()
    n = sum(q_lens)
    assert_close_bf16(out[:n], want[:n], f"one launch {hq}/{hkv}")
    # private copies of blocks 0-3 per sequence: the same bits
    kc, vc, bt = b["kc"], b["vc"], b["bt"].clone()
    nb = kc.shape[0]
    extra = []
    for i in range(len(tables)):
        for j, blk in enumerate(tables[i][:4]):
            if blk < 4:
                bt[i, j] = nb + len(extra)
                extra.append(blk)
    idx = torch.tensor(extra, device=gpu)
    b2 = dict(b, kc=torch.cat([kc, kc[idx]]), vc=torch.cat([vc, vc[idx]]), bt=bt)
    priv = _run(b2, 4 * BS, hint=4 * BS)
    torch.cuda.synchronize()
    assert bits_equal(out[:n], priv[:n])
