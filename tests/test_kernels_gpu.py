"""GPU parity of the HIP kernels against the oracle (pytest -m gpu).

Bars: store and block-table gather bit-exact; attention within 2e-2 max abs and
1e-2 mean abs of the fp32 oracle (and of the fp64 brute-force known answers).
Every call goes through the C-ABI (pagedkv -> libpagedkv.so).
"""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from golden.cases import CASES, build_case, input_digest
from paged_helpers import assert_close_bf16, bits_equal, subset_oracle
from pagedkv.workloads import BLOCK_SIZE, make_workload

pytestmark = pytest.mark.gpu
GOLDEN = __import__("pathlib").Path(__file__).resolve().parent / "golden"


def _dev_bf16(bits, dev):
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).to(dev)


def _dev_i32(a, dev):
    return torch.from_numpy(np.asarray(a, dtype=np.int32).copy()).to(dev)


def _run_case(case, dev):
    bt = _dev_i32(case["block_table"], dev) if case["paged"] else None
    return pagedkv.varlen_attention(
        _dev_bf16(case["q"], dev), _dev_bf16(case["k"], dev), _dev_bf16(case["v"], dev),
        _dev_i32(case["cu_q"], dev), _dev_i32(case["cu_k"], dev),
        max(case["q_lens"]), max(case["k_lens"]), case["scale"], case["causal"], bt)


# ----------------------------------------------------------- known answers ---

@pytest.mark.parametrize("name", sorted(CASES))
def test_kat_against_fp64_bruteforce(gpu, name):
    print(f"[kat] {name}", flush=True)
    case = build_case(name)
    ref = np.load(GOLDEN / f"kat_{name}.npz")
    assert str(ref["digest"]) == input_digest(case)
    out = _run_case(case, gpu)
    torch.cuda.synchronize()
    assert_close_bf16(out, torch.from_numpy(ref["out"]), name)


# ------------------------------------------------------------------ store ----

@pytest.mark.parametrize("name", ["cfg1_store", "cfg2", "cfg3", "cfg4"])
def test_store_bit_exact(gpu, name):
    """Every configuration at its full size (cfg2: the 256 new tokens of the serving batch)."""
    print(f"[store] {name}", flush=True)
    w = make_workload(name, gpu)
    kc_ref, vc_ref = w.k_cache.cpu(), w.v_cache.cpu()
    oracle.store_kvcache(w.k.cpu(), w.v.cpu(), kc_ref, vc_ref, w.slot_mapping.cpu())
    pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, w.slot_mapping)
    torch.cuda.synchronize()
    assert bits_equal(w.k_cache, kc_ref) and bits_equal(w.v_cache, vc_ref)


def test_store_skips_padding_slots(gpu):
    g = torch.Generator(device=gpu).manual_seed(7)
    n, nb = 300, 6
    k = torch.randn(n, 8, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    qkv = torch.randn(n, 4096, generator=g, device=gpu, dtype=torch.bfloat16)
    v = qkv[:, 3072:].view(n, 8, 128)                           # strided like qwen3.py:80-84
    kc = torch.full((nb, BLOCK_SIZE, 8, 128), -3.0, device=gpu, dtype=torch.bfloat16)
    vc = kc.clone()
    perm = torch.randperm(nb * BLOCK_SIZE, generator=torch.Generator().manual_seed(1))[:n]
    slots = perm.to(torch.int32)
    slots[::7] = -1                                             # graph padding rows
    kc_ref, vc_ref = kc.cpu(), vc.cpu()
    oracle.store_kvcache(k.cpu(), v.cpu(), kc_ref, vc_ref, slots)
    pagedkv.store_kvcache(k, v, kc, vc, slots.to(gpu))
    torch.cuda.synchronize()
    assert bits_equal(kc, kc_ref) and bits_equal(vc, vc_ref)


def test_store_bound_check_drops_out_of_range(gpu):
    n = 4
    k = torch.ones(n, 8, 128, device=gpu, dtype=torch.bfloat16)
    kc = torch.zeros(2, BLOCK_SIZE, 8, 128, device=gpu, dtype=torch.bfloat16)
    vc = kc.clone()
    slots = torch.tensor([0, 2 * BLOCK_SIZE, -5, 1], dtype=torch.int32, device=gpu)
    pagedkv.ops.store_kvcache(k, k, kc, vc, slots, check_slots=True)
    torch.cuda.synchronize()
    rows = kc.view(-1, 8, 128)
    assert rows[0].eq(1).all() and rows[1].eq(1).all()
    assert rows[2:].eq(0).all()


def test_store_empty_batch(gpu):
    kc = torch.zeros(1, BLOCK_SIZE, 8, 128, device=gpu, dtype=torch.bfloat16)
    e = torch.empty(0, 8, 128, device=gpu, dtype=torch.bfloat16)
    pagedkv.store_kvcache(e, e, kc, kc.clone(), torch.empty(0, dtype=torch.int32, device=gpu))
    torch.cuda.synchronize()
    assert kc.eq(0).all()


# ----------------------------------------------------------------- gather ----

@pytest.mark.parametrize("name", ["cfg3", "cfg4"])
def test_gather_bit_exact(gpu, name):
    w = make_workload(name, gpu, num_seqs=16)
    got = pagedkv.gather_kv(w.k_cache, w.block_tables, w.cu_seqlens_k, w.max_seqlen_k, sum(w.k_lens))
    want = oracle.gather_kv(w.k_cache.cpu(), w.block_tables.cpu(), w.cu_seqlens_k.cpu())
    torch.cuda.synchronize()
    assert bits_equal(got, want)


# ----------------------------------------------- attention layer (drop-in) ---

def _layer(w):
    layer = pagedkv.Attention(128, 16, 8, 128 ** -0.5)
    layer.k_cache, layer.v_cache = w.k_cache, w.v_cache
    return layer


@pytest.mark.parametrize("name,num_seqs", [("cfg1_decode", None), ("cfg2", 24), ("cfg3", 24),
                                           ("cfg4", None), ("cfg3", None)])
def test_attention_forward_matches_oracle(gpu, name, num_seqs):
    print(f"[forward] {name} num_seqs={num_seqs}", flush=True)
    w = make_workload(name, gpu, num_seqs=num_seqs)
    ids = list(range(len(w.q_lens)))
    rows, want = subset_oracle(w, ids)
    out = _layer(w)(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert_close_bf16(out[torch.tensor(rows, device=gpu)], want, name)


def test_attention_forward_cfg2_full_size(gpu):
    """The serving batch at its full size: all 256 sequences (4.8 GB of K/V) against the
    oracle, through Attention.forward (store of the 256 new tokens, then paged decode)."""
    print("[forward] cfg2 full size, 256 sequences", flush=True)
    w = make_workload("cfg2", gpu)
    rows, want = subset_oracle(w, list(range(len(w.q_lens))))
    assert rows == list(range(256))
    out = _layer(w)(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert_close_bf16(out, want, "cfg2 full")


def test_dense_flat_mode_matches_oracle(gpu):
    # all-fresh prompts: block_tables None, cu_seqlens_k == cu_seqlens_q (model_runner.py:211)
    g = torch.Generator(device=gpu).manual_seed(11)
    lens = [1, 2, 63, 64, 65, 130, 257]
    n = sum(lens)
    q = torch.randn(n, 16, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    qkv = torch.randn(n, 4096, generator=g, device=gpu, dtype=torch.bfloat16)
    k = qkv[:, 2048:3072].reshape(n, 8, 128).clone()
    v = qkv[:, 3072:].view(n, 8, 128)
    cu = torch.tensor([0] + np.cumsum(lens).tolist(), dtype=torch.int32, device=gpu)
    out = pagedkv.varlen_attention(q, k, v, cu, cu, max(lens), max(lens), None, True, None)
    want = oracle.varlen_attention(q.cpu(), k.cpu(), v.cpu(), cu.cpu(), cu.cpu(), None, True, None)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, "flat")


@pytest.mark.parametrize("hq,hkv", [(8, 8), (16, 4), (16, 2), (32, 8)])
def test_gqa_groups(gpu, hq, hkv):
    g = torch.Generator(device=gpu).manual_seed(hq * 100 + hkv)
    seqs = [(1, 700), (1, 33), (129, 300), (40, 40)]           # (Lq, Lk)
    nb_per = [math.ceil(lk / BLOCK_SIZE) for _, lk in seqs]
    nb = sum(nb_per) + 1
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(3)).tolist()
    bt = torch.full((len(seqs), max(nb_per)), -1, dtype=torch.int32)
    pos = 0
    for i, c in enumerate(nb_per):
        bt[i, :c] = torch.tensor(perm[pos:pos + c])
        pos += c
    nq = sum(s[0] for s in seqs)
    q = torch.randn(nq, hq, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    kc = torch.randn(nb, BLOCK_SIZE, hkv, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    vc = torch.randn(nb, BLOCK_SIZE, hkv, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum([s[0] for s in seqs]).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum([s[1] for s in seqs]).tolist(), dtype=torch.int32)
    out = pagedkv.varlen_attention(q, kc, vc, cu_q.to(gpu), cu_k.to(gpu), 129, 700, None, True,
                                   bt.to(gpu))
    want = oracle.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q, cu_k, None, True, bt)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, f"gqa {hq}/{hkv}")


def test_noncausal_paged(gpu):
    case = build_case("noncausal2")
    out = _run_case(case, gpu)
    ref = np.load(GOLDEN / "kat_noncausal2.npz")["out"]
    torch.cuda.synchronize()
    assert_close_bf16(out, torch.from_numpy(ref), "noncausal")


# ------------------------------------------------------------- invariants ---

def test_block_relabelling_bit_identical(gpu):
    w = make_workload("cfg3", gpu, num_seqs=12)
    out1 = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k,
                                    w.max_seqlen_q, w.max_seqlen_k, None, True, w.block_tables)
    nb = w.k_cache.shape[0]
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(9)).to(gpu)
    kc2 = torch.empty_like(w.k_cache)
    vc2 = torch.empty_like(w.v_cache)
    kc2[perm] = w.k_cache
    vc2[perm] = w.v_cache
    bt2 = torch.where(w.block_tables >= 0, perm[w.block_tables.clamp(min=0).long()].int(),
                      w.block_tables)
    out2 = pagedkv.varlen_attention(w.q, kc2, vc2, w.cu_seqlens_q, w.cu_seqlens_k,
                                    w.max_seqlen_q, w.max_seqlen_k, None, True, bt2.contiguous())
    torch.cuda.synchronize()
    assert bits_equal(out1, out2)


def test_shared_prefix_equals_private_copies(gpu):
    w = make_workload("cfg4", gpu, num_seqs=16)
    out_shared = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q,
                                          w.cu_seqlens_k, 1, w.max_seqlen_k, None, True,
                                          w.block_tables)
    shared = w.meta["shared_blocks"]
    nb = w.k_cache.shape[0]
    s = len(w.q_lens)
    extra = torch.tensor(shared, device=gpu).repeat(s)              # a private prefix per sequence
    kc = torch.cat([w.k_cache, w.k_cache[extra]])
    vc = torch.cat([w.v_cache, w.v_cache[extra]])
    bt = w.block_tables.clone()
    bt[:, :len(shared)] = (nb + torch.arange(s * len(shared), device=gpu).view(s, -1)).int()
    out_priv = pagedkv.varlen_attention(w.q, kc, vc, w.cu_seqlens_q, w.cu_seqlens_k, 1,
                                        w.max_seqlen_k, None, True, bt)
    torch.cuda.synchronize()
    assert bits_equal(out_shared, out_priv)


def test_decode_row_matches_prefill_last_row(gpu):
    w = make_workload("cfg3", gpu, num_seqs=8)
    n_dec = 8
    full = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k,
                                    w.max_seqlen_q, w.max_seqlen_k, None, True, w.block_tables)
    cu_q = w.cu_seqlens_q.cpu()
    b = n_dec                                               # first prefill sequence
    last = int(cu_q[b + 1]) - 1
    q1 = w.q[last:last + 1]
    cu1 = torch.tensor([0, 1], dtype=torch.int32, device=gpu)
    cuk = torch.tensor([0, w.k_lens[b]], dtype=torch.int32, device=gpu)
    one = pagedkv.varlen_attention(q1, w.k_cache, w.v_cache, cu1, cuk, 1, w.k_lens[b], None, True,
                                   w.block_tables[b:b + 1].contiguous())
    torch.cuda.synchronize()
    assert_close_bf16(one[0], full[last].float(), "decode vs prefill row")


def test_deterministic(gpu):
    w = make_workload("cfg3", gpu, num_seqs=12)
    a = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k,
                                 w.max_seqlen_q, w.max_seqlen_k, None, True, w.block_tables)
    b = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k,
                                 w.max_seqlen_q, w.max_seqlen_k, None, True, w.block_tables)
    torch.cuda.synchronize()
    assert bits_equal(a, b)


# ------------------------------------------------------------ graph replay ---

def test_graph_capture_padded_decode_replay(gpu):
    """Decode captured once at a padded batch size and replayed with reference-style
    padding (slot -1, cu_seqlens zero tail, block tables -1; model_runner.py:245-259)."""
    bs, graph_bs, max_seq_len = 20, 32, 8192
    w = make_workload("cfg2", gpu, num_seqs=bs)
    width = max_seq_len // BLOCK_SIZE
    layer = _layer(w)
    st = dict(
        q=torch.zeros(graph_bs, 16, 128, device=gpu, dtype=torch.bfloat16),
        k=torch.zeros(graph_bs, 8, 128, device=gpu, dtype=torch.bfloat16),
        qkv=torch.zeros(graph_bs, 4096, device=gpu, dtype=torch.bfloat16),
        slot=torch.zeros(graph_bs, dtype=torch.int32, device=gpu),
        cu_q=torch.zeros(graph_bs + 1, dtype=torch.int32, device=gpu),
        cu_k=torch.zeros(graph_bs + 1, dtype=torch.int32, device=gpu),
        bt=torch.zeros(graph_bs, width, dtype=torch.int32, device=gpu),
    )
    v_static = st["qkv"][:, 3072:].view(graph_bs, 8, 128)
    ctx = pagedkv.Context(cu_seqlens_q=st["cu_q"], cu_seqlens_k=st["cu_k"], max_seqlen_q=1,
                          max_seqlen_k=max_seq_len, slot_mapping=st["slot"], block_tables=st["bt"])

    def fill(qnew):
        st["q"][:bs] = qnew
        st["k"][:bs] = w.k
        st["qkv"][:bs] = w.meta["qkv"]
        st["slot"].fill_(-1)
        st["slot"][:bs] = w.slot_mapping
        st["cu_q"].zero_()
        st["cu_q"][:bs + 1] = w.cu_seqlens_q
        st["cu_k"].zero_()
        st["cu_k"][:bs + 1] = w.cu_seqlens_k
        st["bt"].fill_(-1)
        st["bt"][:bs, :w.block_tables.shape[1]] = w.block_tables

    pagedkv.reserve_workspace(graph_bs, 16, 128, 1, max_seq_len, gpu)
    fill(w.q)
    layer(st["q"], st["k"], v_static, ctx)                       # warmup outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = layer(st["q"], st["k"], v_static, ctx)
    torch.cuda.synchronize()
    cache_before = (w.k_cache.clone(), w.v_cache.clone())
    g = torch.Generator(device=gpu).manual_seed(5)
    for rep in range(3):
        qnew = w.q if rep == 0 else torch.randn(w.q.shape, generator=g, device=gpu, dtype=torch.bfloat16)
        fill(qnew)
        graph.replay()
        torch.cuda.synchronize()
        eager = layer(qnew, w.k, w.v, w.ctx)
        torch.cuda.synchronize()
        assert_close_bf16(out_static[:bs], eager.float(), f"replay {rep}")
    # padded rows store nothing: only the real slots (rewritten with identical bits) changed
    assert bits_equal(w.k_cache, cache_before[0]) and bits_equal(w.v_cache, cache_before[1])


def test_graph_capture_mixed_call_replay(gpu):
    """A call with both decode and prefill sequences (decode split + combine, prefill plan +
    persistent prefill + merge) captured into a graph: every replay is bit-identical to the
    eager call, with eager calls of the same shape in between."""
    w = make_workload("cfg3", gpu, num_seqs=24)
    assert 1 in w.q_lens and max(w.q_lens) > 1
    ws = torch.empty(pagedkv.workspace_bytes(len(w.q_lens), 16, 128, w.max_seqlen_q, w.max_seqlen_k),
                     dtype=torch.uint8, device=gpu)

    def run():
        return pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k,
                                        w.max_seqlen_q, w.max_seqlen_k, None, True, w.block_tables,
                                        workspace=ws)
    want = run()
    torch.cuda.synchronize()
    print("[graph] cfg3 mixed call, 24 sequences", flush=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = run()
    torch.cuda.synchronize()
    for rep in range(3):
        out_static.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert bits_equal(out_static, want), f"replay {rep}"
        again = run()
        torch.cuda.synchronize()
        assert bits_equal(again, want), f"eager call after replay {rep}"


def test_workspace_reuse_across_batch_shapes(gpu):
    """One shared workspace serves calls of different shapes in any order: each result is
    bit-identical to the same call on a fresh (zero-filled) workspace."""
    shapes = [("cfg4", 16), ("cfg2", 24), ("cfg3", None), ("cfg1_decode", None), ("cfg2", 8), ("cfg3", 40)]
    wls = [make_workload(n, gpu, num_seqs=s) for n, s in shapes]

    def need(w):
        return pagedkv.workspace_bytes(len(w.q_lens), 16, 128, w.max_seqlen_q, w.max_seqlen_k)

    def run(w, ws):
        return pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k,
                                        w.max_seqlen_q, w.max_seqlen_k, None, True, w.block_tables,
                                        workspace=ws)
    fresh = [run(w, torch.zeros(max(1, need(w)), dtype=torch.uint8, device=gpu)) for w in wls]
    shared = torch.empty(max(need(w) for w in wls), dtype=torch.uint8, device=gpu)
    for rep in range(2):
        for w, want in zip(wls, fresh):
            got = run(w, shared)
            torch.cuda.synchronize()
            assert bits_equal(got, want), f"{w.name} rep {rep}"


def test_calls_on_two_streams_may_overlap(gpu):
    """Without an explicit workspace every call takes its own scratch, so a decode batch and
    a prefill batch may run concurrently on two streams (one shared per-device buffer would
    let the decode partials overwrite the prefill work list)."""
    w = make_workload("cfg3", gpu, num_seqs=24)
    dec = [i for i, lq in enumerate(w.q_lens) if lq == 1]
    pre = [i for i, lq in enumerate(w.q_lens) if lq > 1]

    def sub(ids):
        cu_q = w.cu_seqlens_q.cpu().tolist()
        rows = [r for i in ids for r in range(cu_q[i], cu_q[i + 1])]
        q = w.q[torch.tensor(rows, device=gpu)]
        lq = [w.q_lens[i] for i in ids]
        lk = [w.k_lens[i] for i in ids]
        cq = torch.tensor([0] + np.cumsum(lq).tolist(), dtype=torch.int32, device=gpu)
        ck = torch.tensor([0] + np.cumsum(lk).tolist(), dtype=torch.int32, device=gpu)
        bt = w.block_tables[torch.tensor(ids, device=gpu)].contiguous()
        return lambda: pagedkv.varlen_attention(q, w.k_cache, w.v_cache, cq, ck, max(lq), max(lk), None, True, bt)
    fd, fp = sub(dec), sub(pre)
    want_d, want_p = fd(), fp()
    torch.cuda.synchronize()
    print("[two streams] cfg3 decode + prefill sub-batches", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    for _ in range(3):
        got_d = fd()
        with torch.cuda.stream(side):
            got_p = fp()
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        assert bits_equal(got_d, want_d) and bits_equal(got_p, want_p)


def test_long_context_small_batch(gpu):
    """40k-key sequences: decode splits grow to fit the combine table, and the prefill
    kernel reads block ids past the 64 it keeps in a register."""
    g = torch.Generator(device=gpu).manual_seed(21)
    seqs = [(1, 40000), (70, 33000), (1, 300)]
    nb_per = [math.ceil(lk / BLOCK_SIZE) for _, lk in seqs]
    nb = sum(nb_per)
    perm = torch.randperm(nb, generator=torch.Generator().manual_seed(4)).tolist()
    bt = torch.full((len(seqs), max(nb_per)), -1, dtype=torch.int32)
    pos = 0
    for i, c in enumerate(nb_per):
        bt[i, :c] = torch.tensor(perm[pos:pos + c])
        pos += c
    nq = sum(s[0] for s in seqs)
    q = torch.randn(nq, 16, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    kc = torch.randn(nb, BLOCK_SIZE, 8, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    vc = torch.randn(nb, BLOCK_SIZE, 8, 128, generator=g, device=gpu, dtype=torch.bfloat16)
    cu_q = torch.tensor([0] + np.cumsum([s[0] for s in seqs]).tolist(), dtype=torch.int32)
    cu_k = torch.tensor([0] + np.cumsum([s[1] for s in seqs]).tolist(), dtype=torch.int32)
    out = pagedkv.varlen_attention(q, kc, vc, cu_q.to(gpu), cu_k.to(gpu), 70, 40000, None, True,
                                   bt.to(gpu))
    want = oracle.varlen_attention(q.cpu(), kc.cpu(), vc.cpu(), cu_q, cu_k, None, True, bt)
    torch.cuda.synchronize()
    assert_close_bf16(out, want, "long context")


@pytest.mark.parametrize("name,num_seqs", [("cfg2", 24), ("cfg3", 12), ("cfg4", 16)])
def test_cache_hint_never_changes_results(gpu, name, num_seqs):
    """pk_varlen_attention_ex's cached_prefix_keys only picks the load flavour (normal or
    streaming) per decode split: outputs are bit-identical to the default entry point for
    every value, including streaming all keys (0) and none (-1)."""
    w = make_workload(name, gpu, num_seqs=num_seqs)
    pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, w.slot_mapping)
    args = (w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k, w.max_seqlen_q,
            w.max_seqlen_k, 128 ** -0.5, True, w.block_tables)
    print(f"[cache_hint] {name} seqs={num_seqs}", flush=True)
    ref = pagedkv.varlen_attention(*args)
    outs = [pagedkv.varlen_attention(*args, cached_prefix_keys=c) for c in (0, -1, 256, 2048, 1 << 20)]
    torch.cuda.synchronize()
    for o in outs:
        assert bits_equal(o, ref)


def test_attention_forward_accepts_reference_context(gpu):
    """The layer takes the reference's eight-field Context (no cache hint) and gives the
    same output as with this package's Context when that states no shared prefix either
    (a stated prefix selects the shared-prefix decode path, tested on its own)."""
    import dataclasses

    @dataclasses.dataclass
    class RefContext:  # the fields of src/utils/context.py:5-14
        is_prefill: bool = False
        cu_seqlens_q: torch.Tensor | None = None
        cu_seqlens_k: torch.Tensor | None = None
        max_seqlen_q: int = 0
        max_seqlen_k: int = 0
        slot_mapping: torch.Tensor | None = None
        context_lens: torch.Tensor | None = None
        block_tables: torch.Tensor | None = None

    w = make_workload("cfg4", gpu)
    c = dataclasses.replace(w.ctx, cached_prefix_keys=None)
    ref_ctx = RefContext(c.is_prefill, c.cu_seqlens_q, c.cu_seqlens_k, c.max_seqlen_q, c.max_seqlen_k,
                         c.slot_mapping, c.context_lens, c.block_tables)
    kc0, vc0 = w.k_cache.clone(), w.v_cache.clone()
    out_a = _layer(w)(w.q, w.k, w.v, ref_ctx)
    w.k_cache.copy_(kc0)
    w.v_cache.copy_(vc0)
    out_b = _layer(w)(w.q, w.k, w.v, c)
    torch.cuda.synchronize()
    assert torch.equal(out_a.view(torch.int16), out_b.view(torch.int16))
