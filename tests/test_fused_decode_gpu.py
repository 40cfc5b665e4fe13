"""GPU parity of the fused decode step (pk_qkv_decode_attention, through the C-ABI) against
its unfused form, pk_qk_norm_rope_store followed by pk_varlen_attention_ex over the block
tables: the attention output and both caches must be bit-identical, for GQA groups 1, 2, 4,
sequences of one to several splits (the last split stores the token's K/V row and reads it
back), and graph-style padding rows (zero-length sequences, slot -1) that must leave the
caches untouched. The unfused path is itself pinned against the oracle by
test_producer_gpu.py and test_kernels_gpu.py.
"""
import math

import pytest
import torch

import pagedkv
from pagedkv import workloads as W

pytestmark = pytest.mark.gpu

D = 128
BS = 256
EPS = 1e-6
MAX_POS = 40960


def _batch(lens, hq, hkv, seed, dev, pad=0):
    g = torch.Generator().manual_seed(seed)
    S = len(lens)
    nb = sum(math.ceil(lk / BS) for lk in lens) + 2
    tables = W._pop_tables(lens, torch.randperm(nb, generator=g).tolist())
    width = max(len(t) for t in tables)
    bt = torch.full((S + pad, width), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    kc = torch.randn(nb, BS, hkv, D, generator=g).to(torch.bfloat16)
    vc = torch.randn(nb, BS, hkv, D, generator=g).to(torch.bfloat16)
    qkv = (torch.randn(S + pad, (hq + 2 * hkv) * D, generator=g) * 3).to(torch.bfloat16)
    pos = torch.tensor([lk - 1 for lk in lens] + [0] * pad, dtype=torch.int64)
    slot = torch.tensor([tables[i][(lk - 1) // BS] * BS + (lk - 1) % BS for i, lk in enumerate(lens)] +
                        [-1] * pad, dtype=torch.int32)
    # graph padding as the reference runner writes it: cumulative lengths, then a zero tail
    cu_q = torch.tensor(list(range(S + 1)) + [0] * pad, dtype=torch.int32)
    cu_k = torch.tensor([0] + list(torch.tensor(lens).cumsum(0).tolist()) + [0] * pad, dtype=torch.int32)
    qw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    to = lambda t: t.to(dev)  # noqa: E731
    return dict(qkv=to(qkv), pos=to(pos), slot=to(slot), cu_q=to(cu_q), cu_k=to(cu_k), bt=to(bt), kc=to(kc),
                vc=to(vc), qw=to(qw), kw=to(kw), maxk=max(lens), S=S)


def _both(b, hq, hkv, cs, hint=0):
    scale = D ** -0.5
    kca, vca = b["kc"].clone(), b["vc"].clone()
    q, _ = pagedkv.qk_norm_rope_store(b["qkv"], b["pos"], cs, hq, hkv, D, b["qw"], b["kw"], EPS, kca, vca,
                                      b["slot"])
    out_a = pagedkv.varlen_attention(q, kca, vca, b["cu_q"], b["cu_k"], 1, b["maxk"], scale, True, b["bt"],
                                     cached_prefix_keys=hint)
    kcb, vcb = b["kc"].clone(), b["vc"].clone()
    out_b = pagedkv.qkv_decode_attention(b["qkv"], b["pos"], cs, hq, hkv, D, b["qw"], b["kw"], EPS, kcb, vcb,
                                         b["slot"], b["cu_q"], b["cu_k"], b["maxk"], scale, b["bt"],
                                         cached_prefix_keys=hint)
    torch.cuda.synchronize()
    return (out_a, kca, vca), (out_b, kcb, vcb)


def _assert_same(a, b, S):
    out_a, kca, vca = a
    out_b, kcb, vcb = b
    assert torch.equal(out_a[:S].view(torch.int16), out_b[:S].view(torch.int16)), "attention output differs"
    assert torch.equal(kca.view(torch.int16), kcb.view(torch.int16)), "K cache differs"
    assert torch.equal(vca.view(torch.int16), vcb.view(torch.int16)), "V cache differs"


# (8, 4), (4, 2), (2, 1): one tensor-parallel rank's share at tp 2, 4, 8 (qwen3.py:30-36)
@pytest.mark.parametrize("hq,hkv", [(16, 8), (8, 8), (16, 4), (16, 2), (8, 4), (4, 2), (2, 1)])
@pytest.mark.parametrize("lens,pad", [([1, 5, 255, 256, 257, 3000], 0), ([700, 12, 4096, 1], 3)])
def test_fused_decode_bit_identical_to_producer_then_attention(gpu, hq, hkv, lens, pad):
    cs = pagedkv.rope_cos_sin(MAX_POS, D, 1000000.0, gpu)
    b = _batch(lens, hq, hkv, seed=len(lens) + hq + pad, dev=gpu, pad=pad)
    a, f = _both(b, hq, hkv, cs)
    _assert_same(a, f, b["S"])


def test_fused_decode_serving_batch_and_cache_hints(gpu):
    """128 sequences of 100-2048 keys (a serving decode step), every cache hint."""
    g = torch.Generator().manual_seed(11)
    lens = W._uniform(g, 100, 2048, 128)
    cs = pagedkv.rope_cos_sin(MAX_POS, D, 1000000.0, gpu)
    b = _batch(lens, 16, 8, seed=12, dev=gpu)
    for hint in (0, -1, 1024):
        a, f = _both(b, 16, 8, cs, hint=hint)
        _assert_same(a, f, b["S"])


def test_fused_decode_in_graph_replays(gpu):
    """Captured once, replayed on new qkv rows: every replay equals the eager unfused step."""
    cs = pagedkv.rope_cos_sin(MAX_POS, D, 1000000.0, gpu)
    b = _batch([40, 600, 2100, 9, 1300], 16, 8, seed=21, dev=gpu, pad=3)
    S = b["S"]
    pagedkv.reserve_workspace(S + 3, 16, 128, 1, b["maxk"], gpu)
    kcg, vcg = b["kc"].clone(), b["vc"].clone()
    qkv = b["qkv"].clone()
    out = torch.empty(S + 3, 16, D, dtype=torch.bfloat16, device=gpu)

    def step():
        pagedkv.qkv_decode_attention(qkv, b["pos"], cs, 16, 8, D, b["qw"], b["kw"], EPS, kcg, vcg, b["slot"],
                                     b["cu_q"], b["cu_k"], b["maxk"], D ** -0.5, b["bt"], out=out,
                                     cached_prefix_keys=0)
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    g = torch.Generator().manual_seed(5)
    for r in range(3):
        qkv.copy_((torch.randn(qkv.shape, generator=g) * 3).to(torch.bfloat16).to(gpu))
        graph.replay()
        torch.cuda.synchronize()
        b2 = dict(b, qkv=qkv.clone(), kc=kcg.clone(), vc=vcg.clone())
        # the replay already stored this step's rows: the unfused step on the same inputs
        # stores the same rows again and must produce the same output
        a, _ = _both(b2, 16, 8, cs)
        assert torch.equal(a[0][:S].view(torch.int16), out[:S].view(torch.int16)), f"replay {r}"
        assert torch.equal(a[1].view(torch.int16), kcg.view(torch.int16)), f"replay {r}: K cache"


@pytest.mark.parametrize("hq,hkv", [(16, 8), (16, 4), (8, 8), (16, 2)])
def test_store_decode_bit_identical_to_store_then_attention(gpu, hq, hkv):
    """pk_store_decode_attention (Attention.forward on a decode step) against
    pk_store_kvcache + pk_varlen_attention_ex: output and caches bit-identical, with graph
    padding rows and a strided value view (as qwen3.py passes v)."""
    b = _batch([1, 5, 255, 256, 257, 3000, 700], hq, hkv, seed=31 + hq, dev=gpu, pad=2)
    S = b["S"]
    g = torch.Generator().manual_seed(3)
    n = S + 2
    q = (torch.randn(n, hq, D, generator=g)).to(torch.bfloat16).to(gpu)
    kv = (torch.randn(n, 2 * hkv * D + 64, generator=g)).to(torch.bfloat16).to(gpu)
    key = kv[:, :hkv * D].view(n, hkv, D)
    value = kv[:, hkv * D:2 * hkv * D].view(n, hkv, D)          # row stride 2 hkv D + 64
    scale = D ** -0.5
    kca, vca = b["kc"].clone(), b["vc"].clone()
    pagedkv.store_kvcache(key, value, kca, vca, b["slot"])
    out_a = pagedkv.varlen_attention(q, kca, vca, b["cu_q"], b["cu_k"], 1, b["maxk"], scale, True, b["bt"],
                                     cached_prefix_keys=0)
    kcb, vcb = b["kc"].clone(), b["vc"].clone()
    layer = pagedkv.Attention(D, hq, hkv, scale)
    layer.k_cache, layer.v_cache = kcb, vcb
    ctx = pagedkv.Context(False, b["cu_q"], b["cu_k"], 1, b["maxk"], b["slot"], None, b["bt"], 0)
    out_b = layer(q, key, value, ctx)
    torch.cuda.synchronize()
    _assert_same((out_a, kca, vca), (out_b, kcb, vcb), S)


class _Spy:
    """Counts calls of the one-launch store + decode that Attention.forward makes."""

    def __init__(self, monkeypatch):
        import pagedkv.attention as A

        self.calls = 0
        real = A.store_decode_attention

        def spy(*a, **k):
            self.calls += 1
            return real(*a, **k)
        monkeypatch.setattr(A, "store_decode_attention", spy)


def _two_launches(q, key, value, kc, vc, ctx, scale):
    """store_kvcache + varlen_attention as Attention.forward calls them (a stated shared
    prefix also selects the shared-prefix decode path)."""
    hint = ctx.cached_prefix_keys
    pagedkv.store_kvcache(key, value, kc, vc, ctx.slot_mapping)
    return pagedkv.varlen_attention(q, kc, vc, ctx.cu_seqlens_q, ctx.cu_seqlens_k, 1, ctx.max_seqlen_k, scale, True,
                                    ctx.block_tables, cached_prefix_keys=hint,
                                    shared_prefix_keys=hint if hint is not None and hint > 0 else None)


def test_shared_token_block_takes_two_launches(gpu, monkeypatch):
    """A decode row whose slot lies in a block another sequence reads (the recomputed last
    token of a fully prefix-cached prompt, scheduler.py:77-80) must not use the one-launch
    path: its store would race with the other sequence's reads of that block. The Context
    then states the shared prefix (cached_prefix_keys > 0) and forward takes store_kvcache +
    varlen_attention, bit-identical to calling the two; with cached_prefix_keys == 0 over
    private blocks it takes the one launch."""
    spy = _Spy(monkeypatch)
    g = torch.Generator().manual_seed(41)
    hq, hkv, scale = 16, 8, D ** -0.5
    nb = 8
    # sequence 0: a 256-token prompt, fully cached, recomputes its last token into block 5;
    # sequence 1 (700 keys) and 2 (300 keys) share block 5 as their first block
    tables = [[5], [5, 2, 7], [5, 0]]
    lens = [256, 700, 300]
    bt = torch.full((3, 3), -1, dtype=torch.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = torch.tensor(t, dtype=torch.int32)
    slot = torch.tensor([t[(lk - 1) // BS] * BS + (lk - 1) % BS for t, lk in zip(tables, lens)], dtype=torch.int32)
    kc = torch.randn(nb, BS, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    vc = torch.randn(nb, BS, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    q = torch.randn(3, hq, D, generator=g).to(torch.bfloat16).to(gpu)
    key = torch.randn(3, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    value = torch.randn(3, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    hint = pagedkv.shared_prefix_keys(bt, BS)
    assert hint == BS
    ctx = pagedkv.Context(False, torch.arange(4, dtype=torch.int32, device=gpu),
                          torch.tensor([0, 256, 956, 1256], dtype=torch.int32, device=gpu), 1, 700,
                          slot.to(gpu), None, bt.to(gpu), hint)
    layer = pagedkv.Attention(D, hq, hkv, scale)
    layer.k_cache, layer.v_cache = kc.clone(), vc.clone()
    out = layer(q, key, value, ctx)
    kc2, vc2 = kc.clone(), vc.clone()
    want = _two_launches(q, key, value, kc2, vc2, ctx, scale)
    torch.cuda.synchronize()
    assert spy.calls == 0, "a batch with a shared block took the one-launch path"
    _assert_same((want, kc2, vc2), (out, layer.k_cache, layer.v_cache), 3)
    # the same batch over private blocks, stated unshared: the one launch, same results
    priv = torch.tensor([[5, -1, -1], [1, 2, 7], [3, 0, -1]], dtype=torch.int32)
    kcp, vcp = kc.clone(), vc.clone()
    kcp[1], vcp[1] = kc[5], vc[5]
    kcp[3], vcp[3] = kc[5], vc[5]
    ctx_p = pagedkv.Context(False, ctx.cu_seqlens_q, ctx.cu_seqlens_k, 1, 700, ctx.slot_mapping, None,
                            priv.to(gpu), pagedkv.shared_prefix_keys(priv, BS))
    assert ctx_p.cached_prefix_keys == 0
    layer.k_cache, layer.v_cache = kcp.clone(), vcp.clone()
    out_p = layer(q, key, value, ctx_p)
    kcp2, vcp2 = kcp.clone(), vcp.clone()
    want_p = _two_launches(q, key, value, kcp2, vcp2, ctx_p, scale)
    torch.cuda.synchronize()
    assert spy.calls == 1
    _assert_same((want_p, kcp2, vcp2), (out_p, layer.k_cache, layer.v_cache), 3)


@pytest.mark.parametrize("hint", [0, None])
def test_forward_graph_under_reference_capture_protocol(gpu, hint):
    """Attention.forward captured the way the reference's runner captures its decode graphs
    (model_runner.py:268-315): static inputs all zero during the warmup run and the capture
    (zero cu_seqlens, slot 0, zero block tables), then every replay after filling the
    reference's padding (slot -1, zero cu_seqlens tail, -1 block tables, :244-259). Each
    replay must equal eager store_kvcache + varlen_attention bit for bit, output and caches.
    hint 0 states unshared blocks (the one-launch path is captured), None is the reference's
    Context (two launches)."""
    hq, hkv, scale = 16, 8, D ** -0.5
    bs, graph_bs, max_k = 5, 8, 4096
    b = _batch([40, 600, 2100, 9, 1300], hq, hkv, seed=51, dev=gpu)
    width = max_k // BS
    st = dict(q=torch.zeros(graph_bs, hq, D, dtype=torch.bfloat16, device=gpu),
              k=torch.zeros(graph_bs, hkv, D, dtype=torch.bfloat16, device=gpu),
              v=torch.zeros(graph_bs, hkv, D, dtype=torch.bfloat16, device=gpu),
              slot=torch.zeros(graph_bs, dtype=torch.int32, device=gpu),
              cu_q=torch.zeros(graph_bs + 1, dtype=torch.int32, device=gpu),
              cu_k=torch.zeros(graph_bs + 1, dtype=torch.int32, device=gpu),
              bt=torch.zeros(graph_bs, width, dtype=torch.int32, device=gpu))
    ctx = pagedkv.Context(False, st["cu_q"], st["cu_k"], 1, max_k, st["slot"], None, st["bt"], hint)
    layer = pagedkv.Attention(D, hq, hkv, scale)
    layer.k_cache, layer.v_cache = b["kc"].clone(), b["vc"].clone()
    pagedkv.reserve_workspace(graph_bs, hq, D, 1, max_k, gpu)
    layer(st["q"], st["k"], st["v"], ctx)                    # the reference's warmup run
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = layer(st["q"], st["k"], st["v"], ctx)
    torch.cuda.synchronize()
    g = torch.Generator().manual_seed(52)
    for rep in range(3):
        q = torch.randn(bs, hq, D, generator=g).to(torch.bfloat16).to(gpu)
        key = torch.randn(bs, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
        value = torch.randn(bs, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
        kc_ref, vc_ref = layer.k_cache.clone(), layer.v_cache.clone()
        st["q"][:bs], st["k"][:bs], st["v"][:bs] = q, key, value
        st["slot"].fill_(-1)
        st["slot"][:bs] = b["slot"]
        st["cu_q"].zero_()
        st["cu_q"][:bs + 1] = b["cu_q"]
        st["cu_k"].zero_()
        st["cu_k"][:bs + 1] = b["cu_k"]
        st["bt"].fill_(-1)
        st["bt"][:bs, :b["bt"].shape[1]] = b["bt"]
        graph.replay()
        torch.cuda.synchronize()
        # eager store_kvcache + varlen_attention on the same padded inputs (same launch bounds)
        ref_ctx = pagedkv.Context(False, st["cu_q"].clone(), st["cu_k"].clone(), 1, max_k, st["slot"].clone(), None,
                                  st["bt"].clone(), hint)
        want = _two_launches(st["q"].clone(), st["k"].clone(), st["v"].clone(), kc_ref, vc_ref, ref_ctx, scale)
        torch.cuda.synchronize()
        _assert_same((want, kc_ref, vc_ref), (out_static, layer.k_cache, layer.v_cache), bs)
