"""GPU parity of the fused producer (q/k RMSNorm + RoPE + K/V store) against the oracle.

Bars: q and k outputs within 1 bf16 ulp of the oracle element-wise and identical on at
least 99% of elements (the reference itself runs these ops under torch.compile, whose
FMA contraction and rsqrt are not pinned, so one ulp is the honest bound); cache rows
bit-identical to the kernel's own k output (K) and to the input row (V); slots -1 and
rows no token maps to keep their sentinel bits. Calls go through the C-ABI.
"""
import pytest
import torch

import pagedkv
from oracle import producer as P
from test_oracle_producer import ulp_diff

pytestmark = pytest.mark.gpu

D = 128
BASE = 1000000.0
EPS = 1e-6
MAX_POS = 40960          # Qwen3 max_position_embeddings
SENTINEL = 0x7BAD


def _inputs(n, hq, hkv, seed, dev, stride_pad=0):
    g = torch.Generator().manual_seed(seed)
    width = (hq + 2 * hkv) * D
    buf = (torch.randn(n, width + stride_pad, generator=g) * 3).to(torch.bfloat16)
    qkv = buf.to(dev)[:, :width]                       # row stride width + stride_pad
    pos = torch.randint(0, MAX_POS, (n,), generator=g)
    pos[: min(n, 3)] = torch.tensor([0, 1, MAX_POS - 1])[: min(n, 3)]
    qw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.3 * torch.randn(D, generator=g)).to(torch.bfloat16)
    return qkv, pos.to(dev), qw.to(dev), kw.to(dev)


def _caches(num_blocks, bs, hkv, dev):
    kc = torch.full((num_blocks, bs, hkv, D), SENTINEL, dtype=torch.int16).view(torch.bfloat16)
    return kc.to(dev), kc.clone().to(dev)


def _slots(n, num_slots, seed, minus_one_every=5):
    g = torch.Generator().manual_seed(seed + 100)
    s = torch.randperm(num_slots, generator=g)[:n].to(torch.int32)
    s[::minus_one_every] = -1
    return s


def _check_close(got, want, what):
    d = ulp_diff(got.cpu(), want.cpu())
    assert int(d.max()) <= 1, f"{what}: max ulp diff {int(d.max())}"
    frac = float((d == 0).float().mean())
    assert frac >= 0.99, f"{what}: only {frac:.4f} identical"


@pytest.mark.parametrize("n,hq,hkv", [(300, 16, 8), (64, 8, 4), (33, 32, 8), (5, 4, 2), (1, 16, 8)])
def test_producer_matches_oracle(gpu, n, hq, hkv):
    qkv, pos, qw, kw = _inputs(n, hq, hkv, seed=n + hq, dev=gpu)
    cs = pagedkv.rope_cos_sin(MAX_POS, D, BASE, gpu)
    kc, vc = _caches(8, 64, hkv, gpu)
    slots = _slots(n, 8 * 64, seed=n).to(gpu)
    kc_ref, vc_ref = kc.cpu().clone(), vc.cpu().clone()
    q, k = pagedkv.qk_norm_rope_store(qkv, pos, cs, hq, hkv, D, qw, kw, EPS, kc, vc, slots,
                                      return_k=True)
    torch.cuda.synchronize()
    rq, rk = P.qk_norm_rope_store(qkv.cpu(), pos, cs, hq, hkv, D, qw, kw, EPS, kc_ref, vc_ref,
                                  slots)
    _check_close(q, rq, "q")
    _check_close(k, rk, "k")
    # cache rows: exactly the kernel's k rows and the raw v rows; everything else untouched
    flat_k, flat_v = kc.cpu().view(-1, hkv, D), vc.cpu().view(-1, hkv, D)
    v_in = qkv.cpu()[:, (hq + hkv) * D:].reshape(n, hkv, D)
    s = slots.cpu().long()
    keep = s != -1
    assert torch.equal(flat_k[s[keep]].view(torch.int16), k.cpu()[keep].view(torch.int16))
    assert torch.equal(flat_v[s[keep]].view(torch.int16), v_in[keep].view(torch.int16))
    mask = torch.ones(flat_k.shape[0], dtype=torch.bool)
    mask[s[keep]] = False
    assert torch.all(flat_k[mask].view(torch.int16) == SENTINEL)
    assert torch.all(flat_v[mask].view(torch.int16) == SENTINEL)


def test_producer_without_norm_weights_is_rope_only(gpu):
    n, hq, hkv = 40, 16, 8
    qkv, pos, _, _ = _inputs(n, hq, hkv, seed=7, dev=gpu)
    cs = pagedkv.rope_cos_sin(MAX_POS, D, BASE, gpu)
    q, k = pagedkv.qk_norm_rope_store(qkv, pos, cs, hq, hkv, D, return_k=True)
    rq, rk = P.qk_norm_rope_store(qkv.cpu(), pos, cs, hq, hkv, D, None, None, EPS)
    _check_close(q, rq, "q")
    _check_close(k, rk, "k")


def test_producer_strided_qkv_and_no_cache(gpu):
    n, hq, hkv = 70, 16, 8
    qkv, pos, qw, kw = _inputs(n, hq, hkv, seed=9, dev=gpu, stride_pad=256)
    assert qkv.stride(0) == (hq + 2 * hkv) * D + 256
    cs = pagedkv.rope_cos_sin(MAX_POS, D, BASE, gpu)
    q, k = pagedkv.qk_norm_rope_store(qkv, pos, cs, hq, hkv, D, qw, kw, EPS, return_k=True)
    rq, rk = P.qk_norm_rope_store(qkv.cpu(), pos, cs, hq, hkv, D, qw, kw, EPS)
    _check_close(q, rq, "q")
    _check_close(k, rk, "k")


def test_producer_slot_bound_check_and_padding(gpu):
    n, hq, hkv = 16, 16, 8
    qkv, pos, qw, kw = _inputs(n, hq, hkv, seed=11, dev=gpu)
    cs = pagedkv.rope_cos_sin(MAX_POS, D, BASE, gpu)
    kc, vc = _caches(2, 64, hkv, gpu)
    slots = torch.arange(n, dtype=torch.int32)
    slots[3] = 128        # one past the last slot: dropped under the bound check
    slots[4] = 1 << 20    # far out of range: dropped
    slots[5] = -1         # graph padding: skipped
    q, k = pagedkv.qk_norm_rope_store(qkv, pos, cs, hq, hkv, D, qw, kw, EPS, kc, vc,
                                      slots.to(gpu), return_k=True, check_slots=True)
    torch.cuda.synchronize()
    flat_k = kc.cpu().view(-1, hkv, D)
    for i in range(n):
        row = flat_k[i].view(torch.int16)
        if i in (3, 4, 5):
            assert torch.all(row == SENTINEL), i
        else:
            assert torch.equal(row, k.cpu()[i].view(torch.int16)), i
    assert torch.all(flat_k[n:].view(torch.int16) == SENTINEL)


def test_producer_feeds_attention_like_the_unfused_path(gpu):
    # store through the fused producer, then decode; compare with the unfused sequence
    # (oracle norm + rope, pk store, same attention) -> identical cache bits and outputs
    n, hq, hkv = 8, 16, 8
    qkv, pos, qw, kw = _inputs(n, hq, hkv, seed=13, dev=gpu)
    pos = torch.arange(n, device=gpu) * 0 + 255   # every sequence appends position 255
    cs = pagedkv.rope_cos_sin(MAX_POS, D, BASE, gpu)
    kc, vc = _caches(n, 256, hkv, gpu)
    g = torch.Generator().manual_seed(5)
    kc[:, :255] = torch.randn(n, 255, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    vc[:, :255] = torch.randn(n, 255, hkv, D, generator=g).to(torch.bfloat16).to(gpu)
    kc2, vc2 = kc.clone(), vc.clone()
    slots = (torch.arange(n, dtype=torch.int32) * 256 + 255).to(gpu)
    q, _ = pagedkv.qk_norm_rope_store(qkv, pos, cs, hq, hkv, D, qw, kw, EPS, kc, vc, slots)
    rq, rk = P.qk_norm_rope_store(qkv.cpu(), pos, cs, hq, hkv, D, qw, kw, EPS)
    v_in = qkv[:, (hq + hkv) * D:].reshape(n, hkv, D)
    pagedkv.store_kvcache(rk.to(gpu), v_in, kc2, vc2, slots)
    cu_q = torch.arange(n + 1, dtype=torch.int32, device=gpu)
    cu_k = (torch.arange(n + 1, dtype=torch.int32) * 256).to(gpu)
    bt = torch.arange(n, dtype=torch.int32, device=gpu).unsqueeze(1)
    o1 = pagedkv.varlen_attention(q, kc, vc, cu_q, cu_k, 1, 256, None, True, bt)
    o2 = pagedkv.varlen_attention(rq.to(gpu), kc2, vc2, cu_q, cu_k, 1, 256, None, True, bt)
    torch.cuda.synchronize()
    assert torch.equal(vc.cpu().view(torch.int16), vc2.cpu().view(torch.int16))
    _check_close(kc.view(-1, hkv, D)[slots.long()], kc2.view(-1, hkv, D)[slots.long()], "cache k")
    assert (o1.float() - o2.float()).abs().max().item() <= 2e-2


def test_producer_empty_batch(gpu):
    cs = pagedkv.rope_cos_sin(16, D, BASE, gpu)
    qkv = torch.empty(0, 32 * D, dtype=torch.bfloat16, device=gpu)
    pos = torch.empty(0, dtype=torch.int64, device=gpu)
    q, k = pagedkv.qk_norm_rope_store(qkv, pos, cs, 16, 8, D, return_k=True)
    assert q.shape == (0, 16, D) and k.shape == (0, 8, D)
