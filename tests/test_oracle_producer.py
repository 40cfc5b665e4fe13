"""Pins the producer oracle (q/k RMSNorm + RoPE + K/V store) on the CPU.

Each check is chosen so that a plausible mistake fails it: fp64 loops with the
reference's rounding points, closed forms (identity at position 0, a constant row
normalises to its sign, a one-hot row rotates onto cos/sin of the textbook frequency
at columns j and j + D/2), the per-pair norm invariant, the store's closed form, and
planted mistakes patched into the oracle.
"""
import math

import numpy as np
import pytest
import torch

from oracle import producer as P

D = 128
BASE = 1000000.0
EPS = 1e-6


def ulp_diff(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """Distance in bf16 units in the last place (monotone integer view of the bits)."""
    def key(t):
        i = t.contiguous().view(torch.int16).to(torch.int32)
        return torch.where(i < 0, -(i & 0x7FFF), i)
    return (key(a) - key(b)).abs()


def make(n=7, hq=4, hkv=2, seed=0, max_pos=4096):
    g = torch.Generator().manual_seed(seed)
    qkv = (torch.randn(n, (hq + 2 * hkv) * D, generator=g) * 2).to(torch.bfloat16)
    pos = torch.randint(0, max_pos, (n,), generator=g)
    qw = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    kw = (1 + 0.2 * torch.randn(D, generator=g)).to(torch.bfloat16)
    return qkv, pos, qw, kw


def inv_freq32(j, base):
    """1 / base^(2j / D) with the fp32 roundings of pos_embedding.py:9."""
    e = np.float32(2 * j) / np.float32(D)
    return np.float32(1.0) / np.float32(np.float64(base) ** np.float64(e))


def brute(qkv, pos, qw, kw, hq, hkv, base=BASE, eps=EPS):
    """fp64 loops; bf16 rounding after the norm and after RoPE (the reference's points)."""
    n = qkv.shape[0]
    x = qkv.double()
    outs = []
    for first, heads, w in ((0, hq, qw), (hq, hkv, kw)):
        o = torch.empty(n, heads, D, dtype=torch.bfloat16)
        for i in range(n):
            p = int(pos[i])
            for h in range(heads):
                row = [float(x[i, (first + h) * D + d]) for d in range(D)]
                ms = sum(v * v for v in row) / D
                r = 1.0 / math.sqrt(ms + eps)
                nrm = torch.tensor([float(w[d]) * row[d] * r for d in range(D)],
                                   dtype=torch.float64).to(torch.bfloat16).double()
                rot = [0.0] * D
                for j in range(D // 2):
                    # the angle as the table holds it: fp32 frequency, fp32 product
                    # (pos_embedding.py:9-12); cos and sin of it in fp64
                    th = float(np.float32(p) * inv_freq32(j, base))
                    c, s = math.cos(th), math.sin(th)
                    rot[j] = nrm[j] * c - nrm[j + D // 2] * s
                    rot[j + D // 2] = nrm[j] * s + nrm[j + D // 2] * c
                o[i, h] = torch.tensor(rot, dtype=torch.float64).to(torch.bfloat16)
        outs.append(o)
    return outs


def run(qkv, pos, qw, kw, hq, hkv, max_pos=4096):
    cs = P.rope_cos_sin(max_pos, D, BASE)
    return P.qk_norm_rope_store(qkv, pos, cs, hq, hkv, D, qw, kw, EPS)


def test_oracle_matches_fp64_loops():
    qkv, pos, qw, kw = make()
    q, k = run(qkv, pos, qw, kw, 4, 2)
    bq, bk = brute(qkv, pos, qw, kw, 4, 2)
    for got, want in ((q, bq), (k, bk)):
        d = ulp_diff(got, want)
        assert int(d.max()) <= 1
        assert float((d == 0).float().mean()) >= 0.99


def test_position_zero_is_identity():
    qkv, _, qw, kw = make(n=5)
    pos = torch.zeros(5, dtype=torch.long)
    q, k = run(qkv, pos, qw, kw, 4, 2)
    nq = P.rms_norm(qkv[:, :4 * D].reshape(5, 4, D), qw, EPS)
    nk = P.rms_norm(qkv[:, 4 * D:6 * D].reshape(5, 2, D), kw, EPS)
    assert torch.equal(q.view(torch.int16), nq.view(torch.int16))
    assert torch.equal(k.view(torch.int16), nk.view(torch.int16))


def test_constant_row_normalises_to_sign():
    x = torch.full((3, 2, D), -2.5).to(torch.bfloat16)
    x[1] = 0.75
    out = P.rms_norm(x, torch.ones(D, dtype=torch.bfloat16), EPS)
    assert torch.equal(out.float(), torch.sign(x.float()))


def test_eps_inside_the_root():
    # constant row c with c^2 = eps: out = c / sqrt(c^2 + eps) = 1 / sqrt(2)
    c = float(torch.tensor(1e-3).to(torch.bfloat16))
    x = torch.full((1, 1, D), c).to(torch.bfloat16)
    out = P.rms_norm(x, torch.ones(D, dtype=torch.bfloat16), c * c)
    want = torch.tensor(1 / math.sqrt(2)).to(torch.bfloat16)
    assert int(ulp_diff(out, want.expand_as(out)).max()) <= 1


def test_one_hot_rotates_onto_textbook_frequency():
    # x = e_j: the norm gives sqrt(D) e_j; RoPE at position p puts sqrt(D) cos(p f_j) at
    # column j and sqrt(D) sin(p f_j) at column j + D/2, f_j = base^(-2j/D), zeros elsewhere
    # (pins rotate-half pairing, the sign of the sine and the frequency formula).
    cs = P.rope_cos_sin(2048, D, BASE)
    w = torch.ones(D, dtype=torch.bfloat16)
    for j, p in ((0, 1), (3, 700), (17, 1500), (40, 2047), (63, 999)):
        x = torch.zeros(1, 1, D, dtype=torch.bfloat16)
        x[0, 0, j] = 1.0
        out = P.rope(P.rms_norm(x, w, 0.0), torch.tensor([p]), cs).float()[0, 0]
        a = float(torch.tensor(math.sqrt(D)).to(torch.bfloat16))
        f = BASE ** (-2 * j / D)
        want = torch.zeros(D)
        want[j] = a * math.cos(p * f)
        want[j + D // 2] = a * math.sin(p * f)
        assert torch.allclose(out, want, atol=0.06, rtol=0.01), (j, p)
        others = [d for d in range(D) if d not in (j, j + D // 2)]
        assert torch.count_nonzero(out[others]) == 0


def test_table_closed_form():
    cs = P.rope_cos_sin(1000, D, BASE)
    p = torch.arange(1000, dtype=torch.float64).unsqueeze(1)
    f = torch.tensor([BASE ** (-2 * j / D) for j in range(D // 2)], dtype=torch.float64)
    assert torch.allclose(cs[:, :D // 2].double(), torch.cos(p * f), atol=1e-4)
    assert torch.allclose(cs[:, D // 2:].double(), torch.sin(p * f), atol=1e-4)


def test_rotation_preserves_pair_norms():
    qkv, pos, qw, kw = make(n=9, seed=3)
    cs = P.rope_cos_sin(4096, D, BASE)
    x = P.rms_norm(qkv[:, :4 * D].reshape(9, 4, D), qw, EPS)
    y = P.rope(x, pos, cs)
    r_in = x.float()[..., :D // 2] ** 2 + x.float()[..., D // 2:] ** 2
    r_out = y.float()[..., :D // 2] ** 2 + y.float()[..., D // 2:] ** 2
    assert torch.allclose(r_in, r_out, rtol=2e-2, atol=1e-2)


def test_store_closed_form():
    qkv, pos, qw, kw = make(n=6, seed=5)
    kc = torch.full((4, 8, 2, D), 7.0).to(torch.bfloat16)
    vc = kc.clone()
    slots = torch.tensor([3, -1, 17, 30, -1, 0], dtype=torch.int32)
    cs = P.rope_cos_sin(4096, D, BASE)
    q, k = P.qk_norm_rope_store(qkv, pos, cs, 4, 2, D, qw, kw, EPS, kc, vc, slots)
    v = qkv[:, 6 * D:].reshape(6, 2, D)
    flat_k, flat_v = kc.view(-1, 2, D), vc.view(-1, 2, D)
    for i, s in enumerate(slots.tolist()):
        if s != -1:
            assert torch.equal(flat_k[s].view(torch.int16), k[i].view(torch.int16))
            assert torch.equal(flat_v[s].view(torch.int16), v[i].view(torch.int16))
    untouched = [r for r in range(32) if r not in (3, 17, 30, 0)]
    assert torch.all(flat_k[untouched].float() == 7.0) and torch.all(flat_v[untouched].float() == 7.0)


# ---- planted mistakes: each must make a check above fail -------------------------------

def _interleaved(x, positions, cos_sin):
    cs = cos_sin[positions].unsqueeze(1)
    cos, sin = cs.chunk(2, dim=-1)
    t1, t2 = x.float()[..., 0::2], x.float()[..., 1::2]
    out = torch.stack((t1 * cos - t2 * sin, t1 * sin + t2 * cos), dim=-1).flatten(-2)
    return out.to(x.dtype)


def _sign_flipped(x, positions, cos_sin):
    cs = cos_sin[positions].unsqueeze(1)
    cos, sin = cs.chunk(2, dim=-1)
    t1, t2 = torch.chunk(x.float(), 2, dim=-1)
    return torch.cat((t1 * cos + t2 * sin, -t1 * sin + t2 * cos), dim=-1).to(x.dtype)


def _eps_outside(x, weight, eps):
    fx = x.float()
    return (weight * (fx * (fx.square().mean(-1, keepdim=True).rsqrt() + eps))).to(x.dtype)


def _no_weight(x, weight, eps):
    fx = x.float()
    return (fx * (fx.square().mean(-1, keepdim=True) + eps).rsqrt()).to(x.dtype)


def _unrounded_chain(qkv, positions, cos_sin, num_heads, num_kv_heads, head_dim, qw, kw, eps,
                     *args):
    def f(x, w):
        fx = x.float()
        n = w.float() * (fx * (fx.square().mean(-1, keepdim=True) + eps).rsqrt())
        cs = cos_sin[positions].unsqueeze(1)
        cos, sin = cs.chunk(2, dim=-1)
        t1, t2 = torch.chunk(n, 2, dim=-1)
        return torch.cat((t1 * cos - t2 * sin, t1 * sin + t2 * cos), dim=-1).to(x.dtype)
    q_size, kv_size = num_heads * head_dim, num_kv_heads * head_dim
    q, k, _ = qkv.split([q_size, kv_size, kv_size], dim=-1)
    return (f(q.reshape(-1, num_heads, head_dim), qw), f(k.reshape(-1, num_kv_heads, head_dim), kw))


@pytest.mark.parametrize("attr,fake,check", [
    ("rope", _interleaved, "test_one_hot_rotates_onto_textbook_frequency"),
    ("rope", _sign_flipped, "test_one_hot_rotates_onto_textbook_frequency"),
    ("rms_norm", _eps_outside, "test_eps_inside_the_root"),
    ("rms_norm", _no_weight, "test_oracle_matches_fp64_loops"),
    ("qk_norm_rope_store", _unrounded_chain, "test_oracle_matches_fp64_loops"),
])
def test_planted_mistake_is_caught(monkeypatch, attr, fake, check):
    monkeypatch.setattr(P, attr, fake)
    with pytest.raises(AssertionError):
        globals()[check]()
