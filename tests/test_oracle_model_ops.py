"""Pins the oracle of the serving loop's other kernels (oracle/model_ops.py) on the CPU."""
import math

import pytest
import torch

from oracle import model_ops as M
from test_oracle_producer import ulp_diff


def _rand(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def test_residual_cancelling_input_gives_zeros():
    x = _rand((4, 256), 0)
    out, res = M.rms_norm_residual(x, -x, torch.ones(256, dtype=torch.bfloat16), 1e-6)
    assert torch.all(out.float() == 0) and torch.all(res.float() == 0)


def test_constant_sum_normalises_to_sign():
    x = torch.full((3, 128), 1.5).to(torch.bfloat16)
    r = torch.full((3, 128), 0.5).to(torch.bfloat16)
    r[1] = -3.0
    out, res = M.rms_norm_residual(x, r, torch.ones(128, dtype=torch.bfloat16), 1e-6)
    assert torch.equal(out.float(), torch.sign(res.float()))
    assert torch.equal(res.float()[0], torch.full((128,), 2.0))


def _norm_loops(x, r, w, eps):
    out = torch.empty_like(x)
    for i in range(x.shape[0]):
        s = [float(x[i, j]) + float(r[i, j]) for j in range(x.shape[1])]
        rs = 1.0 / math.sqrt(sum(v * v for v in s) / len(s) + eps)
        out[i] = torch.tensor([float(w[j]) * s[j] * rs for j in range(len(s))],
                              dtype=torch.float64).to(torch.bfloat16)
    return out


def test_norm_matches_fp64_loops():
    x, r, w = _rand((6, 1024), 1), _rand((6, 1024), 2), _rand((1024,), 3, 0.2) + 1
    got, _ = M.rms_norm_residual(x, r, w.to(torch.bfloat16), 1e-6)
    d = ulp_diff(got, _norm_loops(x, r, w.to(torch.bfloat16), 1e-6))
    assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99


def test_silu_closed_forms():
    g = torch.tensor([0.0, 1.0, -2.0, 3.5, -8.0, 0.25]).to(torch.bfloat16)
    one = torch.ones_like(g)
    out = M.silu_and_mul(torch.cat([g, one]).unsqueeze(0))[0]
    want = torch.tensor([float(v) / (1 + math.exp(-float(v))) for v in g], dtype=torch.float64)
    assert out[0] == 0
    assert int(ulp_diff(out, want.to(torch.bfloat16)).max()) == 0


def test_silu_matches_fp64_single_rounding():
    x = _rand((8, 2 * 3072), 4, 2.0)
    got = M.silu_and_mul(x)
    g, u = x.double().chunk(2, -1)
    want = (g / (1 + torch.exp(-g)) * u).to(torch.bfloat16)
    d = ulp_diff(got, want)
    assert int(d.max()) <= 1 and float((d == 0).float().mean()) >= 0.99


def test_lm_head_one_hot_weights_and_ties():
    # weight row v = e_(v mod 8): logit v = x[v mod 8]; the max of x repeats every 8 ids,
    # so the first id holding it must win
    hidden, vocab = 128, 40
    w = torch.zeros(vocab, hidden)
    for v in range(vocab):
        w[v, v % 8] = 1.0
    x = torch.zeros(3, hidden)
    x[0, 5] = 2.0
    x[1, :8] = torch.tensor([1.0, 3.0, 3.0, 0.0, -1.0, 2.0, 0.5, 3.0])
    x[2, :8] = -1.0
    got = M.lm_head_greedy(x.to(torch.bfloat16), w.to(torch.bfloat16))
    assert got.tolist() == [5, 1, 0]


def test_lm_head_selects_last_token_of_each_sequence():
    hidden, vocab = 128, 16
    w = torch.eye(vocab, hidden).to(torch.bfloat16)
    x = torch.zeros(7, hidden)
    for row, tok in enumerate([3, 9, 1, 14, 2, 7, 11]):
        x[row, tok] = 1.0
    cu = torch.tensor([0, 3, 4, 7], dtype=torch.int32)      # sequences end at rows 2, 3, 6
    got = M.lm_head_greedy(x.to(torch.bfloat16), w, cu)
    assert got.tolist() == [1, 14, 11]


def _double_rounding_silu(x):
    g, u = x.float().chunk(2, -1)
    return ((g / (1.0 + torch.exp(-g))).to(x.dtype).float() * u).to(x.dtype)


def _no_residual(x, residual, weight, eps):
    s = x.float()
    var = s.square().mean(-1, keepdim=True) + eps
    return (weight.float() * (s * var.rsqrt())).to(x.dtype), s.to(x.dtype)


def _last_argmax(logits):
    m = logits.max(dim=-1, keepdim=True).values
    idx = torch.arange(logits.shape[-1]).expand_as(logits)
    return torch.where(logits == m, idx, torch.full_like(idx, -1)).max(dim=-1).values


def _no_selection(hidden, weight, cu_seqlens_q=None):
    logits = (hidden.double() @ weight.double().T).to(torch.bfloat16).float()
    return M.first_argmax(logits)[: (len(cu_seqlens_q) - 1 if cu_seqlens_q is not None else None)]


@pytest.mark.parametrize("attr,fake,check", [
    ("rms_norm_residual", _no_residual, test_residual_cancelling_input_gives_zeros),
    ("silu_and_mul", _double_rounding_silu, test_silu_matches_fp64_single_rounding),
    ("first_argmax", _last_argmax, test_lm_head_one_hot_weights_and_ties),
    ("lm_head_greedy", _no_selection, test_lm_head_selects_last_token_of_each_sequence),
])
def test_planted_mistake_is_caught(monkeypatch, attr, fake, check):
    monkeypatch.setattr(M, attr, fake)
    with pytest.raises(AssertionError):
        check()
