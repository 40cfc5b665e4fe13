"""CPU pinning of oracle/qwen3.py (the model oracle of the end-to-end engine tests).

Checks, each chosen so a plausible mistake in the oracle's composition fails one:
  * an fp64 restatement written from the reference's modules (tests/golden/qwen3_bruteforce.py,
    explicit per-token, per-head attention loops) on a small geometry with GQA group 2;
  * a closed form: with o_proj and down_proj weights zero, every layer adds nothing to the
    residual stream, so the logits are final_norm(embed[ids]) . embed^T (tied head);
  * causality: the logits of position p do not change when later tokens change;
  * the attention step on its own: one token attends only to itself (output = its V row),
    and with zero keys row i is the mean of V rows 0 .. i;
  * planted mistakes (GQA map h % Hkv, no causal mask, no softmax scale, residual not carried)
    patched into the oracle must each fail a check.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import oracle.model_ops as M
import oracle.qwen3 as Q
from golden.qwen3_bruteforce import bf16 as bf16_np
from golden.qwen3_bruteforce import forward_logits as brute_logits

CFG = SimpleNamespace(num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6,
                      rope_theta=10000.0, hidden_size=48, intermediate_size=40, vocab_size=96)
TOKENS = [5, 17, 80, 3, 44, 17, 91, 0]
# |oracle - fp64 restatement| on these logits: both round at the same bf16 points, so they
# differ only where fp32 and fp64 sums land on different sides of a bf16 rounding boundary
# (measured max 2.4e-6 here; the logits span about +-33). Every planted mistake below moves
# some logit by more than 10.
TOL = 1e-3


def _weights(seed: int, layers: int = 2, zero_out: bool = False):
    g = torch.Generator().manual_seed(seed)
    H, D = CFG.hidden_size, CFG.head_dim
    hq, hkv, inter, vocab = CFG.num_attention_heads, CFG.num_key_value_heads, CFG.intermediate_size, CFG.vocab_size

    def rnd(*shape, fan_in=None):
        s = 1.0 if fan_in is None else fan_in ** -0.5
        return (torch.randn(*shape, generator=g) * s).to(torch.bfloat16)

    def norm_w(n):
        return (1.0 + 0.2 * torch.randn(n, generator=g)).to(torch.bfloat16)

    Ls = []
    for _ in range(layers):
        L = dict(input_norm=norm_w(H), post_norm=norm_w(H), q_norm=norm_w(D), k_norm=norm_w(D),
                 qkv=rnd((hq + 2 * hkv) * D, H, fan_in=H), o=rnd(H, hq * D, fan_in=hq * D),
                 gate_up=rnd(2 * inter, H, fan_in=H), down=rnd(H, inter, fan_in=inter))
        if zero_out:
            L["o"].zero_()
            L["down"].zero_()
        Ls.append(L)
    return SimpleNamespace(embed=rnd(vocab, H), final_norm=norm_w(H), layers=Ls)


def _np(w):
    f = lambda t: t.double().numpy()  # noqa: E731
    return SimpleNamespace(embed=f(w.embed), final_norm=f(w.final_norm),
                           layers=[{k: f(v) for k, v in L.items()} for L in w.layers])


def check_bruteforce():
    w = _weights(1)
    got = Q.forward_logits(w, CFG, TOKENS).double().numpy()
    want = brute_logits(_np(w), CFG, TOKENS)
    err = np.abs(got - want).max()
    assert err <= TOL, f"oracle vs fp64 restatement: max |diff| {err:.3e}"


def check_zero_o_down_closed_form():
    w = _weights(2, layers=3, zero_out=True)
    got = Q.forward_logits(w, CFG, TOKENS).double().numpy()
    e = w.embed.double().numpy()
    x = e[TOKENS]
    inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + CFG.rms_norm_eps)
    want = bf16_np(w.final_norm.double().numpy() * x * inv) @ e.T
    err = np.abs(got - want).max()
    assert err <= 1e-2, f"zero o/down closed form: max |diff| {err:.3e}"


def check_causal():
    w = _weights(3)
    full = Q.forward_logits(w, CFG, TOKENS)
    changed = Q.forward_logits(w, CFG, TOKENS[:4] + [t ^ 1 for t in TOKENS[4:]])
    assert torch.equal(full[:4], changed[:4]) or (full[:4] - changed[:4]).abs().max() <= 1e-4, \
        "logits of positions 0-3 depend on tokens 4-7"
    assert (full[4:] - changed[4:]).abs().max() > 1e-2      # and the later rows do change


def check_attention_step():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 4, 16, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 4, 16, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 4, 16, generator=g).to(torch.bfloat16)
    assert torch.equal(Q.causal_attention(q, k, v, 0.25), v), "one token must attend to its own V row"
    n = 6
    v = torch.randn(n, 4, 16, generator=g).to(torch.bfloat16)
    o = Q.causal_attention(torch.randn(n, 4, 16, generator=g).to(torch.bfloat16), torch.zeros(n, 4, 16), v, 0.25)
    mean = v.float().cumsum(0) / torch.arange(1, n + 1).view(n, 1, 1)
    assert (o.float() - mean).abs().max() <= 1e-2, "zero keys: row i must be the mean of V rows 0 .. i"


CHECKS = [check_bruteforce, check_zero_o_down_closed_form, check_causal, check_attention_step]


@pytest.mark.parametrize("check", CHECKS, ids=lambda c: c.__name__)
def test_model_oracle(check):
    check()


def _modulo_gqa(num_heads, num_kv_heads):
    return torch.arange(num_heads) % num_kv_heads


def _no_mask(q, k, v, scale):
    s = torch.einsum("ihd,jhd->hij", q.float(), k.float()) * scale
    return torch.einsum("hij,jhd->ihd", torch.softmax(s, dim=-1), v.float()).to(torch.bfloat16)


def _no_scale(q, k, v, scale):
    return _REAL_ATTENTION(q, k, v, 1.0)


def _residual_dropped(x, residual, weight, eps):
    return _REAL_NORM(x, torch.zeros_like(residual), weight, eps)


_REAL_ATTENTION = Q.causal_attention
_REAL_NORM = M.rms_norm_residual


@pytest.mark.parametrize("target,attr,bad,caught_by", [
    (Q, "kv_head_of", _modulo_gqa, [check_bruteforce]),
    (Q, "causal_attention", _no_mask, [check_bruteforce, check_causal]),
    (Q, "causal_attention", _no_scale, [check_bruteforce]),
    (M, "rms_norm_residual", _residual_dropped, [check_bruteforce, check_zero_o_down_closed_form]),
], ids=["gqa_modulo", "no_causal_mask", "no_scale", "residual_dropped"])
def test_planted_mistakes_are_caught(monkeypatch, target, attr, bad, caught_by):
    monkeypatch.setattr(target, attr, bad)
    for check in caught_by:
        with pytest.raises(AssertionError):
            check()
