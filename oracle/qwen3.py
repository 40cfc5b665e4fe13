"""CPU restatement of the Qwen3 forward pass -- the oracle for the end-to-end engine.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.

Follows src/models/qwen3.py:74-195 with the reference's rounding points: bf16 activations
between operations, fp32 inside the norms (layernorm.py:11-28), RoPE (pos_embedding.py:
30-48) and SiLU * mul (activation.py:6-10), linear layers as bf16 = round(fp32 x . W^T)
(linear.py:135-136), and attention as fp32 softmax(scale q k^T) v over the causal prefix of
one sequence with GQA head h -> h // (Hq / Hkv), rounded to bf16 (the flash-attn call at
attention.py:95-104). Logits are returned in fp32.

It runs one sequence at a time over its whole token list, with no KV cache, so it checks
the engine's paged cache, chunking and graph replay end to end: the logits at position p
predict the token at p + 1.

Pinning (tests/test_oracle_qwen3.py): an fp64 restatement of the decoder written from the
reference's modules (explicit per-token, per-head attention loops) on a small geometry; a
closed form (zero o_proj and down_proj weights reduce the model to the final norm of the
embedding rows times the tied embedding); causality (the logits of position p do not
depend on later tokens); a one-token sequence, whose attention output is its own V row;
and planted mistakes (GQA map h % Hkv, no causal mask, no softmax scale, RoPE positions
shifted by one, residual not carried) that each check must catch.
"""
from __future__ import annotations

import torch

from . import model_ops, producer


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (x.float() @ w.float().T).to(torch.bfloat16)


def kv_head_of(num_heads: int, num_kv_heads: int) -> torch.Tensor:
    """GQA: query head h reads kv head h // (num_heads / num_kv_heads)."""
    return torch.arange(num_heads) // (num_heads // num_kv_heads)


def positions_of(n: int) -> torch.Tensor:
    """Positions of a sequence run from its start: 0 .. n - 1."""
    return torch.arange(n)


def causal_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """q, k, v (n, H, D) with k, v already expanded to the query heads: fp32
    softmax(scale q k^T) v over keys t <= i for row i, rounded to bf16."""
    n = q.shape[0]
    mask = torch.ones(n, n, dtype=torch.bool).tril()
    s = torch.einsum("ihd,jhd->hij", q.float(), k.float()) * scale
    s = s.masked_fill(~mask, float("-inf"))
    return torch.einsum("hij,jhd->ihd", torch.softmax(s, dim=-1), v.float()).to(torch.bfloat16)


def forward_logits(weights, cfg, token_ids: list[int]) -> torch.Tensor:
    """(len(token_ids), vocab) fp32 logits; `weights` holds CPU copies of the parameters
    with the attribute layout of pagedkv.qwen3.Qwen3Weights."""
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps
    n = len(token_ids)
    ids = torch.tensor(token_ids, dtype=torch.long)
    pos = positions_of(n)
    cos_sin = producer.rope_cos_sin(int(pos.max()) + 1, D, cfg.rope_theta)
    h = weights.embed[ids]
    residual = None
    kv_of = kv_head_of(Hq, Hkv)
    for L in weights.layers:
        if residual is None:
            x, residual = producer.rms_norm(h, L["input_norm"], eps), h
        else:
            x, residual = model_ops.rms_norm_residual(h, residual, L["input_norm"], eps)
        qkv = _linear(x, L["qkv"])
        q, k = producer.qk_norm_rope_store(qkv, pos, cos_sin, Hq, Hkv, D, L["q_norm"], L["k_norm"], eps)
        v = qkv[:, (Hq + Hkv) * D:].reshape(n, Hkv, D)
        o = causal_attention(q, k[:, kv_of], v[:, kv_of], D ** -0.5)
        h = _linear(o.reshape(n, Hq * D), L["o"])
        x, residual = model_ops.rms_norm_residual(h, residual, L["post_norm"], eps)
        h = _linear(model_ops.silu_and_mul(_linear(x, L["gate_up"])), L["down"])
    x, _ = model_ops.rms_norm_residual(h, residual, weights.final_norm, eps)
    return x.float() @ weights.embed.float().T
