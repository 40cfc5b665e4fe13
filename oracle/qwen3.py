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
"""
from __future__ import annotations

import torch

from . import model_ops, producer


def _linear(x: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    return (x.float() @ w.float().T).to(torch.bfloat16)


def forward_logits(weights, cfg, token_ids: list[int]) -> torch.Tensor:
    """(len(token_ids), vocab) fp32 logits; `weights` holds CPU copies of the parameters
    with the attribute layout of pagedkv.qwen3.Qwen3Weights."""
    Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    eps = cfg.rms_norm_eps
    n = len(token_ids)
    ids = torch.tensor(token_ids, dtype=torch.long)
    pos = torch.arange(n)
    cos_sin = producer.rope_cos_sin(n, D, cfg.rope_theta)
    h = weights.embed[ids]
    residual = None
    mask = torch.ones(n, n, dtype=torch.bool).tril()
    for L in weights.layers:
        if residual is None:
            x, residual = producer.rms_norm(h, L["input_norm"], eps), h
        else:
            x, residual = model_ops.rms_norm_residual(h, residual, L["input_norm"], eps)
        qkv = _linear(x, L["qkv"])
        q, k = producer.qk_norm_rope_store(qkv, pos, cos_sin, Hq, Hkv, D, L["q_norm"], L["k_norm"], eps)
        v = qkv[:, (Hq + Hkv) * D:].reshape(n, Hkv, D)
        kv_of = torch.arange(Hq) // (Hq // Hkv)
        qf, kf, vf = q.float(), k.float()[:, kv_of], v.float()[:, kv_of]
        s = torch.einsum("ihd,jhd->hij", qf, kf) * (D ** -0.5)
        s = s.masked_fill(~mask, float("-inf"))
        o = torch.einsum("hij,jhd->ihd", torch.softmax(s, dim=-1), vf).to(torch.bfloat16)
        h = _linear(o.reshape(n, Hq * D), L["o"])
        x, residual = model_ops.rms_norm_residual(h, residual, L["post_norm"], eps)
        h = _linear(model_ops.silu_and_mul(_linear(x, L["gate_up"])), L["down"])
    x, _ = model_ops.rms_norm_residual(h, residual, weights.final_norm, eps)
    return x.float() @ weights.embed.float().T
