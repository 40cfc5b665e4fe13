"""fp64 restatement of the Qwen3 decoder forward pass, written from the reference's modules
(not from oracle/qwen3.py) to pin that oracle's composition. Test infrastructure only.

Follows, per token list of one sequence:
  * Qwen3Model.forward (src/models/qwen3.py:180-195): embedding rows, the decoder layers
    with a residual stream that starts as the embedding, the final RMSNorm;
  * Qwen3DecoderLayer.forward (qwen3.py:155-169): input RMSNorm (plain on the first layer,
    residual-add form after), attention, post-attention RMSNorm with residual, MLP;
  * Qwen3Attention.forward (qwen3.py:74-91): fused qkv projection split [q | k | v], per-head
    q_norm / k_norm, rotate-half RoPE at positions 0 .. n - 1, causal attention with GQA
    head h -> h // (Hq / Hkv) and scale D^-0.5, o_proj;
  * RMSNorm (src/layers/layernorm.py:11-28), RoPE (src/layers/pos_embedding.py:6-48),
    SiluAndMul (src/layers/activation.py:6-10), tied LM head (qwen3.py:215-216).
Arithmetic is fp64 with explicit per-(token, head, key) attention loops; values are rounded
to bf16 where the reference's tensors are bf16 (after every linear layer, norm, RoPE,
attention output and SiLU * mul). Logits stay unrounded.
"""
from __future__ import annotations

import math

import numpy as np


def bf16(x) -> np.ndarray:
    """Round to the nearest bf16 value (ties to even), returned as float64."""
    f = np.asarray(x, dtype=np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return (r & 0xFFFFFFFF).astype(np.uint32).view(np.float32).astype(np.float64)


def _rms_norm(rows: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        x = rows[r]
        inv = 1.0 / math.sqrt(float(np.mean(x * x)) + eps)
        out[r] = weight * (x * inv)
    return bf16(out)


def _rope(x: np.ndarray, pos: int, theta: float) -> np.ndarray:
    d = x.shape[-1]
    half = d // 2
    out = np.empty_like(x)
    for j in range(half):
        ang = pos * (1.0 / theta ** (2 * j / d))
        c, s = math.cos(ang), math.sin(ang)
        x1, x2 = x[..., j], x[..., j + half]
        out[..., j] = x1 * c - x2 * s
        out[..., j + half] = x1 * s + x2 * c
    return bf16(out)


def forward_logits(weights, cfg, token_ids) -> np.ndarray:
    """(n, vocab) fp64 logits. `weights`: embed, final_norm and layers[i][name] as float64
    arrays holding bf16 values (names as pagedkv.qwen3.Qwen3Weights)."""
    hq, hkv, d = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    grp = hq // hkv
    eps, theta = cfg.rms_norm_eps, cfg.rope_theta
    n = len(token_ids)
    emb = weights.embed
    h = emb[np.asarray(token_ids)]
    residual = None
    for L in weights.layers:
        if residual is None:
            x, residual = _rms_norm(h, L["input_norm"], eps), h
        else:
            s = h + residual
            x, residual = _rms_norm(s, L["input_norm"], eps), bf16(s)
        qkv = bf16(x @ L["qkv"].T)
        q = qkv[:, :hq * d].reshape(n, hq, d)
        k = qkv[:, hq * d:(hq + hkv) * d].reshape(n, hkv, d)
        v = qkv[:, (hq + hkv) * d:].reshape(n, hkv, d)
        qr = np.empty_like(q)
        kr = np.empty_like(k)
        for i in range(n):
            qr[i] = _rope(_rms_norm(q[i], L["q_norm"], eps), i, theta)
            kr[i] = _rope(_rms_norm(k[i], L["k_norm"], eps), i, theta)
        o = np.zeros((n, hq, d))
        for i in range(n):
            for head in range(hq):
                g = head // grp
                scores = [float(np.dot(qr[i, head], kr[t, g])) * d ** -0.5 for t in range(i + 1)]
                mx = max(scores)
                p = [math.exp(sc - mx) for sc in scores]
                z = sum(p)
                for t in range(i + 1):
                    o[i, head] += (p[t] / z) * v[t, g]
        h = bf16(bf16(o).reshape(n, hq * d) @ L["o"].T)
        s = h + residual
        x, residual = _rms_norm(s, L["post_norm"], eps), bf16(s)
        gu = bf16(x @ L["gate_up"].T)
        inter = gu.shape[1] // 2
        gate, up = gu[:, :inter], gu[:, inter:]
        act = bf16(gate / (1.0 + np.exp(-gate)) * up)
        h = bf16(act @ L["down"].T)
    x = _rms_norm(h + residual, weights.final_norm, eps)
    return x @ emb.T
