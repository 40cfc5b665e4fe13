"""Qwen3 decoder (the reference's model, src/models/qwen3.py) assembled from the gfx950
kernels of this package; the dense projections are hipBLASLt GEMMs through torch.

Per layer (qwen3.py:155-169):
    x, residual = add_rmsnorm(h, input_layernorm, residual)        layernorm.py:18-28
    qkv = x W_qkv^T                                                 linear.py:190-228
    q, k = qk_norm_rope_store(qkv, ...)  (norms, RoPE, K/V store)   qwen3.py:80-88
    o = varlen_attention(q, k | k_cache, v | v_cache, ...)          attention.py:89-105
    h = o W_o^T                                                     qwen3.py:90
    x, residual = add_rmsnorm(h, post_attention_layernorm, residual)
    h = silu_and_mul(x W_gate_up^T) W_down^T                        qwen3.py:119-123
and the final norm (qwen3.py:194). Weights are random (the serving benchmark runs a
random-init model of the Qwen3-0.6B geometry); the LM head is tied to the embedding
(qwen3.py:215-216).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import ops
from .context import Context


@dataclass(frozen=True)
class Qwen3Config:
    """Qwen3-0.6B geometry (the HF config the reference loads, model_config.py:3-4)."""
    vocab_size: int = 151936
    hidden_size: int = 1024
    num_hidden_layers: int = 28
    num_attention_heads: int = 16
    num_key_value_heads: int = 8
    head_dim: int = 128
    intermediate_size: int = 3072
    rms_norm_eps: float = 1e-6
    rope_theta: float = 1000000.0
    max_position_embeddings: int = 40960


class Qwen3Weights:
    """All parameters, bf16 on one device, random-normal (std 0.02) with unit norms."""

    def __init__(self, cfg: Qwen3Config, device: torch.device, seed: int = 5, std: float = 0.02):
        g = torch.Generator(device=device).manual_seed(seed)
        bf = dict(dtype=torch.bfloat16, device=device)

        def randn(*shape):
            return (torch.randn(*shape, generator=g, device=device) * std).to(torch.bfloat16)

        H, D = cfg.hidden_size, cfg.head_dim
        qkv_out = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * D
        self.embed = randn(cfg.vocab_size, H)                    # tied with the LM head
        self.layers = []
        for _ in range(cfg.num_hidden_layers):
            self.layers.append(dict(
                input_norm=torch.ones(H, **bf), post_norm=torch.ones(H, **bf),
                q_norm=torch.ones(D, **bf), k_norm=torch.ones(D, **bf),
                qkv=randn(qkv_out, H), o=randn(H, cfg.num_attention_heads * D),
                gate_up=randn(2 * cfg.intermediate_size, H), down=randn(H, cfg.intermediate_size)))
        self.final_norm = torch.ones(H, **bf)


class Qwen3Model:
    """Forward over one step's tokens; K/V caches are (L, NB, BS, Hkv, D) per operand."""

    def __init__(self, cfg: Qwen3Config, weights: Qwen3Weights, k_caches: torch.Tensor | None,
                 v_caches: torch.Tensor | None, max_position: int):
        """k_caches / v_caches None: no cache yet (the warmup pass before the cache is sized,
        as the reference's Attention skips the store while k_cache is empty,
        attention.py:87-88); bind_caches attaches them later."""
        self.cfg = cfg
        self.w = weights
        self.bind_caches(k_caches, v_caches)
        dev = weights.embed.device
        self.cos_sin = ops.rope_cos_sin(max_position, cfg.head_dim, cfg.rope_theta, dev)
        self.scale = cfg.head_dim ** -0.5

    def bind_caches(self, k_caches: torch.Tensor | None, v_caches: torch.Tensor | None) -> None:
        """Per-layer K/V cache views, (L, NB, BS, Hkv, D) per operand (model_runner.py:161-165)."""
        if (k_caches is None) != (v_caches is None):
            raise ValueError("bind both caches or neither")
        self.k_caches = k_caches
        self.v_caches = v_caches

    def linear_workspace_bytes(self, max_rows: int) -> int:
        """Scratch the decode-step linear layers need for any batch of up to `max_rows`
        tokens (the launch shape, and so the scratch, depends on the row count)."""
        cfg = self.cfg
        H, qd, inter = cfg.hidden_size, cfg.num_attention_heads * cfg.head_dim, cfg.intermediate_size
        qkv_out = (cfg.num_attention_heads + 2 * cfg.num_key_value_heads) * cfg.head_dim
        need = 0
        for rows in range(1, min(max_rows, ops.LINEAR_MAX_ROWS) + 1):
            need = max(need, ops.linear_workspace_bytes(rows, qkv_out, H, ops.LINEAR_STORE),
                       ops.linear_workspace_bytes(rows, H, qd, ops.LINEAR_ADD_RMSNORM),
                       ops.linear_workspace_bytes(rows, inter, H, ops.LINEAR_SILU_MUL),
                       ops.linear_workspace_bytes(rows, H, inter, ops.LINEAR_ADD_RMSNORM))
        return need

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, ctx: Context) -> torch.Tensor:
        """Steps of at most 128 tokens (decode batches) run every projection on the library's
        decode-step linear kernels, each fused with the op after it: qkv_proj; o_proj + the
        post-attention RMSNorm; gate_up_proj + SiluAndMul; down_proj + the next layer's input
        RMSNorm (the final norm after the last layer). Larger steps use F.linear (a library
        GEMM) and the separate norm / activation kernels. Rounding points are the same."""
        cfg, W = self.cfg, self.w
        Hq, Hkv, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        eps = cfg.rms_norm_eps
        flat = ctx.block_tables is None
        small = input_ids.shape[0] <= ops.LINEAR_MAX_ROWS
        # a decode step: every sequence has one new token (cu_seqlens_q = arange), read
        # through block tables; the producer then runs inside the attention launch
        decode = not flat and ctx.max_seqlen_q == 1 and input_ids.shape[0] == ctx.cu_seqlens_q.numel() - 1
        h = F.embedding(input_ids, W.embed)
        residual = None
        nl = len(W.layers)
        for li, L in enumerate(W.layers):
            if residual is None:
                x = ops.add_rmsnorm(h, L["input_norm"], eps)
                residual = h
            elif not small:
                x, residual = ops.add_rmsnorm(h, L["input_norm"], eps, residual=residual)
            qkv = ops.linear(x, L["qkv"]) if small else F.linear(x, L["qkv"])
            kc, vc = (None, None) if self.k_caches is None else (self.k_caches[li], self.v_caches[li])
            if decode:
                # one launch: q/k norm + RoPE, the K/V store and paged decode attention; no
                # block is shared (no prefix cache), so every decode read streams
                o = ops.qkv_decode_attention(qkv, positions, self.cos_sin, Hq, Hkv, D, L["q_norm"], L["k_norm"],
                                             eps, kc, vc, ctx.slot_mapping, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                             ctx.max_seqlen_k, self.scale, ctx.block_tables, cached_prefix_keys=0)
            else:
                q, k = ops.qk_norm_rope_store(qkv, positions, self.cos_sin, Hq, Hkv, D, L["q_norm"],
                                              L["k_norm"], eps, kc, vc, ctx.slot_mapping, return_k=flat)
                if flat:
                    v = qkv[:, (Hq + Hkv) * D:].view(-1, Hkv, D)
                    o = ops.varlen_attention(q, k, v, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                             ctx.max_seqlen_q, ctx.max_seqlen_k, self.scale, True)
                else:
                    o = ops.varlen_attention(q, kc, vc, ctx.cu_seqlens_q, ctx.cu_seqlens_k,
                                             ctx.max_seqlen_q, ctx.max_seqlen_k, self.scale, True,
                                             ctx.block_tables, cached_prefix_keys=0)
            if small:
                x, residual = ops.linear_add_rmsnorm(o.view(-1, Hq * D), L["o"], residual,
                                                     L["post_norm"], eps, residual_out=residual)
                nxt = W.layers[li + 1]["input_norm"] if li + 1 < nl else W.final_norm
                x, residual = ops.linear_add_rmsnorm(ops.linear_silu_mul(x, L["gate_up"]), L["down"],
                                                     residual, nxt, eps, residual_out=residual)
            else:
                h = F.linear(o.view(-1, Hq * D), L["o"])
                x, residual = ops.add_rmsnorm(h, L["post_norm"], eps, residual=residual)
                h = F.linear(ops.silu_and_mul(F.linear(x, L["gate_up"])), L["down"])
        if not small:
            x, _ = ops.add_rmsnorm(h, W.final_norm, eps, residual=residual)
        return x

    def greedy(self, hidden: torch.Tensor, ctx: Context, out: torch.Tensor | None = None) -> torch.Tensor:
        """Next tokens: the last row of each sequence for prefill batches (llm_head.py:61-63)."""
        cu = ctx.cu_seqlens_q if ctx.is_prefill else None
        return ops.lm_head_greedy(hidden, self.w.embed, cu, out=out)
