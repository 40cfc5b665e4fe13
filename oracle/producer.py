"""CPU restatement of the producer of the attention inputs -- the oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/ and bench.py's CPU-baseline leg, never by
the product package.

What each function restates (paths relative to the reference repository):

* rms_norm      -- RMSNorm.normal_forward, src/layers/layernorm.py:11-16: upcast to fp32,
  var = mean(x^2) + eps, x * rsqrt(var), multiply by the (bf16) weight in fp32, round to
  the input dtype.
* rope_cos_sin  -- build_rope_cos_sin, src/layers/pos_embedding.py:6-18: inv_freq_j =
  1 / base^(2j / D), table row p = [cos(p inv_freq) | sin(p inv_freq)] in fp32.
* rope          -- RoPE.forward, src/layers/pos_embedding.py:30-48: rotate-half on the
  fp32 upcast, t1 = x[:D/2], t2 = x[D/2:], out = [t1 cos - t2 sin | t1 sin + t2 cos],
  rounded to the input dtype.
* qk_norm_rope_store -- the sequence of Qwen3Attention.forward, src/models/qwen3.py:80-88
  (split of the fused qkv row, q_norm, k_norm, rotary_emb) followed by the store inside
  Attention.forward (src/layers/attention.py:87-88, kernel :10-34): K (normed, rotated)
  and raw V rows into slot_mapping's slots, -1 skipped.

Rounding points are the reference's: bf16 after the norm, fp32 inside RoPE, bf16 after.
The reference runs these under torch.compile, whose fused code may contract products
into FMAs or use an approximate rsqrt; results can therefore differ from any
restatement by one bf16 ulp, which is the tolerance the kernel tests use.

Pinning (tests/test_oracle_producer.py): fp64 loops with the same rounding points,
closed forms (position 0 is the identity, a constant row normalises to its sign, a
one-hot row rotates onto (cos, sin) at columns j and j + D/2 with the textbook
frequency), the per-pair norm invariant, and planted mistakes (interleaved pairs,
flipped sine sign, eps outside the root, dropped weight, no rounding after the norm)
that each check must catch.
"""
from __future__ import annotations

import torch


def rms_norm(x: torch.Tensor, weight: torch.Tensor | None, eps: float) -> torch.Tensor:
    """layernorm.py:11-16 over the last dimension; weight None means no norm."""
    if weight is None:
        return x
    fx = x.float()
    var = fx.square().mean(-1, keepdim=True) + eps
    return (weight * (fx * var.rsqrt())).to(x.dtype)


def rope_cos_sin(max_position: int, head_dim: int, base: float) -> torch.Tensor:
    """pos_embedding.py:6-18 as a (max_position, head_dim) fp32 table."""
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2).float() / head_dim))
    pos = torch.arange(max_position, dtype=torch.float)
    freqs = torch.outer(pos, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1)


def rope(x: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor) -> torch.Tensor:
    """pos_embedding.py:37-46 on x (N, H, D) with positions (N,)."""
    cs = cos_sin[positions].unsqueeze(1)          # (N, 1, D)
    cos, sin = cs.chunk(2, dim=-1)
    t1, t2 = torch.chunk(x.float(), 2, dim=-1)
    return torch.cat((t1 * cos - t2 * sin, t1 * sin + t2 * cos), dim=-1).to(x.dtype)


def qk_norm_rope_store(qkv: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor,
                       num_heads: int, num_kv_heads: int, head_dim: int,
                       q_weight: torch.Tensor | None, k_weight: torch.Tensor | None, eps: float,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None):
    """Returns (q (N, Hq, D), k (N, Hkv, D)); stores K and V rows into the caches in place."""
    qkv = qkv.cpu()
    positions = positions.cpu().long()
    cos_sin = cos_sin.cpu().reshape(cos_sin.shape[0], -1).float()
    q_size, kv_size = num_heads * head_dim, num_kv_heads * head_dim
    q, k, v = qkv.split([q_size, kv_size, kv_size], dim=-1)
    q = q.reshape(-1, num_heads, head_dim)
    k = k.reshape(-1, num_kv_heads, head_dim)
    v = v.reshape(-1, num_kv_heads, head_dim)
    qw = None if q_weight is None else q_weight.cpu()
    kw = None if k_weight is None else k_weight.cpu()
    q = rope(rms_norm(q, qw, eps), positions, cos_sin)
    k = rope(rms_norm(k, kw, eps), positions, cos_sin)
    if k_cache is not None:
        keep = slot_mapping.cpu().long() != -1                       # attention.py:23
        slots = slot_mapping.cpu().long()[keep]
        k_cache.view(-1, kv_size)[slots] = k.reshape(-1, kv_size)[keep]
        v_cache.view(-1, kv_size)[slots] = v.reshape(-1, kv_size)[keep]
    return q, k
