"""CPU restatement of the serving loop's other kernels -- the oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.

* rms_norm_residual -- RMSNorm.residual_forward, src/layers/layernorm.py:18-28: s = x + r in
  fp32, out = bf16(w * (s * rsqrt(mean(s^2) + eps))), new residual = bf16(s).
* silu_and_mul      -- SiluAndMul.forward, src/layers/activation.py:6-10, as torch.compile
  runs it: both halves upcast, silu(x) * y in fp32, one rounding to bf16.
* lm_head_greedy    -- ParallelLMHead.forward, src/layers/llm_head.py:60-64 (row selection
  cu_seqlens_q[1:] - 1 for prefill batches, logits = F.linear(x, W) rounded to bf16),
  then argmax with the lowest index among equal maxima (torch.argmax's rule).

Pinning (tests/test_oracle_model_ops.py): closed forms (x + r = 0 gives zeros; a constant
sum normalises to its sign; silu(0) = 0 and silu(x) * 1 = x sigmoid(x) against math.exp;
one-hot weight rows make the logits the hidden values themselves), ties resolved to the
lowest index, fp64 loops with the same rounding points, and planted mistakes (residual not
added, two roundings in SiLU * mul, last index on ties, no row selection) that must fail.
"""
from __future__ import annotations

import torch


def rms_norm_residual(x: torch.Tensor, residual: torch.Tensor, weight: torch.Tensor, eps: float):
    s = x.float() + residual.float()
    var = s.square().mean(-1, keepdim=True) + eps
    return (weight.float() * (s * var.rsqrt())).to(x.dtype), s.to(x.dtype)


def silu_and_mul(x: torch.Tensor) -> torch.Tensor:
    g, u = x.float().chunk(2, -1)
    return (g / (1.0 + torch.exp(-g)) * u).to(x.dtype)


def lm_head_greedy(hidden: torch.Tensor, weight: torch.Tensor,
                   cu_seqlens_q: torch.Tensor | None = None) -> torch.Tensor:
    x = hidden.float()
    if cu_seqlens_q is not None:
        x = x[cu_seqlens_q[1:].long() - 1]
    logits = (x.double() @ weight.double().T).to(torch.bfloat16).float()
    return first_argmax(logits)


def first_argmax(logits: torch.Tensor) -> torch.Tensor:
    """Index of the first maximum along the last dimension."""
    m = logits.max(dim=-1, keepdim=True).values
    idx = torch.arange(logits.shape[-1]).expand_as(logits)
    big = torch.full_like(idx, logits.shape[-1])
    return torch.where(logits == m, idx, big).min(dim=-1).values
