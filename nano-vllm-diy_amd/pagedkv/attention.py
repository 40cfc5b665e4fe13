"""Drop-in Attention layer for the paged-KV path.

Same class, constructor and forward(q, k, v, ctx) as the reference's Attention
(src/layers/attention.py:63-105), and the same store_kvcache helper (:36-61), but
every device operation is a hand-written gfx950 HIP kernel from libpagedkv.so:

* forward stores the new K/V rows into the bound cache first (when the runner has
  bound one; attention.py:87-88), so a token attends to itself;
* with ctx.block_tables set it reads K/V from the paged cache, otherwise from the
  fresh k / v rows (attention.py:93-94);
* one call covers a mixed batch: one-row sequences go to the split-K decode kernel
  and longer ones to the MFMA prefill kernel, both bottom-right causal;
* on a decode step (one new token per sequence, paged) whose caller states that no cache
  block is read by two sequences of the batch (ctx.cached_prefix_keys == 0, what
  shared_prefix_keys returns when no block's reference count exceeds 1), the store and the
  attention run in one launch of the split-K kernel (pk_store_decode_attention),
  bit-identical to the two. In that launch a token's row is written while other
  work-groups read the cache, so the one-launch path needs the token's slot to lie in a
  block no other sequence reads. With prefix caching that can fail: a fully cached prompt
  recomputes its last token (scheduler.py:77-80, model_runner.py:185-186) into a block
  other live sequences share. The reference's eight-field Context carries no such
  statement, so it always gets the two launches, whose store is ordered before every read;
* a Context stating a shared prefix (ctx.cached_prefix_keys > 0) also selects the
  shared-prefix decode path: the decode rows' keys below it are computed once per shared
  block for all sequences that hold it (pk_varlen_attention_shared_prefix).

The runner rebinds k_cache / v_cache to per-layer views of its KV tensor
(model_runner.py:159-165), exactly as with the reference layer.
"""
from __future__ import annotations

import torch
from torch import nn

from .context import Context
from .ops import store_kvcache as _store_kvcache
from .ops import store_decode_attention, varlen_attention


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """Reference signature of store_kvcache (attention.py:36-42)."""
    _store_kvcache(key, value, k_cache, v_cache, slot_mapping)


def _contiguous_blocks(cache: torch.Tensor) -> bool:
    """(NB, BS, Hkv, D) with contiguous rows and blocks: the one-launch decode step writes a
    token's row where store_kvcache writes slot * row only for such caches."""
    return cache.dim() == 4 and cache.stride(3) == 1 and cache.stride(2) == cache.shape[3] and \
        cache.stride(1) == cache.shape[2] * cache.shape[3] and cache.stride(0) == cache.shape[1] * cache.stride(1)


class Attention(nn.Module):
    def __init__(self, head_dim: int, num_heads: int, num_kv_heads: int, scale: float = None):
        super().__init__()
        self.head_dim = head_dim
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.scale = scale
        self.k_cache = torch.tensor([])
        self.v_cache = torch.tensor([])

    def forward(self, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, ctx: Context) -> torch.Tensor:
        k_cache, v_cache = self.k_cache, self.v_cache
        bound = k_cache.numel() and v_cache.numel()
        hint = getattr(ctx, "cached_prefix_keys", None)  # absent on the reference Context
        if bound and ctx.block_tables is not None and ctx.max_seqlen_q == 1 and hint == 0 and \
                q.shape[0] == k.shape[0] == ctx.cu_seqlens_q.numel() - 1 and _contiguous_blocks(k_cache) and \
                _contiguous_blocks(v_cache):
            # a decode step (one new token per sequence) over blocks no two sequences share:
            # the store and the attention in one launch, bit-identical to the two
            return store_decode_attention(q, k, v, k_cache, v_cache, ctx.slot_mapping, ctx.cu_seqlens_q,
                                          ctx.cu_seqlens_k, ctx.max_seqlen_k, self.scale, ctx.block_tables,
                                          cached_prefix_keys=hint)
        if bound:
            store_kvcache(k, v, k_cache, v_cache, ctx.slot_mapping)
        shared = None
        if ctx.block_tables is not None:
            k, v = k_cache, v_cache
            shared = hint if hint is not None and hint > 0 else None
        return varlen_attention(
            q, k, v,
            cu_seqlens_q=ctx.cu_seqlens_q,
            cu_seqlens_k=ctx.cu_seqlens_k,
            max_seqlen_q=ctx.max_seqlen_q,
            max_seqlen_k=ctx.max_seqlen_k,
            softmax_scale=self.scale,
            causal=True,
            block_table=ctx.block_tables,
            cached_prefix_keys=hint,
            shared_prefix_keys=shared,
        )
