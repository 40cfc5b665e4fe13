"""Per-step attention metadata -- same fields and meaning as the reference's
Context (src/utils/context.py:5-14), built by the runner (model_runner.py:174-233).

* cu_seqlens_q / cu_seqlens_k: (S + 1,) int32 prefix sums of per-sequence query
  and key lengths; sequence lengths are always derived from these on the device.
* max_seqlen_q / max_seqlen_k: host-side upper bounds (launch sizes only).
* slot_mapping: (N,) int32 cache slot of every new token, -1 = do not store.
* context_lens: (S,) int32 key length per sequence; produced by the runner and,
  as in the reference, not read by Attention.
* block_tables: (S, W) int32, -1 padded; None selects flat (fresh K/V) attention.
* cached_prefix_keys (an addition): the longest prefix the batch's sequences share
  (shared_prefix_keys), in keys. Decode reads past it stream (a cache hint); above 0 it also
  selects the shared-prefix decode path, which computes the shared blocks once for all the
  sequences that hold them (results within the attention tolerance of the plain path).
  0 states that no block is shared (and allows the one-launch store + decode); None keeps
  the library default.
"""
from __future__ import annotations

from dataclasses import dataclass

from torch import Tensor


@dataclass(slots=True)
class Context:
    is_prefill: bool = False
    cu_seqlens_q: Tensor | None = None
    cu_seqlens_k: Tensor | None = None
    max_seqlen_q: int = 0
    max_seqlen_k: int = 0
    slot_mapping: Tensor | None = None
    context_lens: Tensor | None = None
    block_tables: Tensor | None = None
    cached_prefix_keys: int | None = None
