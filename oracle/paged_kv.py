"""CPU restatement of the reference's paged-KV path -- the oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, never by the product package.

What each function restates (paths relative to the reference repository):

* store_kvcache  -- src/layers/attention.py:10-34 (kernel) and :36-61 (wrapper):
  for token i with s = slot_mapping[i] != -1, copy the (num_kv_heads * head_dim)
  element K row i and V row i into cache row s (a bit copy, done on uint16 views
  with numpy so the result is bit-exact by construction).
* gather_kv      -- the paged K/V addressing flash-attn performs for the call at
  src/layers/attention.py:93-104 with block tables from
  src/engine/model_runner.py:168-172: K_b[t] = cache[bt[b, t // BS], t % BS].
* varlen_attention -- flash_attn_varlen_func(q, k, v, cu_seqlens_q, cu_seqlens_k,
  max_seqlen_q, max_seqlen_k, softmax_scale, causal=True, block_table) as called at
  src/layers/attention.py:95-104 (flash-attn 2.8.3, pinned at uv.lock:234-236 and
  absent here). Restated from its documented semantics: per sequence, fp32 scores
  scale * q . k over the sequence's keys, bottom-right-aligned causal mask (row i
  of Lq rows over Lk keys sees t <= i + Lk - Lq), GQA head h -> kv head
  h // (Hq / Hkv), fp32 softmax, fp32 P.V. Sequences with Lq <= 0 or Lk <= 0 are
  skipped (graph padding, model_runner.py:250-257); rows that see no key are 0.

Pinning (tests/test_oracle.py): fp64 brute-force loops on tiny inputs, closed-form
special cases (Lq = Lk = 1 gives V[0]; K = 0 gives the mean of the visible V rows;
constant V rows give that constant), invariants (block relabelling, shared vs
duplicated prefix blocks, decode == last prefill row, flat == paged), and planted
mistakes (wrong mask alignment, wrong GQA map, dropped scale, skipped -1 check)
that each check must catch. The reference ships no tests or golden vectors.
"""
from __future__ import annotations

import numpy as np
import torch


def _keep_slots(slots: np.ndarray) -> np.ndarray:
    """Tokens that are stored: every slot except -1 (attention.py:23)."""
    return slots != -1


def kv_head_of(num_heads: int, num_kv_heads: int) -> torch.Tensor:
    """GQA map: query head h reads kv head h // (Hq / Hkv) (flash-attn's grouping)."""
    return torch.arange(num_heads) // (num_heads // num_kv_heads)


def visible(lq: int, lk: int, causal: bool) -> torch.Tensor:
    """(Lq, Lk) bool: row i sees key t iff t <= i + Lk - Lq (bottom-right causal)."""
    i = torch.arange(lq).unsqueeze(1)
    t = torch.arange(lk).unsqueeze(0)
    if not causal:
        return torch.ones(lq, lk, dtype=torch.bool)
    return t <= i + (lk - lq)


def default_scale(head_dim: int, softmax_scale: float | None) -> float:
    """flash-attn's default softmax_scale is head_dim ** -0.5."""
    return head_dim ** -0.5 if softmax_scale is None else softmax_scale


def _u16(t: torch.Tensor) -> np.ndarray:
    """View a CPU 16-bit tensor as a numpy uint16 array (no copy, no rounding)."""
    assert t.device.type == "cpu" and t.element_size() == 2
    return t.view(torch.int16).numpy().view(np.uint16)


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor) -> None:
    """In-place scatter of token rows into cache slots (attention.py:10-34).

    key, value: (N, Hkv, D), any row stride; k_cache, v_cache: (NB, BS, Hkv, D)
    contiguous; slot_mapping: (N,) int32, -1 = skip.
    """
    n = key.shape[0]
    row = key.shape[1] * key.shape[2]
    assert slot_mapping.numel() == n
    kc = _u16(k_cache).reshape(-1, row)
    vc = _u16(v_cache).reshape(-1, row)
    slots = slot_mapping.numpy().astype(np.int64)
    keep = _keep_slots(slots)
    kc[slots[keep]] = _u16(key.contiguous()).reshape(n, row)[keep]
    vc[slots[keep]] = _u16(value.contiguous()).reshape(n, row)[keep]


def gather_kv(cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_k: torch.Tensor) -> torch.Tensor:
    """Flat (sum Lk, Hkv, D) copy of each sequence's keys read through its block table."""
    nb, bs = cache.shape[0], cache.shape[1]
    rows = _u16(cache).reshape(nb * bs, -1)
    cu = cu_seqlens_k.numpy().astype(np.int64)
    bt = block_table.numpy().astype(np.int64)
    out = np.zeros((int(cu[-1]), rows.shape[1]), dtype=np.uint16)
    for b in range(len(cu) - 1):
        lk = int(cu[b + 1] - cu[b])
        if lk <= 0:
            continue
        t = np.arange(lk)
        out[cu[b]:cu[b] + lk] = rows[bt[b, t // bs] * bs + t % bs]
    return torch.from_numpy(out.view(np.int16)).view(cache.dtype).reshape(-1, *cache.shape[2:])


def _seq_kv(k, v, b, cu_k, block_table):
    k0, lk = int(cu_k[b]), int(cu_k[b + 1] - cu_k[b])
    if block_table is None:
        return k[k0:k0 + lk], v[k0:k0 + lk]
    bs = k.shape[1]
    t = torch.arange(lk)
    blocks = block_table[b].long()[t // bs]
    return k[blocks, t % bs], v[blocks, t % bs]


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                     softmax_scale: float | None = None, causal: bool = True,
                     block_table: torch.Tensor | None = None) -> torch.Tensor:
    """fp32 output (Nq, Hq, D) of causal varlen attention (attention.py:95-104).

    k, v: flat (Nk, Hkv, D) when block_table is None, else caches (NB, BS, Hkv, D).
    Output rows of skipped sequences are left at zero.
    """
    nq, hq, d = q.shape
    hkv = k.shape[-2]
    scale = default_scale(d, softmax_scale)
    cu_q = cu_seqlens_q.tolist()
    cu_k = cu_seqlens_k.tolist()
    out = torch.zeros(nq, hq, d, dtype=torch.float32)
    heads = kv_head_of(hq, hkv)
    for b in range(len(cu_q) - 1):
        q0, lq = cu_q[b], cu_q[b + 1] - cu_q[b]
        lk = cu_k[b + 1] - cu_k[b]
        if lq <= 0 or lk <= 0:
            continue
        kb, vb = _seq_kv(k, v, b, cu_k, block_table)
        kb = kb.float()[:, heads].transpose(0, 1)            # (Hq, Lk, D)
        vb = vb.float()[:, heads].transpose(0, 1)
        qb = q[q0:q0 + lq].float().transpose(0, 1)           # (Hq, Lq, D)
        s = torch.matmul(qb, kb.transpose(1, 2)) * scale     # (Hq, Lq, Lk)
        s = s.masked_fill(~visible(lq, lk, causal), float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        seen = torch.isfinite(m)
        p = torch.exp(s - torch.where(seen, m, torch.zeros_like(m)))
        denom = p.sum(-1, keepdim=True)
        o = torch.matmul(p, vb) / torch.where(seen, denom, torch.ones_like(denom))
        out[q0:q0 + lq] = o.transpose(0, 1)
    return out
