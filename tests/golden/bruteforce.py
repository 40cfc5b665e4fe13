"""fp64 brute-force attention for tiny inputs -- the checker that pins the oracle.

Written independently of oracle/paged_kv.py: explicit Python loops over sequences,
kv heads, the query heads of each kv head, rows and keys; the visible keys of a
row are enumerated one by one; keys are addressed by walking the block table
slot by slot (model_runner.py:200-210 form); math.exp in float64.
"""
from __future__ import annotations

import math

import numpy as np


def attention_fp64(q, k, v, cu_q, cu_k, scale, causal=True, block_table=None, block_size=None):
    """q (Nq, Hq, D); k, v flat (Nk, Hkv, D) or caches flattened to (slots, Hkv, D);
    all float64 numpy. Returns (Nq, Hq, D) float64; skipped rows stay 0."""
    nq, hq, d = q.shape
    hkv = k.shape[1]
    group = hq // hkv
    out = np.zeros((nq, hq, d), dtype=np.float64)
    for b in range(len(cu_q) - 1):
        q0 = cu_q[b]
        lq = cu_q[b + 1] - cu_q[b]
        lk = cu_k[b + 1] - cu_k[b]
        if lq <= 0 or lk <= 0:
            continue
        rows = []
        for t in range(lk):
            if block_table is None:
                rows.append(cu_k[b] + t)
            else:
                rows.append(block_table[b][t // block_size] * block_size + t % block_size)
        for g in range(hkv):
            for h in range(g * group, (g + 1) * group):
                for i in range(lq):
                    allowed = [t for t in range(lk) if (not causal) or t - (lk - lq) <= i]
                    if not allowed:
                        continue
                    scores = [scale * float(np.dot(q[q0 + i, h], k[rows[t], g])) for t in allowed]
                    top = max(scores)
                    w = [math.exp(s - top) for s in scores]
                    z = math.fsum(w)
                    acc = np.zeros(d, dtype=np.float64)
                    for wt, t in zip(w, allowed):
                        acc += wt * v[rows[t], g]
                    out[q0 + i, h] = acc / z
    return out
