"""Shared helpers of the GPU parity tests (not a test module)."""
from __future__ import annotations

import math

import numpy as np
import torch

import oracle
from pagedkv.workloads import BLOCK_SIZE, Workload

ATOL_MAX = 2e-2   # max |gpu - oracle| for bf16 attention outputs
ATOL_MEAN = 1e-2  # mean |gpu - oracle|


def assert_close_bf16(got: torch.Tensor, want: torch.Tensor, what: str = ""):
    diff = (got.float().cpu() - want.float().cpu()).abs()
    assert torch.isfinite(got.float()).all(), f"{what}: non-finite output"
    mx, mean = diff.max().item(), diff.mean().item()
    assert mx <= ATOL_MAX and mean <= ATOL_MEAN, f"{what}: max {mx:.3e} mean {mean:.3e}"
    return mx, mean


def bits_equal(a: torch.Tensor, b: torch.Tensor) -> bool:
    return torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))


def subset_oracle(w: Workload, seq_ids: list[int]):
    """Oracle output of Attention.forward (store, then attend) for the chosen sequences.

    Only the blocks those sequences read are copied to the host (block ids
    renumbered), so this works at full serving size. Call it BEFORE the GPU forward
    (which stores the new tokens into the device caches).
    Returns (row indices into the batch, fp32 output rows).
    """
    bt = w.block_tables.cpu()
    blocks = sorted({int(x) for b in seq_ids
                     for x in bt[b, :math.ceil(w.k_lens[b] / BLOCK_SIZE)].tolist()})
    remap = {old: new for new, old in enumerate(blocks)}
    idx = torch.tensor(blocks, dtype=torch.long, device=w.k_cache.device)
    kc = w.k_cache.index_select(0, idx).cpu()
    vc = w.v_cache.index_select(0, idx).cpu()
    cu_q = w.cu_seqlens_q.cpu().tolist()
    slots = w.slot_mapping.cpu().tolist()
    rows, new_slots, q_lens, k_lens = [], [], [], []
    width = max(math.ceil(w.k_lens[b] / BLOCK_SIZE) for b in seq_ids)
    bt_sub = torch.full((len(seq_ids), width), -1, dtype=torch.int32)
    for j, b in enumerate(seq_ids):
        r = list(range(cu_q[b], cu_q[b + 1]))
        rows += r
        for i in r:
            s = slots[i]
            new_slots.append(-1 if s == -1 else remap[s // BLOCK_SIZE] * BLOCK_SIZE + s % BLOCK_SIZE)
        q_lens.append(len(r))
        k_lens.append(w.k_lens[b])
        nbk = math.ceil(w.k_lens[b] / BLOCK_SIZE)
        bt_sub[j, :nbk] = torch.tensor([remap[int(x)] for x in bt[b, :nbk].tolist()], dtype=torch.int32)
    ridx = torch.tensor(rows, dtype=torch.long, device=w.q.device)
    q = w.q.index_select(0, ridx).cpu()
    k = w.k.index_select(0, ridx).cpu()
    v = w.v.index_select(0, ridx).cpu()
    oracle.store_kvcache(k, v, kc, vc, torch.tensor(new_slots, dtype=torch.int32))
    cu_qs = torch.tensor(np.concatenate([[0], np.cumsum(q_lens)]), dtype=torch.int32)
    cu_ks = torch.tensor(np.concatenate([[0], np.cumsum(k_lens)]), dtype=torch.int32)
    out = oracle.varlen_attention(q, kc, vc, cu_qs, cu_ks, 128 ** -0.5, True, bt_sub)
    return rows, out
