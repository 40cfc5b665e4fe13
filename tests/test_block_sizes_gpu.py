"""GPU parity at cache block sizes other than 256.

The reference accepts any KV block size that is a multiple of 256 (runner_config.py:39); the
kernels accept any multiple of 64 (a 64-key tile never straddles two blocks). The other GPU
tests use 256 (the serving shape) and 64 (the fixtures); these run 128, 512 and 1024 through
the store (bit-exact against the oracle's scatter, attention.py:10-34), a call mixing decode
rows with prefill chunks over cached prefixes, a decode batch on the flat grid, and the
shared-prefix path, each against the oracle (attention.py:95-104).
"""
import math

import numpy as np
import pytest
import torch

import oracle
import pagedkv
from paged_helpers import assert_close_bf16, bits_equal

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5
HQ, HKV, D = 16, 8, 128


def _case(bs, spec, seed, shared_blocks=0):
    """spec: (Lq, Lk) per sequence; the new tokens are each sequence's last Lq positions.
    shared_blocks: leading blocks every sequence maps to the same physical blocks (prefix
    caching); the rest of each table is private and shuffled."""
    g = torch.Generator().manual_seed(seed)
    nb_per = [math.ceil(lk / bs) for _, lk in spec]
    private = [max(0, n - shared_blocks) for n in nb_per]
    nb = shared_blocks + sum(private) + 2
    perm = torch.randperm(nb, generator=g).tolist()
    shared, pool = perm[:shared_blocks], perm[shared_blocks:]
    bt = torch.full((len(spec), max(nb_per)), -1, dtype=torch.int32)
    pos = 0
    for i, n in enumerate(nb_per):
        row = shared[:min(n, shared_blocks)] + pool[pos:pos + private[i]]
        pos += private[i]
        bt[i, :n] = torch.tensor(row, dtype=torch.int32)
    nq = sum(lq for lq, _ in spec)
    slots = []
    for i, (lq, lk) in enumerate(spec):
        for t in range(lk - lq, lk):
            slots.append(int(bt[i, t // bs]) * bs + t % bs)
    return dict(
        q=torch.randn(nq, HQ, D, generator=g).to(torch.bfloat16),
        k=torch.randn(nq, HKV, D, generator=g).to(torch.bfloat16),
        v=torch.randn(nq, HKV, D, generator=g).to(torch.bfloat16),
        kc=torch.randn(nb, bs, HKV, D, generator=g).to(torch.bfloat16),
        vc=torch.randn(nb, bs, HKV, D, generator=g).to(torch.bfloat16),
        bt=bt, slots=torch.tensor(slots, dtype=torch.int32),
        cu_q=torch.tensor([0] + np.cumsum([lq for lq, _ in spec]).tolist(), dtype=torch.int32),
        cu_k=torch.tensor([0] + np.cumsum([lk for _, lk in spec]).tolist(), dtype=torch.int32),
        max_q=max(lq for lq, _ in spec), max_k=max(lk for _, lk in spec))


def _run(c, dev, shared_prefix_keys=None):
    """Store the new rows, then attend (Attention.forward's two steps) on the GPU and in the
    oracle; returns (gpu out, oracle out, gpu caches, oracle caches)."""
    kc, vc = c["kc"].to(dev), c["vc"].to(dev)
    pagedkv.store_kvcache(c["k"].to(dev), c["v"].to(dev), kc, vc, c["slots"].to(dev))
    out = pagedkv.varlen_attention(c["q"].to(dev), kc, vc, c["cu_q"].to(dev), c["cu_k"].to(dev), c["max_q"],
                                   c["max_k"], SCALE, True, c["bt"].to(dev), shared_prefix_keys=shared_prefix_keys)
    kco, vco = c["kc"].clone(), c["vc"].clone()
    oracle.store_kvcache(c["k"], c["v"], kco, vco, c["slots"])
    want = oracle.varlen_attention(c["q"], kco, vco, c["cu_q"], c["cu_k"], SCALE, True, c["bt"])
    torch.cuda.synchronize()
    return out, want, (kc, vc), (kco, vco)


@pytest.mark.parametrize("bs", [128, 512, 1024])
def test_store_and_mixed_call(gpu, bs):
    """Decode rows of 1 to 9000 keys between prefill chunks over cached prefixes (block
    boundaries inside chunks and tiles at every block size): caches bit-exact after the store,
    every row within tolerance of the oracle."""
    spec = [(1, 1), (1, 700), (300, 1000), (1, 3000), (64, 64), (1, 9000), (200, 4600), (1, 5000), (37, 1201)]
    c = _case(bs, spec, seed=bs)
    print(f"[block sizes] mixed call, block_size={bs}", flush=True)
    out, want, (kc, vc), (kco, vco) = _run(c, gpu)
    assert bits_equal(kc, kco) and bits_equal(vc, vco), "store"
    assert_close_bf16(out, want, f"mixed call, block_size {bs}")


@pytest.mark.parametrize("bs", [128, 512, 1024])
def test_decode_batch_on_flat_grid(gpu, bs):
    """48 decode rows of 500-3000 keys (the flat decode grid: pieces cut across block
    boundaries)."""
    lens = torch.randint(500, 3001, (48,), generator=torch.Generator().manual_seed(bs + 1)).tolist()
    c = _case(bs, [(1, lk) for lk in lens], seed=bs + 1)
    print(f"[block sizes] flat decode grid, block_size={bs}", flush=True)
    out, want, _, _ = _run(c, gpu)
    assert_close_bf16(out, want, f"flat decode grid, block_size {bs}")


@pytest.mark.parametrize("bs", [128, 512, 1024])
def test_shared_prefix_path(gpu, bs):
    """24 decode rows whose first 2048 keys lie in blocks they all share, private suffixes of
    100-1500 keys: the shared-prefix path (chunks of whole blocks) against the oracle."""
    nsh = 2048 // bs
    lens = torch.randint(2048 + 100, 2048 + 1501, (24,), generator=torch.Generator().manual_seed(bs + 2)).tolist()
    c = _case(bs, [(1, lk) for lk in lens], seed=bs + 2, shared_blocks=nsh)
    assert pagedkv.shared_prefix_keys(c["bt"], bs) == nsh * bs
    print(f"[block sizes] shared prefix, block_size={bs}", flush=True)
    out, want, _, _ = _run(c, gpu, shared_prefix_keys=nsh * bs)
    assert_close_bf16(out, want, f"shared prefix, block_size {bs}")
