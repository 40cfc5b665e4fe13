"""Known-answer cases for the paged-KV path, at the real head geometry.

Inputs are regenerated from a recipe (numpy PCG64 seed -> standard normal float32
-> bf16 by round-to-nearest-even); each fixture kat_<name>.npz stores the SHA-256
of those input bytes (so a changed generator fails loudly instead of comparing
different data) and the fp64 brute-force outputs (tests/golden/bruteforce.py).
make_golden.py writes the fixtures.

Every case uses Hkv * D = 1024-element token rows and block_size 64 (the kernels
accept any multiple of 64) so short sequences still cross block boundaries.
"""
from __future__ import annotations

import hashlib

import numpy as np

BS = 64
D = 128

# name -> dict(hq, hkv, seqs=[(Lq, Lk)], paged, causal, pad=extra padded sequences)
CASES = {
    "decode3": dict(hq=16, hkv=8, seqs=[(1, 1), (1, 70), (1, 200)], paged=True, causal=True),
    "prefill2": dict(hq=16, hkv=8, seqs=[(5, 5), (37, 150)], paged=True, causal=True),
    "mixed4": dict(hq=16, hkv=8, seqs=[(1, 64), (3, 130), (1, 1), (66, 66)], paged=True, causal=True),
    "flat2": dict(hq=16, hkv=8, seqs=[(7, 7), (70, 70)], paged=False, causal=True),
    "noncausal2": dict(hq=16, hkv=8, seqs=[(4, 100), (1, 65)], paged=True, causal=False),
    "gqa1": dict(hq=8, hkv=8, seqs=[(1, 90), (9, 140)], paged=True, causal=True),
    "gqa4": dict(hq=16, hkv=4, seqs=[(1, 129), (17, 80)], paged=True, causal=True),
    "gqa8": dict(hq=16, hkv=2, seqs=[(1, 77), (20, 200)], paged=True, causal=True),
    "padded": dict(hq=16, hkv=8, seqs=[(1, 100), (2, 66)], paged=True, causal=True, pad=3),
}


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_bits_to_f64(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def build_case(name: str, seed: int = 1234) -> dict:
    """Deterministic inputs of one case (bf16 as uint16 bits, metadata as int32)."""
    c = CASES[name]
    rng = np.random.Generator(np.random.PCG64(seed + sum(map(ord, name))))
    hq, hkv = c["hq"], c["hkv"]
    seqs = list(c["seqs"])
    q_lens = [s[0] for s in seqs]
    k_lens = [s[1] for s in seqs]
    nq = sum(q_lens)
    nblocks = [-(-lk // BS) for lk in k_lens]
    nb = sum(nblocks) + 2                      # two blocks no table points at
    perm = rng.permutation(nb).tolist()
    tables, pos = [], 0
    for n in nblocks:
        tables.append(perm[pos:pos + n])
        pos += n
    width = max(nblocks) + 1                   # one -1 column of padding
    pad = c.get("pad", 0)
    bt = np.full((len(seqs) + pad, width), -1, dtype=np.int32)
    for i, t in enumerate(tables):
        bt[i, :len(t)] = t
    cu_q = np.concatenate([[0], np.cumsum(q_lens)]).astype(np.int32)
    cu_k = np.concatenate([[0], np.cumsum(k_lens)]).astype(np.int32)
    if pad:
        # graph padding (model_runner.py:252-255): the tail of cu_seqlens is zeroed, so
        # padded sequences have length <= 0 (the first one negative)
        cu_q = np.concatenate([cu_q, np.zeros(pad, np.int32)])
        cu_k = np.concatenate([cu_k, np.zeros(pad, np.int32)])
    normal = lambda *shape: f32_to_bf16_bits(rng.standard_normal(shape, dtype=np.float32))  # noqa: E731
    q = normal(nq, hq, D)
    if c["paged"]:
        k = normal(nb, BS, hkv, D)
        v = normal(nb, BS, hkv, D)
    else:
        k = normal(int(cu_k[len(seqs)]), hkv, D)
        v = normal(int(cu_k[len(seqs)]), hkv, D)
    return dict(name=name, hq=hq, hkv=hkv, q=q, k=k, v=v, cu_q=cu_q, cu_k=cu_k,
                block_table=bt if c["paged"] else None, causal=c["causal"], paged=c["paged"],
                scale=D ** -0.5, q_lens=q_lens, k_lens=k_lens)


def input_digest(case: dict) -> str:
    h = hashlib.sha256()
    for key in ("q", "k", "v", "cu_q", "cu_k", "block_table"):
        a = case[key]
        if a is not None:
            h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def expected_fp64(case: dict) -> np.ndarray:
    from golden.bruteforce import attention_fp64

    q = bf16_bits_to_f64(case["q"])
    k = bf16_bits_to_f64(case["k"])
    v = bf16_bits_to_f64(case["v"])
    if case["paged"]:
        k = k.reshape(-1, case["hkv"], D)
        v = v.reshape(-1, case["hkv"], D)
    bt = case["block_table"].tolist() if case["paged"] else None
    return attention_fp64(q, k, v, case["cu_q"].tolist(), case["cu_k"].tolist(), case["scale"],
                          case["causal"], bt, BS)
