"""Seeded synthetic batches for the paged-KV path, shaped like the reference's.

Host-side restatement of how the reference lays a batch out, used by the
benchmarks and tests:

* physical blocks are popped from a shuffled free list, one sequence after the
  other (BlockManager.allocate pops free_block_ids[0], src/engine/block_manager.py:
  183-207), so block tables are non-contiguous; shared prefix blocks appear in
  several tables (refcounted, block_manager.py:141,149);
* the slot of a new token at position p is block_table[p // BS] * BS + p % BS
  (the walk in ModelRunner.prepare_seqs, src/engine/model_runner.py:200-210);
* Lk = cached + scheduled and Lq = scheduled (model_runner.py:186-190), decodes
  first in the batch (scheduler.py:47-110), block tables -1 padded
  (model_runner.py:168-172), all metadata int32;
* v is a strided view into a fused qkv row of (Hq + 2 Hkv) * D elements and q, k
  are contiguous, as at the Qwen3 call site (src/models/qwen3.py:80-88).

Lengths and block permutations come from a CPU generator seeded per workload, so
the same workload is bit-identical on every machine; tensor values come from a
generator on the target device.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch

from .context import Context

HQ, HKV, HEAD_DIM, BLOCK_SIZE = 16, 8, 128, 256   # Qwen3-0.6B attention geometry
ROW_BYTES = HKV * HEAD_DIM * 2                     # one token row of K (or V), bytes
# One GPU's share of the heads under the reference's tensor parallelism, which splits the
# query heads and the KV cache by kv head (src/models/qwen3.py:30-36,
# src/engine/model_runner.py:153; tp defaults to 2 and may go up to 8,
# src/config/runner_config.py:12,40): (Hq / tp, Hkv / tp).
TP_HEADS = {1: (16, 8), 2: (8, 4), 4: (4, 2), 8: (2, 1)}

WORKLOADS = ("cfg1_store", "cfg1_decode", "cfg2", "cfg3", "cfg4", "prefill_steady", "decode_serve")


@dataclass
class Workload:
    name: str
    q: torch.Tensor                 # (N, Hq, D) bf16
    k: torch.Tensor                 # (N, Hkv, D) bf16, new key rows (contiguous)
    v: torch.Tensor                 # (N, Hkv, D) bf16, new value rows (strided view)
    k_cache: torch.Tensor           # (NB, BS, Hkv, D) bf16
    v_cache: torch.Tensor
    slot_mapping: torch.Tensor      # (N,) int32
    block_tables: torch.Tensor | None
    cu_seqlens_q: torch.Tensor      # (S + 1,) int32
    cu_seqlens_k: torch.Tensor
    context_lens: torch.Tensor      # (S,) int32
    max_seqlen_q: int
    max_seqlen_k: int
    q_lens: list[int]
    k_lens: list[int]
    attend: bool = True             # False: store-only workload
    unique_blocks: int = 0          # distinct physical blocks read by the attention
    meta: dict = field(default_factory=dict)

    @property
    def num_heads(self) -> int:
        return int(self.q.shape[1])

    @property
    def num_kv_heads(self) -> int:
        return int(self.k_cache.shape[2])

    @property
    def row_bytes(self) -> int:
        """One token row of K (or V) in the cache, bytes: Hkv * D * 2."""
        return self.num_kv_heads * HEAD_DIM * 2

    @property
    def ctx(self) -> Context:
        return Context(
            is_prefill=self.max_seqlen_q > 1,
            cu_seqlens_q=self.cu_seqlens_q,
            cu_seqlens_k=self.cu_seqlens_k,
            max_seqlen_q=self.max_seqlen_q,
            max_seqlen_k=self.max_seqlen_k,
            slot_mapping=self.slot_mapping,
            context_lens=self.context_lens,
            block_tables=self.block_tables,
            cached_prefix_keys=self.shared_prefix_keys,
        )

    @property
    def shared_prefix_keys(self) -> int:
        """Longest shared leading run of blocks, in keys (0 when no block is shared)."""
        if "shared_prefix_keys" not in self.meta:
            from .ops import shared_prefix_keys
            self.meta["shared_prefix_keys"] = (0 if self.block_tables is None else
                                               shared_prefix_keys(self.block_tables, BLOCK_SIZE))
        return self.meta["shared_prefix_keys"]

    # ---- algorithmic work (per pass) ----
    def store_bytes(self) -> int:
        """Read K and V rows, write K and V rows, read the slot: 4 N R + 4 N."""
        n = int(self.slot_mapping.numel())
        return 4 * n * self.row_bytes + 4 * n

    def decode_kv_bytes(self) -> int:
        """K and V bytes the one-row sequences need: sum Lk * 2R."""
        return sum(lk * 2 * self.row_bytes for lq, lk in zip(self.q_lens, self.k_lens) if lq == 1 and lk > 0)

    def decode_unique_kv_bytes(self) -> int:
        """Distinct K and V bytes the one-row sequences need. With shared prefix blocks
        (meta["shared_prefix"] keys, read by every sequence): (prefix + sum of the
        suffixes) * 2R, the keys themselves, not the whole blocks that hold them."""
        if "shared_prefix" in self.meta:
            p = self.meta["shared_prefix"]
            keys = p + sum(lk - p for lq, lk in zip(self.q_lens, self.k_lens) if lq == 1 and lk > 0)
            return keys * 2 * self.row_bytes
        return self.decode_kv_bytes()

    def decode_unique_block_bytes(self) -> int:
        """Bytes of the distinct cache blocks the one-row sequences read (whole blocks)."""
        return self.unique_blocks * BLOCK_SIZE * 2 * self.row_bytes if self.unique_blocks else self.decode_kv_bytes()

    def prefill_flops(self) -> int:
        """sum 4 Hq D (Lq P + Lq (Lq + 1) / 2) over sequences with Lq > 1 (causal)."""
        tot = 0
        for lq, lk in zip(self.q_lens, self.k_lens):
            if lq > 1:
                p = lk - lq
                tot += 4 * self.num_heads * HEAD_DIM * (lq * p + lq * (lq + 1) // 2)
        return tot

    def to(self, device) -> "Workload":
        mv = lambda t: None if t is None else t.to(device)  # noqa: E731
        # keep v a strided view: move the qkv buffer it lives in
        base = self.meta.get("qkv")
        meta = dict(self.meta)
        if base is not None:
            qkv = base.to(device)
            meta["qkv"] = qkv
            v = _v_view(qkv, self.v.shape[0], self.num_heads, self.num_kv_heads)
        else:
            v = mv(self.v)
        return Workload(self.name, mv(self.q), mv(self.k), v, mv(self.k_cache), mv(self.v_cache),
                        mv(self.slot_mapping), mv(self.block_tables), mv(self.cu_seqlens_q),
                        mv(self.cu_seqlens_k), mv(self.context_lens), self.max_seqlen_q,
                        self.max_seqlen_k, list(self.q_lens), list(self.k_lens), self.attend,
                        self.unique_blocks, meta)


def _v_view(qkv: torch.Tensor, n: int, hq: int = HQ, hkv: int = HKV) -> torch.Tensor:
    return qkv[:, (hq + hkv) * HEAD_DIM:].view(n, hkv, HEAD_DIM)


def slots_for(block_table: list[int], start: int, end: int, block_size: int = BLOCK_SIZE) -> list[int]:
    """Slots of positions [start, end) of one sequence (model_runner.py:200-210)."""
    return [block_table[p // block_size] * block_size + p % block_size for p in range(start, end)]


def _randn(shape, gen: torch.Generator, device) -> torch.Tensor:
    return torch.randn(shape, generator=gen, device=device, dtype=torch.float32).to(torch.bfloat16) \
        if torch.device(device).type == "cpu" else \
        torch.randn(shape, generator=gen, device=device, dtype=torch.bfloat16)


def _assemble(name: str, seqs: list[tuple[int, int, list[int]]], num_blocks: int, seed: int,
              device, attend: bool = True, unique_blocks: int = 0, meta: dict | None = None,
              heads: tuple[int, int] = (HQ, HKV)) -> Workload:
    """seqs: (Lq, Lk, block_table) per sequence in batch order; new tokens are the
    last Lq positions of each sequence. heads = (Hq, Hkv)."""
    hq, hkv = heads
    dev = torch.device(device)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    q_lens = [s[0] for s in seqs]
    k_lens = [s[1] for s in seqs]
    n = sum(q_lens)
    slots: list[int] = []
    for lq, lk, bt in seqs:
        slots += slots_for(bt, lk - lq, lk)
    width = max((len(s[2]) for s in seqs), default=0)
    k_cache = _randn((num_blocks, BLOCK_SIZE, hkv, HEAD_DIM), gen, dev)
    v_cache = _randn((num_blocks, BLOCK_SIZE, hkv, HEAD_DIM), gen, dev)
    qkv = _randn((n, (hq + 2 * hkv) * HEAD_DIM), gen, dev)
    q = qkv[:, :hq * HEAD_DIM].reshape(n, hq, HEAD_DIM).clone()
    k = qkv[:, hq * HEAD_DIM:(hq + hkv) * HEAD_DIM].reshape(n, hkv, HEAD_DIM).clone()
    v = _v_view(qkv, n, hq, hkv)
    bts = torch.full((len(seqs), width), -1, dtype=torch.int32)
    for i, (_, _, bt) in enumerate(seqs):
        bts[i, :len(bt)] = torch.tensor(bt, dtype=torch.int32)
    cu_q = torch.tensor([0] + list(_cumsum(q_lens)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(_cumsum(k_lens)), dtype=torch.int32)
    m = dict(meta or {})
    m["qkv"] = qkv
    return Workload(
        name=name, q=q, k=k, v=v, k_cache=k_cache, v_cache=v_cache,
        slot_mapping=torch.tensor(slots, dtype=torch.int32).to(dev),
        block_tables=bts.to(dev), cu_seqlens_q=cu_q.to(dev), cu_seqlens_k=cu_k.to(dev),
        context_lens=torch.tensor(k_lens, dtype=torch.int32).to(dev),
        max_seqlen_q=max(q_lens, default=0), max_seqlen_k=max(k_lens, default=0),
        q_lens=q_lens, k_lens=k_lens, attend=attend, unique_blocks=unique_blocks, meta=m)


def _cumsum(xs):
    t = 0
    for x in xs:
        t += x
        yield t


def _pop_tables(lengths: list[int], pool: list[int]) -> list[list[int]]:
    """Pop ceil(L / BS) blocks per sequence, in order, from the front of pool."""
    tables, pos = [], 0
    for length in lengths:
        nb = math.ceil(length / BLOCK_SIZE)
        tables.append(pool[pos:pos + nb])
        pos += nb
    return tables


def _uniform(gen: torch.Generator, lo: int, hi: int, n: int) -> list[int]:
    """n integers uniform on [lo, hi] (inclusive, like random.randint)."""
    return torch.randint(lo, hi + 1, (n,), generator=gen).tolist()


def make_workload(name: str, device="cpu", seed: int | None = None,
                  num_seqs: int | None = None, heads: tuple[int, int] = (HQ, HKV)) -> Workload:
    """Build one of WORKLOADS. num_seqs shrinks the batch (tests); None = full size.
    heads = (Hq, Hkv): the whole model's (16, 8) or one tensor-parallel rank's share
    (TP_HEADS); lengths and block tables do not depend on it."""
    if name not in WORKLOADS:
        raise ValueError(f"unknown workload {name!r}; choose from {WORKLOADS}")
    hq, hkv = heads
    if hq <= 0 or hkv <= 0 or hq % hkv:
        raise ValueError(f"heads {heads}: Hq must be a positive multiple of Hkv")
    kw = {"heads": (hq, hkv)}
    cfg_seed = {"cfg1_store": 1, "cfg1_decode": 1, "cfg2": 2, "cfg3": 3, "cfg4": 4, "prefill_steady": 5,
                "decode_serve": 9}[name]
    seed = cfg_seed if seed is None else seed
    host = torch.Generator()
    host.manual_seed(seed)

    if name in ("cfg1_store", "cfg1_decode"):
        # 64-block cache; 2048 new tokens stored into 8 popped blocks, then a decode
        # batch of 8 sequences (Lk ~ U[256, 2048]) over a reshuffled pool.
        nb = 64
        store_pool = torch.randperm(nb, generator=host).tolist()
        n_store = 2048 if num_seqs is None else min(2048, 256 * num_seqs)
        s = 8 if num_seqs is None else num_seqs
        lks = _uniform(host, 256, 2048, s)
        pool = torch.randperm(nb, generator=host).tolist()
        if name == "cfg1_store":
            bt = store_pool[:math.ceil(n_store / BLOCK_SIZE)]
            return _assemble(name, [(n_store, n_store, bt)], nb, seed * 1000 + 11, device, attend=False, **kw)
        tables = _pop_tables(lks, pool)
        return _assemble(name, [(1, lk, bt) for lk, bt in zip(lks, tables)], nb, seed * 1000 + 12, device, **kw)

    if name == "cfg2":
        # decode at serving scale: S = 256, Lk ~ U[1024, 8192], pool = exactly the blocks needed
        s = 256 if num_seqs is None else num_seqs
        lks = _uniform(host, 1024, 8192, s)
        nb = sum(math.ceil(lk / BLOCK_SIZE) for lk in lks)
        pool = torch.randperm(nb, generator=host).tolist()
        tables = _pop_tables(lks, pool)
        return _assemble(name, [(1, lk, bt) for lk, bt in zip(lks, tables)], nb, seed * 1000 + 2, device,
                         unique_blocks=nb, **kw)

    if name == "decode_serve":
        # the serving run's decode steps: 128 live sequences (the scheduler's cap,
        # scheduler.py:37) of prompt + generated tokens, contexts U[100, 2048]
        s = 128 if num_seqs is None else num_seqs
        lks = _uniform(host, 100, 2048, s)
        nb = sum(math.ceil(lk / BLOCK_SIZE) for lk in lks)
        pool = torch.randperm(nb, generator=host).tolist()
        tables = _pop_tables(lks, pool)
        return _assemble(name, [(1, lk, bt) for lk, bt in zip(lks, tables)], nb, seed * 1000 + 9, device,
                         unique_blocks=nb, **kw)

    if name == "cfg3":
        # mixed batch: 128 decodes (Lk ~ U[512, 4096]) first, then 8 prefill chunks of
        # 512 tokens over cached prefixes P ~ U[0, 4096]
        n_dec = 128 if num_seqs is None else num_seqs
        n_pre = 8 if num_seqs is None else max(1, num_seqs // 4)
        dec_lks = _uniform(host, 512, 4096, n_dec)
        prefixes = _uniform(host, 0, 4096, n_pre)
        chunk = 512
        lks = dec_lks + [p + chunk for p in prefixes]
        nb = sum(math.ceil(lk / BLOCK_SIZE) for lk in lks)
        pool = torch.randperm(nb, generator=host).tolist()
        tables = _pop_tables(lks, pool)
        seqs = [(1, lk, bt) for lk, bt in zip(dec_lks, tables[:n_dec])]
        seqs += [(chunk, lk, bt) for lk, bt in zip(lks[n_dec:], tables[n_dec:])]
        return _assemble(name, seqs, nb, seed * 1000 + 3, device, unique_blocks=0,
                         meta={"prefixes": prefixes}, **kw)

    if name == "prefill_steady":
        # chunked prefill large enough to keep every CU busy: 16 chunks of 1024 tokens, each
        # over a 4096-token cached prefix (618 GFLOP of causal attention)
        s = 16 if num_seqs is None else num_seqs
        chunk, prefix = 1024, 4096
        lks = [prefix + chunk] * s
        nb = sum(math.ceil(lk / BLOCK_SIZE) for lk in lks)
        pool = torch.randperm(nb, generator=host).tolist()
        tables = _pop_tables(lks, pool)
        return _assemble(name, [(chunk, lk, bt) for lk, bt in zip(lks, tables)], nb, seed * 1000 + 5, device, **kw)

    # cfg4: 64 sequences share one 2048-token prefix (8 physical blocks, refcount 64);
    # private suffixes of U[256, 1024] tokens.
    s = 64 if num_seqs is None else num_seqs
    prefix = 2048
    suffixes = _uniform(host, 256, 1024, s)
    n_shared = prefix // BLOCK_SIZE
    n_private = sum(math.ceil(x / BLOCK_SIZE) for x in suffixes)
    nb = n_shared + n_private
    pool = torch.randperm(nb, generator=host).tolist()
    shared, private = pool[:n_shared], pool[n_shared:]
    tables = [shared + t for t in _pop_tables(suffixes, private)]
    seqs = [(1, prefix + x, bt) for x, bt in zip(suffixes, tables)]
    return _assemble(name, seqs, nb, seed * 1000 + 4, device, unique_blocks=nb,
                     meta={"shared_blocks": shared, "shared_prefix": prefix}, **kw)


def serving_requests(seed: int = 5, num_requests: int = 256, vocab_size: int = 151936,
                     lo: int = 100, hi: int = 1024) -> tuple[list[list[int]], list[int]]:
    """The offline serving workload: num_requests prompts of token ids uniform in
    [0, vocab_size) with lengths uniform in [lo, hi], and output lengths uniform in [lo, hi]
    (greedy, ignore_eos), drawn from random.Random(seed), prompts first and output lengths
    after, in the order of the reference's bench.py:63-64 (which draws ids below 10000;
    this workload draws them from the whole vocabulary)."""
    import random

    rng = random.Random(seed)
    prompts = [[rng.randrange(vocab_size) for _ in range(rng.randint(lo, hi))] for _ in range(num_requests)]
    max_tokens = [rng.randint(lo, hi) for _ in range(num_requests)]
    return prompts, max_tokens
