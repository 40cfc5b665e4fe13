"""GPU parity at one tensor-parallel rank's share of the heads.

The reference splits the query heads and the KV cache by kv head across its tensor-parallel
ranks (src/models/qwen3.py:30-36, src/engine/model_runner.py:153); tp defaults to 2 and may
go up to 8 (src/config/runner_config.py:12,40). A drop-in Attention on one rank therefore
sees (Hq, Hkv) = (8, 4) at tp 2, (4, 2) at tp 4 and (2, 1) at tp 8, with the same head_dim,
block size and sequence lengths. These tests run the serving configurations at those shares
through the C-ABI against the oracle (2e-2 max / 1e-2 mean abs): the decode batch of 256
sequences of 1k-8k keys (split grid), the mixed chunked-prefill batch (flat decode grid,
prefill kernel and merge), the shared-prefix batch (shared-prefix kernel + suffix grid) and
its bit identity with duplicated prefix blocks, and the one-launch store + decode step.
"""
import numpy as np
import pytest
import torch

import pagedkv
from paged_helpers import assert_close_bf16, bits_equal, subset_oracle
from pagedkv.workloads import TP_HEADS, make_workload

pytestmark = pytest.mark.gpu

SCALE = 128 ** -0.5
SHARES = [2, 4, 8]


def _layer(w):
    layer = pagedkv.Attention(128, w.num_heads, w.num_kv_heads, SCALE)
    layer.k_cache, layer.v_cache = w.k_cache, w.v_cache
    return layer


@pytest.mark.parametrize("tp", SHARES)
def test_decode_batch_at_rank_share(gpu, tp):
    """256 sequences of 1024-8192 keys, store + decode through Attention.forward (one launch),
    every row against the oracle."""
    hq, hkv = TP_HEADS[tp]
    print(f"[tp] decode batch tp={tp} heads={hq}/{hkv}", flush=True)
    w = make_workload("cfg2", gpu, heads=(hq, hkv))
    rows, want = subset_oracle(w, list(range(len(w.q_lens))))
    out = _layer(w)(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, f"decode tp={tp}")


@pytest.mark.parametrize("tp", SHARES)
def test_decode_split_and_flat_grids_at_rank_share(gpu, tp):
    """The decode rows of the mixed batch alone (128 sequences of 512-4096 keys: the flat grid)
    and the first 40 of them (40 x 4096 keys is below the flat grid's bound: the split grid)."""
    hq, hkv = TP_HEADS[tp]
    print(f"[tp] split/flat grids tp={tp}", flush=True)
    w = make_workload("cfg3", gpu, heads=(hq, hkv))
    dec = [i for i, lq in enumerate(w.q_lens) if lq == 1]
    rows, want = subset_oracle(w, dec)
    pagedkv.store_kvcache(w.k, w.v, w.k_cache, w.v_cache, w.slot_mapping)
    for n in (len(dec), 40):
        ids = dec[:n]
        lks = [w.k_lens[i] for i in ids]
        cu_q = torch.arange(n + 1, dtype=torch.int32, device=gpu)
        cu_k = torch.tensor([0] + np.cumsum(lks).tolist(), dtype=torch.int32, device=gpu)
        q = w.q.index_select(0, torch.tensor([rows[i] for i in range(n)], device=gpu))
        bt = w.block_tables[:n].contiguous()
        out = pagedkv.varlen_attention(q, w.k_cache, w.v_cache, cu_q, cu_k, 1, max(lks), SCALE, True, bt,
                                       cached_prefix_keys=0)
        torch.cuda.synchronize()
        assert_close_bf16(out, want[:n], f"decode rows tp={tp} n={n}")


@pytest.mark.parametrize("tp", SHARES)
def test_mixed_batch_at_rank_share(gpu, tp):
    """The mixed chunked-prefill batch at full size: every decode row and two prefill chunks."""
    hq, hkv = TP_HEADS[tp]
    print(f"[tp] mixed batch tp={tp}", flush=True)
    w = make_workload("cfg3", gpu, heads=(hq, hkv))
    ids = list(range(128)) + [128, 133]
    rows, want = subset_oracle(w, ids)
    out = _layer(w)(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, f"mixed tp={tp}")


@pytest.mark.parametrize("tp", SHARES)
def test_shared_prefix_batch_at_rank_share(gpu, tp):
    """64 sequences over one shared 2048-key prefix, through Attention.forward (the Context
    states the shared prefix, so the shared-prefix path runs): every row against the oracle,
    and bit for bit against private copies of the prefix blocks."""
    hq, hkv = TP_HEADS[tp]
    print(f"[tp] shared prefix tp={tp}", flush=True)
    w = make_workload("cfg4", gpu, heads=(hq, hkv))
    assert w.ctx.cached_prefix_keys == 2048
    rows, want = subset_oracle(w, list(range(len(w.q_lens))))
    out = _layer(w)(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert_close_bf16(out[rows], want, f"shared prefix tp={tp}")
    shared = w.meta["shared_blocks"]
    nb, s = w.k_cache.shape[0], len(w.q_lens)
    extra = torch.tensor(shared, device=gpu).repeat(s)
    kc = torch.cat([w.k_cache, w.k_cache[extra]])
    vc = torch.cat([w.v_cache, w.v_cache[extra]])
    bt = w.block_tables.clone()
    bt[:, :len(shared)] = (nb + torch.arange(s * len(shared), device=gpu).view(s, -1)).int()
    shared_out = pagedkv.varlen_attention(w.q, w.k_cache, w.v_cache, w.cu_seqlens_q, w.cu_seqlens_k, 1,
                                          w.max_seqlen_k, SCALE, True, w.block_tables, cached_prefix_keys=2048,
                                          shared_prefix_keys=2048)
    priv = pagedkv.varlen_attention(w.q, kc, vc, w.cu_seqlens_q, w.cu_seqlens_k, 1, w.max_seqlen_k, SCALE, True,
                                    bt, cached_prefix_keys=2048, shared_prefix_keys=2048)
    torch.cuda.synchronize()
    assert bits_equal(shared_out, priv)


@pytest.mark.parametrize("tp", SHARES)
def test_store_decode_step_bit_identical_at_rank_share(gpu, tp):
    """Attention.forward's one-launch store + decode against store_kvcache + varlen_attention
    (two launches) on 64 sequences of the decode batch: output and caches bit for bit."""
    hq, hkv = TP_HEADS[tp]
    w = make_workload("cfg2", gpu, num_seqs=64, heads=(hq, hkv))
    kc, vc = w.k_cache.clone(), w.v_cache.clone()
    pagedkv.store_kvcache(w.k, w.v, kc, vc, w.slot_mapping)
    ref = pagedkv.varlen_attention(w.q, kc, vc, w.cu_seqlens_q, w.cu_seqlens_k, 1, w.max_seqlen_k, SCALE, True,
                                   w.block_tables, cached_prefix_keys=0)
    out = _layer(w)(w.q, w.k, w.v, w.ctx)
    torch.cuda.synchronize()
    assert bits_equal(out, ref)
    assert bits_equal(w.k_cache, kc) and bits_equal(w.v_cache, vc)


@pytest.mark.parametrize("tp", SHARES)
def test_tiny_and_ragged_decode_rows_at_rank_share(gpu, tp):
    """Decode rows of 1, 2, 3, 5, 7, 9 and 33 keys (fewer keys than a step's rows: with 1 or
    2 kv heads some DPP rows of a wavefront see no key at all) beside long ragged rows, on the
    split grid (small batch) and on the flat grid (the same rows in a batch of 128), against
    the oracle."""
    import math

    from pagedkv import workloads as W

    hq, hkv = TP_HEADS[tp]
    tiny = [1, 2, 3, 5, 7, 9, 33, 257, 1000, 4099]
    # 9 rows of at most 1000 keys: below the flat grid's 32768-key bound, the split grid
    for n, lens in ((9, tiny[:9]), (128, (tiny * 13)[:128])):
        g = torch.Generator().manual_seed(300 + tp + n)
        nb = sum(math.ceil(lk / W.BLOCK_SIZE) for lk in lens)
        tables = W._pop_tables(lens, torch.randperm(nb, generator=g).tolist())
        w = W._assemble("tiny", [(1, lk, bt) for lk, bt in zip(lens, tables)], nb, 300 + tp + n, gpu,
                        heads=(hq, hkv))
        rows, want = subset_oracle(w, list(range(n)))
        out = _layer(w)(w.q, w.k, w.v, w.ctx)
        torch.cuda.synchronize()
        assert_close_bf16(out[rows], want, f"tiny rows tp={tp} n={n}")
