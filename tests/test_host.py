"""CPU tests of the host side: the C-ABI library (loads, exports, argument checks that
return before any GPU work), the seeded workloads and their slot / block-table layout."""
import ctypes
import math
import pathlib
import re

import pytest
import torch

from pagedkv import _lib
from pagedkv.workloads import BLOCK_SIZE, HKV, HEAD_DIM, HQ, WORKLOADS, make_workload, slots_for

HEADER = pathlib.Path(__file__).resolve().parents[1] / "include" / "pagedkv.h"


def header_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(pk_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = _lib.lib()
    names = header_functions()
    assert names, "no declarations parsed from include/pagedkv.h"
    for name in names:
        assert hasattr(lib, name), f"{name} declared in pagedkv.h but not exported"
    assert set(names) == set(_lib.SIGNATURES), "ctypes signatures and header disagree"
    assert lib.pk_abi_version() == _lib.ABI_VERSION


def test_error_codes_match_header():
    text = HEADER.read_text()
    for name in ("PK_OK", "PK_ERR_INVALID_ARG", "PK_ERR_UNSUPPORTED", "PK_ERR_WORKSPACE", "PK_ERR_HIP"):
        m = re.search(rf"#define {name} \(?(-?\d+)\)?", text)
        assert m and int(m.group(1)) == getattr(_lib, name)


def _attn(lib, **kw):
    args = dict(q=None, q_row_stride=HQ * HEAD_DIM, k=None, v=None, k_row_stride=HKV * HEAD_DIM,
                v_row_stride=HKV * HEAD_DIM, k_block_stride=BLOCK_SIZE * HKV * HEAD_DIM,
                v_block_stride=BLOCK_SIZE * HKV * HEAD_DIM, block_table=None, bt_stride=0,
                block_size=BLOCK_SIZE, cu_q=None, cu_k=None, num_seqs=1, max_q=1, max_k=1,
                num_heads=HQ, num_kv_heads=HKV, head_dim=HEAD_DIM, scale=0.088, causal=1,
                out=None, out_row_stride=HQ * HEAD_DIM, ws=None, ws_bytes=0, stream=None)
    args.update(kw)
    return lib.pk_varlen_attention(*args.values())


def test_attention_argument_checks_fail_before_launch():
    lib = _lib.lib()
    assert _attn(lib, head_dim=64) == _lib.PK_ERR_UNSUPPORTED
    assert b"head_dim" in lib.pk_last_error()
    assert _attn(lib, num_heads=12, num_kv_heads=8) == _lib.PK_ERR_INVALID_ARG
    assert _attn(lib, num_heads=24, num_kv_heads=8) == _lib.PK_ERR_UNSUPPORTED  # group 3
    assert _attn(lib, num_seqs=-1) == _lib.PK_ERR_INVALID_ARG
    assert _attn(lib, num_seqs=70000) == _lib.PK_ERR_INVALID_ARG
    assert _attn(lib) == _lib.PK_ERR_INVALID_ARG  # null pointers
    assert b"null" in lib.pk_last_error()
    # nothing to do: success without touching any pointer
    assert _attn(lib, num_seqs=0) == _lib.PK_OK
    assert _attn(lib, max_q=0) == _lib.PK_OK


def test_store_argument_checks_fail_before_launch():
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x10000)
    assert lib.pk_store_kvcache(fake, 1024, fake, 1024, fake, fake, fake, 4, 1020, 0, None) == _lib.PK_ERR_INVALID_ARG
    assert lib.pk_store_kvcache(fake, 1000, fake, 1024, fake, fake, fake, 4, 1024, 0, None) == _lib.PK_ERR_INVALID_ARG
    odd = ctypes.c_void_p(0x10008)
    assert lib.pk_store_kvcache(odd, 1024, fake, 1024, fake, fake, fake, 4, 1024, 0, None) == _lib.PK_ERR_INVALID_ARG
    assert b"aligned" in lib.pk_last_error()
    assert lib.pk_store_kvcache(None, 1024, None, 1024, None, None, None, 0, 1024, 0, None) == _lib.PK_OK


def test_workspace_size_formula():
    lib = _lib.lib()
    # one split per sequence needs no workspace
    assert lib.pk_varlen_attention_workspace_bytes(8, HQ, HEAD_DIM, 1, 64) == 0
    ws = lib.pk_varlen_attention_workspace_bytes(256, HQ, HEAD_DIM, 1, 8192)
    split = 512
    units = 256 * (8192 // split) * HQ
    want = math.ceil(units * HEAD_DIM * 2 / 256) * 256 + math.ceil(units * 2 * 4 / 256) * 256
    # (bf16 outputs and fp32 (max, sum) per partial unit and head)
    assert ws == want
    # 128 sequences of <= 2048 keys take the flat decode grid: 896 runs of keys + 128
    # sequences, one partial unit each, after room for shared-prefix chunks (at most the split
    # grid's 128 x 16 units of 128-key splits), and a record of the run length and the 128
    # key-line positions (130 ints in 256-byte lines)
    ws = lib.pk_varlen_attention_workspace_bytes(128, HQ, HEAD_DIM, 1, 2048)
    units = (128 * (2048 // 128) + 128 + 896) * HQ
    want = math.ceil(units * HEAD_DIM * 2 / 256) * 256 + math.ceil(units * 2 * 4 / 256) * 256
    want += math.ceil(130 * 4 / 256) * 256
    assert ws == want


def test_workloads_are_deterministic_and_well_formed():
    for name in WORKLOADS:
        a = make_workload(name, "cpu", num_seqs=4)
        b = make_workload(name, "cpu", num_seqs=4)
        assert torch.equal(a.block_tables, b.block_tables)
        assert torch.equal(a.slot_mapping, b.slot_mapping)
        assert torch.equal(a.q.view(torch.int16), b.q.view(torch.int16))
        assert a.cu_seqlens_q.dtype == torch.int32 and a.block_tables.dtype == torch.int32
        assert int(a.cu_seqlens_q[-1]) == a.q.shape[0] == a.k.shape[0] == a.slot_mapping.numel()
        # v is a strided view into the fused qkv row, as at the Qwen3 call site
        assert a.v.stride(0) == (HQ + 2 * HKV) * HEAD_DIM and a.v.stride(1) == HEAD_DIM
        assert a.k.is_contiguous() and a.q.is_contiguous()


def test_workloads_at_tensor_parallel_shares():
    """heads=(Hq, Hkv) keeps lengths, block tables and slots, and shrinks the rows: q
    (N, Hq, D), k and v (N, Hkv, D) with v a view of the (Hq + 2 Hkv) D qkv row, caches
    (NB, BS, Hkv, D), and the algorithmic bytes scale with Hkv."""
    from pagedkv.workloads import TP_HEADS

    assert TP_HEADS == {1: (16, 8), 2: (8, 4), 4: (4, 2), 8: (2, 1)}
    for name in ("cfg2", "cfg3", "cfg4"):
        full = make_workload(name, "cpu", num_seqs=5)
        for tp, (hq, hkv) in TP_HEADS.items():
            w = make_workload(name, "cpu", num_seqs=5, heads=(hq, hkv))
            assert w.k_lens == full.k_lens and torch.equal(w.block_tables, full.block_tables)
            assert torch.equal(w.slot_mapping, full.slot_mapping)
            assert w.q.shape[1:] == (hq, HEAD_DIM) and w.k.shape[1:] == (hkv, HEAD_DIM)
            assert w.k_cache.shape[1:] == (BLOCK_SIZE, hkv, HEAD_DIM)
            assert w.v.stride(0) == (hq + 2 * hkv) * HEAD_DIM
            assert w.decode_kv_bytes() * tp == full.decode_kv_bytes()
            assert w.prefill_flops() * tp == full.prefill_flops()
    with pytest.raises(ValueError):
        make_workload("cfg2", "cpu", num_seqs=2, heads=(6, 4))


def test_shared_prefix_unique_bytes():
    """cfg4: unique bytes are the distinct keys, (2048 + sum of the suffixes) * 2R; the
    whole-block figure counts the blocks that hold them; logical bytes every sequence's keys."""
    w = make_workload("cfg4", "cpu")
    R = HKV * HEAD_DIM * 2
    suffix = [lk - 2048 for lk in w.k_lens]
    assert all(256 <= x <= 1024 for x in suffix)
    assert w.decode_unique_kv_bytes() == (2048 + sum(suffix)) * 2 * R
    blocks = 8 + sum(math.ceil(x / BLOCK_SIZE) for x in suffix)
    assert w.decode_unique_block_bytes() == blocks * BLOCK_SIZE * 2 * R
    assert w.decode_kv_bytes() == sum(w.k_lens) * 2 * R


@pytest.mark.parametrize("name", ["cfg2", "cfg3", "cfg4"])
def test_block_tables_and_slots(name):
    w = make_workload(name, "cpu", num_seqs=6)
    bt = w.block_tables.tolist()
    used = []
    for b, (lq, lk) in enumerate(zip(w.q_lens, w.k_lens)):
        nb = math.ceil(lk / BLOCK_SIZE)
        assert all(x >= 0 for x in bt[b][:nb]) and all(x == -1 for x in bt[b][nb:])
        used.append(bt[b][:nb])
    # slots of each sequence's new tokens follow the block-table walk (model_runner.py:200-210)
    slots = w.slot_mapping.tolist()
    pos = 0
    for b, (lq, lk) in enumerate(zip(w.q_lens, w.k_lens)):
        assert slots[pos:pos + lq] == slots_for(bt[b], lk - lq, lk)
        pos += lq
    flat = [x for t in used for x in t]
    if name == "cfg4":
        shared = w.meta["shared_blocks"]
        assert all(t[:len(shared)] == shared for t in used)
        private = [x for t in used for x in t[len(shared):]]
        assert len(set(private)) == len(private) and not set(private) & set(shared)
    else:
        assert len(set(flat)) == len(flat), "private blocks are never shared"
    assert len(set(slots)) == len(slots), "no two new tokens share a slot"


def test_slots_for_closed_form():
    bt = [7, 3, 9]
    assert slots_for(bt, 0, 3) == [7 * 256, 7 * 256 + 1, 7 * 256 + 2]
    assert slots_for(bt, 255, 258) == [7 * 256 + 255, 3 * 256, 3 * 256 + 1]
    assert slots_for(bt, 700, 701) == [9 * 256 + 188]


def test_algorithmic_work_formulas():
    w = make_workload("cfg3", "cpu", num_seqs=4)
    row = HKV * HEAD_DIM * 2
    assert w.decode_kv_bytes() == sum(lk * 2 * row for lq, lk in zip(w.q_lens, w.k_lens) if lq == 1)
    fl = 0
    for lq, lk in zip(w.q_lens, w.k_lens):
        if lq > 1:
            p = lk - lq
            # causal: row i sees p + i + 1 keys; QK and PV are 2 flops per MAC each
            fl += sum(2 * 2 * HQ * HEAD_DIM * (p + i + 1) for i in range(lq))
    assert w.prefill_flops() == fl
    n = w.slot_mapping.numel()
    assert w.store_bytes() == 4 * n * row + 4 * n


def test_attention_module_mirrors_reference_constructor():
    import pagedkv

    layer = pagedkv.Attention(128, 16, 8, 128 ** -0.5)
    assert (layer.head_dim, layer.num_heads, layer.num_kv_heads) == (128, 16, 8)
    assert layer.k_cache.numel() == 0 and layer.v_cache.numel() == 0
    ctx = pagedkv.Context()
    assert ctx.block_tables is None and ctx.max_seqlen_q == 0


def _prod(lib, **kw):
    fake = ctypes.c_void_p(0x10000)
    args = dict(qkv=fake, qkv_row_stride=32 * HEAD_DIM, positions=fake, cos_sin=fake, max_position=4096,
                qw=None, kw=None, eps=1e-6, n=4, hq=HQ, hkv=HKV, head_dim=HEAD_DIM, q_out=fake,
                q_out_row_stride=HQ * HEAD_DIM, k_out=None, k_out_row_stride=0, k_cache=None,
                v_cache=None, slots=None, num_slots=0, stream=None)
    args.update(kw)
    return lib.pk_qk_norm_rope_store(*args.values())


def test_producer_argument_checks_fail_before_launch():
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x10000)
    assert _prod(lib, head_dim=64) == _lib.PK_ERR_UNSUPPORTED
    assert _prod(lib, n=-1) == _lib.PK_ERR_INVALID_ARG
    assert _prod(lib, n=0) == _lib.PK_OK
    assert _prod(lib, qkv=None) == _lib.PK_ERR_INVALID_ARG
    assert _prod(lib, k_cache=fake) == _lib.PK_ERR_INVALID_ARG          # one cache only
    assert b"both caches" in lib.pk_last_error()
    assert _prod(lib, k_cache=fake, v_cache=fake) == _lib.PK_ERR_INVALID_ARG  # no slot_mapping
    assert _prod(lib, qkv_row_stride=31 * HEAD_DIM) == _lib.PK_ERR_INVALID_ARG
    assert _prod(lib, qkv=ctypes.c_void_p(0x10008)) == _lib.PK_ERR_INVALID_ARG
    assert b"aligned" in lib.pk_last_error()
    assert _prod(lib, max_position=0) == _lib.PK_ERR_INVALID_ARG
    assert _prod(lib, eps=-1.0) == _lib.PK_ERR_INVALID_ARG


# ---------------------------------------------------------------- decode-step linear ---
_FAKE = 1 << 32  # 16-byte aligned fake device addresses: these calls fail before any HIP call


def _linear(lib, x=_FAKE, xs=1024, w=2 * _FAKE, ws_=1024, rows=8, n_out=4096, k=1024, epi=0,
            out=3 * _FAKE, os_=4096, work=4 * _FAKE, work_bytes=1 << 30):
    return lib.pk_linear(x, xs, w, ws_, rows, n_out, k, epi, out, os_, work, work_bytes, None)


def test_linear_argument_checks():
    lib = _lib.lib()
    assert _linear(lib, rows=129) == _lib.PK_ERR_UNSUPPORTED            # decode batches only
    assert _linear(lib, k=1000) == _lib.PK_ERR_UNSUPPORTED              # k % 256
    assert _linear(lib, n_out=100, os_=104) == _lib.PK_ERR_UNSUPPORTED  # n_out % 32
    assert _linear(lib, epi=2) == _lib.PK_ERR_INVALID_ARG               # norm has its own entry
    assert _linear(lib, xs=1000) == _lib.PK_ERR_INVALID_ARG             # stride below k
    assert _linear(lib, x=_FAKE + 8) == _lib.PK_ERR_INVALID_ARG         # misaligned
    assert _linear(lib, w=None) == _lib.PK_ERR_INVALID_ARG
    # out overlapping x (same buffer) is refused; adjacent buffers are fine up to the launch
    assert _linear(lib, out=_FAKE + 2 * 1024 * 7) == _lib.PK_ERR_INVALID_ARG
    need = lib.pk_linear_workspace_bytes(8, 1024, 2048, 0)  # few weight tiles: K is split
    assert need > 0
    assert _linear(lib, n_out=1024, k=2048, xs=2048, ws_=2048, os_=1024, work_bytes=need - 1) == _lib.PK_ERR_WORKSPACE
    assert _linear(lib, n_out=1024, k=2048, xs=2048, ws_=2048, os_=1024, work=None) == _lib.PK_ERR_WORKSPACE
    assert _linear(lib, rows=0) == _lib.PK_OK
    rc = lib.pk_linear_add_rmsnorm(_FAKE, 2048, 2 * _FAKE, 2048, 8, 1024, 2048, None, 1024,
                                   5 * _FAKE, 1e-6, 3 * _FAKE, 1024, 6 * _FAKE, 1024,
                                   4 * _FAKE, 1 << 30, None)
    assert rc == _lib.PK_ERR_INVALID_ARG                               # residual required
    rc = lib.pk_linear_add_rmsnorm(_FAKE, 8192, 2 * _FAKE, 8192, 8, 8192, 8192, 7 * _FAKE, 8192,
                                   5 * _FAKE, 1e-6, 3 * _FAKE, 8192, 6 * _FAKE, 8192,
                                   4 * _FAKE, 1 << 30, None)
    assert rc == _lib.PK_ERR_UNSUPPORTED                               # hidden above 4096


def test_linear_workspace_sizes():
    lib = _lib.lib()
    f = lib.pk_linear_workspace_bytes
    assert f(0, 4096, 1024, 0) == 0 and f(129, 4096, 1024, 0) == 0
    for n_out, k, epi in [(4096, 1024, 0), (3072, 1024, 1), (1024, 2048, 2), (1024, 3072, 2)]:
        slab = n_out * 4 * (2 if epi == 1 else 1)  # fp32 partial sums of one row
        for rows in (1, 17, 32, 33, 64, 100, 128):
            need = f(rows, n_out, k, epi)
            if need == 0:
                assert epi != 2                   # the norm epilogue always takes the partial path
                continue
            # K splits x rows whole slabs, the split count dividing k / 256
            assert need % (rows * slab) == 0 and (k // 256) % (need // (rows * slab)) == 0
    # enough (weight tile x row group) work-groups without splitting K: no scratch, except
    # for the norm epilogue (whole rows), which keeps one slab per row
    assert f(64, 8192, 1024, 0) == 0
    assert f(128, 4096, 1024, 0) == 0
    assert f(64, 1024, 256, 2) == 64 * 1024 * 4


def test_shared_prefix_keys_from_block_reference_counts():
    from pagedkv import shared_prefix_keys
    # two sequences share their first two blocks, a third shares nothing
    assert shared_prefix_keys([[5, 6, 1], [5, 6, 2, 3], [7, 8]], 256) == 512
    # sharing that does not start at the first block gives no cached prefix
    assert shared_prefix_keys([[1, 9], [2, 9]], 256) == 0
    # padding (-1) never counts, an all-shared table stops at its end
    assert shared_prefix_keys(torch.tensor([[4, 5, -1], [4, 5, 6]], dtype=torch.int32), 16) == 32
    assert shared_prefix_keys([], 256) == 0
    # the seeded workloads: cfg4 shares its 2048-token prefix, cfg1 shares nothing
    w4 = make_workload("cfg4")
    assert w4.shared_prefix_keys == 2048 and w4.ctx.cached_prefix_keys == 2048
    assert make_workload("cfg1_decode").shared_prefix_keys == 0


def _fused(lib, **kw):
    fake = ctypes.c_void_p(0x10000)
    width = (HQ + 2 * HKV) * HEAD_DIM
    args = dict(qkv=fake, qkv_row_stride=width, positions=fake, cos_sin=fake, max_position=40960,
                q_norm=fake, k_norm=fake, eps=1e-6, k_cache=fake, v_cache=fake,
                k_row_stride=HKV * HEAD_DIM, v_row_stride=HKV * HEAD_DIM,
                k_block_stride=BLOCK_SIZE * HKV * HEAD_DIM, v_block_stride=BLOCK_SIZE * HKV * HEAD_DIM,
                slot_mapping=fake, num_slots=0, block_table=fake, bt_stride=8, block_size=BLOCK_SIZE,
                cu_q=fake, cu_k=fake, num_seqs=2, max_k=2048, num_heads=HQ, num_kv_heads=HKV,
                head_dim=HEAD_DIM, scale=0.088, out=fake, out_row_stride=HQ * HEAD_DIM,
                ws=None, ws_bytes=0, hint=0, stream=None)
    args.update(kw)
    return lib.pk_qkv_decode_attention(*args.values())


def test_fused_decode_argument_checks_fail_before_launch():
    lib = _lib.lib()
    assert _fused(lib, qkv=None) == _lib.PK_ERR_INVALID_ARG
    assert b"null" in lib.pk_last_error()
    assert _fused(lib, block_table=None) == _lib.PK_ERR_INVALID_ARG       # paged only
    assert _fused(lib, qkv_row_stride=(HQ + 2 * HKV) * HEAD_DIM - 8) == _lib.PK_ERR_INVALID_ARG
    assert _fused(lib, qkv=ctypes.c_void_p(0x10008)) == _lib.PK_ERR_INVALID_ARG
    assert b"aligned" in lib.pk_last_error()
    assert _fused(lib, max_position=0) == _lib.PK_ERR_INVALID_ARG
    assert _fused(lib, head_dim=64) == _lib.PK_ERR_UNSUPPORTED
    assert _fused(lib, num_heads=24, qkv_row_stride=(24 + 2 * HKV) * HEAD_DIM) == _lib.PK_ERR_UNSUPPORTED  # GQA 3
    assert _fused(lib, block_size=100) == _lib.PK_ERR_INVALID_ARG
    # the token row is written at block * block_stride + offset * row: contiguous caches only
    assert _fused(lib, k_block_stride=2 * BLOCK_SIZE * HKV * HEAD_DIM) == _lib.PK_ERR_INVALID_ARG
    assert b"contiguous" in lib.pk_last_error()
    assert _fused(lib, v_row_stride=2 * HKV * HEAD_DIM) == _lib.PK_ERR_INVALID_ARG
    # the split-K partials need a workspace: refused before any launch
    assert _fused(lib) == _lib.PK_ERR_WORKSPACE
    assert _fused(lib, num_seqs=-1) == _lib.PK_ERR_INVALID_ARG
    assert _fused(lib, num_seqs=0) == _lib.PK_OK



def _store_decode(lib, **kw):
    fake = ctypes.c_void_p(0x10000)
    row = HKV * HEAD_DIM
    args = dict(q=fake, q_row_stride=HQ * HEAD_DIM, key=fake, key_row_stride=row, value=fake,
                value_row_stride=4 * row, k_cache=fake, v_cache=fake, k_row_stride=row, v_row_stride=row,
                k_block_stride=BLOCK_SIZE * row, v_block_stride=BLOCK_SIZE * row, slot_mapping=fake,
                num_slots=0, block_table=fake, bt_stride=8, block_size=BLOCK_SIZE, cu_q=fake, cu_k=fake,
                num_seqs=2, max_k=2048, num_heads=HQ, num_kv_heads=HKV, head_dim=HEAD_DIM, scale=0.088,
                out=fake, out_row_stride=HQ * HEAD_DIM, ws=None, ws_bytes=0, hint=0, stream=None)
    args.update(kw)
    return lib.pk_store_decode_attention(*args.values())


def test_store_decode_argument_checks_fail_before_launch():
    """pk_store_decode_attention refuses bad arguments on the host, before any launch."""
    lib = _lib.lib()
    assert _store_decode(lib, key=None) == _lib.PK_ERR_INVALID_ARG
    assert b"null" in lib.pk_last_error()
    assert _store_decode(lib, q=None) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib, block_table=None) == _lib.PK_ERR_INVALID_ARG     # paged only
    assert _store_decode(lib, key_row_stride=HKV * HEAD_DIM - 8) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib, value_row_stride=HKV * HEAD_DIM + 4) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib, value=ctypes.c_void_p(0x10008)) == _lib.PK_ERR_INVALID_ARG
    assert b"aligned" in lib.pk_last_error()
    assert _store_decode(lib, num_slots=-1) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib, head_dim=64) == _lib.PK_ERR_UNSUPPORTED
    assert _store_decode(lib, block_size=100) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib, v_block_stride=2 * BLOCK_SIZE * HKV * HEAD_DIM) == _lib.PK_ERR_INVALID_ARG
    assert b"contiguous" in lib.pk_last_error()
    assert _store_decode(lib, k_row_stride=2 * HKV * HEAD_DIM,
                         k_block_stride=2 * BLOCK_SIZE * HKV * HEAD_DIM) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib) == _lib.PK_ERR_WORKSPACE    # split-K partials need a workspace
    assert _store_decode(lib, num_seqs=-1) == _lib.PK_ERR_INVALID_ARG
    assert _store_decode(lib, num_seqs=0) == _lib.PK_OK

def test_attention_takes_one_launch_only_over_unshared_contiguous_blocks():
    """Attention.forward's decode-step dispatch: the one-launch store + decode needs caches
    with contiguous blocks and a Context that states no block is shared
    (cached_prefix_keys == 0); anything else takes store_kvcache + varlen_attention."""
    from pagedkv.attention import _contiguous_blocks

    kc = torch.empty(4, BLOCK_SIZE, HKV, HEAD_DIM, dtype=torch.bfloat16)
    assert _contiguous_blocks(kc)
    big = torch.empty(4, 2 * BLOCK_SIZE, HKV, HEAD_DIM, dtype=torch.bfloat16)
    assert not _contiguous_blocks(big[:, :BLOCK_SIZE])           # padded blocks
    both = torch.empty(2, 4, BLOCK_SIZE, HKV, HEAD_DIM, dtype=torch.bfloat16)
    assert _contiguous_blocks(both[0]) and _contiguous_blocks(both[1])   # the runner's per-layer views


def test_no_alloc_refuses_bounds_beyond_its_scratch():
    """pk_varlen_attention_noalloc checks its launch bounds against the static scratch on the
    host: 2048 decode sequences of 8192 keys need 256 MiB of partials, above the 128 MiB, and
    are refused before any device call."""
    lib = _lib.lib()
    need = lib.pk_varlen_attention_workspace_bytes(2048, HQ, HEAD_DIM, 1, 8192)
    assert need > 128 << 20
    assert lib.pk_varlen_attention_workspace_bytes(256, HQ, HEAD_DIM, 1, 8192) <= 128 << 20
    fake = ctypes.c_void_p(0x10000)
    row = HKV * HEAD_DIM
    rc = lib.pk_varlen_attention_noalloc(fake, HQ * HEAD_DIM, fake, fake, row, row, BLOCK_SIZE * row,
                                         BLOCK_SIZE * row, fake, 32, BLOCK_SIZE, fake, fake, 2048, 1, 8192,
                                         HQ, HKV, HEAD_DIM, 0.088, 1, fake, HQ * HEAD_DIM, 0, None)
    assert rc == _lib.PK_ERR_WORKSPACE
    assert b"static scratch" in lib.pk_last_error()
    # nothing to do: success without touching the device
    assert lib.pk_varlen_attention_noalloc(None, HQ * HEAD_DIM, None, None, row, row, 0, 0, None, 0, 0, None, None,
                                           0, 1, 1, HQ, HKV, HEAD_DIM, 0.088, 1, None, HQ * HEAD_DIM, 0, None) == 0


def test_shared_prefix_argument_checks():
    """pk_varlen_attention_shared_prefix refuses a negative bound and a shared prefix in flat
    mode (no block tables to share blocks through) before any launch; 0 sequences is a no-op."""
    lib = _lib.lib()
    fake = ctypes.c_void_p(0x10000)
    row = HKV * HEAD_DIM
    base = [fake, HQ * HEAD_DIM, fake, fake, row, row, BLOCK_SIZE * row, BLOCK_SIZE * row, fake, 32, BLOCK_SIZE,
            fake, fake, 4, 1, 4096, HQ, HKV, HEAD_DIM, 0.088, 1, fake, HQ * HEAD_DIM, None, 0, 2048]
    assert lib.pk_varlen_attention_shared_prefix(*base, -1, None) == _lib.PK_ERR_INVALID_ARG
    flat = list(base)
    flat[8] = None
    assert lib.pk_varlen_attention_shared_prefix(*flat, 512, None) == _lib.PK_ERR_INVALID_ARG
    assert b"paged" in lib.pk_last_error()
    # a workspace is still required (decode partials): refused before any launch
    assert lib.pk_varlen_attention_shared_prefix(*base, 512, None) == _lib.PK_ERR_WORKSPACE
    empty = list(base)
    empty[13] = 0
    assert lib.pk_varlen_attention_shared_prefix(*empty, 512, None) == _lib.PK_OK
