"""Torch-facing wrappers around the libpagedkv C-ABI.

Each wrapper checks layouts the way the reference does (src/layers/attention.py:
51-56) plus what the kernels need (bf16, 16-byte aligned rows, int32 metadata on
the same device), then calls the C entry point on the current torch stream with
raw device pointers. No wrapper synchronises or reads device memory, so all of
them can run under torch.cuda.graph capture.
"""
from __future__ import annotations

from collections import Counter

import torch

from ._lib import check, lib

# pk_varlen_attention's cache hint (include/pagedkv.h): keys below it are read with normal loads
PK_CACHED_PREFIX_KEYS_DEFAULT = 2048

_workspaces: dict[int, torch.Tensor] = {}  # device index -> workspace of graph-captured calls


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _req_i32(name: str, t: torch.Tensor, device: torch.device) -> None:
    if t.dtype != torch.int32:
        raise TypeError(f"{name} must be int32, got {t.dtype}")
    if t.device != device:
        raise ValueError(f"{name} is on {t.device}, expected {device}")


def store_kvcache(key: torch.Tensor, value: torch.Tensor, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                  check_slots: bool = False) -> None:
    """Scatter new K/V token rows into their cache slots.

    Mirrors store_kvcache (src/layers/attention.py:36-61): key/value (N, Hkv, D)
    with contiguous heads (any token row stride), caches (NB, BS, Hkv, D) with
    contiguous token rows, slot_mapping (N,) int32 where -1 skips the token.
    check_slots=True makes the kernel ignore slots outside the cache (the reference
    has no such check; attention.py:59 is commented out).
    """
    batch_seq_len, num_kv_heads, head_dim = key.shape
    row = num_kv_heads * head_dim
    # the reference's layout checks (attention.py:51-56)
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == row and v_cache.stride(1) == row
    assert slot_mapping.numel() == batch_seq_len
    if value.shape != key.shape:
        raise ValueError(f"value shape {tuple(value.shape)} != key shape {tuple(key.shape)}")
    if key.element_size() != 2 or value.dtype != key.dtype or k_cache.dtype != key.dtype or \
            v_cache.dtype != key.dtype:
        raise TypeError("key, value and caches must share one 16-bit dtype")
    if k_cache.stride(-1) != 1 or k_cache.stride(-2) != head_dim or v_cache.stride(-1) != 1 or \
            v_cache.stride(-2) != head_dim:
        raise ValueError("cache rows must be contiguous (heads x head_dim)")
    dev = key.device
    for name, t in (("value", value), ("k_cache", k_cache), ("v_cache", v_cache)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")
    _req_i32("slot_mapping", slot_mapping, dev)
    if batch_seq_len == 0:
        return
    if not slot_mapping.is_contiguous():
        raise ValueError("slot_mapping must be contiguous")
    num_slots = k_cache.numel() // row if check_slots else 0
    check(lib().pk_store_kvcache(
        key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), slot_mapping.data_ptr(),
        batch_seq_len, row, num_slots, _stream(key)), "pk_store_kvcache")


def workspace_bytes(num_seqs: int, num_heads: int, head_dim: int, max_seqlen_q: int,
                    max_seqlen_k: int) -> int:
    """Scratch bytes varlen_attention needs for these launch bounds."""
    return int(lib().pk_varlen_attention_workspace_bytes(
        num_seqs, num_heads, head_dim, max_seqlen_q, max_seqlen_k))


def _workspace(nbytes: int, device: torch.device,
               cache: dict[int, torch.Tensor] = _workspaces) -> torch.Tensor | None:
    """Scratch for one call.

    Outside graph capture every call takes its own buffer from torch's caching allocator,
    which orders reuse by stream, so calls on different streams may overlap. Under capture
    the buffer reserved ahead of it (reserve_workspace / reserve_linear_workspace) is used
    when it is large enough, so all graphs of a device share one buffer instead of holding
    one each; graphs sharing it must not replay concurrently (the rule for torch's shared
    graph memory pools). Without a large enough reservation a buffer from the capture pool
    is used.
    """
    if nbytes == 0:
        return None
    if torch.cuda.is_current_stream_capturing():
        idx = device.index if device.index is not None else torch.cuda.current_device()
        ws = cache.get(idx)
        if ws is not None and ws.numel() >= nbytes:
            return ws
    return torch.empty(nbytes, dtype=torch.uint8, device=device)


def _given_workspace(ws: torch.Tensor, nbytes: int, device: torch.device) -> torch.Tensor:
    if ws.dtype != torch.uint8 or ws.device != device or not ws.is_contiguous() or ws.numel() < nbytes:
        raise ValueError(f"workspace must be a contiguous uint8 tensor of >= {nbytes} bytes on {device}")
    return ws


def _reserve(nbytes: int, device: torch.device, cache: dict[int, torch.Tensor]) -> None:
    """Grow the per-device buffer that captured calls use (outside capture only)."""
    if nbytes == 0 or torch.cuda.is_current_stream_capturing():
        return
    idx = device.index if device.index is not None else torch.cuda.current_device()
    ws = cache.get(idx)
    if ws is None or ws.numel() < nbytes:
        cache[idx] = torch.empty(nbytes, dtype=torch.uint8, device=device)


def reserve_workspace(num_seqs: int, num_heads: int, head_dim: int, max_seqlen_q: int,
                      max_seqlen_k: int, device: torch.device | str = "cuda") -> None:
    """Reserve the workspace that graph-captured attention calls use (call before capture)."""
    _reserve(workspace_bytes(num_seqs, num_heads, head_dim, max_seqlen_q, max_seqlen_k),
             torch.device(device), _workspaces)


def varlen_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor,
                     max_seqlen_q: int, max_seqlen_k: int,
                     softmax_scale: float | None = None, causal: bool = True,
                     block_table: torch.Tensor | None = None,
                     out: torch.Tensor | None = None,
                     cached_prefix_keys: int | None = None,
                     workspace: torch.Tensor | None = None,
                     shared_prefix_keys: int | None = None) -> torch.Tensor:
    """Causal varlen attention with optional paged K/V; bf16 in and out.

    Same arguments and meaning as the flash_attn_varlen_func call of the reference
    (src/layers/attention.py:95-104): q (Nq, Hq, D); k, v flat (Nk, Hkv, D) when
    block_table is None, else caches (NB, BS, Hkv, D) read through block_table
    (S, W) int32; per-sequence lengths from cu_seqlens_q / cu_seqlens_k (S + 1,)
    int32; bottom-right-aligned causal mask; GQA h -> h // (Hq / Hkv).
    Returns out (Nq, Hq, D) bf16.

    cached_prefix_keys (an addition, results unchanged): decode keys from this position on
    are read with streaming loads, earlier ones kept in cache -- the longest prefix the
    caller's block manager may share between sequences (0: none shared, -1: cache every
    read). None keeps the library default (PK_CACHED_PREFIX_KEYS_DEFAULT = 2048).
    workspace: caller-owned uint8 scratch of at least workspace_bytes(...) bytes (as the
    C-ABI takes it); None takes one per call (or the reserved one under graph capture).
    shared_prefix_keys (an addition, paged mode): decode keys below it are computed once per
    shared cache block, the query rows of every sequence that holds the block in one MFMA
    tile (pk_varlen_attention_shared_prefix); results stay within the attention tolerance.
    None or 0: off.
    """
    nq, num_heads, head_dim = q.shape
    dev = q.device
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("q, k and v must be bfloat16")
    if q.stride(-1) != 1 or q.stride(1) != head_dim:
        raise ValueError("q must have contiguous heads (stride(1) == head_dim, stride(2) == 1)")
    for name, t in (("k", k), ("v", v), ("cu_seqlens_k", cu_seqlens_k)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")
    _req_i32("cu_seqlens_q", cu_seqlens_q, dev)
    _req_i32("cu_seqlens_k", cu_seqlens_k, dev)
    if not (cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous()):
        raise ValueError("cu_seqlens_q / cu_seqlens_k must be contiguous")
    num_seqs = cu_seqlens_q.numel() - 1
    if cu_seqlens_k.numel() != num_seqs + 1:
        raise ValueError("cu_seqlens_q and cu_seqlens_k must have the same length")
    if block_table is None:
        if k.dim() != 3 or v.shape != k.shape:
            raise ValueError("flat mode expects k, v of shape (Nk, Hkv, D)")
        num_kv_heads = k.shape[1]
        k_row, v_row, k_blk, v_blk = k.stride(0), v.stride(0), 0, 0
        bt_ptr, bt_stride, block_size = 0, 0, 0
        kv_inner = (k.stride(1), k.stride(2), v.stride(1), v.stride(2))
    else:
        if k.dim() != 4 or v.shape != k.shape:
            raise ValueError("paged mode expects caches of shape (NB, BS, Hkv, D)")
        _req_i32("block_table", block_table, dev)
        if block_table.dim() != 2 or block_table.stride(1) != 1:
            raise ValueError("block_table must be (S, W) with contiguous rows")
        if block_table.shape[0] < num_seqs:
            raise ValueError("block_table has fewer rows than sequences")
        num_kv_heads = k.shape[2]
        block_size = k.shape[1]
        k_row, v_row, k_blk, v_blk = k.stride(1), v.stride(1), k.stride(0), v.stride(0)
        bt_ptr, bt_stride = block_table.data_ptr(), block_table.stride(0)
        kv_inner = (k.stride(2), k.stride(3), v.stride(2), v.stride(3))
    if k.shape[-1] != head_dim:
        raise ValueError(f"k head_dim {k.shape[-1]} != q head_dim {head_dim}")
    if kv_inner != (head_dim, 1, head_dim, 1):
        raise ValueError("k and v must have contiguous heads within a token row")
    if out is None:
        out = torch.empty(nq, num_heads, head_dim, dtype=torch.bfloat16, device=dev)
    elif out.shape != q.shape or out.dtype != torch.bfloat16 or out.stride(-1) != 1 or \
            out.stride(1) != head_dim:
        raise ValueError("out must be (Nq, Hq, D) bf16 with contiguous heads")
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    nbytes = workspace_bytes(num_seqs, num_heads, head_dim, max_seqlen_q, max_seqlen_k)
    ws = _workspace(nbytes, dev) if workspace is None else _given_workspace(workspace, nbytes, dev)
    args = (q.data_ptr(), q.stride(0), k.data_ptr(), v.data_ptr(),
            k_row, v_row, k_blk, v_blk,
            bt_ptr, bt_stride, block_size,
            cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(),
            num_seqs, int(max_seqlen_q), int(max_seqlen_k),
            num_heads, num_kv_heads, head_dim,
            scale, 1 if causal else 0,
            out.data_ptr(), out.stride(0),
            ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0)
    if shared_prefix_keys and block_table is not None:
        hint = PK_CACHED_PREFIX_KEYS_DEFAULT if cached_prefix_keys is None else int(cached_prefix_keys)
        check(lib().pk_varlen_attention_shared_prefix(*args, hint, int(shared_prefix_keys), _stream(q)),
              "pk_varlen_attention_shared_prefix")
    elif cached_prefix_keys is None:
        check(lib().pk_varlen_attention(*args, _stream(q)), "pk_varlen_attention")
    else:
        check(lib().pk_varlen_attention_ex(*args, int(cached_prefix_keys), _stream(q)), "pk_varlen_attention_ex")
    return out


def qkv_decode_attention(qkv: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor,
                         num_heads: int, num_kv_heads: int, head_dim: int,
                         q_norm_weight: torch.Tensor | None, k_norm_weight: torch.Tensor | None, eps: float,
                         k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                         cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_k: int,
                         softmax_scale: float | None, block_table: torch.Tensor,
                         out: torch.Tensor | None = None, cached_prefix_keys: int | None = None,
                         check_slots: bool = False, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """One decode step of an attention layer from the fused qkv projection: q/k RMSNorm +
    RoPE, the new K/V rows stored at slot_mapping and paged decode attention, in one launch.
    Bit-identical to qk_norm_rope_store(qkv, ..., k_cache, v_cache, slot_mapping) followed by
    varlen_attention(q, k_cache, v_cache, ..., max_seqlen_q=1, block_table=...)
    (src/models/qwen3.py:80-89 and src/layers/attention.py:87-104 on a decode step). Every
    sequence has one query row (cu_seqlens_q = arange, graph padding rows aside) and
    slot_mapping[i] is the cache slot of sequence i's last key. Returns out (S, Hq, D) bf16.
    """
    if qkv.dim() != 2 or qkv.dtype != torch.bfloat16 or qkv.stride(1) != 1:
        raise ValueError("qkv must be (S, (Hq + 2 Hkv) * D) bf16 with contiguous rows")
    n = qkv.shape[0]
    dev = qkv.device
    if qkv.shape[1] != (num_heads + 2 * num_kv_heads) * head_dim:
        raise ValueError(f"qkv width {qkv.shape[1]} != (Hq + 2 Hkv) * D")
    if positions.dtype != torch.int64 or positions.device != dev or positions.numel() != n or \
            not positions.is_contiguous():
        raise ValueError("positions must be a contiguous (S,) int64 tensor on the qkv device")
    if cos_sin.dim() == 3:
        cos_sin = cos_sin.squeeze(1)
    if cos_sin.dtype != torch.float32 or cos_sin.shape[-1] != head_dim or \
            not cos_sin.is_contiguous() or cos_sin.device != dev:
        raise ValueError("cos_sin must be a contiguous (P, D) float32 table on the qkv device")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w is not None and (w.dtype != torch.bfloat16 or w.numel() != head_dim or
                              not w.is_contiguous() or w.device != dev):
            raise ValueError(f"{name} must be a contiguous ({head_dim},) bf16 tensor on the qkv device")
    _req_i32("slot_mapping", slot_mapping, dev)
    _req_i32("cu_seqlens_q", cu_seqlens_q, dev)
    _req_i32("cu_seqlens_k", cu_seqlens_k, dev)
    _req_i32("block_table", block_table, dev)
    num_seqs = cu_seqlens_q.numel() - 1
    if slot_mapping.numel() != n or not slot_mapping.is_contiguous() or num_seqs != n or \
            cu_seqlens_k.numel() != n + 1 or not (cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous()):
        raise ValueError("a decode step has one qkv row, one slot and one (q, k) length pair per sequence")
    if block_table.dim() != 2 or block_table.stride(1) != 1 or block_table.shape[0] < num_seqs:
        raise ValueError("block_table must be (S, W) with contiguous rows")
    row = num_kv_heads * head_dim
    for c in (k_cache, v_cache):
        if c.dim() != 4 or c.dtype != torch.bfloat16 or c.device != dev or c.stride(-1) != 1 or \
                c.stride(-2) != head_dim or c.shape[-2] != num_kv_heads or c.shape[-1] != head_dim:
            raise ValueError("caches must be (NB, BS, Hkv, D) bf16 with contiguous heads")
        if c.stride(1) != row or c.stride(0) != c.shape[1] * row:
            raise ValueError("qkv_decode_attention needs caches with contiguous rows and blocks")
    if v_cache.shape != k_cache.shape:
        raise ValueError("k_cache and v_cache shapes differ")
    num_slots = k_cache.shape[0] * k_cache.shape[1] if check_slots else 0
    if out is None:
        out = torch.empty(n, num_heads, head_dim, dtype=torch.bfloat16, device=dev)
    elif out.shape != (n, num_heads, head_dim) or out.dtype != torch.bfloat16 or out.stride(-1) != 1 or \
            out.stride(1) != head_dim:
        raise ValueError("out must be (S, Hq, D) bf16 with contiguous heads")
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    nbytes = workspace_bytes(num_seqs, num_heads, head_dim, 1, max_seqlen_k)
    ws = _workspace(nbytes, dev) if workspace is None else _given_workspace(workspace, nbytes, dev)
    hint = PK_CACHED_PREFIX_KEYS_DEFAULT if cached_prefix_keys is None else int(cached_prefix_keys)
    ptr = lambda t: t.data_ptr() if t is not None else 0  # noqa: E731
    check(lib().pk_qkv_decode_attention(
        qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0],
        ptr(q_norm_weight), ptr(k_norm_weight), float(eps), k_cache.data_ptr(), v_cache.data_ptr(),
        k_cache.stride(1), v_cache.stride(1), k_cache.stride(0), v_cache.stride(0),
        slot_mapping.data_ptr(), num_slots, block_table.data_ptr(), block_table.stride(0), k_cache.shape[1],
        cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_seqs, int(max_seqlen_k),
        num_heads, num_kv_heads, head_dim, scale, out.data_ptr(), out.stride(0),
        ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0, hint, _stream(qkv)),
        "pk_qkv_decode_attention")
    return out


def store_decode_attention(q: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                           k_cache: torch.Tensor, v_cache: torch.Tensor, slot_mapping: torch.Tensor,
                           cu_seqlens_q: torch.Tensor, cu_seqlens_k: torch.Tensor, max_seqlen_k: int,
                           softmax_scale: float | None, block_table: torch.Tensor,
                           out: torch.Tensor | None = None, cached_prefix_keys: int | None = None,
                           check_slots: bool = False, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """Attention.forward on a decode step (src/layers/attention.py:87-104) in one launch:
    the store of store_kvcache (same layout checks, attention.py:51-56) followed by paged
    decode attention; output and caches are bit-identical to store_kvcache + varlen_attention.
    Row i of q, key and value is sequence i's token (one query row per sequence) and
    slot_mapping[i] is the cache slot of sequence i's last key, in a cache block that no other
    sequence of the batch reads (the row is written while other work-groups read the cache;
    with shared prefix blocks call store_kvcache + varlen_attention instead). The caches'
    rows and blocks must be contiguous. Returns out (S, Hq, D) bf16.
    """
    n, num_heads, head_dim = q.shape
    num_kv_heads = key.shape[1]
    row = num_kv_heads * head_dim
    assert key.stride(-1) == 1 and value.stride(-1) == 1
    assert key.stride(1) == head_dim and value.stride(1) == head_dim
    assert k_cache.stride(1) == row and v_cache.stride(1) == row
    assert slot_mapping.numel() == key.shape[0]
    dev = q.device
    if q.dtype != torch.bfloat16 or key.dtype != torch.bfloat16 or value.dtype != torch.bfloat16 or \
            k_cache.dtype != torch.bfloat16 or v_cache.dtype != torch.bfloat16:
        raise TypeError("q, key, value and caches must be bfloat16")
    if value.shape != key.shape or key.shape[0] != n or key.shape[2] != head_dim:
        raise ValueError("q (S, Hq, D), key / value (S, Hkv, D): one token per sequence")
    if q.stride(-1) != 1 or q.stride(1) != head_dim:
        raise ValueError("q must have contiguous heads")
    for c in (k_cache, v_cache):
        if c.dim() != 4 or c.device != dev or c.stride(-1) != 1 or c.stride(-2) != head_dim or \
                c.shape[-2] != num_kv_heads:
            raise ValueError("caches must be (NB, BS, Hkv, D) bf16 with contiguous heads")
        if c.stride(0) != c.shape[1] * row:
            # the one launch writes the token row at block * block_stride + offset * row, where
            # store_kvcache writes slot * row: the same place only for contiguous blocks
            raise ValueError("store_decode_attention needs caches with contiguous blocks "
                             "(stride(0) == block_size * Hkv * D); use store_kvcache + varlen_attention")
    for name, t in (("key", key), ("value", value)):
        if t.device != dev:
            raise ValueError(f"{name} is on {t.device}, expected {dev}")
    _req_i32("slot_mapping", slot_mapping, dev)
    _req_i32("cu_seqlens_q", cu_seqlens_q, dev)
    _req_i32("cu_seqlens_k", cu_seqlens_k, dev)
    _req_i32("block_table", block_table, dev)
    num_seqs = cu_seqlens_q.numel() - 1
    if num_seqs != n or cu_seqlens_k.numel() != n + 1 or not slot_mapping.is_contiguous() or \
            not (cu_seqlens_q.is_contiguous() and cu_seqlens_k.is_contiguous()):
        raise ValueError("a decode step has one row, one slot and one (q, k) length pair per sequence")
    if block_table.dim() != 2 or block_table.stride(1) != 1 or block_table.shape[0] < num_seqs:
        raise ValueError("block_table must be (S, W) with contiguous rows")
    num_slots = k_cache.shape[0] * k_cache.shape[1] if check_slots else 0
    if out is None:
        out = torch.empty(n, num_heads, head_dim, dtype=torch.bfloat16, device=dev)
    elif out.shape != q.shape or out.dtype != torch.bfloat16 or out.stride(-1) != 1 or out.stride(1) != head_dim:
        raise ValueError("out must be (S, Hq, D) bf16 with contiguous heads")
    scale = head_dim ** -0.5 if softmax_scale is None else float(softmax_scale)
    nbytes = workspace_bytes(num_seqs, num_heads, head_dim, 1, max_seqlen_k)
    ws = _workspace(nbytes, dev) if workspace is None else _given_workspace(workspace, nbytes, dev)
    hint = PK_CACHED_PREFIX_KEYS_DEFAULT if cached_prefix_keys is None else int(cached_prefix_keys)
    check(lib().pk_store_decode_attention(
        q.data_ptr(), q.stride(0), key.data_ptr(), key.stride(0), value.data_ptr(), value.stride(0),
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(1), v_cache.stride(1), k_cache.stride(0),
        v_cache.stride(0), slot_mapping.data_ptr(), num_slots, block_table.data_ptr(), block_table.stride(0),
        k_cache.shape[1], cu_seqlens_q.data_ptr(), cu_seqlens_k.data_ptr(), num_seqs, int(max_seqlen_k),
        num_heads, num_kv_heads, head_dim, scale, out.data_ptr(), out.stride(0),
        ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0, hint, _stream(q)),
        "pk_store_decode_attention")
    return out


def shared_prefix_keys(block_tables, block_size: int) -> int:
    """The cached_prefix_keys value for a batch: the longest run of leading blocks that
    some sequence shares with another (block reference count > 1, the count the
    reference's block manager keeps, block_manager.py:141,149), in keys. Only leading
    blocks can be shared (prefix hashes chain from the sequence start,
    block_manager.py:96-181), so keys past this run are read once per step and can stream.
    block_tables: per-sequence lists of block ids, or an (S, W) int tensor, -1 padded."""
    if isinstance(block_tables, torch.Tensor):
        block_tables = block_tables.cpu().tolist()
    refs = Counter(b for row in block_tables for b in set(row) if b >= 0)
    best = 0
    for row in block_tables:
        n = 0
        while n < len(row) and row[n] >= 0 and refs[row[n]] > 1:
            n += 1
        best = max(best, n)
    return best * block_size


def gather_kv(cache: torch.Tensor, block_table: torch.Tensor, cu_seqlens_k: torch.Tensor,
              max_seqlen_k: int, total_k: int | None = None) -> torch.Tensor:
    """Flat (sum Lk, Hkv, D) copy of each sequence's cache rows via its block table.

    total_k (= cu_seqlens_k[-1]) sizes the output; pass it to avoid a device read.
    """
    dev = cache.device
    _req_i32("block_table", block_table, dev)
    _req_i32("cu_seqlens_k", cu_seqlens_k, dev)
    if cache.dim() != 4 or cache.stride(-1) != 1 or cache.stride(-2) != cache.shape[-1] or \
            cache.stride(1) != cache.shape[-1] * cache.shape[-2]:
        raise ValueError("cache must be (NB, BS, Hkv, D) with contiguous token rows")
    if block_table.dim() != 2 or block_table.stride(1) != 1:
        raise ValueError("block_table must be (S, W) with contiguous rows")
    num_seqs = cu_seqlens_k.numel() - 1
    if total_k is None:
        total_k = int(cu_seqlens_k[-1].item())
    row = cache.shape[2] * cache.shape[3]
    dst = torch.empty(total_k, cache.shape[2], cache.shape[3], dtype=cache.dtype, device=dev)
    check(lib().pk_gather_kv(
        cache.data_ptr(), cache.stride(0), cache.shape[1], block_table.data_ptr(),
        block_table.stride(0), cu_seqlens_k.data_ptr(), num_seqs, int(max_seqlen_k), row,
        dst.data_ptr(), _stream(cache)), "pk_gather_kv")
    return dst


def rope_cos_sin(max_position: int, head_dim: int, base: float = 1000000.0,
                 device: torch.device | str = "cuda") -> torch.Tensor:
    """The (max_position, head_dim) fp32 RoPE table [cos | sin] of position x frequency.

    Built the way build_rope_cos_sin does it (src/layers/pos_embedding.py:6-18), as data
    for qk_norm_rope_store; the reference's (P, 1, D) view is accepted there as well.
    """
    inv_freq = 1.0 / (base ** (torch.arange(0, head_dim, 2, device=device).float() / head_dim))
    pos = torch.arange(max_position, dtype=torch.float, device=device)
    freqs = torch.outer(pos, inv_freq)
    return torch.cat((freqs.cos(), freqs.sin()), dim=-1).contiguous()


def qk_norm_rope_store(qkv: torch.Tensor, positions: torch.Tensor, cos_sin: torch.Tensor,
                       num_heads: int, num_kv_heads: int, head_dim: int = 128,
                       q_norm_weight: torch.Tensor | None = None,
                       k_norm_weight: torch.Tensor | None = None, eps: float = 1e-6,
                       k_cache: torch.Tensor | None = None, v_cache: torch.Tensor | None = None,
                       slot_mapping: torch.Tensor | None = None, return_k: bool = False,
                       check_slots: bool = False, q_out: torch.Tensor | None = None,
                       k_out: torch.Tensor | None = None):
    """Fused q/k RMSNorm + RoPE + K/V cache store from the fused qkv projection output.

    Replaces, in one kernel, the sequence of Qwen3Attention.forward
    (src/models/qwen3.py:80-89): split of qkv, q_norm / k_norm (layernorm.py:11-16),
    rotary_emb (pos_embedding.py:30-48) and the store inside Attention.forward
    (attention.py:87-88). qkv (N, (Hq + 2 Hkv) D) bf16; positions (N,) int64;
    cos_sin from rope_cos_sin. With caches given, K (normed, rotated) and raw V rows go
    to slot_mapping's slots (-1 skips). Returns (q (N, Hq, D), k (N, Hkv, D) or None);
    k is produced when return_k (attention over fresh keys needs it).
    """
    if qkv.dim() != 2 or qkv.dtype != torch.bfloat16 or qkv.stride(1) != 1:
        raise ValueError("qkv must be (N, (Hq + 2 Hkv) * D) bf16 with contiguous rows")
    n = qkv.shape[0]
    dev = qkv.device
    if qkv.shape[1] != (num_heads + 2 * num_kv_heads) * head_dim:
        raise ValueError(f"qkv width {qkv.shape[1]} != (Hq + 2 Hkv) * D")
    if positions.dtype != torch.int64 or positions.device != dev or positions.numel() != n or \
            not positions.is_contiguous():
        raise ValueError("positions must be a contiguous (N,) int64 tensor on the qkv device")
    if cos_sin.dim() == 3:
        cos_sin = cos_sin.squeeze(1)
    if cos_sin.dtype != torch.float32 or cos_sin.shape[-1] != head_dim or \
            not cos_sin.is_contiguous() or cos_sin.device != dev:
        raise ValueError("cos_sin must be a contiguous (P, D) float32 table on the qkv device")
    for name, w in (("q_norm_weight", q_norm_weight), ("k_norm_weight", k_norm_weight)):
        if w is not None and (w.dtype != torch.bfloat16 or w.numel() != head_dim or
                              not w.is_contiguous() or w.device != dev):
            raise ValueError(f"{name} must be a contiguous ({head_dim},) bf16 tensor on the qkv device")
    if (k_cache is None) != (v_cache is None):
        raise ValueError("pass both caches or neither")
    row = num_kv_heads * head_dim
    num_slots = 0
    if k_cache is not None:
        if slot_mapping is None:
            raise ValueError("slot_mapping is required with caches")
        _req_i32("slot_mapping", slot_mapping, dev)
        assert slot_mapping.numel() == n and slot_mapping.is_contiguous()
        for c in (k_cache, v_cache):
            if c.dtype != torch.bfloat16 or c.device != dev or c.stride(-1) != 1 or \
                    c.stride(-2) != head_dim or c.stride(1) != row or c.shape[-2] != num_kv_heads:
                raise ValueError("caches must be (NB, BS, Hkv, D) bf16 with contiguous token rows")
        if check_slots:
            num_slots = k_cache.numel() // row
    if q_out is None:
        q_out = torch.empty(n, num_heads, head_dim, dtype=torch.bfloat16, device=dev)
    elif q_out.shape != (n, num_heads, head_dim) or q_out.stride(1) != head_dim or q_out.stride(2) != 1:
        raise ValueError("q_out must be (N, Hq, D) with contiguous heads")
    if return_k and k_out is None:
        k_out = torch.empty(n, num_kv_heads, head_dim, dtype=torch.bfloat16, device=dev)
    if k_out is not None and (k_out.shape != (n, num_kv_heads, head_dim) or
                              k_out.stride(1) != head_dim or k_out.stride(2) != 1):
        raise ValueError("k_out must be (N, Hkv, D) with contiguous heads")
    ptr = lambda t: t.data_ptr() if t is not None else 0  # noqa: E731
    check(lib().pk_qk_norm_rope_store(
        qkv.data_ptr(), qkv.stride(0), positions.data_ptr(), cos_sin.data_ptr(), cos_sin.shape[0],
        ptr(q_norm_weight), ptr(k_norm_weight), float(eps), n, num_heads, num_kv_heads, head_dim,
        q_out.data_ptr(), q_out.stride(0), ptr(k_out), k_out.stride(0) if k_out is not None else 0,
        ptr(k_cache), ptr(v_cache), ptr(slot_mapping), num_slots, _stream(qkv)),
        "pk_qk_norm_rope_store")
    return q_out, k_out


def _rows2d(name: str, t: torch.Tensor) -> None:
    if t.dim() != 2 or t.dtype != torch.bfloat16 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D bf16 tensor with contiguous rows")


def add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float,
                residual: torch.Tensor | None = None, out: torch.Tensor | None = None):
    """RMSNorm.forward (src/layers/layernorm.py:30-39) with the residual add fused.

    residual None: returns bf16(w * x * rsqrt(mean(x^2) + eps)). Otherwise returns
    (normed, new_residual) with new_residual = bf16(x + residual), as residual_forward.
    """
    _rows2d("x", x)
    rows, hidden = x.shape
    if weight.dtype != torch.bfloat16 or weight.numel() != hidden or not weight.is_contiguous():
        raise ValueError("weight must be a contiguous (hidden,) bf16 tensor")
    if out is None:
        out = torch.empty_like(x)
    res_out = None
    if residual is not None:
        _rows2d("residual", residual)
        if residual.shape != x.shape:
            raise ValueError("residual must match x")
        res_out = torch.empty_like(residual)
    check(lib().pk_add_rmsnorm(
        x.data_ptr(), x.stride(0), residual.data_ptr() if residual is not None else 0,
        residual.stride(0) if residual is not None else 0, weight.data_ptr(), float(eps), rows,
        hidden, out.data_ptr(), out.stride(0), res_out.data_ptr() if res_out is not None else 0,
        res_out.stride(0) if res_out is not None else 0, _stream(x)), "pk_add_rmsnorm")
    return out if residual is None else (out, res_out)


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """SiluAndMul.forward (src/layers/activation.py:6-10): silu(first half) * second half."""
    _rows2d("x", x)
    rows, width = x.shape
    inter = width // 2
    if out is None:
        out = torch.empty(rows, inter, dtype=torch.bfloat16, device=x.device)
    check(lib().pk_silu_and_mul(x.data_ptr(), x.stride(0), rows, inter, out.data_ptr(),
                                out.stride(0), _stream(x)), "pk_silu_and_mul")
    return out


_lm_keys: dict[int, torch.Tensor] = {}


def lm_head_greedy(hidden_states: torch.Tensor, weight: torch.Tensor,
                   cu_seqlens_q: torch.Tensor | None = None, num_rows: int | None = None,
                   out: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy next tokens from ParallelLMHead.forward's logits (src/layers/llm_head.py:60-64).

    With cu_seqlens_q, row m is the last token of sequence m (the prefill selection of
    llm_head.py:61-63) and num_rows defaults to len(cu_seqlens_q) - 1; otherwise every row.
    Returns int32 token ids: argmax over the bf16-rounded logits, lowest id on ties.
    """
    _rows2d("hidden_states", hidden_states)
    _rows2d("weight", weight)
    hidden = hidden_states.shape[1]
    if weight.shape[1] != hidden:
        raise ValueError("weight must be (vocab, hidden)")
    dev = hidden_states.device
    if cu_seqlens_q is not None:
        _req_i32("cu_seqlens_q", cu_seqlens_q, dev)
        rows = cu_seqlens_q.numel() - 1 if num_rows is None else num_rows
    else:
        rows = hidden_states.shape[0] if num_rows is None else num_rows
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    keys = _lm_keys.get(idx)
    if keys is None or keys.numel() < rows:
        keys = torch.empty(max(rows, 512), dtype=torch.int64, device=dev)
        if not torch.cuda.is_current_stream_capturing():
            _lm_keys[idx] = keys
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=dev)
    check(lib().pk_lm_head_greedy(
        hidden_states.data_ptr(), hidden_states.stride(0),
        cu_seqlens_q.data_ptr() if cu_seqlens_q is not None else 0, weight.data_ptr(),
        weight.stride(0), rows, weight.shape[0], hidden, keys.data_ptr(), out.data_ptr(),
        _stream(hidden_states)), "pk_lm_head_greedy")
    return out


# ----------------------------------------------------------- decode-step linear layers ---
LINEAR_MAX_ROWS = 128
LINEAR_STORE, LINEAR_SILU_MUL, LINEAR_ADD_RMSNORM = 0, 1, 2
_lin_workspaces: dict[int, torch.Tensor] = {}  # device index -> scratch of graph-captured calls


def linear_workspace_bytes(rows: int, n_out: int, k: int, epilogue: int = LINEAR_STORE) -> int:
    """Scratch bytes of one decode-step linear call (0 when it needs none)."""
    return int(lib().pk_linear_workspace_bytes(rows, n_out, k, epilogue))


def reserve_linear_workspace(nbytes: int, device: torch.device | str = "cuda") -> None:
    """Reserve the scratch that graph-captured linear-layer calls use (call before capture)."""
    _reserve(nbytes, torch.device(device), _lin_workspaces)


def _linear_args(x: torch.Tensor, weight: torch.Tensor, rows_per_out: int):
    _rows2d("x", x)
    _rows2d("weight", weight)
    rows, k = x.shape
    if weight.shape[1] != k or weight.shape[0] % rows_per_out:
        raise ValueError(f"weight {tuple(weight.shape)} does not match x {tuple(x.shape)}")
    if rows > LINEAR_MAX_ROWS:
        raise ValueError(f"decode-step linear layers take at most {LINEAR_MAX_ROWS} rows, got {rows}")
    return rows, k, weight.shape[0] // rows_per_out


def _linear_call(x, weight, rows, k, n_out, epilogue, out, workspace=None):
    nbytes = linear_workspace_bytes(rows, n_out, k, epilogue)
    ws = _workspace(nbytes, x.device, _lin_workspaces) if workspace is None else \
        _given_workspace(workspace, nbytes, x.device)
    check(lib().pk_linear(
        x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, n_out, k, epilogue,
        out.data_ptr(), out.stride(0), ws.data_ptr() if ws is not None else 0, nbytes,
        _stream(x)), "pk_linear")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
           workspace: torch.Tensor | None = None) -> torch.Tensor:
    """F.linear(x, weight) of a decode step (src/layers/linear.py:74-75, :169-170): bf16
    (rows <= 128, k) x (n_out, k)^T with fp32 accumulation, rounded to bf16. workspace:
    optional caller-owned uint8 scratch of linear_workspace_bytes(...) bytes."""
    rows, k, n_out = _linear_args(x, weight, 1)
    if out is None:
        out = torch.empty(rows, n_out, dtype=torch.bfloat16, device=x.device)
    return _linear_call(x, weight, rows, k, n_out, LINEAR_STORE, out, workspace)


def linear_silu_mul(x: torch.Tensor, weight: torch.Tensor, out: torch.Tensor | None = None,
                    workspace: torch.Tensor | None = None) -> torch.Tensor:
    """SiluAndMul(F.linear(x, weight)) for the merged gate/up weight (2 inter, k)
    (qwen3.py:120-121): gate and up outputs are rounded to bf16, then silu(g) * u in fp32."""
    rows, k, inter = _linear_args(x, weight, 2)
    if out is None:
        out = torch.empty(rows, inter, dtype=torch.bfloat16, device=x.device)
    return _linear_call(x, weight, rows, k, inter, LINEAR_SILU_MUL, out, workspace)


def linear_add_rmsnorm(x: torch.Tensor, weight: torch.Tensor, residual: torch.Tensor,
                       norm_weight: torch.Tensor, eps: float, out: torch.Tensor | None = None,
                       residual_out: torch.Tensor | None = None):
    """RMSNorm.residual_forward (layernorm.py:18-28) of h = F.linear(x, weight) and residual:
    returns (bf16(w * s * rsqrt(mean(s^2) + eps)), bf16(s)) with s = h + residual in fp32.
    residual_out may be residual itself (updated in place)."""
    rows, k, hidden = _linear_args(x, weight, 1)
    _rows2d("residual", residual)
    if residual.shape != (rows, hidden):
        raise ValueError(f"residual must be ({rows}, {hidden})")
    if norm_weight.dtype != torch.bfloat16 or norm_weight.numel() != hidden or not norm_weight.is_contiguous():
        raise ValueError("norm_weight must be a contiguous (hidden,) bf16 tensor")
    if out is None:
        out = torch.empty(rows, hidden, dtype=torch.bfloat16, device=x.device)
    if residual_out is None:
        residual_out = torch.empty_like(residual)
    nbytes = linear_workspace_bytes(rows, hidden, k, LINEAR_ADD_RMSNORM)
    ws = _workspace(nbytes, x.device, _lin_workspaces)
    check(lib().pk_linear_add_rmsnorm(
        x.data_ptr(), x.stride(0), weight.data_ptr(), weight.stride(0), rows, hidden, k,
        residual.data_ptr(), residual.stride(0), norm_weight.data_ptr(), float(eps),
        out.data_ptr(), out.stride(0), residual_out.data_ptr(), residual_out.stride(0),
        ws.data_ptr() if ws is not None else 0, nbytes, _stream(x)), "pk_linear_add_rmsnorm")
    return out, residual_out
