"""ctypes binding of libpagedkv.so (the C-ABI declared in include/pagedkv.h).

The library is loaded on first use. If it has not been built the import of any
op fails loudly: there is no CPU or PyTorch fallback for the kernels.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libpagedkv.so")

PK_OK = 0
PK_ERR_INVALID_ARG = -1
PK_ERR_UNSUPPORTED = -2
PK_ERR_WORKSPACE = -3
PK_ERR_HIP = -4

_c_void_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_size_t = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/pagedkv.h one to one.
SIGNATURES = {
    "pk_abi_version": (ctypes.c_int, []),
    "pk_last_error": (ctypes.c_char_p, []),
    "pk_store_kvcache": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _i32, _i32, _i64,
        _c_void_p]),
    "pk_varlen_attention": (ctypes.c_int, [
        _c_void_p, _i64,                    # q, q_row_stride
        _c_void_p, _c_void_p,               # k, v
        _i64, _i64, _i64, _i64,             # k/v row strides, k/v block strides
        _c_void_p, _i32, _i32,              # block_table, its row stride, block_size
        _c_void_p, _c_void_p,               # cu_seqlens_q, cu_seqlens_k
        _i32, _i32, _i32,                   # num_seqs, max_seqlen_q, max_seqlen_k
        _i32, _i32, _i32,                   # num_heads, num_kv_heads, head_dim
        ctypes.c_float, _i32,               # softmax_scale, causal
        _c_void_p, _i64,                    # out, out_row_stride
        _c_void_p, _size_t,                 # workspace, workspace_bytes
        _c_void_p]),                        # stream
    "pk_varlen_attention_ex": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
        _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32,
        _i32, _i32, _i32, ctypes.c_float, _i32, _c_void_p, _i64, _c_void_p, _size_t,
        _i32,                               # cached_prefix_keys
        _c_void_p]),                        # stream
    "pk_varlen_attention_shared_prefix": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
        _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32,
        _i32, _i32, _i32, ctypes.c_float, _i32, _c_void_p, _i64, _c_void_p, _size_t,
        _i32, _i32,                         # cached_prefix_keys, shared_prefix_keys
        _c_void_p]),                        # stream
    "pk_varlen_attention_noalloc": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64,
        _c_void_p, _i32, _i32, _c_void_p, _c_void_p, _i32, _i32, _i32,
        _i32, _i32, _i32, ctypes.c_float, _i32, _c_void_p, _i64,
        _i32,                               # cached_prefix_keys
        _c_void_p]),                        # stream
    "pk_qkv_decode_attention": (ctypes.c_int, [
        _c_void_p, _i64,                    # qkv, qkv_row_stride
        _c_void_p, _c_void_p, _i64,         # positions, cos_sin, max_position
        _c_void_p, _c_void_p, ctypes.c_float,  # q / k norm weights, eps
        _c_void_p, _c_void_p,               # k_cache, v_cache
        _i64, _i64, _i64, _i64,             # k/v row strides, k/v block strides
        _c_void_p, _i64,                    # slot_mapping, num_slots
        _c_void_p, _i32, _i32,              # block_table, its row stride, block_size
        _c_void_p, _c_void_p,               # cu_seqlens_q, cu_seqlens_k
        _i32, _i32,                         # num_seqs, max_seqlen_k
        _i32, _i32, _i32,                   # num_heads, num_kv_heads, head_dim
        ctypes.c_float,                     # softmax_scale
        _c_void_p, _i64,                    # out, out_row_stride
        _c_void_p, _size_t,                 # workspace, its bytes
        _i32, _c_void_p]),                  # cached_prefix_keys, stream
    "pk_store_decode_attention": (ctypes.c_int, [
        _c_void_p, _i64,                    # q, q_row_stride
        _c_void_p, _i64, _c_void_p, _i64,   # key, its row stride, value, its row stride
        _c_void_p, _c_void_p,               # k_cache, v_cache
        _i64, _i64, _i64, _i64,             # k/v row strides, k/v block strides
        _c_void_p, _i64,                    # slot_mapping, num_slots
        _c_void_p, _i32, _i32,              # block_table, its row stride, block_size
        _c_void_p, _c_void_p,               # cu_seqlens_q, cu_seqlens_k
        _i32, _i32,                         # num_seqs, max_seqlen_k
        _i32, _i32, _i32,                   # num_heads, num_kv_heads, head_dim
        ctypes.c_float,                     # softmax_scale
        _c_void_p, _i64,                    # out, out_row_stride
        _c_void_p, _size_t,                 # workspace, its bytes
        _i32, _c_void_p]),                  # cached_prefix_keys, stream
    "pk_varlen_attention_workspace_bytes": (_size_t, [_i32, _i32, _i32, _i32, _i32]),
    "pk_gather_kv": (ctypes.c_int, [
        _c_void_p, _i64, _i32, _c_void_p, _i32, _c_void_p, _i32, _i32, _i32, _c_void_p,
        _c_void_p]),
    "pk_qk_norm_rope_store": (ctypes.c_int, [
        _c_void_p, _i64,                    # qkv, qkv_row_stride
        _c_void_p, _c_void_p, _i64,         # positions, cos_sin, max_position
        _c_void_p, _c_void_p, ctypes.c_float,  # q/k norm weights, eps
        _i32, _i32, _i32, _i32,             # num_tokens, num_heads, num_kv_heads, head_dim
        _c_void_p, _i64, _c_void_p, _i64,   # q_out, its row stride, k_out, its row stride
        _c_void_p, _c_void_p, _c_void_p,    # k_cache, v_cache, slot_mapping
        _i64, _c_void_p]),                  # num_slots, stream
    "pk_add_rmsnorm": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _i64, _c_void_p, ctypes.c_float, _i32, _i32,
        _c_void_p, _i64, _c_void_p, _i64, _c_void_p]),
    "pk_silu_and_mul": (ctypes.c_int, [_c_void_p, _i64, _i32, _i32, _c_void_p, _i64, _c_void_p]),
    "pk_lm_head_greedy": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _i32, _i32, _i32, _c_void_p, _c_void_p,
        _c_void_p]),
    "pk_linear_workspace_bytes": (_size_t, [_i32, _i32, _i32, _i32]),
    "pk_linear": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _i64,   # x, its row stride, weight, its row stride
        _i32, _i32, _i32, _i32,             # rows, n_out, k, epilogue
        _c_void_p, _i64,                    # out, out_row_stride
        _c_void_p, _size_t, _c_void_p]),    # workspace, workspace_bytes, stream
    "pk_linear_add_rmsnorm": (ctypes.c_int, [
        _c_void_p, _i64, _c_void_p, _i64,   # x, its row stride, weight, its row stride
        _i32, _i32, _i32,                   # rows, hidden, k
        _c_void_p, _i64, _c_void_p, ctypes.c_float,  # residual, its row stride, norm weight, eps
        _c_void_p, _i64, _c_void_p, _i64,   # out, its row stride, residual_out, its row stride
        _c_void_p, _size_t, _c_void_p]),    # workspace, workspace_bytes, stream
}

ABI_VERSION = 9

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library, with argument and return types set."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built (expected at {LIB_PATH}); run "
                    "`python -m pagedkv.build` in nano-vllm-diy_amd/ or __graft_entry__.build()")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.pk_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIB_PATH.name} ABI {handle.pk_abi_version()} != {ABI_VERSION}")
            _lib = handle
    return _lib


class PagedKVError(RuntimeError):
    """A libpagedkv entry point returned an error code."""

    def __init__(self, code: int, what: str, message: str):
        super().__init__(f"{what} failed with code {code}: {message}")
        self.code = code


def check(code: int, what: str) -> None:
    if code != PK_OK:
        raise PagedKVError(code, what, lib().pk_last_error().decode(errors="replace"))
