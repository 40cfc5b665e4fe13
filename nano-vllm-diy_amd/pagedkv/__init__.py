"""pagedkv -- MI355X (gfx950) paged-KV attention path for a nano-vLLM-style engine.

Public surface (mirrors the reference's src/layers/attention.py and
src/utils/context.py):
    Attention, store_kvcache, Context,
    varlen_attention (flash_attn_varlen_func semantics), gather_kv,
    workspace_bytes, reserve_workspace,
    qk_norm_rope_store + rope_cos_sin (the fused q/k norm, RoPE and cache store of
    src/models/qwen3.py:80-89),
    add_rmsnorm, silu_and_mul, lm_head_greedy, and the decode-step linear layers linear,
    linear_silu_mul, linear_add_rmsnorm (the serving loop's other kernels), and
    shared_prefix_keys (the decode cache hint a batch's block tables imply), and
    qkv_decode_attention (producer + decode attention of a decode step in one launch).
"""
from .attention import Attention, store_kvcache  # noqa: F401
from .context import Context  # noqa: F401
from .ops import (add_rmsnorm, gather_kv, linear, linear_add_rmsnorm,  # noqa: F401
                  linear_silu_mul, linear_workspace_bytes, lm_head_greedy, qk_norm_rope_store, qkv_decode_attention,
                  store_decode_attention,
                  reserve_linear_workspace, reserve_workspace, rope_cos_sin, shared_prefix_keys,
                  silu_and_mul, varlen_attention, workspace_bytes)

__all__ = ["Attention", "store_kvcache", "Context", "varlen_attention", "gather_kv",
           "workspace_bytes", "reserve_workspace", "qk_norm_rope_store", "rope_cos_sin",
           "add_rmsnorm", "silu_and_mul", "lm_head_greedy", "linear", "linear_silu_mul",
           "linear_add_rmsnorm", "linear_workspace_bytes", "reserve_linear_workspace",
           "shared_prefix_keys", "qkv_decode_attention", "store_decode_attention"]
