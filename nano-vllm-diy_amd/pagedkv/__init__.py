"""pagedkv -- MI355X (gfx950) paged-KV attention path for a nano-vLLM-style engine.

Public surface (mirrors the reference's src/layers/attention.py and
src/utils/context.py):
    Attention, store_kvcache, Context,
    varlen_attention (flash_attn_varlen_func semantics), gather_kv,
    workspace_bytes, reserve_workspace.
"""
from .attention import Attention, store_kvcache  # noqa: F401
from .context import Context  # noqa: F401
from .ops import gather_kv, reserve_workspace, varlen_attention, workspace_bytes  # noqa: F401

__all__ = ["Attention", "store_kvcache", "Context", "varlen_attention", "gather_kv",
           "workspace_bytes", "reserve_workspace"]
