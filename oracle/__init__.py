"""CPU oracle for the paged-KV attention path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg may import
this package, and only as the checker or the timed CPU baseline. The product path
(pagedkv) never calls into it.
"""
from .paged_kv import (  # noqa: F401
    default_scale,
    gather_kv,
    kv_head_of,
    store_kvcache,
    varlen_attention,
    visible,
)
