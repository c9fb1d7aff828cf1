"""Hybrid Sparse Attention on MI355X — public API of ``wan/modules/hsa/__init__.py:3-26``."""

from .attention import (
    HSAAttention,
    compress_kv,
    hsa_attention,
    hsa_parameter_names,
    require_trained_hsa,
    resolve_backend,
)
from .kvcache import kv_append, new_block_sums
from .block_sparse import block_sparse_attention, block_sparse_attention_reference, map_to_index
from .routing import (
    BlockRouting,
    block_attention_map,
    block_mean_pool,
    build_block_routing,
    build_topk_routing,
)

__all__ = [
    "HSAAttention",
    "hsa_attention",
    "compress_kv",
    "resolve_backend",
    "hsa_parameter_names",
    "require_trained_hsa",
    "block_sparse_attention_reference",
    "block_sparse_attention",
    "map_to_index",
    "BlockRouting",
    "build_block_routing",
    "build_topk_routing",
    "block_attention_map",
    "block_mean_pool",
    "kv_append",
    "new_block_sums",
]
