from model.attention.base import BaseAttention, KVCache
from model.attention.hip_sparse import HipSparseAttention, gather_kv_blocks

__all__ = ["BaseAttention", "KVCache", "HipSparseAttention", "gather_kv_blocks"]
