from model.attention.async_offload import AsyncOffloadedKVCache, HipAsyncOffloadAttention
from model.attention.base import BaseAttention, KVCache
from model.attention.hip_sparse import HipSparseAttention, PrototypeKVCache, gather_kv_blocks
from model.attention.offload import HipOffloadAttention, OffloadedKVCache

__all__ = ["BaseAttention", "KVCache", "PrototypeKVCache", "HipSparseAttention", "gather_kv_blocks", "OffloadedKVCache",
           "HipOffloadAttention", "AsyncOffloadedKVCache", "HipAsyncOffloadAttention"]
