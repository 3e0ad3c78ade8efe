"""Attention plugin interface and GPU KV cache (model/attention/base.py:11-73)."""

from abc import ABC, abstractmethod
from typing import Optional, Tuple

import torch
import torch.nn as nn

from model.config import ModelConfig
from model.rope import RotaryEmbedding


class KVCache:
    """Pre-allocated k/v [B, Smax, Hkv, D]; ``update`` appends and returns the
    valid prefix views (model/attention/base.py:11-32)."""

    def __init__(self, max_batch_size: int, max_seq_len: int, n_kv_head: int, head_dim: int,
                 device: torch.device, dtype: torch.dtype):
        self.k = torch.zeros((max_batch_size, max_seq_len, n_kv_head, head_dim), device=device, dtype=dtype)
        self.v = torch.zeros((max_batch_size, max_seq_len, n_kv_head, head_dim), device=device, dtype=dtype)
        self.current_len = 0

    def update(self, xk: torch.Tensor, xv: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        n = xk.shape[1]
        lo, hi = self.current_len, self.current_len + n
        if hi > self.k.shape[1]:
            raise ValueError(f"KVCache overflow: {hi} > capacity {self.k.shape[1]}")
        self.k[:, lo:hi] = xk
        self.v[:, lo:hi] = xv
        self.current_len = hi
        return self.k[:, :hi], self.v[:, :hi]

    def reset(self):
        self.current_len = 0


class BaseAttention(nn.Module, ABC):
    """Backends own wq/wk/wv/wo with the reference's names and shapes, so
    state dicts move across backends (model/attention/base.py:35-73)."""

    def __init__(self, config: ModelConfig, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.n_head = config.n_head
        self.n_kv_head = config.n_kv_head
        self.head_dim = config.head_dim
        self.n_embd = config.n_embd
        self.num_queries_per_kv = config.num_queries_per_kv
        self.wq = nn.Linear(self.n_embd, self.n_head * self.head_dim, bias=False)
        self.wk = nn.Linear(self.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.wv = nn.Linear(self.n_embd, self.n_kv_head * self.head_dim, bias=False)
        self.wo = nn.Linear(self.n_head * self.head_dim, self.n_embd, bias=False)

    @abstractmethod
    def forward(self, x: torch.Tensor, rotary_emb: RotaryEmbedding, kv_cache: Optional[KVCache] = None,
                mask: Optional[torch.Tensor] = None, is_causal: bool = True, **kwargs) -> torch.Tensor:
        """x [B,T,n_embd] -> [B,T,n_embd]."""
