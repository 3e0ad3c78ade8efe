"""Rotary position embedding (rotate-half pairs (i, i + D/2)), as in
model/rope.py:8-98: fp32 cos/sin tables cast to the input dtype."""

from typing import Tuple

import torch
import torch.nn as nn


def rope_tables(head_dim: int, max_seq_len: int, theta: float = 10000.0) -> Tuple[torch.Tensor, torch.Tensor]:
    """cos, sin of shape [max_seq_len, head_dim // 2] in fp32."""
    if head_dim % 2:
        raise ValueError("head_dim must be even for RoPE")
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, dtype=torch.float32) / head_dim))
    ang = torch.arange(max_seq_len, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return torch.cos(ang), torch.sin(ang)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, offset: int = 0) -> torch.Tensor:
    """x [B,T,H,D]; rotates (x1, x2) -> (x1 cos - x2 sin, x2 cos + x1 sin)."""
    T = x.shape[1]
    half = x.shape[-1] // 2
    c = cos[offset:offset + T].to(x.dtype)[None, :, None, :]
    s = sin[offset:offset + T].to(x.dtype)[None, :, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return torch.cat((x1 * c - x2 * s, x2 * c + x1 * s), dim=-1)


class RotaryEmbedding(nn.Module):
    """Caches the tables; grows them when a longer sequence arrives."""

    def __init__(self, head_dim: int, max_seq_len: int = 4096, theta: float = 10000.0):
        super().__init__()
        self.head_dim = head_dim
        self.theta = theta
        self.max_seq_len = max_seq_len
        # plain fp32 attributes, not buffers: Module.to(dtype) would round
        # buffers to the model dtype; tables() moves them to the device in use
        self.cos, self.sin = rope_tables(head_dim, max_seq_len, theta)

    def tables(self, need: int, device) -> Tuple[torch.Tensor, torch.Tensor]:
        """fp32 cos, sin [L, head_dim/2] on `device`, L >= need."""
        if need > self.max_seq_len:
            self.max_seq_len = max(need, 2 * self.max_seq_len)
            cos, sin = rope_tables(self.head_dim, self.max_seq_len, self.theta)
            self.cos, self.sin = cos.to(device), sin.to(device)
        if self.cos.device != torch.device(device):
            self.cos, self.sin = self.cos.to(device), self.sin.to(device)
        return self.cos, self.sin

    def forward(self, xq: torch.Tensor, xk: torch.Tensor, offset: int = 0):
        cos, sin = self.tables(offset + xq.shape[1], xq.device)
        return apply_rope(xq, cos, sin, offset), apply_rope(xk, cos, sin, offset)
