"""Transformer block with the forecast hook and the attention-backend factory
(model/transformer.py:18-131).

The block computes layer L's forecast F_L from its normalised input, hands it
to layer L+1's backend ``prefetch`` (when that backend has one) before running
its own attention and FFN — the window the prefetch overlaps with — and
attends with F_{L-1} (layer 0 receives None).
"""

from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from model.attention.async_offload import HipAsyncOffloadAttention
from model.attention.base import BaseAttention, KVCache
from model.attention.hip_sparse import HipSparseAttention
from model.attention.offload import HipOffloadAttention
from model.config import ModelConfig
from model.forecast import ForecastProjection
from model.norm import RMSNorm
from model.rope import RotaryEmbedding


class SwiGLU(nn.Module):
    """(SiLU(x W_gate) * x W_up) W_down (model/transformer.py:18-31)."""

    def __init__(self, n_embd: int, ffn_dim: int):
        super().__init__()
        self.w_gate = nn.Linear(n_embd, ffn_dim, bias=False)
        self.w_up = nn.Linear(n_embd, ffn_dim, bias=False)
        self.w_down = nn.Linear(ffn_dim, n_embd, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.w_down(F.silu(self.w_gate(x)) * self.w_up(x))


def build_attention_backend(config: ModelConfig, layer_idx: int) -> BaseAttention:
    """Backend by name (model/transformer.py:34-51); unknown names raise ValueError.

    Every name maps onto libsparda's kernels: the dense, static and forecast
    sparse backends onto ``HipSparseAttention``, the offload backends onto the
    pinned-arena engine.
    """
    backend = config.attention_backend.lower()
    if backend == "dense":
        return HipSparseAttention(config, layer_idx, mode="dense")
    if backend in ("static_sparse", "static"):
        return HipSparseAttention(config, layer_idx, mode="static")
    if backend in ("sparse", "forecast", "sparse_forecast", "gpu_forecast", "hip_sparse"):
        mode = getattr(config, "sparse_mode", "forecast")
        if backend in ("sparse", "hip_sparse") and mode == "static":
            return HipSparseAttention(config, layer_idx, mode="static")
        return HipSparseAttention(config, layer_idx, mode="forecast")
    if backend in ("offload", "forecast_offload", "hip_offload"):
        return HipOffloadAttention(config, layer_idx)
    if backend in ("async", "async_offload", "async_prefetch", "hip_async_offload"):
        return HipAsyncOffloadAttention(config, layer_idx)
    raise ValueError(f"Unknown attention backend: {config.attention_backend}")


class TransformerBlock(nn.Module):
    """RMSNorm -> forecast (+ prefetch for layer L+1) -> attention -> residual ->
    RMSNorm -> SwiGLU -> residual (model/transformer.py:56-131)."""

    def __init__(self, config: ModelConfig, layer_idx: int):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.attn_norm = RMSNorm(config.n_embd, eps=config.norm_eps)
        self.attention = build_attention_backend(config, layer_idx)
        self.forecast = ForecastProjection(config)
        self.ffn_norm = RMSNorm(config.n_embd, eps=config.norm_eps)
        self.ffn = SwiGLU(config.n_embd, config.ffn_dim)

    def forward(self, x: torch.Tensor, rotary_emb: RotaryEmbedding, kv_cache: Optional[KVCache] = None,
                mask: Optional[torch.Tensor] = None, is_causal: bool = True,
                prev_layer_forecast: Optional[torch.Tensor] = None,
                next_layer_block: Optional["TransformerBlock"] = None,
                next_kv_cache=None) -> Tuple[torch.Tensor, torch.Tensor]:
        normed_x = self.attn_norm(x)
        current_forecast = self.forecast(normed_x)
        if next_layer_block is not None and next_kv_cache is not None:
            if hasattr(next_layer_block.attention, "prefetch"):
                next_layer_block.attention.prefetch(forecast_vector=current_forecast, offload_cache=next_kv_cache)
        attn_out = self.attention(normed_x, rotary_emb=rotary_emb, kv_cache=kv_cache, mask=mask,
                                  is_causal=is_causal, forecast_vector=prev_layer_forecast)
        x = x + attn_out
        x = x + self.ffn(self.ffn_norm(x))
        return x, current_forecast
