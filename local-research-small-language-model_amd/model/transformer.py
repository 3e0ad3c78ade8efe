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

import sparda


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
        self._fused_w = None
        self._fused_key = None
        self._ffn_w = None
        self._ffn_key = None

    def _use_fused_producer(self, x: torch.Tensor, mask) -> bool:
        a = self.attention
        return (getattr(self.config, "fused_producer", False)
                and type(a) in (HipSparseAttention, HipOffloadAttention, HipAsyncOffloadAttention)
                and mask is None and x.is_cuda and x.dtype == torch.bfloat16 and a.head_dim == 64
                and self.forecast.forecast_dim == 64 and not torch.is_grad_enabled())

    def _fused_weight(self) -> torch.Tensor:
        """[wq; wk; wv; wf] with the attention RMSNorm weight folded into the
        columns, rebuilt when any of the parameters changed."""
        ws = (self.attention.wq.weight, self.attention.wk.weight, self.attention.wv.weight,
              self.forecast.wf.weight, self.attn_norm.weight)
        key = tuple((t.data_ptr(), t._version) for t in ws)
        if key != self._fused_key:
            with torch.no_grad():
                w = torch.cat([t.float() for t in ws[:4]], dim=0) * ws[4].float()[None, :]
                self._fused_w = w.to(torch.bfloat16).contiguous()
            self._fused_key = key
        return self._fused_w

    def _use_fused_ffn(self, x: torch.Tensor) -> bool:
        C = x.shape[-1]
        F_ = self.ffn.w_gate.out_features
        return (getattr(self.config, "fused_ffn", False) and x.is_cuda and x.dtype == torch.bfloat16
                and not torch.is_grad_enabled() and x.shape[0] * x.shape[1] <= 16
                and C % 128 == 0 and C <= 1024 and F_ % 128 == 0 and F_ <= 2048)

    def _fused_ffn_weight(self) -> torch.Tensor:
        """[w_gate; w_up] with the FFN RMSNorm weight folded into the columns,
        rebuilt when any of the parameters changed."""
        ws = (self.ffn.w_gate.weight, self.ffn.w_up.weight, self.ffn_norm.weight)
        key = tuple((t.data_ptr(), t._version) for t in ws)
        if key != self._ffn_key:
            with torch.no_grad():
                w = torch.cat([ws[0].float(), ws[1].float()], dim=0) * ws[2].float()[None, :]
                self._ffn_w = w.to(torch.bfloat16).contiguous()
            self._ffn_key = key
        return self._ffn_w

    def _use_fused_wo(self, x: torch.Tensor, T: int, kv_cache) -> bool:
        """x + wo(attention) as one kernel: single-token decode steps of the
        sparse backend, under the same switch and size limits as the FFN."""
        return (T == 1 and kv_cache is not None and type(self.attention) is HipSparseAttention
                and getattr(self.config, "fused_producer", False) and self._use_fused_ffn(x) and self.attention.n_head * self.attention.head_dim % 128 == 0
                and self.attention.n_head * self.attention.head_dim <= 2048)

    def ffn_residual(self, x: torch.Tensor) -> torch.Tensor:
        """x + SwiGLU(ffn_norm(x)) (transformer.py:126-129); one fused pair of
        kernels for decode-sized batches when the config asks for it."""
        if self._use_fused_ffn(x):
            return sparda.ffn_decode(x, self._fused_ffn_weight(), self.ffn.w_down.weight, self.ffn_norm.eps)
        return x + self.ffn(self.ffn_norm(x))

    def forward(self, x: torch.Tensor, rotary_emb: RotaryEmbedding, kv_cache: Optional[KVCache] = None,
                mask: Optional[torch.Tensor] = None, is_causal: bool = True,
                prev_layer_forecast: Optional[torch.Tensor] = None,
                next_layer_block: Optional["TransformerBlock"] = None,
                next_kv_cache=None) -> Tuple[torch.Tensor, torch.Tensor]:
        if self._use_fused_producer(x, mask):
            # RMSNorm + q / k / v / forecast projections + RoPE in one kernel
            a = self.attention
            B, T, _ = x.shape
            offset = kv_cache.current_len if kv_cache is not None else 0
            cos, sin = rotary_emb.tables(offset + T, x.device)
            xq, xk, xv, f = sparda.produce(x, self._fused_weight(), a.n_head * a.head_dim,
                                           a.n_kv_head * a.head_dim,
                                           self.forecast.forecast_heads * self.forecast.forecast_dim,
                                           self.attn_norm.eps, cos, sin, pos0=offset, f_dtype=x.dtype)
            current_forecast = f.view(B, T, self.forecast.forecast_heads, self.forecast.forecast_dim)
            if next_layer_block is not None and next_kv_cache is not None:
                if hasattr(next_layer_block.attention, "prefetch"):
                    next_layer_block.attention.prefetch(forecast_vector=current_forecast,
                                                        offload_cache=next_kv_cache)
            if self._use_fused_wo(x, T, kv_cache):
                x = a.forward_projected(xq, xk, xv, kv_cache=kv_cache, is_causal=is_causal,
                                        forecast_vector=prev_layer_forecast, residual=x)
            else:
                x = x + a.forward_projected(xq, xk, xv, kv_cache=kv_cache, is_causal=is_causal,
                                            forecast_vector=prev_layer_forecast)
            return self.ffn_residual(x), current_forecast
        normed_x = self.attn_norm(x)
        current_forecast = self.forecast(normed_x)
        if next_layer_block is not None and next_kv_cache is not None:
            if hasattr(next_layer_block.attention, "prefetch"):
                next_layer_block.attention.prefetch(forecast_vector=current_forecast, offload_cache=next_kv_cache)
        attn_out = self.attention(normed_x, rotary_emb=rotary_emb, kv_cache=kv_cache, mask=mask,
                                  is_causal=is_causal, forecast_vector=prev_layer_forecast)
        x = x + attn_out
        return self.ffn_residual(x), current_forecast
