"""Forecast projection, KV block compressor and block selector — the
interfaces of model/forecast.py:11-130, computed by libsparda's HIP kernels.

``KVBlockCompressor`` and ``ForecastBlockSelector`` keep the reference's
constructor and ``forward`` signatures. Differences, all deliberate:
  * prototypes are returned in fp32 (the reference returns the key dtype);
  * scores are fp32 even for bf16 forecasts;
  * tied scores are ordered by lower block index (torch.topk leaves the tie
    order unspecified).
The tensors must be on a GPU device.
"""

from typing import Tuple

import torch
import torch.nn as nn

import sparda
from model.config import ModelConfig


class ForecastProjection(nn.Module):
    """wf: n_embd -> forecast_heads * forecast_dim, viewed [B,T,Hf,Df] (model/forecast.py:11-40)."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.n_embd = config.n_embd
        self.forecast_heads = config.forecast_heads
        self.forecast_dim = config.forecast_dim
        self.wf = nn.Linear(self.n_embd, self.forecast_heads * self.forecast_dim, bias=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        B, T, _ = x.shape
        return self.wf(x).view(B, T, self.forecast_heads, self.forecast_dim)


class KVBlockCompressor(nn.Module):
    """Mean-pooled key prototypes per block (model/forecast.py:43-78).

    forward(k [B,S,Hkv,D]) -> [B,NB,Hkv,Df] fp32; the zero-padded tail block
    is divided by block_size like the reference's padded mean.
    """

    def __init__(self, block_size: int = 32, head_dim: int = 64, forecast_dim: int = 64):
        super().__init__()
        self.block_size = block_size
        self.head_dim = head_dim
        self.forecast_dim = forecast_dim
        self.proj = nn.Linear(head_dim, forecast_dim, bias=False) if head_dim != forecast_dim else nn.Identity()

    def forward(self, k: torch.Tensor) -> torch.Tensor:
        protos = sparda.compress(k, self.block_size)
        if isinstance(self.proj, nn.Identity):
            return protos
        return self.proj(protos.to(self.proj.weight.dtype)).float()


class ForecastBlockSelector(nn.Module):
    """Forecast x prototype scores, causal block mask, top-k (model/forecast.py:81-130).

    forward(forecast [B,Tq,Hf,Df], block_reps [B,NB,Hkv,Df], top_k, is_causal)
      -> (scores fp32 [B,Hkv,Tq,NB], topk int64 [B,Hkv,Tq,min(top_k,NB)])
    Row t is masked beyond block (t + query_pos0) // block_size; the
    reference always uses query_pos0 = 0.
    """

    def __init__(self, block_size: int = 32, forecast_dim: int = 64):
        super().__init__()
        self.block_size = block_size
        self.forecast_dim = forecast_dim

    def forward(self, forecast: torch.Tensor, block_reps: torch.Tensor, top_k: int,
                is_causal: bool = True, query_pos0: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
        n_f_heads = forecast.shape[2]
        n_kv_head = block_reps.shape[2]
        assert n_f_heads == n_kv_head, f"Mismatch: forecast_heads ({n_f_heads}) != n_kv_head ({n_kv_head})"
        topk, scores, _, _ = sparda.route(forecast, block_reps, self.block_size, top_k, causal=is_causal,
                                          score_pos0=query_pos0, query_pos0=query_pos0,
                                          want_topk=True, want_scores=True)
        return scores, topk.long()
