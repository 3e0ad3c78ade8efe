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
import torch.nn.functional as F

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


def _canonical_topk(scores: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest scores, larger first, equal scores by lower index."""
    return torch.sort(scores, dim=-1, descending=True, stable=True).indices[..., :k]


class TeacherBlockSelector(nn.Module):
    """Ground-truth block importance from dense attention (model/forecast.py:133-193).

    forward(attn_weights [B,Hq,Tq,Tk], top_k, is_causal)
      -> (block_scores [B,Hkv,Tq,NB], topk [B,Hkv,Tq,k] int64, target_distribution)
    restates the reference on materialised post-softmax weights. from_qk(q, k,
    top_k, is_causal) returns the same triple from the HIP kernel
    (sparda.teacher_block_mass) without materialising the weights (q
    [B,T,Hq,64], k [B,T,Hkv,64] bf16, block size 64). Ties in the top-k go to
    the lower block index (torch.topk leaves their order unspecified).
    """

    def __init__(self, block_size: int = 32, num_queries_per_kv: int = 3):
        super().__init__()
        self.block_size = block_size
        self.num_queries_per_kv = num_queries_per_kv

    def forward(self, attn_weights: torch.Tensor, top_k: int,
                is_causal: bool = True) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        B, Hq, Tq, Tk = attn_weights.shape
        R = self.num_queries_per_kv
        bs = self.block_size
        per_kv = attn_weights.reshape(B, Hq // R, R, Tq, Tk).mean(dim=2)
        nb = (Tk + bs - 1) // bs
        per_kv = F.pad(per_kv, (0, nb * bs - Tk))
        block_scores = per_kv.reshape(B, Hq // R, Tq, nb, bs).sum(dim=-1)
        if is_causal:
            t = torch.arange(Tq, device=attn_weights.device)[:, None]
            j = torch.arange(nb, device=attn_weights.device)[None, :]
            block_scores = block_scores.masked_fill(j > t // bs, 0.0)
        return self._finish(block_scores, top_k)

    def from_qk(self, q: torch.Tensor, k: torch.Tensor, top_k: int,
                is_causal: bool = True) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        if q.shape[2] != k.shape[2] * self.num_queries_per_kv:
            raise AssertionError(f"Mismatch: {q.shape[2]} query heads vs {k.shape[2]} KV heads x "
                                 f"{self.num_queries_per_kv}")
        mass = sparda.teacher_block_mass(q, k, self.block_size, causal=is_causal)
        return self._finish(mass, top_k)

    @staticmethod
    def _finish(block_scores: torch.Tensor, top_k: int):
        target = block_scores / (block_scores.sum(dim=-1, keepdim=True) + 1e-8)
        kk = min(top_k, block_scores.shape[-1])
        return block_scores, _canonical_topk(block_scores, kk), target


def compute_forecast_loss(pred_scores: torch.Tensor, target_distribution: torch.Tensor,
                          loss_type: str = "kl", temperature: float = 1.0) -> torch.Tensor:
    """Auxiliary loss between forecast scores and the teacher distribution
    (model/forecast.py:196-238): "kl" = KL(target || softmax(pred / temperature)),
    "bce" = BCE with logits against the multi-hot support of the target; both
    averaged over the (row, block) entries with a finite prediction in rows
    whose target has mass."""
    valid = torch.isfinite(pred_scores) & (target_distribution.sum(dim=-1, keepdim=True) > 0)
    n = valid.sum().clamp(min=1)
    if loss_type == "kl":
        logp = F.log_softmax(pred_scores / temperature, dim=-1)
        logp = torch.where(torch.isfinite(logp), logp, torch.zeros_like(logp))
        per = F.kl_div(logp, target_distribution, reduction="none")
    elif loss_type == "bce":
        hot = (target_distribution > 0).to(pred_scores.dtype)
        logits = torch.where(torch.isfinite(pred_scores), pred_scores, torch.full_like(pred_scores, -100.0))
        per = F.binary_cross_entropy_with_logits(logits, hot, reduction="none")
    else:
        raise ValueError(f"compute_forecast_loss: loss_type must be 'kl' or 'bce', got {loss_type!r}")
    return torch.where(valid, per, torch.zeros_like(per)).sum() / n
