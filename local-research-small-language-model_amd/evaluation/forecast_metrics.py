"""Forecast routing metrics against a teacher (evaluation/forecast_metrics.py:8-136):
Recall@K, Precision@K, top-1 accuracy and KL(target || softmax(pred)).

Index tensors are [..., n] block lists (the selector's and the teacher's top-k,
best first); scores / distributions are [..., NB]. Means run over all leading
positions.
"""

from typing import Dict, List, Optional

import torch
import torch.nn.functional as F


def _overlap(pred_indices: torch.Tensor, target_indices: torch.Tensor, k: int):
    """(number of the first k predicted blocks found among the first k target
    blocks per position, kp, kt), or None when either list is empty."""
    kp = min(k, pred_indices.shape[-1])
    kt = min(k, target_indices.shape[-1])
    if kp == 0 or kt == 0:
        return None
    p = pred_indices[..., :kp].unsqueeze(-1)
    t = target_indices[..., :kt].unsqueeze(-2)
    hits = (p == t).any(dim=-1).float().sum(dim=-1)
    return hits, kp, kt


def compute_recall_at_k(pred_indices: torch.Tensor, target_indices: torch.Tensor, k: int) -> float:
    """|Pred_K ∩ Target_K| / |Target_K|, averaged (forecast_metrics.py:8-43)."""
    o = _overlap(pred_indices, target_indices, k)
    return 0.0 if o is None else float((o[0] / float(o[2])).mean().item())


def compute_precision_at_k(pred_indices: torch.Tensor, target_indices: torch.Tensor, k: int) -> float:
    """|Pred_K ∩ Target_K| / |Pred_K|, averaged (forecast_metrics.py:46-70)."""
    o = _overlap(pred_indices, target_indices, k)
    return 0.0 if o is None else float((o[0] / float(o[1])).mean().item())


def compute_block_selection_accuracy(pred_indices: torch.Tensor, target_indices: torch.Tensor) -> float:
    """Share of positions whose first predicted block is the first teacher block
    (forecast_metrics.py:73-82)."""
    return float((pred_indices[..., 0] == target_indices[..., 0]).float().mean().item())


def compute_kl_divergence(pred_scores: torch.Tensor, target_distribution: torch.Tensor,
                          eps: float = 1e-8) -> float:
    """Mean over positions with a finite prediction and a non-empty target of
    sum_j t_j (log t_j - log p_j), t and p clamped at eps and renormalised,
    p = softmax(pred) (forecast_metrics.py:85-108)."""
    valid = torch.isfinite(pred_scores) & (target_distribution.sum(dim=-1, keepdim=True) > 0)
    t = target_distribution.clamp(min=eps)
    t = t / t.sum(dim=-1, keepdim=True).clamp(min=eps)
    p = F.softmax(pred_scores, dim=-1).clamp(min=eps)
    p = p / p.sum(dim=-1, keepdim=True).clamp(min=eps)
    kl = (t * (t.log() - p.log())).sum(dim=-1)
    rows = valid.any(dim=-1)
    return float((kl[rows] if rows.any() else kl).mean().item())


def evaluate_forecast_metrics(pred_scores: torch.Tensor, pred_indices: torch.Tensor,
                              target_indices: torch.Tensor,
                              target_distribution: Optional[torch.Tensor] = None,
                              k_values: Optional[List[int]] = None) -> Dict[str, float]:
    """accuracy_top1, recall@K and precision@K for K in k_values (default
    1, 2, 4, 8), and kl_divergence when a target distribution is given
    (forecast_metrics.py:111-136)."""
    out: Dict[str, float] = {"accuracy_top1": compute_block_selection_accuracy(pred_indices, target_indices)}
    for k in (k_values if k_values is not None else [1, 2, 4, 8]):
        out[f"recall@{k}"] = compute_recall_at_k(pred_indices, target_indices, k)
        out[f"precision@{k}"] = compute_precision_at_k(pred_indices, target_indices, k)
    if target_distribution is not None:
        out["kl_divergence"] = compute_kl_divergence(pred_scores, target_distribution)
    return out
