"""Routing-quality path (model/forecast.py:133-238, evaluation/forecast_metrics.py),
CPU: the teacher restatements against closed forms and the float64 oracle, the
loss and the metrics against hand-computed answers."""

import math

import numpy as np
import torch

from evaluation.forecast_metrics import (compute_block_selection_accuracy, compute_kl_divergence,
                                         compute_precision_at_k, compute_recall_at_k, evaluate_forecast_metrics)
from model.forecast import TeacherBlockSelector, compute_forecast_loss
from oracle import sparda_oracle as O


def test_oracle_teacher_closed_forms():
    # one block: every causal row puts all its mass on block 0
    g = np.random.default_rng(1)
    q, k = g.standard_normal((1, 40, 3, 16)), g.standard_normal((1, 40, 1, 16))
    m = O.teacher_block_mass(q, k, 64)
    assert m.shape == (1, 1, 40, 1) and np.allclose(m, 1.0)
    # identical keys: uniform weights over the t + 1 causal keys, so block j of
    # row t holds (number of keys of block j that are <= t) / (t + 1)
    T, bs = 50, 8
    q = g.standard_normal((1, T, 2, 8))
    k = np.ones((1, T, 1, 8))
    m = O.teacher_block_mass(q, k, bs)
    for t in range(T):
        for j in range((T + bs - 1) // bs):
            n = max(0, min(t, j * bs + bs - 1) - j * bs + 1)
            assert abs(m[0, 0, t, j] - n / (t + 1)) < 1e-12
    # non-causal rows sum to one over all blocks
    m = O.teacher_block_mass(q, g.standard_normal((1, T, 1, 8)), bs, causal=False)
    assert np.allclose(m.sum(-1), 1.0)


def test_oracle_dense_weights_gqa_against_sdpa():
    # SDPA with identity values returns its own weight matrix (softmax(QK^T) @ I),
    # and enable_gqa applies the library's query-head -> KV-head mapping, so
    # this pins the oracle's h // R grouping, scale and causal mask with more
    # than one KV head (a swapped mapping, h % Hkv, fails it)
    g = np.random.default_rng(5)
    B, T, Hq, Hkv, D = 2, 37, 6, 2, 16
    q, k = g.standard_normal((B, T, Hq, D)), g.standard_normal((B, T, Hkv, D))
    eye = torch.eye(T, dtype=torch.float64).expand(B, Hkv, T, T)
    for causal in (True, False):
        want = torch.nn.functional.scaled_dot_product_attention(
            torch.from_numpy(q).transpose(1, 2), torch.from_numpy(k).transpose(1, 2), eye,
            is_causal=causal, enable_gqa=True).numpy()
        got = O.dense_weights(q, k, causal)
        assert got.shape == (B, Hq, T, T)
        assert np.abs(got - want).max() < 1e-12
    # the planted mistake a swapped head mapping would make is visible here
    swapped = O.dense_weights(q[:, :, [0, 3, 1, 4, 2, 5]], k, True)
    assert np.abs(swapped - O.dense_weights(q, k, True)).max() > 1e-3


def test_teacher_selector_forward_matches_oracle():
    g = np.random.default_rng(2)
    q, k = g.standard_normal((2, 100, 6, 16)), g.standard_normal((2, 100, 2, 16))
    for causal in (True, False):
        w = O.dense_weights(q, k, causal)
        want = O.teacher_block_scores(w, 16, 3, causal)
        sel = TeacherBlockSelector(block_size=16, num_queries_per_kv=3)
        scores, topk, target = sel(torch.from_numpy(w), top_k=4, is_causal=causal)
        assert np.abs(scores.numpy() - want).max() < 1e-12
        assert np.allclose(target.numpy(), want / (want.sum(-1, keepdims=True) + 1e-8))
        order = np.argsort(-want, axis=-1, kind="stable")[..., :4]
        assert (topk.numpy() == order).all()


def test_teacher_topk_ties_lower_index():
    s = torch.tensor([[[[0.2, 0.4, 0.4, 0.0, 0.4]]]])
    _, topk, _ = TeacherBlockSelector._finish(s, 3)
    assert topk.flatten().tolist() == [1, 2, 4]


def test_forecast_loss_known_answers():
    target = torch.tensor([[0.5, 0.25, 0.25]])
    # KL is zero when the prediction is the target itself
    assert abs(float(compute_forecast_loss(target.log(), target))) < 1e-7
    # KL(t || softmax(0)) = sum t log(t / (1/3)), averaged over the 3 valid entries
    want = sum(p * math.log(p * 3) for p in (0.5, 0.25, 0.25)) / 3
    assert abs(float(compute_forecast_loss(torch.zeros(1, 3), target)) - want) < 1e-6
    # BCE of logit 0 against hot targets is log 2 per valid entry; -inf predictions are left out
    pred = torch.tensor([[0.0, 0.0, -math.inf]])
    tgt = torch.tensor([[1.0, 0.0, 0.0]])
    assert abs(float(compute_forecast_loss(pred, tgt, "bce")) - math.log(2.0)) < 1e-6
    # a row whose target is empty contributes nothing
    pred2 = torch.tensor([[0.0, 0.0, -math.inf], [5.0, 1.0, 2.0]])
    tgt2 = torch.tensor([[1.0, 0.0, 0.0], [0.0, 0.0, 0.0]])
    assert abs(float(compute_forecast_loss(pred2, tgt2, "bce")) - math.log(2.0)) < 1e-6


def test_metrics_known_answers():
    pred = torch.tensor([[0, 1, 2, 3], [5, 6, 7, 8]])
    tgt = torch.tensor([[2, 0, 9, 10], [5, 7, 6, 1]])
    # K=2: {0,1} vs {2,0} -> 1 hit; {5,6} vs {5,7} -> 1 hit
    assert compute_recall_at_k(pred, tgt, 2) == 0.5
    assert compute_precision_at_k(pred, tgt, 2) == 0.5
    # K=4: 2/4 and 3/4
    assert abs(compute_recall_at_k(pred, tgt, 4) - 0.625) < 1e-12
    # uneven list lengths: 1 of the 2 target blocks among the 4 predicted
    assert compute_recall_at_k(pred[:1], tgt[:1, :2], 4) == 1.0
    assert compute_precision_at_k(pred[:1], tgt[:1, :2], 4) == 0.5
    assert compute_block_selection_accuracy(pred, tgt) == 0.5
    t = torch.tensor([[0.7, 0.2, 0.1]])
    assert abs(compute_kl_divergence(t.log(), t)) < 1e-6
    m = evaluate_forecast_metrics(t.log(), pred, tgt, t, k_values=[2])
    assert set(m) == {"accuracy_top1", "recall@2", "precision@2", "kl_divergence"}
