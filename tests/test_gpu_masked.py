"""GPU parity of the masked prefill with attention weights (the reference's
masked-SDPA path with `mask` and return_attn_weights, model/attention/
sparse.py:206-221, 255-281) and of the backend options that use it, against
the float64 oracle. Outputs within the bf16 / fp32 bars; weights within the
same bars, and exactly zero outside each row's allowed set."""

import numpy as np
import pytest
import torch

import sparda
from sparda import synth
from model.attention import HipSparseAttention
from model.config import ModelConfig
from model.rope import RotaryEmbedding
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def _check(x, sel, n, bs, causal, dtype, mask=None, mask_t=None):
    d = {k_: t_.to(DEV) for k_, t_ in x.items()}
    st = torch.from_numpy(sel).to(DEV) if sel is not None else None
    nt = torch.from_numpy(n).to(DEV) if n is not None else None
    out, w = sparda.prefill_masked(d["q"], d["k"], d["v"], st, nt, bs, causal=causal,
                                   mask=mask_t.to(DEV) if mask_t is not None else None, want_weights=True)
    torch.cuda.synchronize()
    want_o, want_w = O.attention_prefill_masked(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel, n, bs, causal,
                                                mask=mask)
    assert_close_out(np32(out), want_o, dtype)
    assert_close_out(np32(w), want_w, dtype, what="weights")
    assert (np32(w)[want_w == 0] == 0).all(), "weight outside the allowed set"
    return out, w


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_masked_prefill_sparse_forecast_lists_with_mask(dtype):
    case(f"prefill_masked forecast lists + [T,T] mask {dtype}")
    B, T, bs, k = 2, 320, 64, 2
    x = synth.prefill_inputs(B, T, 12, 4, 64, dtype=dtype, seed=301)
    _, _, sel, n = O.route(np32(x["forecast"]), O.compress(np32(x["k"]), bs), bs, k, True)
    m = np.random.default_rng(301).standard_normal((T, T)).astype(np.float32)
    _check(x, sel, n, bs, True, dtype, mask=m, mask_t=torch.from_numpy(m))


def test_masked_prefill_per_kv_head_mask_and_dense_noncausal():
    case("prefill_masked per-KV-head mask, dense non-causal")
    B, T, bs = 1, 200, 32
    x = synth.prefill_inputs(B, T, 8, 2, 32, dtype=torch.float32, seed=302)
    m = np.random.default_rng(302).standard_normal((B, 2, T, T)).astype(np.float32)
    m[:, :, :, 150:] = -np.inf  # some keys excluded outright
    mq = np.repeat(m, 4, axis=1)  # KV head g applies to its query heads, as repeat_interleave does
    _check(x, None, None, bs, False, torch.float32, mask=mq, mask_t=torch.from_numpy(m))


def test_masked_prefill_fully_masked_row():
    # a row whose mask is -inf on every allowed key: with the weights (the
    # reference's F.softmax path) weights and output are NaN there, as the
    # oracle has them; without (the reference's SDPA path) the output row is 0
    case("prefill_masked fully masked row, with and without weights")
    B, T, bs, k = 1, 192, 64, 2
    x = synth.prefill_inputs(B, T, 12, 4, 64, dtype=torch.float32, seed=304)
    _, _, sel, n = O.route(np32(x["forecast"]), O.compress(np32(x["k"]), bs), bs, k, True)
    m = np.random.default_rng(304).standard_normal((B, 12, T, T)).astype(np.float32)
    m[0, 5, 100, :] = -np.inf
    d = {k_: t_.to(DEV) for k_, t_ in x.items()}
    st, nt, mt = (torch.from_numpy(a).to(DEV) for a in (sel, n, m))
    out, w = sparda.prefill_masked(d["q"], d["k"], d["v"], st, nt, bs, causal=True, mask=mt, want_weights=True)
    plain = sparda.prefill_masked(d["q"], d["k"], d["v"], st, nt, bs, causal=True, mask=mt)
    torch.cuda.synchronize()
    want_o, want_w = O.attention_prefill_masked(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel, n, bs, True, mask=m)
    go, gw, gp = np32(out), np32(w), np32(plain)
    assert np.isnan(gw[0, 5, 100]).all() and np.isnan(go[0, 100, 5 * 64:6 * 64]).all()
    assert (np.isnan(gw) == np.isnan(want_w)).all() and (np.isnan(go) == np.isnan(want_o)).all()
    ok_w, ok_o = ~np.isnan(want_w), ~np.isnan(want_o)
    assert_close_out(gw[ok_w], want_w[ok_w], torch.float32, what="weights")
    assert_close_out(go[ok_o], want_o[ok_o], torch.float32)
    assert (gp[0, 100, 5 * 64:6 * 64] == 0).all()
    assert_close_out(gp[ok_o], want_o[ok_o], torch.float32, what="output without weights")


def test_masked_prefill_static_noncausal_window():
    case("prefill_masked static non-causal window")
    B, T, bs, k = 1, 256, 32, 2
    x = synth.prefill_inputs(B, T, 8, 2, 32, dtype=torch.float32, seed=303)
    sel, n = O.sel_fixed(O.SEL_WINDOW_PREFILL, B, T, 2, (T + bs - 1) // bs, bs, k)
    _check(x, sel, n, bs, False, torch.float32)


def _ref_config():
    # the reference's test geometry (tests/test_sparse_attention.py:14-30)
    return ModelConfig(vocab_size=1000, n_layer=4, n_embd=256, n_head=8, n_kv_head=2, head_dim=32, ffn_dim=512,
                       forecast_heads=2, forecast_dim=32, context_length=512, block_size=16, top_k_blocks=2)


def test_backend_return_attn_weights_is_causal():
    # tests/test_sparse_attention.py:80-92: the weights of a causal sparse layer
    # are zero above the diagonal; here also checked against the oracle
    case("backend return_attn_weights causality")
    cfg = _ref_config()
    torch.manual_seed(7)
    attn = HipSparseAttention(cfg, layer_idx=1).to(DEV).eval()
    rot = RotaryEmbedding(cfg.head_dim, 64).to(DEV)
    x = torch.randn(1, 64, cfg.n_embd, device=DEV)
    f = torch.randn(1, 64, cfg.forecast_heads, cfg.forecast_dim, device=DEV)
    with torch.no_grad():
        out, weights = attn(x, rotary_emb=rot, forecast_vector=f, return_attn_weights=True)
        plain = attn(x, rotary_emb=rot, forecast_vector=f)
    assert weights.shape == (1, cfg.n_head, 64, 64)
    assert torch.all(torch.triu(weights[0, 0], diagonal=1) == 0.0)
    assert (out - plain).abs().max().item() < 1e-4
    B, T = 1, 64
    xq = attn.wq(x).view(B, T, 8, 32)
    xk = attn.wk(x).view(B, T, 2, 32)
    xq, xk = rot(xq, xk, offset=0)
    sel, n = O.prefill_selection(np32(xk), np32(f), 16, 2)
    _, want_w = O.attention_prefill_masked(np32(xq), np32(xk), np32(xk), sel, n, 16, True)
    assert np.abs(np32(weights) - want_w).max() < 1e-4


def test_dense_backend_weights_for_the_teacher():
    # scripts/benchmark_forecast.py:86-93: the dense backend's weights feed the
    # routing-quality teacher
    case("dense backend weights")
    cfg = _ref_config()
    torch.manual_seed(8)
    attn = HipSparseAttention(cfg, layer_idx=0, mode="dense").to(DEV).eval()
    rot = RotaryEmbedding(cfg.head_dim, 128).to(DEV)
    x = torch.randn(2, 128, cfg.n_embd, device=DEV)
    with torch.no_grad():
        out, weights = attn(x, rotary_emb=rot, return_attn_weights=True)
    xq = attn.wq(x).view(2, 128, 8, 32)
    xk = attn.wk(x).view(2, 128, 2, 32)
    xq, xk = rot(xq, xk, offset=0)
    want = O.dense_weights(np32(xq), np32(xk), True)
    assert np.abs(np32(weights) - want).max() < 1e-4
    assert np.allclose(np32(weights).sum(-1), 1.0, atol=1e-4)
