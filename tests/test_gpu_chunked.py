"""GPU parity of the chunked-gather prefill (model/attention/sparse.py:284-364):
the per-query-block lists (sparda_select_chunked) bit-exact against the
oracle's, the one-launch kernel (sparda_prefill_chunked: lists built in the
launch, attention over them) against the oracle, against sparda_prefill on the
same lists and against itself (determinism), and HipSparseAttention with
use_chunked_gather=True against the oracle."""

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


@pytest.mark.parametrize("T,bs,k,spread", [(1000, 64, 8, None), (1000, 64, 4, 16), (777, 32, 4, 6),
                                           (64, 64, 8, None), (16384, 64, 8, None), (5000, 16, 2, 40)])
def test_select_chunked_equals_the_oracle(T, bs, k, spread):
    case(f"select_chunked T={T} bs={bs} k={k} spread={spread}")
    B, H = 2, 3
    NB = (T + bs - 1) // bs
    ke = min(k, NB)
    rng = np.random.default_rng(T + k)
    tk = rng.integers(0, spread or NB, size=(B, H, T, ke)).astype(np.int32) % NB
    sel, n = sparda.select_chunked(torch.from_numpy(tk).to(DEV), B, H, T, bs, k)
    sel_o, n_o = O.chunked_selection(tk, B, H, T, bs, k)
    torch.cuda.synchronize()
    assert np.array_equal(n.cpu().numpy(), n_o)
    assert np.array_equal(sel.cpu().numpy(), sel_o)
    # the static window (no forecast)
    sel, n = sparda.select_chunked(None, B, H, T, bs, k, device=DEV)
    sel_o, n_o = O.chunked_selection(None, B, H, T, bs, k)
    torch.cuda.synchronize()
    assert np.array_equal(n.cpu().numpy(), n_o) and np.array_equal(sel.cpu().numpy(), sel_o)


@pytest.mark.parametrize("B,T,bs,k", [(2, 1500, 64, 8), (1, 16384, 64, 8), (1, 2000, 32, 4)])
def test_chunked_prefill_against_the_oracle(B, T, bs, k):
    case(f"chunked prefill B={B} T={T} bs={bs} k={k}")
    Hq, Hkv, D = 12, 4, 64
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=torch.bfloat16, seed=700 + T)
    d = {n: t.to(DEV) for n, t in x.items()}
    protos = sparda.compress(d["k"], bs)
    topk = sparda.route(d["forecast"], protos, bs, k, causal=False)[0]
    sel, n = sparda.select_chunked(topk, B, Hkv, T, bs, k)
    out = sparda.prefill(d["q"], d["k"], d["v"], sel, n, bs, causal=True)
    torch.cuda.synchronize()
    _, tk_o, _, _ = O.route(np32(x["forecast"]), O.compress(np32(x["k"]), bs), bs, k, False)
    assert np.array_equal(topk.cpu().numpy(), tk_o)
    sel_o, n_o = O.chunked_selection(tk_o, B, Hkv, T, bs, k)
    assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
    r = np.random.default_rng(3)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, B, 64), r.integers(0, T, 64))})
    rows += [(0, 0), (0, bs - 1), (0, bs), (B - 1, T - 1)]
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(out), want, torch.bfloat16, mask)


@pytest.mark.parametrize("with_forecast", [True, False])
def test_backend_use_chunked_gather(with_forecast):
    # HipSparseAttention with use_chunked_gather=True: the chunked lists and the
    # prefill over them, then wo (layer 1 with a forecast; without one the
    # static window, as the reference's chunked path takes for layer 0)
    case(f"HipSparseAttention use_chunked_gather forecast={with_forecast}")
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=2048)
    attn = HipSparseAttention(cfg, layer_idx=1).to(DEV, torch.bfloat16).eval()
    rot = RotaryEmbedding(cfg.head_dim, cfg.context_length).to(DEV)
    g = torch.Generator().manual_seed(12)
    B, T = 1, 1200
    x = torch.randn(B, T, cfg.n_embd, generator=g).to(DEV, torch.bfloat16)
    f = (torch.randn(B, T, cfg.n_kv_head, cfg.forecast_dim, generator=g).to(DEV, torch.bfloat16)
         if with_forecast else None)
    with torch.no_grad():
        got = attn(x, rot, forecast_vector=f, use_chunked_gather=True)
        xq = attn.wq(x).view(B, T, attn.n_head, attn.head_dim)
        xk = attn.wk(x).view(B, T, attn.n_kv_head, attn.head_dim)
        xv = attn.wv(x).view(B, T, attn.n_kv_head, attn.head_dim)
        xq, xk = rot(xq, xk, offset=0)
        topk = None
        if with_forecast:
            topk = sparda.route(f, sparda.compress(xk, 64), 64, 8, causal=False)[0]
        o, sel, n = sparda.prefill_chunked(xq, xk, xv, topk, 64, 8, want_sel=True)
        want = attn.wo(o)
        per_token = attn(x, rot, forecast_vector=f)
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    tk = None if topk is None else topk.cpu().numpy()
    sel_o, n_o = O.chunked_selection(tk, B, attn.n_kv_head, T, 64, 8)
    assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
    want_o = O.attention_prefill(np32(xq), np32(xk), np32(xv), sel_o, n_o, 64, True)
    assert_close_out(np32(o), want_o, torch.bfloat16)
    assert not torch.equal(got, per_token)  # the per-token rule is another selection


def test_backend_default_follows_the_length():
    # without the flag the backend takes the chunked path past 8192 tokens and
    # the per-token rule up to it (sparse.py:420); the flag overrides either
    # way, and the chunked path answers a weights request with the output
    # alone, as the reference's does
    case("HipSparseAttention default at T=8192 / 8193")
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=8256)
    attn = HipSparseAttention(cfg, layer_idx=1).to(DEV, torch.bfloat16).eval()
    rot = RotaryEmbedding(cfg.head_dim, cfg.context_length).to(DEV)
    g = torch.Generator().manual_seed(13)
    for T, chunked in ((8192, False), (8193, True)):
        x = torch.randn(1, T, cfg.n_embd, generator=g).to(DEV, torch.bfloat16)
        f = torch.randn(1, T, cfg.n_kv_head, cfg.forecast_dim, generator=g).to(DEV, torch.bfloat16)
        with torch.no_grad():
            default = attn(x, rot, forecast_vector=f)
            as_chunked = attn(x, rot, forecast_vector=f, use_chunked_gather=True)
            per_token = attn(x, rot, forecast_vector=f, use_chunked_gather=False)
            weights_asked = attn(x, rot, forecast_vector=f, return_attn_weights=True) if chunked else None
        torch.cuda.synchronize()
        assert torch.equal(default, as_chunked if chunked else per_token), T
        assert not torch.equal(as_chunked, per_token), T
        if chunked:
            assert isinstance(weights_asked, torch.Tensor) and torch.equal(weights_asked, as_chunked)


@pytest.mark.parametrize("B,T,Hq,Hkv,k,spread,forecast", [
    (2, 1500, 12, 4, 8, None, True), (1, 16384, 12, 4, 8, None, True), (1, 64, 12, 4, 8, None, True),
    (3, 777, 4, 4, 4, None, True), (1, 2000, 16, 4, 8, None, True), (2, 1000, 8, 4, 4, 16, True),
    (2, 1500, 12, 4, 8, None, False), (1, 130, 6, 2, 8, None, False)])
def test_prefill_chunked_one_launch(B, T, Hq, Hkv, k, spread, forecast):
    # the lists built inside the attention launch equal select_chunked's (and
    # the oracle's) bit for bit; the output is within the bf16 bar of the
    # oracle on sampled rows and close to sparda_prefill over the same lists;
    # two calls give the same bits
    case(f"prefill_chunked B={B} T={T} Hq={Hq} Hkv={Hkv} k={k} spread={spread} forecast={forecast}")
    bs, D = 64, 64
    NB = (T + bs - 1) // bs
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=torch.bfloat16, seed=800 + T + Hq)
    d = {n: t.to(DEV) for n, t in x.items()}
    topk = None
    if forecast:
        ke = min(k, NB)
        rng = np.random.default_rng(T + k)
        tk = rng.integers(0, spread or NB, size=(B, Hkv, T, ke)).astype(np.int32) % NB
        topk = torch.from_numpy(tk).to(DEV)
    out, sel, n = sparda.prefill_chunked(d["q"], d["k"], d["v"], topk, bs, k, want_sel=True)
    out2 = sparda.prefill_chunked(d["q"], d["k"], d["v"], topk, bs, k)
    sel_l, n_l = sparda.select_chunked(topk, B, Hkv, T, bs, k, device=DEV)
    lists = sparda.prefill(d["q"], d["k"], d["v"], sel_l, n_l, bs, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(out, out2), "prefill_chunked is not deterministic"
    assert torch.equal(sel, sel_l) and torch.equal(n, n_l)
    sel_o, n_o = O.chunked_selection(None if topk is None else topk.cpu().numpy(), B, Hkv, T, bs, k)
    assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
    r = np.random.default_rng(T)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, B, 96), r.integers(0, T, 96))})
    rows += [(0, 0), (0, min(T - 1, bs - 1)), (0, min(T - 1, bs)), (B - 1, T - 1)]
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(out), want, torch.bfloat16, mask)
    assert_close_out(np32(out), np32(lists), torch.bfloat16, what="against sparda_prefill on the same lists")


def test_prefill_chunked_two_launch_shapes():
    # shapes outside the one-launch kernel (32-key blocks, fp32) run
    # select_chunked + prefill through the hand-off buffers: the same bits
    case("prefill_chunked two-launch shapes")
    for bs, dtype in ((32, torch.bfloat16), (64, torch.float32)):
        B, T, Hq, Hkv, D, k = 2, 700, 12, 4, 64, 4
        NB = (T + bs - 1) // bs
        x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=dtype, seed=900 + bs)
        d = {n: t.to(DEV) for n, t in x.items()}
        tk = np.random.default_rng(bs).integers(0, NB, size=(B, Hkv, T, k)).astype(np.int32)
        topk = torch.from_numpy(tk).to(DEV)
        out, sel, n = sparda.prefill_chunked(d["q"], d["k"], d["v"], topk, bs, k, want_sel=True)
        sel_l, n_l = sparda.select_chunked(topk, B, Hkv, T, bs, k)
        want = sparda.prefill(d["q"], d["k"], d["v"], sel_l, n_l, bs, causal=True)
        torch.cuda.synchronize()
        assert torch.equal(sel, sel_l) and torch.equal(n, n_l)
        assert torch.equal(out, want), (bs, dtype)


@pytest.mark.parametrize("T,Hq,Hkv,k", [(4096 * 64, 3, 1, 8), (5000, 12, 4, 32)])
def test_prefill_chunked_at_its_limits(T, Hq, Hkv, k):
    # 4096 blocks (the list bitmap's capacity) and top-32 (lists of 34 blocks)
    case(f"prefill_chunked limits T={T} Hq={Hq} Hkv={Hkv} k={k}")
    B, bs, D = 1, 64, 64
    NB = (T + bs - 1) // bs
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=torch.bfloat16, seed=41 + k)
    d = {n: t.to(DEV) for n, t in x.items()}
    tk = np.random.default_rng(k).integers(0, NB, size=(B, Hkv, T, k)).astype(np.int32)
    topk = torch.from_numpy(tk).to(DEV)
    out, sel, n = sparda.prefill_chunked(d["q"], d["k"], d["v"], topk, bs, k, want_sel=True)
    sel_l, n_l = sparda.select_chunked(topk, B, Hkv, T, bs, k)
    torch.cuda.synchronize()
    assert torch.equal(sel, sel_l) and torch.equal(n, n_l)
    sel_o, n_o = O.chunked_selection(tk, B, Hkv, T, bs, k)
    assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
    r = np.random.default_rng(T)
    rows = sorted({(0, int(t)) for t in r.integers(0, T, 48)} | {(0, 0), (0, T - 1)})
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(out), want, torch.bfloat16, mask)


@pytest.mark.parametrize("T", [1, 2, 63, 65, 129])
def test_prefill_chunked_tiny_lengths(T):
    # one or two query blocks, ragged: the lists and the output against the oracle
    case(f"prefill_chunked tiny T={T}")
    B, Hq, Hkv, D, bs, k = 2, 12, 4, 64, 64, 8
    NB = (T + bs - 1) // bs
    x = synth.prefill_inputs(B, T, Hq, Hkv, D, dtype=torch.bfloat16, seed=70 + T)
    d = {n: t.to(DEV) for n, t in x.items()}
    for with_topk in (True, False):
        tk = np.random.default_rng(T).integers(0, NB, size=(B, Hkv, T, min(k, NB))).astype(np.int32)
        topk = torch.from_numpy(tk).to(DEV) if with_topk else None
        out, sel, n = sparda.prefill_chunked(d["q"], d["k"], d["v"], topk, bs, k, want_sel=True)
        torch.cuda.synchronize()
        sel_o, n_o = O.chunked_selection(tk if with_topk else None, B, Hkv, T, bs, k)
        assert np.array_equal(sel.cpu().numpy(), sel_o) and np.array_equal(n.cpu().numpy(), n_o)
        want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, True)
        assert_close_out(np32(out), want, torch.bfloat16)


def test_static_mode_backend_past_8192_takes_the_window():
    # the static-window backend past 8192 tokens: the chunked path's window
    # lists (sparse.py:320-328 take the window whenever no forecast routes)
    case("static mode backend T=8200")
    from model.transformer import build_attention_backend
    cfg = ModelConfig(block_size=64, top_k_blocks=8, context_length=8256, attention_backend="static_sparse")
    attn = build_attention_backend(cfg, 1).to(DEV, torch.bfloat16).eval()
    rot = RotaryEmbedding(cfg.head_dim, cfg.context_length).to(DEV)
    g = torch.Generator().manual_seed(14)
    B, T = 1, 8200
    x = torch.randn(B, T, cfg.n_embd, generator=g).to(DEV, torch.bfloat16)
    with torch.no_grad():
        got = attn(x, rot)
        xq = attn.wq(x).view(B, T, attn.n_head, attn.head_dim)
        xk = attn.wk(x).view(B, T, attn.n_kv_head, attn.head_dim)
        xv = attn.wv(x).view(B, T, attn.n_kv_head, attn.head_dim)
        xq, xk = rot(xq, xk, offset=0)
        want = attn.wo(sparda.prefill_chunked(xq, xk, xv, None, 64, 8))
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_prefill_chunked_on_strided_views():
    # q, k and v as slices of one packed [B, T, Hq + 2 Hkv, D] buffer (element
    # strides, no copies): the same output as on contiguous copies
    case("prefill_chunked strided views")
    B, T, Hq, Hkv, D, bs, k = 2, 1000, 12, 4, 64, 64, 8
    g = torch.Generator().manual_seed(15)
    packed = torch.randn(B, T, Hq + 2 * Hkv, D, generator=g).to(DEV, torch.bfloat16)
    q, kk, v = packed[:, :, :Hq], packed[:, :, Hq:Hq + Hkv], packed[:, :, Hq + Hkv:]
    NB = (T + bs - 1) // bs
    topk = torch.from_numpy(np.random.default_rng(15).integers(0, NB, size=(B, Hkv, T, k)).astype(np.int32)).to(DEV)
    got = sparda.prefill_chunked(q, kk, v, topk, bs, k)
    want = sparda.prefill_chunked(q.contiguous(), kk.contiguous(), v.contiguous(), topk, bs, k)
    torch.cuda.synchronize()
    assert not q.is_contiguous() and torch.equal(got, want)
