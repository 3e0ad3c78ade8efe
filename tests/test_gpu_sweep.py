"""Seeded random sweep of the hot path's entry points over shapes the fixed
cases do not pin: the routed prefill (lists bit-exact against the oracle's
router, sampled rows of the output against the oracle's attention), the
decode step in both routings (selection bit-exact, output to the bf16 / fp32
bar), the dense decode split over workgroups, and the chunked-gather prefill
(the non-causal router, then the lists built inside the attention launch:
lists bit-exact against the oracle's, sampled rows to the bf16 bar).

Every configuration comes from seeded generators (2026, 2027, 2028, 2029) and is
printed before it runs, so a failure names a reproducible case."""

import numpy as np
import pytest
import torch

import sparda
from sparda import synth
from oracle import sparda_oracle as O
from helpers import assert_close_out, np32

pytestmark = pytest.mark.gpu
DEV = "cuda"


def case(msg):
    print(f"[case] {msg}", flush=True)


def _draws(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for _ in range(n):
        Hkv = int(r.choice([1, 2, 4]))
        R = int(r.integers(1, 5))
        bs = int(r.choice([32, 64]))
        out.append(dict(B=int(r.integers(1, 4)), Hkv=Hkv, Hq=Hkv * R, bs=bs, k=int(r.integers(1, 9)),
                        seed=int(r.integers(1, 1 << 30))))
    return out


_PREFILL = _draws(12, 2026)


@pytest.mark.parametrize("i", range(len(_PREFILL)))
def test_routed_prefill_random_shapes(i):
    c = _PREFILL[i]
    r = np.random.default_rng(c["seed"])
    T = int(r.integers(1, 2600))
    causal = bool(r.integers(0, 4) != 0)
    fdt = torch.float32 if r.integers(0, 3) == 0 else torch.bfloat16
    B, Hq, Hkv, bs, k = c["B"], c["Hq"], c["Hkv"], c["bs"], c["k"]
    case(f"routed prefill B={B} T={T} Hq={Hq} Hkv={Hkv} bs={bs} k={k} causal={causal} f={fdt} seed={c['seed']}")
    x = synth.prefill_inputs(B, T, Hq, Hkv, 64, dtype=torch.bfloat16, seed=c["seed"] % 100000)
    d = {n: t.to(DEV) for n, t in x.items()}
    f = d["forecast"].to(fdt)
    protos = sparda.compress(d["k"], bs)
    got, sel, n = sparda.prefill_routed(d["q"], d["k"], d["v"], f, protos, bs, k, causal=causal, want_sel=True)
    torch.cuda.synchronize()
    f_np = np32(f)
    _, _, sel_o, n_o = O.route(f_np, O.compress(np32(x["k"]), bs), bs, k, causal)
    n_g, sel_g = n.cpu().numpy(), sel.cpu().numpy()
    assert np.array_equal(n_g, n_o)
    for b in range(B):  # the listed entries (the caller's capacity may exceed the oracle's)
        for g in range(Hkv):
            for t in range(T):
                m = int(n_o[b, g, t])
                assert np.array_equal(sel_g[b, g, t, :m], sel_o[b, g, t, :m]), (b, g, t)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, B, 48), r.integers(0, T, 48))})
    rows += [(0, 0), (B - 1, T - 1)]
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, causal, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(got), want, torch.bfloat16, mask)


_DECODE = _draws(12, 2027)


@pytest.mark.parametrize("i", range(len(_DECODE)))
def test_decode_step_random_shapes(i):
    c = _DECODE[i]
    r = np.random.default_rng(c["seed"])
    S = int(r.integers(1, 7000))
    routing = "absolute" if r.integers(0, 2) else "reference"
    dtype = torch.float32 if r.integers(0, 4) == 0 else torch.bfloat16
    B, Hq, Hkv, bs, k = c["B"], c["Hq"], c["Hkv"], c["bs"], c["k"]
    case(f"decode B={B} S={S} Hq={Hq} Hkv={Hkv} bs={bs} k={k} {routing} {dtype} seed={c['seed']}")
    x = synth.decode_inputs(B, S, Hq, Hkv, 64, dtype=dtype, seed=c["seed"] % 100000)
    d = {n: t.to(DEV) for n, t in x.items()}
    out, ex = sparda.decode(d["q"], d["k_cache"], d["v_cache"], S, d["forecast"], bs, k, routing=routing,
                            want_sel=True)
    torch.cuda.synchronize()
    kc = np32(x["k_cache"])
    sel_o, n_o, _ = O.decode_selection(kc, S, np32(x["forecast"]), bs, k, routing)
    assert np.array_equal(ex["n_sel"].cpu().numpy(), n_o)
    assert np.array_equal(ex["sel"].cpu().numpy(), sel_o)
    want = O.attention_decode(np32(x["q"]), kc, np32(x["v_cache"]), S, sel_o, n_o, bs)
    assert_close_out(np32(out), want, dtype)


_DENSE = _draws(8, 2028)


@pytest.mark.parametrize("i", range(len(_DENSE)))
def test_dense_decode_random_lengths(i):
    c = _DENSE[i]
    r = np.random.default_rng(c["seed"])
    S = int(r.integers(1, 20000))
    B, Hq, Hkv, bs = c["B"], c["Hq"], c["Hkv"], c["bs"]
    case(f"dense decode B={B} S={S} Hq={Hq} Hkv={Hkv} bs={bs} seed={c['seed']}")
    x = synth.decode_inputs(B, S, Hq, Hkv, 64, dtype=torch.bfloat16, seed=c["seed"] % 100000)
    d = {n: t.to(DEV) for n, t in x.items()}
    out = sparda.decode_selected(d["q"], d["k_cache"], d["v_cache"], S, bs)
    torch.cuda.synchronize()
    NB = (S + bs - 1) // bs
    sel = np.broadcast_to(np.arange(NB, dtype=np.int32), (B, Hkv, NB)).copy()
    n = np.full((B, Hkv), NB, np.int32)
    want = O.attention_decode(np32(x["q"]), np32(x["k_cache"]), np32(x["v_cache"]), S, sel, n, bs)
    assert_close_out(np32(out), want, torch.bfloat16)


_CHUNKED = _draws(10, 2029)


@pytest.mark.parametrize("i", range(len(_CHUNKED)))
def test_chunked_prefill_random_shapes(i):
    c = _CHUNKED[i]
    r = np.random.default_rng(c["seed"])
    T = int(r.integers(1, 5000))
    with_forecast = bool(r.integers(0, 4) != 0)
    B, Hq, Hkv, bs, k = c["B"], c["Hq"], c["Hkv"], c["bs"], c["k"]
    case(f"chunked prefill B={B} T={T} Hq={Hq} Hkv={Hkv} bs={bs} k={k} forecast={with_forecast} seed={c['seed']}")
    x = synth.prefill_inputs(B, T, Hq, Hkv, 64, dtype=torch.bfloat16, seed=c["seed"] % 100000)
    d = {n: t.to(DEV) for n, t in x.items()}
    topk = tk_o = None
    if with_forecast:
        topk = sparda.route(d["forecast"], sparda.compress(d["k"], bs), bs, k, causal=False)[0]
        _, tk_o, _, _ = O.route(np32(x["forecast"]), O.compress(np32(x["k"]), bs), bs, k, False)
    got, sel, n = sparda.prefill_chunked(d["q"], d["k"], d["v"], topk, bs, k, want_sel=True)
    torch.cuda.synchronize()
    if with_forecast:
        assert np.array_equal(topk.cpu().numpy(), tk_o)
    sel_o, n_o = O.chunked_selection(tk_o, B, Hkv, T, bs, k)
    assert np.array_equal(n.cpu().numpy(), n_o) and np.array_equal(sel.cpu().numpy(), sel_o)
    rows = sorted({(int(b), int(t)) for b, t in zip(r.integers(0, B, 40), r.integers(0, T, 40))} | {(B - 1, T - 1)})
    want = O.attention_prefill(np32(x["q"]), np32(x["k"]), np32(x["v"]), sel_o, n_o, bs, True, rows=rows)
    mask = np.zeros(want.shape, bool)
    for b, t in rows:
        mask[b, t] = True
    assert_close_out(np32(got), want, torch.bfloat16, mask)
