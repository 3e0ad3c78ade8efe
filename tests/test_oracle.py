"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Each oracle function is checked against something independent of its own
code: closed forms, brute force, exact rational arithmetic, PyTorch library
routines (torch.topk, scaled_dot_product_attention), the op-for-op
restatement of the reference path, and the known-answer assertions of the
reference's tests (tests/test_forecast.py, tests/test_sparse_attention.py).
"""

import math
from fractions import Fraction

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import reference_path as R
from oracle import sparda_oracle as O


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# compressor (model/forecast.py:57-78)
# ---------------------------------------------------------------------------

def test_compress_matches_padded_mean():
    k = rng(0).standard_normal((2, 50, 3, 16)).astype(np.float32)
    bs = 16
    got = O.compress(k, bs)
    pad = np.zeros((2, 64, 3, 16), np.float64)
    pad[:, :50] = k
    want = pad.reshape(2, 4, 16, 3, 16).mean(axis=2)
    assert got.shape == (2, 4, 3, 16)
    np.testing.assert_allclose(got, want, rtol=0, atol=2e-6)


def test_compress_reference_known_answers():
    # tests/test_forecast.py:53-68: S=64, bs=16 -> 4 blocks; S=50 -> ceil = 4 blocks
    assert O.compress(np.zeros((2, 64, 4, 32), np.float32), 16).shape == (2, 4, 4, 32)
    assert O.compress(np.zeros((2, 50, 4, 32), np.float32), 16).shape == (2, 4, 4, 32)
    # partial block divided by bs, not by the present count (zero-padded mean)
    p = O.compress(np.ones((1, 50, 1, 4), np.float32), 16)
    assert np.all(p[0, :3] == 1.0) and np.all(p[0, 3] == np.float32(2 / 16))


def test_compress_exact_on_integers():
    k = rng(1).integers(-50, 50, size=(1, 256, 2, 8)).astype(np.float32)
    got = O.compress(k, 64)
    want = k.reshape(1, 4, 64, 2, 8).sum(axis=2) / 64  # exact: small integers, power-of-2 divisor
    assert np.array_equal(got, want.astype(np.float32))


def test_compress_sequential_order_is_pinned():
    # ((0 + 1e8) + 1) - 1e8 + 1 = 1 sequentially; a pairwise tree gives 0
    k = np.array([1e8, 1.0, -1e8, 1.0], np.float32).reshape(1, 4, 1, 1)
    assert O.compress(k, 4)[0, 0, 0, 0] == np.float32(0.25)


# ---------------------------------------------------------------------------
# scores (model/forecast.py:108-126)
# ---------------------------------------------------------------------------

def _fp32_round(fr: Fraction) -> np.float32:
    x = np.float32(float(fr))
    best = x
    for c in (np.nextafter(x, np.float32(-np.inf)), np.nextafter(x, np.float32(np.inf))):
        dc, db = abs(Fraction(float(c)) - fr), abs(Fraction(float(best)) - fr)
        if dc < db or (dc == db and (int(c.view(np.uint32)) & 1) == 0):
            best = c
    return np.float32(best)


def test_scores_fma_chain_exact():
    r = rng(2)
    f = r.standard_normal((1, 3, 2, 16)).astype(np.float32)
    P = r.standard_normal((1, 5, 2, 16)).astype(np.float32)
    got = O.scores(f, P, bs=1, causal=False, scale=0.25)
    for h in range(2):
        for t in range(3):
            for j in range(5):
                acc = np.float32(0)
                for d in range(16):
                    acc = _fp32_round(Fraction(float(f[0, t, h, d])) * Fraction(float(P[0, j, h, d]))
                                      + Fraction(float(acc)))
                assert got[0, h, t, j] == np.float32(acc * np.float32(0.25))


def test_scores_close_to_float64_matmul():
    r = rng(3)
    f = r.standard_normal((2, 40, 4, 64)).astype(np.float32)
    P = r.standard_normal((2, 5, 4, 64)).astype(np.float32)
    got = O.scores(f, P, bs=8, causal=True)
    want = np.einsum("bthd,bjhd->bhtj", f.astype(np.float64), P.astype(np.float64)) / 8.0
    fin = np.isfinite(got)
    np.testing.assert_allclose(got[fin], want[fin], atol=1e-4)


def test_scores_causal_pattern_reference_known_answer():
    # tests/test_forecast.py:71-92: bs=8, Tq=32, NB=4
    r = rng(4)
    f = r.standard_normal((2, 32, 2, 16)).astype(np.float32)
    P = r.standard_normal((2, 4, 2, 16)).astype(np.float32)
    s = O.scores(f, P, bs=8, causal=True)
    tk = O.topk(s, 2)
    assert s.shape == (2, 2, 32, 4) and tk.shape == (2, 2, 32, 2)
    assert np.isneginf(s[:, :, 0, 1:]).all()
    assert np.isneginf(s[:, :, 7, 1:]).all()
    assert np.isfinite(s[:, :, 8, :2]).all()
    assert np.isneginf(s[:, :, 8, 2:]).all()


def test_scores_position_offset():
    r = rng(5)
    f = r.standard_normal((1, 1, 1, 16)).astype(np.float32)
    P = r.standard_normal((1, 8, 1, 16)).astype(np.float32)
    s0 = O.scores(f, P, bs=4, causal=True, score_pos0=0)
    s1 = O.scores(f, P, bs=4, causal=True, score_pos0=29)
    assert np.isfinite(s0[0, 0, 0, 0]) and np.isneginf(s0[0, 0, 0, 1:]).all()
    assert np.isfinite(s1[0, 0, 0, :8]).all()  # 29 // 4 = 7 -> all 8 blocks


# ---------------------------------------------------------------------------
# top-k (torch.topk at model/forecast.py:128-129, ties by lower index)
# ---------------------------------------------------------------------------

def _brute_topk(row, k):
    key = lambda j: (-(0.0 if row[j] == 0 else float(row[j])), j)
    return sorted(range(len(row)), key=key)[:min(k, len(row))]


def test_topk_equals_torch_on_distinct_values():
    s = rng(6).permutation(4096 * 64).reshape(4096, 64).astype(np.float32) / 7.0
    got = O.topk(s, 8)
    want = torch.topk(torch.from_numpy(s), 8, dim=-1).indices.numpy()
    assert np.array_equal(got, want)


def test_topk_ties_lower_index_first():
    r = rng(7)
    s = r.integers(-3, 3, size=(500, 40)).astype(np.float32)
    s[r.random(s.shape) < 0.2] = -np.inf
    s[:, 5] = -0.0
    got = O.topk(s, 8)
    for i in range(s.shape[0]):
        assert list(got[i]) == _brute_topk(s[i], 8)


def test_topk_k_larger_than_blocks():
    s = np.array([[0.5, -np.inf, 2.0]], np.float32)
    assert O.topk(s, 8).tolist() == [[2, 0, 1]]


# ---------------------------------------------------------------------------
# selection sets (model/attention/sparse.py:126-154, 231-253)
# ---------------------------------------------------------------------------

def test_selection_sets_brute_force():
    r = rng(8)
    B, Tq, H, NB, bs, k = 2, 96, 2, 12, 8, 4
    f = r.standard_normal((B, Tq, H, 16)).astype(np.float32)
    P = r.standard_normal((B, NB, H, 16)).astype(np.float32)
    for causal in (True, False):
        sc, tk, sel, n = O.route(f, P, bs, k, causal=causal)
        for b in range(B):
            for h in range(H):
                for t in range(Tq):
                    own = min(t // bs, NB - 1)
                    want = {0, own} | set(int(x) for x in tk[b, h, t])
                    if causal:
                        want = {j for j in want if j <= own}
                    got = sel[b, h, t, :n[b, h, t]]
                    assert list(got) == sorted(want)
                    assert (sel[b, h, t, n[b, h, t]:] == -1).all()


def test_decode_reference_routing_closed_form():
    # row-0 mask (model/forecast.py:123-126 from model/attention/sparse.py:139):
    # only block 0 is finite, ties by index give {0..k-1}, plus the current block
    r = rng(9)
    S, bs, k = 1000, 16, 5
    kc = r.standard_normal((2, S, 3, 16)).astype(np.float32)
    f = r.standard_normal((2, 3, 16)).astype(np.float32)
    sel, n, _ = O.decode_selection(kc, S, f, bs, k, routing="reference")
    cb = (S - 1) // bs
    for b in range(2):
        for g in range(3):
            assert list(sel[b, g, :n[b, g]]) == list(range(k)) + [cb]


def test_fixed_selections():
    sel, n = O.sel_fixed(O.SEL_WINDOW_DECODE, 1, 1, 1, NB=20, bs=16, k=4, query_pos0=16 * 10 + 3)
    assert list(sel[0, 0, 0, :n[0, 0, 0]]) == [0, 7, 8, 9, 10]
    sel, n = O.sel_fixed(O.SEL_WINDOW_PREFILL, 1, 64, 1, NB=4, bs=16, k=1)
    assert list(sel[0, 0, 63, :n[0, 0, 63]]) == [0, 2, 3]
    assert list(sel[0, 0, 20, :n[0, 0, 20]]) == [0, 1]
    sel, n = O.sel_fixed(O.SEL_DENSE, 1, 40, 1, NB=3, bs=16, k=1)
    assert list(sel[0, 0, 39, :n[0, 0, 39]]) == [0, 1, 2]


# ---------------------------------------------------------------------------
# gather (model/attention/sparse.py:19-62; tests/test_sparse_attention.py:33-60)
# ---------------------------------------------------------------------------

def test_gather_reference_known_answer():
    k = rng(10).standard_normal((2, 2, 48, 32)).astype(np.float32)
    v = rng(11).standard_normal((2, 2, 48, 32)).astype(np.float32)
    idx = np.array([[[0, 2], [1, 2]], [[2, 0], [0, 1]]])
    kg, vg = O.gather_blocks(k, v, idx, 16)
    assert kg.shape == (2, 2, 32, 32)
    assert np.array_equal(kg[0, 0, :16], k[0, 0, 0:16])
    assert np.array_equal(kg[0, 0, 16:], k[0, 0, 32:48])
    assert np.array_equal(vg[1, 0, :16], v[1, 0, 32:48])
    # tail block past S is zero-padded
    kg2, _ = O.gather_blocks(k[:, :, :40], v[:, :, :40], idx, 16)
    assert np.array_equal(kg2[0, 0, 16:24], k[0, 0, 32:40]) and not kg2[0, 0, 24:].any()


# ---------------------------------------------------------------------------
# attention (model/attention/sparse.py:185-282, 99-183)
# ---------------------------------------------------------------------------

def _inputs(seed, B, T, Hq, Hkv, D):
    r = rng(seed)
    q = r.standard_normal((B, T, Hq, D)).astype(np.float32)
    k = r.standard_normal((B, T, Hkv, D)).astype(np.float32)
    v = r.standard_normal((B, T, Hkv, D)).astype(np.float32)
    f = r.standard_normal((B, T, Hkv, D)).astype(np.float32)
    return q, k, v, f


def test_prefill_blockwise_equals_full_mask_textbook():
    B, T, Hq, Hkv, D, bs, k = 2, 70, 6, 2, 16, 8, 3
    q, kk, v, f = _inputs(12, B, T, Hq, Hkv, D)
    sel, n = O.prefill_selection(kk, f, bs, k)
    got = O.attention_prefill(q, kk, v, sel, n, bs)
    # textbook: explicit [T,T] allowed mask, full-row softmax in float64
    R_ = Hq // Hkv
    want = np.zeros_like(got)
    for b in range(B):
        for h in range(Hq):
            g = h // R_
            allowed = np.zeros((T, T), bool)
            for t in range(T):
                blocks = set(sel[b, g, t, :n[b, g, t]].tolist())
                for s in range(t + 1):
                    allowed[t, s] = (s // bs) in blocks
            sc = q[b, :, h].astype(np.float64) @ kk[b, :, g].astype(np.float64).T / math.sqrt(D)
            sc[~allowed] = -np.inf
            p = np.exp(sc - sc.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            want[b, :, h * D:(h + 1) * D] = p @ v[b, :, g].astype(np.float64)
    np.testing.assert_allclose(got, want, atol=1e-12)


def test_prefill_dense_cases_equal_sdpa():
    B, T, Hq, Hkv, D, bs = 1, 50, 4, 2, 16, 8
    q, kk, v, f = _inputs(13, B, T, Hq, Hkv, D)
    tq = torch.from_numpy(q).double().transpose(1, 2)
    tk = torch.repeat_interleave(torch.from_numpy(kk).double().transpose(1, 2), 2, dim=1)
    tv = torch.repeat_interleave(torch.from_numpy(v).double().transpose(1, 2), 2, dim=1)
    want = F.scaled_dot_product_attention(tq, tk, tv, is_causal=True).transpose(1, 2).reshape(B, T, Hq * D)
    # k >= NB: every causal block is selected -> dense causal attention
    sel, n = O.prefill_selection(kk, f, bs, topk_blocks=16)
    np.testing.assert_allclose(O.attention_prefill(q, kk, v, sel, n, bs), want.numpy(), atol=1e-12)
    # sel=None is the dense fallback (model/attention/sparse.py:201-224)
    np.testing.assert_allclose(O.attention_prefill(q, kk, v, None, None, bs), want.numpy(), atol=1e-12)


def test_prefill_matches_reference_path_restatement():
    B, T, Hq, Hkv, D, bs, k = 2, 160, 6, 2, 16, 16, 3
    q, kk, v, f = _inputs(14, B, T, Hq, Hkv, D)
    sel, n = O.prefill_selection(kk, f, bs, k)
    got = O.attention_prefill(q, kk, v, sel, n, bs)
    t = lambda a: torch.from_numpy(a).double()
    want = R.sparse_prefill(t(q).transpose(1, 2), t(kk).transpose(1, 2), t(v).transpose(1, 2), t(f), bs, k)
    np.testing.assert_allclose(got, want.numpy(), atol=1e-10)


def test_prefill_causality_invariant():
    # tests/test_sparse_attention.py:80-92 restated on outputs: future tokens never matter
    B, T, Hq, Hkv, D, bs, k = 1, 96, 4, 2, 16, 8, 3
    q, kk, v, f = _inputs(15, B, T, Hq, Hkv, D)
    sel, n = O.prefill_selection(kk, f, bs, k)
    out = O.attention_prefill(q, kk, v, sel, n, bs)
    kk2, v2 = kk.copy(), v.copy()
    kk2[:, 60:] += 5.0
    v2[:, 60:] -= 3.0
    out2 = O.attention_prefill(q, kk2, v2, sel, n, bs)
    np.testing.assert_array_equal(out[:, :60], out2[:, :60])


def test_decode_dense_fallback_equals_sdpa():
    B, S, Hq, Hkv, D, bs, k = 2, 90, 6, 2, 16, 16, 4  # NB = 6 <= k+2
    r = rng(16)
    q = r.standard_normal((B, Hq, D)).astype(np.float32)
    kc = r.standard_normal((B, 100, Hkv, D)).astype(np.float32)
    vc = r.standard_normal((B, 100, Hkv, D)).astype(np.float32)
    f = r.standard_normal((B, Hkv, D)).astype(np.float32)
    got, sel, n = O.decode_step(q, kc, vc, S, f, bs, k)
    assert (n == 6).all()
    tq = torch.from_numpy(q).double()[:, :, None]
    tk = torch.repeat_interleave(torch.from_numpy(kc[:, :S]).double().transpose(1, 2), 3, dim=1)
    tv = torch.repeat_interleave(torch.from_numpy(vc[:, :S]).double().transpose(1, 2), 3, dim=1)
    want = F.scaled_dot_product_attention(tq, tk, tv).reshape(B, Hq * D)
    np.testing.assert_allclose(got, want.numpy(), atol=1e-12)


def test_decode_absolute_equals_last_prefill_row():
    B, T, Hq, Hkv, D, bs, k = 2, 200, 6, 2, 16, 16, 4
    q, kk, v, f = _inputs(17, B, T, Hq, Hkv, D)
    sel, n = O.prefill_selection(kk, f, bs, k)
    pre = O.attention_prefill(q, kk, v, sel, n, bs, rows=[(b, T - 1) for b in range(B)])
    dec, dsel, dn = O.decode_step(q[:, T - 1], kk, v, T, f[:, T - 1], bs, k, routing="absolute")
    np.testing.assert_allclose(dec, pre[:, T - 1], atol=1e-12)
    for b in range(B):
        for g in range(Hkv):
            assert list(dsel[b, g, :dn[b, g]]) == list(sel[b, g, T - 1, :n[b, g, T - 1]])


def test_decode_matches_reference_restatement_on_its_selection():
    B, S, Hq, Hkv, D, bs, k = 2, 300, 6, 2, 16, 16, 4
    r = rng(18)
    q = r.standard_normal((B, Hq, D)).astype(np.float32)
    kc = r.standard_normal((B, S, Hkv, D)).astype(np.float32)
    vc = r.standard_normal((B, S, Hkv, D)).astype(np.float32)
    f = r.standard_normal((B, 1, Hkv, D)).astype(np.float32)
    t = lambda a: torch.from_numpy(a).double()
    out, idx, valid = R.sparse_decode(t(q)[:, :, None], t(kc).transpose(1, 2), t(vc).transpose(1, 2), S,
                                      t(f), bs, k)
    # same attention on the selection torch.topk made (its -inf tie order is unspecified)
    cap = k + 2
    sel = np.full((B, Hkv, cap), -1, np.int32)
    n = np.zeros((B, Hkv), np.int32)
    for b in range(B):
        for g in range(Hkv):
            s = sorted(int(j) for j, ok in zip(idx[b, g], valid[b, g]) if ok)
            sel[b, g, :len(s)] = s
            n[b, g] = len(s)
            cb = (S - 1) // bs
            assert 0 in s and cb in s and len(s) <= k + 2
    got = O.attention_decode(q, kc, vc, S, sel, n, bs)
    np.testing.assert_allclose(got, out.reshape(B, Hq * D).numpy(), atol=1e-12)
    # absolute routing masks at the query's position: no -inf ties among the
    # 19 causal blocks, so the restatement's selection is the oracle's
    out, idx, valid = R.sparse_decode(t(q)[:, :, None], t(kc).transpose(1, 2), t(vc).transpose(1, 2), S,
                                      t(f), bs, k, routing="absolute")
    sel_o, n_o, _ = O.decode_selection(kc, S, f[:, 0], bs, k, "absolute")
    for b in range(B):
        for g in range(Hkv):
            s = sorted(int(j) for j, ok in zip(idx[b, g], valid[b, g]) if ok)
            assert s == list(sel_o[b, g, :n_o[b, g]])
    got = O.attention_decode(q, kc, vc, S, sel_o, n_o, bs)
    np.testing.assert_allclose(got, out.reshape(B, Hq * D).numpy(), atol=1e-12)


# ---------------------------------------------------------------------------
# prefetch (lookahead) selection
# ---------------------------------------------------------------------------

def test_prefetch_selection_dense_branch():
    # own + 1 <= k + 2: every block 0..own (model/attention/async_offload.py:198-203)
    kc = np.random.default_rng(0).standard_normal((1, 1000, 2, 8)).astype(np.float32)
    f = np.ones((1, 2, 8), np.float32)
    sel, n = O.prefetch_selection(kc, 600, 600, f, 64, 8)
    assert (n == 10).all() and (sel[0, 0, :10] == np.arange(10)).all() and (sel[0, 0, 10:] == -1).all()


def test_prefetch_selection_reference_mode_closed_form():
    # the row-0 mask leaves only block 0 finite: {0..k-1} U {own} under canonical ties
    rng = np.random.default_rng(1)
    kc = rng.standard_normal((2, 2000, 2, 8)).astype(np.float32)
    f = rng.standard_normal((2, 2, 8)).astype(np.float32)
    for L in (1300, 1280):  # own block partial / empty
        sel, n = O.prefetch_selection(kc, L, L, f, 64, 4, "reference")
        own = L // 64
        assert (n == 5).all()
        assert (sel[..., :5] == np.array([0, 1, 2, 3, own])).all()


def test_prefetch_selection_absolute_equals_router_and_brute_force():
    rng = np.random.default_rng(2)
    B, H, D, bs, k = 2, 3, 8, 16, 3
    kc = rng.standard_normal((B, 300, H, D)).astype(np.float32)
    f = rng.standard_normal((B, H, D)).astype(np.float32)
    for L in (200, 208):  # 208 = 13 full blocks: the own block (13) holds no token yet
        sel, n = O.prefetch_selection(kc, L, L, f, bs, k, "absolute")
        P = O.compress(kc[:, :L], bs)
        NB = P.shape[1]
        own = L // bs
        for b in range(B):
            for h in range(H):
                s = np.array([np.float32(sum(np.float64(f[b, h, d]) * np.float64(P[b, j, h, d])
                                             for d in range(D))) for j in range(NB)])
                order = sorted(range(NB), key=lambda j: (-s[j], j))[:k]
                want = sorted({0, own} | set(order))
                assert list(sel[b, h, :n[b, h]]) == want
        if L % bs:
            # with a partial own block the router (own clamped to NB-1 = own) agrees
            _, _, rsel, rn = O.route(f.reshape(B, 1, H, D), P, bs, k, True, L, L)
            assert np.array_equal(rsel[:, :, 0], sel) and np.array_equal(rn[:, :, 0], n)


# ---------------------------------------------------------------------------
# masked prefill with weights (sparse.py:206-221, 255-281)
# ---------------------------------------------------------------------------

def _small(seed, B=1, T=96, Hq=4, Hkv=2, D=16):
    r = np.random.default_rng(seed)
    return (r.standard_normal((B, T, Hq, D)), r.standard_normal((B, T, Hkv, D)),
            r.standard_normal((B, T, Hkv, D)))


def test_masked_prefill_without_mask_equals_prefill():
    q, k, v = _small(1)
    f = np.random.default_rng(2).standard_normal((1, 96, 2, 16))
    _, _, sel, n = O.route(f, O.compress(k, 16), 16, 2, True)
    out, w = O.attention_prefill_masked(q, k, v, sel, n, 16, True)
    assert np.allclose(out, O.attention_prefill(q, k, v, sel, n, 16, True), atol=1e-12)
    # weights: rows sum to one, nothing above the diagonal, out == W V
    assert np.allclose(w.sum(-1), 1.0)
    assert (np.triu(w[0, 0], 1) == 0).all()
    o2 = np.einsum("bhts,bshd->bthd", w, np.repeat(v, 2, axis=2)).reshape(out.shape)
    assert np.allclose(o2, out, atol=1e-12)


def test_masked_prefill_dense_equals_sdpa_with_attn_mask():
    # library pin: dense, non-causal, additive mask == torch SDPA(attn_mask)
    q, k, v = _small(3)
    m = np.random.default_rng(4).standard_normal((1, 4, 96, 96))
    out, _ = O.attention_prefill_masked(q, k, v, None, None, 16, False, mask=m)
    tq, tk, tv = (torch.from_numpy(x).permute(0, 2, 1, 3) for x in (q, k, v))
    tk, tv = (torch.repeat_interleave(x, 2, dim=1) for x in (tk, tv))
    ref = F.scaled_dot_product_attention(tq, tk, tv, attn_mask=torch.from_numpy(m))
    assert np.allclose(out, ref.permute(0, 2, 1, 3).reshape(1, 96, 64).numpy(), atol=1e-10)


def test_masked_prefill_fully_masked_row_is_softmax_nan():
    # library pin: the reference's weights path is F.softmax(scores + mask),
    # which is NaN throughout a row whose scores are all -inf, and the output
    # (weights @ V) is NaN there too; every other row is unaffected
    q, k, v = _small(6)
    T = 96
    m = np.random.default_rng(6).standard_normal((1, 4, T, T))
    m[0, 1, 40, :] = -np.inf
    out, w = O.attention_prefill_masked(q, k, v, None, None, 16, True, mask=m)
    tq, tk = (torch.from_numpy(x).permute(0, 2, 1, 3) for x in (q, k))
    tk = torch.repeat_interleave(tk, 2, dim=1)
    causal = torch.triu(torch.full((T, T), float("-inf"), dtype=torch.float64), 1)
    ref_w = F.softmax(tq @ tk.transpose(-1, -2) / np.sqrt(q.shape[-1]) + causal + torch.from_numpy(m), dim=-1)
    assert torch.isnan(ref_w[0, 1, 40]).all() and np.isnan(w[0, 1, 40]).all()
    assert np.isnan(out[0, 40, 16:32]).all()
    ok = ~np.isnan(ref_w.numpy())
    assert np.allclose(w[ok], ref_w.numpy()[ok], atol=1e-12)
    assert np.isfinite(np.delete(out[0, 40], np.s_[16:32])).all() and np.isfinite(np.delete(out, 40, 1)).all()


def test_masked_prefill_minus_inf_block_equals_dropping_it():
    # -inf over one listed block is the list without it; a constant shift of the
    # mask changes nothing (softmax shift invariance)
    q, k, v = _small(5)
    T, bs = 96, 16
    sel = np.full((1, 2, T, 4), -1, np.int32)
    n = np.zeros((1, 2, T), np.int32)
    sel2, n2 = sel.copy(), n.copy()
    for t in range(T):
        own = t // bs
        lst = sorted({0, own} | ({own - 1} if own >= 1 else set()))
        sel[0, :, t, :len(lst)] = lst
        n[0, :, t] = len(lst)
        keep = [j for j in lst if j != 0] or [0]
        sel2[0, :, t, :len(keep)] = keep
        n2[0, :, t] = len(keep)
    m = np.zeros((T, T))
    m[:, :bs] = -np.inf
    rows = [(0, t) for t in range(bs, T)]  # rows whose lists keep another block
    a, _ = O.attention_prefill_masked(q, k, v, sel, n, bs, True, mask=m, rows=rows)
    b, _ = O.attention_prefill_masked(q, k, v, sel2, n2, bs, True, rows=rows)
    c, _ = O.attention_prefill_masked(q, k, v, sel, n, bs, True, mask=m + 3.5, rows=rows)
    assert np.allclose(a[0, bs:], b[0, bs:], atol=1e-12)
    assert np.allclose(a[0, bs:], c[0, bs:], atol=1e-12)


def test_masked_prefill_repeats_and_out_of_range_entries_count_once():
    q, k, v = _small(6)
    T, bs = 96, 16
    sel = np.full((1, 2, T, 6), -1, np.int32)
    n = np.zeros((1, 2, T), np.int32)
    clean = sel.copy()
    nc = n.copy()
    for t in range(T):
        own = t // bs
        sel[0, :, t, :5] = [own, 0, own, -1, 99]
        n[0, :, t] = 5
        lst = sorted({0, own})
        clean[0, :, t, :len(lst)] = lst
        nc[0, :, t] = len(lst)
    a, wa = O.attention_prefill_masked(q, k, v, sel, n, bs, True)
    b = O.attention_prefill(q, k, v, clean, nc, bs, True)
    assert np.allclose(a, b, atol=1e-12)
