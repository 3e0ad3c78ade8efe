"""The oracle's chunked-gather lists and attention (model/attention/sparse.py:
284-364) pinned against a torch restatement of the reference's steps: the
selection mask built by scatter, future blocks cleared, the cut by
torch.topk over the 0/1 mask, the gather, the validity mask and SDPA per
query block. Where the union fits the cut (no tie among the 1.0 entries
decides) the lists must be the same sets; where it does not, the oracle keeps
the lowest block indices (checked directly), an order torch.topk leaves
unspecified."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import sparda_oracle as O


def _reference_lists(tk, B, H, T, bs, k):
    """The selection steps of sparse.py:303-333 in torch (CPU), per query block:
    (sel_indices, val) as the reference computes them."""
    NB = (T + bs - 1) // bs
    max_sel = min(NB, k + 2)
    out = []
    for bq in range(NB):
        start, end = bq * bs, min(T, (bq + 1) * bs)
        mask = torch.zeros((B, H, NB), dtype=torch.bool)
        mask.scatter_(-1, torch.zeros((B, H, 1), dtype=torch.long), True)
        mask.scatter_(-1, torch.full((B, H, 1), bq, dtype=torch.long), True)
        if tk is not None and bq > 0:
            idx = torch.from_numpy(tk[:, :, start:end, :].astype(np.int64)).reshape(B, H, -1)
            mask.scatter_(-1, idx.clamp(0, NB - 1), True)
        else:
            for j in range(max(0, bq - k + 1), bq + 1):
                mask.scatter_(-1, torch.full((B, H, 1), j, dtype=torch.long), True)
        mask[:, :, torch.arange(NB) > bq] = False
        val, sel = torch.topk(mask.float(), k=max_sel, dim=-1)
        out.append((bq, start, end, sel, val, mask))
    return out


def _random_topk(rng, B, H, T, NB, ke, spread):
    # picks confined to `spread` blocks so that the unions stay small or large on purpose
    return rng.integers(0, spread, size=(B, H, T, ke)).astype(np.int32) % NB


# the last case's unions exceed the cut (min(NB, k+2) = 6 of 16 blocks)
@pytest.mark.parametrize("T,bs,k,spread", [(300, 64, 8, 3), (640, 64, 4, 2), (257, 32, 8, 4), (130, 64, 8, 64),
                                           (1000, 64, 4, 16)])
def test_chunked_lists_equal_the_reference_steps(T, bs, k, spread):
    B, H = 2, 3
    NB = (T + bs - 1) // bs
    rng = np.random.default_rng(T + bs + k)
    tk = _random_topk(rng, B, H, T, NB, min(k, NB), spread)
    sel, n = O.chunked_selection(tk, B, H, T, bs, k)
    for bq, start, end, rsel, val, mask in _reference_lists(tk, B, H, T, bs, k):
        for b in range(B):
            for h in range(H):
                want = sorted(int(j) for j, v in zip(rsel[b, h], val[b, h]) if v > 0.5)
                union = int(mask[b, h].sum())
                for t in range(start, end):
                    got = list(sel[b, h, t, :n[b, h, t]])
                    if union <= rsel.shape[-1]:
                        assert got == want, (bq, b, h, t)
                    else:  # the cut: the lowest indices of the union
                        assert got == sorted(np.flatnonzero(mask[b, h].numpy()))[:rsel.shape[-1]]


def test_chunked_lists_window_without_forecast_and_invariants():
    B, H, T, bs, k = 1, 2, 1000, 64, 8
    NB = (T + bs - 1) // bs
    sel, n = O.chunked_selection(None, B, H, T, bs, k)
    for t in range(T):
        bq = t // bs
        lst = list(sel[0, 0, t, :n[0, 0, t]])
        assert lst == sorted({0} | set(range(max(0, bq - k + 1), bq + 1)))[:min(NB, k + 2)]
    rng = np.random.default_rng(5)
    tk = rng.integers(0, NB, size=(B, H, T, k)).astype(np.int32)
    sel, n = O.chunked_selection(tk, B, H, T, bs, k)
    for t in range(T):
        bq = t // bs
        lst = list(sel[0, 1, t, :n[0, 1, t]])
        assert lst[0] == 0 and lst == sorted(set(lst)) and max(lst) <= bq and len(lst) <= min(NB, k + 2)
        assert (sel[0, 1, t, n[0, 1, t]:] == -1).all()


def test_chunked_attention_equals_the_reference_gather_and_sdpa():
    # the chunked path's attention (gather, validity and causal mask, SDPA per
    # query block, sparse.py:334-359) against the oracle's blockwise attention
    # over the same lists, in float64
    B, T, Hq, Hkv, D, bs, k = 1, 300, 6, 2, 16, 64, 4
    R = Hq // Hkv
    rng = np.random.default_rng(9)
    q = rng.standard_normal((B, T, Hq, D))
    kk = rng.standard_normal((B, T, Hkv, D))
    v = rng.standard_normal((B, T, Hkv, D))
    NB = (T + bs - 1) // bs
    tk = _random_topk(rng, B, Hkv, T, NB, k, NB)
    sel, n = O.chunked_selection(tk, B, Hkv, T, bs, k)
    want = O.attention_prefill(q, kk, v, sel, n, bs, True)
    xq = torch.from_numpy(q).transpose(1, 2)
    xk = torch.from_numpy(kk).transpose(1, 2)
    xv = torch.from_numpy(v).transpose(1, 2)
    got = np.zeros((B, T, Hq * D))
    for bq, start, end, _, _, _ in _reference_lists(tk, B, Hkv, T, bs, k):
        # the lists the oracle cut (the same sets where the union fits)
        lst = torch.from_numpy(sel[:, :, start, :].astype(np.int64))            # [B,Hkv,cap]
        valid = torch.from_numpy(np.arange(sel.shape[-1])[None, None, :] < n[:, :, start][..., None])
        lst = torch.where(valid, lst, torch.zeros_like(lst))
        ms = lst.shape[-1]
        pad = NB * bs - T
        kp = F.pad(xk, (0, 0, 0, pad)).view(B, Hkv, NB, bs, D)
        vp = F.pad(xv, (0, 0, 0, pad)).view(B, Hkv, NB, bs, D)
        ix = lst[..., None, None].expand(-1, -1, -1, bs, D)
        kg = torch.gather(kp, 2, ix).reshape(B, Hkv, ms * bs, D)
        vg = torch.gather(vp, 2, ix).reshape(B, Hkv, ms * bs, D)
        pos = (lst[..., None] * bs + torch.arange(bs)).reshape(B, Hkv, 1, ms * bs)
        bval = valid[..., None].expand(-1, -1, -1, bs).reshape(B, Hkv, 1, ms * bs)
        qpos = torch.arange(start, end).view(1, 1, end - start, 1)
        ok = (pos < T) & (pos <= qpos) & bval
        mask = torch.where(ok, torch.zeros(1, dtype=torch.float64), torch.full((1,), float("-inf"),
                                                                              dtype=torch.float64))
        kg = torch.repeat_interleave(kg, R, dim=1)
        vg = torch.repeat_interleave(vg, R, dim=1)
        mask = torch.repeat_interleave(mask, R, dim=1)
        o = F.scaled_dot_product_attention(xq[:, :, start:end], kg, vg, attn_mask=mask)
        got[:, start:end] = o.transpose(1, 2).reshape(B, end - start, Hq * D).numpy()
    assert np.abs(got - want).max() < 1e-10


def test_chunked_restatement_equals_the_oracle_where_the_union_fits():
    # oracle/reference_path.chunked_prefill (the reference's steps, the CPU
    # baseline of the chunked leg) against the oracle's lists and attention,
    # in float64, with picks confined so that no union exceeds the cut (where
    # torch.topk's choice among equal mask entries would decide)
    from oracle import reference_path as RP
    B, T, Hq, Hkv, D, bs, k = 1, 700, 6, 2, 16, 64, 8
    rng = np.random.default_rng(21)
    q = rng.standard_normal((B, T, Hq, D))
    kk = rng.standard_normal((B, T, Hkv, D))
    v = rng.standard_normal((B, T, Hkv, D))
    f = rng.standard_normal((B, T, Hkv, D))
    xq, xk, xv = (torch.from_numpy(a).transpose(1, 2) for a in (q, kk, v))
    NB = (T + bs - 1) // bs
    # with k + 2 >= NB the cut never binds
    got = RP.chunked_prefill(xq, xk, xv, torch.from_numpy(f), bs, NB).numpy()
    _, tk, _, _ = O.route(f, O.compress(kk, bs), bs, NB, False)
    sel, n = O.chunked_selection(tk, B, Hkv, T, bs, NB)
    want = O.attention_prefill(q, kk, v, sel, n, bs, True)
    assert np.abs(got - want).max() < 1e-10
    # one forecast per query block: every row picks the same k blocks, so the
    # union ({0, own} and k picks) fits the cut exactly and the selection is real
    k = 4
    fb = np.repeat(rng.standard_normal((B, NB, Hkv, D)), bs, axis=1)[:, :T]
    got = RP.chunked_prefill(xq, xk, xv, torch.from_numpy(fb), bs, k).numpy()
    _, tk, _, _ = O.route(fb, O.compress(kk, bs), bs, k, False)
    sel, n = O.chunked_selection(tk, B, Hkv, T, bs, k)
    assert (n < NB).any()
    assert np.abs(got - O.attention_prefill(q, kk, v, sel, n, bs, True)).max() < 1e-10
    got_w = RP.chunked_prefill(xq, xk, xv, None, bs, 3).numpy()
    sel_w, n_w = O.chunked_selection(None, B, Hkv, T, bs, 3)
    assert np.abs(got_w - O.attention_prefill(q, kk, v, sel_w, n_w, bs, True)).max() < 1e-10
