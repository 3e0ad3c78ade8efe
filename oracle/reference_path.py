"""Op-for-op PyTorch CPU restatement of the reference's sparse attention path.

TEST INFRASTRUCTURE. Used by ``tests/`` (semantic cross-check of the oracle)
and by ``bench.py``'s ``cpu_baseline`` leg (the timed CPU baseline). The
product path never imports it.

It performs the same tensor operations and materialisations as the
reference, so its CPU time is the reference's CPU time on the same inputs:

* block mean of zero-padded keys            model/forecast.py:65-78
* matmul scores, future masked_fill, topk   model/forecast.py:108-130
* O(T^2) allowed mask via scatter/gather,
  additive mask via where, repeat_interleave,
  masked scaled_dot_product_attention       model/attention/sparse.py:226-281
* decode: full-cache recompression, sink/current scatter, topk compaction,
  physical gather, additive mask, SDPA      model/attention/sparse.py:99-183
* chunked prefill (past 8192 tokens): per query block, non-causal selector on
  its rows, mask scatter, future blocks cleared, topk over the 0/1 mask,
  physical gather, validity + causal mask, SDPA
                                            model/attention/sparse.py:284-364

``torch.topk`` leaves the order of tied values unspecified; where that
matters (the -inf ties of the decode routing) the selection it produced is
returned so that callers can compare like with like.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn.functional as F


def block_means(k: torch.Tensor, bs: int) -> torch.Tensor:
    """k: [B,S,H,D] -> [B,NB,H,D] (zero-padded tail divided by bs)."""
    B, S, H, D = k.shape
    nb = (S + bs - 1) // bs
    pad = nb * bs - S
    if pad:
        k = torch.cat([k, k.new_zeros(B, pad, H, D)], dim=1)
    return k.reshape(B, nb, bs, H, D).mean(dim=2)


def select_blocks(forecast: torch.Tensor, reps: torch.Tensor, bs: int, top_k: int,
                  causal: bool = True, query_pos0: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
    """forecast [B,Tq,H,Df], reps [B,NB,H,Df] -> scores [B,H,Tq,NB], topk [B,H,Tq,k].
    Row i of the causal mask sits at position query_pos0 + i (0: the
    reference's row index, forecast.py:123-126)."""
    f = forecast.transpose(1, 2)
    r = reps.transpose(1, 2)
    sc = torch.matmul(f, r.transpose(-1, -2)) * (1.0 / math.sqrt(f.shape[-1]))
    nb = r.shape[2]
    if causal:
        tq = f.shape[2]
        fut = torch.arange(nb).view(1, 1, 1, nb) > ((torch.arange(tq).view(1, 1, tq, 1) + query_pos0) // bs)
        sc = sc.masked_fill(fut, float("-inf"))
    return sc, torch.topk(sc, k=min(top_k, nb), dim=-1).indices


def sparse_prefill(xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor,
                   forecast: Optional[torch.Tensor], bs: int, top_k: int,
                   causal: bool = True) -> torch.Tensor:
    """xq [B,Hq,T,D], xk/xv [B,Hkv,T,D] -> [B,T,Hq*D] (before wo)."""
    B, Hq, T, D = xq.shape
    Hkv = xk.shape[1]
    rep = Hq // Hkv
    nb = (T + bs - 1) // bs
    tq = torch.arange(T).view(1, 1, T, 1)
    tk = torch.arange(T).view(1, 1, 1, T)
    bq, bk = tq // bs, tk // bs
    if nb <= 2 or forecast is None:
        k_e = torch.repeat_interleave(xk, rep, dim=1)
        v_e = torch.repeat_interleave(xv, rep, dim=1)
        o = F.scaled_dot_product_attention(xq, k_e, v_e, is_causal=causal)
        return o.transpose(1, 2).reshape(B, T, Hq * D)
    reps = block_means(xk.transpose(1, 2), bs)
    _, top = select_blocks(forecast, reps, bs, top_k, causal)
    chosen = torch.zeros(B, Hkv, T, nb, dtype=torch.bool)
    chosen.scatter_(-1, top.clamp(0, nb - 1), True)
    allowed = (bk == bq) | (bk == 0) | chosen.gather(-1, bk.expand(B, Hkv, T, T))
    if causal:
        allowed = allowed & (tk <= tq)
    add = torch.where(allowed, torch.zeros(1, dtype=xq.dtype),
                      torch.full((1,), float("-inf"), dtype=xq.dtype))
    k_e = torch.repeat_interleave(xk, rep, dim=1)
    v_e = torch.repeat_interleave(xv, rep, dim=1)
    add = torch.repeat_interleave(add, rep, dim=1)
    o = F.scaled_dot_product_attention(xq, k_e, v_e, attn_mask=add)
    return o.transpose(1, 2).reshape(B, T, Hq * D)


def chunked_prefill(xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor,
                    forecast: Optional[torch.Tensor], bs: int, top_k: int) -> torch.Tensor:
    """The chunked-gather prefill, xq [B,Hq,T,D], xk/xv [B,Hkv,T,D], forecast
    [B,T,Hkv,Df] or None -> [B,T,Hq*D] (before wo). One iteration per query
    block of bs rows, each with the reference's own tensor operations."""
    B, Hq, T, D = xq.shape
    Hkv = xk.shape[1]
    rep = Hq // Hkv
    nb = (T + bs - 1) // bs
    reps = block_means(xk.transpose(1, 2), bs)
    max_sel = min(nb, top_k + 2)
    outs = []
    for b_q in range(nb):
        s0, s1 = b_q * bs, min(T, (b_q + 1) * bs)
        mask = torch.zeros((B, Hkv, nb), dtype=torch.bool)
        mask.scatter_(-1, torch.zeros((B, Hkv, 1), dtype=torch.long), True)
        mask.scatter_(-1, torch.full((B, Hkv, 1), b_q, dtype=torch.long), True)
        if forecast is not None and b_q > 0:
            _, top = select_blocks(forecast[:, s0:s1], reps, bs, top_k, causal=False)
            mask.scatter_(-1, top.reshape(B, Hkv, -1).clamp(0, nb - 1), True)
        else:
            for j in range(max(0, b_q - top_k + 1), b_q + 1):
                mask.scatter_(-1, torch.full((B, Hkv, 1), j, dtype=torch.long), True)
        mask[:, :, torch.arange(nb) > b_q] = False
        val, sel = torch.topk(mask.float(), k=max_sel, dim=-1)
        pad = nb * bs - T
        kp = F.pad(xk, (0, 0, 0, pad)).view(B, Hkv, nb, bs, D)
        vp = F.pad(xv, (0, 0, 0, pad)).view(B, Hkv, nb, bs, D)
        ix = sel[..., None, None].expand(-1, -1, -1, bs, D)
        kg = torch.gather(kp, 2, ix).reshape(B, Hkv, max_sel * bs, D)
        vg = torch.gather(vp, 2, ix).reshape(B, Hkv, max_sel * bs, D)
        pos = (sel[..., None] * bs + torch.arange(bs)).reshape(B, Hkv, 1, max_sel * bs)
        ok = (val > 0.5)[..., None].expand(-1, -1, -1, bs).reshape(B, Hkv, 1, max_sel * bs)
        qpos = torch.arange(s0, s1).view(1, 1, s1 - s0, 1)
        valid = (pos < T) & (pos <= qpos) & ok
        add = torch.where(valid, torch.zeros(1, dtype=xq.dtype), torch.full((1,), float("-inf"), dtype=xq.dtype))
        kg = torch.repeat_interleave(kg, rep, dim=1)
        vg = torch.repeat_interleave(vg, rep, dim=1)
        add = torch.repeat_interleave(add, rep, dim=1)
        outs.append(F.scaled_dot_product_attention(xq[:, :, s0:s1], kg, vg, attn_mask=add))
    return torch.cat(outs, dim=2).transpose(1, 2).reshape(B, T, Hq * D)


def sparse_decode(xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor, S: int,
                  forecast: Optional[torch.Tensor], bs: int, top_k: int, routing: str = "reference"):
    """xq [B,Hq,1,D], xk/xv [B,Hkv,S,D] (S includes the new token), forecast
    [B,1,Hkv,Df] -> (out [B,1,Hq*D], selected block indices [B,Hkv,m],
    validity [B,Hkv,m]). routing "reference" masks the scores at row 0 as
    sparse.py:139 does; "absolute" at the query's position S - 1 (the same
    operations, another mask row)."""
    B, Hq, _, D = xq.shape
    Hkv = xk.shape[1]
    rep = Hq // Hkv
    nb = (S + bs - 1) // bs
    cb = (S - 1) // bs
    m = min(nb, top_k + 2)
    if nb <= m:
        o = F.scaled_dot_product_attention(xq, torch.repeat_interleave(xk[:, :, :S], rep, 1),
                                           torch.repeat_interleave(xv[:, :, :S], rep, 1))
        idx = torch.arange(nb).expand(B, Hkv, nb)
        return o.transpose(1, 2).reshape(B, 1, Hq * D), idx, torch.ones(B, Hkv, nb, dtype=torch.bool)
    mark = torch.zeros(B, Hkv, nb, dtype=torch.bool)
    mark[:, :, 0] = True
    mark[:, :, cb] = True
    if forecast is not None:
        reps = block_means(xk.transpose(1, 2), bs)
        _, top = select_blocks(forecast, reps, bs, top_k, causal=True,
                               query_pos0=S - 1 if routing == "absolute" else 0)
        mark.scatter_(-1, top[:, :, 0, :].clamp(0, nb - 1), True)
    else:
        mark[:, :, max(0, cb - top_k + 1):cb + 1] = True
    mark[:, :, cb + 1:] = False
    val, idx = torch.topk(mark.float(), k=m, dim=-1)
    pad = nb * bs - S
    kp = torch.cat([xk, xk.new_zeros(B, Hkv, pad, D)], 2) if pad else xk
    vp = torch.cat([xv, xv.new_zeros(B, Hkv, pad, D)], 2) if pad else xv
    g = idx.view(B, Hkv, m, 1, 1).expand(B, Hkv, m, bs, D)
    kg = torch.gather(kp.view(B, Hkv, nb, bs, D), 2, g).reshape(B, Hkv, m * bs, D)
    vg = torch.gather(vp.view(B, Hkv, nb, bs, D), 2, g).reshape(B, Hkv, m * bs, D)
    pos = (idx.unsqueeze(-1) * bs + torch.arange(bs)).view(B, Hkv, 1, m * bs)
    ok = (pos < S) & (val > 0.5).unsqueeze(-1).expand(B, Hkv, m, bs).reshape(B, Hkv, 1, m * bs)
    add = torch.where(ok, torch.zeros(1, dtype=xq.dtype), torch.full((1,), float("-inf"), dtype=xq.dtype))
    o = F.scaled_dot_product_attention(xq, torch.repeat_interleave(kg, rep, 1),
                                       torch.repeat_interleave(vg, rep, 1),
                                       attn_mask=torch.repeat_interleave(add, rep, 1))
    return o.transpose(1, 2).reshape(B, 1, Hq * D), idx, val > 0.5
