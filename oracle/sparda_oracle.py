"""CPU oracle for SparDA's forecast-guided block-sparse attention path.

TEST INFRASTRUCTURE. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
reference results are compared with (or as the timed CPU baseline). The product path never imports it.

What it restates (citations into tyborra/local-research-Small-Language-Model):

* ``compress``   — KVBlockCompressor.forward, model/forecast.py:57-78
* ``scores``     — ForecastBlockSelector.forward scoring + causal mask,
                   model/forecast.py:108-126
* ``topk``       — torch.topk at model/forecast.py:128-129, ties fixed to
                   "lower block index first"
* ``sel_from_topk`` / ``route`` — the allowed-block rule of the prefill
                   (model/attention/sparse.py:231-253) and the decode
                   selection (model/attention/sparse.py:126-154)
* ``sel_fixed``  — dense fallback and the static windows
                   (model/attention/sparse.py:113-123, 142-147, 250-251)
* ``chunked_selection`` — the per-query-block lists of the chunked-gather
                   prefill (model/attention/sparse.py:303-333): sink + own
                   block + the union of the block's rows' non-causal top-k
                   (or the static window), future blocks dropped, cut to
                   min(NB, k+2) by the lowest block indices
* ``gather_blocks`` — gather_kv_blocks, model/attention/sparse.py:19-62
* ``attention_prefill`` — masked SDPA over the allowed set,
                   model/attention/sparse.py:255-281, computed per query row in
                   float64 over exactly the allowed keys (never an O(T^2) mask)
* ``attention_prefill_masked`` — the same with an explicit additive mask
                   and the attention weights (return_attn_weights),
                   model/attention/sparse.py:206-221, 255-281
* ``attention_decode`` / ``decode_step`` — model/attention/sparse.py:99-183
* ``teacher_block_scores`` — TeacherBlockSelector.forward steps 1-3,
                   model/forecast.py:160-184 (head mean, block sums, causal 0)
* ``dense_weights`` / ``teacher_block_mass`` — the dense softmax weights the
                   teacher consumes (model/attention/dense.py with
                   return_attn_weights), float64, then the block mass

The compressor, scorer and top-k run in C (``sparda_oracle.c``) so that the
fp32 summation / fma order is exactly the documented one; everything else is
numpy.
"""

from __future__ import annotations

import ctypes
import os
import subprocess
from typing import Optional, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

# Selection modes (same numbering as the library's SPARDA_SEL_*).
SEL_DENSE = 0
SEL_WINDOW_DECODE = 1
SEL_WINDOW_PREFILL = 2


def build() -> str:
    """Compile the C restatement (idempotent)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i64, f32, ptr, cint = ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_int
        L.oracle_compress.argtypes = [ptr, i64, i64, i64, i64, i64, i64, i64, i64, ptr]
        L.oracle_scores.argtypes = [ptr, i64, i64, i64, ptr, i64, i64, i64, i64, i64, i64,
                                    cint, i64, f32, ptr]
        L.oracle_topk.argtypes = [ptr, i64, i64, i64, ptr]
        L.oracle_sel_from_topk.argtypes = [ptr, i64, i64, ptr, cint, i64, ptr, ptr]
        for f in (L.oracle_compress, L.oracle_scores, L.oracle_topk, L.oracle_sel_from_topk):
            f.restype = None
        _lib = L
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def num_blocks(S: int, bs: int) -> int:
    return (S + bs - 1) // bs


# --------------------------------------------------------------------------
# compressor / router
# --------------------------------------------------------------------------

def compress(k, bs: int) -> np.ndarray:
    """k: [B,S,H,D] -> prototypes [B,NB,H,D] fp32 (sequential fp32 sum / bs)."""
    k = _f32(k)
    B, S, H, D = k.shape
    NB = num_blocks(S, bs)
    out = np.empty((B, NB, H, D), np.float32)
    lib().oracle_compress(_p(k), B, S, H, D, S * H * D, H * D, D, bs, _p(out))
    return out


def scores(f, protos, bs: int, causal: bool = True, score_pos0: int = 0,
           scale: Optional[float] = None) -> np.ndarray:
    """f: [B,Tq,H,Df], protos: [B,NB,H,Df] -> fp32 scores [B,H,Tq,NB]."""
    f = _f32(f)
    P = _f32(protos)
    B, Tq, H, Df = f.shape
    NB = P.shape[1]
    assert P.shape == (B, NB, H, Df), "forecast heads must equal KV heads (model/forecast.py:110)"
    if scale is None:
        scale = float(np.float32(1.0 / np.sqrt(Df)))
    out = np.empty((B, H, Tq, NB), np.float32)
    lib().oracle_scores(_p(f), Tq * H * Df, H * Df, Df, _p(P), B, Tq, H, Df, NB, bs,
                        int(causal), score_pos0, scale, _p(out))
    return out


def topk(score_rows, k: int) -> np.ndarray:
    """Canonical top-k over the last axis: score desc, then lower index."""
    s = _f32(score_rows)
    lead = s.shape[:-1]
    NB = s.shape[-1]
    rows = int(np.prod(lead)) if lead else 1
    ke = min(k, NB)
    out = np.empty((rows, ke), np.int32)
    lib().oracle_topk(_p(s.reshape(rows, NB)), rows, NB, k, _p(out))
    return out.reshape(*lead, ke)


def own_blocks(Tq: int, bs: int, NB: int, query_pos0: int = 0) -> np.ndarray:
    t = np.arange(Tq, dtype=np.int64)
    return np.minimum((query_pos0 + t) // bs, NB - 1)


def sel_from_topk(tk: np.ndarray, own: np.ndarray, causal: bool, cap: int):
    """tk: [..., Tq, ke]; own: [Tq] broadcast over the leading axes."""
    tk = np.ascontiguousarray(tk, dtype=np.int32)
    lead = tk.shape[:-1]
    ke = tk.shape[-1]
    assert cap >= ke + 2
    rows = int(np.prod(lead))
    own_full = np.ascontiguousarray(np.broadcast_to(own, lead).reshape(rows), dtype=np.int64)
    sel = np.empty((rows, cap), np.int32)
    n = np.empty((rows,), np.int32)
    lib().oracle_sel_from_topk(_p(tk.reshape(rows, ke)), rows, ke, _p(own_full), int(causal),
                               cap, _p(sel), _p(n))
    return sel.reshape(*lead, cap), n.reshape(lead)


def route(f, protos, bs: int, k: int, causal: bool = True, score_pos0: int = 0,
          query_pos0: int = 0, scale: Optional[float] = None, cap: Optional[int] = None):
    """scores [B,H,Tq,NB], topk [B,H,Tq,ke], sel [B,H,Tq,cap], n_sel [B,H,Tq]."""
    sc = scores(f, protos, bs, causal, score_pos0, scale)
    NB = sc.shape[-1]
    tk = topk(sc, k)
    ke = tk.shape[-1]
    cap = cap if cap is not None else ke + 2
    own = own_blocks(sc.shape[2], bs, NB, query_pos0)
    sel, n = sel_from_topk(tk, own, causal, cap)
    return sc, tk, sel, n


def sel_fixed(mode: int, B: int, Tq: int, H: int, NB: int, bs: int, k: int,
              query_pos0: int = 0, cap: Optional[int] = None):
    """Forecast-free selection lists (dense / static windows)."""
    own = own_blocks(Tq, bs, NB, query_pos0)
    if mode == SEL_DENSE:
        need = int(own.max()) + 1
    else:
        need = k + 2
    cap = cap if cap is not None else need
    sel = np.full((Tq, cap), -1, np.int32)
    n = np.zeros((Tq,), np.int32)
    for t in range(Tq):
        o = int(own[t])
        if mode == SEL_DENSE:
            blocks = list(range(0, o + 1))
        elif mode == SEL_WINDOW_DECODE:
            blocks = sorted({0} | set(range(max(0, o - k + 1), o + 1)))
        elif mode == SEL_WINDOW_PREFILL:
            blocks = sorted({0} | set(range(max(0, o - k), o + 1)))
        else:
            raise ValueError(mode)
        assert len(blocks) <= cap
        sel[t, :len(blocks)] = blocks
        n[t] = len(blocks)
    sel = np.broadcast_to(sel, (B, H, Tq, cap)).copy()
    n = np.broadcast_to(n, (B, H, Tq)).copy()
    return sel, n


def chunked_selection(tk, B: int, H: int, T: int, bs: int, k: int):
    """Lists of the chunked-gather prefill (model/attention/sparse.py:303-333).

    For query block bq (rows bq*bs .. min(T, (bq+1)*bs) - 1): {0, bq} U the
    union of those rows' top-k picks (tk [B,H,T,ke], the non-causal per-row
    top-k of sparse.py:321-323) when tk is given and bq > 0, else U the
    static window [max(0, bq-k+1), bq] (sparse.py:324-328); blocks past bq
    dropped (sparse.py:330-331); then cut to min(NB, k+2) entries. The cut is
    torch.topk over a 0/1 mask (sparse.py:333), whose order among equal
    values is unspecified; here the lowest block indices are kept (the
    library's tie rule). Every row of the block gets the block's list.
    Returns sel [B,H,T,cap] (ascending, -1 padded), n [B,H,T], cap = min(NB, k+2).
    """
    NB = num_blocks(T, bs)
    cap = min(NB, k + 2)
    sel = np.full((B, H, T, cap), -1, np.int32)
    n = np.zeros((B, H, T), np.int32)
    for b in range(B):
        for h in range(H):
            for bq in range(NB):
                rows = range(bq * bs, min(T, (bq + 1) * bs))
                blocks = {0, bq}
                if tk is not None and bq > 0:
                    blocks |= {int(j) for t in rows for j in np.asarray(tk[b, h, t]).ravel()}
                else:
                    blocks |= set(range(max(0, bq - k + 1), bq + 1))
                lst = sorted(j for j in blocks if 0 <= j <= bq)[:cap]
                for t in rows:
                    sel[b, h, t, :len(lst)] = lst
                    n[b, h, t] = len(lst)
    return sel, n


# --------------------------------------------------------------------------
# gather
# --------------------------------------------------------------------------

def gather_blocks(k, v, idx, bs: int):
    """k, v: [B,H,S,D]; idx: [B,H,n] -> [B,H,n*bs,D], zero beyond S."""
    k = np.asarray(k)
    v = np.asarray(v)
    B, H, S, D = k.shape
    n = idx.shape[-1]
    ko = np.zeros((B, H, n * bs, D), k.dtype)
    vo = np.zeros((B, H, n * bs, D), v.dtype)
    for b in range(B):
        for h in range(H):
            for i in range(n):
                j = int(idx[b, h, i])
                lo, hi = j * bs, min((j + 1) * bs, S)
                if hi > lo:
                    ko[b, h, i * bs:i * bs + hi - lo] = k[b, h, lo:hi]
                    vo[b, h, i * bs:i * bs + hi - lo] = v[b, h, lo:hi]
    return ko, vo


# --------------------------------------------------------------------------
# attention (float64)
# --------------------------------------------------------------------------

def _softmax_attend(qr: np.ndarray, K: np.ndarray, V: np.ndarray, scale: float) -> np.ndarray:
    """qr: [R,D], K/V: [n,D] (float64) -> [R,D]."""
    s = (qr @ K.T) * scale
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    return (p @ V) / p.sum(axis=1, keepdims=True)


def _keys_for(blocks, bs: int, limit: int) -> np.ndarray:
    """Token indices of the given blocks that are < limit."""
    parts = [np.arange(j * bs, min((j + 1) * bs, limit)) for j in blocks if j * bs < limit]
    return np.concatenate(parts) if parts else np.zeros((0,), np.int64)


def attention_prefill(q, k, v, sel, n_sel, bs: int, causal: bool = True,
                      scale: Optional[float] = None, rows=None) -> np.ndarray:
    """Block-sparse GQA prefill in float64.

    q: [B,T,Hq,D]; k, v: [B,T,Hkv,D]; sel: [B,Hkv,T,cap] or None (dense);
    rows: optional iterable of (b, t) to evaluate (others left NaN).
    Returns [B,T,Hq*D] float64.
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    R = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.full((B, T, Hq * D), np.nan)
    if rows is None:
        rows = [(b, t) for b in range(B) for t in range(T)]
    NB = num_blocks(T, bs)
    for b, t in rows:
        limit = t + 1 if causal else T
        for g in range(Hkv):
            if sel is None:
                blocks = range(NB)
            else:
                blocks = sel[b, g, t, :int(n_sel[b, g, t])]
            keys = _keys_for(blocks, bs, limit)
            qr = q[b, t, g * R:(g + 1) * R]
            o = _softmax_attend(qr, k[b, keys, g], v[b, keys, g], scale)
            out[b, t, g * R * D:(g + 1) * R * D] = o.reshape(-1)
    return out


def attention_prefill_masked(q, k, v, sel, n_sel, bs: int, causal: bool = True, mask=None,
                             scale: Optional[float] = None, rows=None):
    """The masked-SDPA path with an explicit additive mask and the attention
    weights (model/attention/sparse.py:206-221, 255-281), float64.

    Selections have set semantics (repeated entries count once, entries
    outside [0, NB) attend nothing). mask: broadcastable to [B, Hq, T, T]
    (natural-log units, added to the allowed scores). Returns (out
    [B,T,Hq*D], weights [B,Hq,T,T]); rows not evaluated are NaN. A row with
    no finite score (the mask -inf on every allowed key, or no allowed key)
    is NaN throughout, weights and output, as F.softmax over an all -inf
    row gives it in the reference's weights path (sparse.py:266-268).
    """
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    R = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    NB = num_blocks(T, bs)
    m = None if mask is None else np.broadcast_to(np.asarray(mask, np.float64), (B, Hq, T, T))
    out = np.full((B, T, Hq * D), np.nan)
    w = np.full((B, Hq, T, T), np.nan)
    if rows is None:
        rows = [(b, t) for b in range(B) for t in range(T)]
    for b, t in rows:
        limit = t + 1 if causal else T
        for g in range(Hkv):
            if sel is None:
                blocks = range(NB)
            else:
                blocks = sorted({int(j) for j in sel[b, g, t, :int(n_sel[b, g, t])] if 0 <= j < NB})
            keys = _keys_for(blocks, bs, limit)
            for hh in range(R):
                h = g * R + hh
                s = (k[b, keys, g] @ q[b, t, h]) * scale
                if m is not None:
                    s = s + m[b, h, t, keys]
                if len(keys) == 0 or np.all(s == -np.inf):
                    continue  # no finite score: the NaN row stays
                mx = s.max()
                p = np.exp(s - mx)
                p = p / p.sum()
                row = np.zeros(T)
                row[keys] = p
                w[b, h, t] = row
                out[b, t, h * D:(h + 1) * D] = p @ v[b, keys, g]
    return out, w


def attention_decode(q, kc, vc, S: int, sel, n_sel, bs: int,
                     scale: Optional[float] = None) -> np.ndarray:
    """q: [B,Hq,D]; kc, vc: [B,Smax,Hkv,D]; sel: [B,Hkv,cap] -> [B,Hq*D] float64."""
    q = np.asarray(q, np.float64)
    B, Hq, D = q.shape
    Hkv = kc.shape[2]
    R = Hq // Hkv
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    out = np.empty((B, Hq * D))
    for b in range(B):
        for g in range(Hkv):
            keys = _keys_for(sel[b, g, :int(n_sel[b, g])], bs, S)
            K = np.asarray(kc[b, keys, g], np.float64)
            V = np.asarray(vc[b, keys, g], np.float64)
            o = _softmax_attend(q[b, g * R:(g + 1) * R], K, V, scale)
            out[b, g * R * D:(g + 1) * R * D] = o.reshape(-1)
    return out


def decode_selection(kc, S: int, f, bs: int, k: int, routing: str = "reference",
                     scale: Optional[float] = None):
    """Selection of one decode step (model/attention/sparse.py:109-154).

    kc: [B,Smax,Hkv,D] cache (tokens [0,S) valid); f: [B,Hkv,Df] or None.
    routing: "reference" scores with the causal mask at row 0 (as
    model/attention/sparse.py:139 does), "absolute" at position S-1.
    Returns sel [B,Hkv,k+2], n_sel [B,Hkv] and the fp32 scores (or None).
    """
    kc = np.asarray(kc, np.float32)
    B, _, Hkv, D = kc.shape
    NB = num_blocks(S, bs)
    cb = (S - 1) // bs
    cap = k + 2
    if NB <= k + 2:
        sel, n = sel_fixed(SEL_DENSE, B, 1, Hkv, NB, bs, k, query_pos0=S - 1, cap=cap)
        return sel[:, :, 0], n[:, :, 0], None
    if f is None:
        sel, n = sel_fixed(SEL_WINDOW_DECODE, B, 1, Hkv, NB, bs, k, query_pos0=S - 1, cap=cap)
        return sel[:, :, 0], n[:, :, 0], None
    P = compress(kc[:, :S], bs)
    f4 = np.asarray(f, np.float32).reshape(B, 1, Hkv, -1)
    pos0 = 0 if routing == "reference" else S - 1
    sc = scores(f4, P, bs, True, pos0, scale)
    tk = topk(sc, k)
    own = np.array([cb], np.int64)
    sel, n = sel_from_topk(tk, own, True, cap)
    return sel[:, :, 0], n[:, :, 0], sc[:, :, 0]


def prefetch_selection(kc, length: int, pos: int, f, bs: int, k: int, routing: str = "reference",
                       scale: Optional[float] = None):
    """Selection made for the query at position `pos` from the first `length`
    cached tokens (the one-token lookahead of AsyncForecastOffloadAttention.prefetch,
    model/attention/async_offload.py:196-260): own = pos // bs; every block
    0..own when own + 1 <= k + 2 (the small-context branch, 203-239); otherwise
    {0, own} U top-k of the prototypes of blocks [0, ceil(length/bs)) scored
    with the causal mask at row 0 ("reference", forecast.py:120-126) or at pos
    ("absolute"). Returns sel [B,Hkv,k+2], n_sel [B,Hkv]."""
    kc = np.asarray(kc, np.float32)
    B, _, Hkv, D = kc.shape
    own = pos // bs
    cap = k + 2
    if own + 1 <= k + 2:
        sel = np.full((B, Hkv, cap), -1, np.int32)
        sel[:, :, :own + 1] = np.arange(own + 1, dtype=np.int32)
        return sel, np.full((B, Hkv), own + 1, np.int32)
    P = compress(kc[:, :length], bs)
    f4 = np.asarray(f, np.float32).reshape(B, 1, Hkv, -1)
    sc = scores(f4, P, bs, True, 0 if routing == "reference" else pos, scale)
    tk = topk(sc, k)
    sel, n = sel_from_topk(tk, np.array([own], np.int64), True, cap)
    return sel[:, :, 0], n[:, :, 0]


def decode_step(q, kc, vc, S: int, f, bs: int, k: int, routing: str = "reference",
                scale: Optional[float] = None):
    """Full decode step: selection then attention. Returns (out [B,Hq*D], sel, n_sel)."""
    sel, n, _ = decode_selection(kc, S, f, bs, k, routing)
    return attention_decode(q, kc, vc, S, sel, n, bs, scale), sel, n


def prefill_selection(k, f, bs: int, topk_blocks: int, causal: bool = True,
                      scale: Optional[float] = None):
    """Routing of a prefill (model/attention/sparse.py:233-247): returns sel, n_sel."""
    P = compress(k, bs)
    _, _, sel, n = route(f, P, bs, topk_blocks, causal, 0, 0, scale)
    return sel, n


def teacher_block_scores(attn_weights, bs: int, R: int, causal: bool = True) -> np.ndarray:
    """TeacherBlockSelector.forward steps 1-3 (model/forecast.py:160-184) in
    float64: weights [B,Hq,Tq,Tk] -> mean over the R query heads of each KV
    head, zero-padded to whole blocks, summed per block, future blocks 0."""
    w = np.asarray(attn_weights, np.float64)
    B, Hq, Tq, Tk = w.shape
    G = Hq // R
    kv = w.reshape(B, G, R, Tq, Tk).mean(axis=2)
    NB = num_blocks(Tk, bs)
    pad = np.zeros((B, G, Tq, NB * bs), np.float64)
    pad[..., :Tk] = kv
    out = pad.reshape(B, G, Tq, NB, bs).sum(axis=-1)
    if causal:
        t = np.arange(Tq)[:, None]
        j = np.arange(NB)[None, :]
        out[..., (j > t // bs)] = 0.0
    return out


def dense_weights(q, k, causal: bool = True, scale: Optional[float] = None) -> np.ndarray:
    """Post-softmax attention weights [B,Hq,T,T] in float64 from q [B,T,Hq,D],
    k [B,T,Hkv,D] (query head h reads KV head h // (Hq/Hkv)), as the dense
    backend's return_attn_weights gives them."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    B, T, Hq, D = q.shape
    R = Hq // k.shape[2]
    if scale is None:
        scale = 1.0 / np.sqrt(D)
    w = np.empty((B, Hq, T, T), np.float64)
    for b in range(B):
        for h in range(Hq):
            s = (q[b, :, h, :] @ k[b, :, h // R, :].T) * scale
            if causal:
                s[np.triu_indices(T, 1)] = -np.inf
            s = s - s.max(axis=1, keepdims=True)
            e = np.exp(s)
            w[b, h] = e / e.sum(axis=1, keepdims=True)
    return w


def teacher_block_mass(q, k, bs: int, causal: bool = True, scale: Optional[float] = None) -> np.ndarray:
    """Teacher block mass [B,Hkv,T,NB] (float64) from q and k: dense weights,
    then teacher_block_scores."""
    R = np.asarray(q).shape[2] // np.asarray(k).shape[2]
    return teacher_block_scores(dense_weights(q, k, causal, scale), bs, R, causal)
