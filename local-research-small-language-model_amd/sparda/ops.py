"""Tensor-level wrappers over libsparda's C ABI.

PyTorch provides device memory and the current HIP stream; every computation
runs in libsparda's HIP kernels. Tensors must live on a GPU device: a CPU
tensor raises instead of falling back to another implementation.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from . import _lib
from ._lib import call

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def _dtype_code(t: torch.Tensor) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise TypeError(f"sparda: unsupported dtype {t.dtype} (float32 or bfloat16)") from None


def require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not isinstance(t, torch.Tensor):
            raise TypeError(f"sparda: expected a tensor, got {type(t).__name__}")
        if t.device.type != "cuda":
            raise RuntimeError(
                f"sparda: HIP kernels need tensors on a GPU device, got a {t.device.type} tensor "
                "(there is no CPU implementation)")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"sparda: tensors on different devices ({dev} vs {t.device})")
    return dev


def _inference_only(*tensors: Optional[torch.Tensor]) -> None:
    if torch.is_grad_enabled() and any(t is not None and t.requires_grad for t in tensors):
        raise RuntimeError("sparda: the HIP sparse attention path is inference-only; "
                           "run it under torch.no_grad() / torch.inference_mode()")


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _rowmajor(t: torch.Tensor) -> torch.Tensor:
    """Innermost stride 1 (other strides arbitrary)."""
    return t if t.stride(-1) == 1 else t.contiguous()


def default_scale(dim: int) -> float:
    return 1.0 / math.sqrt(dim)


# ---------------------------------------------------------------------------
# compressor / router
# ---------------------------------------------------------------------------

def compress(k: torch.Tensor, block_size: int) -> torch.Tensor:
    """k [B,S,H,D] (fp32/bf16) -> prototypes [B,NB,H,D] fp32 (model/forecast.py:57-78)."""
    dev = require_device(k)
    _inference_only(k)
    k = _rowmajor(k)
    B, S, H, D = k.shape
    NB = (S + block_size - 1) // block_size
    out = torch.empty((B, NB, H, D), dtype=torch.float32, device=dev)
    sb, ss, sh, _ = k.stride()
    call("sparda_compress", k.data_ptr(), _dtype_code(k), B, S, H, D, sb, ss, sh, block_size,
         out.data_ptr(), _stream(dev))
    return out


def route(forecast: torch.Tensor, protos: torch.Tensor, block_size: int, top_k: int,
          causal: bool = True, score_pos0: int = 0, query_pos0: int = 0,
          scale: Optional[float] = None, want_topk: bool = True, want_scores: bool = False,
          want_sel: bool = False, sel_cap: Optional[int] = None):
    """Fused score + top-k router (model/forecast.py:89-130).

    forecast [B,Tq,H,Df], protos [B,NB,H,Df] fp32.
    Returns (topk int32 [B,H,Tq,ke] | None, scores fp32 [B,H,Tq,NB] | None,
    sel int32 [B,H,Tq,cap] | None, n_sel int32 [B,H,Tq] | None).
    """
    dev = require_device(forecast, protos)
    _inference_only(forecast)
    forecast = _rowmajor(forecast)
    if protos.dtype != torch.float32 or not protos.is_contiguous():
        protos = protos.float().contiguous()
    B, Tq, H, Df = forecast.shape
    if protos.shape[0] != B or protos.shape[2] != H or protos.shape[3] != Df:
        raise AssertionError(f"Mismatch: forecast {tuple(forecast.shape)} vs prototypes {tuple(protos.shape)}")
    NB = protos.shape[1]
    ke = min(top_k, NB)
    if scale is None:
        scale = default_scale(Df)
    topk = torch.empty((B, H, Tq, ke), dtype=torch.int32, device=dev) if want_topk else None
    scores = torch.empty((B, H, Tq, NB), dtype=torch.float32, device=dev) if want_scores else None
    sel = n_sel = None
    if want_sel:
        cap = sel_cap if sel_cap is not None else ke + 2
        sel = torch.empty((B, H, Tq, cap), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, H, Tq), dtype=torch.int32, device=dev)
    else:
        cap = 0
    fsb, fst, fsh, _ = forecast.stride()
    call("sparda_route", forecast.data_ptr(), _dtype_code(forecast), fsb, fst, fsh, protos.data_ptr(),
         B, Tq, H, Df, NB, block_size, top_k, int(causal), score_pos0, query_pos0, float(scale),
         topk.data_ptr() if topk is not None else None,
         scores.data_ptr() if scores is not None else None,
         sel.data_ptr() if sel is not None else None,
         n_sel.data_ptr() if n_sel is not None else None, cap, _stream(dev))
    return topk, scores, sel, n_sel


def topk_scores(scores: torch.Tensor, top_k: int, algo: int = _lib.TOPK_AUTO) -> torch.Tensor:
    """Canonical top-k (score desc, lower index on ties) over the last axis of fp32 scores."""
    dev = require_device(scores)
    s = scores.float().contiguous()
    NB = s.shape[-1]
    rows = s.numel() // NB
    ke = min(top_k, NB)
    out = torch.empty(s.shape[:-1] + (ke,), dtype=torch.int32, device=dev)
    call("sparda_topk_scores", s.data_ptr(), rows, NB, top_k, algo, out.data_ptr(), _stream(dev))
    return out


def select_fixed(mode: int, B: int, Tq: int, H: int, NB: int, block_size: int, top_k: int,
                 query_pos0: int = 0, device=None, sel_cap: Optional[int] = None):
    """Forecast-free selection lists (dense / static windows)."""
    dev = torch.device(device) if device is not None else torch.device("cuda")
    if dev.type != "cuda":
        raise RuntimeError("sparda: select_fixed needs a GPU device")
    if sel_cap is None:
        if mode == _lib.SEL_DENSE:
            sel_cap = min((query_pos0 + Tq - 1) // block_size, NB - 1) + 1
        else:
            sel_cap = top_k + 2
    sel = torch.empty((B, H, Tq, sel_cap), dtype=torch.int32, device=dev)
    n_sel = torch.empty((B, H, Tq), dtype=torch.int32, device=dev)
    call("sparda_select_fixed", mode, B, Tq, H, NB, block_size, top_k, query_pos0, sel.data_ptr(),
         n_sel.data_ptr(), sel_cap, _stream(dev))
    return sel, n_sel


def select_chunked(topk: Optional[torch.Tensor], B: int, H: int, T: int, block_size: int, top_k: int,
                   device=None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Lists of the chunked-gather prefill (model/attention/sparse.py:303-333):
    per query block of block_size rows, {0, own} U the union of its rows'
    top-k picks (topk int32 [B,H,T,ke], route(..., causal=False)'s; None: the
    static window of top_k blocks), blocks past the own one dropped, cut to the
    lowest min(NB, top_k+2). Returns sel [B,H,T,cap], n_sel [B,H,T]."""
    if topk is not None:
        dev = require_device(topk)
        if topk.dtype != torch.int32 or tuple(topk.shape[:3]) != (B, H, T):
            raise ValueError("sparda: select_chunked takes int32 top-k picks [B,H,T,ke]")
        topk = topk.contiguous()
    else:
        dev = torch.device(device) if device is not None else torch.device("cuda")
        if dev.type != "cuda":
            raise RuntimeError("sparda: select_chunked needs a GPU device")
    NB = (T + block_size - 1) // block_size
    cap = min(NB, top_k + 2)
    sel = torch.empty((B, H, T, cap), dtype=torch.int32, device=dev)
    n_sel = torch.empty((B, H, T), dtype=torch.int32, device=dev)
    call("sparda_select_chunked", topk.data_ptr() if topk is not None else None,
         topk.shape[-1] if topk is not None else 0, B, H, T, block_size, top_k, sel.data_ptr(), n_sel.data_ptr(),
         cap, _stream(dev))
    return sel, n_sel


def gather_blocks(k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                  block_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """k, v [B,H,S,D]; block_indices [B,H,n] -> [B,H,n*bs,D] (model/attention/sparse.py:19-62)."""
    dev = require_device(k, v, block_indices)
    _inference_only(k, v)
    if k.dtype != v.dtype or k.shape != v.shape:
        raise ValueError("sparda: k and v must share shape and dtype")
    k = _rowmajor(k)
    v = _rowmajor(v)
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    B, H, S, D = k.shape
    n = block_indices.shape[-1]
    idx = block_indices.to(torch.int32).contiguous()
    ko = torch.empty((B, H, n * block_size, D), dtype=k.dtype, device=dev)
    vo = torch.empty_like(ko)
    sb, sh, ss, _ = k.stride()
    call("sparda_gather_blocks", k.data_ptr(), v.data_ptr(), _dtype_code(k), sb, sh, ss, idx.data_ptr(),
         B, H, S, D, n, block_size, ko.data_ptr(), vo.data_ptr(), _stream(dev))
    return ko, vo


# ---------------------------------------------------------------------------
# attention
# ---------------------------------------------------------------------------

def prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sel: Optional[torch.Tensor],
            n_sel: Optional[torch.Tensor], block_size: int, causal: bool = True,
            scale: Optional[float] = None, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Block-sparse GQA prefill.

    q [B,T,Hq,D], k/v [B,T,Hkv,D] (same dtype), sel/n_sel from ``route`` or
    ``select_fixed`` ([B,Hkv,T,cap] / [B,Hkv,T]) or None for dense.
    Returns out [B,T,Hq*D] in q's dtype.
    """
    dev = require_device(q, k, v, sel, n_sel)
    _inference_only(q, k, v)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q, k, v must share a dtype")
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty((B, T, Hq * D), dtype=q.dtype, device=dev)
    cap = 0
    if sel is not None:
        sel = sel.to(torch.int32).contiguous()
        n_sel = n_sel.to(torch.int32).contiguous()
        cap = sel.shape[-1]
    qsb, qst, qsh, _ = q.stride()
    ksb, kst, ksh, _ = k.stride()
    osb, ost, _ = out.stride()
    call("sparda_prefill", q.data_ptr(), qsb, qst, qsh, k.data_ptr(), v.data_ptr(), ksb, kst, ksh,
         _dtype_code(q), sel.data_ptr() if sel is not None else None,
         n_sel.data_ptr() if n_sel is not None else None, cap, B, T, Hq, Hkv, D, block_size,
         int(causal), float(scale), out.data_ptr(), osb, ost, _stream(dev))
    return out


def _routed_one_launch(q, k, v, forecast, protos, out, block_size: int, ke: int) -> bool:
    """Whether sparda_prefill_routed takes its one-launch path for these
    tensors (a subset of the library's own test: outside it the call gets the
    hand-off buffers the two-launch path needs)."""
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if q.dtype != torch.bfloat16 or D != 64 or forecast.shape[-1] != 64 or block_size not in (32, 64):
        return False
    if forecast.dtype not in (torch.bfloat16, torch.float32) or not 1 <= ke <= 8:
        return False
    if Hq % Hkv or not 1 <= Hq // Hkv <= 4 or (T + block_size - 1) // block_size > 1024:
        return False
    ts = (q, k, v, out)
    if any(t.data_ptr() % 16 for t in ts + (protos,)) or any(st % 8 for t in ts for st in t.stride()[:-1]):
        return False
    # the library's own bound on window-relative offsets (128-token windows)
    return (128 * q.stride(1) + (Hq // Hkv) * q.stride(2) + 64 < (1 << 30)
            and 64 * k.stride(1) + 64 < (1 << 30))


def prefill_routed(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, forecast: torch.Tensor,
                   protos: torch.Tensor, block_size: int, top_k: int, causal: bool = True,
                   scale: Optional[float] = None, route_scale: Optional[float] = None, want_sel: bool = False,
                   sel_cap: Optional[int] = None, out: Optional[torch.Tensor] = None):
    """Router + block-sparse prefill (model/forecast.py:89-130 then
    model/attention/sparse.py:231-281): ``route`` at positions 0.. and
    ``prefill`` on its lists, one launch where the shape allows.

    q [B,T,Hq,D], k/v [B,T,Hkv,D], forecast [B,T,Hkv,Df], protos [B,NB,Hkv,Df]
    fp32 (``compress`` of k). Returns out [B,T,Hq*D], or (out, sel, n_sel)
    with want_sel (the lists ``route`` returns with want_sel and the same
    sel_cap, default min(top_k, NB) + 2).
    """
    dev = require_device(q, k, v, forecast, protos)
    _inference_only(q, k, v, forecast)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q, k, v must share a dtype")
    q, k, v, forecast = _rowmajor(q), _rowmajor(k), _rowmajor(v), _rowmajor(forecast)
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    if protos.dtype != torch.float32 or not protos.is_contiguous():
        protos = protos.float().contiguous()
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    Df = forecast.shape[-1]
    NB = (T + block_size - 1) // block_size
    if tuple(forecast.shape[:3]) != (B, T, Hkv) or tuple(protos.shape) != (B, NB, Hkv, Df):
        raise AssertionError(f"Mismatch: forecast {tuple(forecast.shape)} / prototypes {tuple(protos.shape)} "
                             f"for k {tuple(k.shape)} at block size {block_size}")
    ke = min(top_k, NB)
    if scale is None:
        scale = default_scale(D)
    if route_scale is None:
        route_scale = default_scale(Df)
    if out is None:
        out = torch.empty((B, T, Hq * D), dtype=q.dtype, device=dev)
    sel = n_sel = None
    cap = 0
    if want_sel or not _routed_one_launch(q, k, v, forecast, protos, out, block_size, ke):
        cap = sel_cap if sel_cap is not None else ke + 2
        sel = torch.empty((B, Hkv, T, cap), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, Hkv, T), dtype=torch.int32, device=dev)
    qsb, qst, qsh, _ = q.stride()
    ksb, kst, ksh, _ = k.stride()
    fsb, fst, fsh, _ = forecast.stride()
    osb, ost, _ = out.stride()
    call("sparda_prefill_routed", q.data_ptr(), qsb, qst, qsh, k.data_ptr(), v.data_ptr(), ksb, kst, ksh,
         _dtype_code(q), forecast.data_ptr(), _dtype_code(forecast), fsb, fst, fsh, protos.data_ptr(), Df, top_k,
         float(route_scale), sel.data_ptr() if sel is not None else None,
         n_sel.data_ptr() if n_sel is not None else None, cap, B, T, Hq, Hkv, D, block_size, int(causal),
         float(scale), out.data_ptr(), osb, ost, _stream(dev))
    return (out, sel, n_sel) if want_sel else out


def _chunked_one_launch(q, k, v, out, block_size: int) -> bool:
    """Whether sparda_prefill_chunked takes its one-launch path for these
    tensors (the library's own test; outside it the call gets the hand-off
    buffers the two-launch path needs)."""
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if q.dtype != torch.bfloat16 or D != 64 or block_size != 64 or Hq % Hkv or not 1 <= Hq // Hkv <= 4:
        return False
    ts = (q, k, v)
    if any(t.data_ptr() % 16 for t in ts) or out.data_ptr() % 8:
        return False
    return all(st % 8 == 0 for t in ts for st in t.stride()[:-1]) and all(st % 4 == 0 for st in out.stride()[:-1])


def prefill_chunked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, topk: Optional[torch.Tensor],
                    block_size: int, top_k: int, scale: Optional[float] = None, want_sel: bool = False,
                    out: Optional[torch.Tensor] = None):
    """The chunked-gather prefill (model/attention/sparse.py:303-364) after its
    router: per query block of block_size tokens the list of
    ``select_chunked`` (topk [B,Hkv,T,ke] int32 from ``route(...,
    causal=False)``; None: the static window), then causal attention over it,
    in one launch where the shape allows. q [B,T,Hq,D], k/v [B,T,Hkv,D].
    Returns out [B,T,Hq*D], or (out, sel, n_sel) with want_sel (the lists
    ``select_chunked`` returns)."""
    dev = require_device(q, k, v, topk)
    _inference_only(q, k, v)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q, k, v must share a dtype")
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if topk is not None:
        if topk.dtype != torch.int32 or tuple(topk.shape[:3]) != (B, Hkv, T):
            raise ValueError("sparda: prefill_chunked takes int32 top-k picks [B,Hkv,T,ke]")
        topk = topk.contiguous()
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty((B, T, Hq * D), dtype=q.dtype, device=dev)
    NB = (T + block_size - 1) // block_size
    cap = min(NB, top_k + 2)
    sel = n_sel = None
    if want_sel or not _chunked_one_launch(q, k, v, out, block_size):
        sel = torch.empty((B, Hkv, T, cap), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, Hkv, T), dtype=torch.int32, device=dev)
    qsb, qst, qsh, _ = q.stride()
    ksb, kst, ksh, _ = k.stride()
    osb, ost, _ = out.stride()
    call("sparda_prefill_chunked", q.data_ptr(), qsb, qst, qsh, k.data_ptr(), v.data_ptr(), ksb, kst, ksh,
         _dtype_code(q), topk.data_ptr() if topk is not None else None, topk.shape[-1] if topk is not None else 0,
         top_k, sel.data_ptr() if sel is not None else None, n_sel.data_ptr() if n_sel is not None else None,
         cap if sel is not None else 0, B, T, Hq, Hkv, D, block_size, float(scale), out.data_ptr(), osb, ost,
         _stream(dev))
    return (out, sel, n_sel) if want_sel else out


def prefill_masked(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, sel: Optional[torch.Tensor],
                   n_sel: Optional[torch.Tensor], block_size: int, causal: bool = True,
                   scale: Optional[float] = None, mask: Optional[torch.Tensor] = None,
                   want_weights: bool = False, out: Optional[torch.Tensor] = None):
    """Block-sparse GQA prefill with an additive mask and optionally the
    attention weights (model/attention/sparse.py:206-221, 255-281).

    q [B,T,Hq,D], k/v [B,T,Hkv,D]; sel/n_sel as for ``prefill`` (None: dense).
    mask: additive, broadcastable to [B, H, T, T] with H in {1, Hkv, Hq} (a
    per-KV-head mask applies to that head's query heads, as the reference's
    repeat_interleave does). Returns out [B,T,Hq*D], and with want_weights
    also weights [B,Hq,T,T] (q's dtype, zero outside the allowed set).
    """
    dev = require_device(q, k, v, sel, n_sel, mask)
    _inference_only(q, k, v)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q, k, v must share a dtype")
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty((B, T, Hq * D), dtype=q.dtype, device=dev)
    cap = 0
    if sel is not None:
        sel = sel.to(torch.int32).contiguous()
        n_sel = n_sel.to(torch.int32).contiguous()
        cap = sel.shape[-1]
    mptr, mdt, mst = None, _lib.F32, (0, 0, 0, 0)
    if mask is not None:
        if mask.dtype == torch.bool:
            raise TypeError("sparda: the mask is additive (floating point), as in the reference")
        m = mask if mask.dim() == 4 else mask.reshape((1,) * (4 - mask.dim()) + tuple(mask.shape))
        if m.shape[1] == Hkv and Hkv != Hq:
            m = torch.repeat_interleave(m, Hq // Hkv, dim=1)
        if m.dtype not in (torch.float32, torch.bfloat16):
            m = m.float()
        m = torch.broadcast_to(m, (B, Hq, T, T))
        mptr, mdt, mst = m.data_ptr(), _dtype_code(m), tuple(m.stride())
        mask = m  # keep alive through the call
    w = None
    wst = (0, 0, 0)
    if want_weights:
        w = torch.empty((B, Hq, T, T), dtype=q.dtype, device=dev)
        wst = w.stride()[:3]
    qsb, qst, qsh, _ = q.stride()
    ksb, kst, ksh, _ = k.stride()
    osb, ost, _ = out.stride()
    call("sparda_prefill_masked", q.data_ptr(), qsb, qst, qsh, k.data_ptr(), v.data_ptr(), ksb, kst, ksh,
         _dtype_code(q), sel.data_ptr() if sel is not None else None,
         n_sel.data_ptr() if n_sel is not None else None, cap, B, T, Hq, Hkv, D, block_size,
         int(causal), float(scale), mptr, mdt, *mst, out.data_ptr(), osb, ost,
         w.data_ptr() if w is not None else None, *wst, _stream(dev))
    return (out, w) if want_weights else out


class DecodeWorkspace:
    """Device workspace for ``decode``, grown on demand and reused across steps."""

    def __init__(self, device=None):
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        self.buf: Optional[torch.Tensor] = None

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < nbytes:
            self.buf = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=self.device)
        return self.buf


STATUS_PREFILL_WAIT_TIMEOUT = 1


def status(device=None, clear: bool = True) -> int:
    """The device's status word (STATUS_* bits raised by kernels since it was
    last cleared), read on the current stream; clears it unless clear=False.
    Waits for the stream to reach the read (one .item())."""
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else torch.device(device)
    word = torch.zeros(1, dtype=torch.int32, device=dev)
    _lib.call("sparda_status", word.data_ptr(), 1 if clear else 0, _stream(dev))
    return int(word.item()) & 0xffffffff


def decode_workspace_bytes(B: int, S: int, Hq: int, Hkv: int, D: int, block_size: int, top_k: int) -> int:
    return int(_lib.load().sparda_decode_workspace_bytes(B, S, Hq, Hkv, D, block_size, top_k))


def _dense_split_ws(B: int, Hq: int, Hkv: int, D: int, S: int, block_size: int, dev):
    """(pointer, bytes, tensor) of the split partials of a dense decode of up
    to S tokens (sparda_decode_dense_workspace_bytes; (None, 0, None) when it
    does not split). The tensor comes from torch's allocator, so a call under
    graph capture takes it from the graph's pool; the caller keeps it alive
    until the launch is enqueued."""
    nbytes = int(_lib.load().sparda_decode_dense_workspace_bytes(B, Hq, Hkv, D, S, block_size))
    if nbytes == 0:
        return None, 0, None
    ws = torch.empty(nbytes // 4 + 4, dtype=torch.float32, device=dev)
    return ws.data_ptr(), nbytes, ws


def decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, S: int,
           forecast: Optional[torch.Tensor], block_size: int, top_k: int, routing: str = "reference",
           scale: Optional[float] = None, workspace: Optional[DecodeWorkspace] = None,
           protos_in: Optional[torch.Tensor] = None, want_protos: bool = False,
           want_sel: bool = False, out: Optional[torch.Tensor] = None):
    """One decode step (model/attention/sparse.py:99-183 after the projections).

    q [B,Hq,D] at position S-1; caches [B,Smax,Hkv,D] with tokens [0,S) valid;
    forecast [B,Hkv,Df] or None; routing "reference" | "absolute".
    Returns out [B,Hq*D], or (out, extras) when want_protos / want_sel.
    """
    dev = require_device(q, k_cache, v_cache, forecast, protos_in)
    _inference_only(q, k_cache, v_cache)
    if not (q.dtype == k_cache.dtype == v_cache.dtype):
        raise TypeError("sparda: q and the caches must share a dtype")
    q, k_cache, v_cache = _rowmajor(q), _rowmajor(k_cache), _rowmajor(v_cache)
    if k_cache.stride() != v_cache.stride():
        raise ValueError("sparda: k_cache and v_cache must share strides")
    B, Hq, D = q.shape
    Hkv = k_cache.shape[2]
    if S > k_cache.shape[1] or S <= 0:
        raise ValueError(f"sparda: S={S} outside the cache (capacity {k_cache.shape[1]})")
    if routing not in ("reference", "absolute"):
        raise ValueError(f"sparda: routing must be 'reference' or 'absolute', got {routing!r}")
    if scale is None:
        scale = default_scale(D)
    NB = (S + block_size - 1) // block_size
    if forecast is not None:
        forecast = _rowmajor(forecast.reshape(B, Hkv, -1) if forecast.dim() != 3 else forecast)
    if out is None:
        out = torch.empty((B, Hq * D), dtype=q.dtype, device=dev)
    nbytes = decode_workspace_bytes(B, S, Hq, Hkv, D, block_size, top_k)
    ws = (workspace or DecodeWorkspace(dev)).get(nbytes)
    protos_out = torch.empty((B, NB, Hkv, D), dtype=torch.float32, device=dev) if want_protos else None
    sel = n_sel = None
    if want_sel:
        sel = torch.empty((B, Hkv, top_k + 2), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, Hkv), dtype=torch.int32, device=dev)
    if protos_in is not None:
        protos_in = protos_in.float().contiguous()
    qsb, qsh, _ = q.stride()
    ksb, kss, ksh, _ = k_cache.stride()
    fsb = fsh = 0
    fdt = _lib.F32
    if forecast is not None:
        fsb, fsh, _ = forecast.stride()
        fdt = _dtype_code(forecast)
    call("sparda_decode", q.data_ptr(), qsb, qsh, k_cache.data_ptr(), v_cache.data_ptr(), ksb, kss, ksh,
         _dtype_code(q), forecast.data_ptr() if forecast is not None else None, fdt, fsb, fsh,
         B, S, Hq, Hkv, D, block_size, top_k,
         _lib.ROUTE_ABSOLUTE if routing == "absolute" else _lib.ROUTE_REFERENCE, float(scale),
         protos_in.data_ptr() if protos_in is not None else None,
         protos_out.data_ptr() if protos_out is not None else None,
         sel.data_ptr() if sel is not None else None, n_sel.data_ptr() if n_sel is not None else None,
         out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), _stream(dev))
    if want_protos or want_sel:
        return out, {"protos": protos_out, "sel": sel, "n_sel": n_sel}
    return out


def decode_selected(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, S: int, block_size: int,
                    sel: Optional[torch.Tensor] = None, n_sel: Optional[torch.Tensor] = None,
                    compact: bool = False, k_new: Optional[torch.Tensor] = None,
                    v_new: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                    out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode attention of q [B,Hq,D] (position S-1) over the blocks sel[b,g,:n_sel]
    (model/attention/sparse.py:154-181; offload.py:247-278; async_offload.py:380-489).

    compact=False: k/v are caches [B,Smax,Hkv,D] read in place. compact=True:
    k/v are fetched block buffers [B,Hkv,cap,bs,D], slot i holding block
    sel[b,g,i]. sel=None: dense over [0, S). k_new/v_new [B,Hkv,D]: the key and
    value of position S-1 (overriding what k/v hold there).
    """
    dev = require_device(q, k, v, sel, n_sel, k_new, v_new)
    _inference_only(q, k, v, k_new, v_new)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q, k and v must share a dtype")
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    if k.stride() != v.stride():
        raise ValueError("sparda: k and v must share strides")
    B, Hq, D = q.shape
    if compact:
        if sel is None:
            raise ValueError("sparda: compact block buffers need a selection")
        _, Hkv, cap, bs_, _ = k.shape
        if bs_ != block_size or cap != sel.shape[-1]:
            raise ValueError("sparda: compact buffers must be [B,Hkv,sel_cap,block_size,D]")
        kv_sb, kv_sh, _, kv_ss, _ = k.stride()
    else:
        Hkv = k.shape[2]
        if S > k.shape[1] or S <= 0:
            raise ValueError(f"sparda: S={S} outside the cache (capacity {k.shape[1]})")
        kv_sb, kv_ss, kv_sh, _ = k.stride()
    cap = 0
    if sel is not None:
        if sel.dtype != torch.int32 or n_sel is None or n_sel.dtype != torch.int32:
            raise TypeError("sparda: sel / n_sel must be int32 tensors")
        sel, n_sel = sel.contiguous(), n_sel.contiguous()
        cap = sel.shape[-1]
    nsb = nsh = 0
    if k_new is not None:
        k_new = _rowmajor(k_new.reshape(B, Hkv, D))
        v_new = _rowmajor(v_new.reshape(B, Hkv, D))
        if k_new.stride() != v_new.stride():
            raise ValueError("sparda: k_new and v_new must share strides")
        nsb, nsh, _ = k_new.stride()
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty((B, Hq * D), dtype=q.dtype, device=dev)
    qsb, qsh, _ = q.stride()
    # dense (no selection) on the matrix cores: the blocks split over workgroups, partials in a workspace
    split = sel is None and q.dtype == torch.bfloat16 and D == 64 and block_size in (32, 64)
    ws_ptr, ws_bytes, ws = _dense_split_ws(B, Hq, Hkv, D, S, block_size, dev) if split else (None, 0, None)
    call("sparda_decode_selected", q.data_ptr(), qsb, qsh, k.data_ptr(), v.data_ptr(), kv_sb, kv_ss, kv_sh,
         _dtype_code(q), int(compact), sel.data_ptr() if sel is not None else None,
         n_sel.data_ptr() if n_sel is not None else None, cap,
         k_new.data_ptr() if k_new is not None else None, v_new.data_ptr() if v_new is not None else None,
         nsb, nsh, B, S, Hq, Hkv, D, block_size, float(scale), out.data_ptr(), out.stride(0), ws_ptr, ws_bytes,
         _stream(dev))
    del ws
    return out


def teacher_block_mass(q: torch.Tensor, k: torch.Tensor, block_size: int = 64, causal: bool = True,
                       scale: Optional[float] = None) -> torch.Tensor:
    """Dense attention probability per (query row, KV block), averaged over the
    query heads of each KV head (model/forecast.py:141-193, steps 1-3), from
    q [B,T,Hq,64] and k [B,T,Hkv,64] bf16 without materialising the weights.
    Returns [B,Hkv,T,ceil(T/64)] fp32."""
    dev = require_device(q, k)
    _inference_only(q, k)
    q, k = _rowmajor(q), _rowmajor(k)
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    if k.shape[0] != B or k.shape[1] != T or k.shape[3] != D:
        raise AssertionError(f"Mismatch: q {tuple(q.shape)} vs k {tuple(k.shape)}")
    if scale is None:
        scale = default_scale(D)
    NB = (T + block_size - 1) // block_size
    mass = torch.empty((B, Hkv, T, NB), dtype=torch.float32, device=dev)
    qsb, qst, qsh, _ = q.stride()
    ksb, kst, ksh, _ = k.stride()
    call("sparda_teacher_mass", q.data_ptr(), qsb, qst, qsh, k.data_ptr(), ksb, kst, ksh, _dtype_code(q),
         B, T, Hq, Hkv, D, block_size, int(causal), float(scale), mass.data_ptr(), _stream(dev))
    return mass


def produce(x: torch.Tensor, w_stacked: torch.Tensor, n_q: int, n_kv: int, n_f: int, eps: float,
            rope_cos: torch.Tensor, rope_sin: torch.Tensor, pos0: int = 0,
            f_dtype: torch.dtype = torch.bfloat16, pos_dev: Optional[torch.Tensor] = None,
            k_cache: Optional[torch.Tensor] = None, v_cache: Optional[torch.Tensor] = None):
    """RMSNorm + q / k / v / forecast projections + RoPE in one kernel
    (model/transformer.py:104-107; model/norm.py:15-21; model/forecast.py:30-40;
    model/attention/base.py:38-52; model/rope.py:34-65).

    x [B,T,C] bf16; w_stacked [n_q + 2*n_kv + n_f, C] bf16 = [wq; wk; wv; wf]
    with the RMSNorm weight folded into its columns; rope tables [L, 32] fp32.
    Returns q [B,T,n_q/64,64], k, v [B,T,n_kv/64,64] (bf16, q and k rotated at
    positions pos0..pos0+T-1) and f [B,T,n_f/64,64] of f_dtype.

    pos_dev: a one-element int64 device tensor holding the first position,
    read when the kernel runs (pos0 must then be 0; positions are clamped into
    the tables), for launches recorded once and replayed every decode step.
    With pos_dev, k_cache / v_cache ([B,Smax,n_kv/64,64] bf16) also receive
    the new keys and values as rows *pos_dev + t (the cache append of
    KVCache.update, model/attention/base.py:19-29; decode-sized batches,
    B*T <= 16); block sums are then the decode launch's to update."""
    dev = require_device(x, w_stacked, rope_cos, rope_sin, pos_dev)
    _inference_only(x, w_stacked)
    if x.dtype != torch.bfloat16 or w_stacked.dtype != torch.bfloat16:
        raise TypeError("sparda: produce takes bf16 activations and weights")
    B, T, C = x.shape
    x2 = x.reshape(B * T, C)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    w_stacked = w_stacked.contiguous()
    if tuple(w_stacked.shape) != (n_q + 2 * n_kv + n_f, C):
        raise AssertionError(f"Mismatch: stacked weight {tuple(w_stacked.shape)} vs ({n_q + 2 * n_kv + n_f}, {C})")
    rope_cos = rope_cos.float().contiguous()
    rope_sin = rope_sin.float().contiguous()
    if rope_cos.shape[-1] != 32 or rope_sin.shape != rope_cos.shape:
        raise AssertionError("sparda: RoPE tables must be [L, 32] (head dim 64)")
    q = torch.empty((B, T, n_q // 64, 64), dtype=torch.bfloat16, device=dev)
    k = torch.empty((B, T, n_kv // 64, 64), dtype=torch.bfloat16, device=dev)
    v = torch.empty_like(k)
    f = torch.empty((B, T, n_f // 64, 64), dtype=f_dtype, device=dev)
    if (k_cache is None) != (v_cache is None):
        raise ValueError("sparda: k_cache and v_cache go together")
    if k_cache is not None:
        if pos_dev is None or pos0 != 0:
            raise ValueError("sparda: writing the caches needs pos_dev (and pos0 = 0)")
        require_device(k_cache, v_cache)
        if not (k_cache.dtype == v_cache.dtype == torch.bfloat16) or k_cache.stride() != v_cache.stride():
            raise TypeError("sparda: the caches must be bf16 with equal strides")
        if k_cache.shape[0] != B or tuple(k_cache.shape[2:]) != (n_kv // 64, 64) or k_cache.stride(-1) != 1:
            raise AssertionError(f"Mismatch: cache {tuple(k_cache.shape)} for {B} sequences, {n_kv // 64} heads")
        sb, st, sh, _ = k_cache.stride()
        call("sparda_produce_cache_at", x2.data_ptr(), x2.stride(0), w_stacked.data_ptr(), B * T, C, n_q, n_kv,
             n_f, float(eps), rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.shape[0], T, _pos_ptr(pos_dev),
             q.data_ptr(), k.data_ptr(), v.data_ptr(), f.data_ptr(), _DT[f_dtype], k_cache.data_ptr(),
             v_cache.data_ptr(), sb, st, sh, k_cache.shape[1], _stream(dev))
        return q, k, v, f
    if pos_dev is not None:
        if pos0 != 0:
            raise ValueError("sparda: produce takes pos0 or pos_dev, not both")
        call("sparda_produce_at", x2.data_ptr(), x2.stride(0), w_stacked.data_ptr(), B * T, C, n_q, n_kv, n_f,
             float(eps), rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.shape[0], T, _pos_ptr(pos_dev),
             q.data_ptr(), k.data_ptr(), v.data_ptr(), f.data_ptr(), _DT[f_dtype], _stream(dev))
        return q, k, v, f
    call("sparda_produce", x2.data_ptr(), x2.stride(0), w_stacked.data_ptr(), B * T, C, n_q, n_kv, n_f,
         float(eps), rope_cos.data_ptr(), rope_sin.data_ptr(), rope_cos.shape[0], T, pos0,
         q.data_ptr(), k.data_ptr(), v.data_ptr(), f.data_ptr(), _DT[f_dtype], _stream(dev))
    return q, k, v, f


def decode_sums(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, S: int, forecast: torch.Tensor,
                block_sums: torch.Tensor, block_size: int, top_k: int, routing: str = "reference",
                pos_dev: Optional[torch.Tensor] = None, scale: Optional[float] = None,
                want_sel: bool = False, out: Optional[torch.Tensor] = None, update_current: bool = False):
    """One decode step with cached prototypes in a single launch: the blocks
    are scored from the fp32 block sums [B,NBmax,Hkv,D] (sum / bs = the
    prototypes of model/forecast.py:66-78), the top-k + sink + own block
    selected (model/attention/sparse.py:126-154; every block while the cache
    holds at most top_k + 2 blocks) and attended in place, inside the attention
    kernel. q [B,Hq,D] at position S-1, caches [B,Smax,Hkv,D] holding [0, S),
    forecast [B,Hkv,D]. With pos_dev (a one-element int64 GPU tensor) the
    length is *pos_dev + 1, read when the kernel runs, S its bound. With
    update_current the sums of the block holding position S-1 are first
    recomputed from its rows (as block_sums(k, cb*bs, S - cb*bs, ...) does)
    and stored, so the caller needs no separate sums update after appending.
    Returns out [B,Hq*D], or (out, sel, n_sel) with want_sel."""
    dev = require_device(q, k, v, forecast, block_sums, pos_dev)
    _inference_only(q, k, v)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q and the caches must share a dtype")
    if block_sums.dtype != torch.float32 or not block_sums.is_contiguous():
        raise TypeError("sparda: block_sums must be contiguous float32")
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    if k.stride() != v.stride():
        raise ValueError("sparda: k_cache and v_cache must share strides")
    B, Hq, D = q.shape
    Hkv = k.shape[2]
    if S > k.shape[1] or S <= 0:
        raise ValueError(f"sparda: S={S} outside the cache (capacity {k.shape[1]})")
    if routing not in ("reference", "absolute"):
        raise ValueError(f"sparda: routing must be 'reference' or 'absolute', got {routing!r}")
    forecast = _rowmajor(forecast.reshape(B, Hkv, -1) if forecast.dim() != 3 else forecast)
    if forecast.shape[-1] != D or tuple(block_sums.shape[2:]) != (Hkv, D) or block_sums.shape[0] != B:
        raise AssertionError(f"Mismatch: forecast {tuple(forecast.shape)} / block sums {tuple(block_sums.shape)} "
                             f"for head dim {D}")
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty((B, Hq * D), dtype=q.dtype, device=dev)
    sel = n_sel = None
    if want_sel:
        sel = torch.empty((B, Hkv, top_k + 2), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, Hkv), dtype=torch.int32, device=dev)
    qsb, qsh, _ = q.stride()
    ksb, kss, ksh, _ = k.stride()
    fsb, fsh, _ = forecast.stride()
    call("sparda_decode_sums", q.data_ptr(), qsb, qsh, k.data_ptr(), v.data_ptr(), ksb, kss, ksh, _dtype_code(q),
         forecast.data_ptr(), _dtype_code(forecast), fsb, fsh, block_sums.data_ptr(), block_sums.shape[1],
         1 if update_current else 0, B, S,
         _pos_ptr(pos_dev) if pos_dev is not None else None, Hq, Hkv, D, block_size, top_k,
         _lib.ROUTE_ABSOLUTE if routing == "absolute" else _lib.ROUTE_REFERENCE, float(scale),
         float(default_scale(forecast.shape[-1])), sel.data_ptr() if sel is not None else None,
         n_sel.data_ptr() if n_sel is not None else None, out.data_ptr(), out.stride(0), _stream(dev))
    if want_sel:
        return out, sel, n_sel
    return out


def ffn_decode(x: torch.Tensor, w_gate_up: torch.Tensor, w_down: torch.Tensor, eps: float,
               out: Optional[torch.Tensor] = None, prefetch: Optional[tuple] = None,
               pos_dev: Optional[torch.Tensor] = None, block_size: int = 64) -> torch.Tensor:
    """x + SwiGLU(RMSNorm(x)) for decode-sized batches (model/transformer.py:18-31,
    126-129; model/norm.py:15-21): x [B,T,C] bf16 with B*T <= 16, w_gate_up
    [2F, C] = [w_gate; w_up] * norm_weight (folded into the columns), w_down
    [C, F], all bf16. Returns [B,T,C] bf16.

    prefetch: (gate_up_spec, down_spec), either None: shares of the next
    layer's prefetch copy carried by the two launches (sparda_ffn_decode_prefetch),
    each a decode_at prefetch spec with ``stage`` 2 and ``parts`` / ``part``,
    at position pos_dev over arenas of block_size-key blocks."""
    dev = require_device(x, w_gate_up, w_down, out)
    _inference_only(x, w_gate_up, w_down)
    if not (x.dtype == w_gate_up.dtype == w_down.dtype == torch.bfloat16):
        raise TypeError("sparda: ffn_decode takes bf16 activations and weights")
    B, T, C = x.shape
    x2 = x.reshape(B * T, C)
    if x2.stride(-1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    F = w_gate_up.shape[0] // 2
    w_gate_up, w_down = w_gate_up.contiguous(), w_down.contiguous()
    if tuple(w_gate_up.shape) != (2 * F, C) or tuple(w_down.shape) != (C, F):
        raise AssertionError(f"Mismatch: w_gate_up {tuple(w_gate_up.shape)}, w_down {tuple(w_down.shape)} "
                             f"for width {C}")
    act = torch.empty((B * T, F), dtype=torch.bfloat16, device=dev)
    if out is None:
        out = torch.empty((B, T, C), dtype=torch.bfloat16, device=dev)
    o2 = out.view(B * T, C)
    if prefetch is None:
        call("sparda_ffn_decode", x2.data_ptr(), x2.stride(0), w_gate_up.data_ptr(), w_down.data_ptr(), B * T, C, F,
             float(eps), act.data_ptr(), o2.data_ptr(), o2.stride(0), _stream(dev))
        return out
    if pos_dev is None or T != 1:
        raise ValueError("sparda: a carried prefetch needs pos_dev and one token per sequence")
    args, keep = [], []
    for spec in prefetch:
        if spec is None:
            args.append(None)
            continue
        if int(spec.get("stage", 0)) != 2:
            raise ValueError("sparda: the feed-forward launches carry only the copy (stage 2)")
        pf, k = _prefetch_args(spec, B, spec["arena"].Hkv, spec["arena"].D, block_size, dev)
        args.append(ctypes.byref(pf))
        keep.append((pf, k))
    call("sparda_ffn_decode_prefetch", x2.data_ptr(), x2.stride(0), w_gate_up.data_ptr(), w_down.data_ptr(), B * T,
         C, F, float(eps), act.data_ptr(), o2.data_ptr(), o2.stride(0), args[0], args[1], _pos_ptr(pos_dev),
         block_size, _stream(dev))
    del keep
    return out


def rows_residual(a: torch.Tensor, w: torch.Tensor, res: torch.Tensor,
                  out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """res + a . w^T for decode-sized batches in one kernel: the attention's
    output projection and residual (model/transformer.py:118-126 with
    model/attention/sparse.py:183). a [B,T,K], w [N,K], res [B,T,N], all bf16,
    B*T <= 16. The projection is rounded to bf16 before the sum, as the
    unfused pair does. Returns [B,T,N] bf16."""
    dev = require_device(a, w, res, out)
    _inference_only(a, w, res)
    if not (a.dtype == w.dtype == res.dtype == torch.bfloat16):
        raise TypeError("sparda: rows_residual takes bf16 activations and weights")
    B, T, K = a.shape
    N = w.shape[0]
    if tuple(w.shape) != (N, K) or tuple(res.shape) != (B, T, N):
        raise AssertionError(f"Mismatch: a {tuple(a.shape)}, w {tuple(w.shape)}, res {tuple(res.shape)}")
    a2 = a.reshape(B * T, K)
    if a2.stride(-1) != 1 or a2.stride(0) % 8:
        a2 = a2.contiguous()
    r2 = res.reshape(B * T, N)
    if r2.stride(-1) != 1:
        r2 = r2.contiguous()
    w = w.contiguous()
    if out is None:
        out = torch.empty((B, T, N), dtype=torch.bfloat16, device=dev)
    o2 = out.view(B * T, N)
    call("sparda_rows_residual", a2.data_ptr(), a2.stride(0), w.data_ptr(), B * T, K, N, r2.data_ptr(),
         r2.stride(0), o2.data_ptr(), o2.stride(0), _stream(dev))
    return out


def norm_gemv(x: torch.Tensor, w_folded: torch.Tensor, eps: float,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """final_norm(x) . W^T for decode-sized batches in one kernel (the model's
    last RMSNorm and its tied output projection, model/model.py:79-157 with
    model/norm.py:15-21): x [B,T,C] bf16 with B*T <= 16, w_folded [N,C] bf16 =
    W * norm_weight (folded into the columns). Returns [B,T,N] bf16."""
    dev = require_device(x, w_folded, out)
    _inference_only(x, w_folded)
    if not (x.dtype == w_folded.dtype == torch.bfloat16):
        raise TypeError("sparda: norm_gemv takes bf16 activations and weights")
    B, T, C = x.shape
    N = w_folded.shape[0]
    if tuple(w_folded.shape) != (N, C):
        raise AssertionError(f"Mismatch: weight {tuple(w_folded.shape)} for width {C}")
    x2 = x.reshape(B * T, C)
    if x2.stride(-1) != 1 or x2.stride(0) % 8:
        x2 = x2.contiguous()
    w_folded = w_folded.contiguous()
    if out is None:
        out = torch.empty((B, T, N), dtype=torch.bfloat16, device=dev)
    o2 = out.view(B * T, N)
    call("sparda_norm_gemv", x2.data_ptr(), x2.stride(0), w_folded.data_ptr(), B * T, C, N, float(eps),
         o2.data_ptr(), o2.stride(0), _stream(dev))
    return out


def _pos_ptr(pos_dev: torch.Tensor) -> int:
    """Address of a device-held position: one int64 element on the GPU."""
    if pos_dev.dtype != torch.int64 or pos_dev.numel() != 1 or not pos_dev.is_cuda:
        raise TypeError("sparda: pos_dev must be a one-element int64 tensor on the GPU")
    return pos_dev.data_ptr()


def append_at(k_cache: torch.Tensor, v_cache: Optional[torch.Tensor], pos_dev: torch.Tensor, block_size: int,
              block_sums: Optional[torch.Tensor], k_new: Optional[torch.Tensor] = None,
              v_new: Optional[torch.Tensor] = None) -> Optional[torch.Tensor]:
    """Decode-step cache append at token p = pos_dev (a one-element int64 device
    tensor, read when the kernel runs): k_new / v_new ([B,1,Hkv,D] or
    [B,Hkv,D]) written as row p of the caches [B,Smax,Hkv,D] (KVCache.update,
    model/attention/base.py:19-29), and the fp32 sums of the block holding p
    recomputed over [p - p % bs, p] in block_sums (in place; returned). Without
    k_new / v_new only the sums are recomputed; without block_sums only the
    rows are written."""
    dev = require_device(k_cache, v_cache, block_sums, pos_dev, k_new, v_new)
    _inference_only(k_cache, v_cache, k_new, v_new)
    if k_cache.stride(-1) != 1:
        raise ValueError("sparda: the cache's last dimension must be contiguous")
    B, S, Hkv, D = k_cache.shape
    if block_sums is None:
        if k_new is None:
            raise ValueError("sparda: append_at needs new rows or block sums")
        nbs = (S + block_size - 1) // block_size
    else:
        if block_sums.dtype != torch.float32 or not block_sums.is_contiguous():
            raise TypeError("sparda: block sums must be contiguous float32")
        if tuple(block_sums.shape[:1]) != (B,) or tuple(block_sums.shape[2:]) != (Hkv, D):
            raise AssertionError(f"Mismatch: cache {tuple(k_cache.shape)} vs block sums {tuple(block_sums.shape)}")
        nbs = block_sums.shape[1]
    nsb = nsh = 0
    if (k_new is None) != (v_new is None):
        raise ValueError("sparda: k_new and v_new go together")
    if k_new is not None:
        if v_cache is None or v_cache.stride() != k_cache.stride() or v_cache.shape != k_cache.shape:
            raise ValueError("sparda: appending needs a v_cache shaped and strided like k_cache")
        if not (k_new.dtype == v_new.dtype == k_cache.dtype == v_cache.dtype):
            raise TypeError("sparda: the new rows and the caches must share a dtype")
        k_new = _rowmajor(k_new.reshape(B, Hkv, D))
        v_new = _rowmajor(v_new.reshape(B, Hkv, D))
        if k_new.stride() != v_new.stride():
            raise ValueError("sparda: k_new and v_new must share strides")
        nsb, nsh, _ = k_new.stride()
    max_len = min(S, nbs * block_size)
    sb, st, sh, _ = k_cache.stride()
    call("sparda_append_at", k_cache.data_ptr(), v_cache.data_ptr() if v_cache is not None else None,
         _dtype_code(k_cache), sb, st, sh, k_new.data_ptr() if k_new is not None else None,
         v_new.data_ptr() if v_new is not None else None, nsb, nsh, B, Hkv, D, max_len, _pos_ptr(pos_dev),
         block_size, nbs, block_sums.data_ptr() if block_sums is not None else None, _stream(dev))
    return block_sums


def select_decode_at(forecast: torch.Tensor, block_sums: torch.Tensor, pos_dev: torch.Tensor, max_len: int,
                     block_size: int, top_k: int, routing: str = "reference", scale: Optional[float] = None,
                     sel: Optional[torch.Tensor] = None, n_sel: Optional[torch.Tensor] = None,
                     lookahead: bool = False):
    """select_decode for the decode step at token p = pos_dev (a one-element
    int64 device tensor, read when the kernel runs): length p + 1, query
    position p; with lookahead, length p (the prefetch issued before token p
    is appended, model/attention/async_offload.py:196-260). p is clamped below
    max_len."""
    dev = require_device(forecast, block_sums, pos_dev, sel, n_sel)
    if block_sums.dtype != torch.float32 or not block_sums.is_contiguous():
        raise TypeError("sparda: block_sums must be contiguous float32")
    B, nbs, Hkv, D = block_sums.shape
    forecast = _rowmajor(forecast.reshape(B, Hkv, -1) if forecast.dim() != 3 else forecast)
    if routing not in ("reference", "absolute"):
        raise ValueError(f"sparda: routing must be 'reference' or 'absolute', got {routing!r}")
    if scale is None:
        scale = default_scale(forecast.shape[-1])
    if sel is None:
        sel = torch.empty((B, Hkv, top_k + 2), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, Hkv), dtype=torch.int32, device=dev)
    fsb, fsh, _ = forecast.stride()
    call("sparda_select_decode_at", forecast.data_ptr(), _dtype_code(forecast), fsb, fsh, block_sums.data_ptr(),
         B, Hkv, D, nbs, max_len, _pos_ptr(pos_dev), block_size, top_k,
         _lib.ROUTE_ABSOLUTE if routing == "absolute" else _lib.ROUTE_REFERENCE, float(scale),
         sel.data_ptr(), n_sel.data_ptr(), sel.shape[-1], int(bool(lookahead)), _stream(dev))
    return sel, n_sel


def decode_at(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, pos_dev: torch.Tensor, block_size: int,
              sel: Optional[torch.Tensor] = None, n_sel: Optional[torch.Tensor] = None, window: int = 0,
              max_len: Optional[int] = None, scale: Optional[float] = None,
              out: Optional[torch.Tensor] = None, compact: bool = False, k_new: Optional[torch.Tensor] = None,
              v_new: Optional[torch.Tensor] = None, prefetch: Optional[dict] = None) -> torch.Tensor:
    """Decode attention of q [B,Hq,D] at token p = pos_dev (a one-element int64
    device tensor, read when the kernel runs) over the caches [B,Smax,Hkv,D]
    holding p + 1 tokens: the blocks sel[b,g,:n_sel], or with sel None the
    static window of `window` blocks (+ sink; every block while the cache has
    at most window + 2), or every block (window 0). compact: k / v are fetched
    block buffers [B,Hkv,cap,bs,D] (slot i = block sel[b,g,i]); k_new / v_new
    [B,Hkv,D]: the key and value of position p. p is clamped below max_len
    (default: the cache capacity; required with compact).

    prefetch: the next layer's prefetch carried by the same launch
    (sparda_decode_at_prefetch; bf16, D = 64): a dict with ``arena`` (the next
    layer's OffloadArena), ``forecast`` [B,Hkv,Df], ``block_sums`` (its sums),
    ``top_k``, ``routing``, optional ``scale``, and the outputs ``sel`` /
    ``n_sel`` / ``k_dst`` / ``v_dst`` — what select_decode_at(lookahead=True)
    and OffloadArena.fetch_at would write, bit for bit. Optional ``stage``: 0
    (default) selection and copy, 1 the selection only, 2 the copy only of
    the selection already in sel / n_sel."""
    dev = require_device(q, k, v, pos_dev, sel, n_sel, k_new, v_new)
    _inference_only(q, k, v, k_new, v_new)
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("sparda: q, k and v must share a dtype")
    q, k, v = _rowmajor(q), _rowmajor(k), _rowmajor(v)
    if k.stride() != v.stride():
        raise ValueError("sparda: k and v must share strides")
    B, Hq, D = q.shape
    if compact:
        if sel is None or max_len is None:
            raise ValueError("sparda: compact block buffers need a selection and max_len")
        _, Hkv, cap_, bs_, _ = k.shape
        if bs_ != block_size or cap_ != sel.shape[-1]:
            raise ValueError("sparda: compact buffers must be [B,Hkv,sel_cap,block_size,D]")
        kv_sb, kv_sh, _, kv_ss, _ = k.stride()
    else:
        Hkv = k.shape[2]
        if max_len is None:
            max_len = k.shape[1]
        if not 0 < max_len <= k.shape[1]:
            raise ValueError(f"sparda: max_len={max_len} outside the cache (capacity {k.shape[1]})")
        kv_sb, kv_ss, kv_sh, _ = k.stride()
    nsb = nsh = 0
    if (k_new is None) != (v_new is None):
        raise ValueError("sparda: k_new and v_new go together")
    if k_new is not None:
        k_new = _rowmajor(k_new.reshape(B, Hkv, D))
        v_new = _rowmajor(v_new.reshape(B, Hkv, D))
        if k_new.stride() != v_new.stride():
            raise ValueError("sparda: k_new and v_new must share strides")
        nsb, nsh, _ = k_new.stride()
    cap = 0
    if sel is not None:
        if sel.dtype != torch.int32 or n_sel is None or n_sel.dtype != torch.int32:
            raise TypeError("sparda: sel / n_sel must be int32 tensors")
        sel, n_sel = sel.contiguous(), n_sel.contiguous()
        cap = sel.shape[-1]
    if scale is None:
        scale = default_scale(D)
    if out is None:
        out = torch.empty((B, Hq * D), dtype=q.dtype, device=dev)
    qsb, qsh, _ = q.stride()
    args = (q.data_ptr(), qsb, qsh, k.data_ptr(), v.data_ptr(), kv_sb, kv_ss, kv_sh,
            _dtype_code(q), int(bool(compact)), sel.data_ptr() if sel is not None else None,
            n_sel.data_ptr() if n_sel is not None else None, cap, int(window),
            k_new.data_ptr() if k_new is not None else None, v_new.data_ptr() if v_new is not None else None,
            nsb, nsh, B, max_len, _pos_ptr(pos_dev), Hq, Hkv, D, block_size, float(scale), out.data_ptr(),
            out.stride(0))
    # every block (no selection, no window) on the matrix cores: split over workgroups, partials in a workspace
    dense = sel is None and int(window) == 0 and q.dtype == torch.bfloat16 and D == 64 and block_size in (32, 64)
    ws_ptr, ws_bytes, ws = _dense_split_ws(B, Hq, Hkv, D, max_len, block_size, dev) if dense else (None, 0, None)
    if prefetch is None:
        call("sparda_decode_at", *args, ws_ptr, ws_bytes, _stream(dev))
    else:
        pf, keep = _prefetch_args(prefetch, B, Hkv, D, block_size, dev)
        call("sparda_decode_at_prefetch", *args, ctypes.byref(pf), ws_ptr, ws_bytes, _stream(dev))
        del keep
    del ws
    return out


def _prefetch_args(spec: dict, B: int, Hkv: int, D: int, block_size: int, dev):
    """The sparda_prefetch_args of a prefetch spec carried by another launch
    (checked as select_decode_at and OffloadArena.fetch_at check theirs), with
    the tensors it points into."""
    arena = spec["arena"]
    f, sums = spec["forecast"], spec["block_sums"]
    sel, n_sel, k_dst, v_dst = spec["sel"], spec["n_sel"], spec["k_dst"], spec["v_dst"]
    stage = int(spec.get("stage", 0))
    if stage not in (0, 1, 2):
        raise ValueError(f"sparda: prefetch stage must be 0, 1 or 2, got {stage}")
    parts, part = int(spec.get("parts", 1)), int(spec.get("part", 0))
    if not (1 <= parts and 0 <= part < parts) or (parts > 1 and stage != 2):
        raise ValueError(f"sparda: prefetch share {part} of {parts} (shares need stage 2)")
    require_device(f, sums, sel, n_sel, k_dst, v_dst)
    if (arena.B, arena.Hkv, arena.D) != (B, Hkv, D):
        raise ValueError("sparda: the prefetched arena must have the attended layer's batch, KV heads and head dim")
    if sums.dtype != torch.float32 or not sums.is_contiguous() or tuple(sums.shape[:1]) + tuple(sums.shape[2:]) \
            != (B, Hkv, D):
        raise TypeError("sparda: prefetch block_sums must be contiguous float32 [B,nb,Hkv,D]")
    f = _rowmajor(f.reshape(B, Hkv, -1) if f.dim() != 3 else f)
    if tuple(f.shape) != (B, Hkv, D):
        raise ValueError(f"sparda: the prefetch forecast must be [B,Hkv,{D}], got {tuple(f.shape)}")
    routing = spec.get("routing", "reference")
    if routing not in ("reference", "absolute"):
        raise ValueError(f"sparda: routing must be 'reference' or 'absolute', got {routing!r}")
    scale = spec.get("scale")
    if scale is None:
        scale = default_scale(f.shape[-1])
    if sel.dtype != torch.int32 or n_sel.dtype != torch.int32 or not (sel.is_contiguous() and n_sel.is_contiguous()):
        raise TypeError("sparda: prefetch sel / n_sel must be contiguous int32 tensors")
    cap = sel.shape[-1]
    if tuple(sel.shape) != (B, Hkv, cap) or tuple(n_sel.shape) != (B, Hkv):
        raise ValueError("sparda: prefetch sel / n_sel must be [B,Hkv,cap] / [B,Hkv]")
    if not (k_dst.is_contiguous() and v_dst.is_contiguous()) or tuple(k_dst.shape) != (B, Hkv, cap, block_size, D) \
            or k_dst.shape != v_dst.shape:
        raise ValueError("sparda: prefetch destinations must be contiguous [B,Hkv,sel_cap,block_size,D]")
    if k_dst.dtype != arena.dtype or v_dst.dtype != arena.dtype:
        raise TypeError("sparda: prefetch destinations must have the arena dtype")
    fsb, fsh, _ = f.stride()
    pf = _lib.PrefetchArgs(arena.handle.value, f.data_ptr(), _dtype_code(f), fsb, fsh, sums.data_ptr(), sums.shape[1],
                           int(spec["top_k"]), _lib.ROUTE_ABSOLUTE if routing == "absolute" else _lib.ROUTE_REFERENCE,
                           float(scale), sel.data_ptr(), n_sel.data_ptr(), cap, k_dst.data_ptr(), v_dst.data_ptr(),
                           stage, parts, part)
    return pf, (f, sums, sel, n_sel, k_dst, v_dst)


def block_sums(k: torch.Tensor, pos: int, n: int, block_size: int, sums: torch.Tensor) -> torch.Tensor:
    """Accumulate fp32 block sums of tokens [pos, pos+n) of the device cache
    k [B,S,Hkv,D] into sums [B,NBmax,Hkv,D] (in place; returned). A block whose
    first token is in the range restarts from zero, so pos = j*block_size
    recomputes blocks j.. exactly: sums/bs equal compress() bit for bit
    (prototypes of model/forecast.py:66-78 without recompressing the cache)."""
    dev = require_device(k, sums)
    _inference_only(k)
    if sums.dtype != torch.float32 or not sums.is_contiguous():
        raise TypeError("sparda: block sums must be contiguous float32")
    if k.stride(-1) != 1:
        raise ValueError("sparda: the cache's last dimension must be contiguous")
    B, S, Hkv, D = k.shape
    if tuple(sums.shape[:1]) != (B,) or tuple(sums.shape[2:]) != (Hkv, D):
        raise AssertionError(f"Mismatch: cache {tuple(k.shape)} vs block sums {tuple(sums.shape)}")
    if pos < 0 or n < 1 or pos + n > S:
        raise ValueError(f"sparda: tokens [{pos}, {pos + n}) outside the cache of {S}")
    sb, st, sh, _ = k.stride()
    call("sparda_block_sums", k.data_ptr(), _dtype_code(k), sb, st, sh, B, Hkv, D, pos, n, block_size,
         sums.shape[1], sums.data_ptr(), _stream(dev))
    return sums


def select_decode(forecast: torch.Tensor, block_sums: torch.Tensor, length: int, pos: int, block_size: int,
                  top_k: int, routing: str = "reference", scale: Optional[float] = None,
                  sel: Optional[torch.Tensor] = None, n_sel: Optional[torch.Tensor] = None):
    """Decode selection from block sums [B,NBmax,Hkv,D] fp32 covering tokens [0, length),
    for the query at position `pos` (model/attention/async_offload.py:196-260).
    Returns sel [B,Hkv,top_k+2] int32 (ascending, -1 padded) and n_sel [B,Hkv]."""
    dev = require_device(forecast, block_sums, sel, n_sel)
    if block_sums.dtype != torch.float32 or not block_sums.is_contiguous():
        raise TypeError("sparda: block_sums must be contiguous float32")
    B, nbs, Hkv, D = block_sums.shape
    forecast = _rowmajor(forecast.reshape(B, Hkv, -1) if forecast.dim() != 3 else forecast)
    if routing not in ("reference", "absolute"):
        raise ValueError(f"sparda: routing must be 'reference' or 'absolute', got {routing!r}")
    if scale is None:
        scale = default_scale(forecast.shape[-1])
    cap = top_k + 2
    if sel is None:
        sel = torch.empty((B, Hkv, cap), dtype=torch.int32, device=dev)
        n_sel = torch.empty((B, Hkv), dtype=torch.int32, device=dev)
    fsb, fsh, _ = forecast.stride()
    call("sparda_select_decode", forecast.data_ptr(), _dtype_code(forecast), fsb, fsh, block_sums.data_ptr(),
         B, Hkv, D, nbs, length, pos, block_size, top_k,
         _lib.ROUTE_ABSOLUTE if routing == "absolute" else _lib.ROUTE_REFERENCE, float(scale),
         sel.data_ptr(), n_sel.data_ptr(), sel.shape[-1], _stream(dev))
    return sel, n_sel


class OffloadArena:
    """Pinned host KV arena of one layer owned by libsparda (sparda_offload_create).

    Layout of each of K and V: [B][Hkv][max_seq][D]. ``k_host`` / ``v_host`` are
    CPU tensor views of it in the reference's [B,max_seq,Hkv,D] order.
    """

    def __init__(self, B: int, max_seq: int, Hkv: int, D: int, dtype: torch.dtype, device=None):
        self.B, self.max_seq, self.Hkv, self.D, self.dtype = B, max_seq, Hkv, D, dtype
        self.device = torch.device(device) if device is not None else torch.device("cuda")
        with torch.cuda.device(self.device):
            h = ctypes.c_void_p()
            call("sparda_offload_create", B, max_seq, Hkv, D, _DT[dtype], ctypes.byref(h))
        self._h = h
        kp, vp = ctypes.c_void_p(), ctypes.c_void_p()
        call("sparda_offload_host", self._h, ctypes.byref(kp), ctypes.byref(vp))
        n = B * Hkv * max_seq * D
        esz = torch.empty((), dtype=dtype).element_size()

        def view(ptr):
            buf = (ctypes.c_uint8 * (n * esz)).from_address(ptr.value)
            t = torch.frombuffer(buf, dtype=torch.uint8).view(dtype).view(B, Hkv, max_seq, D)
            return t.transpose(1, 2)

        self.k_host = view(kp)
        self.v_host = view(vp)

    @property
    def handle(self):
        if self._h is None:
            raise RuntimeError("sparda: offload arena already destroyed")
        return self._h

    def close(self) -> None:
        if getattr(self, "_h", None) is not None:
            self.k_host = self.v_host = None
            call("sparda_offload_destroy", self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def append(self, k: torch.Tensor, v: torch.Tensor, pos: int, block_size: int = 0,
               block_sums: Optional[torch.Tensor] = None) -> None:
        """Tokens [pos, pos+n) of k, v [B,n,Hkv,D] (device) into the arena (+ block sums)."""
        dev = require_device(k, v, block_sums)
        k, v = _rowmajor(k), _rowmajor(v)
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise TypeError(f"sparda: arena holds {self.dtype}, got {k.dtype}/{v.dtype}")
        if k.stride() != v.stride():
            k, v = k.contiguous(), v.contiguous()
        B, n, Hkv, D = k.shape
        if (B, Hkv, D) != (self.B, self.Hkv, self.D):
            raise ValueError("sparda: k/v shape does not match the arena")
        sb, st, sh, _ = k.stride()
        call("sparda_offload_append", self.handle, k.data_ptr(), v.data_ptr(), sb, st, sh, pos, n, block_size,
             block_sums.data_ptr() if block_sums is not None else None, _stream(dev))

    def rebuild_sums(self, length: int, block_size: int, block_sums: torch.Tensor) -> None:
        dev = require_device(block_sums)
        call("sparda_offload_rebuild_sums", self.handle, length, block_size, block_sums.data_ptr(), _stream(dev))

    def fetch(self, sel: torch.Tensor, n_sel: torch.Tensor, block_size: int, length: int,
              k_dst: torch.Tensor, v_dst: torch.Tensor, method: int = _lib.FETCH_KERNEL) -> None:
        """Blocks sel[b,g,:n_sel] (rows < length) into k_dst/v_dst [B,Hkv,cap,bs,D]."""
        dev = require_device(sel, n_sel, k_dst, v_dst)
        if not (k_dst.is_contiguous() and v_dst.is_contiguous()):
            raise ValueError("sparda: fetch destinations must be contiguous")
        cap = sel.shape[-1]
        if tuple(k_dst.shape) != (self.B, self.Hkv, cap, block_size, self.D) or k_dst.shape != v_dst.shape:
            raise ValueError("sparda: fetch destinations must be [B,Hkv,sel_cap,block_size,D]")
        if k_dst.dtype != self.dtype or v_dst.dtype != self.dtype:
            raise TypeError("sparda: fetch destinations must have the arena dtype")
        call("sparda_offload_fetch", self.handle, sel.contiguous().data_ptr(), n_sel.contiguous().data_ptr(),
             cap, block_size, length, method, k_dst.data_ptr(), v_dst.data_ptr(), _stream(dev))

    def fetch_at(self, sel: torch.Tensor, n_sel: torch.Tensor, block_size: int, len_dev: torch.Tensor,
                 k_dst: torch.Tensor, v_dst: torch.Tensor) -> None:
        """fetch (gather kernel) with the arena length read from device memory
        (len_dev: a one-element int64 GPU tensor, clamped into [0, max_seq])."""
        dev = require_device(sel, n_sel, k_dst, v_dst, len_dev)
        if not (k_dst.is_contiguous() and v_dst.is_contiguous()):
            raise ValueError("sparda: fetch destinations must be contiguous")
        cap = sel.shape[-1]
        if tuple(k_dst.shape) != (self.B, self.Hkv, cap, block_size, self.D) or k_dst.shape != v_dst.shape:
            raise ValueError("sparda: fetch destinations must be [B,Hkv,sel_cap,block_size,D]")
        if k_dst.dtype != self.dtype or v_dst.dtype != self.dtype:
            raise TypeError("sparda: fetch destinations must have the arena dtype")
        if not (sel.is_contiguous() and n_sel.is_contiguous()):
            raise ValueError("sparda: sel / n_sel must be contiguous")
        call("sparda_offload_fetch_at", self.handle, sel.data_ptr(), n_sel.data_ptr(), cap, block_size,
             _pos_ptr(len_dev), k_dst.data_ptr(), v_dst.data_ptr(), _stream(dev))

    def append_at(self, k: torch.Tensor, v: torch.Tensor, pos_dev: torch.Tensor, block_size: int = 0,
                  block_sums: Optional[torch.Tensor] = None, prefetch: Optional[dict] = None,
                  max_len: Optional[int] = None) -> None:
        """One token k, v ([B,1,Hkv,D] or [B,Hkv,D], device) into the arena at row
        pos_dev (a one-element int64 GPU tensor, read when the kernel runs),
        with its block's sums recomputed from the arena when block_sums is given.
        prefetch (with max_len, the positions' bound): the next layer's prefetch
        stage carried by the same launch, a decode_at prefetch dict (normally
        stage 1, the selection; sparda_offload_append_at_prefetch)."""
        dev = require_device(k, v, block_sums, pos_dev)
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise TypeError(f"sparda: arena holds {self.dtype}, got {k.dtype}/{v.dtype}")
        k = _rowmajor(k.reshape(self.B, self.Hkv, self.D))
        v = _rowmajor(v.reshape(self.B, self.Hkv, self.D))
        if k.stride() != v.stride():
            k, v = k.contiguous(), v.contiguous()
        if block_sums is not None and (block_sums.dtype != torch.float32 or not block_sums.is_contiguous()):
            raise TypeError("sparda: block sums must be contiguous float32")
        nsb, nsh, _ = k.stride()
        if prefetch is None:
            call("sparda_offload_append_at", self.handle, k.data_ptr(), v.data_ptr(), nsb, nsh, _pos_ptr(pos_dev),
                 block_size, block_sums.data_ptr() if block_sums is not None else None, _stream(dev))
            return
        if max_len is None or block_size <= 0:
            raise ValueError("sparda: a carried prefetch needs max_len and the block size")
        pf, keep = _prefetch_args(prefetch, self.B, self.Hkv, self.D, block_size, dev)
        call("sparda_offload_append_at_prefetch", self.handle, k.data_ptr(), v.data_ptr(), nsb, nsh, _pos_ptr(pos_dev),
             block_size, block_sums.data_ptr() if block_sums is not None else None, int(max_len), ctypes.byref(pf),
             _stream(dev))
        del keep
