"""Forecast-driven asynchronous KV prefetch — drop-in for AsyncOffloadedKVCache
and AsyncForecastOffloadAttention (model/attention/async_offload.py:28-573).

``prefetch(F_L, cache_{L+1})`` is called by layer L's block before its
attention and FFN (model/transformer.py:110-115). It runs entirely on a side
stream that first waits for the compute stream: decode-time selection from the
GPU block sums, then the fetch of the selected blocks from the pinned host
arena into persistent device buffers, then an event. Layer L+1's decode waits
on that event (``hipStreamWaitEvent``, not a host wait), appends its token, and
attends over the prefetched blocks with the new token supplied separately.
Nothing on this path synchronises the host; overlap is measured from device
events on both streams (``overlap_stats``).
"""

from typing import Dict, List, Optional, Tuple

import torch

import sparda
from model.attention.base import BaseAttention
from model.attention.offload import OffloadedKVCache, dense_from_arena, prefill_dense, resident_dense_decode
from model.config import ModelConfig
from model.forecast import ForecastBlockSelector, KVBlockCompressor
from model.rope import RotaryEmbedding


class AsyncOffloadedKVCache(OffloadedKVCache):
    """Pinned host KV cache with a dedicated transfer stream (async_offload.py:28-112)."""

    def __init__(self, max_batch_size: int, max_seq_len: int, n_kv_head: int, head_dim: int,
                 gpu_device: torch.device, dtype: torch.dtype = torch.bfloat16, pin_memory: bool = True,
                 transfer_stream: Optional[torch.cuda.Stream] = None, block_size: Optional[int] = None):
        super().__init__(max_batch_size, max_seq_len, n_kv_head, head_dim, gpu_device, dtype, pin_memory,
                         block_size)
        # default priority: streams of other priorities are not used anywhere
        self.transfer_stream = transfer_stream or torch.cuda.Stream(device=self.gpu_device)

    def async_transfer_selected_blocks(self, block_indices: torch.Tensor, block_size: int,
                                       stream: Optional[torch.cuda.Stream] = None
                                       ) -> Tuple[torch.Tensor, torch.Tensor, torch.cuda.Event, int]:
        """Fetch blocks [B,Hkv,n] on the transfer stream; returns (gpu_k, gpu_v, event, bytes)
        (async_offload.py:55-112). Consumers must wait on the event."""
        s = stream or self.transfer_stream
        B, H, n = block_indices.shape
        idx = block_indices.to(self.gpu_device, torch.int32).contiguous()
        cnt = torch.full((B, H), n, dtype=torch.int32, device=self.gpu_device)
        shape = (B, H, n, block_size, self.head_dim)
        k = torch.zeros(shape, dtype=self.dtype, device=self.gpu_device)
        v = torch.zeros(shape, dtype=self.dtype, device=self.gpu_device)
        main = torch.cuda.current_stream(self.gpu_device)
        s.wait_stream(main)
        with torch.cuda.stream(s):
            self.arena.fetch(idx, cnt, block_size, self.current_len, k, v)
            ev = torch.cuda.Event()
            ev.record(s)
        for t in (idx, cnt, k, v):
            t.record_stream(s)
        gk = k.view(B, H, n * block_size, self.head_dim)
        gv = v.view(B, H, n * block_size, self.head_dim)
        nbytes = (gk.numel() + gv.numel()) * gk.element_size()
        self.total_bytes_transferred += nbytes
        self.total_transfer_calls += 1
        return gk, gv, ev, nbytes


class HipAsyncOffloadAttention(BaseAttention):
    """Asynchronous forecast-guided offload attention on libsparda
    (model/attention/async_offload.py:115-573)."""

    def __init__(self, config: ModelConfig, layer_idx: int, transfer_stream: Optional[torch.cuda.Stream] = None,
                 fetch_method: int = sparda.FETCH_KERNEL):
        super().__init__(config, layer_idx)
        self.block_size = config.block_size
        self.top_k_blocks = config.top_k_blocks
        self.decode_routing = getattr(config, "decode_routing", "reference")
        self.fetch_method = fetch_method
        self.compressor = KVBlockCompressor(self.block_size, self.head_dim, config.forecast_dim)
        self.selector = ForecastBlockSelector(self.block_size, config.forecast_dim)
        self.transfer_stream = transfer_stream
        # prefetched state (async_offload.py:140-151)
        self.prefetch_event: Optional[torch.cuda.Event] = None
        self.prefetched_gpu_k: Optional[torch.Tensor] = None
        self.prefetched_gpu_v: Optional[torch.Tensor] = None
        self.prefetched_sel_indices: Optional[torch.Tensor] = None
        self.prefetched_n_sel: Optional[torch.Tensor] = None
        self.prefetched_bytes = 0
        self.prefetched_curr_len_at_launch = 0
        self.prefetched_is_small_context = False
        self.stale_prefetches = 0
        self.track_overlap = False
        self._timing: List[Tuple[torch.cuda.Event, torch.cuda.Event, torch.cuda.Event]] = []
        self._pending: Optional[Tuple[torch.cuda.Event, torch.cuda.Event]] = None
        self._bufs: Dict[Tuple, torch.Tensor] = {}
        self.last_profile: Dict[str, float] = {"bytes_transferred": 0, "overlap_pct": 0.0}

    def _ensure_transfer_stream(self, device: torch.device) -> torch.cuda.Stream:
        if self.transfer_stream is None:
            self.transfer_stream = torch.cuda.Stream(device=device)
        return self.transfer_stream

    def _buf(self, name: str, shape, dtype, device) -> torch.Tensor:
        key = (name, tuple(shape), dtype, device)
        t = self._bufs.get(key)
        if t is None:
            t = torch.empty(shape, dtype=dtype, device=device)
            self._bufs[key] = t
        return t

    # -- prefetch (async_offload.py:170-294) ---------------------------------
    @torch.no_grad()
    def prefetch(self, forecast_vector: Optional[torch.Tensor], offload_cache: OffloadedKVCache) -> bool:
        """Issue selection + block fetch for this layer's next decode step on the
        transfer stream; returns False when the cache is empty."""
        if not isinstance(offload_cache, OffloadedKVCache):
            return False
        curr = offload_cache.current_len
        if curr == 0:
            return False
        dev = offload_cache.gpu_device
        side = self._ensure_transfer_stream(dev)
        bs, k = self.block_size, self.top_k_blocks
        B, H, D = offload_cache.max_batch_size, self.n_kv_head, self.head_dim
        own = curr // bs
        small = own + 1 <= k + 2 or forecast_vector is None or self.layer_idx == 0
        # everything the side stream touches is allocated on the compute stream first
        if small:
            nb = own + 1
            sel = torch.arange(nb, dtype=torch.int32, device=dev).repeat(B, H, 1).contiguous()
            n_sel = torch.full((B, H), nb, dtype=torch.int32, device=dev)
            kb = torch.empty((B, H, nb, bs, D), dtype=offload_cache.dtype, device=dev)
            vb = torch.empty_like(kb)
            f = None
            sums = None
            nbytes = 2 * B * H * (curr + 1) * D * kb.element_size()
        else:
            sums = offload_cache.block_sums(bs)
            f = forecast_vector.reshape(B, H, -1)
            sel = self._buf("sel", (B, H, k + 2), torch.int32, dev)
            n_sel = self._buf("n_sel", (B, H), torch.int32, dev)
            kb = self._buf("k", (B, H, k + 2, bs, D), offload_cache.dtype, dev)
            vb = self._buf("v", (B, H, k + 2, bs, D), offload_cache.dtype, dev)
            nbytes = 2 * B * H * (k + 2) * bs * D * kb.element_size()
        main = torch.cuda.current_stream(dev)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            ev0 = torch.cuda.Event(enable_timing=True) if self.track_overlap else None
            if ev0 is not None:
                ev0.record(side)
            if not small:
                sparda.select_decode(f, sums, curr, curr, bs, k, routing=self.decode_routing, sel=sel, n_sel=n_sel)
            method = sparda.FETCH_KERNEL if small else self.fetch_method
            offload_cache.arena.fetch(sel, n_sel, bs, curr, kb, vb, method)
            ev1 = torch.cuda.Event(enable_timing=self.track_overlap)
            ev1.record(side)
        if small:
            for t in (sel, n_sel, kb, vb):
                t.record_stream(side)
        offload_cache.total_bytes_transferred += nbytes
        offload_cache.total_transfer_calls += 1
        self.prefetch_event = ev1
        self.prefetched_gpu_k, self.prefetched_gpu_v = kb, vb
        self.prefetched_sel_indices, self.prefetched_n_sel = sel, n_sel
        self.prefetched_bytes = nbytes
        self.prefetched_curr_len_at_launch = curr
        self.prefetched_is_small_context = small
        self._pending = (ev0, ev1) if self.track_overlap else None
        return True

    def _take_prefetch(self, cache: OffloadedKVCache) -> bool:
        if self.prefetch_event is None:
            return False
        if cache.current_len != self.prefetched_curr_len_at_launch:
            # the cache moved since the prefetch was issued: its blocks are stale
            self.stale_prefetches += 1
            self.prefetch_event = None
            return False
        return True

    # -- decode (async_offload.py:296-519) ----------------------------------
    def _async_decode(self, xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor, cache: OffloadedKVCache,
                      forecast_vector: Optional[torch.Tensor]) -> torch.Tensor:
        B = xq.shape[0]
        bs, k = self.block_size, self.top_k_blocks
        main = torch.cuda.current_stream(xq.device)
        if self._take_prefetch(cache):
            ev_ready = None
            if self._pending is not None:
                ev_ready = torch.cuda.Event(enable_timing=True)
                ev_ready.record(main)
            main.wait_event(self.prefetch_event)
            L = self.prefetched_curr_len_at_launch
            S = cache.update(xk, xv)
            kn, vn = xk[:, 0], xv[:, 0]
            if self.prefetched_is_small_context:
                nb = self.prefetched_gpu_k.shape[2]
                kc = self.prefetched_gpu_k.view(B, self.n_kv_head, nb * bs, self.head_dim).transpose(1, 2)
                vc = self.prefetched_gpu_v.view(B, self.n_kv_head, nb * bs, self.head_dim).transpose(1, 2)
                out = sparda.decode_selected(xq, kc, vc, S, bs, k_new=kn, v_new=vn)
            else:
                out = sparda.decode_selected(xq, self.prefetched_gpu_k, self.prefetched_gpu_v, S, bs,
                                             self.prefetched_sel_indices, self.prefetched_n_sel, compact=True,
                                             k_new=kn, v_new=vn)
            assert S == L + 1
            if ev_ready is not None:
                self._timing.append((self._pending[0], self._pending[1], ev_ready))
            self.prefetch_event = None
            self.prefetched_gpu_k = self.prefetched_gpu_v = None
            self.last_profile = {"bytes_transferred": self.prefetched_bytes}
        else:
            # no usable prefetch: select and fetch on the compute stream (async_offload.py:392-465)
            sums = cache.block_sums(bs)
            S = cache.update(xk, xv)
            nb = (S + bs - 1) // bs
            if nb <= k + 2 or forecast_vector is None or self.layer_idx == 0:
                out = dense_from_arena(cache, xq, S, bs)
                nbytes = 2 * B * self.n_kv_head * S * self.head_dim * xq.element_size()
            else:
                sel, n_sel = sparda.select_decode(forecast_vector.reshape(B, self.n_kv_head, -1), sums, S, S - 1,
                                                  bs, k, routing=self.decode_routing)
                kb, vb = cache.fetch(sel, n_sel, bs, S, self.fetch_method)
                out = sparda.decode_selected(xq, kb, vb, S, bs, sel, n_sel, compact=True)
                nbytes = 2 * B * self.n_kv_head * (k + 2) * bs * self.head_dim * xq.element_size()
            cache.total_bytes_transferred += nbytes
            cache.total_transfer_calls += 1
            self.last_profile = {"bytes_transferred": nbytes}
        return self.wo(out.view(B, 1, self.n_head * self.head_dim))

    def overlap_stats(self, reset: bool = True) -> Dict[str, float]:
        """Transfer time and the part of it the compute stream waited for, from
        device events (needs track_overlap = True before the prefetches):
        overlap = 1 - exposed / transfer."""
        if not self._timing:
            return {"steps": 0, "transfer_ms": 0.0, "exposed_ms": 0.0, "overlap": 0.0}
        self._timing[-1][2].synchronize()
        tr = ex = 0.0
        for e0, e1, er in self._timing:
            t = e0.elapsed_time(e1)
            tr += t
            ex += min(t, max(0.0, er.elapsed_time(e1)))
        n = len(self._timing)
        if reset:
            self._timing = []
        return {"steps": n, "transfer_ms": tr / n, "exposed_ms": ex / n,
                "overlap": 1.0 - ex / tr if tr > 0 else 0.0}

    def forward(self, x: torch.Tensor, rotary_emb: RotaryEmbedding, kv_cache=None, mask=None,
                is_causal: bool = True, forecast_vector: Optional[torch.Tensor] = None, **kwargs) -> torch.Tensor:
        if mask is not None:
            raise NotImplementedError("explicit additive masks are not supported by the HIP backend")
        B, T, _ = x.shape
        xq = self.wq(x).view(B, T, self.n_head, self.head_dim)
        xk = self.wk(x).view(B, T, self.n_kv_head, self.head_dim)
        xv = self.wv(x).view(B, T, self.n_kv_head, self.head_dim)
        offset = kv_cache.current_len if kv_cache is not None else 0
        xq, xk = rotary_emb(xq, xk, offset=offset)
        return self.forward_projected(xq, xk, xv, kv_cache=kv_cache, is_causal=is_causal,
                                      forecast_vector=forecast_vector)

    def forward_projected(self, xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor, kv_cache=None,
                          is_causal: bool = True, forecast_vector: Optional[torch.Tensor] = None) -> torch.Tensor:
        """The attention after the projections and RoPE (q [B,T,Hq,D], k / v
        [B,T,Hkv,D] rotated at the cache's position): from forward, or from a
        block whose fused producer computed them."""
        T = xq.shape[1]
        if isinstance(kv_cache, OffloadedKVCache) and T == 1:
            return self._async_decode(xq[:, 0], xk, xv, kv_cache, forecast_vector)
        if kv_cache is not None and T == 1:
            return resident_dense_decode(self, xq, xk, xv, kv_cache)
        return prefill_dense(self, xq, xk, xv, kv_cache, is_causal)


__all__ = ["AsyncOffloadedKVCache", "HipAsyncOffloadAttention"]
