"""HIP sparse GQA attention backend — drop-in for SparseAttention
(model/attention/sparse.py:65-439) and, in mode "dense", for DenseAttention
(model/attention/dense.py), with the block gather of
gather_kv_blocks (model/attention/sparse.py:19-62).

Prefill: compressor, then the router and the block-sparse attention in one
launch (bf16 MFMA kernel that routes its own query windows, for D = 64 and
blocks of 32 or 64 keys), or router then prefill kernel for other shapes. Up
to 8192 tokens the per-token allowed set is the reference's masked-SDPA rule
(sparse.py:226-281); past that length, or when the caller passes
use_chunked_gather=True, the chunked path (sparse.py:284-364, 420): one list
per query block of block_size rows (the union of its rows' non-causal picks,
cut to k+2 blocks) and causal attention over it; use_chunked_gather=False
keeps the per-token rule at any length.

Decode (T == 1 with a KVCache): one libsparda call — whole-cache
compression, routing, split-K attention over the selected blocks, combine.
"""

from typing import Optional, Tuple

import torch

import sparda
from model.attention.base import BaseAttention, KVCache
from model.config import ModelConfig
from model.forecast import ForecastBlockSelector, KVBlockCompressor
from model.rope import RotaryEmbedding

# prefill lengths above this take the chunked path unless the caller says
# otherwise (model/attention/sparse.py:420)
CHUNKED_GATHER_MIN_T = 8192


def gather_kv_blocks(k: torch.Tensor, v: torch.Tensor, block_indices: torch.Tensor,
                     block_size: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """k, v [B,Hkv,S,D], block_indices [B,Hkv,n] -> [B,Hkv,n*bs,D]; tokens past S are zero."""
    return sparda.gather_blocks(k, v, block_indices, block_size)


class PrototypeKVCache(KVCache):
    """KVCache that keeps fp32 block sums of its keys current: sums / bs are
    the block prototypes of KVBlockCompressor (model/forecast.py:66-78), so a
    decode step selects blocks from the sums instead of recompressing all S
    keys (model/attention/sparse.py:133-135). Each update recomputes the
    blocks it touches from their first token, so the sums equal a fresh
    compression bit for bit.

    A single-token append inside the current block leaves that block's sums
    to the next decode launch (``current_block_stale``; decode_sums with
    update_current recomputes them there); any other update, or a consumer
    that reads ``block_sums`` directly after ``refresh_sums()``, sees them
    current."""

    def __init__(self, max_batch_size: int, max_seq_len: int, n_kv_head: int, head_dim: int,
                 device: torch.device, dtype: torch.dtype, block_size: int = 64):
        super().__init__(max_batch_size, max_seq_len, n_kv_head, head_dim, device, dtype)
        self.block_size = block_size
        nb = (max_seq_len + block_size - 1) // block_size
        self.block_sums = torch.zeros((max_batch_size, nb, n_kv_head, head_dim), device=device,
                                      dtype=torch.float32)
        self.current_block_stale = False

    def refresh_sums(self) -> None:
        """Bring the current block's sums up to date (after deferred appends)."""
        if self.current_block_stale and self.current_len > 0:
            first = ((self.current_len - 1) // self.block_size) * self.block_size
            sparda.block_sums(self.k, first, self.current_len - first, self.block_size, self.block_sums)
        self.current_block_stale = False

    def update(self, xk: torch.Tensor, xv: torch.Tensor):
        pos = self.current_len
        same_block = pos > 0 and pos % self.block_size != 0
        if not (xk.shape[1] == 1 and (same_block or not self.current_block_stale)):
            self.refresh_sums()  # a deferred block that this update would leave behind
        out = super().update(xk, xv)
        if xk.shape[1] == 1:
            self.current_block_stale = True  # the decode launch recomputes it
        else:
            first = (pos // self.block_size) * self.block_size
            sparda.block_sums(self.k, first, self.current_len - first, self.block_size, self.block_sums)
        return out

    def reset(self):
        super().reset()
        self.current_block_stale = False


class HipSparseAttention(BaseAttention):
    """Forecast-guided (or static window) block-sparse GQA on libsparda."""

    def __init__(self, config: ModelConfig, layer_idx: int, mode: Optional[str] = None):
        super().__init__(config, layer_idx)
        self.block_size = config.block_size
        self.top_k_blocks = config.top_k_blocks
        if mode is not None:
            self.mode = mode
        elif config.attention_backend in ("static_sparse", "static"):
            self.mode = "static"
        elif getattr(config, "sparse_mode", "forecast") == "static":
            self.mode = "static"
        else:
            self.mode = "forecast"
        if self.mode not in ("forecast", "static", "dense"):
            raise ValueError(f"unknown sparse mode {self.mode!r}")
        self.decode_routing = getattr(config, "decode_routing", "reference")
        # parameter-free, kept for interface parity with the reference module
        self.compressor = KVBlockCompressor(self.block_size, self.head_dim, config.forecast_dim)
        self.selector = ForecastBlockSelector(self.block_size, config.forecast_dim)
        self._ws = None

    # -- decode ------------------------------------------------------------
    def _project(self, out: torch.Tensor, residual: Optional[torch.Tensor] = None) -> torch.Tensor:
        """wo of a decode step's output [B, Hq*D]; with residual, residual +
        wo(out) in one kernel (sparda.rows_residual)."""
        o = out.view(out.shape[0], 1, self.n_head * self.head_dim)
        if residual is None:
            return self.wo(o)
        return sparda.rows_residual(o, self.wo.weight, residual)

    def _decode(self, xq: torch.Tensor, cache: KVCache, forecast_vector: Optional[torch.Tensor],
                residual: Optional[torch.Tensor] = None):
        B = xq.shape[0]
        if self._ws is None or self._ws.device != xq.device:
            self._ws = sparda.DecodeWorkspace(xq.device)
        if self.mode == "dense":
            out = sparda.decode_selected(xq[:, 0], cache.k, cache.v, cache.current_len, self.block_size)
            return self._project(out, residual)
        f = forecast_vector if (self.mode == "forecast" and forecast_vector is not None) else None
        if f is not None:
            f = f.reshape(B, self.n_kv_head, -1)
        if f is not None and isinstance(cache, PrototypeKVCache) and cache.block_size == self.block_size:
            # cached prototypes: select from the block sums and attend in place, one launch
            out = sparda.decode_sums(xq[:, 0], cache.k, cache.v, cache.current_len, f, cache.block_sums,
                                     self.block_size, self.top_k_blocks, routing=self.decode_routing,
                                     update_current=cache.current_block_stale)
            cache.current_block_stale = False
            return self._project(out, residual)
        out = sparda.decode(xq[:, 0], cache.k, cache.v, cache.current_len, f, self.block_size,
                            self.top_k_blocks, routing=self.decode_routing, workspace=self._ws)
        return self._project(out, residual)

    # -- prefill -----------------------------------------------------------
    def _dense_prefill(self, T, forecast_vector):
        """The dense fallback of sparse.py:201-224: dense mode, at most two
        blocks, or forecast mode without a forecast (and at layer 0)."""
        nb = (T + self.block_size - 1) // self.block_size
        return self.mode == "dense" or nb <= 2 or (
            self.mode == "forecast" and (forecast_vector is None or self.layer_idx == 0))

    def _selection(self, xq, xk, forecast_vector, is_causal):
        """The allowed-block lists of a prefill (sparse.py:201-253): None for
        the dense fallback, else router lists (forecast) or the static window
        {0} U [own-k, own]; without causality every listed block is attended
        in full."""
        B, T = xq.shape[:2]
        nb = (T + self.block_size - 1) // self.block_size
        if self._dense_prefill(T, forecast_vector):
            return None, None
        if self.mode == "forecast":
            protos = sparda.compress(xk, self.block_size)
            _, _, sel, n_sel = sparda.route(forecast_vector, protos, self.block_size, self.top_k_blocks,
                                            causal=is_causal, want_topk=False, want_sel=True)
            return sel, n_sel
        return sparda.select_fixed(sparda.SEL_WINDOW_PREFILL, B, T, self.n_kv_head, nb, self.block_size,
                                   self.top_k_blocks, 0, device=xq.device)

    def _chunked_prefill(self, xq, xk, xv, forecast_vector):
        """The chunked-gather prefill (sparse.py:284-364): per query block of
        block_size rows one list, {0, own} U the union of its rows' non-causal
        top-k (forecast mode with a forecast, from the second block on) or the
        static window, cut to min(NB, k+2) (lowest block indices), then the
        causal attention over it. Like the reference's chunked path it takes no
        mask, causality flag or weights."""
        topk = None
        if self.mode == "forecast" and forecast_vector is not None:
            protos = sparda.compress(xk, self.block_size)
            topk = sparda.route(forecast_vector, protos, self.block_size, self.top_k_blocks, causal=False)[0]
        return self.wo(sparda.prefill_chunked(xq, xk, xv, topk, self.block_size, self.top_k_blocks))

    def _prefill(self, xq, xk, xv, forecast_vector, is_causal, mask=None, return_attn_weights=False,
                 use_chunked_gather=None):
        if use_chunked_gather is None:
            # the reference's default: the chunked path past 8192 tokens
            # (sparse.py:420), whatever mask, causality or weights are asked for
            use_chunked_gather = xq.shape[1] > CHUNKED_GATHER_MIN_T
        if use_chunked_gather and self.mode != "dense":
            return self._chunked_prefill(xq, xk, xv, forecast_vector)
        if (mask is None and not return_attn_weights and self.mode == "forecast"
                and not self._dense_prefill(xq.shape[1], forecast_vector)):
            # compressor, then router and attention in one call (one launch
            # where the shape allows)
            protos = sparda.compress(xk, self.block_size)
            return self.wo(sparda.prefill_routed(xq, xk, xv, forecast_vector, protos, self.block_size,
                                                 self.top_k_blocks, causal=is_causal))
        sel, n_sel = self._selection(xq, xk, forecast_vector, is_causal)
        if mask is None and not return_attn_weights:
            return self.wo(sparda.prefill(xq, xk, xv, sel, n_sel, self.block_size, causal=is_causal))
        # explicit additive mask and/or the weights (sparse.py:206-221, 255-281)
        res = sparda.prefill_masked(xq, xk, xv, sel, n_sel, self.block_size, causal=is_causal, mask=mask,
                                    want_weights=return_attn_weights)
        if return_attn_weights:
            out, weights = res
            return self.wo(out), weights
        return self.wo(res)

    def forward(self, x: torch.Tensor, rotary_emb: RotaryEmbedding, kv_cache: Optional[KVCache] = None,
                mask: Optional[torch.Tensor] = None, is_causal: bool = True,
                forecast_vector: Optional[torch.Tensor] = None, **kwargs) -> torch.Tensor:
        B, T, _ = x.shape
        xq = self.wq(x).view(B, T, self.n_head, self.head_dim)
        xk = self.wk(x).view(B, T, self.n_kv_head, self.head_dim)
        xv = self.wv(x).view(B, T, self.n_kv_head, self.head_dim)
        offset = kv_cache.current_len if kv_cache is not None else 0
        xq, xk = rotary_emb(xq, xk, offset=offset)
        # use_chunked_gather: the per-query-block routing (sparse.py:284-364);
        # absent, it follows the length (past 8192 tokens, sparse.py:420)
        chunked = kwargs.get("use_chunked_gather")
        return self.forward_projected(xq, xk, xv, kv_cache=kv_cache, is_causal=is_causal,
                                      forecast_vector=forecast_vector, mask=mask,
                                      return_attn_weights=kwargs.get("return_attn_weights", False),
                                      use_chunked_gather=None if chunked is None else bool(chunked))

    def forward_projected(self, xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor,
                          kv_cache: Optional[KVCache] = None, is_causal: bool = True,
                          forecast_vector: Optional[torch.Tensor] = None,
                          residual: Optional[torch.Tensor] = None, mask: Optional[torch.Tensor] = None,
                          return_attn_weights: bool = False, use_chunked_gather: Optional[bool] = None):
        """The attention after the projections and RoPE: xq [B,T,Hq,D], xk / xv
        [B,T,Hkv,D] (already rotated at the cache's current position). Entered
        from forward, or directly by a block whose fused producer computed them.
        With residual (single-token decode only) the result is residual +
        attention, the projection and the sum in one kernel. A prefill with an
        additive mask or return_attn_weights returns (out, weights) as the
        reference does; a decode step ignores both, as the reference's does
        (sparse.py:398-410). use_chunked_gather (None: T > 8192) picks the
        chunked prefill, which like the reference's takes no mask, causality
        flag or weights (sparse.py:420-428)."""
        T = xq.shape[1]
        if kv_cache is not None and T == 1:
            kv_cache.update(xk, xv)
            return self._decode(xq, kv_cache, forecast_vector, residual)
        if residual is not None:
            raise ValueError("forward_projected: residual is for single-token decode steps")
        if kv_cache is not None:
            if kv_cache.current_len != 0:
                raise NotImplementedError("prefill into a non-empty cache is not supported")
            kv_cache.update(xk, xv)
        return self._prefill(xq, xk, xv, forecast_vector, is_causal, mask, return_attn_weights, use_chunked_gather)
