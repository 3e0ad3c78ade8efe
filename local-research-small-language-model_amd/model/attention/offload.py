"""KV cache in pinned host memory + forecast-guided block fetch (the
synchronous offload backend) — drop-in for OffloadedKVCache and
ForecastOffloadAttention (model/attention/offload.py:23-294).

The authoritative K/V live in a pinned host arena owned by libsparda
(``sparda.OffloadArena``, layout [B][Hkv][Smax][D], so one KV block of one
head is one contiguous run). ``update`` writes new tokens into it from the GPU
and keeps fp32 block sums on the GPU for the touched blocks, so routing never
needs the full K on the device (the reference copies and recompresses the
whole K cache every step, offload.py:218-223). A decode step selects blocks
from the sums, fetches them into a compact device buffer and attends over it —
all stream-ordered, with no host synchronisation.
"""

from typing import Dict, Optional, Tuple

import torch

import sparda
from model.attention.base import BaseAttention, KVCache
from model.config import ModelConfig
from model.forecast import ForecastBlockSelector, KVBlockCompressor
from model.rope import RotaryEmbedding


class OffloadedKVCache:
    """Authoritative KV cache in pinned host memory (model/attention/offload.py:23-128).

    ``cpu_k`` / ``cpu_v`` are [B,Smax,Hkv,D] CPU views of the library-owned
    arena. ``block_size`` (optional) starts GPU block sums right away; otherwise
    they are built on first use by ``block_sums``.
    """

    def __init__(self, max_batch_size: int, max_seq_len: int, n_kv_head: int, head_dim: int,
                 gpu_device: torch.device, dtype: torch.dtype = torch.bfloat16, pin_memory: bool = True,
                 block_size: Optional[int] = None):
        self.max_batch_size = max_batch_size
        self.max_seq_len = max_seq_len
        self.n_kv_head = n_kv_head
        self.head_dim = head_dim
        self.gpu_device = torch.device(gpu_device)
        self.dtype = dtype
        if self.gpu_device.type != "cuda":
            raise RuntimeError("OffloadedKVCache: the HIP offload path needs a GPU device")
        # the arena is always pinned (hipHostMalloc); pin_memory is accepted for interface parity
        self.arena = sparda.OffloadArena(max_batch_size, max_seq_len, n_kv_head, head_dim, dtype, self.gpu_device)
        self.cpu_k = self.arena.k_host
        self.cpu_v = self.arena.v_host
        self.current_len = 0
        self.total_bytes_transferred = 0
        self.total_transfer_calls = 0
        self._bs: Optional[int] = None
        self._sums: Optional[torch.Tensor] = None
        if block_size is not None:
            self._init_sums(block_size, rebuild=False)

    # -- block sums (prototypes * bs) --------------------------------------
    def _init_sums(self, block_size: int, rebuild: bool) -> None:
        nb = (self.max_seq_len + block_size - 1) // block_size
        self._sums = torch.zeros((self.max_batch_size, nb, self.n_kv_head, self.head_dim), dtype=torch.float32,
                                 device=self.gpu_device)
        self._bs = block_size
        if rebuild and self.current_len > 0:
            self.arena.rebuild_sums(self.current_len, block_size, self._sums)

    def block_sums(self, block_size: int) -> torch.Tensor:
        """fp32 block sums [B, ceil(Smax/bs), Hkv, D] of tokens [0, current_len)."""
        if self._bs != block_size:
            self._init_sums(block_size, rebuild=True)
        return self._sums

    # -- reference interface ------------------------------------------------
    def update(self, xk: torch.Tensor, xv: torch.Tensor) -> int:
        """Append [B,n,Hkv,D] (on the GPU) at current_len (offload.py:67-77)."""
        n = xk.shape[1]
        if self.current_len + n > self.max_seq_len:
            raise ValueError(f"OffloadedKVCache overflow: {self.current_len + n} > capacity {self.max_seq_len}")
        self.arena.append(xk.detach(), xv.detach(), self.current_len, self._bs or 0, self._sums)
        self.current_len += n
        return self.current_len

    def get_full_cpu_kv(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """CPU views of tokens [0, current_len) (offload.py:79-81); reading them
        on the host needs the appends to have completed (synchronise first)."""
        return self.cpu_k[:, :self.current_len], self.cpu_v[:, :self.current_len]

    def fetch(self, sel: torch.Tensor, n_sel: torch.Tensor, block_size: int, length: Optional[int] = None,
              method: int = sparda.FETCH_KERNEL, out: Optional[Tuple[torch.Tensor, torch.Tensor]] = None):
        """Selected blocks into compact [B,Hkv,cap,bs,D] device buffers (stream-ordered)."""
        length = self.current_len if length is None else length
        cap = sel.shape[-1]
        if out is None:
            shape = (self.max_batch_size, self.n_kv_head, cap, block_size, self.head_dim)
            out = (torch.zeros(shape, dtype=self.dtype, device=self.gpu_device),
                   torch.zeros(shape, dtype=self.dtype, device=self.gpu_device))
        self.arena.fetch(sel, n_sel, block_size, length, out[0], out[1], method)
        return out

    def transfer_selected_blocks(self, block_indices: torch.Tensor, block_size: int,
                                 non_blocking: bool = True) -> Tuple[torch.Tensor, torch.Tensor, int]:
        """block_indices [B,Hkv,n] -> gpu_k, gpu_v [B,Hkv,n*bs,D] (offload.py:83-123).

        Tokens at or past current_len read as zeros, as in the reference's
        padded gather; bytes are counted as the reference counts them."""
        B, H, n = block_indices.shape
        idx = block_indices.to(self.gpu_device, torch.int32).contiguous()
        cnt = torch.full((B, H), n, dtype=torch.int32, device=self.gpu_device)
        k, v = self.fetch(idx, cnt, block_size)
        gk = k.view(B, H, n * block_size, self.head_dim)
        gv = v.view(B, H, n * block_size, self.head_dim)
        if not non_blocking:
            torch.cuda.current_stream(self.gpu_device).synchronize()
        nbytes = (gk.numel() + gv.numel()) * gk.element_size()
        self.total_bytes_transferred += nbytes
        self.total_transfer_calls += 1
        return gk, gv, nbytes

    def reset(self):
        self.current_len = 0
        self.total_bytes_transferred = 0
        self.total_transfer_calls = 0


def dense_from_arena(cache: OffloadedKVCache, xq: torch.Tensor, length: int, block_size: int,
                     k_new: Optional[torch.Tensor] = None, v_new: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense decode attention of xq [B,Hq,D] over tokens [0, length+1): blocks
    of tokens [0, length) fetched from the arena, position `length` from
    k_new/v_new when given (else from the arena)."""
    S = length + 1 if k_new is not None else length
    nb = (S + block_size - 1) // block_size
    B, H = cache.max_batch_size, cache.n_kv_head
    sel = torch.arange(nb, dtype=torch.int32, device=xq.device).repeat(B, H, 1).contiguous()
    cnt = torch.full((B, H), nb, dtype=torch.int32, device=xq.device)
    shape = (B, H, nb, block_size, cache.head_dim)
    kb = torch.empty(shape, dtype=cache.dtype, device=xq.device)
    vb = torch.empty(shape, dtype=cache.dtype, device=xq.device)
    cache.arena.fetch(sel, cnt, block_size, length if k_new is not None else S, kb, vb)
    # the fetched blocks form a [B,Hkv,nb*bs,D] cache: view it as [B,S',Hkv,D]
    kc = kb.view(B, H, nb * block_size, cache.head_dim).transpose(1, 2)
    vc = vb.view(B, H, nb * block_size, cache.head_dim).transpose(1, 2)
    return sparda.decode_selected(xq, kc, vc, S, block_size, k_new=k_new, v_new=v_new)


class HipOffloadAttention(BaseAttention):
    """Forecast-guided offload decode on libsparda (model/attention/offload.py:131-320).

    Prefill: the cache is appended and dense causal attention runs on the GPU
    (as the reference's prefill path does). Decode: append the token, select
    blocks from the GPU block sums, fetch them from the arena, attend; dense
    over the whole context when NB <= k+2, without a forecast, or at layer 0.
    """

    def __init__(self, config: ModelConfig, layer_idx: int, fetch_method: int = sparda.FETCH_KERNEL):
        super().__init__(config, layer_idx)
        self.block_size = config.block_size
        self.top_k_blocks = config.top_k_blocks
        self.decode_routing = getattr(config, "decode_routing", "reference")
        self.fetch_method = fetch_method
        self.compressor = KVBlockCompressor(self.block_size, self.head_dim, config.forecast_dim)
        self.selector = ForecastBlockSelector(self.block_size, config.forecast_dim)
        self.last_profile: Dict[str, float] = {}

    def _offload_decode(self, xq: torch.Tensor, xk: torch.Tensor, xv: torch.Tensor, cache: OffloadedKVCache,
                        forecast_vector: Optional[torch.Tensor]) -> torch.Tensor:
        B = xq.shape[0]
        bs, k = self.block_size, self.top_k_blocks
        sums = cache.block_sums(bs)
        S = cache.update(xk, xv)
        nb = (S + bs - 1) // bs
        if nb <= k + 2 or forecast_vector is None or self.layer_idx == 0:
            out = dense_from_arena(cache, xq, S, bs)
            nbytes = 2 * B * self.n_kv_head * S * self.head_dim * xq.element_size()
        else:
            sel, n_sel = sparda.select_decode(forecast_vector.reshape(B, self.n_kv_head, -1), sums, S, S - 1, bs,
                                              k, routing=self.decode_routing)
            kb, vb = cache.fetch(sel, n_sel, bs, S, self.fetch_method)
            out = sparda.decode_selected(xq, kb, vb, S, bs, sel, n_sel, compact=True)
            nbytes = 2 * B * self.n_kv_head * (k + 2) * bs * self.head_dim * xq.element_size()
        cache.total_bytes_transferred += nbytes
        cache.total_transfer_calls += 1
        self.last_profile = {"bytes_transferred": nbytes}
        return self.wo(out.view(B, 1, self.n_head * self.head_dim))

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
            return self._offload_decode(xq[:, 0], xk, xv, kv_cache, forecast_vector)
        if kv_cache is not None and T == 1:
            return resident_dense_decode(self, xq, xk, xv, kv_cache)
        return prefill_dense(self, xq, xk, xv, kv_cache, is_causal)


def resident_dense_decode(attn: BaseAttention, xq, xk, xv, kv_cache: KVCache) -> torch.Tensor:
    """Decode step of an offload backend whose layer keeps a GPU-resident
    KVCache (layer 0, which is never prefetched): dense attention over the
    cache, the attention the reference's offload fallback computes there
    (offload.py:180-214; async_offload.py:392-430)."""
    B = xq.shape[0]
    kv_cache.update(xk, xv)
    out = sparda.decode_selected(xq[:, 0], kv_cache.k, kv_cache.v, kv_cache.current_len, attn.config.block_size)
    return attn.wo(out.view(B, 1, attn.n_head * attn.head_dim))


def prefill_dense(attn: BaseAttention, xq, xk, xv, kv_cache, is_causal: bool) -> torch.Tensor:
    """Prefill of the offload backends: cache append + dense causal attention
    over the prompt (model/attention/offload.py:320-345; async_offload.py:547-573)."""
    if kv_cache is not None:
        if kv_cache.current_len != 0:
            raise NotImplementedError("prefill into a non-empty cache is not supported")
        kv_cache.update(xk, xv)
    out = sparda.prefill(xq, xk, xv, None, None, attn.config.block_size, causal=is_causal and xq.shape[1] > 1)
    return attn.wo(out)


__all__ = ["OffloadedKVCache", "HipOffloadAttention", "KVCache", "dense_from_arena", "prefill_dense",
           "resident_dense_decode"]
