"""Token-by-token generation replayed from one captured HIP graph
(SparDAResearchModel.generate with KV caches, model/model.py:159-195).

The reference's loop runs one host-driven forward per token: every layer
re-reads the cache length on the host (KVCache.update,
model/attention/base.py:11-32; the decode branch of SparseAttention.forward,
model/attention/sparse.py:99-183), so each step is ~15 launches per layer
issued one by one. Here the position of the token being decoded lives in
device memory (``pos``, int64) and every position-dependent launch reads it
when it runs:

  fused producer  RMSNorm + q/k/v/forecast projections + RoPE at *pos
  cache append    k / v row *pos written, and the fp32 sums of the block
                  holding it recomputed from its first token (one launch)
  selection and   layer 0 and static layers: the static window; forecast
  attention       layers: top-k of the previous layer's forecast against the
                  cached prototypes (block sums / bs), sink and own block,
                  scored and selected inside the attention launch; the
                  selected blocks of a cache holding *pos + 1 tokens
  LM head         logits of the step; *pos += 1 last

so one recorded step serves every token: a step is one graph replay.

Layers of HipAsyncOffloadAttention keep their KV in a pinned host arena
(AsyncOffloadedKVCache; layer 0 then keeps a GPU-resident KVCache and attends
densely, as the eager path does). Layer L's block issues the prefetch of
layer L+1 right after its producer has formed F_L (transformer.py:110-115):
the selection from layer L+1's block sums (the lookahead before token *pos
is appended, async_offload.py:196-260) and the gather of the selected blocks
from the arena into device buffers, then an event that layer L+1 waits for.
With overlap="fused" (the default) the selection and the copy over the host
link run as extra workgroups of layer L's attention launch
(sparda_decode_at_prefetch), beside its attention workgroups: the overlap the
reference gets from its transfer stream, without a cross-stream dependency
in the graph. When layer L is offloaded too, the selection rides on layer L's
arena-append launch and only the copy on its attention launch. overlap=False issues them as launches of their own on the
compute stream, overlap=True on a side stream joined by an event. Layer L+1
then appends its token into the arena and attends over the fetched blocks
with the new token supplied separately.

The kernels and their launch shapes are those of the eager decode with the
fused producer (HipSparseAttention with PrototypeKVCache, or
HipAsyncOffloadAttention with AsyncOffloadedKVCache), so a replayed step
reproduces the eager step bit for bit while the cache holds more than
top_k + 2 blocks (below that the eager path attends every block through
another wavefront split).

Requirements: HipSparseAttention or HipAsyncOffloadAttention layers, bf16
weights, head dim 64, forecast dim 64 (the fused producer's shape).

The recorded step reads the parameters and the weight copies folded from
them (each block's stacked producer and FFN weights with their RMSNorm
weights folded in, and the folded output head) at the addresses they had
when it was recorded. The decoder holds a reference to every folded copy, so
that memory stays valid, and keys every parameter by (data_ptr, version): a
step that finds a parameter replaced or changed in place records the step
again from the current weights.
"""

from typing import List, Optional, Sequence

import torch
import torch.nn.functional as F

import sparda
from model.attention.async_offload import AsyncOffloadedKVCache, HipAsyncOffloadAttention
from model.attention.base import KVCache
from model.attention.hip_sparse import HipSparseAttention, PrototypeKVCache

_SPARSE, _RESIDENT_DENSE, _OFFLOAD = "sparse", "resident_dense", "offload"


class GraphDecoder:
    """Owns (or adopts) one cache per layer and the device-held position.

    caches: None (a PrototypeKVCache per sparse layer; for offload layers a
    GPU KVCache at layer 0 and an AsyncOffloadedKVCache elsewhere), or one
    cache per layer of those types, all holding the same number of tokens
    (their contents are decoded on from there). overlap selects where the
    offload prefetch of layer L+1 runs: "fused" (default) inside layer L's
    attention launch; False as launches of its own on the compute stream;
    True on a side stream joined by an event before the layer that needs it
    (each cross-stream dependency inside a replayed graph costs more than the
    selection and host-link copy it would hide).

    taps: layers whose attention inputs and output the recorded step keeps in
    ``tapped[i]`` (q [B,Hq,D], the routing forecast or None, the attention
    output [B,Hq*D], and for an offloaded layer the prefetched selection),
    buffers that every replay rewrites, for checking a replayed step."""

    def __init__(self, model, batch_size: int, max_seq_len: int, caches: Optional[Sequence] = None,
                 overlap="fused", taps: Sequence[int] = ()):
        cfg = model.config
        p = next(model.parameters())
        self.device = p.device
        if not p.is_cuda or p.dtype != torch.bfloat16:
            raise TypeError("GraphDecoder: the model must be bf16 on the GPU")
        kinds = []
        for i, layer in enumerate(model.layers):
            a = layer.attention
            if type(a) is HipSparseAttention:
                kinds.append(_SPARSE)
            elif type(a) is HipAsyncOffloadAttention:
                kinds.append(_RESIDENT_DENSE if i == 0 else _OFFLOAD)
            else:
                raise TypeError(f"GraphDecoder: layer {layer.layer_idx} uses {type(a).__name__}, not "
                                "HipSparseAttention or HipAsyncOffloadAttention")
            if a.head_dim != 64 or layer.forecast.forecast_dim != 64:
                raise ValueError("GraphDecoder: head dim and forecast dim must be 64")
        if max_seq_len > cfg.context_length:
            raise ValueError(f"GraphDecoder: max_seq_len {max_seq_len} beyond the context {cfg.context_length}")
        self.model = model
        self.kinds = kinds
        self.B = batch_size
        self.max_len = max_seq_len
        self.block_size = cfg.block_size
        if overlap not in (False, True, "fused"):
            raise ValueError(f"GraphDecoder: overlap must be False, True or 'fused', got {overlap!r}")
        self.overlap = overlap
        bs, H, D = cfg.block_size, cfg.n_kv_head, cfg.head_dim
        if caches is None:
            caches = []
            for kind in kinds:
                if kind == _SPARSE:
                    caches.append(PrototypeKVCache(batch_size, max_seq_len, H, D, self.device, torch.bfloat16,
                                                   block_size=bs))
                elif kind == _RESIDENT_DENSE:
                    caches.append(KVCache(batch_size, max_seq_len, H, D, self.device, torch.bfloat16))
                else:
                    caches.append(AsyncOffloadedKVCache(batch_size, max_seq_len, H, D, self.device, torch.bfloat16,
                                                        block_size=bs))
        caches = list(caches)
        want = {_SPARSE: PrototypeKVCache, _RESIDENT_DENSE: KVCache, _OFFLOAD: AsyncOffloadedKVCache}
        if len(caches) != len(kinds):
            raise ValueError("GraphDecoder: one cache per layer")
        for i, (kind, c) in enumerate(zip(kinds, caches)):
            if not isinstance(c, want[kind]) or (kind == _SPARSE and c.block_size != bs):
                raise TypeError(f"GraphDecoder: layer {i} needs a {want[kind].__name__}")
            cap = c.max_seq_len if kind == _OFFLOAD else c.k.shape[1]
            nb_ = c.max_batch_size if kind == _OFFLOAD else c.k.shape[0]
            if cap < max_seq_len or nb_ != batch_size:
                raise ValueError(f"GraphDecoder: the cache of layer {i} is smaller than {batch_size} x {max_seq_len}")
        lens = {c.current_len for c in caches}
        if len(lens) != 1:
            raise ValueError("GraphDecoder: the caches hold different numbers of tokens")
        for c in caches:
            if isinstance(c, PrototypeKVCache):
                c.refresh_sums()  # the recorded appends keep the sums current from here on
        self.caches = caches
        self.length = lens.pop()
        self.pos = torch.full((1,), self.length, dtype=torch.int64, device=self.device)
        self.tok = torch.zeros((batch_size, 1), dtype=torch.int64, device=self.device)
        self.cos, self.sin = model.rotary_emb.tables(max_seq_len, self.device)
        # prefetch buffers and events of the offloaded layers
        k = cfg.top_k_blocks
        self._side = torch.cuda.Stream(device=self.device)
        self._pf = {}
        for i, kind in enumerate(kinds):
            if kind == _OFFLOAD:
                self._pf[i] = dict(
                    sel=torch.empty((batch_size, H, k + 2), dtype=torch.int32, device=self.device),
                    n=torch.empty((batch_size, H), dtype=torch.int32, device=self.device),
                    k=torch.empty((batch_size, H, k + 2, bs, D), dtype=torch.bfloat16, device=self.device),
                    v=torch.empty((batch_size, H, k + 2, bs, D), dtype=torch.bfloat16, device=self.device),
                    ev=torch.cuda.Event())
                caches[i].block_sums(bs)  # start the block sums before anything is captured
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.logits: Optional[torch.Tensor] = None
        self._taps = frozenset(taps)
        self.tapped = {}
        self._held: List[torch.Tensor] = []
        self._keys = None

    # -- one decode step, every launch reading *pos --------------------------
    def _producer_appends(self, i: int, a, f: Optional[torch.Tensor]) -> bool:
        """Layer i's producer writes the new row into its cache and the decode
        launch re-sums the current block (the forecast-routed sparse layers)."""
        return self.kinds[i] == _SPARSE and a.mode not in ("dense", "static") and f is not None

    def _attend(self, i: int, a, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                f: Optional[torch.Tensor], carry=None, parts: int = 1) -> torch.Tensor:
        """Layer i's append and attention; carry = (j, f_i): layer j's prefetch
        for this step, carried by the attention launch (on an offloaded layer:
        its selection by the append launch, share 0 of `parts` of its copy by
        the attention launch)."""
        bs = self.block_size
        cache = self.caches[i]
        kind = self.kinds[i]
        nxt = self._prefetch_spec(*carry) if carry is not None else None
        if kind == _OFFLOAD:
            pf = self._pf[i]
            torch.cuda.current_stream().wait_event(pf["ev"])
            # a carried prefetch: its selection rides on the append launch, its
            # host-link copy on the attention launch
            cache.arena.append_at(k, v, self.pos, bs, cache.block_sums(bs),
                                  prefetch=None if nxt is None else {**nxt, "stage": 1}, max_len=self.max_len)
            return sparda.decode_at(q, pf["k"], pf["v"], self.pos, bs, pf["sel"], pf["n"], max_len=self.max_len,
                                    compact=True, k_new=k[:, 0], v_new=v[:, 0],
                                    prefetch=None if nxt is None else {**nxt, "stage": 2, "parts": parts, "part": 0})
        if kind == _RESIDENT_DENSE:
            sparda.append_at(cache.k, cache.v, self.pos, bs, None, k, v)
            return sparda.decode_at(q, cache.k, cache.v, self.pos, bs, window=0, max_len=self.max_len,
                                    prefetch=nxt)
        if self._producer_appends(i, a, f):
            if carry is not None:  # this launch carries no prefetch: issue it first
                self._prefetch(*carry)
            return sparda.decode_sums(q, cache.k, cache.v, self.max_len, f, cache.block_sums, bs, a.top_k_blocks,
                                      routing=a.decode_routing, pos_dev=self.pos, update_current=True)
        # dense / static-window layers: the append keeps the block sums current
        sparda.append_at(cache.k, cache.v, self.pos, bs, cache.block_sums, k, v)
        window = 0 if a.mode == "dense" else a.top_k_blocks
        return sparda.decode_at(q, cache.k, cache.v, self.pos, bs, window=window, max_len=self.max_len,
                                prefetch=nxt)

    def _prefetch_spec(self, i: int, f: torch.Tensor) -> dict:
        """Layer i's prefetch for this step (from layer i-1's forecast), as a
        decode launch carries it."""
        a = self.model.layers[i].attention
        cache, pf = self.caches[i], self._pf[i]
        return dict(arena=cache.arena, forecast=f.reshape(self.B, a.n_kv_head, -1),
                    block_sums=cache.block_sums(self.block_size), top_k=a.top_k_blocks, routing=a.decode_routing,
                    sel=pf["sel"], n_sel=pf["n"], k_dst=pf["k"], v_dst=pf["v"])

    def _prefetch(self, i: int, f: torch.Tensor):
        """Selection + gather of layer i's blocks for this step, from layer i-1's forecast."""
        a = self.model.layers[i].attention
        cache, pf, bs = self.caches[i], self._pf[i], self.block_size
        sparda.select_decode_at(f.reshape(self.B, a.n_kv_head, -1), cache.block_sums(bs), self.pos, self.max_len,
                                bs, a.top_k_blocks, routing=a.decode_routing, sel=pf["sel"], n_sel=pf["n"],
                                lookahead=True)
        cache.arena.fetch_at(pf["sel"], pf["n"], bs, self.pos, pf["k"], pf["v"])

    def _step(self):
        m = self.model
        B = self.B
        main = torch.cuda.current_stream()
        x = m.embeddings.embed(self.tok)
        prev_f = None
        n = len(m.layers)
        for i, layer in enumerate(m.layers):
            a = layer.attention
            fc = layer.forecast
            cache = self.caches[i]
            kc, vc = (cache.k, cache.v) if self._producer_appends(i, a, prev_f) else (None, None)
            q, k, v, f = sparda.produce(x, layer._fused_weight(), a.n_head * a.head_dim, a.n_kv_head * a.head_dim,
                                        fc.forecast_heads * fc.forecast_dim, layer.attn_norm.eps, self.cos,
                                        self.sin, f_dtype=x.dtype, pos_dev=self.pos, k_cache=kc, v_cache=vc)
            carry = None
            if i + 1 < n and self.kinds[i + 1] == _OFFLOAD:
                ev = self._pf[i + 1]["ev"]
                if self.overlap == "fused":
                    carry = (i + 1, f)
                elif self.overlap:
                    self._side.wait_stream(main)
                    with torch.cuda.stream(self._side):
                        self._prefetch(i + 1, f)
                        ev.record(self._side)
                else:
                    self._prefetch(i + 1, f)
                    ev.record(main)
            # an offloaded layer with the fused feed-forward spreads the carried
            # copy over its attention and both feed-forward launches
            parts = 3 if (carry is not None and self.kinds[i] == _OFFLOAD and layer._use_fused_ffn(x)) else 1
            out = self._attend(i, a, q[:, 0], k, v, prev_f, carry, parts)
            if i in self._taps:
                t = dict(q=q[:, 0], f=prev_f, out=out)
                if self.kinds[i] == _OFFLOAD:
                    t.update(sel=self._pf[i]["sel"], n_sel=self._pf[i]["n"])
                self.tapped[i] = t
            if layer._use_fused_wo(x, 1, self.caches[i]):
                x = sparda.rows_residual(out.view(B, 1, a.n_head * a.head_dim), a.wo.weight, x)
            else:
                x = x + a.wo(out.view(B, 1, a.n_head * a.head_dim))
            if parts > 1:
                nxt = self._prefetch_spec(*carry)
                x = sparda.ffn_decode(x, layer._fused_ffn_weight(), layer.ffn.w_down.weight, layer.ffn_norm.eps,
                                      prefetch=tuple({**nxt, "stage": 2, "parts": parts, "part": p}
                                                     for p in (1, 2)),
                                      pos_dev=self.pos, block_size=self.block_size)
            else:
                x = layer.ffn_residual(x)
            if carry is not None:
                self._pf[i + 1]["ev"].record(main)
            prev_f = f
        self.logits = m.logits(x)[:, -1, :]
        self.pos.add_(1)

    def _weight_keys(self):
        return tuple((p.data_ptr(), p._version) for p in self.model.parameters())

    def _capture(self):
        m = self.model
        with torch.no_grad():
            # the folded copies are built outside the graph and held while it lives
            self._held = [m._folded_head()] if getattr(m.config, "fused_ffn", False) else []
            for layer in m.layers:
                self._held += [layer._fused_weight(), layer._fused_ffn_weight()]
            self._keys = self._weight_keys()
            # warm-up step on a side stream (library handles, workspaces), then
            # the position is put back: the replay rewrites the same cache rows
            # and recomputes the same block sums. The prefetch of an offloaded
            # layer selects before its token is appended, so there the sums of
            # the current block are rebuilt without the warm-up's token.
            warm = torch.cuda.Stream()
            warm.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(warm):
                self._step()
                self.pos.sub_(1)
            torch.cuda.current_stream().wait_stream(warm)
            for i, kind in enumerate(self.kinds):
                if kind == _OFFLOAD:
                    c = self.caches[i]
                    c.arena.rebuild_sums(self.length, self.block_size, c.block_sums(self.block_size))
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step()
        self.graph = g

    def reset_graph(self):
        """Drop the recorded step (it is captured again by the next ``step``)."""
        self.graph = None
        self.logits = None
        self.tapped = {}
        self._held = []
        self._keys = None

    # -- public loop ---------------------------------------------------------
    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Run the prompt [B, T] through the model into empty caches (eager,
        sparse prefill); returns the logits of its last position [B, V]."""
        if input_ids.shape[0] != self.B:
            raise ValueError(f"GraphDecoder: batch {input_ids.shape[0]} != {self.B}")
        if self.length != 0:
            raise RuntimeError("GraphDecoder: prefill into non-empty caches; call reset() first")
        T = input_ids.shape[1]
        if T >= self.max_len:
            raise ValueError(f"GraphDecoder: prompt of {T} leaves no room in {self.max_len}")
        logits = self.model(input_ids, kv_caches=self.caches)["logits"][:, -1, :]
        for c in self.caches:
            if isinstance(c, PrototypeKVCache):
                c.refresh_sums()
        self.pos.fill_(T)
        self.length = T
        return logits

    @torch.no_grad()
    def step(self, tokens: torch.Tensor) -> torch.Tensor:
        """Decode tokens [B, 1] at the current position by one graph replay.
        Returns the step's logits [B, V] (a buffer the next step overwrites)."""
        if self.length == 0:
            raise RuntimeError("GraphDecoder: prefill first")
        if self.length >= self.max_len:
            raise ValueError(f"GraphDecoder: the caches are full ({self.max_len} tokens)")
        self.tok.copy_(tokens.reshape(self.B, 1))
        if self.graph is not None and self._weight_keys() != self._keys:
            self.reset_graph()  # a parameter was replaced or changed since the step was recorded
        if self.graph is None:
            self._capture()
        self.graph.replay()
        self.length += 1
        for c in self.caches:
            c.current_len = self.length
        return self.logits

    def reset(self):
        """Empty the caches (the recorded step stays valid: it reads *pos)."""
        for c in self.caches:
            c.reset()
        self.length = 0
        self.pos.zero_()

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 50, temperature: float = 0.8,
                 top_k: int = 50, eos_token_id: Optional[int] = None) -> torch.Tensor:
        """SparDAResearchModel.generate with KV caches (model/model.py:159-195),
        each new token one graph replay."""
        self.model.eval()
        self.reset()
        logits = self.prefill(input_ids)
        for i in range(max_new_tokens):
            if temperature > 0.0:
                logits = logits / temperature
                if top_k is not None and top_k > 0:
                    v, _ = torch.topk(logits, min(top_k, logits.size(-1)))
                    logits = logits.masked_fill(logits < v[:, [-1]], -float("inf"))
                nxt = torch.multinomial(F.softmax(logits.float(), dim=-1), num_samples=1)
            else:
                nxt = torch.argmax(logits, dim=-1, keepdim=True)
            input_ids = torch.cat((input_ids, nxt), dim=1)
            if eos_token_id is not None and (nxt == eos_token_id).all():
                break
            if i + 1 < max_new_tokens:
                logits = self.step(nxt)
        return input_ids
