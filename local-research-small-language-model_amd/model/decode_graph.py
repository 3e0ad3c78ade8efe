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
  selection       layer 0 and static layers: the static window; forecast
                  layers: top-k of the previous layer's forecast against the
                  cached prototypes (block sums / bs), sink and own block
  attention       the selected blocks of a cache holding *pos + 1 tokens
  LM head         logits of the step; *pos += 1 last

so one recorded step serves every token: a step is one graph replay. The
kernels and their launch shapes are those of the eager cached-prototype
decode (HipSparseAttention with PrototypeKVCache and the fused producer), so
a replayed step reproduces the eager step bit for bit while the cache holds
more than top_k + 2 blocks.

Requirements: HipSparseAttention layers, bf16 weights, head dim 64, forecast
dim 64 (the fused producer's shape). Weights are read from the tensors that
exist when the step is captured: capture (the first ``step``) after loading
them, or call ``reset_graph`` after changing them.
"""

from typing import List, Optional

import torch
import torch.nn.functional as F

import sparda
from model.attention.hip_sparse import HipSparseAttention, PrototypeKVCache


class GraphDecoder:
    """Owns one PrototypeKVCache per layer and the device-held position."""

    def __init__(self, model, batch_size: int, max_seq_len: int):
        cfg = model.config
        p = next(model.parameters())
        self.device = p.device
        if not p.is_cuda or p.dtype != torch.bfloat16:
            raise TypeError("GraphDecoder: the model must be bf16 on the GPU")
        for layer in model.layers:
            a = layer.attention
            if type(a) is not HipSparseAttention:
                raise TypeError(f"GraphDecoder: layer {layer.layer_idx} uses {type(a).__name__}, "
                                "not HipSparseAttention")
            if a.head_dim != 64 or layer.forecast.forecast_dim != 64:
                raise ValueError("GraphDecoder: head dim and forecast dim must be 64")
        if max_seq_len > cfg.context_length:
            raise ValueError(f"GraphDecoder: max_seq_len {max_seq_len} beyond the context {cfg.context_length}")
        self.model = model
        self.B = batch_size
        self.max_len = max_seq_len
        self.block_size = cfg.block_size
        self.caches: List[PrototypeKVCache] = [
            PrototypeKVCache(batch_size, max_seq_len, cfg.n_kv_head, cfg.head_dim, self.device, torch.bfloat16,
                             block_size=cfg.block_size) for _ in model.layers]
        self.pos = torch.zeros(1, dtype=torch.int64, device=self.device)
        self.tok = torch.zeros((batch_size, 1), dtype=torch.int64, device=self.device)
        self.length = 0
        self.cos, self.sin = model.rotary_emb.tables(max_seq_len, self.device)
        self.graph: Optional[torch.cuda.CUDAGraph] = None
        self.logits: Optional[torch.Tensor] = None

    # -- one decode step, every launch reading *pos --------------------------
    def _attend(self, a: HipSparseAttention, q: torch.Tensor, cache: PrototypeKVCache,
                f: Optional[torch.Tensor]) -> torch.Tensor:
        bs = self.block_size
        if a.mode == "dense":
            return sparda.decode_at(q, cache.k, cache.v, self.pos, bs, window=0, max_len=self.max_len)
        if a.mode == "static" or f is None:
            return sparda.decode_at(q, cache.k, cache.v, self.pos, bs, window=a.top_k_blocks, max_len=self.max_len)
        sel, n_sel = sparda.select_decode_at(f.reshape(self.B, a.n_kv_head, -1), cache.block_sums, self.pos,
                                             self.max_len, bs, a.top_k_blocks, routing=a.decode_routing)
        return sparda.decode_at(q, cache.k, cache.v, self.pos, bs, sel, n_sel, max_len=self.max_len)

    def _step(self):
        m = self.model
        B = self.B
        x = m.embeddings.embed(self.tok)
        prev_f = None
        for layer, cache in zip(m.layers, self.caches):
            a = layer.attention
            fc = layer.forecast
            q, k, v, f = sparda.produce(x, layer._fused_weight(), a.n_head * a.head_dim, a.n_kv_head * a.head_dim,
                                        fc.forecast_heads * fc.forecast_dim, layer.attn_norm.eps, self.cos,
                                        self.sin, f_dtype=x.dtype, pos_dev=self.pos)
            sparda.append_at(cache.k, cache.v, self.pos, self.block_size, cache.block_sums, k, v)
            out = self._attend(a, q[:, 0], cache, prev_f)
            x = x + a.wo(out.view(B, 1, a.n_head * a.head_dim))
            x = x + layer.ffn(layer.ffn_norm(x))
            prev_f = f
        self.logits = m.embeddings.project(m.final_norm(x))[:, -1, :]
        self.pos.add_(1)

    def _capture(self):
        with torch.no_grad():
            for layer in self.model.layers:
                layer._fused_weight()  # build the stacked weights outside the graph
            # warm-up step on a side stream (library handles, workspaces), then
            # the position is put back: the replay rewrites the same cache rows
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                self._step()
                self.pos.sub_(1)
            torch.cuda.current_stream().wait_stream(side)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self._step()
        self.graph = g

    def reset_graph(self):
        """Drop the recorded step (it is captured again by the next ``step``)."""
        self.graph = None
        self.logits = None

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
