"""Full SparDA language model on the HIP attention backends (model/model.py:17-175).

Layer L's forecast routes layer L+1's blocks; layer 0 attends without a
forecast. Inference-only: the attention backends refuse autograd.
"""

from typing import Dict, List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from model.config import ModelConfig
from model.embeddings import TiedEmbedding
from model.norm import RMSNorm
from model.rope import RotaryEmbedding
from model.transformer import TransformerBlock

import sparda


class SparDAResearchModel(nn.Module):
    """Token embedding -> n_layer forecast-routed blocks -> final RMSNorm ->
    tied output projection. Parameter names and count are the reference's, so
    its state dicts load unchanged."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.embeddings = TiedEmbedding(config.vocab_size, config.n_embd, config.initializer_range)
        self.rotary_emb = RotaryEmbedding(head_dim=config.head_dim, max_seq_len=config.context_length,
                                          theta=config.rope_theta)
        self.layers = nn.ModuleList([TransformerBlock(config, layer_idx=i) for i in range(config.n_layer)])
        self.final_norm = RMSNorm(config.n_embd, eps=config.norm_eps)
        self._draw_projection_weights()
        self._head_key = None
        self._head_w: Optional[torch.Tensor] = None

    @torch.no_grad()
    def _draw_projection_weights(self) -> None:
        """Every projection of the model is a bias-free ``nn.Linear``; each
        weight is drawn from N(0, initializer_range^2), in module order. The
        tied embedding draws its own table when it is built and the norm
        weights start at one."""
        std = self.config.initializer_range
        for proj in self.modules():
            if isinstance(proj, nn.Linear):
                proj.weight.normal_(0.0, std)

    def count_parameters(self) -> Dict[str, int]:
        """Parameter counts: the whole model, the trainable part, the shared
        embedding table, and everything else."""
        sizes = [(p.numel(), p.requires_grad) for p in self.parameters()]
        total = sum(n for n, _ in sizes)
        table = self.embeddings.weight.numel()
        return {"total": total, "trainable": sum(n for n, g in sizes if g),
                "embeddings": table, "layers": total - table}

    def _folded_head(self) -> torch.Tensor:
        """The tied output weight with the final RMSNorm weight folded into its
        columns, rebuilt when either changed."""
        ws = (self.embeddings.weight, self.final_norm.weight)
        key = tuple((t.data_ptr(), t._version) for t in ws)
        if key != self._head_key:
            with torch.no_grad():
                self._head_w = (ws[0].float() * ws[1].float()[None, :]).to(torch.bfloat16).contiguous()
            self._head_key = key
        return self._head_w

    def logits(self, x: torch.Tensor) -> torch.Tensor:
        """final_norm + tied output projection (model/model.py:79-157); one
        kernel for decode-sized bf16 batches under ``fused_ffn``."""
        C = x.shape[-1]
        if (getattr(self.config, "fused_ffn", False) and x.is_cuda and x.dtype == torch.bfloat16
                and not torch.is_grad_enabled() and x.shape[0] * x.shape[1] <= 16 and C % 128 == 0
                and C <= 1024 and self.config.vocab_size % 16 == 0):
            return sparda.norm_gemv(x, self._folded_head(), self.final_norm.eps)
        return self.embeddings.project(self.final_norm(x))

    def forward(self, input_ids: torch.Tensor, targets: Optional[torch.Tensor] = None,
                kv_caches: Optional[List] = None, return_forecasts: bool = False) -> Dict[str, torch.Tensor]:
        """input_ids [B,T] -> {"logits" [B,T,V], "loss"?, "forecasts"?} (model/model.py:79-157).

        Block i receives the forecast block i-1 emitted (None for block 0),
        its own cache, and block i+1 with that block's cache so it can issue
        the next layer's prefetch before its own attention."""
        n = len(self.layers)
        caches: List = list(kv_caches) if kv_caches is not None else []
        caches += [None] * (n + 1 - len(caches))
        followers = list(self.layers)[1:] + [None]
        h = self.embeddings.embed(input_ids)
        emitted: List[torch.Tensor] = []
        forecast: Optional[torch.Tensor] = None
        for block, follower, cache, follower_cache in zip(self.layers, followers, caches, caches[1:]):
            h, forecast_out = block(x=h, rotary_emb=self.rotary_emb, kv_cache=cache, mask=None, is_causal=True,
                                    prev_layer_forecast=forecast, next_layer_block=follower,
                                    next_kv_cache=follower_cache if follower is not None else None)
            forecast = forecast_out
            emitted.append(forecast_out)
        result: Dict[str, torch.Tensor] = {"logits": self.logits(h)}
        if return_forecasts:
            result["forecasts"] = emitted
        if targets is not None:
            vocab = self.config.vocab_size
            result["loss"] = F.cross_entropy(result["logits"].reshape(-1, vocab), targets.reshape(-1),
                                             ignore_index=-100)
        return result

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 50, temperature: float = 0.8,
                 top_k: int = 50, eos_token_id: Optional[int] = None,
                 kv_caches: Optional[List] = None) -> torch.Tensor:
        """Sampling loop (model/model.py:159-195). With ``kv_caches`` (one per
        layer, empty) the prompt is prefilled once and each new token runs one
        cached decode step; without, every step re-runs the full forward as
        the reference does."""
        self.eval()
        if kv_caches is not None:
            logits = self.forward(input_ids, kv_caches=kv_caches)["logits"][:, -1, :]
        for step in range(max_new_tokens):
            if kv_caches is None:
                ctx = input_ids if input_ids.shape[1] <= self.config.context_length else \
                    input_ids[:, -self.config.context_length:]
                logits = self.forward(ctx)["logits"][:, -1, :]
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
            if kv_caches is not None and step + 1 < max_new_tokens:
                logits = self.forward(nxt, kv_caches=kv_caches)["logits"][:, -1, :]
        return input_ids
