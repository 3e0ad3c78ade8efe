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
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.embeddings = TiedEmbedding(config.vocab_size, config.n_embd, config.initializer_range)
        self.rotary_emb = RotaryEmbedding(head_dim=config.head_dim, max_seq_len=config.context_length,
                                          theta=config.rope_theta)
        self.layers = nn.ModuleList([TransformerBlock(config, layer_idx=i) for i in range(config.n_layer)])
        self.final_norm = RMSNorm(config.n_embd, eps=config.norm_eps)
        self.apply(self._init_weights)
        self._head_key = None
        self._head_w: Optional[torch.Tensor] = None

    def _init_weights(self, module: nn.Module):
        if isinstance(module, nn.Linear):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)
            if module.bias is not None:
                nn.init.zeros_(module.bias)
        elif isinstance(module, nn.Embedding):
            nn.init.normal_(module.weight, mean=0.0, std=self.config.initializer_range)

    def count_parameters(self) -> Dict[str, int]:
        total = sum(p.numel() for p in self.parameters())
        emb = self.embeddings.weight.numel()
        return {"total": total, "trainable": sum(p.numel() for p in self.parameters() if p.requires_grad),
                "embeddings": emb, "layers": total - emb}

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
        """input_ids [B,T] -> {"logits" [B,T,V], "loss"?, "forecasts"?} (model/model.py:79-157)."""
        x = self.embeddings.embed(input_ids)
        forecasts: List[torch.Tensor] = []
        prev_forecast: Optional[torch.Tensor] = None
        n = len(self.layers)
        for i, layer in enumerate(self.layers):
            kv_cache = kv_caches[i] if kv_caches is not None else None
            next_layer = self.layers[i + 1] if i + 1 < n else None
            next_cache = kv_caches[i + 1] if (kv_caches is not None and i + 1 < len(kv_caches)) else None
            x, current_forecast = layer(x=x, rotary_emb=self.rotary_emb, kv_cache=kv_cache, mask=None,
                                        is_causal=True, prev_layer_forecast=prev_forecast,
                                        next_layer_block=next_layer, next_kv_cache=next_cache)
            if return_forecasts:
                forecasts.append(current_forecast)
            prev_forecast = current_forecast
        logits = self.logits(x)
        out = {"logits": logits}
        if return_forecasts:
            out["forecasts"] = forecasts
        if targets is not None:
            out["loss"] = F.cross_entropy(logits.view(-1, self.config.vocab_size), targets.view(-1),
                                          ignore_index=-100)
        return out

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
