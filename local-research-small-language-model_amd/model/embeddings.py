"""Tied token embedding / LM head (model/embeddings.py:8-33)."""

import torch
import torch.nn as nn
import torch.nn.functional as F


class TiedEmbedding(nn.Module):
    def __init__(self, vocab_size: int, n_embd: int, initializer_range: float = 0.02):
        super().__init__()
        self.vocab_size = vocab_size
        self.n_embd = n_embd
        self.weight = nn.Parameter(torch.empty(vocab_size, n_embd))
        nn.init.normal_(self.weight, mean=0.0, std=initializer_range)

    def embed(self, input_ids: torch.Tensor) -> torch.Tensor:
        return F.embedding(input_ids, self.weight)

    def project(self, hidden_states: torch.Tensor) -> torch.Tensor:
        return F.linear(hidden_states, self.weight)

    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        return self.embed(input_ids)
