"""Causal language model with RACE blocks, the reference API of misc/lm.py.

Drop-in replacement for LMModel (misc/lm.py:37-74) with attn_type "race":
token and position embeddings, cfg["n_layers"] causal RACEBlocks
(race_attention_amd.race.RACEBlock, misc/race.py:176-206), final LayerNorm
and the vocabulary head.  cfg keys as the reference's GPT_CONFIG_124M:
vocab_size, context_length, emb_dim, n_heads, n_layers, drop_rate, qkv_bias,
K, L, M.
"""
from __future__ import annotations

import torch
from torch import nn

from .race import RACEBlock


class LMModel(nn.Module):
    def __init__(self, cfg, attn_type="race", device="cpu"):
        super().__init__()
        if attn_type != "race":
            raise ValueError("this build implements the RACE blocks only (attn_type='race')")
        self.tok_emb = nn.Embedding(cfg["vocab_size"], cfg["emb_dim"])
        self.pos_emb = nn.Embedding(cfg["context_length"], cfg["emb_dim"])
        self.drop_emb = nn.Dropout(cfg["drop_rate"])
        self.final_norm = nn.LayerNorm(cfg["emb_dim"])
        self.out_head = nn.Linear(cfg["emb_dim"], cfg["vocab_size"], bias=False)
        self.blocks = nn.Sequential(*[RACEBlock(cfg, device) for _ in range(cfg["n_layers"])])

    def forward(self, x):
        B, T = x.shape
        pos = torch.arange(T, device=x.device).unsqueeze(0)
        x = self.drop_emb(self.tok_emb(x) + self.pos_emb(pos))
        x = self.blocks(x)
        return self.out_head(self.final_norm(x))
