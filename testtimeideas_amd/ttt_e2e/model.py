"""The reference TTT model (cloud_ttt_e2e/ttt_e2e/model.py) with its attention
on the HIP kernels: the caller of the attention in the meta-learning step.

Same configuration fields, module tree and parameter names as the reference
(model.py:9-143), so state dicts and ``torch.func.functional_call``
parameter dicts carry over: token + position embeddings, ``prefix_blocks``
(pre-LN attention + GELU MLP), ``suffix_blocks`` (the same with a fast MLP and
an optional slow one whose outputs add), a final LayerNorm and an untied head.
``forward(input_ids, mode=...)`` runs the prefix, the suffix from given
hidden states, or both.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch
from torch import nn

from .attention import WindowedSelfAttention


@dataclasses.dataclass
class ModelConfig:
    vocab_size: int = 4096
    max_seq_len: int = 8192
    window_size: Optional[int] = 512
    d_model: int = 512
    n_heads: int = 8
    n_layers: int = 8
    d_ff: int = 2048
    dropout: float = 0.0
    use_gradgrad_attention: bool = True
    suffix_layers: int = -1  # layers updated by the inner loop (-1: all)
    dual_mlp: bool = True    # suffix blocks add a slow MLP to the fast one


def _mlp(cfg: ModelConfig) -> nn.Sequential:
    return nn.Sequential(nn.Linear(cfg.d_model, cfg.d_ff), nn.GELU(), nn.Linear(cfg.d_ff, cfg.d_model))


def _attention(cfg: ModelConfig) -> WindowedSelfAttention:
    return WindowedSelfAttention(cfg.d_model, cfg.n_heads, cfg.window_size, use_gradgrad=cfg.use_gradgrad_attention)


class PrefixBlock(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.ln1 = nn.LayerNorm(cfg.d_model)
        self.attn = _attention(cfg)
        self.ln2 = nn.LayerNorm(cfg.d_model)
        self.mlp = _mlp(cfg)
        self.dropout = nn.Dropout(cfg.dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.dropout(self.attn(self.ln1(x)))
        return x + self.dropout(self.mlp(self.ln2(x)))


class SuffixBlock(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.ln1 = nn.LayerNorm(cfg.d_model)
        self.attn = _attention(cfg)
        self.ln2 = nn.LayerNorm(cfg.d_model)
        self.mlp_fast = _mlp(cfg)
        self.mlp_slow = _mlp(cfg) if cfg.dual_mlp else None
        self.dropout = nn.Dropout(cfg.dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.dropout(self.attn(self.ln1(x)))
        h = self.ln2(x)
        y = self.mlp_fast(h)
        if self.mlp_slow is not None:
            y = y + self.mlp_slow(h)
        return x + self.dropout(y)


class TTTModel(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.pos = nn.Embedding(cfg.max_seq_len, cfg.d_model)
        n_suffix = cfg.suffix_layers if 0 <= cfg.suffix_layers <= cfg.n_layers else cfg.n_layers
        self.suffix_layers = n_suffix
        self.prefix_layers = cfg.n_layers - n_suffix
        self.prefix_blocks = nn.ModuleList(PrefixBlock(cfg) for _ in range(self.prefix_layers))
        self.suffix_blocks = nn.ModuleList(SuffixBlock(cfg) for _ in range(n_suffix))
        self.ln_f = nn.LayerNorm(cfg.d_model)
        self.head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)

    def prefix_forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        t = input_ids.size(1)
        x = self.embed(input_ids) + self.pos(torch.arange(t, device=input_ids.device)).unsqueeze(0)
        for block in self.prefix_blocks:
            x = block(x)
        return x

    def suffix_forward(self, hidden: torch.Tensor) -> torch.Tensor:
        x = hidden
        for block in self.suffix_blocks:
            x = block(x)
        return self.head(self.ln_f(x))

    def forward(self, input_ids: Optional[torch.Tensor] = None, *, mode: str = "full",
                prefix_hidden: Optional[torch.Tensor] = None) -> torch.Tensor:
        if mode == "prefix":
            if input_ids is None:
                raise ValueError("input_ids required for prefix mode")
            return self.prefix_forward(input_ids)
        if mode == "suffix":
            if prefix_hidden is None:
                raise ValueError("prefix_hidden required for suffix mode")
            return self.suffix_forward(prefix_hidden)
        if input_ids is None:
            raise ValueError("input_ids required for full mode")
        return self.suffix_forward(self.prefix_forward(input_ids))
