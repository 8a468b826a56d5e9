"""The reference TTT model as a caller of the HIP attention — bench and test
harness, not part of the library package.

What is kept from the reference (cloud_ttt_e2e/ttt_e2e/model.py:9-143) is
its interface: the ``ModelConfig`` fields (the keys of its YAML configs), the
parameter names that state dicts and ``torch.func.functional_call``
parameter dicts use (``embed``, ``pos``, ``prefix_blocks.<i>.{ln1, attn.*,
ln2, mlp.{0,2}}``, ``suffix_blocks.<i>.{..., mlp_fast.{0,2},
mlp_slow.{0,2}}``, ``ln_f``, ``head``), and ``forward(input_ids, mode=...,
prefix_hidden=...)`` with modes "prefix", "suffix" and "full".

Computation: token plus learned position embeddings; pre-LayerNorm blocks of
windowed self-attention (``WindowedSelfAttention`` on the HIP kernels) and a
GELU feed-forward; the blocks the inner loop adapts (the last
``suffix_layers``) sum a fast and, optionally, a slow feed-forward; a final
LayerNorm and an untied output projection.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch
from torch import nn

from testtimeideas_amd.ttt_e2e.attention import WindowedSelfAttention


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
    suffix_layers: int = -1  # adapted blocks at the end; out of range (e.g. -1): every block
    dual_mlp: bool = True    # adapted blocks add a slow feed-forward to the fast one


class FeedForward(nn.Sequential):
    """d_model -> d_ff -> d_model with a GELU between (parameters ``0.*`` and ``2.*``)."""

    def __init__(self, d_model: int, d_ff: int):
        super().__init__(nn.Linear(d_model, d_ff), nn.GELU(), nn.Linear(d_ff, d_model))


class Block(nn.Module):
    """Pre-LayerNorm block: x + attn(ln1 x), then x + sum of the feed-forwards
    of ln2 x.  A prefix block has one feed-forward, ``mlp``; an adapted
    (suffix) block has ``mlp_fast`` and, with dual_mlp, ``mlp_slow``."""

    def __init__(self, cfg: ModelConfig, adapted: bool):
        super().__init__()
        self.ln1 = nn.LayerNorm(cfg.d_model)
        self.attn = WindowedSelfAttention(cfg.d_model, cfg.n_heads, cfg.window_size,
                                          use_gradgrad=cfg.use_gradgrad_attention)
        self.ln2 = nn.LayerNorm(cfg.d_model)
        if adapted:
            self.ff_names = ("mlp_fast", "mlp_slow") if cfg.dual_mlp else ("mlp_fast",)
        else:
            self.ff_names = ("mlp",)
        for name in self.ff_names:
            self.add_module(name, FeedForward(cfg.d_model, cfg.d_ff))
        self.dropout = nn.Dropout(cfg.dropout)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = x + self.dropout(self.attn(self.ln1(x)))
        h = self.ln2(x)
        ff = [getattr(self, name)(h) for name in self.ff_names]
        y = ff[0] if len(ff) == 1 else ff[0] + ff[1]
        return x + self.dropout(y)


class TTTModel(nn.Module):
    def __init__(self, cfg: ModelConfig):
        super().__init__()
        self.cfg = cfg
        self.embed = nn.Embedding(cfg.vocab_size, cfg.d_model)
        self.pos = nn.Embedding(cfg.max_seq_len, cfg.d_model)
        n_adapted = cfg.suffix_layers if 0 <= cfg.suffix_layers <= cfg.n_layers else cfg.n_layers
        self.suffix_layers = n_adapted
        self.prefix_layers = cfg.n_layers - n_adapted
        self.prefix_blocks = nn.ModuleList([Block(cfg, adapted=False) for _ in range(self.prefix_layers)])
        self.suffix_blocks = nn.ModuleList([Block(cfg, adapted=True) for _ in range(n_adapted)])
        self.ln_f = nn.LayerNorm(cfg.d_model)
        self.head = nn.Linear(cfg.d_model, cfg.vocab_size, bias=False)

    def prefix_forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Hidden states after the prefix blocks, [B, T, d_model]."""
        x = self.embed(input_ids) + self.pos.weight[: input_ids.size(1)]
        for block in self.prefix_blocks:
            x = block(x)
        return x

    def suffix_forward(self, hidden: torch.Tensor) -> torch.Tensor:
        """Logits, [B, T, vocab], from hidden states after the prefix."""
        for block in self.suffix_blocks:
            hidden = block(hidden)
        return self.head(self.ln_f(hidden))

    def forward(self, input_ids: Optional[torch.Tensor] = None, *, mode: str = "full",
                prefix_hidden: Optional[torch.Tensor] = None) -> torch.Tensor:
        """mode "prefix": hidden states of input_ids; "suffix": logits from
        prefix_hidden; anything else ("full"): logits of input_ids."""
        if mode == "suffix":
            if prefix_hidden is None:
                raise ValueError("mode='suffix' starts from prefix_hidden, which was not given")
            return self.suffix_forward(prefix_hidden)
        if input_ids is None:
            raise ValueError(f"mode={mode!r} starts from input_ids, which were not given")
        hidden = self.prefix_forward(input_ids)
        return hidden if mode == "prefix" else self.suffix_forward(hidden)
