"""Synthetic key-value retrieval batches of the reference TTT model
(cloud_ttt_e2e/ttt_e2e/data.py:1-134): the data format on the far side of
the meta step.  Bench and test harness, not part of the library package.

A sequence is BOS, then `context_len // 5` pairs ``KEY k VAL v SEP`` with
distinct keys, then `query_len // 5` queries ``QRY k VAL v SEP`` that repeat
pairs of the context (drawn from its first `far_frac` share when far_frac >
0), padded with PAD.  input_ids/targets are the sequence shifted by one; the
inner mask marks the targets inside the context, the outer mask the value
tokens of the queries.
"""
from __future__ import annotations

import dataclasses
from typing import Optional

import torch

PAD, BOS, SEP, KEY, VAL, QRY = 0, 1, 2, 3, 4, 5


@dataclasses.dataclass
class KVBatch:
    input_ids: torch.Tensor
    targets: torch.Tensor
    inner_mask: torch.Tensor
    outer_mask: torch.Tensor


def generate_kv_batch(batch_size: int, context_len: int, query_len: int, vocab_size: int, num_keys: int = 256,
                      device="cuda", pad_to: Optional[int] = None, pad_multiple: Optional[int] = None,
                      far_frac: float = 0.0, generator: Optional[torch.Generator] = None) -> KVBatch:
    n_pairs = max(1, context_len // 5)
    n_queries = max(1, query_len // 5)
    key_lo = 6
    key_hi = min(key_lo + num_keys, vocab_size // 2)
    val_lo = key_hi
    val_hi = min(val_lo + num_keys, vocab_size - 1)
    seq_len = 1 + 5 * n_pairs + 5 * n_queries  # tokens incl. BOS; input_ids are one shorter
    if pad_to is not None:
        seq_len = max(seq_len, pad_to + 1)
    if pad_multiple is not None and (seq_len - 1) % pad_multiple:
        seq_len = ((seq_len - 1) // pad_multiple + 1) * pad_multiple + 1
    far = min(max(float(far_frac), 0.0), 1.0)

    seqs = torch.full((batch_size, seq_len), PAD, dtype=torch.long)
    inner = torch.zeros((batch_size, seq_len - 1), dtype=torch.float32)
    outer = torch.zeros((batch_size, seq_len - 1), dtype=torch.float32)
    for b in range(batch_size):
        keys = (torch.randperm(key_hi - key_lo, generator=generator) + key_lo)[:n_pairs]
        n = keys.numel()
        vals = torch.randint(val_lo, val_hi, (n,), generator=generator)
        span = max(1, int(n * far)) if far > 0.0 else n
        pick = torch.randint(0, span, (n_queries,), generator=generator)
        ctx = torch.stack([torch.full_like(keys, KEY), keys, torch.full_like(keys, VAL), vals,
                           torch.full_like(keys, SEP)], dim=1).reshape(-1)
        qk, qv = keys[pick], vals[pick]
        qry = torch.stack([torch.full_like(qk, QRY), qk, torch.full_like(qk, VAL), qv,
                           torch.full_like(qk, SEP)], dim=1).reshape(-1)
        row = torch.cat([torch.tensor([BOS]), ctx, qry])[:seq_len]
        seqs[b, :row.numel()] = row
        # targets index i-1 predicts sequence position i
        c_end = min(1 + ctx.numel(), seq_len)
        inner[b, 0:c_end - 1] = 1.0
        vpos = 1 + ctx.numel() + 5 * torch.arange(n_queries) + 3  # value token of each query
        vpos = vpos[vpos - 1 < seq_len - 1]
        outer[b, vpos - 1] = 1.0
    input_ids = seqs[:, :-1].contiguous().to(device)
    targets = seqs[:, 1:].contiguous().to(device)
    return KVBatch(input_ids, targets, inner.to(device), outer.to(device))
