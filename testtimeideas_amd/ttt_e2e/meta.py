"""The meta-learning step of the reference TTT model
(cloud_ttt_e2e/ttt_e2e/meta.py), the product-level caller of the grad-grad
attention.

One ``meta_step``:
  1. prefix hidden states once, with the current parameters;
  2. an inner scan over sequence chunks: per chunk, `inner_steps` SGD steps
     on the masked next-token loss of the suffix, on the parameters whose
     names contain one of the filter substrings, each gradient taken with
     ``create_graph=True`` so that the updates stay differentiable;
  3. the outer loss of the suffix under the adapted parameters, chunk by
     chunk, weighted by each chunk's mask count.
The caller's ``outer_loss.backward()`` then differentiates through every
inner update, which is where the attention's double backward runs
(reference meta.py:44-177).
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch
from torch.func import functional_call


def compute_loss(logits: torch.Tensor, targets: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Token cross entropy, mean over the tokens where mask is 1 (all tokens
    without a mask).  Reference: cloud_ttt_e2e/ttt_e2e/utils.py:24-37."""
    loss = torch.nn.functional.cross_entropy(logits.reshape(-1, logits.size(-1)), targets.reshape(-1),
                                             reduction="none")
    if mask is None:
        return loss.mean()
    m = mask.reshape(-1).float()
    return (loss * m).sum() / m.sum().clamp_min(1.0)


def split_params(model: torch.nn.Module, param_filter=None) -> Tuple[Dict[str, torch.Tensor], List[str]]:
    """All named parameters, and the names the inner loop updates: those
    containing one of the filter substrings (a comma-separated string or a
    list); every name when there is no filter or nothing matches.
    Reference: meta.py:9-30."""
    params = dict(model.named_parameters())
    if param_filter is None:
        subs = []
    elif isinstance(param_filter, str):
        subs = [x.strip() for x in param_filter.split(",") if x.strip()]
    elif isinstance(param_filter, (list, tuple)):
        subs = [str(x).strip() for x in param_filter if str(x).strip()]
    else:
        subs = [str(param_filter)]
    chosen = [n for n in params if any(s in n for s in subs)] if subs else []
    return params, chosen or list(params)


def chunks(x: torch.Tensor, chunk_size: Optional[int]) -> List[torch.Tensor]:
    """Split the sequence dimension (dim 1) into equal chunks; the whole
    tensor when chunk_size is None.  Reference: meta.py:33-41."""
    if chunk_size is None or x.dim() < 2:
        return [x]
    if x.size(1) % chunk_size:
        raise ValueError(f"seq len {x.size(1)} not divisible by chunk_size {chunk_size}")
    return list(x.split(chunk_size, dim=1))


def inner_update(model, params, trainable, targets, mask, lr: float, create_graph: bool, *,
                 prefix_hidden=None, input_ids=None):
    """One SGD step on the trainable parameters; returns (new params, loss).
    Reference: meta.py:44-73."""
    if prefix_hidden is not None:
        logits = functional_call(model, params, (None,), {"mode": "suffix", "prefix_hidden": prefix_hidden})
    elif input_ids is not None:
        logits = functional_call(model, params, (input_ids,), {"mode": "full"})
    else:
        raise ValueError("input_ids required when prefix_hidden is None")
    loss = compute_loss(logits, targets, mask)
    grads = torch.autograd.grad(loss, [params[n] for n in trainable], create_graph=create_graph,
                                retain_graph=create_graph)
    new = dict(params)
    for n, g in zip(trainable, grads):
        new[n] = new[n] - lr * g
    return new, loss


def inner_scan(model, params, trainable, prefix_hidden, targets, inner_mask, *, inner_lr: float, inner_steps: int,
               chunk_size: Optional[int], create_graph: bool):
    """Inner steps over the chunks in order; returns (adapted params, mean of
    each chunk's last inner loss).  Reference: meta.py:76-109."""
    last = []
    for h, t, m in zip(chunks(prefix_hidden, chunk_size), chunks(targets, chunk_size), chunks(inner_mask, chunk_size)):
        for _ in range(inner_steps):
            params, loss = inner_update(model, params, trainable, t, m, inner_lr, create_graph, prefix_hidden=h)
        last.append(loss)
    inner = torch.stack(last).mean() if last else torch.zeros((), device=targets.device)
    return params, inner


def outer_loss(model, params, prefix_hidden, targets, outer_mask, *, chunk_size: Optional[int]) -> torch.Tensor:
    """Mask-weighted mean of the chunks' outer losses; chunks without masked
    tokens are skipped.  Reference: meta.py:112-137."""
    total = torch.zeros((), device=targets.device)
    count = torch.zeros((), device=targets.device)
    for h, t, m in zip(chunks(prefix_hidden, chunk_size), chunks(targets, chunk_size), chunks(outer_mask, chunk_size)):
        n = m.sum()
        if n.item() <= 0:
            continue
        logits = functional_call(model, params, (None,), {"mode": "suffix", "prefix_hidden": h})
        total = total + compute_loss(logits, t, m) * n
        count = count + n
    return total / count.clamp_min(1.0)


def meta_step(model, input_ids, targets, inner_mask, outer_mask, inner_lr: float, inner_steps: int,
              param_filter=None, chunk_size: Optional[int] = None):
    """(inner_loss, outer_loss) of one meta-learning step; the caller
    backpropagates outer_loss.  Reference: meta.py:140-177."""
    params, trainable = split_params(model, param_filter)
    prefix_hidden = functional_call(model, params, (input_ids,), {"mode": "prefix"})
    params, inner = inner_scan(model, params, trainable, prefix_hidden, targets, inner_mask, inner_lr=inner_lr,
                               inner_steps=inner_steps, chunk_size=chunk_size, create_graph=True)
    return inner, outer_loss(model, params, prefix_hidden, targets, outer_mask, chunk_size=chunk_size)
