"""Test-time-training meta step of the reference TTT model, the product-level
caller of the grad-grad attention — bench and test harness, not part of the
library package.

Semantics (reference cloud_ttt_e2e/ttt_e2e/meta.py:140-222, utils.py:24-37):
  * the prefix hidden states are computed once from the current parameters;
  * the inner loop walks the sequence in chunks of ``chunk_size`` positions
    (the whole sequence when None) and, per chunk, takes ``inner_steps`` SGD
    steps of size ``inner_lr`` on the masked next-token loss of the suffix,
    for the parameters whose names contain one of the ``param_filter``
    substrings (every parameter when none matches or there is no filter);
    with ``create_graph`` the updates stay differentiable;
  * the inner loss is the mean over chunks of the loss each chunk's last step
    saw; the outer loss is the suffix loss under the adapted parameters,
    averaged over the outer-mask tokens of all chunks (chunks without any are
    not run).
``outer_loss.backward()`` then differentiates through every inner update,
which runs the attention's double backward.

The parameters travel as a name -> tensor dict through
``torch.func.functional_call``, so the adapted values never overwrite the
module's own parameters.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Sequence, Tuple

import torch
from torch.func import functional_call

Params = Dict[str, torch.Tensor]


def token_loss(logits: torch.Tensor, targets: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Cross entropy of [B, T, V] logits against [B, T] targets: the mean over
    the positions where mask is nonzero (over all positions without a mask;
    0 when the mask is empty)."""
    ce = torch.nn.functional.cross_entropy(logits.flatten(0, -2), targets.flatten(), reduction="none")
    if mask is None:
        return ce.mean()
    w = mask.flatten().to(ce.dtype)
    return (ce * w).sum() / w.sum().clamp_min(1.0)


def adapted_names(model: torch.nn.Module, param_filter=None) -> List[str]:
    """Names of the parameters the inner loop updates.  param_filter: None,
    a comma-separated string or a sequence of substrings."""
    names = [n for n, _ in model.named_parameters()]
    if param_filter is None:
        subs: Sequence[str] = ()
    elif isinstance(param_filter, str):
        subs = param_filter.split(",")
    elif isinstance(param_filter, (list, tuple)):
        subs = [str(s) for s in param_filter]
    else:
        subs = [str(param_filter)]
    subs = [s.strip() for s in subs if s.strip()]
    picked = [n for n in names if any(s in n for s in subs)]
    return picked or names


def _spans(t: int, chunk_size: Optional[int]) -> List[Tuple[int, int]]:
    if chunk_size is None:
        return [(0, t)]
    if t % chunk_size:
        raise ValueError(f"chunk_size {chunk_size} does not divide the sequence length {t}")
    return [(s, s + chunk_size) for s in range(0, t, chunk_size)]


def _suffix_logits(model, params: Params, hidden: torch.Tensor) -> torch.Tensor:
    return functional_call(model, params, (None,), {"mode": "suffix", "prefix_hidden": hidden})


def inner_update(model, params: Params, trainable: List[str], targets, mask, lr: float, create_graph: bool, *,
                 prefix_hidden=None, input_ids=None) -> Tuple[Params, torch.Tensor]:
    """One SGD step of the trainable parameters on the suffix loss of
    prefix_hidden (or the full model's loss of input_ids); returns the new
    parameter dict and the loss before the step."""
    if prefix_hidden is not None:
        logits = _suffix_logits(model, params, prefix_hidden)
    elif input_ids is not None:
        logits = functional_call(model, params, (input_ids,), {"mode": "full"})
    else:
        raise ValueError("inner_update needs prefix_hidden or input_ids")
    loss = token_loss(logits, targets, mask)
    grads = torch.autograd.grad(loss, [params[n] for n in trainable], create_graph=create_graph,
                                retain_graph=create_graph)
    stepped = dict(params)
    stepped.update({n: params[n] - lr * g for n, g in zip(trainable, grads)})
    return stepped, loss


def adapt(model, params: Params, trainable: List[str], hidden, targets, inner_mask, *, inner_lr: float,
          inner_steps: int, chunk_size: Optional[int], create_graph: bool) -> Tuple[Params, torch.Tensor]:
    """The inner loop over the chunks in order: (adapted parameters, inner loss)."""
    seen = []
    for s0, s1 in _spans(hidden.size(1), chunk_size):
        loss = None
        for _ in range(inner_steps):
            params, loss = inner_update(model, params, trainable, targets[:, s0:s1], inner_mask[:, s0:s1], inner_lr,
                                        create_graph, prefix_hidden=hidden[:, s0:s1])
        if loss is not None:
            seen.append(loss)
    inner = torch.stack(seen).mean() if seen else hidden.new_zeros(())
    return params, inner


def outer_loss(model, params: Params, hidden, targets, outer_mask, *, chunk_size: Optional[int]) -> torch.Tensor:
    """The suffix loss under `params`, averaged over every chunk's outer-mask
    tokens; chunks without any are skipped (their counts are read back in
    one transfer)."""
    spans = _spans(hidden.size(1), chunk_size)
    counts = torch.stack([outer_mask[:, s0:s1].sum() for s0, s1 in spans]).tolist()
    total = hidden.new_zeros(())
    n_all = 0.0
    for (s0, s1), n in zip(spans, counts):
        if n <= 0:
            continue
        logits = _suffix_logits(model, params, hidden[:, s0:s1])
        total = total + token_loss(logits, targets[:, s0:s1], outer_mask[:, s0:s1]) * n
        n_all += n
    return total / max(n_all, 1.0)


def meta_step(model, input_ids, targets, inner_mask, outer_mask, inner_lr: float, inner_steps: int,
              param_filter=None, chunk_size: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(inner_loss, outer_loss) of one meta-learning step; the caller
    backpropagates outer_loss."""
    params = dict(model.named_parameters())
    trainable = adapted_names(model, param_filter)
    hidden = functional_call(model, params, (input_ids,), {"mode": "prefix"})
    params, inner = adapt(model, params, trainable, hidden, targets, inner_mask, inner_lr=inner_lr,
                          inner_steps=inner_steps, chunk_size=chunk_size, create_graph=True)
    return inner, outer_loss(model, params, hidden, targets, outer_mask, chunk_size=chunk_size)


def ttt_apply(model, input_ids, targets, inner_mask, inner_lr: float, inner_steps: int, param_filter=None,
              chunk_size: Optional[int] = None) -> Params:
    """The parameters after test-time training on a sequence (no graph kept)."""
    params = dict(model.named_parameters())
    hidden = functional_call(model, params, (input_ids,), {"mode": "prefix"})
    params, _ = adapt(model, params, adapted_names(model, param_filter), hidden, targets, inner_mask,
                      inner_lr=inner_lr, inner_steps=inner_steps, chunk_size=chunk_size, create_graph=False)
    return params


def ttt_logits(model, params: Params, input_ids, *, chunk_size: Optional[int] = None) -> torch.Tensor:
    """Logits of input_ids under `params`, the suffix run chunk by chunk."""
    hidden = functional_call(model, params, (input_ids,), {"mode": "prefix"})
    return torch.cat([_suffix_logits(model, params, hidden[:, s0:s1])
                      for s0, s1 in _spans(hidden.size(1), chunk_size)], dim=1)
