"""Consumers of per-token negative log-likelihoods.

Reference README.md:110-122: ``linear_cross_entropy(..., reduction="none")``
returns per-token NLLs "useful for" perplexity (``ppl = exp(mean(nll))``) and a
DPO-style preference loss (``-log(sigmoid(nll_rejected.sum() - nll_preferred.sum()))``).

Guarantees of this module:

* ``token_nll`` is float32 and shaped like ``targets`` whatever the dtype of the
  hidden states and classifier rows (bf16 / fp16 / fp32); ignored positions hold 0.
* The consumers compute in float32 (or wider, if their input already is) and stay
  differentiable: their gradients reach ``e``, ``c`` and ``bias`` through the CCE
  backward as an arbitrary per-token upstream gradient.
* The DPO loss uses ``softplus`` instead of ``log(sigmoid(.))``, so large
  log-likelihood gaps neither overflow nor return ``-inf``.
"""

import torch
import torch.nn.functional as F

from . import FILTER_LOG_EPS, linear_cross_entropy

__all__ = ["token_nll", "sequence_nll", "perplexity", "dpo_loss"]


def _as_f32(nll):
    return nll if nll.dtype in (torch.float32, torch.float64) else nll.to(torch.float32)


def token_nll(e, c, targets, bias=None, ignore_index=-100, *, shift=0, filter_eps=FILTER_LOG_EPS):
    """Per-token NLL [...] (fp32, same shape as ``targets`` after ``shift``); ignored positions are 0."""
    nll = linear_cross_entropy(e, c, targets, bias, reduction="none", ignore_index=ignore_index, shift=shift,
                               filter_eps=filter_eps)
    return nll.to(torch.float32)


def sequence_nll(nll, mask=None):
    """Sum of the per-token NLL over the last dimension (one value per sequence).

    ``mask`` (bool or 0/1, broadcastable to ``nll``) selects the tokens that count;
    ignored positions already hold 0, so it is only needed to drop further tokens.
    """
    x = _as_f32(nll)
    if mask is not None:
        x = x * mask.to(x.dtype)
    return x.sum(dim=-1)


def perplexity(nll, mask=None):
    """exp(mean NLL) (README.md:117-118: ``ppl = exp(mean(nll))``).

    Without ``mask`` the mean runs over every entry, as in the README; with
    ``mask`` (e.g. ``targets != ignore_index``) it runs over the selected tokens
    only, dividing by max(count, 1).
    """
    x = _as_f32(nll)
    if mask is None:
        return torch.exp(x.mean())
    m = mask.to(x.dtype)
    return torch.exp((x * m).sum() / m.sum().clamp(min=1.0))


def dpo_loss(nll_preferred, nll_rejected, beta=1.0, reduction="mean"):
    """DPO-style preference loss from per-token NLLs (README.md:120-121).

    Each argument is [..., T] (one row of per-token NLLs per sequence) or [T];
    the per-sequence log-likelihood gap is ``sum(nll_rejected) - sum(nll_preferred)``
    over the last dimension, and the loss per pair is
    ``-log(sigmoid(beta * gap)) = softplus(-beta * gap)``.  For a single pair of
    1-D inputs and beta = 1 this is exactly the README's expression.
    reduction: "mean" | "sum" | "none" over the pairs.
    """
    if reduction not in ("mean", "sum", "none"):
        raise ValueError(f"Unknown reduction: {reduction!r}")
    gap = sequence_nll(nll_rejected) - sequence_nll(nll_preferred)
    loss = F.softplus(-beta * gap)
    if reduction == "mean":
        return loss.mean()
    if reduction == "sum":
        return loss.sum()
    return loss
