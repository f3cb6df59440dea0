"""Materialised-logits cross-entropy: the reference's own comparison path.

``linear_cross_entropy_reference`` restates reference/_reference.py:5-48 (exported by
reference/__init__.py:122-126 and selected with ``linear_cross_entropy(...,
impl="reference")``, reference/__init__.py:58-67) in plain PyTorch, on whatever device
the tensors are on.  It allocates the [N, V] logits and differentiates through
torch's own log-softmax: the memory CCE exists to avoid.  It is a separate path the
caller asks for by name, for side-by-side comparisons like the reference's
benchmarks/bench_synthetic.py:100-190; the CCE path never calls it.

Differences from the MLX original, on purpose: the log-softmax runs in float32 (float64
for float64 inputs; MLX takes it in the logits' dtype), ignored targets are gathered at
index 0 before the mask (MLX's take_along_axis on a negative index is not defined for
torch.gather), and the loss is float32 (float64 for float64 inputs) like the CCE
path's.
"""

import torch

__all__ = ["linear_cross_entropy_reference"]


def linear_cross_entropy_reference(e, c, targets, bias=None, reduction="mean", ignore_index=-100, shift=0,
                                   return_lse=False):
    """Reference reference/_reference.py:5-48: logits = e @ c.T (+ bias), cross-entropy
    per token, ``ignore_index`` rows masked to 0, then ``none`` (shaped like targets),
    ``sum``, or ``mean`` over the kept rows (divided by max(count, 1))."""
    if reduction not in ("none", "sum", "mean"):
        raise ValueError(f"Unknown reduction: {reduction!r}")
    if shift > 0:
        e = e[..., :-shift, :]
        targets = targets[..., shift:]
    orig_shape = targets.shape
    e2 = e.reshape(-1, e.shape[-1])
    t = targets.reshape(-1).to(torch.int64)
    logits = e2 @ c.T
    if bias is not None:
        logits = logits + bias[None, :]
    if logits.dtype != torch.float64:
        logits = logits.float()
    lse = torch.logsumexp(logits, dim=-1)
    valid = torch.ones_like(t, dtype=torch.bool) if ignore_index is None else t != ignore_index
    safe = torch.where(valid, t, torch.zeros_like(t))
    per_token = (lse - logits.gather(1, safe[:, None])[:, 0]) * valid
    if reduction == "none":
        loss = per_token.reshape(orig_shape)
    elif reduction == "sum":
        loss = per_token.sum()
    else:
        loss = per_token.sum() / valid.sum().clamp(min=1)
    if return_lse:
        return loss, lse.detach()
    return loss
