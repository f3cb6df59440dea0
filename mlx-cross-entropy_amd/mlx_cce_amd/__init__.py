"""mlx_cce_amd — Cut Cross-Entropy for AMD Instinct MI355X (gfx950), PyTorch-ROCm.

Drop-in for the reference package ``mlx_cce`` (sb1992/mlx-cross-entropy):

    from mlx_cce_amd import linear_cross_entropy
    loss = linear_cross_entropy(hidden_states, classifier_weight, targets)

loss = logsumexp(e @ c.T + bias) - (e @ c.T + bias)[target], computed by
hand-written HIP kernels (``libcce_mi355x.so``) without materialising the
[N, V] logits.  Gradients dE, dC and dBias are produced for every input that
requires grad; vocabulary tiles whose softmax is below 2^-12 for every row of a
128-row block are skipped in the backward (the reference's filter,
csrc/cce/cce.metal:191-204).

API mirrors (reference file:line):
    linear_cross_entropy   mlx_cce/__init__.py:79-107 (+ shift/return_lse/impl/compute_all_grads of
                           reference/__init__.py:22-85)
    linear_cross_entropy_reference  reference/_reference.py:5-48 (materialised logits, torch)
    cce_loss               mlx_cce/__init__.py:54-76
    cut_cross_entropy      csrc/bindings.cpp:15-56
    cce_forward_raw        csrc/bindings.cpp:58-69
    cce_backward_raw       csrc/bindings.cpp:71-86
    LinearCrossEntropy     reference/__init__.py:88-118

Quantized classifier rows (the reference's callers run mx.dequantize first,
README.md:84-95): pass a ``QuantizedWeight`` as ``c``; the library dequantizes a
bounded chunk of rows at a time (see ``quant.py``).
"""

__version__ = "0.1.0"

import torch

from . import _ext
from ._ext import FILTER_LOG_EPS, cce_backward_raw, cce_forward_raw
from .quant import QuantizedWeight, dequantize, quantize
from .reference import linear_cross_entropy_reference

__all__ = [
    "linear_cross_entropy",
    "cce_loss",
    "cut_cross_entropy",
    "cce_forward_raw",
    "cce_backward_raw",
    "LinearCrossEntropy",
    "linear_cross_entropy_reference",
    "FILTER_LOG_EPS",
    "last_tile_stats",
    "last_filter_stats",
    "QuantizedWeight",
    "quantize",
    "dequantize",
]

_REDUCTIONS = ("none", "sum", "mean")
_IMPLS = ("auto", "fused", "chunked", "reference")
_last_stats = {}


def last_tile_stats(device=None):
    """(kept, total) backward tiles of the most recent backward on `device` (synchronises)."""
    st = last_filter_stats(device)
    return None if st is None else (st["kept"], st["total"])


def last_filter_stats(device=None):
    """Tile-filter counts of the most recent backward on `device` (synchronises):
    kept / total 128x128 tiles, and kept_input_order, the tiles the filter keeps with
    token blocks taken in input order (equal to kept unless the backward grouped the
    rows by target tile)."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    t = _last_stats.get(dev)
    if t is None:
        return None
    kept, total, kept_in = (int(x) for x in t.tolist())
    return {"kept": kept, "total": total, "kept_input_order": kept_in, "sorted_rows": kept != kept_in}


class _CCEFunction(torch.autograd.Function):
    """Autograd glue: replaces the reference's mx.custom_function + vjp (mlx_cce/__init__.py:21-51)."""

    @staticmethod
    def forward(ctx, e, c, bias, targets, ignore_index, reduction, filter_eps, grad_c, grad_bias, zero_dc):
        # Quantized classifier rows (a QuantizedWeight, not a tensor): no gradient for them.
        ctx.qw = c if isinstance(c, QuantizedWeight) else None
        # zero_dc (opt-in, backward_options(dc_zero_fill="forward"), with grad mode on and
        # c requiring grad): the forward's tile kernel zeroes dC, so the backward writes
        # only the rows of vocabulary tiles it keeps.  Off by default: the fill's stores
        # delay the tile kernel's stage barriers more than the backward gains (at N = 4096,
        # D = 2304, V = 256000: forward +0.20 ms, backward -0.02 ms), and with the filter
        # off every row is written by the backward anyway.
        ctx.dc_zeroed = torch.empty_like(c) if (zero_dc and ctx.qw is None and c.is_contiguous()) else None
        if ctx.qw is not None:
            tile_max, _tse, _ntl, lse, nll = _ext.forward_q(e, c, targets, bias, ignore_index)
            c = None
        else:
            tile_max, _tse, _ntl, lse, nll = _ext.forward(e, c, targets, bias, ignore_index, zero_out=ctx.dc_zeroed)
        if reduction == "none":
            loss = nll
            scale = None
        else:  # sum, or mean over the kept rows divided by max(count, 1) (mlx_cce/__init__.py:73-75)
            loss, scale = _ext.reduce_loss(nll, targets, ignore_index, reduction)
        ctx.save_for_backward(e, c, bias, targets, lse, tile_max, scale)
        ctx.cce = (ignore_index, reduction, filter_eps, grad_c, grad_bias)
        ctx.mark_non_differentiable(lse)
        ctx.set_materialize_grads(False)  # no zero-filled cotangent for lse (it has no gradient)
        return loss, lse

    @staticmethod
    def backward(ctx, grad_loss, _grad_lse):
        e, c, bias, targets, lse, tile_max, scale = ctx.saved_tensors
        ignore_index, reduction, filter_eps, grad_c, grad_bias = ctx.cce
        if grad_loss is None:
            return None, None, None, None, None, None, None, None, None, None
        N = e.shape[0]
        if reduction == "none":
            d_nll = grad_loss.to(torch.float32).reshape(N)
        else:
            d_nll = _ext.broadcast_grad(grad_loss, scale, N)
        want_de = ctx.needs_input_grad[0]
        want_dc = ctx.needs_input_grad[1] and grad_c
        want_db = bias is not None and ctx.needs_input_grad[2] and grad_bias
        if not (want_de or want_dc or want_db):
            return None, None, None, None, None, None, None, None, None, None
        stats = torch.empty((3,), dtype=torch.int64, device=e.device)
        if ctx.qw is not None:
            dE, dB = _ext.backward_q(e, ctx.qw, targets, lse, tile_max, d_nll, bias, ignore_index, filter_eps,
                                     want_de, want_db, tile_stats=stats)
            _last_stats[e.device] = stats
            return dE, None, dB, None, None, None, None, None, None, None
        dc_zeroed, ctx.dc_zeroed = ctx.dc_zeroed, None  # used once (a second backward zeroes its own)
        dE, dC, dB = _ext.backward(e, c, targets, lse, tile_max, d_nll, bias, ignore_index, filter_eps,
                                   want_de, want_dc, want_db, tile_stats=stats, dc_zeroed=dc_zeroed)
        _last_stats[e.device] = stats
        return dE, dC, dB, None, None, None, None, None, None, None


def _cce(e, c, targets, bias, reduction, ignore_index, filter_eps, grad_c=True, grad_bias=True):
    if reduction not in _REDUCTIONS:
        raise ValueError(f"Unknown reduction: {reduction!r}")
    if bias is not None and bias.dtype != e.dtype:
        bias = bias.to(e.dtype)
    zero_dc = bool(_ext._bwd_opts["dc_zero_fill"] == "forward" and grad_c and torch.is_grad_enabled()
                   and isinstance(c, torch.Tensor) and c.requires_grad)
    loss, lse = _CCEFunction.apply(e, c, bias, targets, ignore_index, reduction, filter_eps, grad_c, grad_bias,
                                   zero_dc)
    return loss, lse


def cce_loss(e, c, targets, bias=None, reduction="mean", ignore_index=-100, *, filter_eps=FILTER_LOG_EPS):
    """Reference mlx_cce/__init__.py:54-76.  e [N, D], c [V, D], targets [N]; fp32 loss.

    ignore_index=None treats every row as valid.  filter_eps (keyword-only, not in
    the reference) sets the backward tile filter threshold; None disables it.
    """
    if e.dim() != 2:
        raise ValueError(f"[cut_cross_entropy] e must be 2D [B, D], got {e.dim()}D")
    loss, _ = _cce(e, c, targets, bias, reduction, ignore_index, filter_eps)
    return loss


def linear_cross_entropy(e, c, targets, bias=None, reduction="mean", ignore_index=-100, shift=0, return_lse=False,
                         impl="auto", compute_all_grads=None, *, filter_eps=FILTER_LOG_EPS):
    """Memory-efficient cross-entropy that never materializes [N, V] logits.

    Reference mlx_cce/__init__.py:79-107 (the installed API: e, c, targets, bias,
    reduction, ignore_index) and the research API reference/__init__.py:22-85, whose
    further arguments follow in the same order (shift, return_lse, impl,
    compute_all_grads; reference/_ops.py:209-211,238-239).

    Args:
        e: hidden states [..., D] (flattened to [N, D])
        c: classifier weights [V, D], or a QuantizedWeight
        targets: target indices [...] (flattened to [N])
        bias: optional classifier bias [V]
        reduction: "mean", "sum" or "none"
        ignore_index: target value to mask (-100 default); None disables masking
        shift: drop the last `shift` positions of e and the first `shift` targets (causal LM)
        return_lse: also return the per-token logsumexp [N] (fp32, no gradient)
        impl: "auto", "fused" or "chunked" run the HIP kernels (one path serves all
            shapes, so the reference's choice between them has nothing to pick);
            "reference" runs the materialised-logits restatement of
            reference/_reference.py (linear_cross_entropy_reference)
        compute_all_grads: True: gradients for c and bias as well as e; False: for e
            only (LoRA / frozen head: c and bias get no gradient, where the
            reference's VJP returns zeros, reference/_ops.py:31-45); None (default):
            whatever autograd asks for -- dC / dBias exactly when c / bias require
            grad.  The reference defaults to False because an MLX VJP cannot tell
            which inputs are differentiated; torch's autograd can.
        filter_eps: backward tile-filter threshold (ln 2^-12); None disables filtering
    Returns:
        loss (fp32 scalar, or [...] for reduction="none"), optionally (loss, lse)
    """
    if impl not in _IMPLS:
        raise ValueError(f"Unknown impl: {impl!r} (expected one of {_IMPLS})")
    if impl == "reference":
        return linear_cross_entropy_reference(e, c, targets, bias=bias, reduction=reduction,
                                              ignore_index=ignore_index, shift=shift, return_lse=return_lse)
    if shift:
        e = e[..., :-shift, :]
        targets = targets[..., shift:]
    orig_shape = targets.shape
    D = e.shape[-1]
    e_flat = e.reshape(-1, D)
    t_flat = targets.reshape(-1)
    grads = True if compute_all_grads is None else bool(compute_all_grads)
    loss, lse = _cce(e_flat, c, t_flat, bias, reduction, ignore_index, filter_eps, grad_c=grads, grad_bias=grads)
    if reduction == "none":
        loss = loss.reshape(orig_shape)
    if return_lse:
        return loss, lse
    return loss


def cut_cross_entropy(e, c, targets, bias=None, reduction="mean", ignore_index=-100, compute_all_grads=False,
                      *, stream=None):
    """Reference csrc/bindings.cpp:15-56 (one-shot native op).

    compute_all_grads=False differentiates only e (the reference's LoRA /
    frozen-head mode); True also produces dC and dBias.
    """
    ctx = torch.cuda.stream(stream) if stream is not None else _ext._nullctx()
    with ctx:
        loss, _ = _cce(e, c, targets, bias, reduction, ignore_index, FILTER_LOG_EPS,
                       grad_c=compute_all_grads, grad_bias=compute_all_grads)
    return loss


class LinearCrossEntropy(torch.nn.Module):
    """Drop-in module (reference/__init__.py:88-118): ``criterion(e, c, targets, bias=None)``.

    compute_all_grads defaults to None -- gradients for whatever requires grad -- where
    the reference defaults to False (see linear_cross_entropy); pass False for the
    reference's frozen-head behaviour whatever c.requires_grad says.
    """

    def __init__(self, reduction="mean", ignore_index=-100, shift=0, compute_all_grads=None,
                 filter_eps=FILTER_LOG_EPS):
        super().__init__()
        self.reduction = reduction
        self.ignore_index = ignore_index
        self.shift = shift
        self.compute_all_grads = compute_all_grads
        self.filter_eps = filter_eps

    def forward(self, e, c, targets, bias=None):
        return linear_cross_entropy(e, c, targets, bias=bias, reduction=self.reduction,
                                    ignore_index=self.ignore_index, shift=self.shift,
                                    compute_all_grads=self.compute_all_grads, filter_eps=self.filter_eps)
