"""Quantized classifier rows for the loss.

The reference's callers keep the lm_head / tied embedding in MLX's affine group
quantization and dequantize it before calling the loss (README.md:84-95,136;
examples/mlx_lm_lora_test.py:16-21):

    c = mx.dequantize(embed.weight, embed.scales, embed.biases, embed.group_size, embed.bits)
    loss = linear_cross_entropy(hidden, c, targets)

Here the quantized rows go to the loss as they are:

    qw = QuantizedWeight(weight, scales, biases, group_size=64, bits=4)
    loss = linear_cross_entropy(hidden, qw, targets)

and the HIP library dequantizes a bounded chunk of rows at a time (cce_forward_q /
cce_backward_q) instead of materialising the [V, D] matrix.  The rows carry no
gradient (the frozen-head setting of those callers); dE and dBias are produced.

Layout (MLX's, mlx >= 0.22): ``weight`` [V, D * bits / 32] 32-bit words, code j of a
word in bits [j * bits, (j + 1) * bits); ``scales`` and ``biases`` [V, D / group_size]
in the compute dtype; w = scale * q + bias.  bits 2, 4 or 8; group_size 32, 64 or 128.
"""

import torch

from . import _ext

__all__ = ["QuantizedWeight", "quantize", "dequantize"]


class QuantizedWeight:
    """Classifier rows [V, D] in affine group quantization (the triple mx.quantize returns)."""

    def __init__(self, weight, scales, biases, group_size=64, bits=4):
        if bits not in (2, 4, 8):
            raise ValueError(f"bits must be 2, 4 or 8, got {bits}")
        if group_size not in (32, 64, 128):
            raise ValueError(f"group_size must be 32, 64 or 128, got {group_size}")
        self.weight = weight
        self.scales = scales
        self.biases = biases
        self.group_size = int(group_size)
        self.bits = int(bits)

    @property
    def shape(self):
        return (self.weight.shape[0], self.weight.shape[1] * 32 // self.bits)

    @property
    def dtype(self):
        return self.scales.dtype

    @property
    def device(self):
        return self.weight.device

    def dequantize(self):
        return dequantize(self)


def quantize(w, group_size=64, bits=4):
    """QuantizedWeight of dense rows w [V, D] (D a multiple of group_size).

    Per group of group_size elements: bias = min, scale = (max - min) / (2^bits - 1)
    (both rounded to w's dtype), q = round((w - bias) / scale) clipped to the code
    range.  This is a plain min/max quantizer for preparing inputs; it need not pick
    the codes mx.quantize would.  The loss depends only on (weight, scales, biases).
    """
    if w.dim() != 2:
        raise ValueError("w must be [V, D]")
    V, D = w.shape
    if D % group_size != 0:
        raise ValueError(f"D={D} must be a multiple of group_size={group_size}")
    if bits not in (2, 4, 8):
        raise ValueError(f"bits must be 2, 4 or 8, got {bits}")
    levels = (1 << bits) - 1
    g = w.detach().to(torch.float32).reshape(V, D // group_size, group_size)
    lo = g.amin(dim=-1)
    hi = g.amax(dim=-1)
    scales = ((hi - lo) / levels).clamp_min(1e-8).to(w.dtype)
    biases = lo.to(w.dtype)
    s32 = scales.to(torch.float32).unsqueeze(-1)
    b32 = biases.to(torch.float32).unsqueeze(-1)
    q = torch.round((g - b32) / s32).clamp_(0, levels).to(torch.int64).reshape(V, D)
    epw = 32 // bits
    shifts = (torch.arange(epw, device=w.device, dtype=torch.int64) * bits)
    words = (q.reshape(V, D // epw, epw) << shifts).sum(dim=-1)
    words = torch.where(words >= (1 << 31), words - (1 << 32), words).to(torch.int32)
    return QuantizedWeight(words.contiguous(), scales.contiguous(), biases.contiguous(), group_size, bits)


def dequantize(qw):
    """Dense rows [V, D] of a QuantizedWeight, dtype of its scales (HIP kernel; the values
    the quantized loss passes use: fp32 scale * q, plus bias in fp32, rounded to nearest-even)."""
    return _ext.dequantize(qw)
