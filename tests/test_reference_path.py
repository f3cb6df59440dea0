"""linear_cross_entropy_reference (the reference's materialised-logits path, selected
with impl="reference") against the float64 oracle, on CPU tensors: loss for every
reduction, shift, return_lse, bias, ignore_index (and None), and autograd gradients."""

import numpy as np
import pytest
import torch

from oracle import cce_oracle as O


@pytest.fixture(scope="module")
def ref():
    from mlx_cce_amd.reference import linear_cross_entropy_reference
    return linear_cross_entropy_reference


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("shift", [0, 2])
def test_against_oracle(ref, reduction, bias, shift):
    rng = np.random.default_rng(11)
    B, T, D, V = 2, 9, 8, 50
    e = torch.tensor(rng.standard_normal((B, T, D)), requires_grad=True)
    c = torch.tensor(rng.standard_normal((V, D)) * 0.5, requires_grad=True)
    b = torch.tensor(rng.standard_normal(V) * 0.2, requires_grad=True) if bias else None
    t = torch.tensor(rng.integers(0, V, (B, T)))
    t[0, 3] = -100
    loss, lse = ref(e, c, t, b, reduction=reduction, shift=shift, return_lse=True)
    want, want_lse = O.linear_cross_entropy(e.detach().numpy(), c.detach().numpy(), t.numpy(),
                                            None if b is None else b.detach().numpy(), reduction, shift=shift,
                                            return_lse=True)
    np.testing.assert_allclose(loss.detach().numpy(), want, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(lse.numpy(), want_lse, rtol=1e-12)
    assert loss.dtype == torch.float64  # float64 inputs keep float64; 16-bit inputs give float32
    loss.backward(torch.ones_like(loss))
    es = e.detach().numpy()[:, :e.shape[1] - shift, :].reshape(-1, D)
    ts = t.numpy()[:, shift:].reshape(-1)
    rE, rC, rB = O.grads(es, c.detach().numpy(), ts, None if b is None else b.detach().numpy(), reduction)
    gE = e.grad.numpy()[:, :e.shape[1] - shift, :].reshape(-1, D)
    assert O.rel_fro(gE, rE) < 1e-6 and O.rel_fro(c.grad.numpy(), rC) < 1e-6
    if bias:
        assert O.rel_fro(b.grad.numpy(), rB) < 1e-6


def test_16bit_inputs_give_float32_loss(ref):
    e = torch.randn(6, 8).to(torch.bfloat16)
    c = torch.randn(10, 8).to(torch.bfloat16)
    t = torch.randint(0, 10, (6,))
    loss, lse = ref(e, c, t, return_lse=True)
    assert loss.dtype == torch.float32 and lse.dtype == torch.float32
    want = O.linear_cross_entropy(e.double().numpy(), c.double().numpy(), t.numpy(), None, "mean")
    np.testing.assert_allclose(float(loss), want, rtol=1e-2)  # logits rounded to bf16 as in MLX


def test_ignore_index_none_and_all_ignored(ref):
    rng = np.random.default_rng(12)
    e = torch.tensor(rng.standard_normal((6, 4)))
    c = torch.tensor(rng.standard_normal((10, 4)))
    t = torch.tensor(rng.integers(0, 10, 6))
    np.testing.assert_allclose(float(ref(e, c, t, ignore_index=None)),
                               O.linear_cross_entropy(e.numpy(), c.numpy(), t.numpy(), None, "mean", ignore_index=None),
                               rtol=1e-6)
    assert float(ref(e, c, torch.full((6,), -100), reduction="mean")) == 0.0
    with pytest.raises(ValueError, match="reduction"):
        ref(e, c, t, reduction="avg")
