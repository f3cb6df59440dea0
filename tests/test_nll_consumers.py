"""NLL consumers (mlx_cce_amd.nll; reference README.md:110-122).

CPU: the consumers' arithmetic on given NLL tensors against closed forms in
float64 numpy (they are plain torch ops).  GPU: token_nll is the fp32 per-token
loss of the CCE path for every input dtype, and a DPO loss built on it sends
its per-token upstream gradient through the CCE backward (dE / dC against fp64
autograd of the same composition).
"""

import math

import numpy as np
import pytest
import torch

from mlx_cce_amd import nll as NLL
from oracle import cce_oracle as O


def test_perplexity_matches_readme_formula():
    x = torch.rand(3, 17, dtype=torch.float64) * 4
    assert abs(float(NLL.perplexity(x)) - math.exp(x.numpy().mean())) < 1e-12
    m = torch.rand(3, 17) > 0.3
    ref = math.exp(x.numpy()[m.numpy()].sum() / m.numpy().sum())
    assert abs(float(NLL.perplexity(x, m)) - ref) < 1e-12 * ref
    assert float(NLL.perplexity(torch.zeros(4), torch.zeros(4, dtype=torch.bool))) == 1.0  # max(count, 1)


def test_perplexity_promotes_half_inputs_to_fp32():
    x = torch.full((8,), 2.0, dtype=torch.bfloat16)
    p = NLL.perplexity(x)
    assert p.dtype == torch.float32 and abs(float(p) - math.exp(2.0)) < 1e-5


def test_sequence_nll_and_mask():
    x = torch.arange(12, dtype=torch.float32).reshape(2, 6)
    assert NLL.sequence_nll(x).tolist() == [15.0, 51.0]
    m = torch.tensor([1, 1, 0, 0, 0, 1])
    assert NLL.sequence_nll(x, m).tolist() == [6.0, 24.0]


def test_dpo_loss_single_pair_is_readme_expression():
    pref = torch.tensor([0.5, 1.25, 0.25], dtype=torch.float64)
    rej = torch.tensor([2.0, 0.75, 1.0], dtype=torch.float64)
    gap = rej.sum() - pref.sum()
    readme = -math.log(1.0 / (1.0 + math.exp(-float(gap))))
    assert abs(float(NLL.dpo_loss(pref, rej)) - readme) < 1e-14


def test_dpo_loss_batched_beta_and_reductions():
    rng = np.random.default_rng(3)
    pref = torch.tensor(rng.random((5, 9)) * 3)
    rej = torch.tensor(rng.random((5, 9)) * 3)
    gap = rej.numpy().sum(1) - pref.numpy().sum(1)
    per = np.log1p(np.exp(-0.1 * gap))
    assert np.allclose(NLL.dpo_loss(pref, rej, beta=0.1, reduction="none").numpy(), per, rtol=1e-13)
    assert abs(float(NLL.dpo_loss(pref, rej, beta=0.1)) - per.mean()) < 1e-13
    assert abs(float(NLL.dpo_loss(pref, rej, beta=0.1, reduction="sum")) - per.sum()) < 1e-12
    with pytest.raises(ValueError):
        NLL.dpo_loss(pref, rej, reduction="avg")


def test_dpo_loss_is_stable_at_large_gaps():
    pref = torch.tensor([[1000.0]])
    rej = torch.tensor([[0.0]])
    assert float(NLL.dpo_loss(pref, rej)) == 1000.0  # softplus(1000), not inf
    assert float(NLL.dpo_loss(rej, pref)) == 0.0
    g = torch.tensor([[1000.0]], requires_grad=True)
    NLL.dpo_loss(g, torch.zeros(1, 1)).backward()
    assert float(g.grad) == 1.0


# ------------------------------------------------------------------ GPU
@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_token_nll_is_fp32_per_token_loss(cuda, dtype):
    g = torch.Generator(device=cuda).manual_seed(11)
    B, T, D, V = 2, 40, 64, 900
    e = torch.randn((B, T, D), generator=g, device=cuda).to(dtype)
    c = (torch.randn((V, D), generator=g, device=cuda) * 0.1).to(dtype)
    t = torch.randint(0, V, (B, T), generator=g, device=cuda)
    t[:, -3:] = -100
    x = NLL.token_nll(e, c, t)
    torch.cuda.synchronize()
    assert x.dtype == torch.float32 and x.shape == (B, T)
    ref, _, _ = O.per_token(e.reshape(-1, D).double().cpu().numpy(), c.double().cpu().numpy(), t.reshape(-1).cpu().numpy())
    np.testing.assert_allclose(x.reshape(-1).double().cpu().numpy(), ref, rtol=1e-4, atol=1e-4)
    assert float(x[:, -3:].abs().sum()) == 0.0


@pytest.mark.gpu
def test_dpo_gradient_through_cce_backward(cuda):
    """Per-token upstream = d(dpo)/d(nll); filter off, fp32: dE / dC within 1e-4 of fp64 autograd."""
    g = torch.Generator(device=cuda).manual_seed(12)
    T, D, V = 48, 32, 500
    e_p = torch.randn((T, D), generator=g, device=cuda).requires_grad_(True)
    e_r = torch.randn((T, D), generator=g, device=cuda).requires_grad_(True)
    c = (torch.randn((V, D), generator=g, device=cuda) * 0.2).requires_grad_(True)
    t_p = torch.randint(0, V, (T,), generator=g, device=cuda)
    t_r = torch.randint(0, V, (T,), generator=g, device=cuda)
    loss = NLL.dpo_loss(NLL.token_nll(e_p, c, t_p, filter_eps=None), NLL.token_nll(e_r, c, t_r, filter_eps=None),
                        beta=0.5)
    loss.backward()
    torch.cuda.synchronize()

    def ref_nll(e, c, t):
        s = e @ c.T
        return torch.logsumexp(s, dim=1) - s.gather(1, t[:, None])[:, 0]

    ep, er, cc = (x.detach().double().cpu().requires_grad_(True) for x in (e_p, e_r, c))
    rl = NLL.dpo_loss(ref_nll(ep, cc, t_p.cpu()), ref_nll(er, cc, t_r.cpu()), beta=0.5)
    rl.backward()
    assert abs(float(loss.detach()) - float(rl.detach())) < 1e-5 * max(1.0, abs(float(rl.detach())))
    for got, ref in ((e_p.grad, ep.grad), (e_r.grad, er.grad), (c.grad, cc.grad)):
        assert O.rel_fro(got.double().cpu().numpy(), ref.numpy()) < 1e-4
