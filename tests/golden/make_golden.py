"""Write the golden fixtures under tests/golden/ (run from the repo root).

The expected values come from an implementation independent of oracle/: float64
torch autograd through materialised logits and torch.nn.functional.cross_entropy
(the same computation as the reference's oracle, reference/_reference.py:24-44,
which uses mlx.nn.losses.cross_entropy — MLX is not installable here, so its
bits cannot be captured; see the parity notes in the design document).
Inputs are exactly representable in bfloat16 so every dtype path can use them.

Cases mirror the reference tests' shapes and options
(tests/test_correctness.py:25-104, tests/test_gradients.py:34-115), shrunk in V,
plus ragged and integer-valued cases.
"""

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def bf16_exact(x):
    return x.to(torch.bfloat16).to(torch.float64)


def case(name, N, D, V, seed, reduction="mean", ignore_index=-100, n_ignored=0, bias=False, integer=False,
         c_std=1.0, boost=None):
    g = torch.Generator().manual_seed(seed)
    if integer:
        e = torch.randint(-3, 4, (N, D), generator=g).double()
        c = torch.randint(-3, 4, (V, D), generator=g).double()
        b = torch.randint(-4, 5, (V,), generator=g).double() if bias else None
    else:
        c = bf16_exact(torch.randn((V, D), generator=g, dtype=torch.float64) * c_std)
        e = torch.randn((N, D), generator=g, dtype=torch.float64)
        b = bf16_exact(torch.randn((V,), generator=g, dtype=torch.float64)) if bias else None
    t = torch.randint(0, V, (N,), generator=g)
    if boost is not None:
        ct = c[t]
        e = 0.5 * e + boost * ct / ct.pow(2).sum(1, keepdim=True)
    e = bf16_exact(e) if not integer else e
    if n_ignored:
        t[N - n_ignored:] = ignore_index
    ec = e.clone().requires_grad_(True)
    cc = c.clone().requires_grad_(True)
    bc = b.clone().requires_grad_(True) if b is not None else None
    logits = ec @ cc.T
    if bc is not None:
        logits = logits + bc
    lse = torch.logsumexp(logits, dim=1)
    nll = F.cross_entropy(logits, t, reduction="none", ignore_index=ignore_index)
    valid = (t != ignore_index).double()
    nll = nll * valid
    if reduction == "none":
        loss = nll
        loss.backward(torch.ones_like(loss))
    elif reduction == "sum":
        loss = nll.sum()
        loss.backward()
    else:
        loss = nll.sum() / valid.sum().clamp(min=1)
        loss.backward()
    out = dict(e=e.float().numpy(), c=c.float().numpy(), targets=t.numpy().astype(np.int64),
               reduction=np.array(reduction), ignore_index=np.array(ignore_index),
               loss=loss.detach().numpy(), nll=nll.detach().numpy(), lse=lse.detach().numpy(),
               dE=ec.grad.numpy(), dC=cc.grad.numpy())
    if b is not None:
        out["bias"] = b.float().numpy()
        out["dBias"] = bc.grad.numpy()
    np.savez_compressed(os.path.join(HERE, f"{name}.npz"), **out)
    print(name, N, D, V, float(loss.detach().sum()))


if __name__ == "__main__":
    case("g_mean", 32, 64, 512, 42)
    case("g_sum_bias_ignore", 32, 64, 512, 43, reduction="sum", n_ignored=16, bias=True)
    case("g_none_ragged", 37, 24, 300, 44, reduction="none", n_ignored=5)
    case("g_int_bias_none", 40, 16, 260, 45, reduction="none", bias=True, integer=True)
    case("g_peaked", 64, 64, 640, 46, c_std=0.02, boost=12.0)
