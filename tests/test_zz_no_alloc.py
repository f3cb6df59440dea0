"""cce_backward_noalloc (no workspace, no allocation: a static device scratch) against
cce_backward_ex on the same inputs, through the C ABI: two calls in a row, the second
with a smaller problem, each bit for bit equal to the workspace entry point's output
(same plan: both problems' default workspace fits the static scratch).  A problem too
large for the scratch is refused with CCE_ERR_WORKSPACE before any device work."""

import numpy as np
import pytest
import torch

from oracle import cce_oracle as O

pytestmark = pytest.mark.gpu


def _case(dev, N, D, V, dtype, seed, bias):
    g = torch.Generator(device=dev).manual_seed(seed)
    e = torch.randn((N, D), generator=g, device=dev).to(dtype)
    c = (torch.randn((V, D), generator=g, device=dev) * 0.05).to(dtype)
    b = (torch.randn((V,), generator=g, device=dev) * 0.1).to(dtype) if bias else None
    t = torch.randint(0, V, (N,), generator=g, device=dev)
    t[::17] = -100
    return e, c, b, t


def test_noalloc_matches_workspace_backward_twice(cuda):
    import mlx_cce_amd as m
    ext = m._ext
    assert ext.lib().cce_backward_noalloc_scratch_size() == 64 << 20
    cases = [(1000, 256, 5000, torch.bfloat16, 1, True, m.FILTER_LOG_EPS), (300, 128, 2000, torch.bfloat16, 2, False,
                                                                           None)]
    for N, D, V, dtype, seed, bias, feps in cases:
        assert ext.workspace_size(torch.empty(N, D, dtype=dtype), torch.empty(V, D, dtype=dtype), True, True,
                                  bias) <= 64 << 20
        e, c, b, t = _case(cuda, N, D, V, dtype, seed, bias)
        tm, _, _, lse, _ = ext.forward(e, c, t, b, -100)
        d_nll = torch.full((N,), 1.0 / N, device=cuda)
        st_ws = torch.zeros(3, dtype=torch.int64, device=cuda)
        st_na = torch.zeros(3, dtype=torch.int64, device=cuda)
        ref = ext.backward(e, c, t, lse, tm, d_nll, b, -100, feps, True, True, True, tile_stats=st_ws)
        got = ext.backward_noalloc(e, c, t, lse, tm, d_nll, b, -100, feps, True, True, True, tile_stats=st_na)
        torch.cuda.synchronize()
        print(f"N={N} D={D} V={V}: tiles {st_na.tolist()}")
        assert torch.equal(st_ws, st_na)
        for name, x, y in zip(("dE", "dC", "dBias"), got, ref):
            if y is None:
                assert x is None
                continue
            assert torch.equal(x.view(torch.int16), y.view(torch.int16)), name
        if feps is None:  # dense: against the oracle too
            rE, rC, _ = O.grads(e.double().cpu().numpy(), c.double().cpu().numpy(), t.cpu().numpy(), None,
                                d_nll=np.where(t.cpu().numpy() != -100, 1.0 / N, 0.0))
            assert O.rel_fro(got[0].double().cpu().numpy(), rE) < 2e-2
            assert O.rel_fro(got[1].double().cpu().numpy(), rC) < 2e-2


def test_noalloc_refuses_problems_past_the_scratch(cuda):
    import mlx_cce_amd as m
    ext = m._ext
    e = torch.zeros((8192, 4096), dtype=torch.bfloat16, device=cuda)  # the fp32 dE carry alone is 128 MiB
    c = torch.zeros((128256, 4096), dtype=torch.bfloat16, device=cuda)
    t = torch.zeros(8192, dtype=torch.int64, device=cuda)
    lse = torch.zeros(8192, device=cuda)
    tm = torch.zeros((1002, 8192), device=cuda)
    with pytest.raises(ValueError, match="static scratch"):
        ext.backward_noalloc(e, c, t, lse, tm, lse, None, -100, None, True, True, False)


def test_noalloc_refuses_outputs_unlike_their_inputs(cuda):
    """Caller-provided outputs are written through raw pointers, so each must be a
    contiguous tensor of its input's shape, dtype and device (and tile_stats int64[3]):
    anything else raises before the library is called."""
    import mlx_cce_amd as m
    ext = m._ext
    e, c, b, t = _case(cuda, 256, 64, 1000, torch.bfloat16, 3, True)
    tm, _, _, lse, _ = ext.forward(e, c, t, b, -100)
    d_nll = torch.full((256,), 1.0 / 256, device=cuda)
    bad = {"dE": torch.empty((255, 64), dtype=torch.bfloat16, device=cuda),
           "dC": torch.empty((1000, 64), dtype=torch.float32, device=cuda),
           "dB": torch.empty((2000,), dtype=torch.bfloat16, device=cuda)[::2]}
    for name, out in bad.items():
        with pytest.raises(ValueError, match=name):
            ext.backward_noalloc(e, c, t, lse, tm, d_nll, b, **{name: out})
    with pytest.raises(ValueError, match="tile_stats"):
        ext.backward_noalloc(e, c, t, lse, tm, d_nll, b, tile_stats=torch.zeros(3, dtype=torch.int32, device=cuda))
