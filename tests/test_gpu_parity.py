"""GPU parity: the HIP path (libcce_mi355x.so via the C ABI) against the float64 oracle.

Tolerances (written per test):
  * loss: 1e-3 relative (reference tests/test_correctness.py:34-40) — the fp32
    path is checked at 1e-5;
  * dE / dC / dBias: relative Frobenius error <= 1e-3 with the filter disabled for
    fp32 inputs, <= 2e-2 for bf16 (measured values are
    printed), cosine > 0.9999 for the reference's own dE test shapes
    (tests/test_gradients.py:34-46);
  * exact: target gather, tile max and the ignore mask on integer-valued inputs
    (every product and sum is exact in fp32), and the kept-tile set recomputed
    from the kernel's own fp32 statistics.
"""

import glob
import math
import os

import numpy as np
import pytest
import torch

import workloads
from oracle import cce_oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


@pytest.fixture(scope="module")
def m(cuda):
    import mlx_cce_amd
    mlx_cce_amd._ext.lib()
    return mlx_cce_amd


def f64(t):
    return None if t is None else t.detach().double().cpu().numpy()


def run(m, e, c, t, bias=None, reduction="mean", ignore_index=-100, filter_eps=None, grads=True, upstream=None):
    e = e.detach().clone().requires_grad_(grads)
    c = c.detach().clone().requires_grad_(grads)
    b = bias.detach().clone().requires_grad_(grads) if bias is not None else None
    loss = m.linear_cross_entropy(e, c, t, b, reduction=reduction, ignore_index=ignore_index, filter_eps=filter_eps)
    if grads:
        g = torch.ones_like(loss) if upstream is None else upstream
        loss.backward(g)
    torch.cuda.synchronize()
    return loss.detach(), (e.grad if grads else None), (c.grad if grads else None), (b.grad if (grads and b is not None) else None)


def cosine(a, b):
    a, b = np.ravel(a), np.ravel(b)
    return float(np.dot(a, b) / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))


def normal_case(B, D, V, dtype, dev, seed=42, std=1.0):
    g = torch.Generator(device=dev).manual_seed(seed)
    e = torch.randn((B, D), generator=g, device=dev).to(dtype)
    c = (torch.randn((V, D), generator=g, device=dev) * std).to(dtype)
    t = torch.randint(0, V, (B,), generator=g, device=dev)
    return e, c, t


# ------------------------------------------------------------ golden fixtures
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(p)[:-4] for p in GOLDEN])
def test_golden(m, cuda, path, dtype):
    z = np.load(path)
    e = torch.tensor(z["e"], device=cuda).to(dtype)
    c = torch.tensor(z["c"], device=cuda).to(dtype)
    b = torch.tensor(z["bias"], device=cuda).to(dtype) if "bias" in z else None
    t = torch.tensor(z["targets"], device=cuda)
    red = str(z["reduction"])
    loss, dE, dC, dB = run(m, e, c, t, b, red, int(z["ignore_index"]))
    tol_loss = 1e-5 if dtype == torch.float32 else 1e-3
    np.testing.assert_allclose(f64(loss), z["loss"], rtol=tol_loss, atol=1e-6)
    # fp32: the north-star bound with the filter off (1e-3).  The peaked fixture's target
    # gradient p_t - 1 is ~0.02, so one ulp of lse moves dE by ~5e-5 relative.
    tol = 1e-3 if dtype == torch.float32 else 2e-2
    for name, got, ref in (("dE", dE, z["dE"]), ("dC", dC, z["dC"])) + ((("dBias", dB, z["dBias"]),) if b is not None else ()):
        err = O.rel_fro(f64(got), ref)
        print(f"{os.path.basename(path)} {dtype} {name} rel_fro={err:.3e}")
        assert err < tol, (name, err)


ROUND = {torch.bfloat16: O.round_bf16, torch.float16: O.round_f16}
DENSE16_CASES = [os.path.basename(p)[:-4] for p in GOLDEN] + ["n300_d264_v9000_bias", "n2048_d256_v16384_mean",
                                                               "c2_rows_mean_scale"]


def _dense16_case(case, dtype, dev):
    """(e, c, targets, bias, reduction, ignore_index, upstream) of a 16-bit dense case."""
    up = 1.0
    if case.startswith("n300"):
        e, c, t = normal_case(300, 264, 9000, dtype, dev, seed=23, std=0.05)
        t[::13] = -100
        b = (torch.randn(9000, device=dev) * 0.1).to(dtype)
        red, ign = "sum", -100
    elif case.startswith("n2048"):
        # mean over 2048 rows of a near-uniform softmax: G = p / N ~ 3e-8 sits below
        # fp16's smallest subnormal unless the G tiles are scaled
        e, c, t = normal_case(2048, 256, 16384, dtype, dev, seed=29, std=0.02)
        b, red, ign = None, "mean", -100
    elif case.startswith("c2_rows"):
        # 128 rows of the c2 workload (full D = 2048, V = 128256) with the cotangent the
        # full batch's mean gives (1 / 3973 per row): the upstream gradient 1 / 32
        w = workloads.make("c2", device=dev, scale=1 / 32)
        e = w["e"].reshape(-1, w["D"]).to(dtype)
        c, t, b = w["c"].to(dtype), w["targets"].reshape(-1), None
        red, ign, up = "mean", -100, 1 / 32
    else:
        z = np.load(os.path.join(os.path.dirname(__file__), "golden", case + ".npz"))
        e = torch.tensor(z["e"], device=dev).to(dtype)
        c = torch.tensor(z["c"], device=dev).to(dtype)
        b = torch.tensor(z["bias"], device=dev).to(dtype) if "bias" in z else None
        t = torch.tensor(z["targets"], device=dev)
        red, ign = str(z["reduction"]), int(z["ignore_index"])
    return e, c, t, b, red, ign, up


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", DENSE16_CASES)
def test_dense_16bit_matches_reference_rounding(m, cuda, case, dtype):
    """Filter off, 16-bit inputs: dE / dC / dBias against the reference's semantics --
    the float64 gradient of the same (16-bit) inputs, rounded once to the output dtype,
    as the reference keeps the softmax weight in fp32 through both products and casts
    the fp32 sums (csrc/cce/cce.metal:275-305, cce.cpp:178,442-446;
    reference/_fused_backward.py:1535-1564,1652-1654) -- at 1e-3 relative Frobenius
    (north star, filter disabled).  The G tiles carry G as a hi + lo pair of the input
    dtype (fp16 scaled by a power of two), so only the sums' fp32 arithmetic is left.
    A backward that rounds G to the input dtype once misses this bound on these cases
    (tests/test_oracle.py::test_single_rounded_g_misses_the_dense_16bit_bound)."""
    e, c, t, b, red, ign, up = _dense16_case(case, dtype, cuda)
    loss_up = None if up == 1.0 else torch.tensor(up, device=cuda)
    if red == "none":
        loss_up = torch.full((t.numel(),), up, device=cuda)
    _, dE, dC, dB = run(m, e, c, t, b, red, ign, filter_eps=None, upstream=loss_up)
    rnd = ROUND[dtype]
    ee, cc = f64(e).reshape(-1, e.shape[-1]), f64(c)
    pE, pC, pB = O.grads(ee, cc, t.cpu().numpy().reshape(-1), f64(b), red, ign)
    pairs = [("dE", dE, pE), ("dC", dC, pC)] + ([("dBias", dB, pB)] if b is not None else [])
    for name, got, plain in pairs:
        g = f64(got).reshape(np.shape(plain))
        err = O.rel_fro(g, rnd(plain * up))
        print(f"{case} {dtype} {name}: vs rounded float64 {err:.2e}, vs float64 {O.rel_fro(g, plain * up):.2e}")
        assert err <= 1e-3, (name, err)


def _single_g_model(dtype, d_nll):
    """The one rounding of G a backward with CCE_BWD_G_SINGLE applies: bf16 as it is; fp16
    after scaling by 2^s with max |d_nll| 2^s in [2^13, 2^14) (the compaction's rule),
    taken back out after the products."""
    if dtype == torch.bfloat16:
        return O.round_bf16
    gmax = float(np.max(np.abs(d_nll)))
    s = 0 if gmax == 0.0 else 14 - math.frexp(gmax)[1]
    return lambda g: O.round_f16(g * 2.0 ** s) / 2.0 ** s


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("case", DENSE16_CASES[:-2])
def test_single_rounded_g_matches_its_model(m, cuda, case, dtype):
    """CCE_BWD_G_SINGLE with the filter off (the fast, lower-precision mode): dE / dC
    against the float64 oracle with G rounded once where the kernel rounds it (fp16 with
    its power-of-two scale, so no subnormal G), then to the output dtype, at 1e-3.  What
    is left is the kernels' own fp32 arithmetic."""
    e, c, t, b, red, ign, up = _dense16_case(case, dtype, cuda)
    assert up == 1.0
    with m._ext.backward_options(g_precision="single"):
        _, dE, dC, dB = run(m, e, c, t, b, red, ign, filter_eps=None)
    rnd = ROUND[dtype]
    ee, cc, tt = f64(e), f64(c), t.cpu().numpy()
    dn = O.upstream(O.valid_mask(tt, ign), red)  # max |d_nll| sets the fp16 scale
    sE, sC, sB = O.grads_staged(ee, cc, tt, f64(b), red, ign, stage=_single_g_model(dtype, dn))
    pairs = [("dE", dE, sE), ("dC", dC, sC)] + ([("dBias", dB, sB)] if b is not None else [])
    for name, got, staged in pairs:
        err = O.rel_fro(f64(got), rnd(staged))
        print(f"{case} {dtype} single G {name}: vs its model {err:.2e}")
        assert err <= 1e-3, (name, err)


def test_integer_inputs_exact(m, cuda):
    """Integer inputs: every logit is exact in fp32, so the gather, tile max and mask must match bit for bit."""
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "g_int_bias_none.npz"))
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        e = torch.tensor(z["e"], device=cuda).to(dtype)
        c = torch.tensor(z["c"], device=cuda).to(dtype)
        b = torch.tensor(z["bias"], device=cuda).to(dtype)
        t = torch.tensor(z["targets"], device=cuda)
        t[::7] = -100
        tm, ts, ntl, lse = m.cce_forward_raw(e, c, t, b, ignore_index=-100)  # the reference's layout
        tm128, _, ntl128, _ = m.cce_forward_raw(e, c, t, b, ignore_index=-100, layout="tiles128")
        torch.cuda.synchronize()
        S = z["e"].astype(np.float64) @ z["c"].astype(np.float64).T + z["bias"]
        tt = t.cpu().numpy()
        valid = tt != -100
        rows = np.nonzero(valid)[0]
        np.testing.assert_array_equal(f64(ntl)[rows], -S[rows, tt[rows]])
        np.testing.assert_array_equal(f64(ntl128)[rows], -S[rows, tt[rows]])  # masked rows are not written
        tm_ref, _ = O.tile_stats(z["e"], z["c"], z["bias"])
        np.testing.assert_array_equal(f64(tm128), tm_ref)
        tm32_ref, _ = O.tile_stats(z["e"], z["c"], z["bias"], tile=32)  # V = 260: a ragged last tile
        np.testing.assert_array_equal(f64(tm), tm32_ref.T.reshape(-1))
        _, _, _, _, nll = m._ext.forward(e, c, t, b, -100)
        nll = f64(nll)
        assert (nll[~valid] == 0.0).all()
        np.testing.assert_allclose(nll[valid], O.per_token(z["e"], z["c"], tt, z["bias"])[0][valid], rtol=1e-5)


# -------------------------------------------- the reference's own test suite
SHAPES = [(32, 64, 1024), (64, 128, 4096), (128, 256, 32000), (32, 2048, 128256)]


@pytest.mark.parametrize("B,D,V", SHAPES)
def test_reference_shapes_loss_and_dE(m, cuda, B, D, V):
    """tests/test_correctness.py:34-40 (loss rtol 1e-3) and tests/test_gradients.py:34-46 (dE cosine)."""
    e, c, t = normal_case(B, D, V, torch.float32, cuda)
    loss, dE, _, _ = run(m, e, c, t, filter_eps=m.FILTER_LOG_EPS)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "mean")
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-3)
    rE, _, _ = O.grads(f64(e), f64(c), t.cpu().numpy(), None, "mean")
    assert cosine(f64(dE), rE) > 0.9999


@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
def test_reduction_modes(m, cuda, reduction):
    e, c, t = normal_case(32, 64, 1024, torch.float32, cuda)
    loss, dE, dC, _ = run(m, e, c, t, reduction=reduction)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, reduction)
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-5, atol=1e-5)
    rE, rC, _ = O.grads(f64(e), f64(c), t.cpu().numpy(), None, reduction)
    assert O.rel_fro(f64(dE), rE) < 1e-4 and O.rel_fro(f64(dC), rC) < 1e-4


def test_ignore_index(m, cuda):
    """tests/test_correctness.py:50-63 and tests/test_gradients.py:48-61."""
    e, c, t = normal_case(32, 64, 1024, torch.float32, cuda)
    tm = torch.where(torch.arange(32, device=cuda) < 16, t, torch.full_like(t, -100))
    loss, dE, dC, _ = run(m, e, c, tm, ignore_index=-100)
    full = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "none")
    np.testing.assert_allclose(f64(loss), full[:16].sum() / 16.0, rtol=1e-5)
    assert (f64(dE)[16:] == 0).all()


def test_ignore_index_none(m, cuda):
    e, c, t = normal_case(32, 64, 1024, torch.float32, cuda)
    got = m.cce_loss(e, c, t, ignore_index=None)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "mean", ignore_index=None)
    np.testing.assert_allclose(f64(got), ref, rtol=1e-5)


def test_bias(m, cuda):
    e, c, t = normal_case(32, 64, 1024, torch.float32, cuda)
    b = torch.randn(1024, device=cuda)
    loss, dE, dC, dB = run(m, e, c, t, b)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), f64(b), "mean")
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-5)
    rE, rC, rB = O.grads(f64(e), f64(c), t.cpu().numpy(), f64(b), "mean")
    for got, r in ((dE, rE), (dC, rC), (dB, rB)):
        assert O.rel_fro(f64(got), r) < 1e-4


def test_batched_sequence(m, cuda):
    """tests/test_correctness.py:82-96: e [4, 128, 256], V=4096."""
    g = torch.Generator(device=cuda).manual_seed(42)
    e = torch.randn((4, 128, 256), generator=g, device=cuda)
    c = torch.randn((4096, 256), generator=g, device=cuda)
    t = torch.randint(0, 4096, (4, 128), generator=g, device=cuda)
    loss, dE, _, _ = run(m, e, c, t)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "mean")
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-3)
    rE, _, _ = O.grads(f64(e).reshape(-1, 256), f64(c), t.cpu().numpy().reshape(-1), None, "mean")
    assert cosine(f64(dE).reshape(-1, 256), rE) > 0.9999
    none = m.linear_cross_entropy(e, c, t, reduction="none")
    assert none.shape == (4, 128)


def test_cut_cross_entropy_matches_cce_loss(m, cuda):
    """tests/test_correctness.py:98-104 (rtol 1e-5)."""
    e, c, t = normal_case(32, 64, 1024, torch.float32, cuda)
    a = m.cut_cross_entropy(e, c, t)
    b = m.cce_loss(e, c, t)
    np.testing.assert_allclose(f64(a), f64(b), rtol=1e-5)


def test_shift_and_return_lse(m, cuda):
    g = torch.Generator(device=cuda).manual_seed(3)
    e = torch.randn((2, 40, 64), generator=g, device=cuda)
    c = torch.randn((500, 64), generator=g, device=cuda)
    t = torch.randint(0, 500, (2, 40), generator=g, device=cuda)
    loss, lse = m.linear_cross_entropy(e, c, t, reduction="none", shift=1, return_lse=True)
    assert loss.shape == (2, 39) and lse.shape == (78,)
    ref, rlse = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "none", shift=1, return_lse=True)
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-5)
    np.testing.assert_allclose(f64(lse), rlse, rtol=1e-6)


def test_float16(m, cuda):
    e, c, t = normal_case(128, 256, 4000, torch.float16, cuda, std=0.1)
    loss, dE, dC, _ = run(m, e, c, t)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "mean")
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-3)
    rE, rC, _ = O.grads(f64(e), f64(c), t.cpu().numpy(), None, "mean")
    assert O.rel_fro(f64(dE), rE) < 2e-2 and O.rel_fro(f64(dC), rC) < 2e-2


# ------------------------------------------------------------------- edges
@pytest.mark.parametrize("N,D,V", [(1, 8, 1), (3, 16, 5), (130, 40, 257), (300, 8, 129)])
def test_ragged_shapes(m, cuda, N, D, V):
    e, c, t = normal_case(N, D, V, torch.float32, cuda, seed=N + V)
    b = torch.randn(V, device=cuda)
    loss, dE, dC, dB = run(m, e, c, t, b, reduction="sum")
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), f64(b), "sum")
    np.testing.assert_allclose(f64(loss), ref, rtol=1e-5, atol=1e-5)
    rE, rC, rB = O.grads(f64(e), f64(c), t.cpu().numpy(), f64(b), "sum")
    for got, r in ((dE, rE), (dC, rC), (dB, rB)):
        assert O.rel_fro(f64(got), r) < 1e-4 or np.abs(f64(got) - r).max() < 1e-6


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("V", [2048, 2000, 1001])
def test_forward_bias_staged_in_lds(m, cuda, dtype, V):
    """The forward starts the accumulators from a 16-byte aligned bias whose V * element
    size is a multiple of 16, staged in LDS (one LDS-DMA copy per tile, zeros past V:
    V = 2000 ends in a partial vocabulary block); any other bias it adds after the
    contraction, from global memory.  An unaligned view of the same values takes the
    global path: the two orders of the fp32 sums agree to a few ulps (measured at c4:
    lse within 1.9e-6), each path is deterministic, and the loss matches the oracle.
    With V = 1001 (2002 bytes) both views take the global path: bit for bit."""
    ext = m._ext
    N, D = 300, 96
    e, c, t = normal_case(N, D, V, dtype, cuda, seed=V, std=0.1)
    g = torch.Generator(device=cuda).manual_seed(V + 1)
    store = (torch.randn(V + 8, generator=g, device=cuda) * 0.5).to(dtype)
    b_al = store[:V]
    off = torch.empty(V + 8, dtype=dtype, device=cuda)
    off[1:V + 1] = b_al
    b_un = off[1:V + 1]  # the same values, 2 or 4 bytes past a 16-byte boundary
    assert b_al.data_ptr() % 16 == 0 and b_un.data_ptr() % 16 != 0
    lds = ext.forward(e, c, t, b_al, -100)
    lds2 = ext.forward(e, c, t, b_al, -100)
    glob = ext.forward(e, c, t, b_un, -100)
    torch.cuda.synchronize()
    same_path = V * b_al.element_size() % 16 != 0
    for k, name in ((0, "tile_max"), (1, "tile_sum_exp"), (3, "lse"), (4, "nll")):
        assert torch.equal(lds[k], lds2[k]), name
        if same_path:
            assert torch.equal(lds[k], glob[k]), name
        else:
            err = (lds[k] - glob[k]).abs().max().item()
            print(f"V={V} {dtype}: {name} LDS vs global path max diff {err:.2e}")
            torch.testing.assert_close(lds[k], glob[k], rtol=1e-5, atol=1e-5)
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), f64(b_al), "none")
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    np.testing.assert_allclose(f64(lds[4]), ref, rtol=tol, atol=tol)


def test_all_rows_ignored(m, cuda):
    e, c, t = normal_case(64, 32, 300, torch.bfloat16, cuda)
    t[:] = -100
    loss, dE, dC, _ = run(m, e, c, t)
    assert f64(loss) == 0.0
    assert not f64(dE).any() and not f64(dC).any()


def test_out_of_range_target_is_nan(m, cuda):
    e, c, t = normal_case(16, 32, 100, torch.float32, cuda)
    t[3] = 100
    loss = m.linear_cross_entropy(e, c, t, reduction="none")
    torch.cuda.synchronize()
    assert math.isnan(float(loss[3])) and np.isfinite(f64(loss)[[0, 1, 2, 4]]).all()


def test_reduce_loss_and_broadcast_grad(m, cuda):
    """cce_reduce_loss / cce_broadcast_grad against fp64 numpy: sum, mean / max(count, 1), ignore_index
    (and None), all rows ignored, NaN propagation; d_nll = grad / scale."""
    from mlx_cce_amd import _ext
    g = torch.Generator(device=cuda).manual_seed(5)
    N = 5000
    nll = torch.rand(N, generator=g, device=cuda) * 10
    t = torch.randint(0, 50, (N,), generator=g, device=cuda)
    t[::7] = -100
    nll[t == -100] = 0.0  # the forward writes 0 for masked rows
    x = nll.double().cpu().numpy()
    kept = int((t != -100).sum())
    loss, scale = _ext.reduce_loss(nll, t, -100, "mean")
    assert abs(float(loss) - x.sum() / kept) <= 1e-6 * abs(x.sum() / kept) and float(scale) == kept
    loss, scale = _ext.reduce_loss(nll, t, -100, "sum")
    assert abs(float(loss) - x.sum()) <= 1e-6 * x.sum() and scale is None
    loss, scale = _ext.reduce_loss(nll, t, None, "mean")
    assert abs(float(loss) - x.sum() / N) <= 1e-6 * x.sum() / N and float(scale) == N
    t_all = torch.full_like(t, -100)
    loss, scale = _ext.reduce_loss(torch.zeros_like(nll), t_all, -100, "mean")
    assert float(loss) == 0.0 and float(scale) == 1.0
    nll[11] = float("nan")
    loss, _ = _ext.reduce_loss(nll, t, -100, "sum")
    assert math.isnan(float(loss))
    up = torch.tensor(3.0, device=cuda)
    d = _ext.broadcast_grad(up, torch.tensor(8.0, device=cuda), N)
    assert d.shape == (N,) and bool((d == 0.375).all())
    d = _ext.broadcast_grad(up, None, 7)
    assert bool((d == 3.0).all())


def test_only_dE_requested(m, cuda):
    e, c, t = normal_case(64, 64, 1000, torch.bfloat16, cuda)
    e.requires_grad_(True)
    loss = m.linear_cross_entropy(e, c, t)
    loss.backward()
    torch.cuda.synchronize()
    rE, _, _ = O.grads(f64(e), f64(c), t.cpu().numpy(), None, "mean")
    assert O.rel_fro(f64(e.grad), rE) < 2e-2 and c.grad is None


def test_upstream_gradient_none_reduction(m, cuda):
    e, c, t = normal_case(96, 64, 700, torch.float32, cuda)
    b = torch.randn(700, device=cuda)
    up = torch.randn(96, device=cuda)
    loss, dE, dC, dB = run(m, e, c, t, b, reduction="none", upstream=up)
    rE, rC, rB = O.grads(f64(e), f64(c), t.cpu().numpy(), f64(b), "none", grad_out=f64(up))
    for got, r in ((dE, rE), (dC, rC), (dB, rB)):
        assert O.rel_fro(f64(got), r) < 1e-4


# ------------------------------------------------------------------ filter
def _peaked(dev, N=512, D=256, V=8192, boost=12.0, dtype=torch.bfloat16, seed=5):
    g = torch.Generator(device=dev).manual_seed(seed)
    c = (torch.randn((V, D), generator=g, device=dev) * 0.02).to(dtype)
    t = workloads.zipf_targets(g, N, V, device=dev)
    ct = c.float()[t]
    e = (0.5 * torch.randn((N, D), generator=g, device=dev) + boost * ct / ct.pow(2).sum(1, keepdim=True)).to(dtype)
    return e, c, t


def _sorted_rows(tt, d_nll, V, ignore_index=-100, head_run=16):
    """The token order the backward may run its tile filter in: rows sorted (stably) by
    the 128-column vocabulary tile of their target, rows without gradient (ignored,
    out-of-range target, d_nll == 0) keyed past the last tile; then the rows whose key
    has fewer than head_run rows are spread evenly over the 128-row blocks (block b
    takes tail rows [tb(b), tb(b+1)), tb(b) = floor(min(128 b, N) nT / N), followed by
    the next rows of the longer runs).  Returns perm: position p holds input row perm[p]."""
    N = len(tt)
    nvt = (V + 127) // 128
    act = (d_nll != 0) & (tt != ignore_index) & (tt >= 0) & (tt < V)
    key = np.where(act, tt // 128, nvt)
    srt = np.argsort(key, kind="stable")
    head = np.bincount(key, minlength=nvt + 1)[key[srt]] >= head_run
    heads, tails = srt[head], srt[~head]
    nT = len(tails)
    nrb = (N + 127) // 128
    tb = [min(128 * b, N) * nT // N for b in range(nrb + 1)]
    perm = np.empty(N, dtype=np.int64)
    h = 0
    for b in range(nrb):
        p0 = 128 * b
        nt = tb[b + 1] - tb[b]
        perm[p0:p0 + nt] = tails[tb[b]:tb[b + 1]]
        nh = min(128 * (b + 1), N) - p0 - nt
        perm[p0 + nt:p0 + nt + nh] = heads[h:h + nh]
        h += nh
    return perm


@pytest.mark.parametrize("precision", [None, "pair"])
@pytest.mark.parametrize("order", ["input", "sorted"])
def test_filtered_backward_matches_filter_emulation(m, cuda, order, precision):
    """Kept-tile set is exact against the kernel's own fp32 statistics (token blocks of the
    input order, or of the rows sorted by target tile); gradients match the oracle over it:
    within the bf16 tolerance with G rounded once (the filter-on default), and within 1e-3
    of the emulation rounded to bf16 with G as the hi + lo pair (CCE_BWD_G_PAIR)."""
    e, c, t = _peaked(cuda)
    tm, _, _, lse, _ = m._ext.forward(e, c, t, None, -100)
    N, V = e.shape[0], c.shape[0]
    d_nll = torch.full((N,), 1.0 / N, device=cuda)
    stats = torch.zeros(3, dtype=torch.int64, device=cuda)
    with m._ext.backward_options(token_order=order, g_precision=precision):
        dE, dC, _ = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, m.FILTER_LOG_EPS, True, True, False,
                                    tile_stats=stats)
    torch.cuda.synchronize()
    tm_np, lse_np = tm.cpu().numpy(), lse.cpu().numpy()
    tt = t.cpu().numpy()
    dn = np.full(N, 1.0 / N)
    perm = _sorted_rows(tt, dn, V) if order == "sorted" else np.arange(N)
    keep = O.keep_mask(tm_np[:, perm], lse_np[perm], tt[perm], dn[perm], eps=np.float32(m.FILTER_LOG_EPS))
    # the kernel's comparison is fp32 (tile_max - lse >= eps): replay it in fp32
    hot = (tm_np - lse_np[None, :]).astype(np.float32) >= np.float32(m.FILTER_LOG_EPS)
    kept, total, kept_in = stats.tolist()
    keep_in = O.keep_mask(tm_np, lse_np, tt, dn, eps=np.float32(m.FILTER_LOG_EPS))
    assert total == keep.size
    assert kept == int(keep.sum()), (kept, int(keep.sum()))
    assert kept_in == int(keep_in.sum()), (kept_in, int(keep_in.sum()))
    assert 0 < kept < total
    if order == "sorted":  # the peaked Zipf case is the one the sorted order is for
        assert kept * 10 <= kept_in * 9, (kept, kept_in)
    print(f"filter ({order} order): kept {kept}/{total} tiles (skip {1 - kept / total:.3f}); "
          f"hot fraction {hot.mean():.4f}")
    ee, cc = f64(e), f64(c)
    fE_p, fC, _ = O.grads_filtered(ee[perm], cc, tt[perm], keep, 128, 128, None, d_nll=dn[perm])
    fE = np.empty_like(fE_p)
    fE[perm] = fE_p
    emu = [O.rel_fro(f64(dE), fE), O.rel_fro(f64(dC), fC)]
    emu_r = [O.rel_fro(f64(dE), O.round_bf16(fE)), O.rel_fro(f64(dC), O.round_bf16(fC))]
    print(f"kernel vs filter emulation ({precision or 'default'} G): dE {emu[0]:.3e} dC {emu[1]:.3e}; "
          f"vs the emulation rounded to bf16: dE {emu_r[0]:.3e} dC {emu_r[1]:.3e}")
    assert emu[0] < 2e-2 and emu[1] < 2e-2  # bf16 tolerance against the same kept-tile set
    if precision == "pair":
        assert emu_r[0] <= 1e-3 and emu_r[1] <= 1e-3
    # The 2^-12 filter itself drops softmax mass; against the dense gradient the error must be
    # no larger than the reference's own 32x32 filter produces on the same inputs.
    dense = O.grads(ee, cc, tt, None, "mean")
    errs = [O.rel_fro(f64(x), y) for x, y in zip((dE, dC), dense[:2])]
    ref_keep = O.reference_keep_mask(ee, cc, tt)
    rE, rC, _ = O.grads_filtered(ee, cc, tt, ref_keep, 32, 32, None, d_nll=np.full(N, 1.0 / N))
    ref_errs = [O.rel_fro(rE, dense[0]), O.rel_fro(rC, dense[1])]
    print(f"filtered vs dense: dE {errs[0]:.3e} dC {errs[1]:.3e}; reference filter: "
          f"dE {ref_errs[0]:.3e} dC {ref_errs[1]:.3e}")
    assert errs[0] <= ref_errs[0] + 2e-3 and errs[1] <= ref_errs[1] + 2e-3


@pytest.mark.parametrize("name", ["c2", "c4"])
def test_filter_on_near_uniform_softmax(m, cuda, name):
    """c2 / c4 row slices (N = 128 rows, full D and V) with the 2^-12 filter ON: the softmax
    is near uniform there (c ~ N(0, 0.02^2)), every p is close to the threshold, and the
    filter drops most of the mass of G outside the targets.  The filtered dE / dC / dBias
    against the dense float64 gradient must be no worse than the reference's own 32 x 32
    filter on the same rows (cce.metal:191-204) + 2e-3; both errors are printed."""
    w = workloads.make(name, device="cuda", scale=1 / 32)
    e, c, t, b = w["e"], w["c"], w["targets"], w["bias"]
    red = w["reduction"]
    _, dE, dC, dB = run(m, e, c, t, b, red, -100, filter_eps=m.FILTER_LOG_EPS)
    fs = m.last_filter_stats()
    ee = f64(e).reshape(-1, w["D"])
    cc, bb = f64(c), f64(b)
    tt = t.cpu().numpy().reshape(-1)
    dense = O.grads(ee, cc, tt, bb, red)
    valid = O.valid_mask(tt, -100)
    ref_keep = O.reference_keep_mask(ee, cc, tt, bb)
    ref = O.grads_filtered(ee, cc, tt, ref_keep, 32, 32, bb, d_nll=O.upstream(valid, red))
    got = [dE.reshape(-1, w["D"]), dC] + ([dB] if b is not None else [])
    names = ["dE", "dC", "dBias"][:len(got)]
    print(f"{name} slice N={ee.shape[0]}: kept {fs['kept']}/{fs['total']} tiles of 128x128 "
          f"(reference 32x32 keeps {int(ref_keep.sum())}/{ref_keep.size})")
    for nm, x, d, r in zip(names, got, dense, ref):
        err, rerr = O.rel_fro(f64(x), d), O.rel_fro(r, d)
        print(f"{name} {nm}: filtered vs dense {err:.3e}; reference filter vs dense {rerr:.3e}")
        assert err <= rerr + 2e-3, (nm, err, rerr)


def test_filter_disabled_is_dense(m, cuda):
    e, c, t = _peaked(cuda, N=256, V=4096)
    tm, _, _, lse, _ = m._ext.forward(e, c, t, None, -100)
    d_nll = torch.full((256,), 1.0 / 256, device=cuda)
    stats = torch.zeros(3, dtype=torch.int64, device=cuda)
    m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, None, True, True, False, tile_stats=stats)
    kept, total, kept_in = stats.tolist()
    assert kept == total == kept_in == 2 * 32


SPLITS = {"one": {}, "chunks": dict(max_chunk_tiles=32), "passes": dict(max_g_tiles=1),
          "both": dict(max_chunk_tiles=32, max_g_tiles=8)}


@pytest.mark.parametrize("split", ["one", "chunks", "passes"])
def test_forward_zero_fill_and_backward_into_zeroed_dc(m, cuda, split):
    """cce_forward_ex fills its buffer with zeros (every byte, whatever it held) and leaves
    the forward's outputs unchanged; cce_backward_ex with CCE_BWD_DC_ZEROED writes only the
    kept vocabulary tiles' dC rows into it, and the result equals the ordinary backward's
    dC bit for bit (filtered, so that most rows are left untouched); in one pass, in
    vocabulary chunks of 32 tiles, or in passes of the smallest G scratch.  The autograd
    op gives the same dC with the fill in its forward (opt-in) and without it."""
    with m._ext.backward_options(**SPLITS[split]):
        _zero_fill_case(m, cuda, split)


def _zero_fill_case(m, cuda, split):
    e, c, t = _peaked(cuda, N=384, D=256, V=9000, seed=13)
    plain = m._ext.forward(e, c, t, None, -100)
    buf = torch.full_like(c, float("nan"))
    outs = m._ext.forward(e, c, t, None, -100, zero_out=buf)
    torch.cuda.synchronize()
    assert int((buf.view(torch.int16) != 0).sum()) == 0
    for x, y in zip(outs, plain):
        assert torch.equal(x, y)
    tm, _, _, lse, _ = plain
    d_nll = torch.full((384,), 1.0 / 384, device=cuda)
    _, dC_ref, _ = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, m.FILTER_LOG_EPS, True, True, False)
    stats = torch.zeros(3, dtype=torch.int64, device=cuda)
    _, dC, _ = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, m.FILTER_LOG_EPS, True, True, False,
                               tile_stats=stats, dc_zeroed=buf)
    torch.cuda.synchronize()
    assert dC.data_ptr() == buf.data_ptr()
    kept, total, _ = stats.tolist()
    assert 0 < kept < total
    assert torch.equal(dC.view(torch.int16), dC_ref.view(torch.int16))
    # the autograd path, with the fill in the forward (opt-in) or not (the default):
    # the same gradients as through the ordinary backward
    for fill in ("forward", "backward"):
        e2 = e.detach().clone().requires_grad_(True)
        c2 = c.detach().clone().requires_grad_(True)
        with m._ext.backward_options(**SPLITS[split], dc_zero_fill=fill):
            m.linear_cross_entropy(e2, c2, t).backward()
        assert torch.equal(c2.grad.view(torch.int16), dC_ref.view(torch.int16)), fill


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("filtered", [False, True])
@pytest.mark.parametrize("split", ["one", "passes", "both"])
def test_host_and_device_pass_schedules_agree(m, cuda, dtype, filtered, split):
    """The host waits for the compaction's pass count and launches only the passes
    (and the dC geometry) the data needs; CCE_BWD_DEVICE_PASSES launches the dense
    worst case and lets the device skip the rest.  Same kernels, same plan: the
    gradients agree bit for bit, in one pass, in several passes, and in several
    passes of several vocabulary chunks."""
    N, D, V = 300, 264, 9000
    if filtered:
        e, c, t = _peaked(cuda, N=N, D=D, V=V, dtype=dtype, seed=17)
    else:
        e, c, t = normal_case(N, D, V, dtype, cuda, seed=17, std=0.05)
    t[5] = -100
    b = (torch.randn(V, device=cuda) * 0.1).to(dtype)
    feps = m.FILTER_LOG_EPS if filtered else None
    opts = {"one": {}, "passes": {"max_g_tiles": 8}, "both": {"max_g_tiles": 8, "max_chunk_tiles": 32}}[split]
    with m._ext.backward_options(**opts):
        host = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
    with m._ext.backward_options(passes="device", **opts):
        dev = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    for x, y in zip(host[1:], dev[1:]):
        assert torch.equal(x.view(bits), y.view(bits))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("filtered", [False, True])
@pytest.mark.parametrize("de_sums", ["narrow", "wide"])
@pytest.mark.parametrize("split", ["chunks", "passes", "both"])
def test_vocabulary_chunks(m, cuda, dtype, filtered, de_sums, split):
    """Several vocabulary chunks (max_chunk_tiles 32), several passes of the smallest G
    scratch (max_g_tiles), or both: dE carried in fp32 between passes, dC / dBias final
    per pass; equal to the one-pass result and the oracle.  Both sum geometries, for dE
    and dC together; D = 264 leaves a ragged column slice in each."""
    N, D, V = 300, 264, 9000
    if filtered:
        e, c, t = _peaked(cuda, N=N, D=D, V=V, dtype=dtype, seed=11)
    else:
        e, c, t = normal_case(N, D, V, dtype, cuda, seed=11, std=0.05)
    t[7] = -100
    gb = torch.Generator(device=cuda).manual_seed(12)  # seeded: the chunked-vs-single error depends on the data
    b = (torch.randn(V, generator=gb, device=cuda) * 0.1).to(dtype)
    feps = m.FILTER_LOG_EPS if filtered else None
    with m._ext.backward_options(de_sums=de_sums, dc_sums=de_sums):
        one = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
    with m._ext.backward_options(de_sums=de_sums, dc_sums=de_sums, **SPLITS[split]):
        assert m._ext.workspace_size(e, c, True, True, True) < m._ext.workspace_size(e, c, True, True, True, 0, 0) \
            or split == "chunks"
        many = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
    np.testing.assert_allclose(f64(many[0]), f64(one[0]), rtol=1e-6)
    tol_same = 1e-5 if dtype == torch.float32 else 1e-2  # fp32 partial sums per chunk reassociate
    for x, y, name in zip(many[1:], one[1:], ("dE", "dC", "dBias")):
        err = O.rel_fro(f64(x), f64(y))
        print(f"chunked vs single {name}: {err:.2e}")
        assert err < tol_same, (name, err)
    if filtered:
        return
    rE, rC, rB = O.grads(f64(e), f64(c), t.cpu().numpy(), f64(b), "sum")
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for got, r, name in zip(many[1:], (rE, rC, rB), ("dE", "dC", "dBias")):
        err = O.rel_fro(f64(got), r)
        print(f"chunked vs oracle {name}: {err:.2e}")
        assert err < tol, (name, err)


DE_SPLITS = {"one": {}, "passes": dict(max_g_tiles=1), "chunks": dict(max_chunk_tiles=32)}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("split", ["one", "passes", "chunks"])
@pytest.mark.parametrize("order", ["sorted", "input"])
def test_de_pieces_match_whole_tasks(m, cuda, dtype, split, order):
    """With few dE tasks (here 3 token blocks x 2 D slices for 256 workgroups) the narrow
    dE sums cut each task into pieces along its kept tiles, whose fp32 sums a finishing
    kernel adds in order: dE equals the whole tasks' (CCE_BWD_DE_WHOLE_TASKS) to the
    fp32 sums' reassociation, in one pass (written directly), in passes and chunks (the
    fp32 carry's store / add / finish modes), with the rows sorted by target tile or in
    input order; repeated runs are equal bit for bit, and dC / dBias do not change."""
    N, D, V = 300, 264, 9000
    e, c, t = normal_case(N, D, V, dtype, cuda, seed=31, std=0.05)
    t[5] = -100
    gb = torch.Generator(device=cuda).manual_seed(32)
    b = (torch.randn(V, generator=gb, device=cuda) * 0.1).to(dtype)
    feps = m.FILTER_LOG_EPS
    with m._ext.backward_options(token_order=order, **DE_SPLITS[split]):
        pieces = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
        again = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
    with m._ext.backward_options(token_order=order, de_tasks="whole", **DE_SPLITS[split]):
        whole = run(m, e, c, t, b, reduction="sum", filter_eps=feps)
    for x, y in zip(pieces[1:], again[1:]):
        assert torch.equal(x, y)
    err = O.rel_fro(f64(pieces[1]), f64(whole[1]))
    print(f"{dtype} {split} {order}: dE pieces vs whole {err:.2e}")
    assert err < (1e-5 if dtype == torch.float32 else 2e-3), err
    assert torch.equal(pieces[2], whole[2]) and torch.equal(pieces[3], whole[3])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_de_pieces_two_per_task(m, cuda, dtype):
    """96 dE tasks (32 token blocks x 3 D slices, the last one ragged) for 256 workgroups:
    each task in 2 pieces, 192 slots, the finishing kernel's grid reaching all 96 tasks.
    dE equals the whole tasks' to the fp32 sums' reassociation and repeats bit for bit."""
    N, D, V = 4000, 520, 9000
    e, c, t = normal_case(N, D, V, dtype, cuda, seed=33, std=0.05)
    feps = m.FILTER_LOG_EPS
    pieces = run(m, e, c, t, None, reduction="sum", filter_eps=feps)
    again = run(m, e, c, t, None, reduction="sum", filter_eps=feps)
    with m._ext.backward_options(de_tasks="whole"):
        whole = run(m, e, c, t, None, reduction="sum", filter_eps=feps)
    assert torch.equal(pieces[1], again[1]) and torch.equal(pieces[2], again[2])
    err = O.rel_fro(f64(pieces[1]), f64(whole[1]))
    print(f"{dtype}: dE two pieces vs whole {err:.2e}")
    assert err < (1e-5 if dtype == torch.float32 else 2e-3), err
    assert torch.equal(pieces[2], whole[2])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_de_pieces_of_tasks_past_the_grid(m, cuda, dtype):
    """288 dE tasks (32 token blocks x 9 D slices) for 256 workgroups: one launch runs a
    whole task per workgroup, a second the 32 tasks past the grid cut into 8 pieces each
    (the last owners, with the fewest kept tiles), and the finishing kernel adds those.
    dE equals the whole tasks' (two rounds on some workgroups) to the fp32 sums'
    reassociation and repeats bit for bit; dC is unchanged."""
    if torch.cuda.get_device_properties(cuda).multi_processor_count != 256:
        pytest.skip("the task counts are laid out for a 256-workgroup grid")
    N, D, V = 4096, 2304, 9000
    e, c, t = normal_case(N, D, V, dtype, cuda, seed=35, std=0.05)
    feps = m.FILTER_LOG_EPS
    pieces = run(m, e, c, t, None, reduction="sum", filter_eps=feps)
    again = run(m, e, c, t, None, reduction="sum", filter_eps=feps)
    with m._ext.backward_options(de_tasks="whole"):
        whole = run(m, e, c, t, None, reduction="sum", filter_eps=feps)
    assert torch.equal(pieces[1], again[1]) and torch.equal(pieces[2], again[2])
    err = O.rel_fro(f64(pieces[1]), f64(whole[1]))
    print(f"{dtype}: dE overflow pieces vs whole {err:.2e}")
    assert err < (1e-5 if dtype == torch.float32 else 2e-3), err
    assert torch.equal(pieces[2], whole[2])


@pytest.mark.parametrize("sizing", ["exact", "pair", "least"])
def test_rounded_once_g_workspace_sizes(m, cuda, sizing):
    """A bf16 backward with the filter on keeps G rounded once in 32 KiB tile slots.
    Given a workspace of exactly cce_backward_workspace_size_flags's size for the
    smallest passes, the larger one of the hi / lo pair's 64 KiB slots for the same
    passes (cce_backward_workspace_size_ex: the plan then takes larger passes), or the
    least size the call accepts (named by its error), the backward keeps the same tiles
    and its gradients equal the default workspace's to the passes' fp32 reassociation
    (2.3e-5, 7.8e-6 and 3.2e-5 relative for dE; dC and dBias, final per pass, bit for
    bit)."""
    import ctypes
    import re
    ext = m._ext
    lib = ext.lib()
    N, D, V = 300, 264, 9000
    e, c, t = _peaked(cuda, N=N, D=D, V=V, seed=11)
    t = t.to(torch.int64).contiguous()
    gb = torch.Generator(device=cuda).manual_seed(12)
    b = (torch.randn(V, generator=gb, device=cuda) * 0.1).to(torch.bfloat16)
    tm, _, _, lse, _ = ext.forward(e, c, t, b, -100)
    d_nll = torch.full((N,), 1.0 / N, device=cuda)
    eps = m.FILTER_LOG_EPS
    st0 = torch.zeros(3, dtype=torch.int64, device=cuda)
    # the least workspace has no room for the sorted token order: its reference keeps
    # the tiles of the input order's token blocks
    with ext.backward_options(token_order="input" if sizing == "least" else None):
        ref = ext.backward(e, c, t, lse, tm, d_nll, b, -100, eps, True, True, True, tile_stats=st0)
    exact = lib.cce_backward_workspace_size_flags(2, N, D, V, 1, 1, 1, 1, 0, ctypes.c_float(eps), 0)
    pair = lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, 1, 0)
    assert 0 < exact < pair
    dE, dC, dB = torch.empty_like(e), torch.empty_like(c), torch.empty_like(b)
    st = torch.zeros(3, dtype=torch.int64, device=cuda)
    stream = torch.cuda.current_stream(cuda).cuda_stream

    def call(ws, nbytes):
        return lib.cce_backward_ex(2, ext._ptr(e), ext._ptr(c), ext._ptr(b), ext._ptr(t), -100, 1, N, D, V,
                                   ext._ptr(lse), ext._ptr(tm), ext._ptr(d_nll), ctypes.c_float(eps), ext._ptr(dE),
                                   ext._ptr(dC), ext._ptr(dB), ext._ptr(ws), ctypes.c_size_t(nbytes), ext._ptr(st),
                                   0, 0, ctypes.c_void_p(stream))

    if sizing == "least":
        small = torch.empty((256,), dtype=torch.uint8, device=cuda)
        assert call(small, 256) == ext.CCE_ERR_WORKSPACE  # refused before any device work
        nbytes = int(re.search(rb"at least (\d+)", lib.cce_last_error()).group(1))
        assert 0 < nbytes <= exact
    else:
        nbytes = exact if sizing == "exact" else pair
    ws = torch.empty((nbytes,), dtype=torch.uint8, device=cuda)
    assert call(ws, nbytes) == ext.CCE_OK, lib.cce_last_error()
    torch.cuda.synchronize()
    print(f"{sizing}: workspace {nbytes} bytes, tiles {st.tolist()} (default {st0.tolist()})")
    assert torch.equal(st, st0)
    for x, y, name in zip((dE, dC, dB), ref, ("dE", "dC", "dBias")):
        err = O.rel_fro(f64(x), f64(y))
        print(f"{sizing} vs default {name}: {err:.2e}")
        assert err < 1e-3, (name, err)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("case", ["skewed", "uniform"])
def test_dc_geometry_chosen_per_pass(m, cuda, case, dtype):
    """With the filter on the compaction picks the dC sums' geometry per pass: narrow
    when the largest owner's kept blocks times the grid exceed the pass's kept tiles
    times the 512-column slices (Zipf targets: vocabulary tile 0 keeps every token
    block), else wide (uniform targets with a peaked softmax: each tile keeps at most
    a few blocks).  The default run equals both forced geometries bit for bit (both sum
    an owner's tiles in the same order with the same instructions)."""
    if case == "skewed":
        e, c, t = _peaked(cuda, N=4096, D=512, V=16000, dtype=dtype, seed=21)
    else:
        N, D, V = 1024, 2048, 32000
        g = torch.Generator(device=cuda).manual_seed(22)
        c = (torch.randn((V, D), generator=g, device=cuda) * 0.02).to(dtype)
        t = torch.randint(0, V, (N,), generator=g, device=cuda)
        ct = c.float()[t]
        e = (0.5 * torch.randn((N, D), generator=g, device=cuda) + 12.0 * ct / ct.pow(2).sum(1, keepdim=True)).to(
            dtype)
    N = e.shape[0]
    tm, _, _, lse, _ = m._ext.forward(e, c, t, None, -100)
    d_nll = torch.full((N,), 1.0 / N, device=cuda)
    outs = {}
    for geo in (None, "wide", "narrow"):
        with m._ext.backward_options(dc_sums=geo):
            outs[geo] = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, m.FILTER_LOG_EPS, True, True, False)
    torch.cuda.synchronize()
    for geo in ("wide", "narrow"):
        assert torch.equal(outs[None][0], outs[geo][0]), ("dE", geo)
        assert torch.equal(outs[None][1], outs[geo][1]), ("dC", geo)
    assert float(outs[None][1].float().abs().sum()) > 0


def test_many_passes_pass_table_in_global_memory(m, cuda):
    """The smallest G scratch (2 tiles per 128-row block) on a dense problem runs one pass
    per vocabulary tile: 157 passes of 64 token blocks, more (pass, block) slot starts
    than the compaction holds in LDS.  Equal to the one-pass result (fp32), and
    <E, dE> = <C, dC> (both equal sum G * S without bias)."""
    N, D, V = 8192, 64, 20000
    e, c, t = normal_case(N, D, V, torch.float32, cuda, seed=17, std=0.05)
    t[::97] = -100
    one = run(m, e, c, t, reduction="sum", filter_eps=None)
    with m._ext.backward_options(max_g_tiles=1):
        many = run(m, e, c, t, reduction="sum", filter_eps=None)
    for x, y, name in zip(many[1:3], one[1:3], ("dE", "dC")):
        err = O.rel_fro(f64(x), f64(y))
        print(f"157 passes vs one pass {name}: {err:.2e}")
        assert err < 1e-5, (name, err)
    ip_e = float((e.double() * many[1].double()).sum())
    ip_c = float((c.double() * many[2].double()).sum())
    assert abs(ip_e - ip_c) <= 1e-4 * max(abs(ip_e), abs(ip_c))
    assert int((many[1][::97].abs() > 0).sum()) == 0  # ignored rows


# --------------------------------------------------- benchmark configurations
def _cfg_check(m, name, scale, tol_grad):
    w = workloads.make(name, device="cuda", scale=scale)
    e, c, t, b = w["e"], w["c"], w["targets"], w["bias"]
    red = w["reduction"]
    loss, dE, dC, dB = run(m, e, c, t, b, red, -100, filter_eps=None)
    ee = f64(e).reshape(-1, w["D"])
    cc = f64(c)
    tt = t.cpu().numpy().reshape(-1)
    bb = f64(b)
    ref = O.linear_cross_entropy(ee, cc, tt, bb, red)
    np.testing.assert_allclose(f64(loss).reshape(-1), np.ravel(ref), rtol=1e-3, atol=1e-5)
    rE, rC, rB = O.grads(ee, cc, tt, bb, red)
    errs = {"dE": O.rel_fro(f64(dE).reshape(-1, w["D"]), rE), "dC": O.rel_fro(f64(dC), rC)}
    if b is not None:
        errs["dBias"] = O.rel_fro(f64(dB), rB)
    print(name, {k: f"{v:.3e}" for k, v in errs.items()})
    for k, v in errs.items():
        assert v < tol_grad, (k, v)


def test_config_c1_fp32_full(m, cuda):
    _cfg_check(m, "c1", 1.0, 1e-3)


def test_config_c2_slice(m, cuda):
    _cfg_check(m, "c2", 1 / 16, 2e-2)


def test_config_c4_slice_bias(m, cuda):
    _cfg_check(m, "c4", 1 / 32, 2e-2)


def test_config_c3_full_size_properties(m, cuda):
    """c3 at full size: loss is ~0 (target logit ~40, F2 degeneracy), lse of sampled rows matches the oracle."""
    w = workloads.make("c3", device="cuda")
    e = w["e"].reshape(-1, w["D"])
    c, t = w["c"], w["targets"].reshape(-1)
    tm, ts, ntl, lse, nll = m._ext.forward(e, c, t, None, -100)
    rows = torch.arange(0, w["N"], 997, device=cuda)
    ref_nll, ref_lse, _ = O.per_token(f64(e[rows]), f64(c), t[rows].cpu().numpy())
    ulp = np.spacing(np.float32(np.abs(ref_lse).max()))
    np.testing.assert_allclose(f64(lse[rows]), ref_lse, rtol=0, atol=8 * ulp)
    assert np.abs(f64(nll[rows]) - ref_nll).max() < 16 * ulp
    e2 = e.detach().clone().requires_grad_(True)
    c2 = c.detach().clone().requires_grad_(True)
    loss = m.linear_cross_entropy(e2, c2, t)
    loss.backward()
    torch.cuda.synchronize()
    kept, total = m.last_tile_stats()
    print(f"c3: loss {loss.item():.3e} kept {kept}/{total} skip {1 - kept / total:.4f}")
    assert 0 < kept < total and torch.isfinite(e2.grad).all() and torch.isfinite(c2.grad).all()


def test_config_c5_full_size_properties(m, cuda):
    """c5 at full size (N=32768, D=8192, V=128256, bf16, reduction sum, the last 410
    positions of each sequence ignored): lse / nll of sampled rows against float64
    (computed with torch on the device in vocabulary chunks: a host float64 copy of C
    would be 8.4 GB), within 32 / 48 ulp; the backward keeps 0 < kept < total tiles,
    gives finite gradients and exactly zero dE rows for the ignored positions."""
    w = workloads.make("c5", device="cuda")
    N, D = w["N"], w["D"]
    e = w["e"].reshape(N, D)
    c, t = w["c"], w["targets"].reshape(N)
    assert w["reduction"] == "sum"
    tm, ts, ntl, lse, nll = m._ext.forward(e, c, t, None, -100)
    rows = torch.arange(5, N, 1021, device=cuda)
    rows = rows[t[rows] != -100]
    er = e[rows].double()
    lse_ref = torch.full((len(rows),), -math.inf, dtype=torch.float64, device=cuda)
    for v0 in range(0, c.shape[0], 16384):
        lse_ref = torch.logaddexp(lse_ref, torch.logsumexp(er @ c[v0:v0 + 16384].double().T, dim=1))
    tgt = (er * c[t[rows]].double()).sum(1)
    # fp32 accumulation of 8192-term dot products (target logits ~40): measured up to
    # 12 ulp of lse (1.1e-6 relative); bounds 32 / 48 ulp (c3, D = 4096: 8 / 16)
    ulp = np.spacing(np.float32(lse_ref.abs().max().item()))
    np.testing.assert_allclose(f64(lse[rows]), f64(lse_ref), rtol=0, atol=32 * ulp)
    assert np.abs(f64(nll[rows]) - f64(lse_ref - tgt)).max() < 48 * ulp
    del tm, ts, ntl, lse, nll
    e2 = e.detach().clone().requires_grad_(True)
    c2 = c.detach().clone().requires_grad_(True)
    loss = m.linear_cross_entropy(e2, c2, t, reduction="sum")
    loss.backward()
    torch.cuda.synchronize()
    kept, total = m.last_tile_stats()
    print(f"c5: loss {loss.item():.3e} kept {kept}/{total} skip {1 - kept / total:.4f}")
    assert 0 < kept < total and torch.isfinite(e2.grad).all() and torch.isfinite(c2.grad).all()
    ign = t == -100
    assert int(ign.sum()) == 8 * 410
    assert int((e2.grad[ign].view(torch.int16) != 0).sum()) == 0


def test_config_c3_full_size_moderate_peak_sampled_grads(m, cuda):
    """c3 at full size (N=8192, D=4096, V=128256, bf16, filter on) with the target boost
    lowered from 40 to 12 so the softmax is peaked but the gradients are not ~0.

    Checks, with the filter on:
      * the kept-tile count equals the filter predicate evaluated on the CPU from the
        kernel's own fp32 tile_max / lse (exact);
      * dE on sampled rows against float64 G_r . C restricted to the kept tiles
        (2e-2 relative Frobenius, bf16);
      * dC on sampled vocabulary rows (hot Zipf targets, untargeted and untouched rows)
        against float64 G[:, v]^T . E restricted to the kept tiles, normalised by the
        kernel's lse (itself checked against float64 on sampled rows, 8 ulp);
      * <E, dE> = <C, dC> (both equal sum G * S; no bias) to 5e-3 relative.
    """
    w = workloads.make("c3", device="cuda", target_boost=12.0)
    N, D, V = w["N"], w["D"], w["V"]
    e = w["e"].reshape(N, D)
    c, t = w["c"], w["targets"].reshape(N)
    tm, ts, ntl, lse, nll = m._ext.forward(e, c, t, None, -100)
    e2 = e.detach().clone().requires_grad_(True)
    c2 = c.detach().clone().requires_grad_(True)
    loss = m.linear_cross_entropy(e2, c2, t)
    loss.backward()
    torch.cuda.synchronize()
    fs = m.last_filter_stats()
    kept, total = fs["kept"], fs["total"]
    dE, dC = e2.grad, c2.grad

    # kept-tile set, from the kernel's fp32 statistics (float32 comparison, as on the GPU),
    # over the token blocks the backward used: with this peaked Zipf input the rows
    # grouped by target tile keep far fewer tiles than the input-order blocks, so the
    # backward picks them
    tn = t.cpu().numpy()
    d_nll = np.full(N, np.float32(1.0 / N), dtype=np.float32)
    tm_np, lse_np = tm.cpu().numpy(), lse.cpu().numpy()
    keep_in = O.keep_mask(tm_np, lse_np, tn, d_nll)
    perm = _sorted_rows(tn, d_nll, V) if fs["sorted_rows"] else np.arange(N)
    keep = O.keep_mask(tm_np[:, perm], lse_np[perm], tn[perm], d_nll[perm])
    blk = np.empty(N, dtype=np.int64)
    blk[perm] = np.arange(N) // 128  # token block of every row in the order used
    print(f"c3 boost 12: loss {loss.item():.4f} kept {kept}/{total} (cpu predicate: order used "
          f"{int(keep.sum())}, input order {int(keep_in.sum())}, rows grouped {fs['sorted_rows']})")
    assert int(keep.sum()) == kept and total == keep.size and fs["kept_input_order"] == int(keep_in.sum())
    assert fs["sorted_rows"] and kept * 10 <= int(keep_in.sum()) * 9

    cc = f64(c)
    lse64 = f64(lse)
    g = 1.0 / N

    # dE rows
    rows = np.array([0, 1, 127, 128, 4095, 5000, 8191])
    S = O.logits(f64(e[rows]), cc)
    ref_lse = O.logsumexp_rows(S)
    ulp = np.spacing(np.float32(np.abs(ref_lse).max()))
    np.testing.assert_allclose(lse64[rows], ref_lse, rtol=0, atol=8 * ulp)
    G = g * np.exp(S - ref_lse[:, None])
    G[np.arange(len(rows)), tn[rows]] -= g
    mask = np.repeat(keep[:, blk[rows]], 128, axis=0)[:V].T  # [rows, V]
    refE = np.where(mask, G, 0.0) @ cc
    errE = O.rel_fro(f64(dE[rows]), refE)

    # dC vocabulary rows: the hottest targets, a mid-frequency one, an untargeted one, the last
    ee = f64(e)
    counts = np.bincount(tn, minlength=V)
    untargeted = int(np.nonzero(counts == 0)[0][len(np.nonzero(counts == 0)[0]) // 2])
    vs = np.array(sorted({0, 1, 2, 7, 63, 128, 1000, untargeted, V - 1}))
    Sc = ee @ cc[vs].T  # [N, len(vs)]
    Gc = g * np.exp(Sc - lse64[:, None])
    Gc -= g * (tn[:, None] == vs[None, :])
    maskc = keep[vs // 128][:, blk].T  # [N, len(vs)]
    refC = np.where(maskc, Gc, 0.0).T @ ee
    errC = O.rel_fro(f64(dC[vs]), refC)

    ip_e = float((e.double() * dE.double()).sum())
    ip_c = float((c.double() * dC.double()).sum())
    rel_ip = abs(ip_e - ip_c) / max(abs(ip_e), abs(ip_c))
    print(f"c3 boost 12: dE rows {errE:.3e}  dC rows {errC:.3e}  <E,dE> {ip_e:.6e} <C,dC> {ip_c:.6e} ({rel_ip:.2e})")
    assert errE < 2e-2 and errC < 2e-2
    assert rel_ip < 5e-3
    assert torch.isfinite(dE).all() and torch.isfinite(dC).all()


# ----------------------------------------------- API of the research tree (f1)
def test_linear_cross_entropy_module_with_shift(m, cuda):
    """LinearCrossEntropy (reference/__init__.py:88-118) with shift=1 on [B, T, D] inputs,
    against the float64 oracle (reference/_reference.py:15-17 shift): loss, dE, dC."""
    g = torch.Generator(device=cuda).manual_seed(41)
    B, T, D, V = 3, 50, 64, 3000
    e = torch.randn((B, T, D), generator=g, device=cuda).requires_grad_(True)
    c = (torch.randn((V, D), generator=g, device=cuda) * 0.1).requires_grad_(True)
    t = torch.randint(0, V, (B, T), generator=g, device=cuda)
    t[:, -3:] = -100
    crit = m.LinearCrossEntropy(reduction="mean", shift=1, filter_eps=None)
    loss = crit(e, c, t)
    loss.backward()
    ref = O.linear_cross_entropy(f64(e), f64(c), t.cpu().numpy(), None, "mean", shift=1)
    np.testing.assert_allclose(float(loss), ref, rtol=1e-5)
    es = f64(e)[:, :-1, :].reshape(-1, D)
    ts = t.cpu().numpy()[:, 1:].reshape(-1)
    rE, rC, _ = O.grads(es, f64(c), ts, None, "mean")
    gE = f64(e.grad)
    assert (gE[:, -1, :] == 0).all()  # the dropped last position gets no gradient
    assert O.rel_fro(gE[:, :-1, :].reshape(-1, D), rE) < 1e-3
    assert O.rel_fro(f64(c.grad), rC) < 1e-3
    # compute_all_grads=False: the frozen-head mode -- no gradient for c
    c.grad = None
    e.grad = None
    m.LinearCrossEntropy(shift=1, compute_all_grads=False, filter_eps=None)(e, c, t).backward()
    assert c.grad is None and O.rel_fro(f64(e.grad)[:, :-1, :].reshape(-1, D), rE) < 1e-3


@pytest.mark.parametrize("compute_all_grads", [False, True])
def test_cut_cross_entropy_gradients(m, cuda, compute_all_grads):
    """cut_cross_entropy(..., compute_all_grads) (csrc/bindings.cpp:15-56): dE always; dC and
    dBias only when asked for (the reference returns zeros for them otherwise)."""
    e, c, t = normal_case(64, 128, 4096, torch.float32, cuda, seed=43, std=0.1)
    b = (torch.randn(4096, device=cuda) * 0.1).requires_grad_(True)
    t[5] = -100
    e.requires_grad_(True)
    c.requires_grad_(True)
    loss = m.cut_cross_entropy(e, c, t, b, "sum", -100, compute_all_grads)
    loss.backward()
    rE, rC, rB = O.grads(f64(e), f64(c), t.cpu().numpy(), f64(b), "sum")
    # the default filter drops sub-threshold entries: bounded by its own error here
    assert O.rel_fro(f64(e.grad), rE) < 2e-2
    if compute_all_grads:
        assert O.rel_fro(f64(c.grad), rC) < 2e-2 and O.rel_fro(f64(b.grad), rB) < 5e-2
    else:
        assert c.grad is None and b.grad is None


def test_linear_cross_entropy_compute_all_grads_keyword(m, cuda):
    """The research API's keywords (reference/__init__.py:22-33): compute_all_grads=False
    leaves c and bias without gradient even when they require it; True and the default
    (None: what autograd asks for) give the same dC / dBias."""
    e, c, t = normal_case(40, 64, 1000, torch.float32, cuda, seed=44, std=0.1)
    b = torch.randn(1000, device=cuda) * 0.1
    outs = {}
    for cag in (None, True, False):
        ee, cc, bb = (x.detach().clone().requires_grad_(True) for x in (e, c, b))
        m.linear_cross_entropy(ee, cc, t, bb, "mean", -100, 0, False, "auto", cag, filter_eps=None).backward()
        outs[cag] = (ee.grad, cc.grad, bb.grad)
    assert outs[False][1] is None and outs[False][2] is None
    for k in range(3):
        assert torch.equal(outs[None][k], outs[True][k])
    assert torch.equal(outs[False][0], outs[True][0])
    with pytest.raises(ValueError, match="impl"):
        m.linear_cross_entropy(e, c, t, impl="metal")


def test_train_validation_call_pattern(m, cuda):
    """The reference's own caller examples/train_validation.py:65-72 runs unchanged:
    linear_cross_entropy(x, head.weight, targets, compute_all_grads=True, reduction="mean")
    on [B, T, D] hidden states; its loss and head gradient equal the materialised path's
    (loss_reference, :57-63) -- here impl="reference", the reference's own comparison."""
    g = torch.Generator(device=cuda).manual_seed(45)
    B, T, D, V = 4, 33, 64, 512
    head = torch.nn.Linear(D, V, bias=False).to(cuda)
    x = torch.randn((B, T, D), generator=g, device=cuda, requires_grad=True)
    tokens = torch.randint(0, V, (B, T + 1), generator=g, device=cuda)
    targets = tokens[:, 1:]
    loss = m.linear_cross_entropy(x, head.weight, targets, compute_all_grads=True, reduction="mean")
    loss.backward()
    gx, gw = x.grad.clone(), head.weight.grad.clone()
    x.grad, head.weight.grad = None, None
    ref = m.linear_cross_entropy(x, head.weight, targets, impl="reference", reduction="mean")
    ref.backward()
    assert abs(float(loss) - float(ref)) <= 1e-5 * abs(float(ref))
    assert O.rel_fro(f64(gx), f64(x.grad)) < 2e-2 and O.rel_fro(f64(gw), f64(head.weight.grad)) < 2e-2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_reference_layout_statistics_and_glue(m, cuda, dtype):
    """cce_forward_raw's default layout is the reference's: per 32 columns, flat
    [N * ceil(V/32)], row major per row (cce.cpp:123-145), which the reference's glue
    reshapes to (B, (V + 31) // 32) and flattens back into cce_backward_raw
    (mlx_cce/__init__.py:22-49).  tile_max / tile_sum_exp against the oracle's 32-column
    statistics; lse, nll and the target logit against the 128-column forward; the glue's
    round trip gives the same dE, bit for bit, as the 128-column statistics with the same
    lse (the filter takes a 128-column tile's max as the max of its four 32-column maxima:
    the same fp32 logits, so the same kept tiles)."""
    N, D, V = 200, 96, 3000  # V % 32 != 0 and V % 128 != 0: ragged last tiles of both widths
    e, c, t = normal_case(N, D, V, dtype, cuda, seed=51, std=0.2)
    b = (torch.randn(V, device=cuda) * 0.5).to(dtype)
    t[::11] = -100
    tm, ts, ntl, lse = m.cce_forward_raw(e, c, t, b, ignore_index=-100)
    tm128, ts128, ntl128, lse128 = m.cce_forward_raw(e, c, t, b, ignore_index=-100, layout="tiles128")
    _, _, _, _, nll = m._ext.forward(e, c, t, b, -100, ref_stats=True)
    _, _, _, _, nll128 = m._ext.forward(e, c, t, b, -100)
    torch.cuda.synchronize()
    nt = (V + 31) // 32
    assert tm.shape == (N * nt,) and ts.shape == (N * nt,)
    tm_o, ts_o = O.tile_stats(f64(e), f64(c), f64(b), tile=32)
    np.testing.assert_allclose(f64(tm), tm_o.T.reshape(-1), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(f64(ts), ts_o.T.reshape(-1), rtol=1e-5)
    rows = (t != -100).nonzero().flatten()  # neg_target_logit of masked rows is not written
    assert torch.equal(ntl[rows], ntl128[rows])
    np.testing.assert_allclose(f64(lse), f64(lse128), rtol=1e-6)
    np.testing.assert_allclose(f64(nll), f64(nll128), rtol=1e-5, atol=1e-6)
    # the 128-column maxima are the maxima of the 32-column ones, exactly
    t32 = tm.reshape(N, nt)
    pad = torch.full((N, 4 * ((V + 127) // 128) - nt), -float("inf"), device=cuda)
    assert torch.equal(torch.cat([t32, pad], 1).reshape(N, -1, 4).amax(-1).T.contiguous(), tm128)
    # the reference glue: reshape(B, num_v_tiles), then reshape(-1) back into the backward
    tile_max_2d = tm.reshape(N, nt)
    d_nll = torch.linspace(0.5, 1.5, N, device=cuda)
    dE = m.cce_backward_raw(e, c, lse, t, d_nll, tile_max_2d.reshape(-1), b, ignore_index=-100)
    dE128 = m.cce_backward_raw(e, c, lse, t, d_nll, tm128, b, ignore_index=-100)
    torch.cuda.synchronize()
    assert torch.equal(dE, dE128)
    with pytest.raises(ValueError, match="tile_max must be"):
        m.cce_backward_raw(e, c, lse, t, d_nll, tile_max_2d, b, ignore_index=-100)


def test_raw_forward_then_raw_backward(m, cuda):
    """cce_forward_raw -> cce_backward_raw (csrc/bindings.cpp:58-86), the reference's
    own two-step use: dE (and with compute_all_grads dC, dBias) against the oracle for
    a given per-token cotangent."""
    e, c, t = normal_case(96, 64, 2000, torch.bfloat16, cuda, seed=46, std=0.1)
    b = (torch.randn(2000, device=cuda) * 0.1).to(torch.bfloat16)
    t[::9] = -100
    tm, ts, ntl, lse = m.cce_forward_raw(e, c, t, b, ignore_index=-100)
    d_nll = torch.linspace(0.5, 1.5, 96, device=cuda)
    dE = m.cce_backward_raw(e, c, lse, t, d_nll, tm, b, ignore_index=-100, filter_eps=None)
    dE2, dC, dB = m.cce_backward_raw(e, c, lse, t, d_nll, tm, b, ignore_index=-100, filter_eps=None,
                                     compute_all_grads=True)
    torch.cuda.synchronize()
    assert torch.equal(dE, dE2) and dE.dtype == torch.bfloat16
    tt = t.cpu().numpy()
    dn = np.where(tt != -100, np.linspace(0.5, 1.5, 96), 0.0)
    rE, rC, rB = O.grads(f64(e), f64(c), tt, f64(b), d_nll=dn)
    for name, got, r in (("dE", dE, rE), ("dC", dC, rC), ("dBias", dB, rB)):
        err = O.rel_fro(f64(got), O.round_bf16(r))
        print(f"raw backward {name}: {err:.2e}")
        assert err <= 1e-3, (name, err)
    np.testing.assert_allclose(f64(lse), O.per_token(f64(e), f64(c), tt, f64(b))[1], rtol=1e-6)



@pytest.mark.parametrize("filtered", [False, True])
def test_backward_captured_in_a_graph(m, cuda, filtered):
    """The backward inside HIP graph capture: the host cannot wait for the pass count
    there, so the library launches the worst case of passes and the device skips the
    empty ones.  Replays (with eager work and synchronisation between them) equal the
    eager backward bit for bit; the passes are several (max_g_tiles) so that the
    skipped ones are exercised."""
    e, c, t = _peaked(cuda, N=300, D=264, V=9000, seed=19) if filtered else \
        normal_case(300, 264, 9000, torch.bfloat16, cuda, seed=19, std=0.05)
    t[3] = -100
    feps = m.FILTER_LOG_EPS if filtered else None
    tm, _, _, lse, _ = m._ext.forward(e, c, t, None, -100)
    d_nll = torch.full((300,), 1.0 / 300, device=cuda)
    with m._ext.backward_options(max_g_tiles=8):
        ref = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, feps, True, True, False)
        torch.cuda.synchronize()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):  # warm-up off the capturing stream
            m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, feps, True, True, False)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, feps, True, True, False)
    for rep in range(3):
        junk = torch.randn(1 << 20, device=cuda).sum()  # eager work between the replays
        graph.replay()
        torch.cuda.synchronize()
        assert bool(torch.isfinite(junk))
        for x, y in zip(out[:2], ref[:2]):
            assert torch.equal(x.view(torch.int16), y.view(torch.int16)), rep


@pytest.mark.parametrize("case", ["plain", "ragged_bias", "passes"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_g_tile_tasks_match_block_tasks(m, cuda, case, dtype):
    """Uniform targets over 1002 vocabulary tiles with c2's logit spread keep each tile
    for ~6 token blocks, so the G kernel takes a tile with up to 4 of its blocks per
    task (the tile's C rows read once).  dE / dC / dBias agree with the token-block
    tasks (CCE_BWD_G_TASKS_BY_BLOCK) to the rounding of reordered fp32 sums and repeat
    bit for bit.  Cases: aligned shapes; ragged N, V and D with a bias (the column sums
    of dBias); several passes of a small G scratch."""
    N, D, V = (4096, 512, 128256) if case != "ragged_bias" else (4000, 520, 128000 - 77)
    e, c, t = normal_case(N, D, V, dtype, cuda, seed=41, std=0.04)
    t[9] = -100
    gb = torch.Generator(device=cuda).manual_seed(3)
    b = (torch.randn(V, generator=gb, device=cuda) * 0.1).to(dtype) if case == "ragged_bias" else None
    lse_tm = m._ext.forward(e, c, t, b, -100)
    tm, lse = lse_tm[0], lse_tm[3]
    d_nll = torch.linspace(0.5, 1.5, N, device=cuda) / N
    stats = torch.zeros(3, dtype=torch.int64, device=cuda)
    opts = {"max_g_tiles": 2048} if case == "passes" else {}
    want_db = b is not None
    run_bwd = lambda: m._ext.backward(e, c, t, lse, tm, d_nll, b, -100, m.FILTER_LOG_EPS, True, True, want_db,
                                      tile_stats=stats)
    with m._ext.backward_options(**opts):
        g1 = run_bwd()
        g2 = run_bwd()
    with m._ext.backward_options(g_tasks="blocks", **opts):
        gb_ = run_bwd()
    torch.cuda.synchronize()
    kept = int(stats[0])
    ntiles = (V + 127) // 128
    print(f"{case} {dtype}: kept tiles {kept} over {ntiles} vocabulary tiles")
    assert kept >= 3 * ntiles  # the tile tasks' condition
    bits = torch.int32 if dtype == torch.float32 else torch.int16
    tol = 1e-5 if dtype == torch.float32 else 2e-3
    for x, y, z, name in zip(g1, g2, gb_, ("dE", "dC", "dBias")):
        if x is None:
            continue
        assert torch.equal(x.view(bits), y.view(bits)), name
        err = O.rel_fro(f64(x), f64(z))
        print(f"  {name}: tile tasks vs block tasks {err:.2e}")
        assert err < tol, (name, err)
        assert float(x.float().abs().sum()) > 0


@pytest.mark.parametrize("case", ["peaked", "uniform", "passes"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_dc_block_tasks_match_owner_tasks(m, cuda, case, dtype):
    """The narrow dC sums run the owners that keep one token block as tasks per (token
    block, D slice); the same owners as tasks of their own (CCE_BWD_DC_OWNER_TASKS)
    give dC bit for bit: the same MFMAs in the same order.  Cases: skewed targets (a
    few owners keep many blocks, most keep one), near-uniform targets with the narrow
    geometry forced, and several passes of a small G scratch; D = 264 has a ragged
    last slice."""
    if case == "peaked":
        e, c, t = _peaked(cuda, N=1000, D=264, V=20000, dtype=dtype, seed=23)
    else:
        e, c, t = normal_case(1000, 264, 20000, dtype, cuda, seed=23, std=0.05)
    t[5] = -100
    lse_tm = m._ext.forward(e, c, t, None, -100)
    tm, lse = lse_tm[0], lse_tm[3]
    d_nll = torch.linspace(0.5, 1.5, 1000, device=cuda) / 1000
    opts = {"dc_sums": "narrow", "g_precision": "single"}
    if case == "passes":
        opts["max_g_tiles"] = 24
    stats = torch.zeros(3, dtype=torch.int64, device=cuda)
    with m._ext.backward_options(**opts):
        dE1, dC1, _ = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, m.FILTER_LOG_EPS, True, True, False,
                                      tile_stats=stats)
    with m._ext.backward_options(dc_tasks="owners", **opts):
        dE2, dC2, _ = m._ext.backward(e, c, t, lse, tm, d_nll, None, -100, m.FILTER_LOG_EPS, True, True, False)
    torch.cuda.synchronize()
    print(f"{case} {dtype}: kept tiles {int(stats[0])} of {int(stats[1])}")
    assert int(stats[0]) > 0
    assert torch.equal(dC1.view(torch.int16), dC2.view(torch.int16))
    assert torch.equal(dE1.view(torch.int16), dE2.view(torch.int16))
    assert float(dC1.float().abs().sum()) > 0
