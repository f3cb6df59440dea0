"""Quantized classifier rows (affine group quantization, MLX's mx.quantize layout).

The reference's callers dequantize the quantized lm_head / tied embedding with
mx.dequantize before the loss (README.md:84-95,136; examples/mlx_lm_lora_test.py:
16-21).  This build takes the quantized rows and dequantizes a bounded chunk at a
time inside the library (cce_forward_q / cce_backward_q).

Bars:
  * CPU: the oracle's dequantize equals a bit-by-bit pure-Python brute force; on
    inputs exact in every rounding order (power-of-two scales, small integer biases)
    it equals integer arithmetic; a planted code-order mistake is caught; the
    host-side quantizer's codes round-trip within half a step; the C ABI rejects
    bad layouts before touching memory.
  * GPU: the dequantize kernel equals the oracle bit for bit after rounding to the
    compute dtype; the quantized passes equal the plain passes over the dequantized
    rows bit for bit (same chunking), including multi-chunk and ragged V; against
    the float64 oracle at small sizes with the tolerances of the plain path.
  MLX's own rounding of scale * q + bias is parity unpinned (MLX cannot run here).
"""

import ctypes
import math
import os

import numpy as np
import pytest
import torch

from oracle import cce_oracle as O

FAKE = 1 << 20  # 16-byte aligned, never dereferenced: validation fails first


def _brute_dequant(words, scales, biases, group_size, bits):
    """Element by element, bit by bit: code j of word w of row r is bits
    [j*bits, (j+1)*bits) of that word; value float32(float32(s) * q) + float32(b)."""
    V, W = len(words), len(words[0])
    epw = 32 // bits
    out = np.zeros((V, W * epw), dtype=np.float32)
    for r in range(V):
        for w in range(W):
            word = int(words[r][w]) & 0xFFFFFFFF
            for j in range(epw):
                q = 0
                for k in range(bits):
                    q |= ((word >> (j * bits + k)) & 1) << k
                d = w * epw + j
                s = np.float32(scales[r][d // group_size])
                b = np.float32(biases[r][d // group_size])
                out[r, d] = np.float32(np.float32(s * np.float32(q)) + b)
    return out


def _random_quant(rng, V, D, group_size, bits):
    words = rng.integers(0, 1 << 32, size=(V, D * bits // 32), dtype=np.int64)
    scales = rng.standard_normal((V, D // group_size)).astype(np.float32) * 0.01
    biases = rng.standard_normal((V, D // group_size)).astype(np.float32) * 0.05
    return words, scales, biases


@pytest.mark.parametrize("bits", [2, 4, 8])
@pytest.mark.parametrize("group_size", [32, 64, 128])
def test_oracle_dequantize_matches_brute_force(bits, group_size):
    rng = np.random.default_rng(bits * 1000 + group_size)
    V, D = 3, 2 * group_size
    words, scales, biases = _random_quant(rng, V, D, group_size, bits)
    got = O.dequantize(words, scales, biases, group_size, bits)
    want = _brute_dequant(words, scales, biases, group_size, bits)
    assert got.dtype == np.float32
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_oracle_dequantize_exact_cases():
    """Scales 2^-k and integer biases: every product and sum is exact in float32 (and
    in bf16 for these magnitudes), so any implementation of w = s q + b agrees."""
    rng = np.random.default_rng(3)
    for bits in (2, 4, 8):
        V, D, gs = 5, 128, 32
        q = rng.integers(0, 1 << bits, size=(V, D))
        k = rng.integers(0, 6, size=(V, D // gs))
        bias_i = rng.integers(-4, 5, size=(V, D // gs))
        epw = 32 // bits
        words = np.zeros((V, D // epw), dtype=np.int64)
        for j in range(epw):
            words |= q[:, j::epw] << (bits * j)
        got = O.dequantize(words, 2.0 ** -k, bias_i, gs, bits)
        want = q * np.repeat(2.0 ** -k, gs, axis=1) + np.repeat(bias_i, gs, axis=1)
        assert np.array_equal(got, want.astype(np.float32))


def test_planted_code_order_mistake_is_caught():
    rng = np.random.default_rng(11)
    words, scales, biases = _random_quant(rng, 2, 64, 32, 4)

    def wrong(words, scales, biases, gs, bits):  # codes read from the high end of the word
        w = np.asarray(words) & 0xFFFFFFFF
        epw = 32 // bits
        sh = (epw - 1 - np.arange(epw)) * bits
        q = ((w[:, :, None] >> sh) & ((1 << bits) - 1)).reshape(w.shape[0], -1)
        return np.repeat(scales, gs, 1).astype(np.float32) * q + np.repeat(biases, gs, 1).astype(np.float32)

    want = _brute_dequant(words, scales, biases, 32, 4)
    assert not np.array_equal(wrong(words, scales, biases, 32, 4), want)
    assert np.array_equal(O.dequantize(words, scales, biases, 32, 4), want)


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_host_quantizer_round_trip(bits):
    from mlx_cce_amd.quant import quantize
    g = torch.Generator().manual_seed(bits)
    w = torch.randn((6, 256), generator=g) * 0.02
    qw = quantize(w, group_size=64, bits=bits)
    assert qw.shape == (6, 256) and qw.weight.dtype == torch.int32
    deq = O.dequantize(qw.weight.numpy(), qw.scales.numpy(), qw.biases.numpy(), 64, bits)
    step = np.repeat(qw.scales.numpy(), 64, axis=1)
    assert np.all(np.abs(deq - w.numpy()) <= 0.5 * step + 1e-6)


# ------------------------------------------------------------------ C ABI (no GPU needed)
@pytest.fixture(scope="module")
def ext():
    from mlx_cce_amd import _build, _ext
    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    _ext.lib()
    return _ext


def _fq(lib, dtype=2, bits=4, gs=64, N=64, D=256, V=512, scratch=FAKE, sbytes=1 << 40, chunk=0, w=FAKE):
    return lib.cce_forward_q(dtype, FAKE, w, FAKE, FAKE, gs, bits, None, FAKE, -100, 1, N, D, V,
                             FAKE, FAKE, FAKE, FAKE, FAKE, scratch, ctypes.c_size_t(sbytes), chunk, None)


def test_quantized_abi_validation(ext):
    lib = ext.lib()
    assert _fq(lib, bits=3) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"bits" in lib.cce_last_error()
    assert _fq(lib, gs=16) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"group_size" in lib.cce_last_error()
    assert _fq(lib, D=96) == ext.CCE_ERR_INVALID_ARGUMENT  # not a multiple of group_size 64
    assert _fq(lib, chunk=1000) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"chunk_rows" in lib.cce_last_error()
    assert _fq(lib, w=None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _fq(lib, sbytes=16) == ext.CCE_ERR_WORKSPACE
    assert lib.cce_dequantize(2, FAKE, FAKE, FAKE, 64, 5, 4, 256, FAKE, None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert lib.cce_dequantize(2, FAKE, FAKE, FAKE, 64, 4, 4, 256, FAKE + 8, None) == ext.CCE_ERR_INVALID_ARGUMENT
    rc = lib.cce_backward_q(2, FAKE, FAKE, FAKE, FAKE, 64, 4, None, FAKE, -100, 1, 64, 256, 512, FAKE, FAKE, FAKE,
                            ctypes.c_float(-8.3), FAKE, None, FAKE, ctypes.c_size_t(16), 0, None, None)
    assert rc == ext.CCE_ERR_WORKSPACE


def test_quantized_scratch_and_workspace_sizes(ext):
    lib = ext.lib()
    N, D, V = 1000, 256, 100000
    assert lib.cce_forward_q_scratch_size(2, V, D, 0) == 32768 * D * 2
    assert lib.cce_forward_q_scratch_size(2, V, D, 4096) == 4096 * D * 2
    assert lib.cce_forward_q_scratch_size(0, 300, D, 4096) == 300 * D * 4
    assert lib.cce_forward_q_scratch_size(2, V, D, 100) == 0
    plain = lib.cce_backward_workspace_size(2, N, D, V, 1, 0, 0)
    q = lib.cce_backward_q_workspace_size(2, N, D, V, 1, 0, 4096)
    assert q >= 4096 * D * 2
    assert lib.cce_backward_q_workspace_size(2, N, D, V, 1, 0, 4095) == 0
    assert plain > 0


# ------------------------------------------------------------------ GPU
def _gpu_quant(dev, V, D, gs, bits, dtype, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    words = torch.randint(-(1 << 31), (1 << 31) - 1, (V, D * bits // 32), generator=g, device=dev,
                          dtype=torch.int64).to(torch.int32)
    scales = (torch.rand((V, D // gs), generator=g, device=dev) * 0.004 + 0.001).to(dtype)
    biases = (torch.randn((V, D // gs), generator=g, device=dev) * 0.02).to(dtype)
    from mlx_cce_amd.quant import QuantizedWeight
    return QuantizedWeight(words, scales, biases, gs, bits)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("bits,gs", [(2, 32), (4, 64), (4, 128), (8, 32), (8, 128)])
def test_dequantize_kernel_bitwise(cuda, dtype, bits, gs):
    import mlx_cce_amd as m
    qw = _gpu_quant(cuda, 300, 256, gs, bits, dtype, seed=bits + gs)
    got = m.dequantize(qw)
    torch.cuda.synchronize()
    ref = O.dequantize(qw.weight.cpu().numpy(), qw.scales.float().cpu().numpy(), qw.biases.float().cpu().numpy(),
                       gs, bits)
    want = torch.from_numpy(ref).to(dtype)
    assert got.dtype == dtype and got.shape == (300, 256)
    assert torch.equal(got.cpu().view(torch.uint8), want.view(torch.uint8))


def _peaked_q(dev, N, D, V, dtype, seed, gs=64, bits=4, bias=False):
    """Peaked logits (as the headline workload) from quantized rows: e leans on the
    dequantized row of its target."""
    import mlx_cce_amd as m
    import workloads
    g = torch.Generator(device=dev).manual_seed(seed)
    c = (torch.randn((V, D), generator=g, device=dev) * 0.02).to(dtype)
    qw = m.quantize(c, group_size=gs, bits=bits)
    cd = m.dequantize(qw).float()
    t = workloads.zipf_targets(g, N, V, device=dev)
    ct = cd[t]
    e = (0.5 * torch.randn((N, D), generator=g, device=dev) + 12.0 * ct / ct.pow(2).sum(1, keepdim=True)).to(dtype)
    b = (torch.randn((V,), generator=g, device=dev) * 0.1).to(dtype) if bias else None
    return e, qw, t, b


@pytest.mark.gpu
@pytest.mark.parametrize("bias", [False, True])
def test_forward_q_equals_plain_forward(cuda, bias):
    """One chunk (the default 32768 rows hold V = 9000): every output bit equal to the
    plain forward over the dequantized rows.  Three chunks of 4096 rows (the last
    ragged): the tile kernel starts each tile's contraction at a slice that depends on
    the XCD it runs on, and the chunked launches place tiles on other XCDs, so the fp32
    sums differ in order only: 1e-5 relative."""
    import mlx_cce_amd as m
    e, qw, t, b = _peaked_q(cuda, 300, 256, 9000, torch.bfloat16, seed=21, bias=bias)
    t[::7] = -100
    cd = m.dequantize(qw)
    plain = m._ext.forward(e, cd, t, b, -100)
    one = m._ext.forward_q(e, qw, t, b, -100)
    three = m._ext.forward_q(e, qw, t, b, -100, chunk_rows=4096)
    torch.cuda.synchronize()
    valid = t != -100  # neg_target_logit is left unwritten on ignored rows (their nll is 0)
    pick = lambda outs: [o if i != 2 else o[valid] for i, o in enumerate(outs)]
    for x, y in zip(pick(one), pick(plain)):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))
    names = ("tile_max", "tile_sum_exp", "neg_target_logit", "lse", "nll")
    for name, x, y in zip(names, pick(three), pick(plain)):
        # nll = lse + neg_target_logit cancels two values near +-12: its error is absolute,
        # a few ulp of lse (ulp(12) = 9.5e-7)
        torch.testing.assert_close(x, y, rtol=1e-5, atol=2e-5 if name == "nll" else 1e-6, msg=name)


@pytest.mark.gpu
@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("filtered", [False, True])
def test_backward_q_equals_plain_backward(cuda, bias, filtered):
    """dE and dBias bit for bit equal to the plain backward over the dequantized rows
    with the same vocabulary chunks (32 tiles = 4096 rows)."""
    import mlx_cce_amd as m
    e, qw, t, b = _peaked_q(cuda, 384, 256, 9000, torch.bfloat16, seed=22, bias=bias)
    t[::11] = -100
    cd = m.dequantize(qw)
    tm, _, _, lse, _ = m._ext.forward(e, cd, t, b, -100)
    d_nll = torch.full((384,), 1.0 / 384, device=cuda)
    eps = m.FILTER_LOG_EPS if filtered else None
    st_p = torch.zeros(3, dtype=torch.int64, device=cuda)
    st_q = torch.zeros(3, dtype=torch.int64, device=cuda)
    with m._ext.backward_options(max_chunk_tiles=32):
        dE_p, _, dB_p = m._ext.backward(e, cd, t, lse, tm, d_nll, b, -100, eps, True, False, True, tile_stats=st_p)
    dE_q, dB_q = m._ext.backward_q(e, qw, t, lse, tm, d_nll, b, -100, eps, True, True, tile_stats=st_q,
                                   chunk_rows=4096)
    torch.cuda.synchronize()
    assert torch.equal(st_p, st_q)
    assert torch.equal(dE_q.view(torch.int16), dE_p.view(torch.int16))
    if bias:
        assert torch.equal(dB_q.view(torch.int16), dB_p.view(torch.int16))
    else:
        assert dB_q is None


@pytest.mark.gpu
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
def test_autograd_with_quantized_rows(cuda, reduction):
    """linear_cross_entropy(e, QuantizedWeight, ...) against the same call on the
    dequantized rows (default chunking: one chunk at this size): loss, dE, dBias equal."""
    import mlx_cce_amd as m
    e, qw, t, b = _peaked_q(cuda, 256, 256, 5000, torch.bfloat16, seed=23, bias=True)
    t[::5] = -100
    cd = m.dequantize(qw)
    outs = []
    for c in (qw, cd):
        ee = e.detach().clone().requires_grad_(True)
        bb = b.detach().clone().requires_grad_(True)
        loss = m.linear_cross_entropy(ee, c, t, bb, reduction=reduction)
        loss.backward(torch.ones_like(loss))
        torch.cuda.synchronize()
        outs.append((loss.detach(), ee.grad, bb.grad))
    bits = lambda x: x.view(torch.int16) if x.element_size() == 2 else x.view(torch.int32)
    for x, y in zip(*outs):
        assert x.dtype == y.dtype and torch.equal(bits(x), bits(y))


@pytest.mark.gpu
def test_quantized_against_oracle(cuda):
    """fp32 compute dtype, filter off: loss and dE against the float64 oracle over the
    oracle's own dequantization of the same words (1e-5 loss, 1e-3 dE)."""
    import mlx_cce_amd as m
    qw = _gpu_quant(cuda, 700, 128, 32, 4, torch.float32, seed=24)
    g = torch.Generator(device=cuda).manual_seed(25)
    e = torch.randn((96, 128), generator=g, device=cuda)
    t = torch.randint(0, 700, (96,), generator=g, device=cuda)
    t[::9] = -100
    ee = e.clone().requires_grad_(True)
    loss = m.linear_cross_entropy(ee, qw, t, filter_eps=None)
    loss.backward()
    torch.cuda.synchronize()
    c = O.dequantize(qw.weight.cpu().numpy(), qw.scales.cpu().numpy(), qw.biases.cpu().numpy(), 32, 4)
    en, tn = e.cpu().numpy(), t.cpu().numpy()
    ref = O.linear_cross_entropy(en, c, tn)
    gE, _, _ = O.grads(en, c, tn)
    np.testing.assert_allclose(float(loss), ref, rtol=1e-5)
    assert O.rel_fro(ee.grad.double().cpu().numpy(), gE) < 1e-3


@pytest.mark.gpu
def test_quantized_rows_get_no_gradient(cuda):
    import mlx_cce_amd as m
    e, qw, t, _ = _peaked_q(cuda, 64, 128, 600, torch.bfloat16, seed=26)
    ee = e.detach().clone().requires_grad_(True)
    m.linear_cross_entropy(ee, qw, t).backward()
    assert ee.grad is not None and not qw.weight.requires_grad and qw.scales.grad is None


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,D,gs,bits", [(torch.bfloat16, 96, 32, 4), (torch.float16, 160, 32, 8),
                                               (torch.float32, 64, 32, 2)])
def test_quantized_ragged_shapes_multi_chunk(cuda, dtype, D, gs, bits):
    """Rows that are not a whole number of 128-byte slices (the zero-padded slice path),
    N not a multiple of the 128-row block, several chunks, ignore_index=None:
    the quantized passes equal the plain passes over the dequantized rows (forward to
    1e-5 across chunks, backward bit for bit with the same chunks)."""
    import mlx_cce_amd as m
    qw = _gpu_quant(cuda, 8500, D, gs, bits, dtype, seed=D + bits)
    g = torch.Generator(device=cuda).manual_seed(31)
    e = torch.randn((333, D), generator=g, device=cuda).to(dtype)
    t = torch.randint(0, 8500, (333,), generator=g, device=cuda)
    cd = m.dequantize(qw)
    plain = m._ext.forward(e, cd, t, None, None)
    quant = m._ext.forward_q(e, qw, t, None, None, chunk_rows=4096)
    torch.cuda.synchronize()
    for x, y in zip(quant, plain):
        torch.testing.assert_close(x, y, rtol=1e-5, atol=2e-5)
    tm, _, _, lse, _ = plain
    d_nll = torch.full((333,), 1.0 / 333, device=cuda)
    with m._ext.backward_options(max_chunk_tiles=32):
        dE_p, _, _ = m._ext.backward(e, cd, t, lse, tm, d_nll, None, None, m.FILTER_LOG_EPS, True, False, False)
    dE_q, _ = m._ext.backward_q(e, qw, t, lse, tm, d_nll, None, None, m.FILTER_LOG_EPS, True, False,
                                chunk_rows=4096)
    torch.cuda.synchronize()
    bits_of = lambda x: x.view(torch.int16) if x.element_size() == 2 else x.view(torch.int32)
    assert torch.equal(bits_of(dE_q), bits_of(dE_p))


@pytest.mark.gpu
def test_quantized_rejects_bad_layouts(cuda):
    import mlx_cce_amd as m
    qw = _gpu_quant(cuda, 300, 128, 64, 4, torch.bfloat16, seed=40)
    e = torch.randn((16, 96), device=cuda).to(torch.bfloat16)
    t = torch.zeros((16,), dtype=torch.int64, device=cuda)
    with pytest.raises(ValueError):
        m.linear_cross_entropy(e, qw, t)  # D mismatch
    e = torch.randn((16, 128), device=cuda).to(torch.float16)
    with pytest.raises(TypeError):
        m.linear_cross_entropy(e, qw, t)  # dtype of e differs from the scales
