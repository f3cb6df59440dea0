"""Host-side tests of the C ABI and the Python API — CPU only, no kernel launches.

* the library loads and exports every function include/cce_mi355x.h declares;
* validation errors come back as negative codes + messages before any HIP call
  (reference: std::invalid_argument / runtime_error, csrc/cce/cce.cpp:41-73,222-227);
* the Python layer refuses CPU tensors and malformed shapes loudly (no fallback).
"""

import ctypes
import math
import os
import re

import pytest
import torch

from conftest import ROOT, gpu_available

HEADER = os.path.join(ROOT, "include", "cce_mi355x.h")


@pytest.fixture(scope="module")
def ext():
    from mlx_cce_amd import _build, _ext
    if not os.path.exists(_build.LIB_PATH):
        _build.build()
    _ext.lib()
    return _ext


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(cce_[a-z_0-9]+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    fns = header_functions()
    assert {"cce_forward", "cce_backward", "cce_backward_workspace_size", "cce_last_error"} <= set(fns)


def test_library_exports_every_declared_symbol(ext):
    lib = ext.lib()
    for name in header_functions():
        assert hasattr(lib, name), name
    assert sorted(ext.SIGNATURES) == header_functions()


def test_version_and_geometry(ext):
    assert "gfx950" in ext.version()
    cfg = ext.tile_config()
    assert cfg == dict(fwd_tokens=256, fwd_vocab=256, stat_tile=128, bwd_tokens=128, bwd_vocab=128)
    lib = ext.lib()
    for V in (1, 127, 128, 129, 128256, 256000):
        assert lib.cce_num_vocab_tiles(V) == math.ceil(V / 128)


def test_forward_workspace_size(ext):
    """Fragment-order copy of E: whole 256-token tiles x row bytes rounded up to the
    128-byte slice; zero for empty shapes and unknown dtypes."""
    lib = ext.lib()
    assert lib.cce_forward_workspace_size(2, 8192, 4096) == 8192 * 8192
    assert lib.cce_forward_workspace_size(0, 300, 40) == 512 * 256  # fp32 rows of 160 B -> 2 slices
    assert lib.cce_forward_workspace_size(1, 1, 8) == 256 * 128
    assert lib.cce_forward_workspace_size(2, 0, 4096) == 0
    assert lib.cce_forward_workspace_size(7, 8192, 4096) == 0


def test_workspace_size_layout(ext):
    lib = ext.lib()
    N, D, V = 1000, 64, 3000
    base = lib.cce_backward_workspace_size(2, N, D, V, 0, 0, 0)
    tiles = math.ceil(N / 128) * math.ceil(V / 128)
    assert base >= tiles * 5 + 256
    full = lib.cce_backward_workspace_size(2, N, D, V, 1, 1, 1)
    assert full - base >= 4 * (N * D + V * D + V)
    assert lib.cce_backward_workspace_size(2, 0, D, V, 1, 1, 1) == 0


FAKE = 1 << 20  # 16-byte aligned, never dereferenced: validation fails first


def _fwd(lib, dtype=2, N=64, D=64, V=256, e=FAKE, c=FAKE, t=FAKE, outs=FAKE):
    return lib.cce_forward(dtype, e, c, None, t, -100, 1, N, D, V, outs, outs, outs, outs, outs, None)


def test_forward_validation_errors(ext):
    lib = ext.lib()
    assert _fwd(lib, dtype=7) == ext.CCE_ERR_UNSUPPORTED_DTYPE
    assert b"unsupported dtype" in lib.cce_last_error()
    assert _fwd(lib, D=12) == ext.CCE_ERR_INVALID_ARGUMENT  # bf16 rows must be 16-byte multiples
    assert b"multiple of 8" in lib.cce_last_error()
    assert _fwd(lib, N=0) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _fwd(lib, V=-3) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _fwd(lib, e=None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _fwd(lib, e=FAKE + 2) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"16-byte aligned" in lib.cce_last_error()
    assert _fwd(lib, outs=None) == ext.CCE_ERR_INVALID_ARGUMENT


def _bwd(lib, ext, ws=FAKE, ws_bytes=1 << 40, dbias=None, bias=None, eps=-8.3, dtype=2, N=64, D=64, V=256):
    return lib.cce_backward(dtype, FAKE, FAKE, bias, FAKE, -100, 1, N, D, V, FAKE, FAKE, FAKE, ctypes.c_float(eps),
                            FAKE, FAKE, dbias, ws, ctypes.c_size_t(ws_bytes), None, None)


def test_backward_validation_errors(ext):
    lib = ext.lib()
    assert _bwd(lib, ext, ws_bytes=16) == ext.CCE_ERR_WORKSPACE
    assert b"workspace" in lib.cce_last_error()
    assert _bwd(lib, ext, ws=None) == ext.CCE_ERR_WORKSPACE
    assert _bwd(lib, ext, dbias=FAKE) == ext.CCE_ERR_INVALID_ARGUMENT  # dBias without bias
    assert _bwd(lib, ext, eps=float("nan")) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _bwd(lib, ext, dtype=3) == ext.CCE_ERR_UNSUPPORTED_DTYPE


def test_reduction_helpers_validation_errors(ext):
    lib = ext.lib()
    assert lib.cce_reduce_loss(FAKE, FAKE, -100, 1, 0, ext.CCE_REDUCE_MEAN, FAKE, None, None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"positive" in lib.cce_last_error()
    assert lib.cce_reduce_loss(FAKE, FAKE, -100, 1, 8, 3, FAKE, None, None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"mode" in lib.cce_last_error()
    assert lib.cce_reduce_loss(FAKE, None, -100, 1, 8, ext.CCE_REDUCE_SUM, FAKE, None, None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert lib.cce_broadcast_grad(FAKE, None, 0, FAKE, None) == ext.CCE_ERR_INVALID_ARGUMENT
    assert lib.cce_broadcast_grad(None, None, 8, FAKE, None) == ext.CCE_ERR_INVALID_ARGUMENT


@pytest.mark.skipif(gpu_available(), reason="would launch on fake pointers when a GPU is present")
def test_no_device_is_reported(ext):
    lib = ext.lib()
    assert _fwd(lib) == ext.CCE_ERR_NO_DEVICE
    assert b"no HIP device" in lib.cce_last_error()


def test_last_error_is_cleared_on_next_call(ext):
    lib = ext.lib()
    _fwd(lib, dtype=9)
    assert lib.cce_last_error() != b""
    lib.cce_num_vocab_tiles(5)  # not an error-reporting call: message persists
    _fwd(lib, N=0)
    assert b"positive" in lib.cce_last_error()


# ------------------------------------------------------------- Python layer
def test_python_api_refuses_cpu_tensors(ext):
    import mlx_cce_amd as m
    e = torch.randn(8, 16)
    c = torch.randn(32, 16)
    t = torch.randint(0, 32, (8,))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        m.linear_cross_entropy(e, c, t)


def test_python_api_validates_shapes(ext):
    import mlx_cce_amd as m
    e = torch.randn(8, 16)
    with pytest.raises(ValueError, match="2D"):
        m.cce_loss(torch.randn(2, 8, 16), torch.randn(32, 16), torch.randint(0, 32, (16,)))
    with pytest.raises(ValueError, match="D"):
        m.linear_cross_entropy(e, torch.randn(32, 8), torch.randint(0, 32, (8,)))
    with pytest.raises(ValueError, match="Unknown reduction"):
        m.linear_cross_entropy(e, torch.randn(32, 16), torch.randint(0, 32, (8,)), reduction="avg")
    with pytest.raises(ValueError, match="bias"):
        m.linear_cross_entropy(e, torch.randn(32, 16), torch.randint(0, 32, (8,)), bias=torch.randn(31))
    with pytest.raises(TypeError, match="dtype"):
        m.linear_cross_entropy(e, torch.randn(32, 16, dtype=torch.float64).to(torch.bfloat16),
                               torch.randint(0, 32, (8,)))
    with pytest.raises(RuntimeError, match="unsupported dtype"):
        m.linear_cross_entropy(e.double(), torch.randn(32, 16).double(), torch.randint(0, 32, (8,)))


def test_package_exports_reference_api(ext):
    import mlx_cce_amd as m
    for name in ("linear_cross_entropy", "cce_loss", "cut_cross_entropy", "cce_forward_raw", "cce_backward_raw",
                 "LinearCrossEntropy", "FILTER_LOG_EPS"):
        assert hasattr(m, name), name
    assert abs(m.FILTER_LOG_EPS - math.log(2.0 ** -12)) < 1e-9
