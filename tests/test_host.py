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


def test_workspace_size_layout(ext):
    lib = ext.lib()
    N, D, V = 1000, 64, 3000
    base = lib.cce_backward_workspace_size(2, N, D, V, 0, 0, 0)
    tiles = math.ceil(N / 128) * math.ceil(V / 128)
    assert base >= tiles * 5 + 256
    full = lib.cce_backward_workspace_size(2, N, D, V, 1, 1, 1)
    assert full - base >= 4 * (N * D + V * D + V)
    assert lib.cce_backward_workspace_size(2, 0, D, V, 1, 1, 1) == 0


G_BUDGET = 512 << 20  # default G-tile budget of one backward pass (CCE_G_SCRATCH_MIB)


@pytest.mark.parametrize("N,D,V", [(8192, 4096, 128256), (32768, 8192, 128256), (65536, 4096, 128256),
                                   (4096, 2304, 256000), (1 << 20, 4096, 128256)],
                         ids=["c3", "c5", "N65536", "c4", "N1M"])
def test_backward_workspace_is_bounded(ext, N, D, V):
    """The backward's workspace is the G-tile budget + O(N*D + V) + per-pair lists of a
    few bytes per 128 x 128 tile (bounded per chunk), never a logits-sized G scratch."""
    lib = ext.lib()
    nrb, nvt = -(-N // 128), -(-V // 128)
    nwords = -(-nvt // 32)
    chunk_pairs = min(nrb * nvt, nrb * 32 * (8192 // nrb))
    for dtype, es in ((2, 2), (0, 4)):
        ws = lib.cce_backward_workspace_size(dtype, N, D, V, 1, 1, 1)
        tile = 128 * 128 * 4  # fp32 G, or the hi and lo halves of a 16-bit G
        g_slots = max(G_BUDGET // tile, 2 * nrb)
        bound = (g_slots * (tile + 512)  # G tiles + their column sums
                 + N * D * (4 + es)                # fp32 dE carry + the sorted copy of E
                 + N * nwords * 4 + 2 * nrb * nwords * 4  # keep bits per row / per block
                 + 40 * chunk_pairs + 64 * N + (4 << 20)
                 + (32 << 20))  # the dE pieces' slots (few dE tasks, or up to 1.5 grids of them)
        print(f"N={N} D={D} V={V} dtype {dtype}: workspace {ws / 2**30:.3f} GiB (bound {bound / 2**30:.3f}, "
              f"logits {N * V * es / 2**30:.2f})")
        assert 0 < ws <= bound
        assert ws < N * V * es / 2
    # the same plan with the smallest passes is smaller still, and sizes grow with the pass size
    sizes = [lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, k, 0) for k in (1, 4 * nrb, 16 * nrb)]
    assert sizes == sorted(sizes) and sizes[-1] <= lib.cce_backward_workspace_size(2, N, D, V, 1, 1, 1)


def test_backward_workspace_small_problems_fit_one_pass(ext):
    """Below the budget the plan keeps every pair in one pass: no fp32 dE carry."""
    lib = ext.lib()
    N, D, V = 1000, 64, 3000
    one = lib.cce_backward_workspace_size(2, N, D, V, 1, 1, 1)
    assert one == lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, 0, 0)
    tiles = math.ceil(N / 128) * math.ceil(V / 128)
    assert one >= tiles * 128 * 128 * 2  # every pair's G tile
    few = lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, 1, 0)  # smallest passes: carry + 16 tiles
    assert few < one and few >= N * D * 4
    assert lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, -1, 0) == 0
    assert lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, 0, -32) == 0


@pytest.mark.parametrize("N,D,V", [(8192, 4096, 128256), (1000, 64, 3000)], ids=["c3", "small"])
def test_workspace_size_follows_the_g_layout(ext, N, D, V):
    """A 16-bit G rounded once (the filter on, or CCE_BWD_G_SINGLE) takes 32 KiB a
    tile slot, the hi / lo pair (the filter off, or CCE_BWD_G_PAIR) and fp32 64 KiB:
    the same passes, so the sizes differ by exactly half the G slots' bytes, and the
    layout-free size is the pair's."""
    lib = ext.lib()
    nrb, nvt = -(-N // 128), -(-V // 128)
    cap = min(max(8192, 2 * nrb), nrb * nvt)  # G tiles of one pass (the default plan)
    eps, off = ctypes.c_float(-8.3), ctypes.c_float(float("-inf"))

    def size(dtype, e, flags=0, g=0):
        return lib.cce_backward_workspace_size_flags(dtype, N, D, V, 1, 1, 1, g, 0, e, flags)

    pair, single = size(2, off), size(2, eps)
    assert pair == lib.cce_backward_workspace_size(2, N, D, V, 1, 1, 1) == size(2, eps, ext.CCE_BWD_G_PAIR)
    assert single == size(2, off, ext.CCE_BWD_G_SINGLE) == size(1, eps)
    assert pair - single == cap * 128 * 128 * 2
    assert size(0, eps) == size(0, off) == lib.cce_backward_workspace_size(0, N, D, V, 1, 1, 1)
    # passes of 2 tiles per token block: the same halving of their (fewer) slots
    small = min(2 * nrb, nrb * nvt)
    assert size(2, off, 0, 1) - size(2, eps, 0, 1) == small * 128 * 128 * 2
    assert size(2, off, 0, 1) == lib.cce_backward_workspace_size_ex(2, N, D, V, 1, 1, 1, 1, 0)
    # invalid filter or flags: 0
    assert size(2, ctypes.c_float(float("nan"))) == 0
    assert size(2, eps, 1 << 14) == 0
    assert size(2, eps, ext.CCE_BWD_G_PAIR | ext.CCE_BWD_G_SINGLE) == 0
    assert size(2, eps, ext.CCE_BWD_TOKENS_INPUT | ext.CCE_BWD_TOKENS_SORTED) == 0


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


def _bwd_ex(lib, flags=0, chunk_tiles=0, ws_bytes=1 << 40):
    return lib.cce_backward_ex(2, FAKE, FAKE, None, FAKE, -100, 1, 64, 64, 256, FAKE, FAKE, FAKE, ctypes.c_float(-8.3),
                               FAKE, FAKE, None, FAKE, ctypes.c_size_t(ws_bytes), None, flags, chunk_tiles, None)


def test_backward_validation_errors(ext):
    lib = ext.lib()
    assert _bwd(lib, ext, ws_bytes=16) == ext.CCE_ERR_WORKSPACE
    assert b"workspace" in lib.cce_last_error() and b"at least" in lib.cce_last_error()
    assert _bwd(lib, ext, ws=None) == ext.CCE_ERR_WORKSPACE
    assert _bwd(lib, ext, dbias=FAKE) == ext.CCE_ERR_INVALID_ARGUMENT  # dBias without bias
    assert _bwd(lib, ext, eps=float("nan")) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _bwd(lib, ext, dtype=3) == ext.CCE_ERR_UNSUPPORTED_DTYPE
    assert _bwd_ex(lib, flags=1 << 14) == ext.CCE_ERR_INVALID_ARGUMENT  # unknown flag
    assert b"unknown flags" in lib.cce_last_error()
    assert _bwd_ex(lib, flags=ext.CCE_BWD_G_PAIR | ext.CCE_BWD_G_SINGLE) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _bwd_ex(lib, flags=ext.CCE_BWD_TOKENS_INPUT | ext.CCE_BWD_TOKENS_SORTED) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _bwd_ex(lib, flags=ext.CCE_BWD_DE_SUMS_WIDE | ext.CCE_BWD_DE_SUMS_NARROW) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _bwd_ex(lib, chunk_tiles=48) == ext.CCE_ERR_INVALID_ARGUMENT
    assert b"max_chunk_tiles" in lib.cce_last_error()
    # the error names the least workspace; one byte less is refused
    assert _bwd_ex(lib, ws_bytes=16) == ext.CCE_ERR_WORKSPACE
    least = int(re.search(rb"at least (\d+)", lib.cce_last_error()).group(1))
    assert 0 < least <= lib.cce_backward_workspace_size_ex(2, 64, 64, 256, 1, 1, 0, 1, 0)
    assert _bwd_ex(lib, ws_bytes=least - 1) == ext.CCE_ERR_WORKSPACE
    if not gpu_available():  # no device: the call passes the workspace check and stops at the device check
        assert _bwd_ex(lib, ws_bytes=least) == ext.CCE_ERR_NO_DEVICE


def _noalloc(lib, N=64, D=64, V=256, flags=0):
    return lib.cce_backward_noalloc(2, FAKE, FAKE, None, FAKE, -100, 1, N, D, V, FAKE, FAKE, FAKE,
                                    ctypes.c_float(-8.3), FAKE, FAKE, None, None, flags, None)


def test_reference_statistic_tiles(ext):
    """The reference's statistic tile is 32 columns: ceil(V / 32) of them."""
    lib = ext.lib()
    assert [lib.cce_num_ref_tiles(v) for v in (0, 1, 32, 33, 260, 128256)] == [0, 1, 1, 2, 9, 4008]
    assert ext.REF_STAT_TILE == 32 and ext.CCE_BWD_REF_STATS == 128


def test_noalloc_validation(ext):
    """cce_backward_noalloc refuses a problem past its static scratch before any device
    work (the fp32 dE carry of N=8192, D=4096 alone is 128 MiB of its 64 MiB)."""
    lib = ext.lib()
    assert lib.cce_backward_noalloc_scratch_size() == 64 << 20
    assert _noalloc(lib, N=8192, D=4096, V=128256) == ext.CCE_ERR_WORKSPACE
    msg = lib.cce_last_error()
    assert b"static scratch" in msg and b"N=8192" in msg
    assert _noalloc(lib, flags=1 << 14) == ext.CCE_ERR_INVALID_ARGUMENT
    assert _noalloc(lib, N=0) == ext.CCE_ERR_INVALID_ARGUMENT
    if not gpu_available():  # fits: stops at the device lookup
        assert _noalloc(lib) == ext.CCE_ERR_NO_DEVICE


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


def test_backward_options_are_scoped_and_validated(ext):
    """backward_options sets the overrides inside its block only (the dC zero fill in
    the backward by default) and refuses unknown values before anything runs."""
    assert ext._bwd_opts["dc_zero_fill"] == "backward" and ext._bwd_opts["flags"] == 0
    with ext.backward_options(dc_zero_fill="forward", g_tasks="blocks", max_g_tiles=7):
        assert ext._bwd_opts["dc_zero_fill"] == "forward"
        assert ext._bwd_opts["flags"] == ext.CCE_BWD_G_TASKS_BY_BLOCK and ext._bwd_opts["max_g_tiles"] == 7
    assert ext._bwd_opts == {"flags": 0, "max_g_tiles": 0, "max_chunk_tiles": 0, "dc_zero_fill": "backward"}
    with pytest.raises(ValueError, match="dc_zero_fill"):
        with ext.backward_options(dc_zero_fill="sometimes"):
            pass
    with pytest.raises(KeyError):
        with ext.backward_options(g_precision="triple"):
            pass
    assert ext._bwd_opts["dc_zero_fill"] == "backward"


def test_python_workspace_size_follows_the_filter(ext):
    """_ext.workspace_size: without a filter argument the size any filter needs (the hi /
    lo pair's slots); with filter_eps (None: the filter off) the exact size of that
    backward, which is what backward() allocates."""
    N, D, V = 8192, 4096, 128256
    e = torch.empty((N, D), dtype=torch.bfloat16)
    c = torch.empty((V, D), dtype=torch.bfloat16)
    lib = ext.lib()
    anyf = ext.workspace_size(e, c, True, True, False)
    assert anyf == lib.cce_backward_workspace_size(2, N, D, V, 1, 1, 0)
    assert ext.workspace_size(e, c, True, True, False, filter_eps=None) == anyf
    on = ext.workspace_size(e, c, True, True, False, filter_eps=ext.FILTER_LOG_EPS)
    assert on == anyf - 8192 * 128 * 128 * 2  # 8192 slots of 32 KiB instead of 64
    with ext.backward_options(g_precision="pair"):
        assert ext.workspace_size(e, c, True, True, False, filter_eps=ext.FILTER_LOG_EPS) == anyf
    with ext.backward_options(g_precision="single"):
        assert ext.workspace_size(e, c, True, True, False, filter_eps=None) == on
    f32 = torch.empty((N, D), dtype=torch.float32), torch.empty((V, D), dtype=torch.float32)
    assert ext.workspace_size(*f32, True, True, False, filter_eps=ext.FILTER_LOG_EPS) == \
        ext.workspace_size(*f32, True, True, False)
