"""ctypes binding of ``libcce_mi355x.so`` — the C ABI declared in ``include/cce_mi355x.h``.

This module is the PyTorch-side replacement of the reference's nanobind module
``mlx_cce._ext`` (csrc/bindings.cpp:12-87).  It only moves pointers and the
current HIP stream across the boundary; every FLOP runs in the HIP library.
There is no fallback: if the library is missing or the tensors are not on a
ROCm device, the call raises.
"""

import contextlib
import ctypes
import math
import os

import torch

from ._build import LIB_PATH

FILTER_LOG_EPS = -8.3177661667  # ln(2^-12); reference csrc/cce/cce.metal:143
STAT_TILE = 128

CCE_OK = 0
CCE_ERR_INVALID_ARGUMENT = -1
CCE_ERR_UNSUPPORTED_DTYPE = -2
CCE_ERR_WORKSPACE = -3
CCE_ERR_LAUNCH = -4
CCE_ERR_NO_DEVICE = -5

DTYPE_CODES = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

# Every symbol include/cce_mi355x.h declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int
SIGNATURES = {
    "cce_last_error": (ctypes.c_char_p, []),
    "cce_version": (ctypes.c_char_p, []),
    "cce_tile_config": (None, [_P, _P, _P, _P, _P]),
    "cce_num_vocab_tiles": (_I64, [_I64]),
    "cce_num_ref_tiles": (_I64, [_I64]),
    "cce_forward_ref": (_INT, [_INT, _P, _P, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "cce_forward": (_INT, [_INT, _P, _P, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P]),
    "cce_backward_workspace_size": (ctypes.c_size_t, [_INT, _I64, _I64, _I64, _INT, _INT, _INT]),
    "cce_backward_workspace_size_ex": (ctypes.c_size_t, [_INT, _I64, _I64, _I64, _INT, _INT, _INT, _I64, _I64]),
    "cce_backward_workspace_size_flags": (ctypes.c_size_t, [_INT, _I64, _I64, _I64, _INT, _INT, _INT, _I64, _I64,
                                                            ctypes.c_float, _INT]),
    "cce_backward": (_INT, [_INT, _P, _P, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, ctypes.c_float,
                            _P, _P, _P, _P, ctypes.c_size_t, _P, _P]),
    "cce_forward_ex": (_INT, [_INT, _P, _P, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _I64,
                              _P]),
    "cce_backward_ex": (_INT, [_INT, _P, _P, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, ctypes.c_float,
                               _P, _P, _P, _P, ctypes.c_size_t, _P, _INT, _I64, _P]),
    "cce_backward_noalloc_scratch_size": (ctypes.c_size_t, []),
    "cce_backward_noalloc": (_INT, [_INT, _P, _P, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, ctypes.c_float,
                                    _P, _P, _P, _P, _INT, _P]),
    "cce_dequantize": (_INT, [_INT, _P, _P, _P, _INT, _INT, _I64, _I64, _P, _P]),
    "cce_forward_q_scratch_size": (ctypes.c_size_t, [_INT, _I64, _I64, _I64]),
    "cce_forward_q": (_INT, [_INT, _P, _P, _P, _P, _INT, _INT, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P, _P,
                             _P, _P, ctypes.c_size_t, _I64, _P]),
    "cce_backward_q_workspace_size": (ctypes.c_size_t, [_INT, _I64, _I64, _I64, _INT, _INT, _I64]),
    "cce_backward_q": (_INT, [_INT, _P, _P, _P, _P, _INT, _INT, _P, _P, _I64, _INT, _I64, _I64, _I64, _P, _P, _P,
                              ctypes.c_float, _P, _P, _P, ctypes.c_size_t, _I64, _P, _P]),
    "cce_reduce_loss": (_INT, [_P, _P, _I64, _INT, _I64, _INT, _P, _P, _P]),
    "cce_broadcast_grad": (_INT, [_P, _P, _I64, _P, _P]),
}

CCE_REDUCE_SUM = 1
CCE_REDUCE_MEAN = 2
CCE_BWD_DC_ZEROED = 1
CCE_BWD_TOKENS_INPUT = 2
CCE_BWD_TOKENS_SORTED = 4
CCE_BWD_DE_SUMS_WIDE = 8
CCE_BWD_DE_SUMS_NARROW = 16
CCE_BWD_DC_SUMS_WIDE = 32
CCE_BWD_DC_SUMS_NARROW = 64
CCE_BWD_REF_STATS = 128
CCE_BWD_DEVICE_PASSES = 256
CCE_BWD_G_PAIR = 512
CCE_BWD_G_SINGLE = 1024
CCE_BWD_DC_OWNER_TASKS = 2048
CCE_BWD_G_TASKS_BY_BLOCK = 4096
CCE_BWD_DE_WHOLE_TASKS = 8192
REF_STAT_TILE = 32

# Overrides of choices the backward otherwise makes itself, for tests and tuning
# (results agree to rounding either way).  They travel explicitly with every
# cce_backward_ex call and its workspace-size query, so the two always agree.
_bwd_opts = {"flags": 0, "max_g_tiles": 0, "max_chunk_tiles": 0, "dc_zero_fill": "backward"}


@contextlib.contextmanager
def backward_options(token_order=None, de_sums=None, dc_sums=None, max_g_tiles=0, max_chunk_tiles=0,
                     passes=None, g_precision=None, dc_tasks=None, g_tasks=None, dc_zero_fill=None,
                     de_tasks=None):
    """Within the block, backward() calls run with these overrides:
    token_order "input" | "sorted" (128-row token blocks of the input order, or of the
    rows grouped by target tile); de_sums / dc_sums "wide" | "narrow" (512- or
    256-column sum tasks); max_g_tiles (passes of at most that many G tiles);
    max_chunk_tiles (vocabulary chunks of at most that many tiles, a multiple of 32);
    passes "device" (launch the worst case of passes and let the device skip the
    empty ones, instead of the host waiting for the pass count); g_precision "pair" |
    "single" (16-bit inputs: the softmax gradient between the two products as a hi +
    lo pair, fp32-accurate, or rounded once to the input dtype; by default the pair
    with the filter off and a single rounding with it on); dc_tasks "owners" (the
    narrow dC sums run one-tile owners as owner tasks, not grouped by token block);
    g_tasks "blocks" (the G kernel's tasks are token blocks with up to 4 kept tiles,
    never vocabulary tiles with up to 4 kept blocks); de_tasks "whole" (the dE sums never
    cut a (token block, D slice) task into pieces); dc_zero_fill "forward" (the
    autograd op has the forward's tile kernel zero dC, cce_forward_ex, and the backward
    write only the rows of kept tiles, CCE_BWD_DC_ZEROED) | "backward" (the default:
    the backward zeroes the rows no kept tile touches)."""
    flags = 0
    flags |= {None: 0, "pair": CCE_BWD_G_PAIR, "single": CCE_BWD_G_SINGLE}[g_precision]
    flags |= {None: 0, "host": 0, "device": CCE_BWD_DEVICE_PASSES}[passes]
    flags |= {None: 0, "blocks": 0, "owners": CCE_BWD_DC_OWNER_TASKS}[dc_tasks]
    flags |= {None: 0, "tiles": 0, "blocks": CCE_BWD_G_TASKS_BY_BLOCK}[g_tasks]
    flags |= {None: 0, "pieces": 0, "whole": CCE_BWD_DE_WHOLE_TASKS}[de_tasks]
    flags |= {None: 0, "input": CCE_BWD_TOKENS_INPUT, "sorted": CCE_BWD_TOKENS_SORTED}[token_order]
    flags |= {None: 0, "wide": CCE_BWD_DE_SUMS_WIDE, "narrow": CCE_BWD_DE_SUMS_NARROW}[de_sums]
    flags |= {None: 0, "wide": CCE_BWD_DC_SUMS_WIDE, "narrow": CCE_BWD_DC_SUMS_NARROW}[dc_sums]
    if dc_zero_fill not in (None, "forward", "backward"):
        raise ValueError(f"dc_zero_fill must be 'forward' or 'backward', got {dc_zero_fill!r}")
    saved = dict(_bwd_opts)
    _bwd_opts.update(flags=flags, max_g_tiles=int(max_g_tiles), max_chunk_tiles=int(max_chunk_tiles),
                     dc_zero_fill=dc_zero_fill or "backward")
    try:
        yield
    finally:
        _bwd_opts.clear()
        _bwd_opts.update(saved)

_lib = None

# Opt-in timing: when enabled, every cce_forward / cce_backward call is bracketed
# by HIP events recorded on the stream the kernels are launched on.
_timing = {"on": False, "forward": [], "backward": []}


def set_timing(on, kinds=("forward", "backward")):
    """Enable/disable event timing of the library calls (of the given kinds) and clear
    recorded events."""
    _timing["on"] = bool(on)
    _timing["kinds"] = tuple(kinds)
    _timing["forward"].clear()
    _timing["backward"].clear()


def timings_ms():
    """{'forward': [ms...], 'backward': [ms...]} of the recorded calls (synchronises)."""
    torch.cuda.synchronize()
    return {k: [a.elapsed_time(b) for a, b in _timing[k]] for k in ("forward", "backward")}


def _event_pair(kind):
    if not _timing["on"] or kind not in _timing.get("kinds", ("forward", "backward")):
        return None
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _timing[kind].append((a, b))
    return a, b


def lib():
    """Load the HIP library once (after torch, so it binds to torch's HIP runtime)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing. Build it with `python mlx-cross-entropy_amd/mlx_cce_amd/_build.py` "
                "(hipcc, --offload-arch=gfx950).")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def version():
    return lib().cce_version().decode()


def tile_config():
    vals = [ctypes.c_int() for _ in range(5)]
    lib().cce_tile_config(*[ctypes.byref(v) for v in vals])
    keys = ("fwd_tokens", "fwd_vocab", "stat_tile", "bwd_tokens", "bwd_vocab")
    return {k: v.value for k, v in zip(keys, vals)}


def _raise(rc, fn):
    msg = lib().cce_last_error().decode() or f"{fn} failed with code {rc}"
    if rc == CCE_ERR_INVALID_ARGUMENT or rc == CCE_ERR_WORKSPACE:
        raise ValueError(msg)
    raise RuntimeError(msg)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _check_device(name, t, device):
    if t.device.type != "cuda":
        raise RuntimeError(
            f"[cce] {name} is on {t.device}; this op runs only on a ROCm GPU (HIP) device "
            "(the reference likewise has no CPU evaluation)")
    if device is not None and t.device != device:
        raise ValueError(f"[cce] {name} is on {t.device}, expected {device}")


def _prep(e, c, targets, bias):
    """Validate and normalise operands to the library's layout; returns dtype code."""
    if e.dim() != 2:
        raise ValueError(f"[cut_cross_entropy] e must be 2D [B, D], got {e.dim()}D")
    if c.dim() != 2:
        raise ValueError(f"[cut_cross_entropy] c must be 2D [V, D], got {c.dim()}D")
    if targets.dim() != 1:
        raise ValueError(f"[cut_cross_entropy] targets must be 1D [B], got {targets.dim()}D")
    if c.shape[1] != e.shape[1]:
        raise ValueError("[cut_cross_entropy] c.shape[1] must equal e.shape[1] (D)")
    if targets.shape[0] != e.shape[0]:
        raise ValueError("[cut_cross_entropy] targets.shape[0] must equal e.shape[0] (B)")
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != c.shape[0]):
        raise ValueError("[cut_cross_entropy] bias must be 1D [V]")
    if e.dtype not in DTYPE_CODES:
        raise RuntimeError(f"CCE: unsupported dtype {e.dtype}")
    if c.dtype != e.dtype or (bias is not None and bias.dtype != e.dtype):
        raise TypeError(f"[cut_cross_entropy] e, c and bias must share one dtype, got {e.dtype}, {c.dtype}"
                        + (f", {bias.dtype}" if bias is not None else ""))
    dev = e.device
    _check_device("e", e, None)
    _check_device("c", c, dev)
    _check_device("targets", targets, dev)
    if bias is not None:
        _check_device("bias", bias, dev)
    return DTYPE_CODES[e.dtype]


def forward(e, c, targets, bias=None, ignore_index=-100, zero_out=None, ref_stats=False):
    """Run the fused forward.  Returns (tile_max, tile_sum_exp, neg_target_logit, lse, nll).

    tile_max / tile_sum_exp are [ceil(V/128), N] fp32 (vocab-tile major), or with
    ref_stats=True per 32 columns, flat [N * ceil(V/32)] (the reference's layout,
    cce_forward_ref); nll is the per-token loss, 0 on rows whose target equals
    ignore_index.  zero_out (optional, a contiguous device tensor of a multiple of 16
    bytes) is filled with zeros by the forward's tile kernel (cce_forward_ex).
    """
    code = _prep(e, c, targets, bias)
    e = e.contiguous()
    c = c.contiguous()
    targets = targets.to(torch.int64).contiguous()
    if bias is not None:
        bias = bias.contiguous()
    N, D = e.shape
    V = c.shape[0]
    nvt = (V + STAT_TILE - 1) // STAT_TILE
    f32 = dict(dtype=torch.float32, device=e.device)
    shape = (N * ((V + REF_STAT_TILE - 1) // REF_STAT_TILE),) if ref_stats else (nvt, N)
    tile_max = torch.empty(shape, **f32)
    tile_sum_exp = torch.empty(shape, **f32)
    neg_tl = torch.empty((N,), **f32)
    lse = torch.empty((N,), **f32)
    nll = torch.empty((N,), **f32)
    has_ignore = ignore_index is not None
    with torch.cuda.device(e.device):
        stream = torch.cuda.current_stream(e.device).cuda_stream
        ev = _event_pair("forward")
        if ev:
            ev[0].record()
        if zero_out is not None and (not zero_out.is_contiguous() or zero_out.device != e.device):
            raise ValueError("[cce_forward] zero_out must be a contiguous tensor on the device of e")
        if ref_stats and zero_out is not None:
            raise ValueError("[cce_forward_ref] takes no zero_out")
        if ref_stats:
            rc = lib().cce_forward_ref(code, _ptr(e), _ptr(c), _ptr(bias), _ptr(targets),
                                       int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                       N, D, V, _ptr(tile_max), _ptr(tile_sum_exp), _ptr(neg_tl), _ptr(lse),
                                       _ptr(nll), ctypes.c_void_p(stream))
        elif zero_out is not None:
            rc = lib().cce_forward_ex(code, _ptr(e), _ptr(c), _ptr(bias), _ptr(targets),
                                      int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                      N, D, V, _ptr(tile_max), _ptr(tile_sum_exp), _ptr(neg_tl), _ptr(lse),
                                      _ptr(nll), _ptr(zero_out), zero_out.numel() * zero_out.element_size(),
                                      ctypes.c_void_p(stream))
        else:
            rc = lib().cce_forward(code, _ptr(e), _ptr(c), _ptr(bias), _ptr(targets),
                                   int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                   N, D, V, _ptr(tile_max), _ptr(tile_sum_exp), _ptr(neg_tl), _ptr(lse), _ptr(nll),
                                   ctypes.c_void_p(stream))
        if ev:
            ev[1].record()
    if rc != CCE_OK:
        _raise(rc, "cce_forward")
    return tile_max, tile_sum_exp, neg_tl, lse, nll


_ANY_FILTER = object()


def workspace_size(e, c, want_de, want_dc, want_db, max_g_tiles=None, max_chunk_tiles=None,
                   filter_eps=_ANY_FILTER, flags=None):
    """Bytes of the backward's workspace; the backward_options in force unless given.
    Without filter_eps: enough for any filter (cce_backward_workspace_size_ex); with
    it (None: the filter off), the size of a backward with that filter and flags
    (cce_backward_workspace_size_flags: 16-bit G rounded once takes half the G
    bytes)."""
    N, D = e.shape
    V = c.shape[0]
    g = _bwd_opts["max_g_tiles"] if max_g_tiles is None else int(max_g_tiles)
    ch = _bwd_opts["max_chunk_tiles"] if max_chunk_tiles is None else int(max_chunk_tiles)
    code = DTYPE_CODES.get(e.dtype, -1)
    if filter_eps is _ANY_FILTER:
        return int(lib().cce_backward_workspace_size_ex(code, N, D, V, int(want_de), int(want_dc), int(want_db),
                                                        g, ch))
    eps = -math.inf if filter_eps is None else float(filter_eps)
    fl = _bwd_opts["flags"] if flags is None else int(flags)
    return int(lib().cce_backward_workspace_size_flags(code, N, D, V, int(want_de), int(want_dc), int(want_db),
                                                       g, ch, ctypes.c_float(eps), fl))


def _ref_stats_layout(tile_max, N, V, fn):
    """True when tile_max is in the reference's layout (flat [N * ceil(V/32)]), False
    for [ceil(V/128), N]; raises for any other shape."""
    nt = (V + REF_STAT_TILE - 1) // REF_STAT_TILE
    if tile_max.dim() == 1 and tile_max.numel() == N * nt:
        return True
    if tile_max.dim() == 2 and tuple(tile_max.shape) == ((V + STAT_TILE - 1) // STAT_TILE, N):
        return False
    raise ValueError(f"[{fn}] tile_max must be flat [N * ceil(V/32)] (reference layout) or "
                     f"[ceil(V/128), N], got {tuple(tile_max.shape)}")


def backward(e, c, targets, lse, tile_max, d_nll, bias=None, ignore_index=-100,
             filter_eps=FILTER_LOG_EPS, want_de=True, want_dc=True, want_db=True, tile_stats=None,
             dc_zeroed=None):
    """Run the filtered backward.  Returns (dE, dC, dBias), each None when not wanted.

    d_nll is the fp32 cotangent of the per-token loss [N].  tile_max is forward()'s,
    in either layout (the flat reference layout runs with CCE_BWD_REF_STATS).
    filter_eps=None or -inf disables the 2^-12 tile filter.  tile_stats, if given, is
    a device int64[3] tensor that receives (kept tiles, total tiles, kept tiles of the
    input-order token blocks).  dc_zeroed, if given, is a tensor like c that already
    holds zeros (from forward(..., zero_out=)): it becomes dC, and only its rows of
    vocabulary tiles with kept tiles are written (cce_backward_ex).
    """
    code = _prep(e, c, targets, bias)
    e = e.contiguous()
    c = c.contiguous()
    targets = targets.to(torch.int64).contiguous()
    if bias is not None:
        bias = bias.contiguous()
    want_db = bool(want_db and bias is not None)
    N, D = e.shape
    V = c.shape[0]
    lse = lse.contiguous()
    tile_max = tile_max.contiguous()
    ref = _ref_stats_layout(tile_max, N, V, "cce_backward")
    d_nll = d_nll.to(torch.float32).contiguous()
    if d_nll.shape != (N,) or lse.shape != (N,):
        raise ValueError("[cce_backward] lse and d_nll must be [N]")
    dE = torch.empty_like(e) if want_de else None
    if dc_zeroed is not None and want_dc:
        if dc_zeroed.shape != c.shape or dc_zeroed.dtype != c.dtype or not dc_zeroed.is_contiguous():
            raise ValueError("[cce_backward] dc_zeroed must be a contiguous tensor like c")
        dC = dc_zeroed
    else:
        dc_zeroed = None
        dC = torch.empty_like(c) if want_dc else None
    dB = torch.empty_like(bias) if want_db else None
    eps = -math.inf if filter_eps is None else float(filter_eps)
    has_ignore = ignore_index is not None
    flags = _bwd_opts["flags"] | (CCE_BWD_DC_ZEROED if dc_zeroed is not None else 0) | (CCE_BWD_REF_STATS if ref else 0)
    ws_bytes = workspace_size(e, c, want_de, want_dc, want_db, filter_eps=eps, flags=flags)
    ws = torch.empty((ws_bytes,), dtype=torch.uint8, device=e.device)
    with torch.cuda.device(e.device):
        stream = torch.cuda.current_stream(e.device).cuda_stream
        ev = _event_pair("backward")
        if ev:
            ev[0].record()
        rc = lib().cce_backward_ex(code, _ptr(e), _ptr(c), _ptr(bias), _ptr(targets),
                                   int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                   N, D, V, _ptr(lse), _ptr(tile_max), _ptr(d_nll), ctypes.c_float(eps),
                                   _ptr(dE), _ptr(dC), _ptr(dB), _ptr(ws), ctypes.c_size_t(ws_bytes),
                                   _ptr(tile_stats), flags, _bwd_opts["max_chunk_tiles"], ctypes.c_void_p(stream))
        if ev:
            ev[1].record()
    if rc != CCE_OK:
        _raise(rc, "cce_backward")
    return dE, dC, dB


def backward_noalloc(e, c, targets, lse, tile_max, d_nll, bias=None, ignore_index=-100,
                     filter_eps=FILTER_LOG_EPS, want_de=True, want_dc=True, want_db=True, tile_stats=None,
                     dE=None, dC=None, dB=None):
    """backward() through cce_backward_noalloc: the library takes no workspace and
    allocates nothing (its static device scratch of cce_backward_noalloc_scratch_size()
    bytes); the outputs are allocated here unless passed in.  Returns (dE, dC, dBias)."""
    code = _prep(e, c, targets, bias)
    for name, t in (("e", e), ("c", c), ("targets", targets), ("lse", lse), ("tile_max", tile_max),
                    ("d_nll", d_nll)):
        if not t.is_contiguous():
            raise ValueError(f"[cce_backward_noalloc] {name} must be contiguous")
    if d_nll.dtype != torch.float32 or lse.dtype != torch.float32 or targets.dtype != torch.int64:
        raise TypeError("[cce_backward_noalloc] lse and d_nll must be float32, targets int64")
    want_db = bool(want_db and bias is not None)
    N, D = e.shape
    if d_nll.shape != (N,) or lse.shape != (N,):
        raise ValueError("[cce_backward_noalloc] lse and d_nll must be [N]")
    ref = _ref_stats_layout(tile_max, N, c.shape[0], "cce_backward_noalloc")
    # caller-provided outputs are written through as raw pointers: they must be exactly
    # like the tensor whose gradient they hold
    for name, out, like in (("dE", dE, e), ("dC", dC, c), ("dB", dB, bias)):
        if out is not None and like is not None and (
                out.shape != like.shape or out.dtype != like.dtype or out.device != like.device
                or not out.is_contiguous()):
            raise ValueError(f"[cce_backward_noalloc] {name} must be a contiguous tensor like its input "
                             f"({tuple(like.shape)}, {like.dtype}, {like.device}), got "
                             f"{tuple(out.shape)}, {out.dtype}, {out.device}")
    if tile_stats is not None and (tile_stats.shape != (3,) or tile_stats.dtype != torch.int64
                                   or tile_stats.device != e.device or not tile_stats.is_contiguous()):
        raise ValueError("[cce_backward_noalloc] tile_stats must be a contiguous int64 [3] tensor on e's device")
    if want_de and dE is None:
        dE = torch.empty_like(e)
    if want_dc and dC is None:
        dC = torch.empty_like(c)
    if want_db and dB is None:
        dB = torch.empty_like(bias)
    dE, dC, dB = (dE if want_de else None), (dC if want_dc else None), (dB if want_db else None)
    eps = -math.inf if filter_eps is None else float(filter_eps)
    has_ignore = ignore_index is not None
    with torch.cuda.device(e.device):
        stream = torch.cuda.current_stream(e.device).cuda_stream
        rc = lib().cce_backward_noalloc(code, _ptr(e), _ptr(c), _ptr(bias), _ptr(targets),
                                        int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                        N, D, c.shape[0], _ptr(lse), _ptr(tile_max), _ptr(d_nll), ctypes.c_float(eps),
                                        _ptr(dE), _ptr(dC), _ptr(dB), _ptr(tile_stats),
                                        _bwd_opts["flags"] | (CCE_BWD_REF_STATS if ref else 0),
                                        ctypes.c_void_p(stream))
    if rc != CCE_OK:
        _raise(rc, "cce_backward_noalloc")
    return dE, dC, dB


# --------------------------------------------------------------------------
# Quantized classifier rows (MLX affine group quantization; see quant.py).

def _quant_parts(qw, D=None):
    w, sc, bi = qw.weight, qw.scales, qw.biases
    if w.dtype not in (torch.int32, torch.uint32):
        raise TypeError(f"[cce] quantized weight must be int32/uint32 words, got {w.dtype}")
    if sc.dtype not in DTYPE_CODES or bi.dtype != sc.dtype:
        raise TypeError("[cce] scales and biases must share one float dtype")
    if w.dim() != 2 or sc.dim() != 2 or bi.shape != sc.shape or sc.shape[0] != w.shape[0]:
        raise ValueError("[cce] weight [V, D*bits/32], scales and biases [V, D/group_size] expected")
    Dq = w.shape[1] * 32 // qw.bits
    if D is not None and Dq != D:
        raise ValueError(f"[cut_cross_entropy] quantized rows hold D={Dq}, e has D={D}")
    if sc.shape[1] * qw.group_size != Dq:
        raise ValueError("[cce] scales.shape[1] * group_size must equal D")
    return w.contiguous(), sc.contiguous(), bi.contiguous(), Dq


def dequantize(qw):
    """Dense [V, D] rows (dtype of the scales) of a QuantizedWeight (cce_dequantize)."""
    w, sc, bi, D = _quant_parts(qw)
    _check_device("weight", w, None)
    _check_device("scales", sc, w.device)
    _check_device("biases", bi, w.device)
    V = w.shape[0]
    out = torch.empty((V, D), dtype=sc.dtype, device=w.device)
    with torch.cuda.device(w.device):
        stream = torch.cuda.current_stream(w.device).cuda_stream
        rc = lib().cce_dequantize(DTYPE_CODES[sc.dtype], _ptr(w), _ptr(sc), _ptr(bi), qw.group_size, qw.bits, V, D,
                                  _ptr(out), ctypes.c_void_p(stream))
    if rc != CCE_OK:
        _raise(rc, "cce_dequantize")
    return out


def _prep_q(e, qw, targets, bias):
    if e.dim() != 2:
        raise ValueError(f"[cut_cross_entropy] e must be 2D [B, D], got {e.dim()}D")
    if targets.dim() != 1 or targets.shape[0] != e.shape[0]:
        raise ValueError("[cut_cross_entropy] targets must be 1D [B] with B = e.shape[0]")
    w, sc, bi, _ = _quant_parts(qw, e.shape[1])
    V = w.shape[0]
    if bias is not None and (bias.dim() != 1 or bias.shape[0] != V):
        raise ValueError("[cut_cross_entropy] bias must be 1D [V]")
    if e.dtype not in DTYPE_CODES:
        raise RuntimeError(f"CCE: unsupported dtype {e.dtype}")
    if sc.dtype != e.dtype or (bias is not None and bias.dtype != e.dtype):
        raise TypeError(f"[cut_cross_entropy] e, the scales and bias must share one dtype, got {e.dtype}, {sc.dtype}")
    dev = e.device
    _check_device("e", e, None)
    for name, t in (("weight", w), ("scales", sc), ("biases", bi), ("targets", targets)):
        _check_device(name, t, dev)
    if bias is not None:
        _check_device("bias", bias, dev)
    return DTYPE_CODES[e.dtype], w, sc, bi, V


def forward_q(e, qw, targets, bias=None, ignore_index=-100, chunk_rows=0):
    """forward() with quantized classifier rows (cce_forward_q): returns the same five tensors."""
    code, w, sc, bi, V = _prep_q(e, qw, targets, bias)
    e = e.contiguous()
    targets = targets.to(torch.int64).contiguous()
    if bias is not None:
        bias = bias.contiguous()
    N, D = e.shape
    nvt = (V + STAT_TILE - 1) // STAT_TILE
    f32 = dict(dtype=torch.float32, device=e.device)
    tile_max = torch.empty((nvt, N), **f32)
    tile_sum_exp = torch.empty((nvt, N), **f32)
    neg_tl = torch.empty((N,), **f32)
    lse = torch.empty((N,), **f32)
    nll = torch.empty((N,), **f32)
    sbytes = int(lib().cce_forward_q_scratch_size(code, V, D, int(chunk_rows)))
    scratch = torch.empty((max(sbytes, 1),), dtype=torch.uint8, device=e.device)
    has_ignore = ignore_index is not None
    with torch.cuda.device(e.device):
        stream = torch.cuda.current_stream(e.device).cuda_stream
        ev = _event_pair("forward")
        if ev:
            ev[0].record()
        rc = lib().cce_forward_q(code, _ptr(e), _ptr(w), _ptr(sc), _ptr(bi), qw.group_size, qw.bits, _ptr(bias),
                                 _ptr(targets), int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                 N, D, V, _ptr(tile_max), _ptr(tile_sum_exp), _ptr(neg_tl), _ptr(lse), _ptr(nll),
                                 _ptr(scratch), ctypes.c_size_t(sbytes), int(chunk_rows), ctypes.c_void_p(stream))
        if ev:
            ev[1].record()
    if rc != CCE_OK:
        _raise(rc, "cce_forward_q")
    return tile_max, tile_sum_exp, neg_tl, lse, nll


def backward_q(e, qw, targets, lse, tile_max, d_nll, bias=None, ignore_index=-100, filter_eps=FILTER_LOG_EPS,
               want_de=True, want_db=True, tile_stats=None, chunk_rows=0):
    """backward() with quantized classifier rows (cce_backward_q): returns (dE, dBias); the rows get no gradient."""
    code, w, sc, bi, V = _prep_q(e, qw, targets, bias)
    e = e.contiguous()
    targets = targets.to(torch.int64).contiguous()
    if bias is not None:
        bias = bias.contiguous()
    want_db = bool(want_db and bias is not None)
    N, D = e.shape
    lse = lse.contiguous()
    tile_max = tile_max.contiguous()
    d_nll = d_nll.to(torch.float32).contiguous()
    if d_nll.shape != (N,) or lse.shape != (N,):
        raise ValueError("[cce_backward] lse and d_nll must be [N]")
    dE = torch.empty_like(e) if want_de else None
    dB = torch.empty_like(bias) if want_db else None
    ws_bytes = int(lib().cce_backward_q_workspace_size(code, N, D, V, int(want_de), int(want_db), int(chunk_rows)))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=e.device)
    eps = -math.inf if filter_eps is None else float(filter_eps)
    has_ignore = ignore_index is not None
    with torch.cuda.device(e.device):
        stream = torch.cuda.current_stream(e.device).cuda_stream
        ev = _event_pair("backward")
        if ev:
            ev[0].record()
        rc = lib().cce_backward_q(code, _ptr(e), _ptr(w), _ptr(sc), _ptr(bi), qw.group_size, qw.bits, _ptr(bias),
                                  _ptr(targets), int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                  N, D, V, _ptr(lse), _ptr(tile_max), _ptr(d_nll), ctypes.c_float(eps),
                                  _ptr(dE), _ptr(dB), _ptr(ws), ctypes.c_size_t(ws_bytes), int(chunk_rows),
                                  _ptr(tile_stats), ctypes.c_void_p(stream))
        if ev:
            ev[1].record()
    if rc != CCE_OK:
        _raise(rc, "cce_backward_q")
    return dE, dB


# --------------------------------------------------------------------------
# Mirrors of the reference's native entry points (csrc/bindings.cpp:58-86).

def cce_forward_raw(e, c, targets, bias=None, *, ignore_index=None, stream=None, layout="reference"):
    """Reference csrc/bindings.cpp:58-69: returns [tile_max, tile_sum_exp, neg_target_logit, lse].

    layout "reference" (default): the statistics per 32 columns, flat [N * ceil(V/32)],
    row major per row of e -- the reference's own layout, which its glue reshapes to
    (B, (V + 31) // 32) (mlx_cce/__init__.py:25-30).  layout "tiles128": per 128
    columns, [ceil(V/128), N] (the layout the fused path keeps internally).  targets
    may be any integer dtype.
    """
    if layout not in ("reference", "tiles128"):
        raise ValueError(f"[cce_forward_raw] layout must be 'reference' or 'tiles128', got {layout!r}")
    ctx = torch.cuda.stream(stream) if stream is not None else _nullctx()
    with ctx:
        tm, ts, ntl, lse, _ = forward(e, c, targets, bias, ignore_index, ref_stats=layout == "reference")
    return [tm, ts, ntl, lse]


def cce_backward_raw(e, c, lse, targets, d_nll, tile_max, bias=None, *, ignore_index=None,
                     filter_eps=FILTER_LOG_EPS, compute_all_grads=False, stream=None):
    """Reference csrc/bindings.cpp:71-86: returns dE (in e.dtype).

    tile_max is cce_forward_raw's in either layout: the reference's flat
    [N * ceil(V/32)] (as its glue passes it back, tile_max.reshape(-1)) or
    [ceil(V/128), N].  With compute_all_grads=True returns (dE, dC, dBias) — the
    semantics of the reference's full-gradient kernel, reference/_fused_backward.py:1618-1655.
    """
    ctx = torch.cuda.stream(stream) if stream is not None else _nullctx()
    with ctx:
        dE, dC, dB = backward(e, c, targets, lse, tile_max, d_nll, bias, ignore_index, filter_eps,
                              True, compute_all_grads, compute_all_grads)
    if compute_all_grads:
        return dE, dC, dB
    return dE


class _nullctx:
    def __enter__(self):
        return self

    def __exit__(self, *a):
        return False


def reduce_loss(nll, targets, ignore_index, reduction):
    """Reduced loss of the per-token nll ('sum' or 'mean'); returns (loss, scale).

    scale is max(count of rows kept by the ignore mask, 1) for 'mean', else None.
    Both are fp32 device tensors of shape () (one deterministic workgroup reduction).
    """
    N = nll.shape[0]
    mode = CCE_REDUCE_MEAN if reduction == "mean" else CCE_REDUCE_SUM
    loss = torch.empty((), dtype=torch.float32, device=nll.device)
    scale = torch.empty((), dtype=torch.float32, device=nll.device) if mode == CCE_REDUCE_MEAN else None
    has_ignore = ignore_index is not None
    t = targets.to(torch.int64).contiguous()
    with torch.cuda.device(nll.device):
        stream = torch.cuda.current_stream(nll.device).cuda_stream
        rc = lib().cce_reduce_loss(_ptr(nll), _ptr(t), int(ignore_index) if has_ignore else 0, 1 if has_ignore else 0,
                                   N, mode, _ptr(loss), _ptr(scale), ctypes.c_void_p(stream))
    if rc != CCE_OK:
        _raise(rc, "cce_reduce_loss")
    return loss, scale


def broadcast_grad(grad, scale, N):
    """d_nll [N] fp32 = grad / scale (scale None: grad) for a scalar upstream gradient."""
    g = grad.to(torch.float32).reshape(1).contiguous()
    d_nll = torch.empty((N,), dtype=torch.float32, device=g.device)
    with torch.cuda.device(g.device):
        stream = torch.cuda.current_stream(g.device).cuda_stream
        rc = lib().cce_broadcast_grad(_ptr(g), _ptr(scale), N, _ptr(d_nll), ctypes.c_void_p(stream))
    if rc != CCE_OK:
        _raise(rc, "cce_broadcast_grad")
    return d_nll
