"""CPU oracle for Cut Cross-Entropy — TEST INFRASTRUCTURE, NOT THE PRODUCT.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker (or the timed CPU
baseline).  The HIP library never calls into it.

A float64 numpy restatement of the reference's semantics, computed from the
exact (already dtype-rounded) inputs, so its own rounding error (~1e-15) is far
below every tolerance it checks:

* ``linear_cross_entropy``: reference/_reference.py:5-48 (shift :15-17, flatten
  :19-22, logits + bias :24-26, per-sample CE :28, lse :30-31, ignore mask :33-34,
  reductions :36-44 with mean = sum / max(count, 1)) and the drop-in API
  mlx_cce/__init__.py:54-107 (ignore_index=None means all rows valid :62-64).
* ``grads``: the closed form of the CE gradient, G = g (softmax - onehot),
  dE = G C, dC = G^T E, dBias = colsum G — the quantities the reference's full
  gradient kernel accumulates (reference/_fused_backward.py:1519-1553, weight
  formula w = d_nll exp(S + b - lse) - d_nll [v == t] at :1512-1517).
* ``tile_stats``: per-(vocab tile, row) max and sum-exp (csrc/cce/cce.metal:117-133,
  combined per cce.metal:339-354), here at this build's 128-column tiles.
* ``keep_mask``: this build's filter at (128 rows x 128 columns) granularity.
* ``reference_keep_mask``: the reference's own filter at 32 x 32 granularity
  (cce.metal:191-204), including its treatment of ignored rows as target 0
  (mlx_cce/__init__.py:61).
* ``grads_filtered``: the gradients restricted to kept tiles (what a filtered
  backward computes).
* ``round_bf16`` / ``round_f16``: round-to-nearest-even to the 16-bit types through
  float32, the rounding of the library's 16-bit stores.  Pinned against torch's own
  conversion on every kind of value (ties, subnormals, overflow) and by a planted
  truncation that must fail.
* ``grads_staged``: the gradients with G rounded to a 16-bit type before the two
  products, as a backward that stores its G tiles in the input dtype computes them
  (dBias from the unrounded G, as the column sums are taken before the store).
  Pinned by reducing to ``grads`` with the identity as the rounding, and by a case
  where the rounding of G provably moves dE.
* ``dequantize``: affine group dequantization of quantized classifier rows, the
  layout of MLX's mx.quantize / mx.dequantize (mlx >= 0.22, absent here), which the
  reference's callers apply before the loss (README.md:84-95,136;
  examples/mlx_lm_lora_test.py:16-21): code j of a uint32 word in bits
  [j bits, (j + 1) bits), w = scale q + bias.  The product and the add are float32
  (the library's rounding).  Pinned by a pure-Python bit-by-bit brute force, by
  cases exact in any rounding order (power-of-two scales, small integer biases),
  and by a planted code-order mistake; MLX's own rounding of scale q + bias is
  parity unpinned (MLX cannot run here).

How each function is pinned (tests/test_oracle.py): pure-Python brute force on
tiny inputs, an independent float64 torch autograd of materialised logits,
central finite differences, closed-form special cases (zero weights give
nll = log V exactly; equal logits; V = 1), invariants (rows of G sum to 0, so
sum(dBias) = 0; <E, dE> = <C, dC> without bias; linearity in the upstream
gradient), and planted mistakes that those checks must catch.
"""

import numpy as np

FILTER_LOG_EPS = -8.3177661667  # ln(2^-12), reference csrc/cce/cce.metal:143
STAT_TILE = 128
BWD_ROWS = 128
REF_TILE = 32  # reference tile (cce.metal:34,168)


def _f64(x):
    return None if x is None else np.asarray(x, dtype=np.float64)


def logits(e, c, bias=None):
    """S = e c^T (+ bias) in float64 (reference/_reference.py:24-26)."""
    s = _f64(e) @ _f64(c).T
    if bias is not None:
        s = s + _f64(bias)[None, :]
    return s


def logsumexp_rows(s):
    m = np.max(s, axis=1, keepdims=True)
    m = np.where(np.isfinite(m), m, 0.0)
    return (m + np.log(np.sum(np.exp(s - m), axis=1, keepdims=True)))[:, 0]


def valid_mask(targets, ignore_index):
    t = np.asarray(targets).reshape(-1)
    if ignore_index is None:
        return np.ones(t.shape, dtype=bool)
    return t != ignore_index


def per_token(e, c, targets, bias=None, ignore_index=-100):
    """(nll [N] masked to 0 on ignored rows, lse [N], valid [N]) for e [N, D]."""
    s = logits(e, c, bias)
    lse = logsumexp_rows(s)
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    valid = valid_mask(t, ignore_index)
    safe = np.where(valid, t, 0)
    tgt = s[np.arange(s.shape[0]), safe]
    nll = np.where(valid, lse - tgt, 0.0)
    return nll, lse, valid


def reduce_loss(nll, valid, reduction):
    if reduction == "none":
        return nll
    if reduction == "sum":
        return nll.sum()
    if reduction == "mean":
        return nll.sum() / max(int(valid.sum()), 1)
    raise ValueError(f"Unknown reduction: {reduction!r}")


def linear_cross_entropy(e, c, targets, bias=None, reduction="mean", ignore_index=-100, shift=0,
                         return_lse=False):
    """reference/_reference.py:5-48 in float64 (e [..., D], targets [...])."""
    e = _f64(e)
    t = np.asarray(targets)
    if shift > 0:
        e = e[..., :-shift, :]
        t = t[..., shift:]
    orig_shape = t.shape
    nll, lse, valid = per_token(e.reshape(-1, e.shape[-1]), c, t.reshape(-1), bias, ignore_index)
    loss = reduce_loss(nll, valid, reduction)
    if reduction == "none":
        loss = loss.reshape(orig_shape)
    return (loss, lse) if return_lse else loss


def upstream(valid, reduction, grad_out=1.0):
    """d loss / d nll_r for the given reduction (the d_nll the backward receives)."""
    n = valid.shape[0]
    if reduction == "none":
        g = np.broadcast_to(np.asarray(grad_out, dtype=np.float64), (n,)).copy()
    elif reduction == "sum":
        g = np.full(n, float(grad_out))
    elif reduction == "mean":
        g = np.full(n, float(grad_out) / max(int(valid.sum()), 1))
    else:
        raise ValueError(f"Unknown reduction: {reduction!r}")
    return np.where(valid, g, 0.0)


def grad_logits(e, c, targets, bias=None, d_nll=None, ignore_index=-100):
    """G = d_nll (softmax - onehot) [N, V] in float64."""
    s = logits(e, c, bias)
    lse = logsumexp_rows(s)
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    valid = valid_mask(t, ignore_index)
    p = np.exp(s - lse[:, None])
    rows = np.nonzero(valid)[0]
    p[rows, t[rows]] -= 1.0
    g = np.where(valid, np.asarray(d_nll, dtype=np.float64), 0.0)
    return p * g[:, None]


def grads(e, c, targets, bias=None, reduction="mean", ignore_index=-100, grad_out=1.0, d_nll=None):
    """(dE, dC, dBias) in float64 for e [N, D]; dBias is None without bias."""
    t = np.asarray(targets).reshape(-1)
    valid = valid_mask(t, ignore_index)
    if d_nll is None:
        d_nll = upstream(valid, reduction, grad_out)
    G = grad_logits(e, c, t, bias, d_nll, ignore_index)
    dE = G @ _f64(c)
    dC = G.T @ _f64(e)
    dB = G.sum(axis=0) if bias is not None else None
    return dE, dC, dB


def tile_stats(e, c, bias=None, tile=STAT_TILE):
    """(tile_max, tile_sum_exp), each [ceil(V/tile), N], float64."""
    s = logits(e, c, bias)
    N, V = s.shape
    nvt = (V + tile - 1) // tile
    tm = np.empty((nvt, N))
    ts = np.empty((nvt, N))
    for k in range(nvt):
        blk = s[:, k * tile:(k + 1) * tile]
        m = blk.max(axis=1)
        tm[k] = m
        ts[k] = np.exp(blk - m[:, None]).sum(axis=1)
    return tm, ts


def keep_mask(tile_max, lse, targets, d_nll, ignore_index=-100, rows=BWD_ROWS, cols=STAT_TILE,
              eps=FILTER_LOG_EPS):
    """This build's filter: keep[vt, rb] for cols-wide vocab tiles x rows-row token blocks.

    Kept iff some row r of the block with d_nll[r] != 0 (and not ignored) has its
    target in the tile or tile_max[vt, r] - lse[r] >= eps.
    """
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    N = t.shape[0]
    nvt = tile_max.shape[0]
    nrb = (N + rows - 1) // rows
    active = (np.asarray(d_nll) != 0) & valid_mask(t, ignore_index)
    keep = np.zeros((nvt, nrb), dtype=bool)
    for vt in range(nvt):
        hit = (t >= vt * cols) & (t < (vt + 1) * cols)
        hot = (tile_max[vt] - lse) >= eps
        row_keep = active & (hit | hot)
        for rb in range(nrb):
            keep[vt, rb] = row_keep[rb * rows:(rb + 1) * rows].any()
    return keep


def reference_keep_mask(e, c, targets, bias=None, ignore_index=-100, eps=FILTER_LOG_EPS):
    """Reference filter (csrc/cce/cce.metal:191-204) on 32 x 32 tiles: keep[vt32, rb32].

    Follows the reference exactly: targets of ignored rows are sanitised to 0
    (mlx_cce/__init__.py:61) and still mark tile 0; d_nll is not consulted.
    """
    s = logits(e, c, bias)
    lse = logsumexp_rows(s)
    N, V = s.shape
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    safe = np.where(valid_mask(t, ignore_index), t, 0)
    nvt = (V + REF_TILE - 1) // REF_TILE
    nrb = (N + REF_TILE - 1) // REF_TILE
    keep = np.zeros((nvt, nrb), dtype=bool)
    for vt in range(nvt):
        m = s[:, vt * REF_TILE:(vt + 1) * REF_TILE].max(axis=1)
        hit = (safe >= vt * REF_TILE) & (safe < (vt + 1) * REF_TILE)
        row_keep = hit | ((m - lse) >= eps)
        for rb in range(nrb):
            keep[vt, rb] = row_keep[rb * REF_TILE:(rb + 1) * REF_TILE].any()
    return keep


def grads_filtered(e, c, targets, keep, rows, cols, bias=None, d_nll=None, ignore_index=-100):
    """(dE, dC, dBias) using only the G entries inside kept (cols x rows) tiles."""
    G = grad_logits(e, c, targets, bias, d_nll, ignore_index)
    N, V = G.shape
    mask = np.zeros((N, V), dtype=bool)
    nvt, nrb = keep.shape
    for vt in range(nvt):
        for rb in range(nrb):
            if keep[vt, rb]:
                mask[rb * rows:(rb + 1) * rows, vt * cols:(vt + 1) * cols] = True
    G = np.where(mask, G, 0.0)
    dE = G @ _f64(c)
    dC = G.T @ _f64(e)
    dB = G.sum(axis=0) if bias is not None else None
    return dE, dC, dB


def round_bf16(x):
    """x rounded to the nearest bfloat16 (ties to even) through float32, as float64.
    NaN and infinities pass through; values past the largest bfloat16 round to inf."""
    x32 = np.asarray(x, dtype=np.float32)
    b = x32.view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return np.where(np.isnan(x32), x32, r).astype(np.float64)


def round_f16(x):
    """x rounded to the nearest float16 (ties to even) through float32, as float64."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float64)


def grads_staged(e, c, targets, bias=None, reduction="mean", ignore_index=-100, grad_out=1.0, d_nll=None,
                 stage=None):
    """(dE, dC, dBias) with G passed through `stage` (a rounding, or None for none)
    before dE = G C and dC = G^T E; dBias sums the unrounded G."""
    t = np.asarray(targets).reshape(-1)
    valid = valid_mask(t, ignore_index)
    if d_nll is None:
        d_nll = upstream(valid, reduction, grad_out)
    G = grad_logits(e, c, t, bias, d_nll, ignore_index)
    Gs = G if stage is None else stage(G)
    dE = Gs @ _f64(c)
    dC = Gs.T @ _f64(e)
    dB = G.sum(axis=0) if bias is not None else None
    return dE, dC, dB


def rel_fro(got, ref):
    """Relative Frobenius error ||got - ref|| / ||ref|| (0 if both are 0)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    num = np.linalg.norm(got - ref)
    if den == 0.0:
        return 0.0 if num == 0.0 else float("inf")
    return float(num / den)


def dequantize(words, scales, biases, group_size, bits):
    """float32 [V, D] rows from quantized words [V, D bits / 32] (uint32 bit patterns,
    any integer dtype) and scales / biases [V, D / group_size]: code j of a word in
    bits [j bits, (j + 1) bits), w = float32(float32(scale) q) + float32(bias)."""
    w = np.asarray(words).astype(np.int64) & 0xFFFFFFFF
    V, W = w.shape
    epw = 32 // bits
    shifts = np.arange(epw, dtype=np.int64) * bits
    q = ((w[:, :, None] >> shifts) & ((1 << bits) - 1)).reshape(V, W * epw)
    D = W * epw
    s = np.repeat(np.asarray(scales, dtype=np.float32), group_size, axis=1)[:, :D]
    b = np.repeat(np.asarray(biases, dtype=np.float32), group_size, axis=1)[:, :D]
    return (s * q.astype(np.float32)).astype(np.float32) + b

