"""Pin the oracle's filter emulation -- CPU only.

The GPU kept-tile assertions and the filtered-gradient bounds rest on three oracle
functions: ``keep_mask`` (this build's blocking), ``reference_keep_mask`` (the
reference's 32 x 32 predicate, csrc/cce/cce.metal:191-204, with ignored rows'
targets sanitised to 0 as mlx_cce/__init__.py:59-61 does) and ``grads_filtered``.
They are checked here against what they were not written from:

* a pure-Python brute force that states the predicate over individual softmax
  probabilities -- a (block, tile) pair is kept iff some counted row of the block
  has its target in the tile or some probability there of at least 2^-12 -- on
  logits built by hand (E = the logits, C = the identity), with planted entries a
  little above and below the threshold, a tile kept only by a target, an ignored
  row, a row with zero cotangent, and ragged last tiles and blocks;
* known answers written out for those inputs, and the exact-threshold case
  (tile_max - lse == ln 2^-12, kept: the reference compares with >=);
* loops that zero G outside the kept tiles and form dE, dC, dBias entry by entry;
* one planted mutant per clause (the target clause dropped, > for >=, inactive rows
  counted, ignored rows not marking tile 0, the row and column blockings swapped),
  each of which must fail these checks while the oracle passes them.
"""

import math

import numpy as np
import pytest

from oracle import cce_oracle as O

EPS = O.FILTER_LOG_EPS  # ln 2^-12 (csrc/cce/cce.metal:143)
P_EPS = 2.0 ** -12
DELTA = 1e-3  # planted log-probabilities sit this far from the threshold
N = V = 300   # 3 blocks / tiles of 128 (the last 44 wide), 10 of 32 (the last 12 wide)


def _plant(S, r, v, logprob):
    """Set S[r, v] so that S[r, v] - lse(S[r]) == logprob (fixed point; p << 1)."""
    x = logprob
    for _ in range(60):
        S[r, v] = x
        m = S[r].max()
        lse = m + math.log(np.exp(S[r] - m).sum())
        x = logprob + lse
    S[r, v] = x


def hand_case():
    """Logits [N, V], targets, d_nll of the hand-built case, and what each row does.

    Every row puts its bulk (logit 0, p ~ 1) on its target, column 64 + r % 32 (the
    128-wide tile 0, the 32-wide tile 2); every other logit is -20 (p ~ 2e-9), except:
      row 5    p = 2^-12 e^+d at column 140  (128-tile 1, 32-tile 4): hot
      row 6    p = 2^-12 e^-d at column 260  (128-tile 2, 32-tile 8): cold
      row 10   ignored (target -100), hot at column 280 (128-tile 2, 32-tile 8)
      row 40   ignored, no planted entry (32-tile 0 of block 1 only by the reference's
               sanitised target 0)
      row 130  target 200 (128-tile 1, 32-tile 6) with p ~ 2e-9 there: kept by the
               target alone; its bulk on column 3 (32-tile 0)
      row 140  hot at column 270 (128-tile 2, 32-tile 8)
      row 280  d_nll = 0, hot at column 299 (the ragged last column)
      row 290  hot at column 150 (128-tile 1, 32-tile 4), in the ragged last block
    """
    S = np.full((N, V), -20.0)
    bulk = np.array([64 + r % 32 for r in range(N)])
    bulk[130] = 3
    S[np.arange(N), bulk] = 0.0
    t = bulk.astype(np.int64)
    t[10] = -100
    t[40] = -100
    t[130] = 200
    for r, v, lp in ((5, 140, EPS + DELTA), (6, 260, EPS - DELTA), (10, 280, EPS + DELTA), (140, 270, EPS + DELTA),
                     (280, 299, EPS + DELTA), (290, 150, EPS + DELTA)):
        _plant(S, r, v, lp)
    dn = np.full(N, 1.0 / N)
    dn[280] = 0.0
    return S, t, dn


def brute_keep(S, t, dn, rows, cols, counted_by_dnll, ignored_marks_tile0, ignore_index=-100):
    """keep[tile][block] by the predicate over individual probabilities, in Python loops."""
    n, nv = len(S), len(S[0])
    lse = []
    for r in range(n):
        m = max(S[r])
        lse.append(m + math.log(sum(math.exp(x - m) for x in S[r])))
    nvt, nrb = -(-nv // cols), -(-n // rows)
    keep = [[False] * nrb for _ in range(nvt)]
    for rb in range(nrb):
        for r in range(rb * rows, min((rb + 1) * rows, n)):
            ignored = t[r] == ignore_index
            if counted_by_dnll and (ignored or dn[r] == 0):
                continue
            tr = 0 if (ignored and ignored_marks_tile0) else t[r]
            for vt in range(nvt):
                if keep[vt][rb]:
                    continue
                if vt * cols <= tr < (vt + 1) * cols:
                    keep[vt][rb] = True
                    continue
                for v in range(vt * cols, min((vt + 1) * cols, nv)):
                    if math.exp(S[r][v] - lse[r]) >= P_EPS:
                        keep[vt][rb] = True
                        break
    return np.array(keep)


def build_keep(fn, S, t, dn, rows, cols):
    """fn (keep_mask or a mutant) on the statistics of S at `cols`-wide tiles."""
    eye = np.eye(V)
    tm, _ = O.tile_stats(S, eye, None, tile=cols)
    _, lse = O.linear_cross_entropy(S, eye, t, None, "none", return_lse=True)
    return fn(tm, lse, t, dn, rows=rows, cols=cols)


# ------------------------------------------------------------------- mutants
def keep_no_target_clause(tile_max, lse, targets, d_nll, ignore_index=-100, rows=128, cols=128, eps=EPS):
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    active = (np.asarray(d_nll) != 0) & O.valid_mask(t, ignore_index)
    nrb = -(-t.shape[0] // rows)
    keep = np.zeros((tile_max.shape[0], nrb), dtype=bool)
    for vt in range(tile_max.shape[0]):
        row_keep = active & ((tile_max[vt] - lse) >= eps)
        for rb in range(nrb):
            keep[vt, rb] = row_keep[rb * rows:(rb + 1) * rows].any()
    return keep


def keep_strict(tile_max, lse, targets, d_nll, ignore_index=-100, rows=128, cols=128, eps=EPS):
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    active = (np.asarray(d_nll) != 0) & O.valid_mask(t, ignore_index)
    nrb = -(-t.shape[0] // rows)
    keep = np.zeros((tile_max.shape[0], nrb), dtype=bool)
    for vt in range(tile_max.shape[0]):
        hit = (t >= vt * cols) & (t < (vt + 1) * cols)
        row_keep = active & (hit | ((tile_max[vt] - lse) > eps))
        for rb in range(nrb):
            keep[vt, rb] = row_keep[rb * rows:(rb + 1) * rows].any()
    return keep


def keep_all_rows(tile_max, lse, targets, d_nll, ignore_index=-100, rows=128, cols=128, eps=EPS):
    t = np.asarray(targets).reshape(-1).astype(np.int64)
    nrb = -(-t.shape[0] // rows)
    keep = np.zeros((tile_max.shape[0], nrb), dtype=bool)
    for vt in range(tile_max.shape[0]):
        hit = (t >= vt * cols) & (t < (vt + 1) * cols)
        row_keep = hit | ((tile_max[vt] - lse) >= eps)
        for rb in range(nrb):
            keep[vt, rb] = row_keep[rb * rows:(rb + 1) * rows].any()
    return keep


def ref_keep_no_tile0(e, c, targets, bias=None, ignore_index=-100, eps=EPS):
    s = O.logits(e, c, bias)
    lse = O.logsumexp_rows(s)
    n, nv = s.shape
    t = np.asarray(targets).reshape(-1).astype(np.int64)  # not sanitised: ignored rows hit nothing
    nvt, nrb = -(-nv // 32), -(-n // 32)
    keep = np.zeros((nvt, nrb), dtype=bool)
    for vt in range(nvt):
        m = s[:, vt * 32:(vt + 1) * 32].max(axis=1)
        row_keep = ((t >= vt * 32) & (t < (vt + 1) * 32)) | ((m - lse) >= eps)
        for rb in range(nrb):
            keep[vt, rb] = row_keep[rb * 32:(rb + 1) * 32].any()
    return keep


def grads_filtered_swapped(e, c, targets, keep, rows, cols, bias=None, d_nll=None, ignore_index=-100):
    G = O.grad_logits(e, c, targets, bias, d_nll, ignore_index)
    n, nv = G.shape
    mask = np.zeros((n, nv), dtype=bool)
    for vt in range(keep.shape[0]):
        for rb in range(keep.shape[1]):
            if keep[vt, rb]:
                mask[vt * cols:(vt + 1) * cols, rb * rows:(rb + 1) * rows] = True  # blockings swapped
    G = np.where(mask, G, 0.0)
    return G @ O._f64(c), G.T @ O._f64(e), (G.sum(axis=0) if bias is not None else None)


# -------------------------------------------------------------------- checks
def check_build_keep(fn):
    """fn agrees with the brute force at 128 x 128 (the backward's blocking), 32 x 32 and
    64 x 32, and with the known answers; returns False on the first disagreement."""
    S, t, dn = hand_case()
    for rows, cols in ((128, 128), (32, 32), (64, 32)):
        got = build_keep(fn, S, t, dn, rows, cols)
        want = brute_keep(S, t, dn, rows, cols, counted_by_dnll=True, ignored_marks_tile0=False)
        if got.shape != want.shape or not (got == want).all():
            return False
    got = build_keep(fn, S, t, dn, 128, 128)
    known = np.array([[1, 1, 1],   # tile 0: every row's bulk
                      [1, 1, 1],   # tile 1: row 5 hot, row 130's target alone, row 290 hot
                      [0, 1, 0]],  # tile 2: row 6 cold, row 10 ignored; row 140 hot; row 280 d_nll = 0
                     dtype=bool)
    if not (got == known).all():
        return False
    # exactly at the threshold: kept (the reference's comparison is >=)
    tm = np.full((1, 4), -30.0)
    tm[0, 2] = EPS
    lse = np.zeros(4)
    at = fn(tm, lse, np.array([900, 901, 902, 903]), np.ones(4), rows=2, cols=128)
    return bool((at == np.array([[False, True]])).all())


def check_reference_keep(fn):
    S, t, dn = hand_case()
    got = fn(S, np.eye(V), t)
    want = brute_keep(S, t, dn, 32, 32, counted_by_dnll=False, ignored_marks_tile0=True)
    if got.shape != want.shape or not (got == want).all():
        return False
    # known answers ([tile][block] of 32): the ignored row 40 alone keeps tile 0 of block
    # 1 (its target sanitised to 0); the d_nll = 0 row 280 and the ignored row 10 still
    # count with their hot entries (the reference does not consult d_nll); row 130's
    # target alone keeps tile 6 of block 4; nothing keeps tile 7 of block 4 or tile 8 of
    # block 1
    kept = (got[0, 1], got[9, 8], got[8, 0], got[8, 4], got[6, 4], got[4, 0], got[4, 9])
    return bool(all(kept) and not got[7, 4] and not got[8, 1])


def _loops_filtered(S, t, dn, keep, rows, cols):
    """G of logits S by loops, zero outside the kept [tile][block] pairs."""
    n, nv = S.shape
    lse = [max(S[r]) + math.log(sum(math.exp(x - max(S[r])) for x in S[r])) for r in range(n)]
    G = [[0.0] * nv for _ in range(n)]
    for r in range(n):
        if t[r] == -100:
            continue
        for v in range(nv):
            if keep[v // cols][r // rows]:
                G[r][v] = dn[r] * (math.exp(S[r][v] - lse[r]) - (1.0 if v == t[r] else 0.0))
    return G


def check_grads_filtered(fn):
    """fn against loops over a small ragged case (rows 8 x cols 16 tiles, 20 x 40) with a
    bias and an ignored row, and a keep pattern that is not symmetric."""
    rng = np.random.default_rng(31)
    n, nv, d = 20, 40, 6
    e = rng.standard_normal((n, d))
    c = rng.standard_normal((nv, d))
    b = rng.standard_normal(nv) * 0.3
    t = rng.integers(0, nv, n)
    t[4] = -100
    dn = np.where(t != -100, 1.0 / n, 0.0)
    rows, cols = 8, 16
    keep = np.zeros((3, 3), dtype=bool)  # [tile][block]
    keep[0, 0] = keep[2, 1] = keep[1, 2] = keep[0, 2] = True
    S = (e @ c.T + b[None, :]).tolist()
    G = _loops_filtered(np.array(S), t, dn, keep, rows, cols)
    dE = [[sum(G[r][v] * c[v][k] for v in range(nv)) for k in range(d)] for r in range(n)]
    dC = [[sum(G[r][v] * e[r][k] for r in range(n)) for k in range(d)] for v in range(nv)]
    dB = [sum(G[r][v] for r in range(n)) for v in range(nv)]
    got = fn(e, c, t, keep, rows, cols, b, d_nll=dn)
    return all(np.allclose(x, np.array(y), rtol=1e-12, atol=1e-15) for x, y in zip(got, (dE, dC, dB)))


# --------------------------------------------------------------------- tests
def test_hand_case_is_what_it_claims():
    """The planted entries sit DELTA on either side of ln 2^-12 and the rest far below."""
    S, t, dn = hand_case()
    lse = O.logsumexp_rows(S)
    lp = S - lse[:, None]
    for r, v, side in ((5, 140, 1), (6, 260, -1), (10, 280, 1), (140, 270, 1), (280, 299, 1), (290, 150, 1)):
        assert abs(lp[r, v] - (EPS + side * DELTA)) < 1e-12
    assert lp[130, 200] < -19 and t[130] == 200  # row 130's target carries no probability


def test_keep_mask_pinned():
    assert check_build_keep(O.keep_mask)


def test_reference_keep_mask_pinned():
    assert check_reference_keep(O.reference_keep_mask)


def test_grads_filtered_pinned():
    assert check_grads_filtered(O.grads_filtered)


@pytest.mark.parametrize("mutant", [keep_no_target_clause, keep_strict, keep_all_rows], ids=lambda f: f.__name__)
def test_keep_mask_mutants_are_caught(mutant):
    assert not check_build_keep(mutant)


def test_reference_keep_mask_mutant_is_caught():
    assert not check_reference_keep(ref_keep_no_tile0)


def test_grads_filtered_mutant_is_caught():
    assert not check_grads_filtered(grads_filtered_swapped)
