"""CPU restatements of the backward's index logic, checked against what it must compute.

Each function below restates, step for step, the indexing of one piece of device code
(the kernel named in its docstring), so that a mistake in the restated scheme -- a lost
row, an index past its array, two writers of one slot -- fails here, on the CPU:

- the counting sort of the token order (`csort_rows`, cce_bwd.hip) against the stable
  sort by target tile with the rare targets spread over the blocks, the order the
  backward's token blocks are defined by (the reference has no counterpart: it runs
  its filter on input-order blocks, cce.metal:191-204);
- the dC block tasks (the compaction's lists, `bwd_compact_kernel`, and the walk of the
  narrow dC sums, `bwd_sum_narrow_kernel`) against the set of one-tile owners and slices;
- the 16-bit epilogue's transpose through LDS (`bwd_sum_narrow_kernel`): a bijection from
  the MFMA register layout to whole 128-byte row pieces, free of LDS bank conflicts;
- the G task lists (`bwd_compact_kernel`) in their three kinds, against the slots they
  must cover: every kept pair once, in runs of at most R slots of one (pass, token block),
  or of at most 4 vt_slot entries of one vocabulary tile;
- the dE sums' pieces (`bwd_sum_narrow_kernel`, `bwd_de_pieces_kernel`): with few tasks
  each is cut along its kept tiles, every tile summed by one piece, every piece's fp32
  partial in its own slot and added once, in order, by the finishing kernel.
"""
import numpy as np
import pytest

HEAD_RUN = 16  # kSortHeadRun
BLOCK = 128    # kBwdTokens == kBwdVocab


def token_order(tt, d_nll, V, ignore_index=-100):
    """The definition: rows stably sorted by the 128-column tile of their target (rows
    without gradient keyed past the last tile); rows of keys with fewer than HEAD_RUN
    rows dealt evenly over the 128-row blocks, each block taking its share of them
    first, then the next rows of the long runs.  perm[p] = input row at position p."""
    N = len(tt)
    nvt = (V + BLOCK - 1) // BLOCK
    act = (d_nll != 0) & (tt != ignore_index) & (tt >= 0) & (tt < V)
    key = np.where(act, tt // BLOCK, nvt)
    srt = np.argsort(key, kind="stable")
    head = np.bincount(key, minlength=nvt + 1)[key[srt]] >= HEAD_RUN
    heads, tails = srt[head], srt[~head]
    nT, nrb = len(tails), (N + BLOCK - 1) // BLOCK
    tb = [min(BLOCK * b, N) * nT // N for b in range(nrb + 1)]
    perm, h = np.empty(N, dtype=np.int64), 0
    for b in range(nrb):
        p0, nt = BLOCK * b, tb[b + 1] - tb[b]
        perm[p0:p0 + nt] = tails[tb[b]:tb[b + 1]]
        nh = min(BLOCK * (b + 1), N) - p0 - nt
        perm[p0 + nt:p0 + nt + nh] = heads[h:h + nh]
        h += nh
    return perm


def lifting_search(r, f, nrb, maxr, top=None):
    """The kernel's block search: binary lifting over the steps top = 4 MAXR, ..., 1
    (every candidate c <= 8 MAXR - 1 reads the table at min(c, nrb))."""
    lo, step = 0, 4 * maxr if top is None else top
    while step >= 1:
        c = lo + step
        if c < nrb and f(min(c, nrb)) <= r:
            lo = c
        step >>= 1
    return lo


def bisection_search(r, f, nrb):
    lo, hi = 0, nrb - 1
    while lo < hi:
        mid = (lo + hi + 1) >> 1
        if f(mid) <= r:
            lo = mid
        else:
            hi = mid - 1
    return lo


@pytest.mark.parametrize("seed", range(6))
def test_block_search_lifting_equals_bisection(seed):
    """For every non-decreasing table from 0 (the head and tail rows before each block)
    and every rank, the lifting search finds the bisection's block; starting one step
    short (2 MAXR) misses the last blocks once nrb > 4 MAXR."""
    rng = np.random.default_rng(seed)
    for maxr in (8, 16):
        for nrb in (1, 2, 3, 31, 32, 33, 4 * maxr, 4 * maxr + 1, 8 * maxr - 1, 8 * maxr):
            steps = rng.integers(0, 130, nrb + 1)
            steps[0] = 0
            tab = np.cumsum(steps)
            f = lambda b: int(tab[b])
            for r in range(0, int(tab[nrb]) + 2, max(1, int(tab[nrb]) // 300)):
                assert lifting_search(r, f, nrb, maxr) == bisection_search(r, f, nrb)
    tab = np.arange(0, 128 * 65, 128)  # 64 blocks of 128 rows
    f = lambda b: int(tab[b])
    r = int(tab[63]) + 5
    assert bisection_search(r, f, 64) == 63
    assert lifting_search(r, f, 64, 8) == 63
    assert lifting_search(r, f, 64, 8, top=16) != 63  # the short-step mutant


def csort_restated(tt, d_nll, V, ignore_index=-100, maxr=16, nkeys=2048, wave_prefix=True):
    """csort_rows: wave w holds rows [w S, (w+1) S), S = ceil(N / 16), 64 per round;
    per round a lane's rank is its wave's running count of its key plus the lower lanes
    with that key (the highest of them advances the 16-bit counter); per key the 16
    counters become a prefix over the waves; head / tail starts come from scans over
    the keys; the block placement searches the per-block head / tail counts by binary
    lifting over the steps 4 MAXR, ..., 2, 1 (MAXR 8 up to N = 8192, else 16)."""
    N = len(tt)
    nvt = (V + BLOCK - 1) // BLOCK
    assert nvt < nkeys and N <= 1024 * maxr
    act = (d_nll != 0) & (tt != ignore_index) & (tt >= 0) & (tt < V)
    key = np.where(act, tt // BLOCK, nvt)
    S = (N + 15) >> 4
    cnt = np.zeros((16, nkeys), dtype=np.int64)
    rank = np.zeros(N, dtype=np.int64)
    for w in range(16):
        for j in range(maxr):
            if j * 64 >= S:
                continue
            lanes = [l for l in range(64) if j * 64 + l < S and w * S + j * 64 + l < N]
            seen = {}
            for l in lanes:  # lanes in order: the lower lanes with the key come first
                row = w * S + j * 64 + l
                k = key[row]
                rank[row] = cnt[w, k] + seen.get(k, 0)
                seen[k] = seen.get(k, 0) + 1
            for k, c in seen.items():
                cnt[w, k] += c
                assert cnt[w, k] < 1 << 16  # 16-bit counters
    tot = np.zeros(nkeys, dtype=np.int64)
    for k in range(nvt + 1):
        run = 0
        for w in range(16):
            c = cnt[w, k]
            cnt[w, k] = run if wave_prefix else 0
            run += c
        tot[k] = run
    is_head = tot >= HEAD_RUN
    hs = np.concatenate([[0], np.cumsum(np.where(is_head, tot, 0))])
    allst = np.concatenate([[0], np.cumsum(tot)])
    nH = int(hs[nkeys])
    nT, nrb = N - nH, (N + BLOCK - 1) // BLOCK
    tbl = [min(b * BLOCK, N) * nT // N for b in range(nrb + 1)]

    def last_block(r, before):  # the last block b < nrb with before(b) <= r
        return lifting_search(r, before, nrb, 8 if N <= 8192 else 16)

    perm = np.full(N, -1, dtype=np.int64)
    for row in range(N):
        k, w = key[row], row // S
        start = hs[k] if is_head[k] else allst[k] - hs[k]
        r = start + cnt[w, k] + rank[row]
        if is_head[k]:
            hb = lambda b: min(b * BLOCK, N) - tbl[b]
            b = last_block(r, hb)
            pos = b * BLOCK + (tbl[b + 1] - tbl[b]) + (r - hb(b))
        else:
            b = last_block(r, lambda b: tbl[b])
            pos = b * BLOCK + (r - tbl[b])
        assert 0 <= pos < N and perm[pos] == -1
        perm[pos] = row
    return perm


@pytest.mark.parametrize("seed", range(24))
def test_counting_sort_equals_the_token_order(seed):
    rng = np.random.default_rng(seed)
    N = int(rng.choice([1, 15, 16, 17, 127, 128, 129, 1000, 4096, 8191, 8192, 12345, 16384]))
    V = int(rng.choice([128, 1000, 20000, 128256, 256000, 262015]))
    kind = seed % 3
    if kind == 0:
        tt = rng.integers(0, V, N)
    elif kind == 1:  # Zipf: long head runs
        tt = np.minimum(rng.zipf(1.3, N) - 1, V - 1)
    else:  # few keys
        tt = rng.integers(0, min(V, 300), N)
    tt[rng.random(N) < 0.05] = -100
    d = rng.random(N).astype(np.float32)
    d[rng.random(N) < 0.03] = 0
    assert np.array_equal(csort_restated(tt, d, V), token_order(tt, d, V))


def test_counting_sort_mutant_is_caught():
    """A counting sort that forgets the earlier waves' rows of a key (no prefix over the
    waves) places two rows at one position or differs from the definition."""
    rng = np.random.default_rng(5)
    N, V = 4096, 20000
    tt = rng.integers(0, 300, N)
    d = np.ones(N, dtype=np.float32)
    assert np.array_equal(csort_restated(tt, d, V), token_order(tt, d, V))
    try:
        bad = csort_restated(tt, d, V, wave_prefix=False)
    except AssertionError:
        return
    assert not np.array_equal(bad, token_order(tt, d, V))


def block_tasks_restated(cnts, vt0, vt1, rb_of, slot_of, chunk=4):
    """bwd_compact_kernel's block tasks of one pass: the pass's tiles that keep one
    token block, counted per block (any order among a block's tiles: LDS atomics), then
    tasks of at most `chunk` of one block's tiles in token-block order.  Returns the
    tasks (rb, e0, e1) and the (owner, slot) pairs by entry."""
    order = [v for v in range(vt0, vt1) if cnts[v] == 1]
    rng = np.random.default_rng(vt0 + 7)
    rng.shuffle(order)
    nrb = max(rb_of.values()) + 1 if rb_of else 1
    cntb = [0] * nrb
    place = {}
    for v in order:
        place[v] = cntb[rb_of[v]]
        cntb[rb_of[v]] += 1
    tasks, first, ob = [], [0] * nrb, 0
    for r in range(nrb):
        c = cntb[r]
        for e in range(0, c, chunk):
            tasks.append((r, ob + e, ob + min(c, e + chunk)))
        first[r] = ob
        ob += c
    own = {}
    for v in order:
        e = first[rb_of[v]] + place[v]
        assert e not in own and 0 <= e < len(order)
        own[e] = (v, slot_of[(rb_of[v], v)])
    assert len(tasks) <= vt1 - vt0  # the tasks of a pass fit its tiles' entries
    return tasks, own


@pytest.mark.parametrize("seed", range(40))
def test_block_tasks_cover_every_one_tile_owner_once(seed):
    rng = np.random.default_rng(seed)
    nrb = int(rng.choice([1, 2, 7, 64, 300]))
    nvt = int(rng.integers(1, 3000))
    cnts = [int(min(nrb, rng.choice([0, 1, 1, 1, 2, 46, int(rng.integers(0, 60))]))) for _ in range(nvt)]
    slot, slot_of, rb_of = 0, {}, {}
    for v in range(nvt):
        for rb in sorted(rng.choice(nrb, cnts[v], replace=False).tolist()):
            slot_of[(rb, v)] = slot
            slot += 1
            if cnts[v] == 1:
                rb_of[v] = rb
    vt0 = int(rng.integers(0, nvt))
    vt1 = int(rng.integers(vt0 + 1, nvt + 1))
    tasks, own = block_tasks_restated(cnts, vt0, vt1, rb_of, slot_of)
    nds = int(rng.choice([1, 8, 16, 23]))
    seen = set()
    for t in range(len(tasks) * nds):  # the kernel's walk: task t = (tasks[t / nds], slice t % nds)
        (rb, e0, e1), ds = tasks[t // nds], t % nds
        assert e0 < e1 and e1 - e0 <= 4
        for e in range(e0, e1):
            v, s = own[e]
            assert rb_of[v] == rb and slot_of[(rb, v)] == s
            assert (v, ds) not in seen
            seen.add((v, ds))
    assert seen == {(v, ds) for v in range(vt0, vt1) if cnts[v] == 1 for ds in range(nds)}
    # the owners dealt to bins are exactly those before the one-tile ones in own_vt
    own_vt = sorted((v for v in range(vt0, vt1) if cnts[v] > 0), key=lambda v: -cnts[v])
    deal = len(own_vt) - len(own)
    assert all(cnts[v] >= 2 for v in own_vt[:deal]) and all(cnts[v] == 1 for v in own_vt[deal:])


def test_epilogue_transpose_is_a_conflict_free_bijection():
    """The 16-bit epilogue: lane (n, h) of a wave holds, per (il, pq), 8 consecutive
    columns 32 il + 16 pq + 8 h of row n of a 32-row x 64-column unit; it writes them to
    16-byte chunk c = 4 il + 2 pq + h of row n, at chunk c ^ ((n >> 1) & 7) of a
    128-byte LDS row; lane l then reads row 8 t + (l >> 3), chunk l & 7 (same swizzle)
    and stores it.  Every chunk is written once and read back by the lane that stores
    its row piece; each group of 8 lanes of a 16-byte access hits 8 distinct 4-bank
    groups of the 64 banks."""
    slot = {}
    for lane in range(64):
        n, h = lane & 31, lane >> 5
        for il in range(2):
            for pq in range(2):
                ck = 4 * il + 2 * pq + h
                addr = n * 128 + ((ck ^ ((n >> 1) & 7)) << 4)
                assert 0 <= addr and addr + 16 <= 4096 and addr not in slot
                slot[addr] = (n, 32 * il + 16 * pq + 8 * h)
    assert len(slot) == 256
    for t in range(4):
        for lane in range(64):
            r, cl = 8 * t + (lane >> 3), lane & 7
            assert slot[r * 128 + ((cl ^ ((r >> 1) & 7)) << 4)] == (r, 8 * cl)
    groups = lambda addrs: {((a // 4) % 64) // 4 for a in addrs}
    for il in range(2):
        for pq in range(2):
            for g in range(8):
                lanes = range(8 * g, 8 * g + 8)
                addrs = [(l & 31) * 128 + (((4 * il + 2 * pq + (l >> 5)) ^ (((l & 31) >> 1) & 7)) << 4) for l in lanes]
                assert len(groups(addrs)) == 8
    for t in range(4):
        for g in range(8):
            addrs = [(8 * t + (l >> 3)) * 128 + (((l & 7) ^ (((8 * t + (l >> 3)) >> 1) & 7)) << 4)
                     for l in range(8 * g, 8 * g + 8)]
            assert len(groups(addrs)) == 8


def g_tasks_restated(bits, cap, maxp, gwg, order=None):
    """bwd_compact_kernel's slots and G tasks for one chunk: bits[rb, v] the kept pairs;
    passes cut by the prefix P[v] of kept pairs per tile (tile v in pass P[v] // (cap -
    nrb) when maxp > 1); slots by pass, block, tile; runs of R slots of one (pass, block),
    R the shortest run whose tasks fit gwg, else 4; listed by (pass, run index, block)
    when kept > 2 * (tiles keeping a pair), else by (pass, block, run index).  Returns
    (rb_start, tasks as (first slot, block), per-pass [task0, task1), R, order)."""
    nrb, nv = bits.shape
    kept_v = bits.sum(0)
    vpre = np.concatenate([[0], np.cumsum(kept_v)])
    kept = int(vpre[nv])
    cp = cap - nrb if maxp > 1 else 1 << 62
    pass_of = vpre[:nv] // cp
    npass = int(pass_of[nv - 1]) + 1
    assert npass <= maxp
    pcnt = np.zeros((npass, nrb), dtype=np.int64)
    for p in range(npass):
        pcnt[p] = bits[:, pass_of == p].sum(1)
    rb_start = np.concatenate([[0], np.cumsum(pcnt.reshape(-1))])
    ntr = [int(((pcnt + r) // (r + 1)).sum()) for r in range(4)]
    R = 1 if ntr[0] <= gwg else 2 if ntr[1] <= gwg else 3 if ntr[2] <= gwg else 4
    ntiles = int((kept_v > 0).sum())
    if order is None:
        order = "block" if kept <= 2 * ntiles else "run"
    tasks, t0 = [], []
    if order == "block":
        for p in range(npass):
            t0.append(len(tasks))
            for rb in range(nrb):
                i = p * nrb + rb
                b0, c = int(rb_start[i]), int(rb_start[i + 1] - rb_start[i])
                for k4 in range(0, c, R):
                    tasks.append((b0 + k4, rb))
    else:
        for p in range(npass):
            t0.append(len(tasks))
            kmax = max(1, -(-int(pcnt[p].max()) // R))
            for k in range(kmax):
                for rb in range(nrb):
                    i = p * nrb + rb
                    b0, c = int(rb_start[i]), int(rb_start[i + 1] - rb_start[i])
                    if c > R * k:
                        tasks.append((b0 + R * k, rb))
    ranges = [(t0[p], t0[p + 1] if p + 1 < npass else len(tasks)) for p in range(npass)]
    return rb_start, tasks, ranges, R, order, npass


@pytest.mark.parametrize("seed", range(30))
def test_g_tasks_cover_every_kept_pair_once(seed):
    """Both task orders: each task is a run of min(R, the rest of its block's slots in
    the pass) slots inside one (pass, block); the runs of a pass's tasks cover exactly
    the pass's slots; the orders list the same runs."""
    rng = np.random.default_rng(seed)
    nrb = int(rng.choice([1, 3, 32, 64]))
    nv = int(rng.choice([1, 5, 33, 200, 1002]))
    dens = float(rng.choice([0.01, 0.05, 0.2, 1.0]))
    bits = rng.random((nrb, nv)) < dens
    if seed % 5 == 0:  # one popular tile
        bits[:, nv // 2] = True
    if not bits.any():
        bits[0, 0] = True
    kept = int(bits.sum())
    maxp = int(rng.choice([1, 2, 8]))
    cap = max(2 * nrb, -(-kept // maxp) + nrb + 1) if maxp > 1 else kept
    gwg = 256
    runs = {}
    for order in ("block", "run", None):
        rb_start, tasks, ranges, R, got, npass = g_tasks_restated(bits, cap, maxp, gwg, order)
        cover = np.zeros(kept, dtype=np.int64)
        for p, (a0, a1) in enumerate(ranges):
            for s0, rb in tasks[a0:a1]:
                i = p * nrb + rb
                lo, hi = int(rb_start[i]), int(rb_start[i + 1])
                assert lo <= s0 < hi  # inside its own (pass, block)
                cnt = min(R, hi - s0)  # the G kernel's count
                cover[s0:s0 + cnt] += 1
        assert (cover == 1).all()
        runs[order] = sorted(tasks)
    assert runs["block"] == runs["run"]


def g_tile_tasks_restated(bits, cap, maxp):
    """bwd_compact_kernel's vocabulary-tile G tasks: per tile (in order), runs of up to 4
    of its vt_slot entries (its kept blocks ascending, as slots); the pass's tasks start
    at its first tile.  Returns (vt_slot, vt_start, slot_rb, tasks (q, tile),
    per-pass [task0, task1), rb_start)."""
    nrb, nv = bits.shape
    kept_v = bits.sum(0)
    vpre = np.concatenate([[0], np.cumsum(kept_v)])
    cp = cap - nrb if maxp > 1 else 1 << 62
    pass_of = vpre[:nv] // cp
    npass = int(pass_of[nv - 1]) + 1
    # slots by (pass, block, tile)
    slot_of, slot_rb, s = {}, [], 0
    rb_start = []
    for p in range(npass):
        for rb in range(nrb):
            rb_start.append(s)
            for v in range(nv):
                if pass_of[v] == p and bits[rb, v]:
                    slot_of[(rb, v)] = s
                    slot_rb.append(rb)
                    s += 1
    rb_start.append(s)
    vt_slot = [slot_of[(rb, v)] for v in range(nv) for rb in range(nrb) if bits[rb, v]]
    tasks, t0 = [], {}
    for v in range(nv):
        p = int(pass_of[v])
        if p not in t0:
            t0[p] = len(tasks)
        for q in range(int(vpre[v]), int(vpre[v + 1]), 4):
            tasks.append((q, v))
    ranges = [(t0[p], t0[p + 1] if p + 1 < npass else len(tasks)) for p in range(npass)]
    return vt_slot, vpre, slot_rb, tasks, ranges, rb_start, npass


@pytest.mark.parametrize("seed", range(30))
def test_g_tile_tasks_cover_every_kept_pair_once(seed):
    """The G kernel's tile tasks: task (q, v) takes cnt = min(4, vt_start[v + 1] - q)
    entries, all of tile v, each a slot of the task's pass whose block is slot_rb of it;
    a pass's tasks cover exactly its slots (every kept pair's G tile is formed once)."""
    rng = np.random.default_rng(seed)
    nrb = int(rng.choice([1, 3, 32, 64]))
    nv = int(rng.choice([1, 5, 33, 200]))
    bits = rng.random((nrb, nv)) < float(rng.choice([0.05, 0.2, 0.6, 1.0]))
    if not bits.any():
        bits[0, 0] = True
    kept = int(bits.sum())
    maxp = int(rng.choice([1, 2, 8]))
    cap = max(2 * nrb, -(-kept // maxp) + nrb + 1) if maxp > 1 else kept
    vt_slot, vt_start, slot_rb, tasks, ranges, rb_start, npass = g_tile_tasks_restated(bits, cap, maxp)
    cover = np.zeros(kept, dtype=np.int64)
    for p, (a0, a1) in enumerate(ranges):
        s_lo, s_hi = rb_start[p * nrb], rb_start[(p + 1) * nrb]
        for q, v in tasks[a0:a1]:
            cnt = min(4, int(vt_start[v + 1]) - q)
            assert cnt >= 1
            for i in range(cnt):
                sl = vt_slot[q + i]
                assert s_lo <= sl < s_hi  # the pass's G scratch
                assert bits[slot_rb[sl], v]  # a kept pair of this tile
                cover[sl] += 1
            # the segments of the task's loads: the blocks of its first cnt entries
            blocks = [slot_rb[vt_slot[q + min(i, cnt - 1)]] for i in range(4)]
            assert blocks[:cnt] == sorted(blocks[:cnt])
    assert (cover == 1).all()


DE_PART_SLOTS = 256  # kDePartSlots: fp32 partial sums of 128 x 256 outputs each
DE_PIECES_PER_TASK = 128 // 4  # kDePiecesPerTask: 4 of a task's 128 rows per workgroup
DE_PIECES_GRID = DE_PIECES_PER_TASK * (DE_PART_SLOTS // 2)  # kDePiecesGrid: bwd_de_pieces_kernel


def de_pieces_of(ntasks, nwg):
    """de_pieces_of (cce_bwd.hip): (tbase, ncut, npc) -- npc pieces each of the cut tasks
    [tbase, tbase + ncut); all of few tasks (2 ntasks <= cap), or the ones past the grid
    when they overflow it by at most half (2 (ntasks - nwg) <= cap); cap = min(nwg, 256)."""
    cap = min(nwg, DE_PART_SLOTS)
    if ntasks <= 0:
        return 0, 0, 1
    if 2 * ntasks <= cap:
        return 0, ntasks, cap // ntasks
    if ntasks > nwg and 2 * (ntasks - nwg) <= cap:
        return nwg, ntasks - nwg, cap // (ntasks - nwg)
    return 0, 0, 1


def de_pieces_restated(own_cnt, nds, nwg):
    """The narrow dE sums' work items (bwd_sum_narrow_kernel, PHASE 0), over its one or
    two launches (de_stage 0, and 1 when tasks overflow the grid).  Stage 0 runs the
    whole tasks (all of them; with an overflow the first nwg) or, when all are cut,
    their pieces; stage 1 the overflow's pieces.  A launch's items: workgroup v walks
    q = 0, 1, ... over p = q nwg + v (q even) or q nwg + nwg - 1 - v (q odd) while
    p < nitems; a cut item p is piece p % npc, tiles [k cnt // npc, (k + 1) cnt // npc),
    of task tbase + p // npc (skipped when empty), with slot p.  Returns (npc, pieces
    {slot: (v, task, j0, j1)}, whole [(v, task)], and per cut task the slots
    bwd_de_pieces_kernel adds)."""
    ntasks = len(own_cnt) * nds
    tbase, ncut, npc = de_pieces_of(ntasks, nwg)
    pieces, whole = {}, []
    stages = [0, 1] if (npc > 1 and tbase > 0) else [0]
    for stage in stages:
        cut = npc > 1 and (stage == 1 or tbase == 0)
        nitems = ncut * npc if stage == 1 else (ntasks * npc if cut else (tbase if npc > 1 else ntasks))
        for v in range(nwg):
            q = 0
            while True:
                p = q * nwg + (nwg - 1 - v if q & 1 else v)
                if p >= nitems:
                    break
                q += 1
                if not cut:
                    whole.append((v, p))
                    continue
                task = tbase + p // npc
                cnt = own_cnt[task // nds]
                k = p - (p // npc) * npc
                j0, j1 = k * cnt // npc, (k + 1) * cnt // npc
                if j0 == j1:
                    continue
                assert p not in pieces
                pieces[p] = (v, task, j0, j1)
    fin = {}
    if npc > 1:
        for ti in range(ncut):
            cnt = own_cnt[(tbase + ti) // nds]
            fin[tbase + ti] = [ti * npc + k for k in range(npc) if k * cnt // npc < (k + 1) * cnt // npc]
    return npc, pieces, whole, fin


@pytest.mark.parametrize("seed", range(60))
def test_de_pieces_cover_every_task_tile_once(seed):
    rng = np.random.default_rng(seed)
    nown = int(rng.choice([1, 2, 3, 4, 8, 16, 32, 64, 65, 128, 288, 300, 384, 400]))
    nds = int(rng.choice([1, 1, 2, 9, 16]))
    nwg = int(rng.choice([8, 200, 256, 304]))
    own_cnt = [int(x) for x in rng.integers(1, 400, nown)]
    own_cnt[-1] = int(rng.choice([1, 2, own_cnt[-1]]))  # owners with fewer tiles than pieces
    npc, pieces, whole, fin = de_pieces_restated(own_cnt, nds, nwg)
    ntasks = nown * nds
    tbase, ncut, _ = de_pieces_of(ntasks, nwg)
    cap = min(nwg, DE_PART_SLOTS)
    if 2 * ntasks <= cap or (ntasks > nwg and 2 * (ntasks - nwg) <= cap):
        assert npc >= 2 and ncut * npc <= cap
    else:
        assert npc == 1
    cover = {t: np.zeros(own_cnt[t // nds], dtype=np.int64) for t in range(ntasks)}
    for v, task in whole:
        assert 0 <= v < nwg and not (tbase <= task < tbase + ncut and npc > 1)
        cover[task][:] += 1
    for p, (v, task, j0, j1) in pieces.items():
        assert 0 <= v < nwg and 0 <= j0 < j1 <= own_cnt[task // nds]
        assert p < DE_PART_SLOTS and tbase + p // npc == task  # the piece's own slot
        cover[task][j0:j1] += 1
    for t in range(ntasks):
        assert (cover[t] == 1).all()
    if npc > 1:  # the finisher adds exactly the slots written, once each
        assert sorted(sum(fin.values(), [])) == sorted(pieces)
        # its workgroups (cut task index = block // 32, rows 4 (block % 32) + wave) reach
        # every row of every cut task
        rows = {(b // DE_PIECES_PER_TASK, 4 * (b % DE_PIECES_PER_TASK) + w) for b in range(DE_PIECES_GRID) for w in range(4)}
        assert rows >= {(ti, m) for ti in range(ncut) for m in range(128)}
    # each workgroup runs at most one item per launch when anything is cut
    if npc > 1:
        assert len({v for v, _ in whole}) == len(whole)


def test_de_pieces_mutant_is_caught():
    """A piece bound off by one (j1 = (k + 1) cnt // P + 1) sums a tile twice."""
    own_cnt, nds, P = [10], 1, 4
    cover = np.zeros(10, dtype=np.int64)
    for k in range(P):
        j0, j1 = k * 10 // P, min((k + 1) * 10 // P + 1, 10)
        cover[j0:j1] += 1
    assert not (cover == 1).all()
