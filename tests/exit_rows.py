"""Synthetic inputs for the walk's exit-face order and search (shared by the
CPU pins and the GPU probes): random rows plus the hard cases, namely near-ties,
exact ties, subnormal and overflowing quotients, and NaN."""
import numpy as np

F = np.float32


def order_cases(rng, m=1 << 16):
    """(n, 4) float32 rows (num, dp, bnum, bdp), dp and bdp in (0, 2^17)."""
    out = []
    with np.errstate(all="ignore"):
        num = (rng.standard_normal(m) * 10.0 ** rng.uniform(-6, 6, m)).astype(F)
        dp = (10.0 ** rng.uniform(-8, 5, m)).astype(F)
        bnum = (rng.standard_normal(m) * 10.0 ** rng.uniform(-6, 6, m)).astype(F)
        bdp = (10.0 ** rng.uniform(-8, 5, m)).astype(F)
        out.append(np.stack([num, dp, bnum, bdp], 1))
        for lo, hi, dlo, dhi in ((-3, 3, -4, 4), (-45, -25, -38, 0), (-40, -30, -20, -5)):
            bnum = (rng.standard_normal(m) * 10.0 ** rng.uniform(lo, hi, m)).astype(F)
            bdp = (10.0 ** rng.uniform(dlo, dhi, m)).astype(F)
            dp = (10.0 ** rng.uniform(dlo, dhi, m)).astype(F)
            k = rng.integers(-24, 25, m)
            t = bnum.astype(np.float64) / bdp.astype(np.float64) * (1.0 + k * 2.0 ** -22)
            out.append(np.stack([(t * dp).astype(F), dp, bnum, bdp], 1))
            s = (2.0 ** rng.integers(-6, 7, m)).astype(F)  # exact ties
            out.append(np.stack([bnum * s, bdp * s, bnum, bdp], 1))
        dp = (10.0 ** rng.uniform(-12, 4, m)).astype(F)  # the first best (2^64, 2^-64), quotients near 2^128
        k = rng.integers(-64, 65, m)
        num = (dp.astype(np.float64) * 2.0 ** 128 * (1.0 + k * 2.0 ** -27)).astype(F)
        out.append(np.stack([num, dp, np.full(m, 2.0 ** 64, F), np.full(m, 2.0 ** -64, F)], 1))
        sp = F([np.nan, 0.0, -0.0, 1.0, -1.0, 1e-45, -1e-45, 3.4e38, -3.4e38])
        g = np.array(np.meshgrid(sp, F([1e-30, 1.0, 1e5]), sp, F([1e-30, 1.0, 1e5, 2.0 ** -64])))
        out.append(g.reshape(4, -1).T.astype(F))
    a = np.concatenate(out)
    return np.ascontiguousarray(a[np.isfinite(a[:, 1]) & np.isfinite(a[:, 3]) & (a[:, 1] > 0) & (a[:, 3] > 0)])


def order_want(a):
    """RN(num/dp) < RN(bnum/bdp) in IEEE float32 (numpy divides correctly rounded)."""
    with np.errstate(all="ignore"):
        return (a[:, 0] / a[:, 1]) < (a[:, 2] / a[:, 3])


def _row(p, o, d, recs):
    r = np.zeros(26, F)
    r[0:3], r[3:6], r[6:9] = p, o, d
    r[9:10] = np.array([len(recs)], np.uint32).view(F)
    h = np.zeros((8, 4), np.float16)
    h[:len(recs), :3] = np.asarray(recs, np.float32).astype(np.float16)
    r[10:26] = h.view(np.uint16).reshape(-1).view(F)
    return r


def face_rows(rng, m=1 << 14):
    """(n, 26) float32 rows for the exit-face search probe."""
    rows = []
    for _ in range(m):
        nf = int(rng.integers(0, 9))
        d = rng.standard_normal(3)
        d = (d / np.linalg.norm(d)).astype(F)
        recs = rng.standard_normal((nf, 3)) * 10.0 ** rng.uniform(-2, 1)
        if nf >= 2 and rng.random() < 0.25:
            recs[int(rng.integers(1, nf))] = recs[0]  # duplicate face: an exact tie
        rows.append(_row(rng.uniform(-3, 3, 3), rng.uniform(-3, 3, 3), d, recs))
    # quotients that round to -inf: origin far along +x, a direction almost
    # along +y, faces that the ray meets at a grazing angle
    d = np.array([1e-9, 1.0, 1e-9], np.float64)
    d = (d / np.linalg.norm(d)).astype(F)
    for ox in (1e30, 3e33, 1e36):
        o = (ox, 0.0, 0.0)
        rows.append(_row((0, 0, 0), o, d, [(1, 0, 1), (1, 0, 0)]))           # -5e38 then -1e39: keep face 0
        rows.append(_row((0, 0, 0), o, d, [(1, 0, 0), (1, 0, 1), (2, 0, 0)]))
        rows.append(_row((0, 0, 0), o, d, [(0, -1, 0), (1, 0, 1), (-1, 0, 0), (1, 0, 0)]))
        rows.append(_row((0, 0, 0), o, d, [(0, 1, 0), (1, 0, 1), (1, 0, 0)]))  # a finite face first
    # NaN site
    rows.append(_row((np.nan, 0, 0), (0, 0, 0), F([0, 0, 1]), [(0, 0, 1), (0, 0, 2)]))
    return np.ascontiguousarray(np.stack(rows))


def packed_rows(rows, rng):
    """Op 6 rows reordered into the packed walk's slots: (n, 30) float32, the
    records of each row put in a new slot order (by the z half, stably, as
    vt_walk_layout_fill's face order 3 lays a list out; reversed; or at
    random), zero records past the count, then the slots' original indices
    as 8 u16 (0xffff for empty slots)."""
    n = rows.shape[0]
    out = np.zeros((n, 30), F)
    out[:, :10] = rows[:, :10]
    recs = np.ascontiguousarray(rows[:, 10:26]).view(np.uint16).reshape(n, 8, 4)
    nf = np.minimum(rows[:, 9].view(np.uint32), 8)
    slots = np.zeros((n, 8, 4), np.uint16)
    orig = np.full((n, 8), 0xffff, np.uint16)
    kind = rng.integers(0, 3, n)
    for i in range(n):
        k = int(nf[i])
        if kind[i] == 0:
            perm = np.argsort(recs[i, :k, 2].view(np.float16).astype(np.float32), kind="stable")
        elif kind[i] == 1:
            perm = np.arange(k)[::-1]
        else:
            perm = rng.permutation(k)
        slots[i, :k] = recs[i, perm]
        orig[i, :k] = perm
    out[:, 10:26] = slots.reshape(n, 16 * 2).view(F)
    out[:, 26:30] = orig.view(F)
    return np.ascontiguousarray(out)
