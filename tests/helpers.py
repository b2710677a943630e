"""Shared test helpers: scenes as device tensors, oracle calls on the same inputs."""
from __future__ import annotations

import functools

import numpy as np
import torch

from oracle import core, host_ops
from vorotracing_amd import camera, native, scene


@functools.lru_cache(maxsize=None)
def c1_scene():
    return scene.config1()


@functools.lru_cache(maxsize=None)
def mini_heightfield(n=40000, seed=3):
    """Config-3 distribution at test size (same generator, 3% of the sites)."""
    return scene.heightfield(seed=seed, n=n, name="mini_c3")


@functools.lru_cache(maxsize=None)
def mini_heightfield_r8(n=40000, seed=3):
    """The mini height field with the reference's only compiled map
    resolution, 8x8 diffuse and 8x8 specular (tracing_octmap.cu:27-28)."""
    return scene.heightfield(seed=seed, n=n, R=8, name="mini_c3_r8")


@functools.lru_cache(maxsize=None)
def small_random(n=600, seed=7, R=4, Rs=None, grid=None):
    return scene.random_scene(n, seed=seed, R=R, Rs=Rs, grid=grid)


def start_for(s, rays):
    """Nearest site of each ray origin (brute force), as uint32 [...]."""
    o = rays[..., :3].reshape(-1, 3)
    uo, inv = np.unique(o, axis=0, return_inverse=True)
    nn = host_ops.nearest_site(s.points, uo)
    return nn[inv.reshape(-1)].astype(np.uint32).reshape(rays.shape[:-1])


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to(dev)


def f16_maps(s):
    return (host_ops.pad_3to4(s.diffuse.astype(np.float16), s.diff_res),
            host_ops.pad_3to4(s.specular.astype(np.float16), s.spec_res))


def stats_np(t: torch.Tensor):
    """(num_rays, native.STATS_WORDS) u32 device tensor -> numpy structured stats."""
    a = t.cpu().numpy().view(np.uint32).reshape(-1, native.STATS_WORDS)
    return np.ascontiguousarray(a).view(core.STATS_DTYPE).reshape(-1)


def tile_order_keys(cost):
    """Ascending sort key of the tile launch order: 8 buckets per octave of the
    tile cost over [16, 2^20) (below: the last bucket, above: the first),
    costliest bucket first."""
    c = np.maximum(np.asarray(cost, dtype=np.int64), 1)
    lb = np.frexp(c.astype(np.float64))[1].astype(np.int64) - 1  # floor(log2 c), exact below 2**53
    frac = (c >> np.maximum(lb - 3, 0)) & 7
    key = 127 - (((lb - 4) << 3) | frac)
    return np.where(lb < 4, 127, np.where(lb >= 20, 0, key))


def assert_stats_equal(got, want):
    for k in ("n", "visits", "faces", "exits", "integrated", "shaded", "visit_hash", "first_cells"):
        diff = got[k] != want[k]
        bad = np.nonzero(diff.reshape(diff.shape[0], -1).any(axis=1))[0]
        assert bad.size == 0, f"stats field {k} differs on {bad.size} rays, first {bad[:5]}: " \
                              f"{got[k][bad[:5]]} vs {want[k][bad[:5]]}"


def assert_infer_rgba(got, want):
    """fp16 RGBA of an inference kernel against the oracle.

    Alpha is 1 - T, which the kernels compute exactly: bit-identical.  RGB is
    shaded with hardware approximations (rsq, rcp, exp2), so each channel may
    sit one fp16 ulp of the oracle's value away (the north star's bound is
    2e-3); almost all values are identical, so the mean difference stays tiny.
    """
    g = np.asarray(got.cpu().numpy() if hasattr(got, "cpu") else got)
    w = np.asarray(want)
    assert g.shape == w.shape and g.dtype == np.float16 and w.dtype == np.float16
    assert np.array_equal(g[..., 3].view(np.uint16), w[..., 3].view(np.uint16)), "alpha differs from the oracle"
    gr, wr = g[..., :3].astype(np.float32), w[..., :3].astype(np.float32)
    assert np.isnan(gr).sum() == 0 and np.isnan(wr).sum() == 0
    d = np.abs(gr - wr)
    ulp = np.spacing(np.abs(w[..., :3])).astype(np.float32)
    bad = np.nonzero(d > ulp)
    assert bad[0].size == 0, f"{bad[0].size} RGB values more than one fp16 ulp from the oracle, " \
                             f"first {gr[bad][:5]} vs {wr[bad][:5]}"
    assert d.max(initial=0.0) <= 2e-3
    assert d.mean() <= 1e-4 if d.size else True, f"mean |rgb - oracle| = {d.mean()}"


def nn_tie_set(n=300000, seed=11):
    """Sites and queries whose nearest sites tie, for the all-sites scan of the
    start-cell lookup (1024 blocks x 256 lanes stride over the sites, so site i
    and i + 262144 fall on one lane, i and i + 256 on two blocks, i and i + 64
    on two waves of a block, i and i + 1 on two lanes of a wave).

    Background sites lie in [5, 9]^3; tie groups sit near x in [-3, 3]:
    exact duplicates at index pairs and triples of each spacing above, and
    pairs exactly equidistant (offsets of +-0.25 along one axis, exact in
    fp32) from their query.  Returns (points (n,3) f32, queries (q,3) f32)."""
    rng = np.random.default_rng(seed)
    pts = rng.uniform(5.0, 9.0, size=(n, 3)).astype(np.float32)
    queries = []
    spacings = [1, 64, 256, 256 * 1023, 262144, 7, 300]
    base = 1000
    g = 0
    for sp in spacings:
        for reps in (2, 3):
            idx = [base + k * sp for k in range(reps)]
            if idx[-1] >= n:
                continue
            c = np.array([-3.0 + 0.25 * g, 0.5, -0.5], np.float32)
            for i in idx:
                pts[i] = c
            queries.append(c)                                   # distance 0 to every copy
            queries.append(c + np.float32([0.0, 0.03125, 0.0]))  # equal distance to every copy
            base += 17
            g += 1
    for e, sp in enumerate((1, 64, 256, 262144)):
        lo, hi = base, base + sp
        if hi >= n:
            continue
        c = np.array([-3.0 + 1.0 * e, -1.5, 1.0], np.float32)  # groups 1.0 apart: no site of one near another
        off = np.float32([0.25, 0.0, 0.0])
        # the higher index on the - side in every other group: the rule must not depend on the side
        pts[lo], pts[hi] = (c + off, c - off) if g % 2 else (c - off, c + off)
        queries.append(c)
        base += 17
        g += 1
    return pts, np.stack(queries).astype(np.float32)


# Per-element allowance in units of the element's absolute sum (the sum of
# |v| over the values scattered into it, oracle absolute-sum mode): about 300
# f32 ulps of that sum, far above what reordering an f32 sum of a few
# thousand terms moves it, and below any single term of an element with fewer
# than 1/COND_RTOL = 50,000 terms, so one wrong or missing term still fails.
COND_RTOL = 2e-5


def assert_grad_close(got, want, name="", rtol=1e-3, atol_frac=1e-6, abs_sum=None):
    """Gradient parity: the largest difference within rtol of the tensor's
    largest magnitude (atomics add in another order than the serial CPU
    loop), and every element within rtol of its own value plus atol_frac of
    that scale, so that a small element cannot be wrong by 100 % unnoticed.
    With ``abs_sum`` (the oracle's absolute sums of the same call), an
    element whose terms cancel is also allowed COND_RTOL of its absolute
    sum: two summation orders differ in proportion to that, not to the
    result."""
    g = np.asarray(got, np.float64)
    w = np.asarray(want, np.float64)
    assert g.shape == w.shape, (name, g.shape, w.shape)
    assert np.isfinite(g).all(), f"{name}: non-finite gradient"
    scale = max(float(np.abs(w).max(initial=0.0)), 1e-30)
    d = np.abs(g - w)
    assert d.max(initial=0.0) <= rtol * scale, f"{name}: max |diff| {d.max():.3g} > {rtol} x scale {scale:.3g}"
    allow = rtol * np.abs(w) + atol_frac * scale
    if abs_sum is not None:
        a = np.asarray(abs_sum, np.float64)
        assert a.shape == w.shape, (name, a.shape, w.shape)
        allow = allow + COND_RTOL * a
    bad = np.nonzero(d > allow)
    assert bad[0].size == 0, (f"{name}: {bad[0].size} elements outside {rtol} x |want| + {atol_frac} x scale"
                              f"{'' if abs_sum is None else f' + {COND_RTOL} x abs sum'}, first "
                              f"{list(zip(g[bad][:4], w[bad][:4]))}")


def quant_ties(per_channel):
    """q8 inputs whose quantised values land exactly on k + 0.5 steps, and the
    codes torch.round (half to even) gives them (vorotracing.py:495-503).
    Each channel spans exactly 255 (scale 1, reciprocal 1), shifted by an
    exact offset, so (x - vmin) * (1 / scale) is the listed value exactly; a
    half-away-from-zero rounding gives 1, 3, 5, ... where these give 0, 2, 4."""
    vals = np.array([0.0, 255.0, 0.5, 1.5, 2.5, 3.5, 4.5, 126.5, 127.5, 128.5, 253.5, 254.5, 100.0, 7.25, 7.75,
                     99.5], np.float32)
    want = np.rint(vals).astype(np.uint8)  # numpy rounds half to even, like torch.round
    assert list(want[2:7]) == [0, 2, 2, 4, 4]
    shift = (-1.0, 0.0, 3.0) if per_channel else (0.0, 0.0, 0.0)
    x = np.stack([vals + np.float32(shift[c]) for c in range(3)], axis=1).reshape(1, -1)  # texel-major
    x = np.repeat(x, 4, axis=0)
    q = np.repeat(np.stack([want] * 3, axis=1).reshape(1, -1), 4, axis=0)
    return x.astype(np.float32), q


# Half-precision accumulation (f16 attribute storage; the reference's
# atomicAdd on __half, ray_integrator_octmap.cuh:1004-1007,1021-1024): each
# term is rounded to half once and each add rounds the sum once, to nearest.
F16_U = 2.0 ** -11      # unit roundoff of binary16
F16_SUB = 2.0 ** -25    # largest rounding error in the subnormal range (half its spacing 2^-24)


def f16_sum_bound(abs_sum, count):
    """Per-element bound on |a - b| for two half-precision accumulations a, b
    of the same ``count`` terms (absolute sum ``abs_sum``, both from the
    oracle's sum modes) in any two orders and groupings.  Against the exact
    sum each side is off by at most sum_i (u|v_i| + s) for the terms' rounding
    plus sum_j (u|P_j| + s) for the adds, with |P_j| <= (1 + u) abs_sum (plus
    the terms' own rounding): (k + 1) u (1 + 2u) A + 2 k s.  A side that
    first sums some terms in f32 (the GPU's same-cell combining) adds at most
    k 2^-23 A.  The bound is that of both sides added."""
    A = np.asarray(abs_sum, np.float64)
    k = np.asarray(count, np.float64)
    one = (k + 1.0) * F16_U * (1.0 + 2.0 * F16_U) * A + 2.0 * k * F16_SUB
    return 2.0 * one + k * 2.0 ** -23 * A


def assert_f16_sum_close(got, want, abs_sum, count, name=""):
    """Every element of a half-precision accumulation within f16_sum_bound of
    the oracle's (same terms: the walks are bit-exact), elements nothing was
    added to exactly zero on both sides."""
    g = np.asarray(got, np.float32).astype(np.float64)
    w = np.asarray(want, np.float32).astype(np.float64)
    assert g.shape == w.shape, (name, g.shape, w.shape)
    assert np.isfinite(g).all(), f"{name}: non-finite value"
    k = np.asarray(count, np.float64)
    assert k.shape == w.shape and (k >= 0).all() and (k == np.round(k)).all(), f"{name}: bad counts"
    allow = f16_sum_bound(abs_sum, k)
    d = np.abs(g - w)
    bad = np.nonzero(d > allow)
    assert bad[0].size == 0, (f"{name}: {bad[0].size} elements outside the half-precision accumulation bound, "
                              f"first (got, want, allowed, adds) {list(zip(g[bad][:4], w[bad][:4], allow[bad][:4], k[bad][:4]))}")
    none = k == 0
    assert not g[none].any() and not w[none].any(), f"{name}: a value where nothing was added"


def f16_train_sums(s, rays, start, thr, fw16, g16, contribution=False, **bwd_kw):
    """Absolute sums and add counts (oracle sum modes) of the f16-storage
    training call whose forward outputs are ``fw16`` and upstream gradient
    ``g16``: the same terms, run with f32 copies of the f16 values (so no sum
    is itself rounded to half).  Returns (abs_sums, counts), dicts of the
    backward's outputs, plus "contribution" when asked for."""
    f32 = lambda a: None if a is None else np.asarray(a).astype(np.float32)  # noqa: E731
    d, sp = f32(s.diffuse.astype(np.float16)), f32(s.specular.astype(np.float16))
    kw = {k: (f32(v) if isinstance(v, np.ndarray) and v.dtype == np.float16 else v) for k, v in bwd_kw.items()}
    out = []
    for count in (False, True):
        with core.abs_sums(count=count):
            r = core.trace_bwd(s.points, d, sp, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets, rays,
                               start, f32(fw16["rgba"]), f32(g16), distortion=fw16["distortion"],
                               W_total=fw16["W_total"], S_total=fw16["S_total"], t_far=fw16["t_far"],
                               weight_threshold=thr, **kw)
            if contribution:
                r["contribution"] = core.trace_fwd(s.points, d, sp, s.diff_res, s.spec_res, s.density, s.adjacency,
                                                   s.offsets, rays, start, weight_threshold=thr,
                                                   return_contribution=True)["contribution"]
        out.append(r)
    return out[0], out[1]


def face_order_key(h):
    """The walk layout's sort key of f16 bits h: a total order that is the
    numeric one on non-NaN values, -0 taken as +0, NaNs past the infinities
    of their sign."""
    h = np.asarray(h, np.uint32)
    h = np.where(h == 0x8000, 0, h)
    return np.where(h & 0x8000, 0x7FFF - (h & 0x7FFF), h | 0x8000)


def walk_layout_np(points, density, adjacency, offsets, adj_diff, face_order=0):
    """The packed walk layout (vt_walk_layout) built on the host with numpy:
    (first_chunk (n + 2), chunks (C, 12) u32, links (8C, 2) u32, heads (n, 2)
    u32, cells (n, 4) f32, orig (8C,) u16).  adj_diff: the f16 records (rows
    of 4 halves).  face_order 1..3 lays out lists of at most 64 faces in the
    order of the x, y or z half of their offsets (face_order_key, ties in list
    order)."""
    offsets = np.asarray(offsets, np.int64)
    n = offsets.size - 1
    nf = np.diff(offsets)
    nch = (nf + 7) // 8
    first = np.zeros(n + 2, np.int64)
    first[1:n + 1] = np.cumsum(nch)
    total = int(first[n])
    first[n + 1] = nch.max() if n else 0
    F = int(offsets[n])
    halves = np.ascontiguousarray(adj_diff).view(np.uint16).reshape(-1, 4)[:F]
    # the face of each slot of each cell (list position within the cell)
    src = np.arange(F) - np.repeat(offsets[:-1], nf)
    if face_order:
        key = face_order_key(halves[:, face_order - 1])
        for c in np.nonzero((nf > 1) & (nf <= 64))[0]:
            b, e = offsets[c], offsets[c + 1]
            src[b:e] = np.argsort(key[b:e], kind="stable")
    cell_of = np.repeat(np.arange(n), nf)
    slot = 8 * first[cell_of] + (np.arange(F) - offsets[cell_of])
    face = offsets[cell_of] + src  # the face record placed at each slot
    rows = np.zeros((max(total, 0), 8, 3), np.uint16)
    for axis in range(3):
        rows[slot // 8, slot % 8, axis] = halves[face, axis]
    nb = np.asarray(adjacency, np.int64)[face]
    links = np.zeros((8 * total, 2), np.uint32)
    links[slot, 0] = (nb | (nch[nb] << 24)).astype(np.uint32)
    links[slot, 1] = first[nb].astype(np.uint32)
    orig = np.full(8 * total, 0xFFFF, np.uint16)
    orig[slot] = src.astype(np.uint16)
    heads = np.stack([np.arange(n) | (nch << 24), first[:n]], 1).astype(np.uint32)
    cells = np.concatenate([np.asarray(points, np.float32).reshape(n, 3),
                            np.asarray(density, np.float32).reshape(n, 1)], 1)
    return first.astype(np.uint32), rows.reshape(total, 24).view(np.uint32), links, heads, cells, orig
