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
