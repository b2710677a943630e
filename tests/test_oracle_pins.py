"""Pins of the CPU oracle (no GPU): each check is chosen so that a plausible
mistake in the restatement (a dropped term, a wrong sign or index, a swapped
operand) fails it.  The reference ships no tests or golden vectors, so the
pins are numpy / float64 libm, closed forms on exact scenes, brute-force
geometry and finite differences."""
import math

import numpy as np
import pytest

from oracle import core, host_ops
from tests import helpers as H
from vorotracing_amd import camera, scene


# --------------------------------------------------------------------------- scalar math

def test_f16_decode_all_halves():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = np.array([core.lib().or_f16_to_f32(int(x)) for x in h[::7]], np.float32)
    w = want[::7]
    ok = (got.view(np.uint32) == w.view(np.uint32)) | (np.isnan(got) & np.isnan(w))
    assert ok.all()


def test_f16_encode_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([
        (rng.standard_normal(1 << 18) * np.exp2(rng.integers(-30, 17, 1 << 18))).astype(np.float32),
        np.float32([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25,
                    2.0 ** -25 * 1.0000001, 3 * 2.0 ** -26, 6.1e-5, 6.103515625e-05, np.inf, -np.inf]),
        # exact halfway cases between adjacent halves
        ((np.arange(1024, 2048, dtype=np.float64) + 0.5) * 2.0 ** -10).astype(np.float32),
    ])
    got = core.f32_to_f16_bits(x)
    want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def _ulps(a, b):
    """distance in float32 ulps of b (float64 reference)"""
    b32 = np.float32(b)
    ulp = np.spacing(np.abs(b32)).astype(np.float64)
    return np.abs(a.astype(np.float64) - b) / ulp


def test_expf_within_two_ulp():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.uniform(-87.0, 88.7, 1 << 20), rng.uniform(-1, 1, 1 << 16), [0.0, 1.0, -1.0, 1e-7]]
                       ).astype(np.float32)
    got = core.expf(x)
    want = np.exp(x.astype(np.float64))
    assert _ulps(got, want).max() <= 2.0
    assert core.expf(np.float32([0.0]))[0] == 1.0
    # subnormal range, overflow, NaN, -inf
    xs = np.float32([-100.0, -103.0, -104.0, 89.0, np.inf, -np.inf, np.nan])
    g = core.expf(xs)
    assert abs(g[0] - np.exp(-100.0)) <= 2 * 2.0 ** -149 + np.exp(-100.0) * 2 ** -22
    assert g[2] == 0.0 and g[3] == np.inf and g[4] == np.inf and g[5] == 0.0 and np.isnan(g[6])


def test_logf_within_two_ulp():
    rng = np.random.default_rng(2)
    x = np.concatenate([np.exp2(rng.uniform(-140, 127, 1 << 20)), rng.uniform(0.5, 2.0, 1 << 16), [1.0, 2.0]]
                       ).astype(np.float32)
    x = x[x > 0]
    got = core.logf(x)
    want = np.log(x.astype(np.float64))
    nz = np.abs(want) > 1e-3
    assert _ulps(got[nz], want[nz]).max() <= 2.0
    # near 1, the absolute error is within 2 ulp of the argument's spacing
    assert (np.abs(got[~nz] - want[~nz]) <= 2 * np.spacing(np.float32(1.0))).all()
    assert core.logf(np.float32([1.0]))[0] == 0.0
    g = core.logf(np.float32([0.0, -1.0, np.inf]))
    assert g[0] == -np.inf and np.isnan(g[1]) and g[2] == np.inf


# --------------------------------------------------------------------------- octahedral map

def _oct_decode(u, v):
    """Octahedral decode of plane coordinates in [-1,1]^2 (Cigolle et al. 2014)."""
    z = 1.0 - abs(u) - abs(v)
    x, y = u, v
    if z < 0:
        x, y = (1 - abs(v)) * math.copysign(1, u), (1 - abs(u)) * math.copysign(1, v)
    n = math.sqrt(x * x + y * y + z * z)
    return np.array([x / n, y / n, z / n])


def _smooth(d):
    a = np.array([0.3, -0.7, 0.5])
    b = np.array([0.6, 0.2, -0.4])
    return float(d @ a + 0.8 * (d @ b) ** 2)


def _interp_error(R, wrap, n=3000, seed=0):
    """Max error of bilinear lookup (oracle encode + `wrap`) of a smooth
    function sampled at texel centres; a wrong fold or index is O(1)."""
    tex = np.empty(R * R)
    for j in range(R):
        for i in range(R):
            tex[j * R + i] = _smooth(_oct_decode((i + 0.5) / R * 2 - 1, (j + 0.5) / R * 2 - 1))
    rng = np.random.default_rng(seed)
    err = 0.0
    for _ in range(n):
        d = rng.normal(size=3)
        d /= np.linalg.norm(d)
        tu, tv = core.oct_encode(d.astype(np.float32), R)
        u0, v0 = math.floor(tu), math.floor(tv)
        fu, fv = tu - u0, tv - v0
        val = ((1 - fu) * (1 - fv) * tex[wrap(u0, v0, R)] + fu * (1 - fv) * tex[wrap(u0 + 1, v0, R)]
               + (1 - fu) * fv * tex[wrap(u0, v0 + 1, R)] + fu * fv * tex[wrap(u0 + 1, v0 + 1, R)])
        err = max(err, abs(val - _smooth(d)))
    return err


@pytest.mark.parametrize("R", [4, 8])
def test_oct_wrap_bilinear_is_continuous(R):
    err = _interp_error(R, core.oct_wrap_index)
    # interpolation error of a smooth function shrinks with R; broken wraps do not
    assert err < (0.45 if R == 4 else 0.16)

    def no_flip(u, v, R):  # plausible mistake: wrap without the mirror fold
        return (v % R) * R + (u % R)

    assert _interp_error(R, no_flip) > 2 * err


@pytest.mark.parametrize("R", [4, 8])
def test_oct_wrap_range_and_identity(R):
    for u in range(-1, R + 1):
        for v in range(-1, R + 1):
            k = core.oct_wrap_index(u, v, R)
            assert 0 <= k < R * R
            if 0 <= u < R and 0 <= v < R:
                assert k == v * R + u


def test_oct_encode_axes():
    # +z maps to the centre, -z to the corners, +x/-x to the edge midpoints
    for R in (4, 8):
        c = (R - 1) / 2.0
        assert np.allclose(core.oct_encode(np.float32([0, 0, 1]), R), [c, c])
        assert np.allclose(core.oct_encode(np.float32([1, 0, 0]), R), [R - 0.5, c])
        assert np.allclose(core.oct_encode(np.float32([-1, 0, 0]), R), [-0.5, c])
        assert np.allclose(core.oct_encode(np.float32([0, 1, 0]), R), [c, R - 0.5])
        uv = core.oct_encode(np.float32([0, 0, -1]), R)
        assert np.allclose(np.abs(uv - c), [R / 2.0, R / 2.0])


# --------------------------------------------------------------------------- walk + compositing on exact scenes

def _render_fwd(s, rays, start, **kw):
    return core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency,
                          s.offsets, rays, start, **kw)


def _const_texture_scene(s, logits):
    s.diffuse[:] = np.repeat(logits[:, None], s.diffuse.shape[1] // 3, 1).reshape(-1, 3).reshape(s.diffuse.shape) \
        if logits.ndim == 2 else logits[:, None]
    s.specular[:] = 0.0
    return s


def test_lattice_axis_ray_closed_form():
    """Sites on a 6x3x3 integer lattice, ray from site (0,1,1) along +x:
    exits at t = 0.5, 1.5, ..., 4.5; the last cell is unbounded in +x and is
    never integrated (tracing_octmap.cu:102-105); n counts the breaking step."""
    s = scene.cubic_lattice(6, 3, 3, raw_density=math.log(0.4))
    sig = np.float32(0.4)
    s.density_raw[:] = np.log(sig)
    dens = np.full((s.num_points, 1), sig, np.float32)
    lg = np.linspace(-1.0, 1.0, s.num_points).astype(np.float32)
    s.diffuse[:] = lg[:, None]
    s.specular[:] = 0.0
    start = int(np.argmin(np.linalg.norm(s.points - np.array([0, 1, 1]), axis=1)))
    rays = np.float32([[0, 1, 1, 1, 0, 0]])
    out = core.trace_fwd(s.points, s.diffuse, s.specular, 4, 4, dens, s.adjacency, s.offsets, rays,
                         np.uint32([start]), depth_quantiles=np.float32([[0.5]]), weight_threshold=1e-6)
    cells = [int(np.argmin(np.linalg.norm(s.points - np.array([x, 1, 1]), axis=1))) for x in range(6)]
    dts = [0.5, 1, 1, 1, 1]
    T, acc = 1.0, 0.0
    for c, dt in zip(cells, dts):
        a = 1 - math.exp(-0.4 * dt)
        acc += T * a / (1 + math.exp(-lg[c]))
        T *= 1 - a
    assert out["n"][0, 0] == 6
    assert abs(out["rgba"][0, 0] - acc) < 2e-6 and abs(out["rgba"][0, 3] - (1 - T)) < 2e-6
    # depth where T crosses 0.5: T(t) = exp(-0.4 t) on [0, 4.5]
    assert abs(out["depth"][0, 0] - math.log(2) / 0.4) < 2e-5
    # distortion (mip-NeRF 360 eq. 15) in s = 1 - 1/(1+t), brute force O(n^2)
    ts = [0.0, 0.5, 1.5, 2.5, 3.5, 4.5]
    w, m, dsv = [], [], []
    T = 1.0
    for i in range(5):
        a = 1 - math.exp(-0.4 * (ts[i + 1] - ts[i]))
        w.append(T * a)
        T *= 1 - a
        s0, s1 = 1 - 1 / (1 + ts[i]), 1 - 1 / (1 + ts[i + 1])
        m.append(0.5 * (s0 + s1))
        dsv.append(s1 - s0)
    L = sum(w[i] * w[j] * abs(m[i] - m[j]) for i in range(5) for j in range(5)) + sum(
        w[i] ** 2 * dsv[i] for i in range(5)) / 3
    assert abs(out["distortion"][0, 0] - L) < 1e-6
    assert abs(out["W_total"][0, 0] - sum(w)) < 1e-6 and out["t_far"][0, 0] == 4.5


def test_lattice_diagonal_tie_and_zero_length_steps():
    """Diagonal ray through lattice corners: at each corner the +x and +y
    planes tie and the lower face index (+x, listed before +y) wins; the
    following step has t1 == t0, is counted and advances without
    integration (tracing_octmap.cu:110-117)."""
    s = scene.cubic_lattice(4, 4, 1)
    s.diffuse[:] = 0.0
    s.specular[:] = 0.0
    dens = np.full((s.num_points, 1), 0.3, np.float32)
    d = np.float32([1, 1, 0]) / np.float32(math.sqrt(2))
    rays = np.float32([[0, 0, 0, d[0], d[1], 0]])
    start = np.uint32([0])
    adj = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    d4 = host_ops.pad_3to4(s.diffuse.astype(np.float16), 4)
    rgba, st, log = core.trace_infer_f16(s.points, d4, d4, 4, 4, dens, s.adjacency, s.offsets, adj, rays, start,
                                         weight_threshold=1e-6, want_stats=True, max_log=16)
    idx = lambda x, y: x * 4 + y  # noqa: E731 (lattice index (i*ny + j)*nz + k)
    want = [idx(0, 0), idx(1, 0), idx(1, 1), idx(2, 1), idx(2, 2), idx(3, 2), idx(3, 3)]
    assert log[0, :7].tolist() == want
    # integrated: (0,0), (1,1), (2,2); the t1 == t0 steps and the unbounded last cell are not
    assert st["visits"][0] == 7 and st["integrated"][0] == 3
    assert st["n"][0] == 7


def test_two_site_single_bisector():
    pts = np.float32([[0, 0, 0], [1, 0, 0]])
    adj = np.uint32([1, 0] + [0] * 32)
    off = np.uint32([0, 1, 2])
    dens = np.float32([[2.0], [5.0]])
    R = 4
    dif = np.zeros((2, 3 * R * R), np.float32)
    dif[0] = 0.7
    spe = np.zeros_like(dif)
    d = np.float64([1, 0.3, -0.2])
    d /= np.linalg.norm(d)
    rays = np.float32([[0, 0, 0, *d]])
    out = core.trace_fwd(pts, dif, spe, R, R, dens, adj, off, rays, np.uint32([0]), weight_threshold=1e-6)
    t = 0.5 / np.float32(d[0])
    a = 1 - math.exp(-2.0 * t)
    assert out["n"][0, 0] == 2
    assert abs(out["rgba"][0, 3] - a) < 2e-6
    assert abs(out["rgba"][0, 0] - a / (1 + math.exp(-0.7))) < 2e-6


def _seg_t(o, d, p, q):
    """float64 exit distance of the ray through the bisector of sites p, q"""
    n = q - p
    return float(((p + q) / 2 - o) @ n / (n @ d))


def test_walk_follows_voronoi_cells_bruteforce():
    """Sites on a 1/64 grid (every site offset exact in fp16): along every
    ray, the midpoint of each integrated segment is nearest to the cell the
    walk attributes it to, and the cell after each exit is nearest just past
    the exit."""
    s = scene.random_scene(500, seed=3, extent=2.0, grid=1 / 64)
    rng = np.random.default_rng(4)
    o = np.float32([0.1, -3.0, 0.2])
    dirs = rng.normal(size=(150, 3)) * [0.25, 0, 0.25] + [0, 1, 0]
    dirs = (dirs / np.linalg.norm(dirs, axis=1, keepdims=True)).astype(np.float32)
    rays = np.concatenate([np.broadcast_to(o, dirs.shape), dirs], 1).astype(np.float32)
    start = host_ops.nearest_site(s.points, o[None])
    adj = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    assert np.array_equal(adj[: s.num_faces, :3].astype(np.float64),
                          (s.points[s.adjacency[: s.num_faces]] - np.repeat(
                              s.points, np.diff(s.offsets.astype(np.int64)), 0)).astype(np.float64))
    d4 = host_ops.pad_3to4(s.diffuse.astype(np.float16), 4)
    _, st, log = core.trace_infer_f16(s.points, d4, d4, 4, 4, np.zeros((s.num_points, 1), np.float32),
                                      s.adjacency, s.offsets, adj, rays, np.repeat(start, len(rays)).astype(np.uint32),
                                      want_stats=True, max_log=256)
    P = s.points.astype(np.float64)
    checked = 0
    for r in range(len(rays)):
        oo = rays[r, :3].astype(np.float64)
        dd = rays[r, 3:].astype(np.float64)
        dd /= np.linalg.norm(dd)
        cells = [c for c in log[r] if c != 0xFFFFFFFF]
        t0 = 0.0
        for a, b in zip(cells[:-1], cells[1:]):
            t1 = _seg_t(oo, dd, P[a], P[b])
            if t1 > t0 + 1e-6:
                mid = oo + 0.5 * (t0 + t1) * dd
                dist = np.linalg.norm(P - mid, axis=1)
                assert dist[a] <= dist.min() + 1e-9
                checked += 1
            after = oo + (max(t0, t1) + 1e-5) * dd
            dist = np.linalg.norm(P - after, axis=1)
            assert dist[b] <= dist.min() + 1e-6
            t0 = max(t0, t1)
    assert checked > 500


def test_morton_and_perm_invariance_oracle():
    """Morton-reordered scene and any lane permutation give the bit-identical
    image with the visit sequence mapped through the permutation."""
    s = scene.random_scene(2000, seed=8, R=4)
    rays = camera.pinhole_rays(40, 30, eye=(0.0, -3.5, 0.2))
    start = host_ops.nearest_site(s.points, rays[0, 0, :3])
    sp = np.full(rays.shape[:-1], start[0], np.uint32)
    d4, s4 = host_ops.pad_3to4(s.diffuse.astype(np.float16), 4), host_ops.pad_3to4(s.specular.astype(np.float16), 4)
    adj = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    a, sta, _ = core.trace_infer_f16(s.points, d4, s4, 4, 4, s.density, s.adjacency, s.offsets, adj, rays, sp,
                                     weight_threshold=0.01, want_stats=True)
    perm, pts, adj2, off2, (d42, s42, den2) = host_ops.morton_reorder(s.points, s.adjacency, s.offsets,
                                                                     rows=[d4, s4, s.density])
    inv = np.empty_like(perm)
    inv[perm] = np.arange(len(perm))
    ad2 = core.prefetch_adj(pts, adj2, off2)
    b, stb, _ = core.trace_infer_f16(pts, d42, s42, 4, 4, den2, adj2, off2, ad2, rays,
                                     inv[sp].astype(np.uint32), weight_threshold=0.01, want_stats=True)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    assert np.array_equal(sta["n"], stb["n"]) and np.array_equal(sta["faces"], stb["faces"])
    tp = host_ops.tile_perm(30, 40, 8, 8)
    c, _, _ = core.trace_infer_f16(s.points, d4, s4, 4, 4, s.density, s.adjacency, s.offsets, adj, rays, sp,
                                   ray_perm=tp, weight_threshold=0.01)
    assert np.array_equal(a.view(np.uint16), c.view(np.uint16))


def test_morton_restatement_csr_invariants():
    s = scene.random_scene(3000, seed=12)
    perm, pts, adj, off, _ = host_ops.morton_reorder(s.points, s.adjacency, s.offsets)
    n = s.num_points
    assert np.array_equal(np.sort(perm), np.arange(n))
    keys = host_ops.morton_keys(s.points)[perm]
    assert (np.diff(keys) >= 0).all()
    inv = np.empty_like(perm)
    inv[perm] = np.arange(n)
    # neighbour sets map through the permutation, list order preserved
    for new in range(0, n, 97):
        old = perm[new]
        a = s.adjacency[s.offsets[old]:s.offsets[old + 1]]
        b = adj[off[new]:off[new + 1]]
        assert np.array_equal(inv[a], b)
    assert not adj[off[-1]:].any()


def test_tile_perm_restatement_shape():
    p = host_ops.tile_perm(822, 1237, 8, 8)
    assert np.array_equal(np.sort(p), np.arange(822 * 1237))
    # the first 64 lanes cover the 8x8 square at the origin
    ys, xs = np.divmod(p[:64], 1237)
    assert set(ys.tolist()) == set(range(8)) and set(xs.tolist()) == set(range(8))


@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_error_bound(per_channel):
    rng = np.random.default_rng(5)
    x = rng.normal(size=(500, 48)).astype(np.float32)
    x[:, 0::3] *= 3.0
    q, sc, of = host_ops.quantize_u8(x, per_channel)
    scv = np.broadcast_to(np.asarray(sc, np.float32), (3,))
    ofv = np.broadcast_to(np.asarray(of, np.float32), (3,))
    deq = scv[None, None, :] * q.reshape(500, 16, 3).astype(np.float32) + ofv[None, None, :]
    err = np.abs(deq - x.reshape(500, 16, 3))
    assert (err <= scv[None, None, :] * 0.5 + 1e-6).all()
    assert q.min() == 0 and q.max() == 255


@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_rounds_ties_to_even(per_channel):
    """torch.round is half to even (vorotracing.py:495-503): inputs landing
    exactly on k + 0.5 steps take the even code."""
    x, want = H.quant_ties(per_channel)
    q, sc, of = host_ops.quantize_u8(x, per_channel)
    assert np.all(np.asarray(sc) == np.float32(1.0))
    assert np.array_equal(q, want)


# --------------------------------------------------------------------------- backward vs finite differences

def _fd_case():
    s = scene.random_scene(300, seed=21, R=4, extent=1.5, density_mu=-0.5)
    rays = camera.pinhole_rays(12, 10, eye=(0.0, -2.8, 0.1), fov_y_deg=40)
    start = host_ops.nearest_site(s.points, rays[0, 0, :3])
    sp = np.full(rays.shape[:-1], start[0], np.uint32)
    g = np.random.default_rng(3).normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    return s, rays, sp, g


def _loss(s, rays, sp, g, dens, dif, spe, q=None, gd=None, gdist=None):
    out = core.trace_fwd(s.points, dif, spe, 4, 4, dens, s.adjacency, s.offsets, rays, sp, depth_quantiles=q,
                         weight_threshold=1e-4)
    L = float((out["rgba"].astype(np.float64) * g).sum())
    if gd is not None:
        L += float((out["depth"].astype(np.float64) * gd).sum())
    if gdist is not None:
        L += float((out["distortion"].astype(np.float64) * gdist).sum())
    return L, out


def test_backward_density_and_texture_vs_central_differences():
    s, rays, sp, g = _fd_case()
    dens = s.density.copy()
    q = np.tile(np.float32([0.6]), rays.shape[:-1] + (1,))
    gd = np.random.default_rng(6).normal(size=rays.shape[:-1] + (1,)).astype(np.float32) * 0.1
    gdist = np.random.default_rng(7).uniform(0, 1, size=rays.shape[:-1] + (1,)).astype(np.float32)
    L, out = _loss(s, rays, sp, g, dens, s.diffuse, s.specular, q, gd, gdist)
    bw = core.trace_bwd(s.points, s.diffuse, s.specular, 4, 4, dens, s.adjacency, s.offsets, rays, sp, out["rgba"],
                        g, depth_quantiles=q, depth_idx=out["depth_idx"], depth_grad=gd,
                        distortion=out["distortion"], distortion_grad=gdist, W_total=out["W_total"],
                        S_total=out["S_total"], t_far=out["t_far"], weight_threshold=1e-4)
    dg = bw["density_grad"][:, 0]
    cells = np.argsort(-np.abs(dg))[:12]
    for c in cells:
        h = np.float32(max(1e-3 * dens[c, 0], 1e-5))
        dp = dens.copy()
        dm = dens.copy()
        dp[c] += h
        dm[c] -= h
        fd = (_loss(s, rays, sp, g, dp, s.diffuse, s.specular, q, gd, gdist)[0]
              - _loss(s, rays, sp, g, dm, s.diffuse, s.specular, q, gd, gdist)[0]) / (float(dp[c, 0]) - float(dm[c, 0]))
        assert abs(fd - dg[c]) <= 2e-2 * abs(dg[c]) + 2e-3 * np.abs(dg).max(), (c, fd, dg[c])
    tg = bw["diffuse_grad"]
    for (c, k) in zip(*np.unravel_index(np.argsort(-np.abs(tg).ravel())[:10], tg.shape)):
        h = np.float32(1e-2)
        dp = s.diffuse.copy()
        dm = s.diffuse.copy()
        dp[c, k] += h
        dm[c, k] -= h
        fd = (_loss(s, rays, sp, g, dens, dp, s.specular)[0] - _loss(s, rays, sp, g, dens, dm, s.specular)[0]) / (
            2 * float(h))
        # texture logits do not touch depth or distortion
        assert abs(fd - tg[c, k]) <= 2e-2 * abs(tg[c, k]) + 1e-3 * np.abs(tg).max(), (c, k, fd, tg[c, k])


def test_cell_intersection_grad_vs_central_differences():
    rng = np.random.default_rng(11)
    for _ in range(50):
        prim = rng.normal(size=3)
        opp = prim + rng.normal(size=3) * 0.3
        o = rng.normal(size=3) * 2
        d = rng.normal(size=3)
        d /= np.linalg.norm(d)
        if abs((opp - prim) @ d) < 0.05:
            continue
        got = core.cell_intersection_grad(prim, opp, o, d).astype(np.float64)
        P, Q, O, D = [np.float32(v).astype(np.float64) for v in (prim, opp, o, d)]
        fd = np.zeros(3)
        for k in range(3):
            e = np.zeros(3)
            e[k] = 1e-6
            fd[k] = (_seg_t(O, D, P + e, Q) - _seg_t(O, D, P - e, Q)) / 2e-6
        assert np.allclose(got, fd, rtol=2e-3, atol=2e-3 * np.abs(fd).max())


@pytest.mark.parametrize("R", [4, 8])
def test_oct_wrap_edge_form_equals_general_on_tap_domain(R):
    """The kernels use a reduced wrap valid for texel coordinates in [-1, R]
    (every bilinear tap of an encoded direction): u mod R and one fold per
    coordinate outside [0, R).  It must equal the general wrap there."""
    for u in range(-1, R + 1):
        for v in range(-1, R + 1):
            wu, wv = u & (R - 1), v & (R - 1)
            if (not 0 <= u < R) != (not 0 <= v < R):
                wu, wv = R - 1 - wu, R - 1 - wv
            assert wv * R + wu == core.oct_wrap_index(u, v, R), (u, v)


def test_probe_length_test_on_squared_length():
    """The inference kernel replaces probe_dir's `sqrtf(x) > 1e-8f` by
    `x > 0x1.cd2b2ap-54f` (vt_infer.hip PROBE_LEN2_MIN); numpy's float32 sqrt
    is correctly rounded like the kernel's, so checking every float in a wide
    band around the boundary, and the special values, shows the two agree."""
    x0 = np.float32(float.fromhex("0x1.cd2b2ap-54"))
    lo, hi = np.float32(x0 / 64).view(np.int32), np.float32(x0 * 64).view(np.int32)
    x = np.arange(lo, hi, dtype=np.int32).view(np.float32)
    t = np.float32(1e-8)
    assert np.array_equal(np.sqrt(x) > t, x > x0)
    sp = np.array([0.0, -0.0, np.inf, np.nan, 1e-45, 1.0, 3e38], np.float32)
    with np.errstate(invalid="ignore"):
        assert np.array_equal(np.sqrt(sp) > t, sp > x0)


def test_exit_face_rows_closed_forms():
    """The oracle's exit-face search on hand-made cells: a unit cube seen from
    inside exits through the face the ray points at; a duplicated face ties
    to the lower index; faces behind the ray (dp <= 0) are skipped; quotients
    that round to -inf keep the first such face (strict t < t_1)."""
    from tests import exit_rows as X
    cube = [(2, 0, 0), (-2, 0, 0), (0, 2, 0), (0, -2, 0), (0, 0, 2), (0, 0, -2)]
    d = np.float32([0.0, 0.0, 1.0])
    rows = np.stack([X._row((0, 0, 0), (0, 0, 0), d, cube),
                     X._row((0, 0, 0), (0, 0, 0), np.float32([0.0, -1.0, 0.0]), cube),
                     X._row((0, 0, 0), (0, 0, 0), d, cube[:4] + [(0, 0, 2), (0, 0, 2)]),
                     X._row((0, 0, 0), (0, 0, 0), d, [(2, 0, 0), (0, 0, -2)])])
    dn = np.array([1e-9, 1.0, 1e-9])
    dn = (dn / np.linalg.norm(dn)).astype(np.float32)
    rows = np.concatenate([rows, np.stack([X._row((0, 0, 0), (1e30, 0, 0), dn, [(1, 0, 1), (1, 0, 0)]),
                                           X._row((0, 0, 0), (1e30, 0, 0), dn, [(0, 1, 0), (1, 0, 1), (1, 0, 0)])])])
    out = core.exit_face_rows(rows)
    t1 = out[:, 1].view(np.float32)
    assert list(out[:4, 0]) == [4, 3, 4, 0xffffffff]
    assert t1[0] == 1.0 and t1[1] == 1.0 and t1[2] == 1.0
    assert list(out[4:, 0]) == [0, 1] and np.all(np.isneginf(t1[4:]))
    # exactly: face 0 of row 4 is -5e38 and face 1 is -1e39, both below -FLT_MAX
    x0 = (0.5 - 1e30) / dn[0].astype(np.float64) / 2
    assert x0 < -np.finfo(np.float32).max


def test_packed_rows_need_the_tie_rule():
    """The reordered rows of the packed-search probe keep each row's faces
    (de-permuted through their original indices they are the row's records),
    and the reordering matters: searched plainly in slot order (first of equal
    quotients wins), many rows take a face other than the one the original
    order takes, so the probe's agreement with the oracle checks the
    original-index tie rule and does not hold by construction."""
    from tests import exit_rows as X
    rows = X.face_rows(np.random.default_rng(11), m=4096)
    packed = X.packed_rows(rows, np.random.default_rng(12))
    n = rows.shape[0]
    recs = np.ascontiguousarray(rows[:, 10:26]).view(np.uint16).reshape(n, 8, 4)
    slots = np.ascontiguousarray(packed[:, 10:26]).view(np.uint16).reshape(n, 8, 4)
    orig = np.ascontiguousarray(packed[:, 26:30]).view(np.uint16)
    nf = np.minimum(rows[:, 9].view(np.uint32), 8)
    for i in range(n):
        k = int(nf[i])
        assert sorted(orig[i, :k]) == list(range(k)) and np.all(orig[i, k:] == 0xFFFF)
        assert np.array_equal(slots[i, :k], recs[i, orig[i, :k]]) and not slots[i, k:].any()
    want = core.exit_face_rows(rows)
    plain = core.exit_face_rows(np.ascontiguousarray(packed[:, :26]))
    hit = plain[:, 0] != 0xFFFFFFFF
    mapped = np.where(hit, orig[np.arange(n), np.where(hit, plain[:, 0], 0)], 0xFFFFFFFF)
    assert np.array_equal(plain[:, 1], want[:, 1])  # the same quotient wins
    assert (mapped != want[:, 0]).sum() >= 500  # of 4109 rows; about a quarter hold a duplicated face


# --------------------------------------------------------------------------- absolute-sum mode

def test_abs_sum_mode():
    """The oracle's absolute-sum mode (the conditioning the GPU parity tests
    scale their per-element tolerance by): single-threaded, so every sum has
    one order.  The backward's terms are linear in the upstream gradient, so
    their magnitudes do not change when it flips sign and double when it
    doubles; the absolute sums bound the plain ones; and point_error's terms
    w * ray_error >= 0 give absolute sums equal to the plain ones."""
    s = scene.random_scene(400, seed=3, R=4)
    rays = camera.pinhole_rays(24, 16, eye=(0.1, -3.3, 0.2))
    o = rays[..., :3].reshape(-1, 3)
    start = host_ops.nearest_site(s.points, o[:1]).astype(np.uint32)[0] * np.ones(rays.shape[:-1], np.uint32)
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        rays, start, weight_threshold=0.001, threads=1)
    g = np.random.default_rng(1).normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    rerr = np.random.default_rng(2).uniform(0, 1, size=rays.shape[:-1]).astype(np.float32)

    def bwd(gg):
        return core.trace_bwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency,
                              s.offsets, rays, start, fw["rgba"], gg, ray_error=rerr, distortion=fw["distortion"],
                              W_total=fw["W_total"], S_total=fw["S_total"], t_far=fw["t_far"], threads=1)

    plain = bwd(g)
    with core.abs_sums():
        a = bwd(g)
        a_neg = bwd(-g)
        a_two = bwd(2 * g)
    again = bwd(g)  # the mode is off again after the context
    keys = ("points_grad", "diffuse_grad", "specular_grad", "density_grad")
    for k in keys:
        assert np.array_equal(a[k], a_neg[k]), k
        assert np.array_equal(a_two[k], 2 * a[k]), k
        assert (a[k] >= 0).all() and (a[k] >= np.abs(plain[k]) * (1 - 1e-6)).all(), k
        assert np.array_equal(again[k], plain[k]), k
    assert np.abs(plain["diffuse_grad"]).max() > 0
    assert (a["diffuse_grad"] > np.abs(plain["diffuse_grad"]) * 1.5).any()  # some texel sums cancel
    assert np.array_equal(a["point_error"], plain["point_error"])
