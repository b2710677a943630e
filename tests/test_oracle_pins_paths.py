"""Pins of the oracle paths that closed-form compositing alone leaves open
(no GPU): the specular lookup direction, the inference density and skip
gates, site-position gradients (including the reference's first-cell term and
unflushed tail), point_error, contribution and contribution_alpha_grad.

Each expectation comes from float64 closed forms or finite differences of the
scene geometry, not from the oracle's formulas.  Each test also switches on
the planted slip it is meant to catch (oracle.h OR_PLANT_*) and asserts that
the check then fails."""
import math

import numpy as np
import pytest

from oracle import core, host_ops
from vorotracing_amd import scene


def _sig(x):
    return 1.0 / (1.0 + math.exp(-x))


# --------------------------------------------------------------------------- specular lookup direction

def _two_site(far=1.0):
    """Sites 0 at the origin and 1 at (-far, 0, 0): cell 0 is the half-space
    x > -far/2, cell 1 the other half (unbounded, never integrated)."""
    pts = np.float32([[0, 0, 0], [-far, 0, 0]])
    adj = np.uint32([1, 0] + [0] * 32)
    off = np.uint32([0, 1, 2])
    return pts, adj, off


def _spec_case(R):
    """A ray from site 0 whose -d encodes exactly onto the centre of texel
    (c, c) of an R x R octahedral map (plane coordinate u = v = a, z part
    1 - 2a): c = 2 for R = 4 (a = 1/4), c = 4 for R = 8 (a = 1/8)."""
    a = 0.25 if R == 4 else 0.125
    c = 2 if R == 4 else 4
    m = np.array([a, a, 1.0 - 2.0 * a])
    d = -(m / np.linalg.norm(m))
    return d.astype(np.float32), c * R + c


@pytest.mark.parametrize("R", [4, 8])
def test_specular_sampled_at_minus_d(R):
    """Colour of the one integrated cell: sigmoid(diffuse + specular(-d)) with
    the specular map zero except at the texel -d encodes onto.  Checked on the
    training forward (f32), the fp16 and q8 inference kernels and, for the
    backward, where the specular gradient lands."""
    pts, adj, off = _two_site()
    d, texel = _spec_case(R)
    rays = np.concatenate([np.zeros(3, np.float32), d])[None].astype(np.float32)
    sigma = np.float32(1.3)
    dens = np.float32([[sigma], [0.5]])
    n3 = 3 * R * R
    dif = np.full((2, n3), 0.25, np.float32)
    spe = np.zeros((2, n3), np.float32)
    vals = np.float32([1.5, -1.0, 0.5])
    spe[0, 3 * texel:3 * texel + 3] = vals
    t1 = 0.5 / abs(float(d[0]))  # bisector x = -1/2
    a = 1.0 - math.exp(-float(sigma) * t1)
    want = np.array([a * _sig(0.25 + float(v)) for v in vals] + [a])

    def fwd():
        return core.trace_fwd(pts, dif, spe, R, R, dens, adj, off, rays, np.uint32([0]), weight_threshold=1e-6)

    def infer_f16():
        ad = core.prefetch_adj(pts, adj, off)
        d4 = host_ops.pad_3to4(dif.astype(np.float16), R)
        s4 = host_ops.pad_3to4(spe.astype(np.float16), R)
        return core.trace_infer_f16(pts, d4, s4, R, R, dens, adj, off, ad, rays, np.uint32([0]),
                                    weight_threshold=1e-6)[0]

    def infer_q8():
        ad = core.prefetch_adj(pts, adj, off)
        # scale 1/64, offset -2: the map's values (0, 0.25, 1.5, -1, 0.5) are exact
        qd = np.round((dif + 2.0) * 64).astype(np.uint8)
        qs = np.round((spe + 2.0) * 64).astype(np.uint8)
        sc, of = [1.0 / 64] * 3, [-2.0] * 3
        return core.trace_infer_q8(pts, qd, qs, R, R, sc, of, sc, of, dens, adj, off, ad, rays, np.uint32([0]),
                                   weight_threshold=1e-6)[0]

    def check(tol):
        ok = []
        ok.append(np.abs(fwd()["rgba"][0].astype(np.float64) - want).max() < 1e-5)
        for f in (infer_f16, infer_q8):
            ok.append(np.abs(f()[0].astype(np.float64) - want).max() < tol)
        return ok

    assert all(check(1e-3)), check(1e-3)
    # backward: with dL/drgb = (1, 1, 1), only the sampled texel's specular
    # logits get gradient w * sigmoid'(logit)
    out = fwd()
    g = np.float32([[1, 1, 1, 0]])
    bw = core.trace_bwd(pts, dif, spe, R, R, dens, adj, off, rays, np.uint32([0]), out["rgba"], g,
                        distortion=out["distortion"], W_total=out["W_total"], S_total=out["S_total"],
                        t_far=out["t_far"], weight_threshold=1e-6)
    sg = bw["specular_grad"][0].reshape(R * R, 3).astype(np.float64)
    wg = np.array([a * _sig(0.25 + float(v)) * (1 - _sig(0.25 + float(v))) for v in vals])
    assert np.abs(sg[texel] - wg).max() < 2e-5 * max(1.0, np.abs(wg).max())
    assert np.abs(np.delete(sg, texel, 0)).max() < 1e-4 * np.abs(wg).max()
    with core.plant(core.PLANT_SPEC_PLUS_D):
        assert not any(check(1e-3))
        bwp = core.trace_bwd(pts, dif, spe, R, R, dens, adj, off, rays, np.uint32([0]), out["rgba"], g,
                             weight_threshold=1e-6)
        assert np.abs(bwp["specular_grad"][0].reshape(R * R, 3)[texel] - wg).max() > 1e-2


# --------------------------------------------------------------------------- inference gates

def _infer_two_site(sigma0, far=200.0, skip=0.0):
    pts, adj, off = _two_site(far)
    R = 4
    dif = np.full((2, 48), 0.3, np.float32)
    spe = np.zeros((2, 48), np.float32)
    dens = np.float32([[sigma0], [2.0]])
    rays = np.float32([[0, 0, 0, -1, 0, 0]])
    ad = core.prefetch_adj(pts, adj, off)
    d4 = host_ops.pad_3to4(dif.astype(np.float16), R)
    s4 = host_ops.pad_3to4(spe.astype(np.float16), R)
    f16 = core.trace_infer_f16(pts, d4, s4, R, R, dens, adj, off, ad, rays, np.uint32([0]), weight_threshold=1e-6,
                               cell_skip_threshold=skip)[0][0]
    q = np.full((2, 48), 128, np.uint8)
    q8 = core.trace_infer_q8(pts, q, q, R, R, [0.01] * 3, [-1.0] * 3, [0.01] * 3, [-1.28] * 3, dens, adj, off, ad,
                             rays, np.uint32([0]), weight_threshold=1e-6, cell_skip_threshold=skip)[0][0]
    tr = core.trace_fwd(pts, dif, spe, R, R, dens, adj, off, rays, np.uint32([0]), weight_threshold=1e-6)
    return f16, q8, tr["rgba"][0]


def test_inference_density_gate_leaves_transmittance():
    """Inference skips a cell of density <= 1e-6 entirely (T untouched,
    ray_integrator_octmap.cuh:323-327, :495-499); the training forward still
    applies alpha = 1 - exp(-s dt).  One 100-unit segment of density 1e-6:
    inference alpha is exactly 0, training alpha is 1 - exp(-1e-4)."""
    f16, q8, tr = _infer_two_site(1e-6)
    assert np.all(f16.view(np.uint16) == 0) and np.all(q8.view(np.uint16) == 0)
    assert abs(float(tr[3]) - (1 - math.exp(-1e-4))) < 2e-7
    # just above the gate the segment counts
    f16b, q8b, _ = _infer_two_site(np.nextafter(np.float32(1e-6), np.float32(1)))
    assert abs(float(f16b[3]) - (1 - math.exp(-1e-4))) < 1e-7 and float(q8b[3]) == float(f16b[3])
    with core.plant(core.PLANT_INFER_NO_DENSITY_GATE):
        f16p, q8p, _ = _infer_two_site(1e-6)
        assert float(f16p[3]) > 0 and float(q8p[3]) > 0


def _lattice_ray(nx=6, sigmas=None, R=4, diff_logits=None):
    """Sites (x, 1, 1), x = 0..nx-1, of an nx x 3 x 3 lattice; the ray from
    (0, 1, 1) along +x exits cell x at t = x + 1/2; the last cell is unbounded
    and never integrated.  Constant textures per cell."""
    s = scene.cubic_lattice(nx, 3, 3, R=R)
    cells = [int(np.argmin(np.linalg.norm(s.points - np.array([x, 1, 1]), axis=1))) for x in range(nx)]
    dens = np.full((s.num_points, 1), 0.5, np.float32)
    sig = np.full(nx, 0.4) if sigmas is None else np.asarray(sigmas, np.float64)
    for c, v in zip(cells, sig):
        dens[c, 0] = np.float32(v)
    lg = np.linspace(-1.2, 1.5, nx) if diff_logits is None else np.asarray(diff_logits)
    dif = np.zeros((s.num_points, 3 * R * R), np.float32)
    for c, v in zip(cells, lg):
        dif[c] = np.float32(v)
    spe = np.zeros_like(dif)
    rays = np.float32([[0, 1, 1, 1, 0, 0]])
    return s, cells, dens, dif, spe, rays


def _closed_weights(sig, dts):
    T, w, a = 1.0, [], []
    for sv, dt in zip(sig, dts):
        al = 1.0 - math.exp(-float(np.float32(sv)) * dt)
        w.append(T * al)
        a.append(al)
        T *= 1.0 - al
    return np.array(w), np.array(a), T


def test_inference_skip_gate_removes_exactly_the_skipped_colour():
    """With skip s, a cell of weight w < s adds no colour but still
    attenuates (tracing_octmap.cu:567-609, ray_integrator_octmap.cuh:336-340):
    RGB(0) - RGB(s) = sum of w_i c_i over w_i < s, alpha identical."""
    s, cells, dens, dif, spe, rays = _lattice_ray()
    ad = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    d4 = host_ops.pad_3to4(dif.astype(np.float16), 4)
    s4 = host_ops.pad_3to4(spe.astype(np.float16), 4)
    start = np.uint32([cells[0]])
    w, a, _ = _closed_weights([0.4] * 5, [0.5, 1, 1, 1, 1])
    lg = np.linspace(-1.2, 1.5, 6)
    colour = np.array([_sig(float(np.float16(v))) for v in lg[:5]])
    skip = 0.15  # skips cells 3 and 4 (w = 0.121, 0.081); their alpha (0.33) is above it

    def render(sk):
        return core.trace_infer_f16(s.points, d4, s4, 4, 4, dens, s.adjacency, s.offsets, ad, rays, start,
                                    weight_threshold=1e-6, cell_skip_threshold=sk)[0][0].astype(np.float64)

    def check():
        full, cut = render(0.0), render(skip)
        removed = float((w * colour)[w < skip].sum())
        return (full[3] == cut[3] and np.all(np.abs((full[:3] - cut[:3]) - removed) < 2e-3)
                and abs(full[0] - float((w * colour).sum())) < 2e-3)

    assert (w < skip).sum() == 2 and (a[w < skip] >= skip).all()
    assert check()
    with core.plant(core.PLANT_SKIP_ON_ALPHA):
        assert not check()


# --------------------------------------------------------------------------- site-position gradients

SHIFT = np.array([1.0, 0.5, 0.25])  # keeps the zero vector off every site (the first-cell term divides by dp)


def _plane_t(prim, opp, o, d):
    n = opp - prim
    return float(((prim + opp) / 2 - o) @ n / (n @ d))


def _plane_grad_fd(prim, opp, o, d, h=1e-6):
    """d t / d prim of the bisector plane of (prim, opp), float64 central differences."""
    g = np.zeros(3)
    for k in range(3):
        e = np.zeros(3)
        e[k] = h
        g[k] = (_plane_t(prim + e, opp, o, d) - _plane_t(prim - e, opp, o, d)) / (2 * h)
    return g


def _grad_lattice(nx, sig, lg, ga, gc, o_x, thr, max_int=1024, ray_error=None, cag=0.0):
    """Oracle forward and backward of one +x ray through a shifted lattice."""
    s, cells, dens, dif, spe, _ = _lattice_ray(nx, sig, diff_logits=lg)
    pts = (s.points.astype(np.float64) + SHIFT).astype(np.float32)
    o = np.array([o_x, 1.0, 1.0]) + SHIFT
    rays = np.concatenate([o, [1.0, 0.0, 0.0]])[None].astype(np.float32)
    start = np.uint32([cells[0]])
    out = core.trace_fwd(pts, dif, spe, 4, 4, dens, s.adjacency, s.offsets, rays, start, weight_threshold=thr,
                         max_intersections=max_int, want_stats=True, return_contribution=True)
    g = np.float32([[gc[0], gc[1], gc[2], ga]])
    bw = core.trace_bwd(pts, dif, spe, 4, 4, dens, s.adjacency, s.offsets, rays, start, out["rgba"], g,
                        ray_error=None if ray_error is None else np.float32([[ray_error]]),
                        contribution_alpha_grad=cag, distortion=out["distortion"], W_total=out["W_total"],
                        S_total=out["S_total"], t_far=out["t_far"], weight_threshold=thr, max_intersections=max_int)
    return s, cells, pts, o, out, bw


def _closed_segment_grads(sig, lg, ga, gc, o_x, k):
    """float64 loss L = g_rgb . rgb + g_a alpha of the first k segments of the
    lattice ray as a function of the segment lengths, and h_i = dL/dlen_i by
    central differences."""
    b = [0.0] + [x + 0.5 - o_x for x in range(k)]           # boundaries t_0 = 0, t_x = x + 1/2 - o_x
    lens = np.diff(np.array(b))
    col = np.array([[_sig(float(np.float32(v)))] * 3 for v in lg[:k]])

    def L(ln):
        T, acc = 1.0, np.zeros(3)
        for i in range(k):
            al = 1.0 - math.exp(-float(np.float32(sig[i])) * ln[i])
            acc += T * al * col[i]
            T *= 1.0 - al
        return float(np.dot(gc, acc) + ga * (1.0 - T))

    h = np.zeros(k)
    for i in range(k):
        e = np.zeros(k)
        e[i] = 1e-6
        h[i] = (L(lens + e) - L(lens - e)) / 2e-6
    return h


@pytest.mark.parametrize("ending", ["opacity", "exit", "cap"])
def test_position_gradient_closed_form_with_reference_quirks(ending):
    """Site gradients on a lattice ray against float64 closed forms: a site's
    x-gradient is (dL/dt_entry + dL/dt_exit) / 2 with dL/dt at a boundary
    h_before - h_after (h_i = dL/dlen_i); the reference's quirks then apply
    (ray_integrator_octmap.cuh:805-855): the first cell also gets -h_0 times
    d t / d site of the bisector against the zero vector (the initial
    'previous site', :816, :875), an opacity stop flushes the current cell but
    not the cell behind its exit (:851-855), and an exit or the step cap
    flushes neither the last integrated cell nor the one behind it."""
    nx = 10
    sig = np.array([0.35, 0.6, 0.5, 0.8, 0.45, 0.7, 0.9, 0.55, 0.6, 0.5])
    lg = np.linspace(-0.8, 1.1, nx)
    ga, gc, o_x = 0.37, np.array([0.9, -0.4, 0.25]), 0.15
    if ending == "opacity":
        thr, max_int = 0.05, 1024
    elif ending == "exit":
        sig = sig * 0.1
        thr, max_int = 1e-6, 1024
    else:
        thr, max_int = 1e-6, 5
    s, cells, pts, o, out, bw = _grad_lattice(nx, sig, lg, ga, gc, o_x, thr, max_int)
    k = int(out["stats"]["integrated"][0])  # integrated cells 0..k-1
    if ending == "opacity":
        assert 2 <= k < nx - 1 and float(out["rgba"][0, 3]) > 1 - thr - 1e-6
    elif ending == "exit":
        assert k == nx - 1
    else:
        assert k == max_int and int(out["n"][0, 0]) == max_int + 1
    h = _closed_segment_grads(sig, lg, ga, gc, o_x, k)
    hx = np.concatenate([h, [0.0]])
    want = np.zeros((nx, 3))
    for i in range(k + 1):
        entry = (hx[i - 1] - hx[i]) if i >= 1 else 0.0
        exit_ = (hx[i] - hx[i + 1]) if i < k else 0.0
        want[i, 0] = 0.5 * (entry + exit_)
    p0 = pts[cells[0]].astype(np.float64)
    want[0] += -h[0] * _plane_grad_fd(p0, np.zeros(3), o, np.array([1.0, 0, 0]))
    if ending == "opacity":
        want[k] = 0.0          # the cell behind the stopping cell's exit is never flushed
    else:
        want[k - 1] = 0.0      # neither is the last integrated cell, on exit or at the cap
        want[k] = 0.0
    got = bw["points_grad"][cells].astype(np.float64)
    scale = np.abs(want).max()
    assert np.abs(got - want).max() <= 1e-4 * scale, (got, want)
    # every other site is untouched
    rest = np.setdiff1d(np.arange(s.num_points), cells)
    assert not bw["points_grad"][rest].any()

    # planted slips the check catches
    plants = [core.PLANT_NO_FIRST_CELL_TERM, core.PLANT_NO_DT0_PREV]
    if ending == "opacity":
        plants.append(core.PLANT_FLUSH_CUR_ON_STOP)
    for code in plants:
        with core.plant(code):
            _, _, _, _, _, bwp = _grad_lattice(nx, sig, lg, ga, gc, o_x, thr, max_int)
        gp = bwp["points_grad"][cells].astype(np.float64)
        assert np.abs(gp - want).max() > 1e-2 * scale, code


def _fd_scene():
    """Sites on a 1/64 grid.  The diffuse map is constant over each cell's
    texels: the reference's backward does not differentiate the diffuse lookup
    direction normalize(o + t0 d - site) with respect to the site, so only a
    direction-independent diffuse colour makes the loss's site derivative the
    one it computes.  The specular lookup depends on d alone and stays random."""
    s = scene.random_scene(400, seed=31, R=4, extent=1.5, grid=1 / 64, density_mu=0.3)
    s.diffuse[:] = np.repeat(s.diffuse[:, :3], 16, axis=0).reshape(s.diffuse.shape)
    return s


def _fd_position_checks(max_checks=60):
    """(fd, backward) pairs of site-gradient components: single-ray losses,
    interior cells of opacity-stopped rays whose every step integrates."""
    s = _fd_scene()
    rng = np.random.default_rng(5)
    dens = s.density
    o = np.float32([0.05, -2.6, 0.1])
    start = host_ops.nearest_site(s.points, o[None]).astype(np.uint32)
    h = 2.0 ** -10
    off64 = s.offsets.astype(np.int64)
    src = np.repeat(np.arange(s.num_points), np.diff(off64))
    dst = s.adjacency[:off64[-1]].astype(np.int64)

    def offsets_exact(c, ax):
        """Every face offset touching site c stays exact in fp16 when c moves by
        up to 2h along ax (then the forward sees the exact geometry)."""
        sel = (src == c) | (dst == c)
        dlt = (s.points[dst[sel], ax].astype(np.float64) - s.points[src[sel], ax].astype(np.float64))
        for m in (-2, -1, 1, 2):
            moved = dlt + np.where(src[sel] == c, -m * h, m * h)
            if not np.array_equal(moved.astype(np.float16).astype(np.float64), moved):
                return False
        return True

    pairs = []
    for trial in range(40):
        d = rng.normal(size=3) * [0.22, 0, 0.22] + [0, 1, 0]
        d = (d / np.linalg.norm(d)).astype(np.float32)
        ray = np.concatenate([o, d])[None].astype(np.float32)
        g = rng.normal(size=(1, 4)).astype(np.float32)
        thr = 0.02

        def fwd(pts):
            return core.trace_fwd(pts, s.diffuse, s.specular, 4, 4, dens, s.adjacency, s.offsets, ray, start,
                                  weight_threshold=thr, want_stats=True)

        base = fwd(s.points)
        if not float(base["rgba"][0, 3]) >= 1 - thr:
            continue  # not an opacity stop
        _, _, log = core.trace_infer_f16(s.points, host_ops.pad_3to4(s.diffuse.astype(np.float16), 4),
                                         host_ops.pad_3to4(s.specular.astype(np.float16), 4), 4, 4,
                                         np.zeros_like(dens), s.adjacency, s.offsets,
                                         core.prefetch_adj(s.points, s.adjacency, s.offsets), ray, start,
                                         max_log=512)
        k = int(base["stats"]["integrated"][0])
        if k < 5 or int(base["stats"]["visits"][0]) != k:
            continue  # only walks whose every step integrates (then path[i] is the i-th integrated cell)
        path = [int(c) for c in log[0][:k]]
        bw = core.trace_bwd(s.points, s.diffuse, s.specular, 4, 4, dens, s.adjacency, s.offsets, ray, start,
                            base["rgba"], g, distortion=base["distortion"], W_total=base["W_total"],
                            S_total=base["S_total"], t_far=base["t_far"], weight_threshold=thr)
        gfull = bw["points_grad"]
        for c in path[1:k - 1]:
            for ax in range(3):
                if not offsets_exact(c, ax):
                    continue
                vals = []
                for m in (-2, -1, 1, 2):
                    p = s.points.copy()
                    p[c, ax] = np.float32(float(p[c, ax]) + m * h)
                    out = fwd(p)
                    if out["stats"]["visit_hash"][0] != base["stats"]["visit_hash"][0]:
                        break
                    vals.append(float((out["rgba"][0].astype(np.float64) * g[0]).sum()))
                if len(vals) < 4:
                    continue
                fd = (vals[0] - 8 * vals[1] + 8 * vals[2] - vals[3]) / (12 * h)
                pairs.append((fd, float(gfull[c, ax]), float(np.abs(gfull).max())))
        if len(pairs) >= max_checks:
            break
    return pairs


def _fd_bad(pairs):
    return [(fd, got) for fd, got, m in pairs if abs(fd - got) > 2e-3 * abs(fd) + 2e-4 * m]


def test_position_gradient_vs_central_differences_interior_cells():
    """Single-ray losses on a scene whose sites lie on a 1/64 grid: moving a
    site by multiples of 2^-10 keeps its fp16 face offsets exact (checked per
    site), so the forward sees the exact geometry (diffuse colour constant per
    cell, see _fd_scene).  On opacity-stopped rays, the gradient of each
    interior cell's site (neither the first cell nor the last) equals the
    fourth-order central difference of the forward's loss; dropping the
    previous site's t0 term (a planted slip) breaks it."""
    pairs = _fd_position_checks()
    assert len(pairs) >= 30
    assert not _fd_bad(pairs), _fd_bad(pairs)[:5]
    with core.plant(core.PLANT_NO_DT0_PREV):
        assert len(_fd_bad(_fd_position_checks(20))) >= 5


# --------------------------------------------------------------------------- point_error, contribution

def test_point_error_and_contribution_are_weights():
    """point_error[cell] = w * ray_error (ray_integrator_octmap.cuh:733-736)
    and the forward's contribution[cell] = w (:131-134), w the closed-form
    compositing weight of the lattice ray's cells."""
    nx = 6
    sig = np.array([0.4, 0.9, 0.3, 0.6, 0.5, 0.5])
    lg = np.linspace(-0.5, 0.5, nx)
    err = 0.7
    _, cells, _, _, out, bw = _grad_lattice(nx, sig, lg, 0.0, np.zeros(3), 0.15, 1e-6, ray_error=err)
    dts = [0.5 - 0.15] + [1.0] * (nx - 2)   # the first cell from o_x = 0.15 to its exit at 1/2
    w, a, _ = _closed_weights(sig[:nx - 1], dts)
    got_pe = bw["point_error"][cells[:nx - 1], 0].astype(np.float64)
    got_c = out["contribution"][cells[:nx - 1], 0].astype(np.float64)
    assert np.abs(got_pe - err * w).max() < 1e-6 and np.abs(got_c - w).max() < 1e-6
    assert bw["point_error"][cells[nx - 1], 0] == 0 and out["contribution"][cells[nx - 1], 0] == 0
    with core.plant(core.PLANT_POINT_ERROR_ALPHA):
        _, _, _, _, _, bwp = _grad_lattice(nx, sig, lg, 0.0, np.zeros(3), 0.15, 1e-6, ray_error=err)
    assert np.abs(bwp["point_error"][cells[:nx - 1], 0] - err * w).max() > 1e-2


def test_contribution_alpha_grad_is_an_alpha_gradient():
    """contribution_alpha_grad c is added to every ray's alpha gradient
    (tracing_octmap.cu:281, _wrapper.py:113-117): with no other upstream
    gradient, density gradients equal c * d(alpha)/d(density) by central
    differences of the forward."""
    nx = 6
    sig = np.array([0.4, 0.9, 0.3, 0.6, 0.5, 0.5])
    lg = np.linspace(-0.5, 0.5, nx)
    c = 1.7
    s, cells, pts, o, out, bw = _grad_lattice(nx, sig, lg, 0.0, np.zeros(3), 0.15, 1e-6, cag=c)
    rays = np.concatenate([o, [1.0, 0, 0]])[None].astype(np.float32)
    _, _, dens, dif, spe, _ = _lattice_ray(nx, sig, diff_logits=lg)

    def alpha(dd):
        r = core.trace_fwd(pts, dif, spe, 4, 4, dd, s.adjacency, s.offsets, rays, np.uint32([cells[0]]),
                           weight_threshold=1e-6)
        return float(r["rgba"][0, 3])

    for cell in cells[:nx - 1]:
        e = np.float32(1e-3)
        dp, dm = dens.copy(), dens.copy()
        dp[cell] += e
        dm[cell] -= e
        fd = c * (alpha(dp) - alpha(dm)) / (float(dp[cell, 0]) - float(dm[cell, 0]))
        got = float(bw["density_grad"][cell, 0])
        assert abs(fd - got) <= 2e-3 * abs(fd) + 1e-5, (cell, fd, got)
    with core.plant(core.PLANT_IGNORE_CONTRIB_GRAD):
        _, _, _, _, _, bwp = _grad_lattice(nx, sig, lg, 0.0, np.zeros(3), 0.15, 1e-6, cag=c)
    assert not bwp["density_grad"].any()
