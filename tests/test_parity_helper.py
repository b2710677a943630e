"""The inference RGBA check itself (CPU): it accepts one fp16 ulp of RGB and
rejects two, a changed alpha bit, or a systematic shift within tolerance."""
import numpy as np
import pytest

from tests import helpers as H


def _img(seed=0):
    rng = np.random.default_rng(seed)
    return rng.uniform(0.0, 1.0, (24, 32, 4)).astype(np.float16)


def _step(a, k):
    """a moved k fp16 ulps up (k > 0) or down."""
    b = a.copy()
    for _ in range(abs(k)):
        b = np.nextafter(b, np.float16(np.inf if k > 0 else -np.inf))
    return b


def test_accepts_identical_and_one_ulp():
    w = _img()
    H.assert_infer_rgba(w.copy(), w)
    g = w.copy()
    g[3, 5, 1] = _step(g[3, 5, 1:2], 1)[0]
    g[7, 2, 0] = _step(g[7, 2, 0:1], -1)[0]
    H.assert_infer_rgba(g, w)


def test_rejects_two_ulps_alpha_and_bias():
    w = _img(1)
    g = w.copy()
    g[1, 1, 2] = _step(g[1, 1, 2:3], 2)[0]
    with pytest.raises(AssertionError):
        H.assert_infer_rgba(g, w)
    g = w.copy()
    g[4, 4, 3] = _step(g[4, 4, 3:4], 1)[0]
    with pytest.raises(AssertionError):
        H.assert_infer_rgba(g, w)
    # every RGB value one ulp up: within the per-value bound, but a mean shift
    # of about 2.4e-4 is far above what approximate shading produces
    with pytest.raises(AssertionError):
        H.assert_infer_rgba(np.concatenate([_step(w[..., :3], 1), w[..., 3:]], -1), w)


# ---- the half-precision accumulation bound (f16 attribute storage)


def _f16_case():
    """Oracle backward of a mini C3 frame with f16 maps, and the same terms
    summed in f32 (f16-valued maps held as f32), with their absolute sums and
    add counts."""
    from oracle import core
    from vorotracing_amd import camera

    s = H.mini_heightfield()
    rays = camera.orbit_rays(5, 48, 40)
    start = H.start_for(s, rays)
    d16, s16 = s.diffuse.astype(np.float16), s.specular.astype(np.float16)
    fw = core.trace_fwd(s.points, d16, s16, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets, rays, start,
                        weight_threshold=0.001)
    g = np.random.default_rng(1).normal(size=rays.shape[:-1] + (4,)).astype(np.float16)

    def bwd(f16):
        d, sp = (d16, s16) if f16 else (d16.astype(np.float32), s16.astype(np.float32))
        rgba, gg = (fw["rgba"], g) if f16 else (fw["rgba"].astype(np.float32), g.astype(np.float32))
        return core.trace_bwd(s.points, d, sp, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets, rays,
                              start, rgba, gg, distortion=fw["distortion"], W_total=fw["W_total"],
                              S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=0.001)

    o16, o32 = bwd(True), bwd(False)
    with core.abs_sums():
        A = bwd(False)
    with core.abs_sums(count=True):
        K = bwd(False)
    return bwd, o16, o32, A, K


def test_f16_bound_holds_for_the_oracles_own_orders():
    """The half-precision sums against the f32 sums of the same terms stay
    within one side's share of the bound; the counts are whole numbers and
    elements with no adds are zero on both sides."""
    _, o16, o32, A, K = _f16_case()
    for key in ("diffuse_grad", "specular_grad"):
        assert o16[key].dtype == np.float16
        half = H.f16_sum_bound(A[key], K[key]) / 2
        d = np.abs(o16[key].astype(np.float64) - o32[key].astype(np.float64))
        assert (d <= half).all(), key
        H.assert_f16_sum_close(o16[key], o32[key], A[key], K[key], key)
        # and the bound is tight where it matters: half of the elements get
        # less than 1 % of their own magnitude
        nz = K[key] > 0
        assert np.median(half[nz] / np.maximum(np.abs(o32[key][nz]), 1e-30)) < 1e-2, key


def test_f16_bound_rejects_a_wrong_term():
    """The specular map sampled at +d instead of -d (one planted slip in the
    oracle) moves most texture gradients far outside the bound."""
    from oracle import core

    bwd, o16, _, A, K = _f16_case()
    with core.plant(core.PLANT_SPEC_PLUS_D):
        bad = bwd(True)
    for key in ("diffuse_grad", "specular_grad"):
        with pytest.raises(AssertionError, match="outside the half-precision accumulation bound"):
            H.assert_f16_sum_close(bad[key], o16[key], A[key], K[key], key)
