"""GPU parity of the training forward / backward against the CPU oracle.

Forward outputs are deterministic and compared bit-for-bit (rgba, n, depth,
depth_idx, distortion, W/S totals, t_far); atomically accumulated outputs
(contribution, all gradients) are compared with the north star's 1e-3
relative tolerance, per element (helpers.assert_grad_close: within 1e-3 of
the element plus 1e-6 of the tensor's largest magnitude; the GPU adds in a
different order than the serial-per-ray CPU loop).
"""
import numpy as np
import pytest
import torch

from oracle import core
from tests import helpers as H
from vorotracing_amd import _C, camera, native, ops
from vorotracing_amd.model import VoroTracing

pytestmark = pytest.mark.gpu

GRAD_RTOL = 1e-3


def _rel_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    scale = max(np.abs(want).max(), 1e-30)
    return float(np.abs(got - want).max() / scale)


def _scene_tensors(s, dev, f16):
    adt = np.float16 if f16 else np.float32
    return (H.to_dev(s.points, dev), H.to_dev(s.diffuse.astype(adt), dev), H.to_dev(s.specular.astype(adt), dev),
            H.to_dev(s.density, dev), H.to_dev(s.adjacency, dev), H.to_dev(s.offsets, dev))


def _case(which):
    if which == "c1":
        s = H.c1_scene()
        rays = camera.pinhole_rays(64, 48, eye=(0.0, -4.0, 0.0))
        thr = 0.01
    elif which == "r8":
        s = H.small_random(1500, seed=5, R=8, Rs=4)
        rays = camera.pinhole_rays(48, 40, eye=(0.3, -3.2, 0.4))
        thr = 0.001
    else:
        s = H.mini_heightfield()
        rays = camera.orbit_rays(5, 64, 48)
        thr = 0.001
    return s, rays, H.start_for(s, rays), thr


@pytest.mark.parametrize("which,f16", [("c1", False), ("r8", False), ("mini_c3", False), ("c1", True)])
def test_fwd_parity(gpu, which, f16):
    s, rays, start, thr = _case(which)
    q = np.tile(np.array([0.9, 0.5, 0.1], np.float32), rays.shape[:-1] + (1,))
    adt = np.float16 if f16 else np.float32
    want = core.trace_fwd(s.points, s.diffuse.astype(adt), s.specular.astype(adt), s.diff_res, s.spec_res,
                          s.density, s.adjacency, s.offsets, rays, start, depth_quantiles=q, weight_threshold=thr,
                          return_contribution=True, want_stats=True)
    pts, dif, spe, den, adj, off = _scene_tensors(s, gpu, f16)
    st = native.new_stats(rays.size // 6, gpu)
    rgba, depth, depth_idx, contrib, n, dist, W, S, tf = _C.trace_vorotracing_fwd(
        pts, dif, spe, den, adj, off, H.to_dev(rays, gpu), H.to_dev(start, gpu), H.to_dev(q, gpu), thr, 1024, True,
        stats=st)
    torch.cuda.synchronize()
    H.assert_stats_equal(H.stats_np(st), want["stats"])  # the walk record through the _C entry
    assert rgba.dtype == (torch.float16 if f16 else torch.float32)
    assert np.array_equal(n.cpu().numpy(), want["n"])
    assert np.array_equal(rgba.cpu().numpy(), want["rgba"])
    assert np.array_equal(depth_idx.cpu().numpy(), want["depth_idx"])
    for got, key in ((depth, "depth"), (dist, "distortion"), (W, "W_total"), (S, "S_total"), (tf, "t_far")):
        g = got.cpu().numpy()
        assert np.array_equal(g.view(np.uint32), want[key].view(np.uint32)), key
    # f16 storage: contribution is summed with half-precision atomics (as in the
    # reference), so once a cell's sum is large, small weights are absorbed and
    # the result depends on the add order; only f32 is held to a tight bound.
    tol = 0.15 if f16 else 1e-5
    assert _rel_err(contrib.cpu().numpy().astype(np.float32), want["contribution"].astype(np.float32)) <= tol


@pytest.mark.parametrize("which,f16,extras", [("c1", False, True), ("r8", False, True), ("mini_c3", False, False),
                                              ("c1", True, False)])
def test_bwd_parity(gpu, which, f16, extras):
    s, rays, start, thr = _case(which)
    rng = np.random.default_rng(1)
    adt = np.float16 if f16 else np.float32
    q = np.tile(np.array([0.8, 0.3], np.float32), rays.shape[:-1] + (1,)) if extras else None
    fw = core.trace_fwd(s.points, s.diffuse.astype(adt), s.specular.astype(adt), s.diff_res, s.spec_res, s.density,
                        s.adjacency, s.offsets, rays, start, depth_quantiles=q, weight_threshold=thr)
    g = rng.normal(size=rays.shape[:-1] + (4,)).astype(adt)
    dg = rng.normal(size=rays.shape[:-1] + (2,)).astype(np.float32) * 0.1 if extras else None
    distg = (rng.uniform(0, 1, size=rays.shape[:-1] + (1,)).astype(np.float32)) if extras else None
    rerr = rng.uniform(0, 1, size=rays.shape[:-1]).astype(adt) if extras else None
    cag = 0.25 if extras else 0.0
    want = core.trace_bwd(s.points, s.diffuse.astype(adt), s.specular.astype(adt), s.diff_res, s.spec_res, s.density,
                          s.adjacency, s.offsets, rays, start, fw["rgba"], g, depth_quantiles=q,
                          depth_idx=fw["depth_idx"], depth_grad=dg, ray_error=rerr, contribution_alpha_grad=cag,
                          distortion=fw["distortion"], distortion_grad=distg, W_total=fw["W_total"],
                          S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr, want_stats=True)
    pts, dif, spe, den, adj, off = _scene_tensors(s, gpu, f16)
    d = lambda a, dt=None: None if a is None else H.to_dev(a, gpu)  # noqa: E731
    st = native.new_stats(rays.size // 6, gpu)
    pg, dgd, sgd, deng, rayg, perr = _C.trace_vorotracing_bwd(
        pts, dif, spe, den, adj, off, d(rays), d(start), d(fw["rgba"]), d(g), d(q), d(fw["depth_idx"]), d(dg),
        d(rerr), cag, d(fw["distortion"]), d(distg), d(fw["W_total"]), d(fw["S_total"]), d(fw["t_far"]), thr, 1024,
        stats=st)
    torch.cuda.synchronize()
    H.assert_stats_equal(H.stats_np(st), want["stats"])
    assert not rayg.cpu().numpy().any()
    if not f16:
        H.assert_grad_close(pg.cpu().numpy(), want["points_grad"], "points_grad")
        H.assert_grad_close(deng.cpu().numpy(), want["density_grad"], "density_grad")
        H.assert_grad_close(dgd.cpu().numpy(), want["diffuse_grad"], "diffuse_grad")
        H.assert_grad_close(sgd.cpu().numpy(), want["specular_grad"], "specular_grad")
    else:
        # f16 storage (as in the reference): the texture gradients are summed
        # with half-precision atomics, each add rounding to 11 bits, so once a
        # texel's sum is large the result depends on the add order; points and
        # density stay f32 atomics.
        assert _rel_err(pg.cpu().numpy(), want["points_grad"]) <= GRAD_RTOL * 10
        assert _rel_err(deng.cpu().numpy(), want["density_grad"]) <= GRAD_RTOL * 10
        assert _rel_err(dgd.cpu().numpy().astype(np.float32), want["diffuse_grad"].astype(np.float32)) <= 5e-2
        assert _rel_err(sgd.cpu().numpy().astype(np.float32), want["specular_grad"].astype(np.float32)) <= 5e-2
    if extras:
        H.assert_grad_close(perr.cpu().numpy(), want["point_error"], "point_error")
    else:
        assert perr is None


@pytest.mark.parametrize("n", [23, 87])
def test_bwd_parity_partial_waves(gpu, n):
    """Flat ray batches keep ray order: 23 rays make one wave of 23 lanes, 87
    a full wave and one of 23.  Fewer scattering lanes than the record's 29
    columns make each lane sum several columns; consecutive pixels of one
    row share cells, so the groups are real.  point_error on."""
    s, rays, _, thr = _case("r8")
    flat = rays[20, 8:8 + n].reshape(-1, 6) if n <= 40 else np.concatenate(
        [rays[20, 4:44], rays[21, 4:44], rays[22, 4:4 + n - 80]]).reshape(-1, 6)
    flat = np.ascontiguousarray(flat, np.float32)
    assert flat.shape == (n, 6)
    start = H.start_for(s, flat)
    rng = np.random.default_rng(3)
    dif32, spe32 = s.diffuse.astype(np.float32), s.specular.astype(np.float32)
    fw = core.trace_fwd(s.points, dif32, spe32, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        flat, start, weight_threshold=thr)
    g = rng.normal(size=(n, 4)).astype(np.float32)
    rerr = rng.uniform(0, 1, size=(n,)).astype(np.float32)
    want = core.trace_bwd(s.points, dif32, spe32, s.diff_res, s.spec_res, s.density, s.adjacency,
                          s.offsets, flat, start, fw["rgba"], g, ray_error=rerr, distortion=fw["distortion"],
                          W_total=fw["W_total"], S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    pts, dif, spe, den, adj, off = _scene_tensors(s, gpu, False)
    d = lambda a: None if a is None else H.to_dev(a, gpu)  # noqa: E731
    pg, dgd, sgd, deng, _, perr = _C.trace_vorotracing_bwd(
        pts, dif, spe, den, adj, off, d(flat), d(start), d(fw["rgba"]), d(g), None, None, None, d(rerr), 0.0,
        d(fw["distortion"]), None, d(fw["W_total"]), d(fw["S_total"]), d(fw["t_far"]), thr, 1024)
    torch.cuda.synchronize()
    H.assert_grad_close(pg.cpu().numpy(), want["points_grad"], "points_grad")
    H.assert_grad_close(deng.cpu().numpy(), want["density_grad"], "density_grad")
    H.assert_grad_close(dgd.cpu().numpy(), want["diffuse_grad"], "diffuse_grad")
    H.assert_grad_close(sgd.cpu().numpy(), want["specular_grad"], "specular_grad")
    H.assert_grad_close(perr.cpu().numpy(), want["point_error"], "point_error")
    assert np.abs(want["diffuse_grad"]).max() > 0 and np.abs(want["point_error"]).max() > 0


def test_c5_shape_fisheye_rolling_shutter(gpu):
    """Config-5 shape at test size: equidistant fisheye rays with a rolling
    shutter (a different origin per image row), start cells from the LBVH for
    every distinct origin (equal to brute force), forward bit for bit and
    backward within tolerance against the oracle."""
    s = H.mini_heightfield()
    rays = camera.fisheye_rolling_rays(80, 53, eye=camera.orbit_eye(3))
    assert len(np.unique(rays[..., :3].reshape(-1, 3), axis=0)) == rays.shape[0]  # one origin per row
    thr = 0.001
    model = VoroTracing.from_scene(s, device=gpu)
    rays_d = H.to_dev(rays, gpu)
    sp = model.get_starting_point(rays_d)
    start = H.start_for(s, rays)
    assert np.array_equal(sp.cpu().numpy(), start)
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        rays, start, weight_threshold=thr)
    pts, dif, spe, den, adj, off = _scene_tensors(s, gpu, False)
    rgba, depth, depth_idx, contrib, n, dist, W, S, tf = _C.trace_vorotracing_fwd(
        pts, dif, spe, den, adj, off, rays_d, sp, None, thr, 1024, False)
    assert np.array_equal(n.cpu().numpy(), fw["n"])
    assert np.array_equal(rgba.cpu().numpy().view(np.uint32), fw["rgba"].view(np.uint32))
    assert np.array_equal(dist.cpu().numpy().view(np.uint32), fw["distortion"].view(np.uint32))
    g = np.random.default_rng(4).normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    want = core.trace_bwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                          rays, start, fw["rgba"], g, distortion=fw["distortion"], W_total=fw["W_total"],
                          S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    d = lambda a: None if a is None else H.to_dev(a, gpu)  # noqa: E731
    pg, dgd, sgd, deng, rayg, perr = _C.trace_vorotracing_bwd(
        pts, dif, spe, den, adj, off, rays_d, sp, d(fw["rgba"]), d(g), None, None, None, None, 0.0,
        d(fw["distortion"]), None, d(fw["W_total"]), d(fw["S_total"]), d(fw["t_far"]), thr, 1024)
    torch.cuda.synchronize()
    H.assert_grad_close(pg.cpu().numpy(), want["points_grad"], "points_grad")
    H.assert_grad_close(deng.cpu().numpy(), want["density_grad"], "density_grad")
    H.assert_grad_close(dgd.cpu().numpy(), want["diffuse_grad"], "diffuse_grad")
    H.assert_grad_close(sgd.cpu().numpy(), want["specular_grad"], "specular_grad")


def test_autograd_model_forward_backward(gpu):
    """VoroTracing.forward -> TraceVoroTracing -> loss.backward matches the oracle bwd."""
    s, rays, start, thr = _case("c1")
    model = VoroTracing.from_scene(s, device=gpu)
    rays_d = H.to_dev(rays, gpu)
    sp = model.get_starting_point(rays_d)
    assert np.array_equal(sp.cpu().numpy(), start)
    rgba, depth, contrib, n, errbox, dist = model(rays_d, start_point=sp, weight_threshold=thr)
    gr = np.random.default_rng(2).normal(size=rgba.shape).astype(np.float32)
    (rgba * torch.from_numpy(gr).to(gpu)).sum().backward()
    dens = model.activated_density().detach().cpu().numpy()  # exp on the device, as the model feeds the kernel
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, 4, 4, dens, s.adjacency, s.offsets, rays, start,
                        weight_threshold=thr)
    want = core.trace_bwd(s.points, s.diffuse, s.specular, 4, 4, dens, s.adjacency, s.offsets, rays, start,
                          fw["rgba"], gr, distortion=fw["distortion"], W_total=fw["W_total"], S_total=fw["S_total"],
                          t_far=fw["t_far"], weight_threshold=thr)
    assert np.array_equal(rgba.detach().cpu().numpy(), fw["rgba"])
    H.assert_grad_close(model.primal_points.grad.cpu().numpy(), want["points_grad"], "points_grad")
    H.assert_grad_close(model.att_diffuse.grad.cpu().numpy(), want["diffuse_grad"], "diffuse_grad")
    H.assert_grad_close(model.att_specular.grad.cpu().numpy(), want["specular_grad"], "specular_grad")
    # density enters through exp: d/draw = d/ds * s
    ds = want["density_grad"] * dens
    H.assert_grad_close(model.density.grad.cpu().numpy(), ds, "density")


def test_train_errors_reference_messages(gpu):
    s, rays, start, thr = _case("c1")
    pts, dif, spe, den, adj, off = _scene_tensors(s, gpu, False)
    r = H.to_dev(rays, gpu)
    sp = H.to_dev(start, gpu)
    with pytest.raises(RuntimeError, match="diffuse and specular must have the same dtype"):
        _C.trace_vorotracing_fwd(pts, dif, spe.half(), den, adj, off, r, sp, None, thr, 1024, False)
    with pytest.raises(RuntimeError, match="rays must have 6 as the last dimension"):
        _C.trace_vorotracing_fwd(pts, dif, spe, den, adj, off, r[..., :5].contiguous(), sp, None, thr, 1024, False)
    with pytest.raises(RuntimeError, match="start_point must have the same batch size as rays"):
        _C.trace_vorotracing_fwd(pts, dif, spe, den, adj, off, r, sp[:3], None, thr, 1024, False)
    with pytest.raises(RuntimeError, match="Unsupported color dtype"):
        _C.trace_vorotracing_fwd(pts, dif.double(), spe.double(), den, adj, off, r, sp, None, thr, 1024, False)
    out = _C.trace_vorotracing_fwd(pts, dif, spe, den, adj, off, r, sp, None, thr, 1024, False)
    with pytest.raises(RuntimeError, match="rgb_grad_in must have 4 as the last dimension"):
        _C.trace_vorotracing_bwd(pts, dif, spe, den, adj, off, r, sp, out[0], out[0][..., :3].contiguous(), None,
                                 None, None, None, 0.0, out[5], None, out[6], out[7], out[8], thr, 1024)
    with pytest.raises(RuntimeError, match="depth_grad must be provided if depth_quantiles is provided"):
        qd = torch.full(rays.shape[:-1] + (1,), 0.5, device=gpu)
        _C.trace_vorotracing_bwd(pts, dif, spe, den, adj, off, r, sp, out[0], out[0], qd, out[2], None, None, 0.0,
                                 out[5], None, out[6], out[7], out[8], thr, 1024)


def test_start_cells_any_ray_order(gpu):
    """VoroTracing.get_starting_point queries one origin per run of equal
    consecutive origins; rays of three cameras shuffled together (short runs,
    origins repeated out of order) still get each origin's nearest site."""
    s = H.small_random(3000, seed=13)
    model = VoroTracing.from_scene(s, device=gpu)
    eyes = ((0.0, -3.0, 0.5), (2.5, 1.0, -0.4), (0.3, 0.2, 0.1))
    rays = np.concatenate([camera.pinhole_rays(20, 12, eye=e).reshape(-1, 6) for e in eyes])
    rays = rays[np.random.default_rng(3).permutation(rays.shape[0])]
    got = model.get_starting_point(H.to_dev(rays, gpu)).cpu().numpy()
    assert np.array_equal(got, H.start_for(s, rays))
    # an image in order: one run per image
    img = camera.pinhole_rays(20, 12, eye=eyes[1])
    assert np.array_equal(model.get_starting_point(H.to_dev(img, gpu)).cpu().numpy(), H.start_for(s, img))


def test_backward_reuses_the_forward_prefetch(gpu):
    """adj_diff_out / adj_diff: the forward's face-offset prefetch (equal to
    the oracle's) handed to the backward, which then skips its own; the
    gradients are the oracle's."""
    s, rays, start, thr = _case("r8")
    rng = np.random.default_rng(6)
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        rays, start, weight_threshold=thr)
    g = rng.normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    want = core.trace_bwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency,
                          s.offsets, rays, start, fw["rgba"], g, distortion=fw["distortion"], W_total=fw["W_total"],
                          S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    scene = _scene_tensors(s, gpu, False)
    rd, sd = H.to_dev(rays, gpu), H.to_dev(start, gpu)
    ad = torch.full((s.adjacency.shape[0] + 32, 4), float("nan"), dtype=torch.float16, device=gpu)
    got = _C.trace_vorotracing_fwd(*scene, rd, sd, None, thr, 1024, False, adj_diff_out=ad)
    torch.cuda.synchronize()
    m = s.num_faces
    pre = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    assert np.array_equal(ad.cpu().numpy()[:m].view(np.uint16), pre[:m].view(np.uint16))
    assert np.array_equal(got[0].cpu().numpy(), fw["rgba"])
    pg, dgd, sgd, deng, _, _ = _C.trace_vorotracing_bwd(
        *scene, rd, sd, got[0], H.to_dev(g, gpu), None, None, None, None, 0.0, got[5], None, got[6], got[7], got[8],
        thr, 1024, adj_diff=ad)
    torch.cuda.synchronize()
    for t, key in ((pg, "points_grad"), (deng, "density_grad"), (dgd, "diffuse_grad"), (sgd, "specular_grad")):
        H.assert_grad_close(t.cpu().numpy(), want[key], key)
    with pytest.raises(RuntimeError, match="adj_diff must be"):
        _C.trace_vorotracing_bwd(*scene, rd, sd, got[0], H.to_dev(g, gpu), None, None, None, None, 0.0, got[5], None,
                                 got[6], got[7], got[8], thr, 1024, adj_diff=ad[:-1])
