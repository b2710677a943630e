"""GPU parity of the training forward / backward against the CPU oracle.

Forward outputs are deterministic and compared bit-for-bit (rgba, n, depth,
depth_idx, distortion, W/S totals, t_far); atomically accumulated outputs
(contribution, all gradients) are compared with the north star's 1e-3
relative tolerance, per element (helpers.assert_grad_close: within 1e-3 of
the element plus 1e-6 of the tensor's largest magnitude; the GPU adds in a
different order than the serial-per-ray CPU loop).  Outputs accumulated in
half precision (f16 attribute storage) are held per element to the
half-precision accumulation bound of their absolute sum and add count
(helpers.f16_sum_bound).  The "hf8" case has the reference's 8x8 diffuse and
8x8 specular maps.
"""
import types

import numpy as np
import pytest
import torch

from oracle import core
from tests import helpers as H
from vorotracing_amd import _C, _lib, camera, native, ops
from vorotracing_amd.model import VoroTracing

pytestmark = pytest.mark.gpu

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
    elif which == "hf8":  # 8x8 diffuse and specular maps, the reference's compiled resolution
        s = H.mini_heightfield_r8()
        rays = camera.orbit_rays(5, 128, 96)
        thr = 0.001
    else:
        s = H.mini_heightfield()
        rays = camera.orbit_rays(5, 64, 48)
        thr = 0.001
    return s, rays, H.start_for(s, rays), thr


@pytest.mark.parametrize("which,f16", [("c1", False), ("r8", False), ("mini_c3", False), ("hf8", False), ("c1", True),
                                      ("mini_c3", True), ("hf8", True)])
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
    if not f16:
        # weights are >= 0: the sum is its own absolute sum
        H.assert_grad_close(contrib.cpu().numpy(), want["contribution"], "contribution",
                            abs_sum=want["contribution"])
    else:
        # f16 storage: contribution is summed with half-precision atomics (as in
        # the reference), one rounding per add, in another order than the
        # oracle's: per element within the half-precision accumulation bound
        # of its weight sum and count
        with core.abs_sums(count=True):
            k = core.trace_fwd(s.points, s.diffuse.astype(adt).astype(np.float32),
                               s.specular.astype(adt).astype(np.float32), s.diff_res, s.spec_res, s.density,
                               s.adjacency, s.offsets, rays, start, weight_threshold=thr,
                               return_contribution=True)["contribution"]
        w32 = core.trace_fwd(s.points, s.diffuse.astype(adt).astype(np.float32),
                             s.specular.astype(adt).astype(np.float32), s.diff_res, s.spec_res, s.density,
                             s.adjacency, s.offsets, rays, start, weight_threshold=thr,
                             return_contribution=True)["contribution"]  # the weights are >= 0: their own sum
        H.assert_f16_sum_close(contrib.cpu().numpy(), want["contribution"], w32, k, "contribution")


@pytest.mark.parametrize("which,f16,extras,gscale", [
    ("c1", False, True, 1.0), ("r8", False, True, 1.0), ("mini_c3", False, False, 1.0), ("hf8", False, True, 1.0),
    ("c1", True, False, 1.0), ("c1", True, True, 1.0), ("mini_c3", True, True, 1.0), ("hf8", True, True, 1.0),
    ("hf8", True, False, 2.0 ** -12)])
def test_bwd_parity(gpu, which, f16, extras, gscale):
    """``gscale`` 2^-12 scales the upstream gradient so that most texel
    gradients of the f16-storage backward are f16 subnormals (below 2^-14):
    the half-precision atomic must keep them, and its +0 into the other half
    of each word must leave a subnormal neighbour as it is."""
    s, rays, start, thr = _case(which)
    rng = np.random.default_rng(1)
    adt = np.float16 if f16 else np.float32
    q = np.tile(np.array([0.8, 0.3], np.float32), rays.shape[:-1] + (1,)) if extras else None
    fw = core.trace_fwd(s.points, s.diffuse.astype(adt), s.specular.astype(adt), s.diff_res, s.spec_res, s.density,
                        s.adjacency, s.offsets, rays, start, depth_quantiles=q, weight_threshold=thr)
    g = (rng.normal(size=rays.shape[:-1] + (4,)) * gscale).astype(adt)
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
        if extras:
            H.assert_grad_close(perr.cpu().numpy(), want["point_error"], "point_error")
    else:
        # f16 storage (as in the reference): texture gradients and point_error
        # are summed with half-precision atomics, one rounding per add, in
        # another order than the oracle's: per element within the
        # half-precision accumulation bound of the element's absolute sum and
        # add count.  Points and density stay f32 atomics.
        A, K = H.f16_train_sums(s, rays, start, thr, fw, g, depth_quantiles=q, depth_idx=fw["depth_idx"],
                                depth_grad=dg, ray_error=rerr, contribution_alpha_grad=cag, distortion_grad=distg)
        H.assert_grad_close(pg.cpu().numpy(), want["points_grad"], "points_grad", abs_sum=A["points_grad"])
        H.assert_grad_close(deng.cpu().numpy(), want["density_grad"], "density_grad", abs_sum=A["density_grad"])
        for got, key in ((dgd, "diffuse_grad"), (sgd, "specular_grad")) + (((perr, "point_error"),) if extras else ()):
            H.assert_f16_sum_close(got.cpu().numpy(), want[key], A[key], K[key], key)
        if gscale < 1.0:
            for key in ("diffuse_grad", "specular_grad"):
                w = np.abs(want[key].astype(np.float32))
                sub = (w > 0) & (w < 2.0 ** -14)
                assert sub.sum() > 0.5 * (w > 0).sum(), f"{key}: too few of the gradients are f16 subnormals"
                got = np.abs(dgd.cpu().numpy() if key == "diffuse_grad" else sgd.cpu().numpy()).astype(np.float32)
                assert ((got > 0) & (got < 2.0 ** -14)).sum() >= 0.9 * sub.sum(), f"{key}: subnormals lost"
    if not extras:
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
    # a larger shuffled batch: runs about as many as rays, one query each
    big = np.concatenate([camera.pinhole_rays(48, 32, eye=e).reshape(-1, 6) for e in eyes])
    big = big[np.random.default_rng(4).permutation(big.shape[0])]
    assert np.array_equal(model.get_starting_point(H.to_dev(big, gpu)).cpu().numpy(), H.start_for(s, big))
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


def _f16_atomic(halves, index, values):
    h = H.to_dev(halves.view(np.uint16), torch.device("cuda:0"))
    # the device tensors stay referenced until the kernel has run (a freed
    # temporary's block would be handed to the next allocation)
    idx = H.to_dev(index.astype(np.uint32), h.device)
    val = H.to_dev(values.astype(np.float32), h.device)
    _lib.call("vt_debug_f16_atomic_add", h.data_ptr(), h.numel(), idx.data_ptr(), val.data_ptr(), index.size,
              torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return h.cpu().numpy().view(np.float16)


def test_f16_atomic_keeps_subnormals(gpu):
    """The f16-storage backward's half atomic (the reference's atomicAdd on
    __half): one add per 32-bit word, into either half, of values whose
    halves and sums are f16 subnormals (below 2^-14), zero, or normal.  The
    target half is RN(half + RN_half(v)) with subnormals kept, computed in
    float64 (exact for two halves), and the other half of the word, which
    receives +0, keeps its bits (subnormals included)."""
    print("case: vt_debug_f16_atomic_add, 8192 words of one add each", flush=True)
    rng = np.random.default_rng(3)
    m = 8192
    sub = lambda n: (rng.integers(1, 1024, n) * rng.choice([-1.0, 1.0], n) * 2.0 ** -24)  # noqa: E731
    init = np.concatenate([sub(m // 2), rng.normal(0, 1e-3, m // 4), np.zeros(m // 8),
                           rng.normal(0, 1, m // 8)]).astype(np.float16)
    halves = rng.permutation(np.concatenate([init, sub(m).astype(np.float16)]))
    halves[halves == 0] = np.float16(0.0)  # +0 only (the backward's buffers start at +0 and never hold -0)
    parity = rng.integers(0, 2, m)
    index = 2 * np.arange(m) + parity
    values = np.concatenate([
        sub(m // 2) * rng.uniform(0.5, 1.5, m // 2),          # rounding to subnormal halves (or to 0)
        rng.uniform(-2.0 ** -25, 2.0 ** -25, m // 8),          # below half the smallest subnormal
        rng.normal(0, 2.0 ** -14, m // 8),                     # across the normal / subnormal boundary
        rng.normal(0, 1e-2, m // 4)]).astype(np.float32)
    values = rng.permutation(values)
    got = _f16_atomic(halves, index, values)
    target = (halves[index].astype(np.float64) + values.astype(np.float16).astype(np.float64)).astype(np.float16)
    assert np.array_equal(got[index].view(np.uint16), target.view(np.uint16)), \
        f"target halves differ at {np.nonzero(got[index].view(np.uint16) != target.view(np.uint16))[0][:8]}"
    other = index ^ 1
    assert np.array_equal(got[other].view(np.uint16), halves[other].view(np.uint16)), "the other half changed"
    assert (np.abs(target[(target != 0)]) < 2.0 ** -14).mean() > 0.3  # the case is mostly subnormal sums


def test_f16_atomic_same_half_exact_in_any_order(gpu):
    """Many lanes adding subnormal multiples of 2^-24 to the same halves:
    below 2^-13 every such sum is a multiple of 2^-24 that f16 holds exactly,
    so the result is the exact total whatever the order, unless the atomic
    unit flushed subnormals."""
    print("case: vt_debug_f16_atomic_add, 64 halves x 96 adds", flush=True)
    rng = np.random.default_rng(4)
    nh, per = 64, 96
    k = rng.integers(0, 8, (nh, per))
    k[:, 0] = 1
    index = np.repeat(np.arange(nh), per)
    order = rng.permutation(index.size)
    values = (k.reshape(-1) * 2.0 ** -24).astype(np.float32)
    got = _f16_atomic(np.zeros(nh, np.float16), index[order], values[order])
    want = (k.sum(axis=1) * 2.0 ** -24)
    assert (want < 2.0 ** -13).all()
    assert np.array_equal(got.astype(np.float64), want), f"{got[:6]} vs {want[:6]}"


def test_backward_in_forward_cost_order(gpu):
    """The backward of a forward over the same rays tensor launches its tiles
    by the forward's recorded costs (18 x longest walk + most face records per
    tile): per-ray walk statistics equal the screen-order backward's, and the
    gradients agree with it and with the oracle."""
    s, rays, start, thr = _case("hf8")
    scene_t = _scene_tensors(s, gpu, False)
    rd, sd = H.to_dev(rays, gpu), H.to_dev(start, gpu)
    g = H.to_dev(np.random.default_rng(8).normal(size=rays.shape[:-1] + (4,)).astype(np.float32), gpu)
    saved = _C.TRAIN_TILE_ORDER
    try:
        res = {}
        for flag in (False, True):
            _C.TRAIN_TILE_ORDER = flag
            _C._TRAIN_SCHEDULES.clear()
            fst = native.new_stats(rays.size // 6, gpu)
            out = _C.trace_vorotracing_fwd(*scene_t, rd, sd, None, thr, 1024, False, stats=fst)
            st = native.new_stats(rays.size // 6, gpu)
            grads = _C.trace_vorotracing_bwd(*scene_t, rd, sd, out[0], g, None, None, None, None, 0.0, out[5], None,
                                             out[6], out[7], out[8], thr, 1024, stats=st)
            torch.cuda.synchronize()
            res[flag] = (out[0].cpu().numpy(), [x.cpu().numpy() for x in grads[:4]], H.stats_np(st), H.stats_np(fst))
        sch = next(iter(_C._TRAIN_SCHEDULES.values()))
    finally:
        _C.TRAIN_TILE_ORDER = saved
    assert np.array_equal(res[True][0], res[False][0])
    H.assert_stats_equal(res[True][2], res[False][2])
    for a, b, name in zip(res[True][1], res[False][1], ("points", "diffuse", "specular", "density")):
        H.assert_grad_close(a, b, name)
    # the order the backward used: tiles by the forward's costs (2-wide strips)
    Hh, W = rays.shape[:2]
    TX, TY = (W + 7) // 8, (Hh + 7) // 8
    yy, xx = np.meshgrid(np.arange(Hh), np.arange(W), indexing="ij")
    tx, ty = xx // 8, yy // 8
    sp = tx // 2
    wd = np.where((sp + 1) * 2 <= TX, 2, TX - sp * 2)
    tile_of = (sp * 2 * TY + ty * wd + (tx - sp * 2)).reshape(-1)
    fs = res[True][3]
    nmax, fmax = np.zeros(TX * TY, np.int64), np.zeros(TX * TY, np.int64)
    np.maximum.at(nmax, tile_of, fs["n"].astype(np.int64))
    np.maximum.at(fmax, tile_of, fs["faces"].astype(np.int64))
    cost = 18 * nmax + fmax
    assert np.array_equal(sch.cost.cpu().numpy().astype(np.int64), cost)
    assert np.array_equal(sch.order[:TX * TY].cpu().numpy().astype(np.int64),
                          np.argsort(H.tile_order_keys(cost), kind="stable"))
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        rays, start, weight_threshold=thr)
    want = core.trace_bwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                          rays, start, fw["rgba"], g.cpu().numpy(), distortion=fw["distortion"],
                          W_total=fw["W_total"], S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    for a, key in zip(res[True][1], ("points_grad", "diffuse_grad", "specular_grad", "density_grad")):
        H.assert_grad_close(a, want[key], key)


@pytest.mark.parametrize("split", ["all", "part"])
def test_forward_split_tiles(gpu, split):
    """A forward of rays rendered again launches by the previous forward's
    tile costs and runs the tiles above the split share as two half-waves
    (TRAIN_SPLIT_WAVES forces splits on a small frame): every per-ray output
    and walk statistic equals the screen-order forward's, bit for bit; the
    split count follows from the previous costs; a whole tile records 18 x
    its longest walk + its most face records, a split tile the larger of its
    halves' (rows 0-3, rows 4-7) such costs (an atomic max into cleared
    costs)."""
    s, rays, start, thr = _case("hf8")
    scene_t = _scene_tensors(s, gpu, False)
    rd, sd = H.to_dev(rays, gpu), H.to_dev(start, gpu)
    q = H.to_dev(np.tile(np.array([0.7, 0.2], np.float32), rays.shape[:-1] + (1,)), gpu)
    Hh, W = rays.shape[:2]
    TX, TY = (W + 7) // 8, (Hh + 7) // 8
    tiles = TX * TY
    waves = (1 << 23) if split == "all" else tiles
    saved = (_C.TRAIN_TILE_ORDER, _C.TRAIN_SPLIT_WAVES)
    try:
        _C.TRAIN_TILE_ORDER = True
        _C.TRAIN_SPLIT_WAVES = waves
        _C._TRAIN_SCHEDULES.clear()
        runs = []
        for _ in range(3):  # screen order, then twice by the recorded costs
            st = native.new_stats(rays.size // 6, gpu)
            out = _C.trace_vorotracing_fwd(*scene_t, rd, sd, q, thr, 1024, False, stats=st)
            sch = next(iter(_C._TRAIN_SCHEDULES.values()))
            torch.cuda.synchronize()
            runs.append(([None if x is None else x.cpu().numpy() for x in out], H.stats_np(st),
                         sch.cost.cpu().numpy().astype(np.int64), sch.order.cpu().numpy().astype(np.int64)))
    finally:
        _C.TRAIN_TILE_ORDER, _C.TRAIN_SPLIT_WAVES = saved
        _C._TRAIN_SCHEDULES.clear()
    assert int(_lib.load().vt_train_fwd_resident_waves()) >= tiles  # the launch had a wave for every half
    # per-tile and per-half maxima of the walk statistics (2-wide tile strips)
    yy, xx = np.meshgrid(np.arange(Hh), np.arange(W), indexing="ij")
    tx, ty = xx // 8, yy // 8
    sp = tx // 2
    wd = np.where((sp + 1) * 2 <= TX, 2, TX - sp * 2)
    tile_of = (sp * 2 * TY + ty * wd + (tx - sp * 2)).reshape(-1)
    half_of = ((yy % 8) // 4).reshape(-1)
    st0 = runs[0][1]
    def cost_of(sel):
        nmax, fmax = np.zeros(tiles, np.int64), np.zeros(tiles, np.int64)
        np.maximum.at(nmax, tile_of[sel], st0["n"][sel].astype(np.int64))
        np.maximum.at(fmax, tile_of[sel], st0["faces"][sel].astype(np.int64))
        return 18 * nmax + fmax
    whole = cost_of(np.ones(tile_of.size, bool))
    halves = np.maximum(cost_of(half_of == 0), cost_of(half_of == 1))
    assert np.array_equal(runs[0][2], whole)
    for i in (1, 2):
        out, stats, cost, order = runs[i]
        for a, b in zip(out, runs[0][0]):
            assert (a is None and b is None) or np.array_equal(a, b)
        H.assert_stats_equal(stats, runs[0][1])
        prev = runs[i - 1][2]
        k = int(np.sum(5 * prev * waves > 4 * prev.sum()))
        assert 0 < k == order[tiles], (k, order[tiles])
        assert np.array_equal(order[:tiles], np.argsort(H.tile_order_keys(prev), kind="stable"))
        split_set = np.zeros(tiles, bool)
        split_set[order[:k]] = True
        assert np.array_equal(cost, np.where(split_set, halves, whole)), i


@pytest.mark.parametrize("split,f16", [("all", False), ("all", True), ("part", False)])
def test_backward_split_tiles(gpu, split, f16):
    """The backward's costliest tiles run as two half-waves (vt_tile_order's
    split count; TRAIN_SPLIT_WAVES forces it on a small frame: every tile,
    or the tiles above 4/5 of the mean cost): per-ray walk statistics equal
    the screen-order backward's, and the gradients agree with it and with
    the oracle."""
    s, rays, start, thr = _case("hf8")
    scene_t = _scene_tensors(s, gpu, f16)
    rd, sd = H.to_dev(rays, gpu), H.to_dev(start, gpu)
    gn = np.random.default_rng(12).normal(size=rays.shape[:-1] + (4,)).astype(np.float16 if f16 else np.float32)
    g = H.to_dev(gn, gpu)
    Hh, W = rays.shape[:2]
    tiles = ((W + 7) // 8) * ((Hh + 7) // 8)
    saved = (_C.TRAIN_TILE_ORDER, _C.TRAIN_SPLIT_WAVES)
    try:
        res = {}
        for flag in (False, True):
            _C.TRAIN_TILE_ORDER = flag
            _C.TRAIN_SPLIT_WAVES = (1 << 23) if split == "all" else tiles
            _C._TRAIN_SCHEDULES.clear()
            out = _C.trace_vorotracing_fwd(*scene_t, rd, sd, None, thr, 1024, False)
            st = native.new_stats(rays.size // 6, gpu)
            grads = _C.trace_vorotracing_bwd(*scene_t, rd, sd, out[0], g, None, None, None, None, 0.0, out[5], None,
                                             out[6], out[7], out[8], thr, 1024, stats=st)
            torch.cuda.synchronize()
            res[flag] = ([x.float().cpu().numpy() for x in grads[:4]], H.stats_np(st))
        sch = next(iter(_C._TRAIN_SCHEDULES.values()))
    finally:
        _C.TRAIN_TILE_ORDER, _C.TRAIN_SPLIT_WAVES = saved
        _C._TRAIN_SCHEDULES.clear()
    cost = sch.cost.cpu().numpy().astype(np.int64)
    k = int(sch.order[tiles].item())
    want_k = tiles if split == "all" else int(np.sum(5 * cost * tiles > 4 * cost.sum()))
    assert k == want_k and 0 < k, (k, want_k)
    resident = int(_lib.load().vt_train_bwd_resident_waves())
    assert resident >= tiles  # every counted tile was split (the launch adds min(tiles, resident) waves)
    H.assert_stats_equal(res[True][1], res[False][1])
    adt = np.float16 if f16 else np.float32
    fw = core.trace_fwd(s.points, s.diffuse.astype(adt), s.specular.astype(adt), s.diff_res, s.spec_res, s.density,
                        s.adjacency, s.offsets, rays, start, weight_threshold=thr)
    want = core.trace_bwd(s.points, s.diffuse.astype(adt), s.specular.astype(adt), s.diff_res, s.spec_res,
                          s.density, s.adjacency, s.offsets, rays, start, fw["rgba"], gn, distortion=fw["distortion"],
                          W_total=fw["W_total"], S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    keys = ("points_grad", "diffuse_grad", "specular_grad", "density_grad")
    if not f16:
        for a, b, key in zip(res[True][0], res[False][0], keys):
            H.assert_grad_close(a, b, key)
            H.assert_grad_close(a, want[key], key)
    else:
        # half-precision texture sums: each run within the accumulation bound
        # of the oracle's absolute sums and add counts
        A, K = H.f16_train_sums(s, rays, start, thr, fw, gn)
        for flag in (False, True):
            for a, key in zip(res[flag][0], keys):
                if key in ("points_grad", "density_grad"):
                    H.assert_grad_close(a, want[key], key, abs_sum=A[key])
                else:
                    H.assert_f16_sum_close(a, want[key], A[key], K[key], key)


@pytest.mark.parametrize("split", ["all", "part"])
def test_backward_split_waves_ray_perm(gpu, split):
    """A flat batch in a ray_perm lane order: the forward records the cost of
    each wave of 64 consecutive ray_perm entries, and the backward of the same
    rays and permutation tensors launches those waves by cost, the ones above
    the split share (forced by TRAIN_SPLIT_WAVES) as two half-waves of 32
    entries.  Per-ray walk statistics equal the batch-order backward's and
    the gradients agree with it and with the oracle."""
    s, rays, start, thr = _case("hf8")
    flat = rays.reshape(-1, 6)
    shuffle = np.random.default_rng(13).permutation(flat.shape[0])
    flat, fstart = np.ascontiguousarray(flat[shuffle]), np.ascontiguousarray(start.reshape(-1)[shuffle])
    scene_t = _scene_tensors(s, gpu, False)
    rd, sd = H.to_dev(flat, gpu), H.to_dev(fstart, gpu)
    perm = _C.ray_order(rd, sd, s.points.shape[0])
    gn = np.random.default_rng(14).normal(size=(flat.shape[0], 4)).astype(np.float32)
    g = H.to_dev(gn, gpu)
    tiles = (flat.shape[0] + 63) // 64
    saved = (_C.TRAIN_TILE_ORDER, _C.TRAIN_SPLIT_WAVES)
    try:
        res = {}
        for flag in (False, True):
            _C.TRAIN_TILE_ORDER = flag
            _C.TRAIN_SPLIT_WAVES = (1 << 23) if split == "all" else tiles
            _C._TRAIN_SCHEDULES.clear()
            out = _C.trace_vorotracing_fwd(*scene_t, rd, sd, None, thr, 1024, False, ray_perm=perm)
            st = native.new_stats(flat.shape[0], gpu)
            grads = _C.trace_vorotracing_bwd(*scene_t, rd, sd, out[0], g, None, None, None, None, 0.0, out[5], None,
                                             out[6], out[7], out[8], thr, 1024, stats=st, ray_perm=perm)
            torch.cuda.synchronize()
            res[flag] = ([x.cpu().numpy() for x in grads[:4]], H.stats_np(st))
        sch = next(iter(_C._TRAIN_SCHEDULES.values()))
        cost = sch.cost.cpu().numpy().astype(np.int64)
        k = int(sch.order[tiles].item())
    finally:
        _C.TRAIN_TILE_ORDER, _C.TRAIN_SPLIT_WAVES = saved
        _C._TRAIN_SCHEDULES.clear()
    assert sch.tiles == tiles
    want_k = tiles if split == "all" else int(np.sum(5 * cost * tiles > 4 * cost.sum()))
    assert 0 < k == want_k, (k, want_k)
    H.assert_stats_equal(res[True][1], res[False][1])
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        flat, fstart, weight_threshold=thr)
    want = core.trace_bwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency,
                          s.offsets, flat, fstart, fw["rgba"], gn, distortion=fw["distortion"], W_total=fw["W_total"],
                          S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    for a, b, key in zip(res[True][0], res[False][0], ("points_grad", "diffuse_grad", "specular_grad", "density_grad")):
        H.assert_grad_close(a, b, key)
        H.assert_grad_close(a, want[key], key)


def test_model_sort_morton(gpu):
    """VoroTracing.sort_morton: the model's rows and CSR in Morton order (the
    oracle's morton_reorder permutation), the LBVH rebuilt, gradients and
    Adam's moments permuted with them; the same rays then render the same
    image bit for bit and get the permuted gradients."""
    from oracle import host_ops

    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    rays = H.to_dev(camera.orbit_rays(4, 96, 72), gpu)
    g = torch.from_numpy(np.random.default_rng(9).normal(size=(72, 96, 4)).astype(np.float32)).to(gpu)
    opt = torch.optim.Adam(model.parameters(), lr=0.0)  # moments only: the parameters stay as they are
    rgba, *_ = model(rays)
    (rgba * g).sum().backward()
    opt.step()
    rgba0 = rgba.detach().clone()
    grads0 = [p.grad.clone() for p in (model.primal_points, model.density, model.att_diffuse, model.att_specular)]
    params0 = [p.detach().clone() for p in (model.primal_points, model.density, model.att_diffuse,
                                            model.att_specular)]
    moments0 = [opt.state[p]["exp_avg"].clone() for p in (model.primal_points, model.att_diffuse)]
    perm = model.sort_morton(opt)
    torch.cuda.synchronize()
    want_perm, _, want_adj, want_off, _ = host_ops.morton_reorder(params0[0].cpu().numpy(), s.adjacency, s.offsets)
    pi = perm.view(torch.int32).long()
    assert np.array_equal(pi.cpu().numpy(), want_perm)
    assert np.array_equal(model.point_adjacency_offsets.cpu().numpy().astype(np.int64), want_off.astype(np.int64))
    m = int(want_off[-1])
    assert np.array_equal(model.point_adjacency.cpu().numpy()[:m].astype(np.int64), want_adj[:m].astype(np.int64))
    for p, p0, g0 in zip((model.primal_points, model.density, model.att_diffuse, model.att_specular), params0,
                         grads0):
        assert torch.equal(p.detach(), p0[pi]) and torch.equal(p.grad, g0[pi])
    for p, m0 in zip((model.primal_points, model.att_diffuse), moments0):
        assert torch.equal(opt.state[p]["exp_avg"], m0[pi])
    model.zero_grad(set_to_none=True)
    rgba1, *_ = model(rays)
    (rgba1 * g).sum().backward()
    torch.cuda.synchronize()
    assert torch.equal(rgba1.detach(), rgba0)
    for p, g0, name in zip((model.primal_points, model.att_diffuse), (grads0[0], grads0[2]), ("points", "diffuse")):
        H.assert_grad_close(p.grad.cpu().numpy(), g0[pi].cpu().numpy(), name)
    # the start cells come from the rebuilt LBVH
    sites = types.SimpleNamespace(points=model.primal_points.detach().cpu().numpy())
    assert np.array_equal(model.get_starting_point(rays).cpu().numpy(), H.start_for(sites, rays.cpu().numpy()))
