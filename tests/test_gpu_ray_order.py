"""Lane order of flat training batches: vt_ray_order and the ray_perm
extension of the training entries.

The reference traces ray i on thread i (tracing_octmap.cu:175-179, :264-268)
and its default trainer batches random pixels of random images
(datasets.py:185-222, trainer.py:52).  Tracing such a batch in another lane
order must leave every per-ray output bit-identical and change the atomically
summed outputs only by the order of their additions, so both are checked
against the CPU oracle under a random permutation, under ray_order's
permutation, and through the default ("auto") path at a batch size that
triggers it.
"""
import functools

import numpy as np
import pytest
import torch

from oracle import core
from tests import helpers as H
from vorotracing_amd import _C, camera

pytestmark = pytest.mark.gpu

DIR_BITS = 7  # octahedral grid bits per axis of vt_ray_order's direction key


def _spread(q):
    q = q.astype(np.uint64)
    out = np.zeros_like(q)
    for b in range(DIR_BITS):
        out |= ((q >> np.uint64(b)) & np.uint64(1)) << np.uint64(2 * b)
    return out


def _grid_directions(rng, n):
    """Directions at octahedral grid-cell centres, with random lengths, so
    that the cell of each is known exactly (half a cell from any edge)."""
    cells = 1 << DIR_BITS
    qu = rng.integers(0, cells, n)
    qv = rng.integers(0, cells, n)
    u = (2 * qu + 1) / cells - 1.0
    v = (2 * qv + 1) / cells - 1.0
    z = 1.0 - np.abs(u) - np.abs(v)
    x = np.where(z < 0, (1.0 - np.abs(v)) * np.sign(u), u)
    y = np.where(z < 0, (1.0 - np.abs(u)) * np.sign(v), v)
    d = np.stack([x, y, z], -1) * rng.uniform(0.5, 2.0, (n, 1))
    return d.astype(np.float32), _spread(qu) | (_spread(qv) << np.uint64(1))


@pytest.mark.parametrize("num_points,num_rays,distinct", [
    (1000, 70001, 7),        # cell and direction in one 24-bit key
    (300000, 70001, 0),      # 19 + 14 bits: direction pass, then a stable cell pass
    (300000, 5000, 11),
    (1, 3000, 1),            # a single site: direction only
    (1000, 1, 1),
])
def test_ray_order_is_stable_cell_then_direction(gpu, num_points, num_rays, distinct):
    rng = np.random.default_rng(num_points + num_rays)
    d, dkey = _grid_directions(rng, num_rays)
    o = rng.normal(size=(num_rays, 3)).astype(np.float32)
    rays = np.ascontiguousarray(np.concatenate([o, d], 1), np.float32)
    if distinct:
        cams = rng.integers(0, num_points, distinct)
        start = cams[rng.integers(0, distinct, num_rays)].astype(np.uint32)
    else:
        start = rng.integers(0, num_points, num_rays).astype(np.uint32)
    perm = _C.ray_order(H.to_dev(rays, gpu), H.to_dev(start, gpu), num_points)
    torch.cuda.synchronize()
    got = perm.view(torch.int32).cpu().numpy().astype(np.int64)
    idx = np.arange(num_rays)
    want = np.lexsort((idx, dkey, start.astype(np.uint64)))
    assert np.array_equal(np.sort(got), idx)
    assert np.array_equal(got, want)


def _multi_camera_batch(rng, num_rays, cams=8, w=64, h=48):
    """Random pixels of random orbit cameras, as the reference's sample_batch draws them."""
    allr = np.stack([camera.orbit_rays(k, w, h, radius=3.0) for k in range(cams)])
    img = rng.integers(0, cams, num_rays)
    y = rng.integers(0, h, num_rays)
    x = rng.integers(0, w, num_rays)
    return np.ascontiguousarray(allr[img, y, x], np.float32)


def _check_fwd(got, want):
    rgba, depth, depth_idx, contrib, n, dist, W, S, tf = got
    assert np.array_equal(n.cpu().numpy(), want["n"])
    assert np.array_equal(rgba.cpu().numpy(), want["rgba"])
    assert np.array_equal(depth_idx.cpu().numpy(), want["depth_idx"])
    for t, key in ((depth, "depth"), (dist, "distortion"), (W, "W_total"), (S, "S_total"), (tf, "t_far")):
        assert np.array_equal(t.cpu().numpy().view(np.uint32), want[key].view(np.uint32)), key
    c = contrib.cpu().numpy().reshape(-1)
    wc = want["contribution"].reshape(-1)
    assert np.abs(c - wc).max() <= 1e-5 * max(np.abs(wc).max(), 1e-30)


def _parity(gpu, num_rays, order):
    s = H.small_random(1500, seed=5, R=8, Rs=4)
    thr = 0.001
    rng = np.random.default_rng(11)
    rays = _multi_camera_batch(rng, num_rays)
    start = H.start_for(s, rays)
    q = np.tile(np.array([0.8, 0.3], np.float32), (num_rays, 1))
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                        rays, start, depth_quantiles=q, weight_threshold=thr, return_contribution=True)
    g = rng.normal(size=(num_rays, 4)).astype(np.float32)
    dg = rng.normal(size=(num_rays, 2)).astype(np.float32) * 0.1
    distg = rng.uniform(0, 1, size=(num_rays, 1)).astype(np.float32)
    rerr = rng.uniform(0, 1, size=(num_rays,)).astype(np.float32)
    bwd = functools.partial(core.trace_bwd, s.points, s.diffuse, s.specular, s.diff_res, s.spec_res, s.density,
                            s.adjacency, s.offsets, rays, start, fw["rgba"], g, depth_quantiles=q,
                            depth_idx=fw["depth_idx"], depth_grad=dg, ray_error=rerr, contribution_alpha_grad=0.25,
                            distortion=fw["distortion"], distortion_grad=distg, W_total=fw["W_total"],
                            S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr)
    want = bwd()
    with core.abs_sums():
        cond = bwd()
    dev = lambda a: H.to_dev(a, gpu)  # noqa: E731
    scene = (dev(s.points), dev(s.diffuse), dev(s.specular), dev(s.density), dev(s.adjacency), dev(s.offsets))
    r, st = dev(rays), dev(start)
    if order == "random":
        perm = torch.from_numpy(rng.permutation(num_rays).astype(np.int32)).to(gpu)
    elif order == "ray_order":
        perm = _C.ray_order(r, st, s.points.shape[0])
    else:
        perm = "auto"
        assert _C.default_ray_perm(r, st, s.points.shape[0]) is not None
    got = _C.trace_vorotracing_fwd(*scene, r, st, dev(q), thr, 1024, True, ray_perm=perm)
    torch.cuda.synchronize()
    _check_fwd(got, fw)
    pg, dgd, sgd, deng, _, perr = _C.trace_vorotracing_bwd(
        *scene, r, st, dev(fw["rgba"]), dev(g), dev(q), dev(fw["depth_idx"]), dev(dg), dev(rerr), 0.25,
        dev(fw["distortion"]), dev(distg), dev(fw["W_total"]), dev(fw["S_total"]), dev(fw["t_far"]), thr, 1024,
        ray_perm=perm)
    torch.cuda.synchronize()
    for got, key in ((pg, "points_grad"), (deng, "density_grad"), (dgd, "diffuse_grad"), (sgd, "specular_grad"),
                     (perr, "point_error")):
        H.assert_grad_close(got.cpu().numpy(), want[key], key, abs_sum=cond[key])
    assert np.abs(want["points_grad"]).max() > 0 and np.abs(want["diffuse_grad"]).max() > 0


@pytest.mark.parametrize("order", ["random", "ray_order"])
def test_permuted_lanes_match_oracle(gpu, order):
    _parity(gpu, 4000, order)


def test_default_order_of_large_flat_batch_matches_oracle(gpu):
    _parity(gpu, _C.ORDER_MIN_RAYS + 4465, "auto")


def test_default_order_choice(gpu):
    s = H.small_random(300, seed=2)
    rays = camera.pinhole_rays(320, 240, eye=(0.2, -3.0, 0.1))
    start = H.to_dev(H.start_for(s, rays), gpu)
    r = H.to_dev(rays, gpu)
    n = s.points.shape[0]
    assert _C.default_ray_perm(r, start, n) is None  # image-shaped: 8x8 screen tiles
    flat = r.reshape(-1, 6)
    assert flat.shape[0] >= _C.ORDER_MIN_RAYS
    perm = _C.default_ray_perm(flat, start.reshape(-1), n)
    assert perm is not None
    assert np.array_equal(np.sort(perm.view(torch.int32).cpu().numpy()), np.arange(flat.shape[0]))
    assert _C.default_ray_perm(flat[:1000], start.reshape(-1)[:1000], n) is None  # small batch: batch order
    with pytest.raises(RuntimeError, match="ray_perm must"):
        _C.trace_vorotracing_fwd(*[H.to_dev(a, gpu) for a in (s.points, s.diffuse, s.specular, s.density,
                                                              s.adjacency, s.offsets)],
                                 flat, start.reshape(-1), None, 0.001, 1024, False, ray_perm=perm[:10])


def _aa_rays(w, h, eye):
    """Five rays per pixel, shaped (H, W, 5, 6) as the reference's full
    antialiasing makes them: the pixel's ray and four perturbed directions."""
    base = camera.pinhole_rays(w, h, eye=eye)
    r = np.repeat(base[:, :, None, :], 5, axis=2)
    r[:, :, 1:, 3:] += np.random.default_rng(4).normal(scale=2e-3, size=(h, w, 4, 3)).astype(np.float32)
    return np.ascontiguousarray(r, np.float32)


def test_antialiased_ray_shapes_equal_flat(gpu):
    """(H, W, 5, 6) rays are traced as H x 5W images, in training and in
    inference; every per-ray output equals the flat batch's in batch order,
    bit for bit."""
    from vorotracing_amd.infer import VoroTracingInfer
    from vorotracing_amd.model import VoroTracing

    s = H.small_random(1500, seed=5, R=8, Rs=4)
    rays = _aa_rays(48, 40, (0.3, -3.2, 0.4))
    assert _C._image_dims(torch.from_numpy(rays)) == (40, 240)
    start = H.start_for(s, rays)
    dev = lambda a: H.to_dev(a, gpu)  # noqa: E731
    scene = (dev(s.points), dev(s.diffuse), dev(s.specular), dev(s.density), dev(s.adjacency), dev(s.offsets))
    img = _C.trace_vorotracing_fwd(*scene, dev(rays), dev(start), None, 0.001, 1024, False)
    flat = _C.trace_vorotracing_fwd(*scene, dev(rays.reshape(-1, 6)), dev(start.reshape(-1)), None, 0.001, 1024,
                                    False, ray_perm=None)
    torch.cuda.synchronize()
    compared = 0
    for a, b in zip(img, flat):
        if a is None:
            assert b is None
            continue
        assert torch.equal(a.reshape(-1).view(torch.int32), b.reshape(-1).view(torch.int32))
        compared += 1
    assert compared == 6  # rgba, n, distortion, W_total, S_total, t_far

    inf = VoroTracingInfer(VoroTracing.from_scene(s, device=gpu), sort_morton=True, quantize="fp16")
    r = dev(rays)
    got = inf.render(r, weight_threshold=0.001, cell_skip_threshold=1e-3)
    want = inf.render(r.reshape(-1, 6), weight_threshold=0.001, cell_skip_threshold=1e-3)
    torch.cuda.synchronize()
    assert tuple(got.shape) == (40, 48, 5, 4)
    assert torch.equal(got.reshape(-1, 4).view(torch.int16), want.view(torch.int16))
    assert (got[..., 3] > 0).any()
