"""GPU parity of the inference path against the CPU oracle.

The walk's arithmetic restates the oracle's op for op, so visited-cell
sequences (hash + counters), per-ray statistics and the alpha channel must be
bit-identical.  The colour of a shaded cell uses hardware approximations
(rsq, rcp, exp2), so RGB must lie within one fp16 ulp of the oracle's value,
inside the north star's 2e-3 for fp16/q8 (tests.helpers.assert_infer_rgba).
"""
import numpy as np
import pytest
import torch

from oracle import core, host_ops
from tests import helpers as H
from vorotracing_amd import _C, _lib, camera, native
from vorotracing_amd.infer import VoroTracingInfer
from vorotracing_amd.model import VoroTracing

pytestmark = pytest.mark.gpu


def test_exit_order_probe(gpu):
    """exit_before, the walk's division-free face order, against IEEE float32
    quotients on random rows, near-ties, exact ties, subnormal and overflowing
    quotients and NaN.  Rows whose best quotient rounds to -inf are outside its
    contract (the walk redoes that search with IEEE quotients; see
    test_exit_face_probe)."""
    from tests import exit_rows as X
    a = X.order_cases(np.random.default_rng(7))
    with np.errstate(all="ignore"):
        keep = ~np.isneginf(a[:, 2] / a[:, 3])
    a = np.ascontiguousarray(a[keep])
    got = native.math_probe(5, torch.from_numpy(a).to(gpu)).cpu().numpy()
    want = X.order_want(a)
    bad = np.nonzero(got.astype(bool) != want)[0]
    assert bad.size == 0, f"{bad.size} of {len(a)} rows differ, first {a[bad[:3]]}"


def test_exit_face_probe(gpu):
    """The walk's exit-face search (chunked reads, exit_before, the IEEE redo
    for quotients rounding to -inf) equals the oracle's plain search: face
    index and t1 bits, on random cells, duplicated faces and the -inf cases."""
    from tests import exit_rows as X
    rows = X.face_rows(np.random.default_rng(11))
    got = native.math_probe(6, torch.from_numpy(rows).to(gpu)).cpu().numpy()
    want = core.exit_face_rows(rows)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} of {len(rows)} rows differ, first {bad[:5]}: {got[bad[:5]]} vs {want[bad[:5]]}"
    assert (want[-13:-1, 1] == np.float32(-np.inf).view(np.uint32)).all()


def test_packed_exit_face_probe(gpu):
    """The packed walk's search over a reordered chunk (exact ties noted and
    settled by original index in the IEEE redo, the -inf redo) picks the face
    the oracle's plain search over the original list picks: original index and
    t1 bits, with the faces sorted by z, reversed and shuffled."""
    from tests import exit_rows as X
    rows = X.face_rows(np.random.default_rng(11))
    packed = X.packed_rows(rows, np.random.default_rng(12))
    got = native.math_probe(7, torch.from_numpy(packed).to(gpu)).cpu().numpy()
    want = core.exit_face_rows(rows)
    bad = np.nonzero((got != want).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} of {len(rows)} rows differ, first {bad[:5]}: {got[bad[:5]]} vs {want[bad[:5]]}"


def _dev_scene(s, dev):
    d4, s4 = H.f16_maps(s)
    return dict(points=H.to_dev(s.points, dev), diffuse4=H.to_dev(d4, dev), specular4=H.to_dev(s4, dev),
                density=H.to_dev(s.density.reshape(-1), dev), adjacency=H.to_dev(s.adjacency, dev),
                offsets=H.to_dev(s.offsets, dev))


def test_math_probe_exp_log_f16(gpu):
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.uniform(-110, 90, 1 << 20).astype(np.float32),
                        (rng.standard_normal(1 << 18) * 3).astype(np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 88.7, 88.73, -87.3, -103.9, -104.0, np.inf, -np.inf,
                                  np.nan], np.float32)])
    xd = torch.from_numpy(x).to(gpu)
    got = native.math_probe(0, xd).cpu().numpy().view(np.float32)
    want = core.expf(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    xl = np.abs(x)
    xl = np.concatenate([xl, rng.uniform(1e-38, 1e-30, 4096).astype(np.float32), np.float32([1e-44, 1.0, 2.0])])
    got = native.math_probe(1, torch.from_numpy(xl).to(gpu)).cpu().numpy().view(np.float32)
    want = core.logf(xl)
    ok = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert ok.all()
    xf = np.concatenate([x, rng.uniform(-70000, 70000, 1 << 16).astype(np.float32),
                         (rng.standard_normal(1 << 16) * 1e-5).astype(np.float32)])
    got = native.math_probe(2, torch.from_numpy(xf).to(gpu)).cpu().numpy().astype(np.uint16)
    want = core.f32_to_f16_bits(xf)
    nan = np.isnan(xf)
    assert np.array_equal(got[~nan], want[~nan])


@pytest.mark.parametrize("which", ["c1", "mini_c3"])
def test_prefetch_bit_exact(gpu, which):
    s = H.c1_scene() if which == "c1" else H.mini_heightfield()
    d = _dev_scene(s, gpu)
    got = _C.trace_vorotracing_prefetch_adj(d["points"], d["adjacency"], d["offsets"]).cpu().numpy()
    want = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    m = s.num_faces
    assert got.shape == (s.adjacency.shape[0] + 32, 4)
    assert np.array_equal(got[:m].view(np.uint16), want[:m].view(np.uint16))
    assert not got[m:].view(np.uint16).any()  # padding rows zero-filled


def test_prefetch_bit_exact_synthetic_csr(gpu):
    """Face lists of every length the prefetch's two owner paths meet: blocks
    of 256 cells whose entries fit its owner table, a block of 256 cells with
    70 faces each (17,920 entries, past the table: binary search), a
    900-face list, empty lists and a partial last block."""
    rng = np.random.default_rng(12)
    n = 1100
    deg = rng.integers(0, 30, n)
    deg[256:512] = 70
    deg[600] = 900
    deg[700:710] = 0
    offsets = np.concatenate([[0], np.cumsum(deg)]).astype(np.uint32)
    m = int(offsets[-1])
    adjacency = np.concatenate([rng.integers(0, n, m), np.zeros(32)]).astype(np.uint32)
    points = rng.normal(size=(n, 3)).astype(np.float32)
    got = _C.trace_vorotracing_prefetch_adj(H.to_dev(points, gpu), H.to_dev(adjacency, gpu),
                                            H.to_dev(offsets, gpu)).cpu().numpy()
    want = core.prefetch_adj(points, adjacency, offsets)
    assert np.array_equal(got[:m].view(np.uint16), want[:m].view(np.uint16))
    assert not got[m:].view(np.uint16).any()


def _c1_rays(W=128, Hh=128):
    return camera.pinhole_rays(W, Hh, eye=(0.0, -4.0, 0.0))


@pytest.mark.parametrize("mode", ["linear", "perm48", "perm88", "tiled88"])
def test_infer_f16_c1_parity(gpu, mode):
    s = H.c1_scene()
    rays = _c1_rays()
    start = H.start_for(s, rays)
    d = _dev_scene(s, gpu)
    adj = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    d4, s4 = H.f16_maps(s)
    want, wst, _ = core.trace_infer_f16(s.points, d4, s4, 4, 4, s.density, s.adjacency, s.offsets,
                                        adj.cpu().numpy(), rays, start, weight_threshold=0.01, want_stats=True)
    rays_d = H.to_dev(rays, gpu)
    start_d = H.to_dev(start, gpu)
    stats = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
    perm = None
    tiled = None
    if mode == "perm48":
        perm = H.to_dev(host_ops.tile_perm(128, 128, 4, 8).view(np.uint32), gpu)
    elif mode == "perm88":
        perm = H.to_dev(host_ops.tile_perm(128, 128, 8, 8).view(np.uint32), gpu)
    elif mode == "tiled88":
        tiled = (8, 8)
    got = native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"],
                           adj, rays_d, start_d, ray_perm=perm, weight_threshold=0.01, stats=stats, tiled=tiled)
    torch.cuda.synchronize()
    H.assert_stats_equal(H.stats_np(stats), wst)
    g = got.cpu().numpy()
    H.assert_infer_rgba(g, want)


def test_infer_f16_reference_surface(gpu):
    """_C.trace_vorotracing_infer with the reference arguments (int32 tile perm)."""
    s = H.c1_scene()
    rays = _c1_rays(96, 64)
    start = H.start_for(s, rays)
    d = _dev_scene(s, gpu)
    adj = _C.trace_vorotracing_prefetch_adj(d["points"], d["adjacency"], d["offsets"])
    perm = H.to_dev(host_ops.tile_perm(64, 96, 4, 8), gpu)
    got = _C.trace_vorotracing_infer(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                                     d["offsets"], H.to_dev(rays, gpu), H.to_dev(start, gpu), adj, perm, 0.01, 1024,
                                     0.0)
    d4, s4 = H.f16_maps(s)
    want, _, _ = core.trace_infer_f16(s.points, d4, s4, 4, 4, s.density, s.adjacency, s.offsets,
                                      adj.cpu().numpy(), rays, start, weight_threshold=0.01)
    assert got.shape == (64, 96, 4) and got.dtype == torch.float16
    H.assert_infer_rgba(got, want)
    # the image above went through the in-kernel tiles; the same rays as a flat
    # batch go through the linear kernel, lane t on ray perm[t]
    flat = _C.trace_vorotracing_infer(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                                      d["offsets"], H.to_dev(rays.reshape(-1, 6), gpu),
                                      H.to_dev(start.reshape(-1), gpu), adj, perm, 0.01, 1024, 0.0)
    torch.cuda.synchronize()
    assert np.array_equal(flat.cpu().numpy().view(np.uint16).reshape(got.shape),
                          got.cpu().numpy().view(np.uint16))
    # a lane order that repeats a ray (so leaves another untraced) is refused
    dup = perm.clone()
    dup[7] = dup[8]
    for r_, s_ in ((rays, start), (rays.reshape(-1, 6), start.reshape(-1))):
        with pytest.raises(RuntimeError, match="ray_perm must be a permutation"):
            _C.trace_vorotracing_infer(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                                       d["offsets"], H.to_dev(r_, gpu), H.to_dev(s_, gpu), adj, dup, 0.01, 1024, 0.0)


@pytest.mark.parametrize("R", [4, 8])
def test_infer_f16_mini_c3_skip(gpu, R):
    """Config-3 distribution (heightfield, skip gate 1e-3, thr 0.01) on two orbit poses."""
    s = H.mini_heightfield() if R == 4 else H.small_random(3000, seed=11, R=8, Rs=4)
    d = _dev_scene(s, gpu)
    adj = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    d4, s4 = H.f16_maps(s)
    adj_np = adj.cpu().numpy()
    for k in (0, 9):
        rays = camera.orbit_rays(k, 160, 120)
        start = H.start_for(s, rays)
        want, wst, _ = core.trace_infer_f16(s.points, d4, s4, s.diff_res, s.spec_res, s.density, s.adjacency,
                                            s.offsets, adj_np, rays, start, weight_threshold=0.01,
                                            cell_skip_threshold=1e-3, want_stats=True)
        stats = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
        got = native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                               d["offsets"], adj, H.to_dev(rays, gpu), H.to_dev(start, gpu), weight_threshold=0.01,
                               cell_skip_threshold=1e-3, stats=stats, tiled=(8, 8))
        torch.cuda.synchronize()
        H.assert_stats_equal(H.stats_np(stats), wst)
        H.assert_infer_rgba(got, want)


@pytest.mark.parametrize("quantize", ["fp16", "q8"])
@pytest.mark.parametrize("lanes", ["linear", "tiled"])
def test_infer_8x8_maps(gpu, quantize, lanes):
    """The reference's only compiled map resolution, 8x8 diffuse and 8x8
    specular (tracing_octmap.cu:27-28, vorotracing.py:12-18), on the mini
    height field: fp16 and q8 through the _C entries, in ray order (no lane
    order) and in in-kernel tiles (a lane order given), two orbit poses,
    skip gate 1e-3.  Walk statistics and alpha bit for bit, RGB to one fp16
    ulp of the oracle."""
    s = H.mini_heightfield_r8()
    assert s.diff_res == 8 and s.spec_res == 8
    d = _dev_scene(s, gpu)
    adj = _C.trace_vorotracing_prefetch_adj(d["points"], d["adjacency"], d["offsets"])
    adj_np = adj.cpu().numpy()
    if quantize == "q8":
        dq, dsc, dof = host_ops.quantize_u8(s.diffuse, True)
        sq, ssc, sof = host_ops.quantize_u8(s.specular, True)
    else:
        d4, s4 = H.f16_maps(s)
    for k in (0, 9):
        print(f"case: {quantize} {lanes} 8x8 maps, pose {k}", flush=True)
        rays = camera.orbit_rays(k, 160, 120)
        start = H.start_for(s, rays)
        rd, sd = H.to_dev(rays, gpu), H.to_dev(start, gpu)
        perm = torch.arange(rays.size // 6, dtype=torch.int32, device=gpu) if lanes == "tiled" else None
        if quantize == "q8":
            want, _ = core.trace_infer_q8(s.points, dq, sq, 8, 8, dsc, dof, ssc, sof, s.density, s.adjacency,
                                          s.offsets, adj_np, rays, start, weight_threshold=0.01,
                                          cell_skip_threshold=1e-3, want_stats=True)
            got = _C.trace_vorotracing_infer_q8(d["points"], H.to_dev(dq, gpu), H.to_dev(sq, gpu), d["density"],
                                                d["adjacency"], d["offsets"], rd, sd, adj, dsc, dof, ssc, sof, 0.01,
                                                1024, 1e-3, ray_perm_in=perm)
        else:
            want, _, _ = core.trace_infer_f16(s.points, d4, s4, 8, 8, s.density, s.adjacency, s.offsets, adj_np,
                                              rays, start, weight_threshold=0.01, cell_skip_threshold=1e-3,
                                              want_stats=True)
            empty = torch.empty(0, dtype=torch.int32, device=gpu)
            got = _C.trace_vorotracing_infer(d["points"], d["diffuse4"], d["specular4"], d["density"],
                                             d["adjacency"], d["offsets"], rd, sd, adj,
                                             empty if perm is None else perm, 0.01, 1024, 1e-3)
        torch.cuda.synchronize()
        H.assert_infer_rgba(got, want)
        assert (want[..., 3] > 0).mean() > 0.3  # the camera sees the surface
    # the walk record of the last pose, through the tiled kernel with statistics
    st = native.new_stats(rays.size // 6, gpu)
    if quantize == "fp16":
        want, wst, _ = core.trace_infer_f16(s.points, d4, s4, 8, 8, s.density, s.adjacency, s.offsets, adj_np, rays,
                                            start, weight_threshold=0.01, cell_skip_threshold=1e-3, want_stats=True)
        native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"], adj,
                         rd, sd, weight_threshold=0.01, cell_skip_threshold=1e-3, stats=st,
                         tiled=(8, 8) if lanes == "tiled" else None)
        torch.cuda.synchronize()
        H.assert_stats_equal(H.stats_np(st), wst)


@pytest.mark.parametrize("per_channel", [False, True])
def test_infer_q8_parity(gpu, per_channel):
    s = H.mini_heightfield()
    dq, dsc, dof = host_ops.quantize_u8(s.diffuse, per_channel)
    sq, ssc, sof = host_ops.quantize_u8(s.specular, per_channel)
    d = _dev_scene(s, gpu)
    adj = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    rays = camera.orbit_rays(3, 128, 96)
    start = H.start_for(s, rays)
    want, wst = core.trace_infer_q8(s.points, dq, sq, 4, 4, dsc, dof, ssc, sof, s.density, s.adjacency, s.offsets,
                                    adj.cpu().numpy(), rays, start, weight_threshold=0.01, cell_skip_threshold=1e-3,
                                    want_stats=True)
    stats = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
    got = native.infer_q8(d["points"], H.to_dev(dq, gpu), H.to_dev(sq, gpu),
                          (np.broadcast_to(dsc, 3), np.broadcast_to(dof, 3), np.broadcast_to(ssc, 3),
                           np.broadcast_to(sof, 3)),
                          d["density"], d["adjacency"], d["offsets"], adj, H.to_dev(rays, gpu),
                          H.to_dev(start, gpu), weight_threshold=0.01, cell_skip_threshold=1e-3, stats=stats)
    torch.cuda.synchronize()
    H.assert_stats_equal(H.stats_np(stats), wst)
    H.assert_infer_rgba(got, want)
    # _C with a lane order over these image-shaped rays renders them in
    # in-kernel tiles: the same image bit for bit
    perm = torch.from_numpy(np.random.default_rng(2).permutation(rays.size // 6).astype(np.int32)).to(gpu)
    viac = _C.trace_vorotracing_infer_q8(d["points"], H.to_dev(dq, gpu),
                                        H.to_dev(sq, gpu), d["density"], d["adjacency"], d["offsets"],
                                        H.to_dev(rays, gpu), H.to_dev(start, gpu), adj, dsc, dof, ssc, sof, 0.01, 1024,
                                        1e-3, ray_perm_in=perm)
    torch.cuda.synchronize()
    assert np.array_equal(viac.cpu().numpy().view(np.uint16), got.cpu().numpy().view(np.uint16))


def test_infer_errors_reference_messages(gpu):
    s = H.c1_scene()
    d = _dev_scene(s, gpu)
    rays = H.to_dev(_c1_rays(8, 8), gpu)
    start = torch.zeros((8, 8), dtype=torch.uint32, device=gpu)
    adj = _C.trace_vorotracing_prefetch_adj(d["points"], d["adjacency"], d["offsets"])
    empty = torch.empty(0, dtype=torch.int32, device=gpu)
    args = [d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"], rays, start, adj,
            empty, 0.01, 1024, 0.0]
    bad = list(args)
    bad[1] = d["diffuse4"].float()
    with pytest.raises(RuntimeError, match="inference kernel requires float16 diffuse"):
        _C.trace_vorotracing_infer(*bad)
    bad = list(args)
    bad[7] = start.to(torch.int32)
    with pytest.raises(RuntimeError, match="start_point must have uint32 dtype"):
        _C.trace_vorotracing_infer(*bad)
    bad = list(args)
    bad[5] = d["offsets"][:-1]
    with pytest.raises(RuntimeError, match="point_adjacency_offsets must have num_points"):
        _C.trace_vorotracing_infer(*bad)
    bad = list(args)
    bad[0] = d["points"].double()
    with pytest.raises(RuntimeError, match="points had dtype Double, expected float32"):
        _C.trace_vorotracing_infer(*bad)
    # empty ray batch is a no-op (kernel_utils.cuh:31-34)
    out = _C.trace_vorotracing_infer(*(args[:6] + [rays[:0], start[:0], adj, empty, 0.01, 1024, 0.0]))
    assert out.shape == (0, 8, 4)


def test_infer_f16_origins_on_sites_ragged(gpu):
    """Rays that start exactly on their start site: the first probe point is the
    site itself, so the probe direction falls back to the ray direction (probe_dir's
    |hit - site| <= 1e-8 branch).  1000 rays, not a multiple of the wave size,
    with no skip gate so that every integrated cell is shaded."""
    s = H.small_random(600, seed=5)
    rng = np.random.default_rng(8)
    n = 1000
    idx = rng.integers(0, s.points.shape[0], n)
    d = rng.normal(size=(n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    rays = np.concatenate([s.points[idx], d.astype(np.float32)], axis=1).astype(np.float32).reshape(1, n, 6)
    start = idx.astype(np.uint32).reshape(1, n)
    dd = _dev_scene(s, gpu)
    adj = native.prefetch(dd["points"], dd["adjacency"], dd["offsets"])
    d4, s4 = H.f16_maps(s)
    want, wst, _ = core.trace_infer_f16(s.points, d4, s4, 4, 4, s.density, s.adjacency, s.offsets,
                                        adj.cpu().numpy(), rays, start, weight_threshold=0.01, want_stats=True)
    stats = native.new_stats(n, gpu)
    got = native.infer_f16(dd["points"], dd["diffuse4"], dd["specular4"], dd["density"], dd["adjacency"],
                           dd["offsets"], adj, H.to_dev(rays, gpu), H.to_dev(start, gpu), weight_threshold=0.01,
                           stats=stats)
    torch.cuda.synchronize()
    H.assert_stats_equal(H.stats_np(stats), wst)
    assert (H.stats_np(stats)["integrated"] > 0).all()
    H.assert_infer_rgba(got, want)


@pytest.mark.parametrize("cap", [1, 5, 13])
def test_infer_f16_step_cap(gpu, cap):
    """max_intersections ends walks mid-scene (tracing_octmap.cu:58-62): the step
    count, the cells integrated up to the cap, and the shades still queued when a
    walk stops all match the oracle, tiled and linear."""
    s = H.mini_heightfield()
    d = _dev_scene(s, gpu)
    adj = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    d4, s4 = H.f16_maps(s)
    rays = camera.orbit_rays(5, 96, 64)
    start = H.start_for(s, rays)
    want, wst, _ = core.trace_infer_f16(s.points, d4, s4, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                                        adj.cpu().numpy(), rays, start, weight_threshold=0.01, max_intersections=cap,
                                        cell_skip_threshold=1e-3, want_stats=True)
    assert (wst["n"] == cap + 1).any()  # some walks do reach the cap
    for tiled in (None, (8, 8)):
        stats = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
        got = native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                               d["offsets"], adj, H.to_dev(rays, gpu), H.to_dev(start, gpu), weight_threshold=0.01,
                               max_intersections=cap, cell_skip_threshold=1e-3, stats=stats, tiled=tiled)
        torch.cuda.synchronize()
        H.assert_stats_equal(H.stats_np(stats), wst)
        H.assert_infer_rgba(got, want)


def test_infer_empty_batch(gpu):
    """A batch of zero rays launches nothing and returns an empty image."""
    s = H.c1_scene()
    d = _dev_scene(s, gpu)
    adj = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    rays = torch.empty((0, 6), dtype=torch.float32, device=gpu)
    start = H.to_dev(np.zeros(0, np.uint32), gpu)
    got = native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"],
                           adj, rays, start, weight_threshold=0.01)
    torch.cuda.synchronize()
    assert tuple(got.shape) == (0, 4)


@pytest.mark.parametrize("in_flight", [2, 3])
def test_render_frames_overlapped_equal_serial(gpu, in_flight):
    """Frames rendered with several in flight on side streams (start-cell
    queries included, each with its own scan workspace) equal serial renders
    bit for bit."""
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    inf = VoroTracingInfer(model, sort_morton=True, quantize="fp16")
    frames = [H.to_dev(camera.orbit_rays(k, 96, 64), gpu) for k in range(9)]
    want = [inf.render(r, weight_threshold=0.01, cell_skip_threshold=1e-3) for r in frames]
    got = inf.render_frames(frames, in_flight=in_flight, weight_threshold=0.01, cell_skip_threshold=1e-3)
    torch.cuda.synchronize()
    assert len(got) == len(want)
    for a, b in zip(got, want):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def _strip_tiles(Hh, W, strip=4):
    """Tile index (4-wide vertical strips of 8x8 tiles, row by row inside a
    strip, as the tiled kernels number them) of every pixel of an H x W image."""
    TX, TY = (W + 7) // 8, (Hh + 7) // 8
    yy, xx = np.meshgrid(np.arange(Hh), np.arange(W), indexing="ij")
    tx, ty = xx // 8, yy // 8
    s = tx // strip
    w = np.where((s + 1) * strip <= TX, strip, TX - s * strip)
    return (s * strip * TY + ty * w + (tx - s * strip)).reshape(-1), TX * TY


def test_tile_order_sorts_by_cost(gpu):
    """vt_tile_order: tiles by decreasing cost bucket (4 per octave), equal
    buckets in tile order, against numpy's stable argsort of the bucket key."""
    rng = np.random.default_rng(3)
    for tiles, hi in ((1, 10), (777, 50), (16095, 40000), (70000, 1 << 20), (5000, 1 << 32)):
        cost = rng.integers(0, hi, tiles).astype(np.uint32)
        cost[: tiles // 3] = cost[0]  # many ties
        cost[-3:] = (0, 1, 0xFFFFFFFF)[: min(3, tiles)]
        c = H.to_dev(cost, gpu)
        order = torch.empty(tiles + 1, dtype=torch.uint32, device=gpu)
        ws = torch.empty(int(_lib.load().vt_tile_order_workspace_size(tiles)), dtype=torch.uint8, device=gpu)
        want = np.argsort(H.tile_order_keys(cost), kind="stable")
        for split_waves in (0, 1, 4096, tiles, (1 << 24) - 1):
            _lib.call("vt_tile_order", c.data_ptr(), tiles, split_waves, order.data_ptr(), ws.data_ptr(),
                      torch.cuda.current_stream().cuda_stream)
            torch.cuda.synchronize()
            got = order.cpu().numpy().astype(np.int64)
            assert np.array_equal(got[:tiles], want), tiles
            # the split count: tiles costing more than 4/5 of the mean share of one of split_waves waves
            c64, total = cost.astype(np.int64), int(cost.astype(np.int64).sum())
            k = int(np.sum(5 * c64 * split_waves > 4 * total)) if split_waves else 0
            assert got[tiles] == k, (tiles, split_waves)


def test_tile_order_and_costs_of_a_render(gpu):
    """A tiled render launched in any tile order gives the same image bit for
    bit; the tile costs it writes are 18 x the longest walk + the most face
    records of a ray of the tile (from the same launch's walk statistics)."""
    s = H.mini_heightfield()
    d = _dev_scene(s, gpu)
    adj = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    Hh, W = 100, 132
    rays = H.to_dev(camera.orbit_rays(3, W, Hh), gpu)
    start = H.to_dev(H.start_for(s, rays.cpu().numpy()), gpu)
    tile_of, tiles = _strip_tiles(Hh, W)
    args = (d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"], adj, rays, start)
    ref = native.infer_f16(*args, weight_threshold=0.01, cell_skip_threshold=1e-3, tiled=(8, 8))
    sch = native.TileSchedule(tiles, gpu)
    st = native.new_stats(Hh * W, gpu)
    got = native.infer_f16(*args, weight_threshold=0.01, cell_skip_threshold=1e-3, tiled=(8, 8), schedule=sch,
                           stats=st)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    stn = H.stats_np(st)
    nmax, fmax = np.zeros(tiles, np.int64), np.zeros(tiles, np.int64)
    np.maximum.at(nmax, tile_of, stn["n"].astype(np.int64))
    np.maximum.at(fmax, tile_of, stn["faces"].astype(np.int64))
    assert np.array_equal(sch.cost.cpu().numpy().astype(np.int64), 18 * nmax + fmax)
    # the same rays again: launched by decreasing cost, same image
    for _ in range(2):
        again = native.infer_f16(*args, weight_threshold=0.01, cell_skip_threshold=1e-3, tiled=(8, 8), schedule=sch)
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), ref.view(torch.int16))
    want = np.argsort(H.tile_order_keys(18 * nmax + fmax), kind="stable")
    assert np.array_equal(sch.order[:tiles].cpu().numpy().astype(np.int64), want)
    # a random launch order through the C ABI: same image
    order = H.to_dev(np.random.default_rng(5).permutation(tiles).astype(np.uint32), gpu)
    out = torch.empty_like(ref)
    _lib.call("vt_trace_infer_f16_tiled", d["points"].data_ptr(), d["diffuse4"].data_ptr(), d["specular4"].data_ptr(),
              4, 4, d["density"].data_ptr(), d["adjacency"].data_ptr(), d["offsets"].data_ptr(), s.num_points,
              adj.data_ptr(), rays.data_ptr(), 1, Hh, W, 8, 8, start.data_ptr(), 0, 0.01, 1024, 1e-3, out.data_ptr(),
              order.data_ptr(), None, None, None, None, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
