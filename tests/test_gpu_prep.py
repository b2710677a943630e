"""GPU parity of the preparation kernels (LBVH start cell, Morton reorder,
tile permutation, q8 quantisation, fp16 padding) against the numpy / C
restatements, and the render invariances they must preserve."""
import numpy as np
import pytest
import torch

from oracle import core, host_ops
from tests import helpers as H
from vorotracing_amd import _C, _lib, camera, native, ops
from vorotracing_amd.infer import VoroTracingInfer
from vorotracing_amd.model import VoroTracing

pytestmark = pytest.mark.gpu


# up to 2^26 query-site pairs the query scans all sites, above it walks the tree
@pytest.mark.parametrize("n,nq,seed", [(1, 5, 0), (2, 50, 1), (37, 300, 2), (300000, 3, 5), (5000, 20000, 3),
                                       (200000, 50000, 4)])
def test_bvh_exact_nearest(gpu, n, nq, seed):
    rng = np.random.default_rng(seed)
    pts = rng.normal(size=(n, 3)).astype(np.float32) * rng.uniform(0.1, 3.0, size=(1, 3)).astype(np.float32)
    q = np.concatenate([rng.normal(size=(nq, 3)).astype(np.float32) * 2,
                        pts[rng.integers(0, n, size=min(nq, 64))]])  # queries exactly on sites
    bvh = ops.NNBVH()
    pd = H.to_dev(pts, gpu)
    bvh.build(pd)
    got = bvh.query(pd, H.to_dev(q, gpu)).cpu().numpy()
    want = host_ops.nearest_site(pts, q)
    assert got.dtype == np.int32
    assert np.array_equal(got, want)


def test_start_cells_runs(gpu):
    """NNBVH.start_cells (vt_start_cells): the nearest site of every ray's
    origin, against the brute-force oracle, for runs of equal consecutive
    origins of lengths 300, 1, 2 and 7, an origin repeated after other runs,
    origins on duplicated sites (lowest index), and 600,000 single-ray runs
    (more than one pass of the grid-stride query: 2048 blocks x 256 lanes);
    the batch's shape is kept, and an empty batch gives an empty result."""
    rng = np.random.default_rng(21)
    n = 5000
    pts = rng.normal(size=(n, 3)).astype(np.float32)
    pts[20] = pts[30] = pts[10]  # duplicates: the lowest index wins
    a, b, c = rng.normal(size=(3, 3)).astype(np.float32)
    runs = [(a, 300), (b, 1), (c, 2), (pts[30], 7), (a, 5), (b, 3)]
    o = np.concatenate([np.repeat(x[None], k, 0) for x, k in runs] +
                       [rng.normal(size=(600000, 3)).astype(np.float32) * 1.5])
    rays = np.concatenate([o, rng.normal(size=o.shape).astype(np.float32)], axis=1)
    assert rays.shape[0] % 256 != 0
    bvh = ops.NNBVH()
    pd = H.to_dev(pts, gpu)
    bvh.build(pd)
    got = bvh.start_cells(pd, H.to_dev(rays, gpu))
    assert got.dtype == torch.uint32 and tuple(got.shape) == (rays.shape[0],)
    want = host_ops.nearest_site(pts, o)
    assert np.array_equal(got.cpu().numpy().astype(np.int64), want.astype(np.int64))
    assert int(got[300 + 1 + 2].item()) == 10
    img = H.to_dev(rays[:12 * 20].reshape(12, 20, 6), gpu)
    assert np.array_equal(bvh.start_cells(pd, img).cpu().numpy().astype(np.int64).reshape(-1), want[:240])
    assert bvh.start_cells(pd, torch.empty((0, 6), device=gpu)).numel() == 0


def test_bvh_ties_lowest_index(gpu):
    """Duplicate sites and equidistant sites: lowest index wins (brute force rule)."""
    base = np.array([[0, 0, 0], [1, 0, 0], [0, 1, 0], [1, 1, 0]], np.float32)
    pts = np.concatenate([base, base, base[::-1]]).astype(np.float32)  # triplicates
    q = np.array([[0.5, 0.5, 0], [0, 0, 0], [1, 1, 0], [0.5, 0, 0], [2, 2, 2]], np.float32)
    bvh = ops.NNBVH()
    pd = H.to_dev(pts, gpu)
    bvh.build(pd)
    got = bvh.query(pd, H.to_dev(q, gpu)).cpu().numpy()
    assert np.array_equal(got, host_ops.nearest_site(pts, q))
    assert got.tolist() == [0, 0, 3, 0, 3]
    # rebuild on a different, larger set reuses the handle
    pts2 = np.random.default_rng(9).uniform(-1, 1, size=(3000, 3)).astype(np.float32)
    bvh.build(H.to_dev(pts2, gpu))
    got = bvh.query(H.to_dev(pts2, gpu), H.to_dev(q, gpu)).cpu().numpy()
    assert np.array_equal(got, host_ops.nearest_site(pts2, q))
    assert np.array_equal(_C.nearest_neighbor_bvh(H.to_dev(pts2, gpu), H.to_dev(q, gpu)).cpu().numpy(), got)


@pytest.mark.parametrize("path", ["scan", "tree"])
def test_bvh_ties_across_strides_and_blocks(gpu, path):
    """Duplicate and equidistant sites at index spacings of a lane, a wave, a
    block and a whole scan stride (300,000 sites): the lowest index wins on the
    all-sites scan (28 queries) and on the tree walk (the same queries repeated
    past 2^26 query-site pairs)."""
    pts, q = H.nn_tie_set()
    if path == "tree":
        q = np.tile(q, (10, 1))
        assert q.shape[0] * pts.shape[0] > (1 << 26)
    else:
        assert q.shape[0] * pts.shape[0] <= (1 << 26)
    bvh = ops.NNBVH()
    pd = H.to_dev(pts, gpu)
    bvh.build(pd)
    got = bvh.query(pd, H.to_dev(q, gpu)).cpu().numpy()
    assert np.array_equal(got, host_ops.nearest_site(pts, q))


@pytest.mark.parametrize("limit", [1, 2, 5])
def test_bvh_stack_overflow_answers_exactly(gpu, limit):
    """A query whose traversal stack would overflow answers by a scan of all
    sites instead of dropping a subtree.  The stack is capped from the host
    (test hook) so the tree walk reaches that path on an ordinary tree."""
    import ctypes as C

    rng = np.random.default_rng(20 + limit)
    pts = rng.normal(size=(20000, 3)).astype(np.float32)
    pts[100:110] = pts[5000]  # duplicates: ties to the lowest index through the fallback too
    q = np.concatenate([rng.normal(size=(700, 3)).astype(np.float32), pts[[5000, 100, 7]]])
    pd, qd = H.to_dev(pts, gpu), H.to_dev(q, gpu)
    h = C.c_void_p()
    _lib.call("vt_bvh_create", C.byref(h))
    try:
        s = torch.cuda.current_stream(gpu).cuda_stream
        _lib.call("vt_bvh_build", h, pd.data_ptr(), pts.shape[0], s)
        _lib.call("vt_bvh_debug_stack_limit", h, limit, 1)
        out = torch.full((q.shape[0],), -7, dtype=torch.int32, device=gpu)
        _lib.call("vt_bvh_query", h, pd.data_ptr(), pts.shape[0], qd.data_ptr(), q.shape[0], out.data_ptr(), s)
        torch.cuda.synchronize()
        with pytest.raises(_lib.VTError, match="above the compiled 64"):
            _lib.call("vt_bvh_debug_stack_limit", h, 65, 1)
    finally:
        _lib.load().vt_bvh_destroy(h)
    assert np.array_equal(out.cpu().numpy(), host_ops.nearest_site(pts, q))


def test_short_adjacent_diff_rejected(gpu):
    """The walk reads face records 8 at a time past a list end: an adjacent_diff
    shorter than the prefetch layout (adjacency rows + 32) is refused."""
    s = H.small_random()
    pts, adj, off = H.to_dev(s.points, gpu), H.to_dev(s.adjacency, gpu), H.to_dev(s.offsets, gpu)
    ad = _C.trace_vorotracing_prefetch_adj(pts, adj, off)
    assert ad.shape[0] == adj.shape[0] + 32
    d4, s4 = (H.to_dev(m, gpu) for m in H.f16_maps(s))
    rays = H.to_dev(camera.pinhole_rays(8, 8, eye=(0.0, -3.0, 0.2)), gpu)
    sp = torch.zeros(rays.shape[:-1], dtype=torch.uint32, device=gpu)
    dens = H.to_dev(s.density.reshape(-1), gpu)
    empty = torch.empty(0, dtype=torch.int32, device=gpu)
    with pytest.raises(RuntimeError, match="adjacency_size \\+ 32 rows"):
        _C.trace_vorotracing_infer(pts, d4, s4, dens, adj, off, rays, sp, ad[:-1].contiguous(), empty, 0.01, 1024, 0.0)
    _C.trace_vorotracing_infer(pts, d4, s4, dens, adj, off, rays, sp, ad, empty, 0.01, 1024, 0.0)
    torch.cuda.synchronize()


def test_morton_reorder_matches_restatement(gpu):
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    inf = VoroTracingInfer(model, sort_morton=True, quantize="fp16")
    perm, pts, adj, off, _ = host_ops.morton_reorder(s.points, s.adjacency, s.offsets)
    assert np.array_equal(inf.morton_perm.cpu().numpy().astype(np.int64), perm)
    assert np.array_equal(inf.primal_points.cpu().numpy(), pts)
    assert np.array_equal(inf.point_adjacency_offsets.cpu().numpy(), off)
    assert np.array_equal(inf.point_adjacency.cpu().numpy(), adj)
    dens_dev = torch.exp(model.density).detach().cpu().numpy()  # activation as computed on the device
    assert np.array_equal(inf.density.cpu().numpy(), dens_dev[perm])
    d4, _ = H.f16_maps(s)
    assert np.array_equal(inf.diffuse_fp16.cpu().numpy().view(np.uint16), d4[perm].view(np.uint16))


def test_morton_render_invariance(gpu):
    """A Morton-permuted scene renders the bit-identical image (face-list
    order is preserved, so every exit choice is the same)."""
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    a = VoroTracingInfer(model, sort_morton=False)
    b = VoroTracingInfer(model, sort_morton=True)
    rays = H.to_dev(camera.orbit_rays(7, 120, 90), gpu)
    for skip in (0.0, 1e-3):
        ia = a.render(rays, weight_threshold=0.01, cell_skip_threshold=skip)
        ib = b.render(rays, weight_threshold=0.01, cell_skip_threshold=skip)
        torch.cuda.synchronize()
        assert np.array_equal(ia.cpu().numpy().view(np.uint16), ib.cpu().numpy().view(np.uint16))


@pytest.mark.parametrize("Hh,W,TH,TW", [(822, 1237, 8, 8), (822, 1237, 4, 8), (5, 7, 8, 8), (64, 64, 8, 8),
                                        (33, 17, 4, 8)])
def test_tile_perm(gpu, Hh, W, TH, TW):
    perm = torch.empty(Hh * W, dtype=torch.int32, device=gpu)
    _lib.call("vt_tile_perm", Hh, W, TH, TW, perm.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert np.array_equal(perm.cpu().numpy(), host_ops.tile_perm(Hh, W, TH, TW))


@pytest.mark.parametrize("per_channel", [False, True])
def test_quantize_and_pad(gpu, per_channel):
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    inf = VoroTracingInfer(model, sort_morton=False, quantize="q8", per_channel_q8=per_channel)
    q, sc, of = host_ops.quantize_u8(s.diffuse, per_channel)
    assert np.array_equal(inf.diffuse_q8.cpu().numpy(), q)
    assert np.allclose(np.float32(inf.diff_scale), sc, rtol=0, atol=0)
    assert np.allclose(np.float32(inf.diff_offset), of, rtol=0, atol=0)
    # values landing exactly on k + 0.5 steps take the even code (torch.round)
    x, want = H.quant_ties(per_channel)
    qt, sct, oft = inf._quantize_to_uint8(H.to_dev(x, gpu), per_channel)
    assert np.all(np.asarray(sct, np.float32) == np.float32(1.0))
    assert np.array_equal(qt.cpu().numpy(), want)
    f = VoroTracingInfer(model, sort_morton=False, quantize="fp16")
    d4, s4 = H.f16_maps(s)
    assert np.array_equal(f.diffuse_fp16.cpu().numpy().view(np.uint16), d4.view(np.uint16))
    assert np.array_equal(f.specular_fp16.cpu().numpy().view(np.uint16), s4.view(np.uint16))


def test_render_q8_batch_per_camera_start(gpu):
    """C4 shape at test size: a batch of cameras rendered in one launch with a
    per-camera start cell, equal to rendering each camera alone; q8 walk
    statistics equal the fp16 ones (density is fp32 in both)."""
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    inf = VoroTracingInfer(model, sort_morton=True, quantize="q8")
    inf16 = VoroTracingInfer(model, sort_morton=True, quantize="fp16")
    batch = np.stack([camera.orbit_rays(k, 96, 64) for k in (0, 4, 8)])
    bd = H.to_dev(batch, gpu)
    st = native.new_stats(batch.size // 6, gpu)
    out = inf.render(bd, weight_threshold=0.01, cell_skip_threshold=0.0, stats=st)
    st16 = native.new_stats(batch.size // 6, gpu)
    inf16.render(bd, weight_threshold=0.01, cell_skip_threshold=0.0, stats=st16)
    for i in range(3):
        one = inf.render(bd[i], weight_threshold=0.01, cell_skip_threshold=0.0)
        assert np.array_equal(one.cpu().numpy().view(np.uint16), out[i].cpu().numpy().view(np.uint16))
    a, b = H.stats_np(st), H.stats_np(st16)
    for k in ("n", "visits", "visit_hash", "integrated", "first_cells"):
        assert np.array_equal(a[k], b[k])
    # oracle on the first camera
    r0 = batch[0]
    sp = np.full(r0.shape[:-1], host_ops.nearest_site(inf.primal_points.cpu().numpy(), r0[0, 0, :3])[0], np.uint32)
    want, _ = core.trace_infer_q8(inf.primal_points.cpu().numpy(), inf.diffuse_q8.cpu().numpy(),
                                  inf.specular_q8.cpu().numpy(), 4, 4, inf.diff_scale, inf.diff_offset,
                                  inf.spec_scale, inf.spec_offset, inf.density.reshape(-1).cpu().numpy(),
                                  inf.point_adjacency.cpu().numpy(), inf.point_adjacency_offsets.cpu().numpy(),
                                  inf.adjacent_diff.cpu().numpy(), r0, sp, weight_threshold=0.01)
    H.assert_infer_rgba(out[0].cpu().numpy(), want)
