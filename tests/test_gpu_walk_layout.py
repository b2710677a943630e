"""The packed walk layout (vt_walk_layout, native.WalkLayout): its arrays
against a numpy construction, its limits, and renders through it, which must
be the renders of the reference's arrays bit for bit (walk statistics,
alpha and RGB), and within the oracle's bounds."""
import numpy as np
import pytest
import torch

from oracle import core, host_ops
from tests import helpers as H
from vorotracing_amd import _C, camera, native

pytestmark = pytest.mark.gpu


def _dev(s, gpu):
    d4, s4 = H.f16_maps(s)
    d = dict(points=H.to_dev(s.points, gpu), diffuse4=H.to_dev(d4, gpu), specular4=H.to_dev(s4, gpu),
             density=H.to_dev(s.density.reshape(-1), gpu), adjacency=H.to_dev(s.adjacency, gpu),
             offsets=H.to_dev(s.offsets, gpu))
    d["adj"] = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    return d


def _check_arrays(wl, points, density, adjacency, offsets, adj_diff):
    first, chunks, links, heads, cells, orig = H.walk_layout_np(points, density, adjacency, offsets, adj_diff,
                                                                face_order=wl.face_order)
    assert wl.num_chunks == int(first[len(offsets) - 1])
    assert np.array_equal(wl.chunks.cpu().numpy().view(np.uint32)[:wl.num_chunks], chunks)
    assert np.array_equal(wl.links.cpu().numpy().view(np.uint32)[:8 * wl.num_chunks], links)
    assert np.array_equal(wl.heads.cpu().numpy().view(np.uint32), heads)
    assert np.array_equal(wl.cells.cpu().numpy().view(np.uint32), cells.view(np.uint32))
    assert np.array_equal(wl.orig.cpu().numpy().view(np.uint16)[:8 * wl.num_chunks], orig)


def test_walk_layout_arrays(gpu):
    """The GPU build against numpy on a height-field scene (lists of every
    length it has, several chunks each)."""
    s = H.mini_heightfield()
    d = _dev(s, gpu)
    for order in (0, 1, 2, 3):
        wl = native.WalkLayout.build(d["points"], d["density"], d["adjacency"], d["offsets"], d["adj"],
                                     face_order=order)
        assert wl is not None
        torch.cuda.synchronize()
        _check_arrays(wl, s.points, s.density, s.adjacency, s.offsets, d["adj"].cpu().numpy())
    nf = np.diff(s.offsets)
    assert nf.min() < 8 < nf.max() and (nf % 8 == 0).any()


def test_walk_layout_ragged_lists(gpu):
    """Empty lists, lists of exactly 8 and 16 faces, one face past a chunk,
    and the largest list the layout holds (255 chunks); one face more and
    build() declines."""
    rng = np.random.default_rng(4)
    for top in (2040, 2041):
        nf = np.array([0, 8, 9, 16, 1, 0, 17, top, 3], np.int64)
        n = nf.size
        offsets = np.concatenate([[0], np.cumsum(nf)]).astype(np.uint32)
        F = int(offsets[-1])
        adjacency = np.concatenate([rng.integers(0, n, F), np.zeros(32, np.int64)]).astype(np.uint32)
        points = rng.standard_normal((n, 3)).astype(np.float32)
        density = rng.random(n).astype(np.float32)
        pd, ad, od = H.to_dev(points, gpu), H.to_dev(adjacency, gpu), H.to_dev(offsets, gpu)
        adj = native.prefetch(pd, ad, od)
        wl = native.WalkLayout.build(pd, H.to_dev(density, gpu), ad, od, adj)
        if top > 8 * native.WalkLayout.MAX_CHUNKS_PER_CELL:
            assert wl is None
            continue
        torch.cuda.synchronize()
        _check_arrays(wl, points, density, adjacency, offsets, adj.cpu().numpy())


@pytest.mark.parametrize("scene", ["heightfield", "random_r8"])
def test_packed_walk_parity(gpu, scene):
    """Tiled fp16 renders through the layout: statistics (visited cells,
    face counts, step counts) equal to the oracle's, RGBA within its bound,
    and every output bit equal to the renders of the reference's arrays."""
    s = H.mini_heightfield() if scene == "heightfield" else H.small_random(3000, seed=11, R=8, Rs=4)
    d = _dev(s, gpu)
    wl = native.WalkLayout.build(d["points"], d["density"], d["adjacency"], d["offsets"], d["adj"])
    d4, s4 = H.f16_maps(s)
    adj_np = d["adj"].cpu().numpy()
    for k in (0, 9):
        print(f"case: packed walk, {scene}, pose {k}", flush=True)
        rays = camera.orbit_rays(k, 160, 120)
        start = H.start_for(s, rays)
        want, wst, _ = core.trace_infer_f16(s.points, d4, s4, s.diff_res, s.spec_res, s.density, s.adjacency,
                                            s.offsets, adj_np, rays, start, weight_threshold=0.01,
                                            cell_skip_threshold=1e-3, want_stats=True)
        outs = []
        for walk in (wl, None):
            st = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
            got = native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                                   d["offsets"], d["adj"], H.to_dev(rays, gpu), H.to_dev(start, gpu),
                                   weight_threshold=0.01, cell_skip_threshold=1e-3, stats=st, tiled=(8, 8),
                                   walk=walk)
            torch.cuda.synchronize()
            H.assert_stats_equal(H.stats_np(st), wst)
            H.assert_infer_rgba(got, want)
            outs.append(got)
            # without statistics (the kernel the renders run)
            outs.append(native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"],
                                         d["offsets"], d["adj"], H.to_dev(rays, gpu), H.to_dev(start, gpu),
                                         weight_threshold=0.01, cell_skip_threshold=1e-3, tiled=(8, 8), walk=walk))
        torch.cuda.synchronize()
        for o in outs[1:]:
            assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))


def test_packed_walk_q8_drop_in(gpu):
    """The q8 drop-in with a lane order walks the layout (cached per scene):
    the same image bit for bit as with the layout off, within the oracle's
    bound, and the cache rebuilds when the density changes in place."""
    s = H.mini_heightfield()
    d = _dev(s, gpu)
    dq, dsc, dof = host_ops.quantize_u8(s.diffuse, True)
    sq, ssc, sof = host_ops.quantize_u8(s.specular, True)
    dqd, sqd = H.to_dev(dq, gpu), H.to_dev(sq, gpu)
    rays = camera.orbit_rays(5, 160, 120)
    start = H.start_for(s, rays)
    rd, sd = H.to_dev(rays, gpu), H.to_dev(start, gpu)
    perm = torch.arange(rays.size // 6, dtype=torch.int32, device=gpu)

    def render():
        return _C.trace_vorotracing_infer_q8(d["points"], dqd, sqd, d["density"], d["adjacency"], d["offsets"], rd,
                                             sd, d["adj"], dsc, dof, ssc, sof, 0.01, 1024, 1e-3, ray_perm_in=perm)

    want, _ = core.trace_infer_q8(s.points, dq, sq, 4, 4, dsc, dof, ssc, sof, s.density, s.adjacency, s.offsets,
                                  d["adj"].cpu().numpy(), rays, start, weight_threshold=0.01,
                                  cell_skip_threshold=1e-3, want_stats=True)
    try:
        _C.DROP_IN_WALK = False
        general = render()
        _C.DROP_IN_WALK = True
        packed = render()
        torch.cuda.synchronize()
        assert torch.equal(packed.view(torch.int16), general.view(torch.int16))
        H.assert_infer_rgba(packed, want)
        # an in-place change of the density: the cached layout must not be reused
        d["density"].mul_(0.5)
        _C.DROP_IN_WALK = False
        general = render()
        _C.DROP_IN_WALK = True
        packed = render()
        torch.cuda.synchronize()
        assert torch.equal(packed.view(torch.int16), general.view(torch.int16))
    finally:
        _C.DROP_IN_WALK = True


@pytest.mark.parametrize("quantize", ["fp16", "q8"])
def test_render_start_cell_forms(gpu, quantize):
    """render() with start cells given per ray, per camera ((B, 1, 1)), as one
    cell for all rays, or not given: the tiled kernels read a per-camera array
    through rays_per_start, and every form renders the same image bit for bit
    (one camera, and a batch of two cameras)."""
    from vorotracing_amd.infer import VoroTracingInfer
    from vorotracing_amd.model import VoroTracing
    s = H.mini_heightfield()
    inf = VoroTracingInfer(VoroTracing.from_scene(s, device=gpu), sort_morton=True, quantize=quantize)
    kw = dict(weight_threshold=0.01, cell_skip_threshold=1e-3)
    one = H.to_dev(camera.orbit_rays(2, 96, 72), gpu)
    two = torch.stack([one, H.to_dev(camera.orbit_rays(11, 96, 72), gpu)])
    for rays in (one, two):
        print(f"case: {quantize} start cell forms, rays {tuple(rays.shape)}", flush=True)
        per_ray = inf.get_starting_point(rays)
        cells = inf.start_cells(rays)
        assert cells.numel() == (rays.shape[0] if rays.dim() == 4 else 1)
        assert inf._rays_per_start(rays, cells) > 0
        outs = [inf.render(rays, **kw), inf.render(rays, start_point=per_ray, **kw),
                inf.render(rays, start_point=cells, **kw)]
        if rays.dim() == 3:
            outs.append(inf.render(rays, start_point=cells.reshape(1), **kw))
        # the same cells through the general path (no lane order): the reference's per-ray form
        outs.append(inf.render(rays, start_point=per_ray, use_warp_perm=False, **kw))
        torch.cuda.synchronize()
        for o in outs[1:]:
            assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
