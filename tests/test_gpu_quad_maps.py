"""Footprint tables of the maps (vt_quad_maps, native.QuadMaps; fp16 and q8):
the tables against a numpy construction through the oracle's octahedral wrap,
and renders that read them, which must equal the renders that read the maps'
texels bit for bit (buffer, camera and drop-in renders, 4x4 and 8x8 maps) and
stay within the oracle's bound."""
import numpy as np
import pytest
import torch

from oracle import core, host_ops
from tests import helpers as H
from vorotracing_amd import _C, _lib, camera, native

pytestmark = pytest.mark.gpu


def _table_np(maps4, R):
    """The footprint table of Half4Texel maps (N, 4 R^2) f16: entry
    (ex, ey) = the texels at (ex - 1, ey - 1), (ex, ey - 1), (ex - 1, ey),
    (ex, ey), each through the oracle's oct_wrap_index."""
    tex = np.ascontiguousarray(maps4).view(np.uint16).reshape(maps4.shape[0], R * R, 4)
    idx = np.array([[core.oct_wrap_index(ex + du - 1, ey + dv - 1, R) for dv in (0, 1) for du in (0, 1)]
                    for ey in range(R + 1) for ex in range(R + 1)], np.int64)
    return tex[:, idx, :].reshape(maps4.shape[0], -1)


def _table_q8_np(maps, R):
    """The q8 table of u8 maps (N, 3 R^2): per entry the four wrapped texels as
    (r, g, b, 0) bytes."""
    tex = np.zeros((maps.shape[0], R * R, 4), np.uint8)
    tex[..., :3] = np.ascontiguousarray(maps).reshape(maps.shape[0], R * R, 3)
    idx = np.array([[core.oct_wrap_index(ex + du - 1, ey + dv - 1, R) for dv in (0, 1) for du in (0, 1)]
                    for ey in range(R + 1) for ex in range(R + 1)], np.int64)
    return tex[:, idx, :].reshape(maps.shape[0], -1)


@pytest.mark.parametrize("R", [4, 8])
def test_quad_tables_q8(gpu, R):
    rng = np.random.default_rng(10 + R)
    n = 555
    maps = rng.integers(0, 256, (n, 3 * R * R), dtype=np.uint8)
    got = native.QuadMaps.table_q8(H.to_dev(maps, gpu))
    torch.cuda.synchronize()
    assert got.shape == (n, 16 * (R + 1) ** 2)
    assert np.array_equal(got.cpu().numpy(), _table_q8_np(maps, R))


@pytest.mark.parametrize("R", [4, 8])
def test_quad_tables(gpu, R):
    """The GPU tables equal the numpy construction for random texel bits
    (every half pattern, NaNs included: the tables copy bits)."""
    rng = np.random.default_rng(R)
    n = 777
    maps = rng.integers(0, 1 << 16, (n, 4 * R * R), dtype=np.uint16).view(np.float16)
    got = native.QuadMaps.table(H.to_dev(maps, gpu))
    torch.cuda.synchronize()
    assert got.shape == (n, 16 * (R + 1) ** 2)
    assert np.array_equal(got.cpu().numpy().view(np.uint16), _table_np(maps, R))


@pytest.mark.parametrize("scene", ["heightfield", "random_r8"])
def test_quad_render_parity(gpu, scene):
    """Tiled fp16 renders reading the tables: within the oracle's bound and
    bit-identical to the renders reading the maps, with the packed walk and
    with the reference's arrays, with and without statistics."""
    s = H.mini_heightfield() if scene == "heightfield" else H.small_random(3000, seed=11, R=8, Rs=8)
    d4, s4 = H.f16_maps(s)
    d = dict(points=H.to_dev(s.points, gpu), diffuse4=H.to_dev(d4, gpu), specular4=H.to_dev(s4, gpu),
             density=H.to_dev(s.density.reshape(-1), gpu), adjacency=H.to_dev(s.adjacency, gpu),
             offsets=H.to_dev(s.offsets, gpu))
    d["adj"] = native.prefetch(d["points"], d["adjacency"], d["offsets"])
    wl = native.WalkLayout.build(d["points"], d["density"], d["adjacency"], d["offsets"], d["adj"])
    qm = native.QuadMaps.build(d["diffuse4"], d["specular4"])
    adj_np = d["adj"].cpu().numpy()
    for k in (0, 9):
        print(f"case: quad maps, {scene}, pose {k}", flush=True)
        rays = camera.orbit_rays(k, 160, 120)
        start = H.start_for(s, rays)
        want, _, _ = core.trace_infer_f16(s.points, d4, s4, s.diff_res, s.spec_res, s.density, s.adjacency,
                                          s.offsets, adj_np, rays, start, weight_threshold=0.01,
                                          cell_skip_threshold=1e-3, want_stats=True)
        outs = []
        for walk in (wl, None):
            for quads in (qm, None):
                for stats in (True, False):
                    st = native.new_stats(rays.shape[0] * rays.shape[1], gpu) if stats else None
                    outs.append(native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"],
                                                 d["adjacency"], d["offsets"], d["adj"], H.to_dev(rays, gpu),
                                                 H.to_dev(start, gpu), weight_threshold=0.01,
                                                 cell_skip_threshold=1e-3, stats=st, tiled=(8, 8), walk=walk,
                                                 quads=quads))
        torch.cuda.synchronize()
        H.assert_infer_rgba(outs[0], want)
        for o in outs[1:]:
            assert torch.equal(o.view(torch.int16), outs[0].view(torch.int16))
    # tables of another scene (fewer cells) or of the other format are refused before any launch
    few = native.QuadMaps.build(d["diffuse4"][:100], d["specular4"][:100])
    with pytest.raises(_lib.VTError, match="quad maps of 100 cells"):
        native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"],
                         d["adj"], H.to_dev(rays, gpu), H.to_dev(start, gpu), tiled=(8, 8), quads=few)
    dq = H.to_dev(host_ops.quantize_u8(s.diffuse, True)[0], gpu)
    sq = H.to_dev(host_ops.quantize_u8(s.specular, True)[0], gpu)
    with pytest.raises(_lib.VTError, match="format 1"):
        native.infer_f16(d["points"], d["diffuse4"], d["specular4"], d["density"], d["adjacency"], d["offsets"],
                         d["adj"], H.to_dev(rays, gpu), H.to_dev(start, gpu), tiled=(8, 8),
                         quads=native.QuadMaps.build(dq, sq))


def test_quad_renders_infer_camera_drop_in(gpu):
    """VoroTracingInfer's buffer and camera renders and the fp16 drop-in with
    a lane order: the same image with the tables on and off; the drop-in's
    cached tables are rebuilt after an in-place change of the maps."""
    from vorotracing_amd.infer import VoroTracingInfer
    from vorotracing_amd.model import VoroTracing
    s = H.mini_heightfield_r8()
    inf = VoroTracingInfer(VoroTracing.from_scene(s, device=gpu), sort_morton=True, quantize="fp16")
    assert inf.quad_tables() is not None
    kw = dict(weight_threshold=0.01, cell_skip_threshold=1e-3)
    rays = H.to_dev(camera.orbit_rays(3, 128, 96), gpu)
    cams = [camera.Camera.orbit(3, 128, 96)]
    outs = {}
    try:
        for on in (True, False):
            VoroTracingInfer.quad_maps = on
            print(f"case: VoroTracingInfer renders, quad maps {on}", flush=True)
            outs[on] = (inf.render(rays, **kw), inf.render_cameras(cams, **kw))
    finally:
        VoroTracingInfer.quad_maps = True
    torch.cuda.synchronize()
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))

    sp = inf.get_starting_point(rays)
    perm = torch.arange(rays.numel() // 6, dtype=torch.int32, device=gpu)
    diffuse = inf.diffuse_fp16.clone()

    def render():
        return _C.trace_vorotracing_infer(inf.primal_points, diffuse, inf.specular_fp16, inf.density,
                                          inf.point_adjacency, inf.point_adjacency_offsets, rays, sp,
                                          inf.adjacent_diff, perm, 0.01, 1024, 1e-3)

    try:
        for step in range(2):
            print(f"case: fp16 drop-in, quad maps on/off, maps changed {bool(step)}", flush=True)
            _C.DROP_IN_QUADS = False
            plain = render()
            _C.DROP_IN_QUADS = True
            quad = render()
            torch.cuda.synchronize()
            assert torch.equal(quad.view(torch.int16), plain.view(torch.int16))
            if step == 0:
                assert torch.equal(quad.view(torch.int16), outs[True][0].view(torch.int16))
                diffuse.mul_(0.5)  # in place: the cached tables must not be reused
    finally:
        _C.DROP_IN_QUADS = True


@pytest.mark.parametrize("res", ["r4", "r8"])
def test_quad_q8_renders(gpu, res):
    """q8 renders of VoroTracingInfer (buffer and camera) and the q8 drop-in
    with a lane order: the same image with the q8 tables on and off (the q8
    parity tests against the oracle run with the tables on, the default)."""
    from vorotracing_amd.infer import VoroTracingInfer
    from vorotracing_amd.model import VoroTracing
    s = H.mini_heightfield() if res == "r4" else H.mini_heightfield_r8()
    inf = VoroTracingInfer(VoroTracing.from_scene(s, device=gpu), sort_morton=True, quantize="q8",
                           per_channel_q8=True)
    qt = inf.quad_tables()
    assert qt is not None and qt.format == native.QUAD_Q8
    kw = dict(weight_threshold=0.01, cell_skip_threshold=1e-3)
    rays = H.to_dev(camera.orbit_rays(5, 128, 96), gpu)
    cams = [camera.Camera.orbit(5, 128, 96)]
    outs = {}
    try:
        for on in (True, False):
            VoroTracingInfer.quad_maps = on
            print(f"case: q8 {res} renders, quad maps {on}", flush=True)
            outs[on] = (inf.render(rays, **kw), inf.render_cameras(cams, **kw))
    finally:
        VoroTracingInfer.quad_maps = True
    torch.cuda.synchronize()
    for a, b in zip(outs[True], outs[False]):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    sp = inf.get_starting_point(rays)
    perm = torch.arange(rays.numel() // 6, dtype=torch.int32, device=gpu)

    def render():
        return _C.trace_vorotracing_infer_q8(inf.primal_points, inf.diffuse_q8, inf.specular_q8, inf.density,
                                             inf.point_adjacency, inf.point_adjacency_offsets, rays, sp,
                                             inf.adjacent_diff, inf.diff_scale, inf.diff_offset, inf.spec_scale,
                                             inf.spec_offset, 0.01, 1024, 1e-3, ray_perm_in=perm)

    try:
        print(f"case: q8 {res} drop-in, quad maps on/off", flush=True)
        _C.DROP_IN_QUADS = False
        plain = render()
        _C.DROP_IN_QUADS = True
        quad = render()
        torch.cuda.synchronize()
    finally:
        _C.DROP_IN_QUADS = True
    assert torch.equal(quad.view(torch.int16), plain.view(torch.int16))
    assert torch.equal(quad.view(torch.int16), outs[True][0].view(torch.int16))


def test_quad_tables_memory_guard(gpu):
    """Tables that would take more than QuadMaps.MAX_FREE_SHARE of the free
    memory are not built; the renders then read the maps, with the same image."""
    from vorotracing_amd.infer import VoroTracingInfer
    from vorotracing_amd.model import VoroTracing
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    kw = dict(weight_threshold=0.01, cell_skip_threshold=1e-3)
    rays = H.to_dev(camera.orbit_rays(7, 96, 64), gpu)
    inf = VoroTracingInfer(model, sort_morton=True, quantize="fp16")
    assert inf.quad_tables() is not None
    with_tables = inf.render(rays, **kw)
    share = native.QuadMaps.MAX_FREE_SHARE
    try:
        native.QuadMaps.MAX_FREE_SHARE = 0.0
        lean = VoroTracingInfer(model, sort_morton=True, quantize="fp16")
        assert lean.quad_tables() is None
        without = lean.render(rays, **kw)
    finally:
        native.QuadMaps.MAX_FREE_SHARE = share
    torch.cuda.synchronize()
    assert torch.equal(with_tables.view(torch.int16), without.view(torch.int16))
