"""GPU parity of in-kernel ray generation: vt_camera_rays against the CPU
restatement (bit-exact), and the camera renders (vt_trace_infer_*_camera)
against the buffer renders of the same rays and against the oracle
(bit-exact images and walk statistics)."""
import numpy as np
import pytest
import torch

from oracle import core as oc
from tests import helpers as H
from vorotracing_amd import camera, native
from vorotracing_amd.infer import VoroTracingInfer
from vorotracing_amd.model import VoroTracing

pytestmark = pytest.mark.gpu


def _cams(kind, W, Hh):
    if kind == "orbit":
        return [camera.Camera.orbit(k, W, Hh) for k in (0, 7, 13)]
    if kind == "fisheye_rolling":
        return [camera.Camera.fisheye_rolling(W, Hh, eye=camera.orbit_eye(k)) for k in (0, 9)]
    if kind == "mixed":
        return [camera.Camera.orbit(2, W, Hh),
                camera.Camera.fisheye_rolling(W, Hh, eye=camera.orbit_eye(3), k1=-0.05, k2=0.002,
                                              diag_fov_deg=150.0, shutter_shift=0.0)]
    if kind == "many":  # a larger batch
        return [camera.Camera.orbit(k, W, Hh, n=18) for k in range(18)]
    raise ValueError(kind)


def test_math_probe_sin_cos(gpu):
    x = np.concatenate([np.linspace(0.0, np.pi, 1 << 18),
                        [0.0, 0.785398185, 0.78539824, 2.3561945, 2.35619473, 1.5707964, 3.1415927]])
    x = x.astype(np.float32)
    for op, cos in ((3, False), (4, True)):
        got = native.math_probe(op, torch.from_numpy(x).to(gpu)).cpu().numpy()
        assert np.array_equal(got, oc.sincos(x, cos).view(np.uint32))


@pytest.mark.parametrize("kind", ["orbit", "fisheye_rolling", "mixed", "many"])
def test_camera_rays_bit_exact(gpu, kind):
    W, Hh = 40, 24
    cams = _cams(kind, W, Hh)
    got = native.camera_rays(cams, gpu).cpu().numpy()
    want = oc.camera_rays(camera.pack_cameras(cams), len(cams), Hh, W)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _infer(gpu, quantize, R=4):
    s = H.mini_heightfield() if R == 4 else H.mini_heightfield_r8()
    model = VoroTracing.from_scene(s, device=gpu)
    return VoroTracingInfer(model, sort_morton=True, quantize=quantize)


@pytest.mark.parametrize("quantize", ["fp16", "q8"])
@pytest.mark.parametrize("kind", ["orbit", "fisheye_rolling", "many"])
def test_camera_render_equals_buffer_render(gpu, quantize, kind):
    """Same image and walk statistics as render() on the rays of vt_camera_rays with
    the same start cells (per image, or per row for rolling shutters)."""
    W, Hh = (72, 40) if kind != "many" else (24, 16)
    cams = _cams(kind, W, Hh)
    inf = _infer(gpu, quantize)
    start, per_row = inf.camera_start_points(cams)
    assert per_row == any(c.rolling_shutter for c in cams)
    rays = native.camera_rays(cams, gpu)
    B = len(cams)
    sp_rays = (start.view(B, Hh, 1) if per_row else start.view(B, 1, 1)).expand(B, Hh, W).contiguous()
    n = B * Hh * W
    st_cam, st_buf = native.new_stats(n, gpu), native.new_stats(n, gpu)
    got = inf.render_cameras(cams, weight_threshold=0.01, cell_skip_threshold=1e-3, stats=st_cam)
    want = inf.render(rays, start_point=sp_rays, weight_threshold=0.01, cell_skip_threshold=1e-3, stats=st_buf)
    torch.cuda.synchronize()
    assert got.shape == (B, Hh, W, 4)
    H.assert_stats_equal(H.stats_np(st_cam), H.stats_np(st_buf))
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    assert (H.stats_np(st_cam)["integrated"] > 0).mean() > 0.3  # the cameras see the scene


@pytest.mark.parametrize("R", [4, 8])
def test_camera_render_equals_oracle(gpu, R):
    """fp16 camera render of a fisheye rolling-shutter camera against the oracle
    rendering the oracle's own rays from the oracle's start cells; R = 8 has
    the reference's 8x8 diffuse and specular maps."""
    W, Hh = 64, 40
    cams = _cams("fisheye_rolling", W, Hh)[:1]
    inf = _infer(gpu, "fp16", R)
    rays = oc.camera_rays(camera.pack_cameras(cams), 1, Hh, W)
    pts = inf.primal_points.cpu().numpy()
    row_origins = rays[0, :, 0, :3]
    from oracle import host_ops

    start_rows = host_ops.nearest_site(pts, row_origins).astype(np.uint32)
    start_rays = np.broadcast_to(start_rows[None, :, None], (1, Hh, W)).copy()
    want, wst, _ = oc.trace_infer_f16(pts, inf.diffuse_fp16.cpu().numpy(), inf.specular_fp16.cpu().numpy(), R, R,
                                      inf.density.reshape(-1).cpu().numpy(), inf.point_adjacency.cpu().numpy(),
                                      inf.point_adjacency_offsets.cpu().numpy(), inf.adjacent_diff.cpu().numpy(),
                                      rays, start_rays, weight_threshold=0.01, cell_skip_threshold=1e-3,
                                      want_stats=True)
    st = native.new_stats(Hh * W, gpu)
    got = inf.render_cameras(cams, weight_threshold=0.01, cell_skip_threshold=1e-3,
                             start_point=torch.from_numpy(start_rows).to(gpu), stats=st)
    torch.cuda.synchronize()
    H.assert_stats_equal(H.stats_np(st), wst)
    H.assert_infer_rgba(got.cpu().numpy(), want)


def test_camera_render_argument_errors(gpu):
    inf = _infer(gpu, "fp16")
    bad = camera.Camera.orbit(0, 16, 8)
    bad.model = "orthographic"
    with pytest.raises(ValueError, match="unknown camera model"):
        inf.render_cameras([bad])
    with pytest.raises(ValueError):
        inf.render_cameras([camera.Camera.orbit(0, 16, 8), camera.Camera.orbit(1, 8, 8)])
    from vorotracing_amd import _lib

    with pytest.raises(_lib.VTError, match="null pointer"):
        _lib.call("vt_camera_rays", None, 1, 8, 16, None, None)
