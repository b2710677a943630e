"""CPU pins of the camera ray generator's restatement (oracle or_camera_rays,
or_sinf / or_cosf) against independent float64 computations: camera.py's
numpy generators and the reference's pinhole formula
(vorotracing/utils/__init__.py:85-130), and of the vt_camera record layout."""
import math
import struct

import numpy as np
import pytest

from oracle import core as oc
from vorotracing_amd import camera


def test_sin_cos_against_float64():
    x = np.concatenate([np.linspace(0, np.pi, 200001), [0.0, np.pi / 2, np.pi]]).astype(np.float32)
    for cos in (False, True):
        got = oc.sincos(x, cos).astype(np.float64)
        ref = np.cos(x.astype(np.float64)) if cos else np.sin(x.astype(np.float64))
        assert np.abs(got - ref).max() <= 1e-7
        big = np.abs(ref) >= 1e-6  # relative error, also next to the zero crossings
        ulp = np.spacing(np.abs(ref[big]).astype(np.float32)).astype(np.float64)
        assert (np.abs(got[big] - ref[big]) / ulp).max() <= 2.0
    assert oc.sincos(np.float32(0.0))[0] == 0.0 and oc.sincos(np.float32(0.0), True)[0] == 1.0


def _unit(d):
    return d / np.linalg.norm(d, axis=-1, keepdims=True)


@pytest.mark.parametrize("k", [0, 5, 17])
def test_orbit_pinhole_matches_float64(k):
    W, H = 96, 64
    c = camera.Camera.orbit(k, W, H)
    got = oc.camera_rays(c.pack(), 1, H, W)[0]
    want = camera.orbit_rays(k, W, H)
    assert np.abs(_unit(got[..., 3:]) - want[..., 3:]).max() <= 3e-7
    assert np.array_equal(got[..., :3], want[..., :3])


def test_fisheye_rolling_matches_float64():
    W, H = 160, 108
    c = camera.Camera.fisheye_rolling(W, H)
    got = oc.camera_rays(c.pack(), 1, H, W)[0]
    want = camera.fisheye_rolling_rays(W, H)
    assert np.abs(_unit(got[..., 3:]) - want[..., 3:]).max() <= 5e-7
    assert np.abs(got[..., :3] - want[..., :3]).max() <= 1e-6
    # rolling shutter: row 0 at the centre, last row shifted by the full shift along x_cam
    assert np.array_equal(got[0, :, :3], np.broadcast_to(np.float32(c.t), (W, 3)))
    assert np.abs(got[-1, 0, :3] - (c.t + c.rolling)).max() <= 1e-6


def test_reference_pinhole_formula():
    """generate_camera_rays (utils/__init__.py:85-130): pixel u without an offset,
    x = (u - cx) / fx, dirs normalised in camera space, rotated by T_c2w, normalised."""
    W, H = 40, 30
    fx, fy, cx, cy = 35.0, 31.0, 18.5, 16.25
    ang = 0.3
    R = np.array([[math.cos(ang), 0, math.sin(ang)], [0, 1, 0], [-math.sin(ang), 0, math.cos(ang)]])
    t = np.array([0.5, -1.0, 2.0])
    c = camera.Camera(W, H, fx, fy, cx, cy, R, t, pixel_offset=0.0)
    got = oc.camera_rays(c.pack(), 1, H, W)[0]
    u, v = np.meshgrid(np.arange(W, dtype=np.float64), np.arange(H, dtype=np.float64), indexing="xy")
    dc = _unit(np.stack([(u - cx) / fx, (v - cy) / fy, np.ones_like(u)], -1))
    dw = _unit(dc @ R.T)
    assert np.abs(_unit(got[..., 3:]) - dw).max() <= 3e-7
    assert np.abs(got[..., :3] - t).max() <= 1e-7


def test_fisheye_unprojection_inverts_projection():
    """Project known directions with the OpenCV fisheye model (float64), place the pixel
    there, and recover the direction: theta_d = theta (1 + k1 theta^2 + ... + k4 theta^8)."""
    k = (-0.05, 0.004, -0.0003, 0.00002)
    f = 200.0
    rng = np.random.default_rng(2)
    th = rng.uniform(0.0, 1.5, 64)
    ph = rng.uniform(-np.pi, np.pi, 64)
    td = th * (1 + k[0] * th ** 2 + k[1] * th ** 4 + k[2] * th ** 6 + k[3] * th ** 8)
    # one camera per direction: principal point chosen so pixel (0, 0) sits on it
    packed = b""
    for i in range(64):
        x, y = f * td[i] * np.cos(ph[i]), f * td[i] * np.sin(ph[i])
        c = camera.Camera(1, 1, f, f, 0.5 - x, 0.5 - y, np.eye(3), np.zeros(3), "fisheye", k)
        packed += c.pack()
    got = oc.camera_rays(packed, 64, 1, 1).reshape(64, 6)
    want = np.stack([np.sin(th) * np.cos(ph), np.sin(th) * np.sin(ph), np.cos(th)], -1)
    assert np.abs(_unit(got[:, 3:]) - want).max() <= 2e-6


def test_camera_record_layout():
    c = camera.Camera.fisheye_rolling(64, 48)
    b = c.pack()
    assert len(b) == 100
    f = struct.unpack("<I5f4f9f3f3f", b)
    assert f[0] == 1 and f[5] == np.float32(0.5)
    assert np.allclose(f[10:19], np.asarray(c.R).reshape(9), atol=1e-7)
    assert np.allclose(f[22:25], c.rolling, atol=1e-7)
    with pytest.raises(ValueError):
        camera.pack_cameras([camera.Camera.orbit(0, 8, 8), camera.Camera.orbit(1, 8, 16)])
