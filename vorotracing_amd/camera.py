"""Ray generation for the benchmark cameras (host side, float64 then f32),
and ``Camera``, the record the in-kernel ray generation takes
(``vt_camera`` in include/vt_abi.h).

Rays are ``[..., 6]`` f32 = origin xyz + direction xyz, the layout of
``Ray`` (camera.h:5-8) the traversal reads.  Pinhole rays follow
vorotracing/utils/__init__.py:85-130 (OpenCV axes: x right, y down, z
forward; ``dir = R (x, y, 1)``, normalised) with pixel centres at +0.5.
"""
from __future__ import annotations

import dataclasses
import math
import struct

import numpy as np


def look_at(eye, target=(0.0, 0.0, 0.0), up=(0.0, 0.0, 1.0)) -> np.ndarray:
    """Camera-to-world rotation (columns right, down, forward) for OpenCV axes."""
    eye = np.asarray(eye, np.float64)
    f = np.asarray(target, np.float64) - eye
    f /= np.linalg.norm(f)
    r = np.cross(f, np.asarray(up, np.float64))
    if np.linalg.norm(r) < 1e-12:
        r = np.cross(f, np.array([0.0, 1.0, 0.0]))
    r /= np.linalg.norm(r)
    d = np.cross(f, r)
    return np.stack([r, d, f], 1)


def orbit_eye(k: int, n: int = 32, radius: float = 7.0, elevation_deg: float = 35.0) -> np.ndarray:
    az = 2.0 * math.pi * k / n
    el = math.radians(elevation_deg)
    return np.array([radius * math.cos(el) * math.cos(az), radius * math.cos(el) * math.sin(az),
                     radius * math.sin(el)])


def pinhole_rays(width: int, height: int, eye, target=(0.0, 0.0, 0.0), up=(0.0, 0.0, 1.0),
                 fov_y_deg: float = 60.0) -> np.ndarray:
    """(H, W, 6) f32 rays of a pinhole camera at ``eye`` looking at ``target``."""
    Rcw = look_at(eye, target, up)
    f = (height / 2.0) / math.tan(math.radians(fov_y_deg) / 2.0)
    u, v = np.meshgrid(np.arange(width, dtype=np.float64), np.arange(height, dtype=np.float64), indexing="xy")
    x = (u + 0.5 - width / 2.0) / f
    y = (v + 0.5 - height / 2.0) / f
    dc = np.stack([x, y, np.ones_like(x)], -1)
    dc /= np.linalg.norm(dc, axis=-1, keepdims=True)
    dw = dc @ Rcw.T
    dw /= np.linalg.norm(dw, axis=-1, keepdims=True)
    o = np.broadcast_to(np.asarray(eye, np.float64), dw.shape)
    return np.concatenate([o, dw], -1).astype(np.float32)


def orbit_rays(k: int, width: int, height: int, n: int = 32, radius: float = 7.0, elevation_deg: float = 35.0,
               fov_y_deg: float = 60.0) -> np.ndarray:
    """Pose k of the config-3 orbit: radius 7, elevation 35 deg, azimuth 2 pi k / n,
    looking at the origin, +z up, 60 deg vertical FOV."""
    return pinhole_rays(width, height, orbit_eye(k, n, radius, elevation_deg), fov_y_deg=fov_y_deg)


def fisheye_rolling_rays(width: int = 1558, height: int = 1039, eye=None, k1: float = -0.1, k2: float = 0.01,
                         diag_fov_deg: float = 180.0, shutter_shift: float = 0.05) -> np.ndarray:
    """Config-5 rays: equidistant fisheye theta_d = theta (1 + k1 theta^2 + k2 theta^4),
    r_px = f theta_d with f set so the image diagonal spans ``diag_fov_deg``;
    unprojection by Newton on theta.  Rolling shutter: the origin of row r is
    eye + (r / (H-1)) * shutter_shift * x_cam."""
    if eye is None:
        eye = orbit_eye(0)
    Rcw = look_at(eye)
    half_diag = math.hypot(width / 2.0, height / 2.0)
    tmax = math.radians(diag_fov_deg) / 2.0
    f = half_diag / (tmax * (1 + k1 * tmax ** 2 + k2 * tmax ** 4))
    u, v = np.meshgrid(np.arange(width, dtype=np.float64), np.arange(height, dtype=np.float64), indexing="xy")
    px = u + 0.5 - width / 2.0
    py = v + 0.5 - height / 2.0
    r = np.hypot(px, py)
    td = r / f
    th = td.copy()
    for _ in range(20):
        g = th * (1 + k1 * th ** 2 + k2 * th ** 4) - td
        dg = 1 + 3 * k1 * th ** 2 + 5 * k2 * th ** 4
        th = th - g / dg
    phi = np.arctan2(py, px)
    st = np.sin(th)
    dc = np.stack([st * np.cos(phi), st * np.sin(phi), np.cos(th)], -1)
    dw = dc @ Rcw.T
    dw /= np.linalg.norm(dw, axis=-1, keepdims=True)
    shift = (v / (height - 1)) * shutter_shift
    o = np.asarray(eye, np.float64)[None, None, :] + shift[..., None] * Rcw[:, 0][None, None, :]
    return np.concatenate([o, dw], -1).astype(np.float32)


_CAMERA_FMT = struct.Struct("<I5f4f9f3f3f")  # vt_camera, 100 bytes
CAMERA_MODELS = {"pinhole": 0, "fisheye": 1}


@dataclasses.dataclass
class Camera:
    """A camera for in-kernel ray generation (``vt_camera``).  Pixel (u, v)
    samples (u + pixel_offset, v + pixel_offset); ``R`` is camera-to-world
    (OpenCV axes: x right, y down, z forward), ``t`` the centre; ``k`` the
    OpenCV fisheye distortion k1..k4; row v's origin is
    ``t + v / (height - 1) * rolling`` (rolling shutter)."""

    width: int
    height: int
    fx: float
    fy: float
    cx: float
    cy: float
    R: np.ndarray
    t: np.ndarray
    model: str = "pinhole"
    k: tuple = (0.0, 0.0, 0.0, 0.0)
    pixel_offset: float = 0.5
    rolling: np.ndarray = dataclasses.field(default_factory=lambda: np.zeros(3))

    @property
    def rolling_shutter(self) -> bool:
        return bool(np.any(np.asarray(self.rolling) != 0))

    def pack(self) -> bytes:
        """The 100-byte vt_camera record (f32 fields)."""
        k = list(self.k) + [0.0] * (4 - len(self.k))
        if self.model not in CAMERA_MODELS:
            raise ValueError(f"unknown camera model {self.model!r} (known: {sorted(CAMERA_MODELS)})")
        return _CAMERA_FMT.pack(CAMERA_MODELS[self.model], self.fx, self.fy, self.cx, self.cy, self.pixel_offset,
                                *k[:4], *np.asarray(self.R, np.float64).reshape(9), *np.asarray(self.t).reshape(3),
                                *np.asarray(self.rolling).reshape(3))

    @classmethod
    def look_at(cls, width: int, height: int, eye, target=(0.0, 0.0, 0.0), up=(0.0, 0.0, 1.0),
                fov_y_deg: float = 60.0) -> "Camera":
        """The pinhole camera of ``pinhole_rays``."""
        f = (height / 2.0) / math.tan(math.radians(fov_y_deg) / 2.0)
        return cls(width, height, f, f, width / 2.0, height / 2.0, look_at(eye, target, up),
                   np.asarray(eye, np.float64))

    @classmethod
    def orbit(cls, k: int, width: int, height: int, n: int = 32, radius: float = 7.0, elevation_deg: float = 35.0,
              fov_y_deg: float = 60.0) -> "Camera":
        """Pose k of the config-3 orbit (``orbit_rays``)."""
        return cls.look_at(width, height, orbit_eye(k, n, radius, elevation_deg), fov_y_deg=fov_y_deg)

    @classmethod
    def fisheye_rolling(cls, width: int = 1558, height: int = 1039, eye=None, k1: float = -0.1, k2: float = 0.01,
                        diag_fov_deg: float = 180.0, shutter_shift: float = 0.05) -> "Camera":
        """The config-5 camera of ``fisheye_rolling_rays``."""
        if eye is None:
            eye = orbit_eye(0)
        Rcw = look_at(eye)
        half_diag = math.hypot(width / 2.0, height / 2.0)
        tmax = math.radians(diag_fov_deg) / 2.0
        f = half_diag / (tmax * (1 + k1 * tmax ** 2 + k2 * tmax ** 4))
        return cls(width, height, f, f, width / 2.0, height / 2.0, Rcw, np.asarray(eye, np.float64), "fisheye",
                   (k1, k2, 0.0, 0.0), 0.5, shutter_shift * Rcw[:, 0])


def pack_cameras(cameras) -> bytes:
    """vt_camera array of a batch of cameras of one image size."""
    cams = list(cameras)
    if not cams:
        raise ValueError("no cameras")
    if any((c.width, c.height) != (cams[0].width, cams[0].height) for c in cams):
        raise ValueError("all cameras of a batch must have the same image size")
    return b"".join(c.pack() for c in cams)
