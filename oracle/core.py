"""ctypes binding of liboracle.so (the C restatement in oracle.c).

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.  Arrays are numpy; every
function mirrors the corresponding entry of oracle.h, which cites the
reference file:line it restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

STATS_DTYPE = np.dtype(
    [
        ("n", "<u4"),
        ("visits", "<u4"),
        ("faces", "<u4"),
        ("exits", "<u4"),
        ("integrated", "<u4"),
        ("shaded", "<u4"),
        ("visit_hash", "<u8"),
        ("first_cells", "<u4", (24,)),  # OR_STATS_LOG
    ]
)
assert STATS_DTYPE.itemsize == 128


def build(force: bool = False) -> str:
    """Compile liboracle.so with oracle/Makefile (gcc)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-B" if force else "-s", "-C", _HERE, "liboracle.so"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = C.CDLL(_LIB_PATH)
        f = C.c_float
        u32 = C.c_uint32
        _lib.or_expf.restype = f
        _lib.or_expf.argtypes = [f]
        _lib.or_logf.restype = f
        _lib.or_logf.argtypes = [f]
        _lib.or_f32_to_f16.restype = C.c_uint16
        _lib.or_f32_to_f16.argtypes = [f]
        _lib.or_f16_to_f32.restype = f
        _lib.or_f16_to_f32.argtypes = [C.c_uint16]
        _lib.or_oct_wrap_index.restype = C.c_int
        _lib.or_oct_wrap_index.argtypes = [C.c_int, C.c_int, C.c_int]
        _lib.or_trace_infer_f16.argtypes = None
        del u32
    return _lib


class plant:
    """Context manager switching on one of oracle.h's planted mistakes
    (OR_PLANT_*) for the pin tests: ``with core.plant(core.PLANT_SPEC_PLUS_D): ...``."""

    def __init__(self, code: int):
        self.code = int(code)

    def __enter__(self):
        lib().or_set_plant(C.c_int(self.code))
        return self

    def __exit__(self, *exc):
        lib().or_set_plant(C.c_int(0))
        return False


class abs_sums:
    """Context manager for oracle.h's absolute-sum mode: inside it, trace_bwd
    returns per element the sum of |v| over the values scattered into it
    (``with core.abs_sums(): cond = core.trace_bwd(...)``); with
    ``count=True`` the number of values scattered into it instead."""

    def __init__(self, count: bool = False):
        self.mode = 2 if count else 1

    def __enter__(self):
        lib().or_set_abs_sums(C.c_int(self.mode))
        return self

    def __exit__(self, *exc):
        lib().or_set_abs_sums(C.c_int(0))
        return False


PLANT_SPEC_PLUS_D = 1
PLANT_INFER_NO_DENSITY_GATE = 2
PLANT_SKIP_ON_ALPHA = 3
PLANT_NO_FIRST_CELL_TERM = 4
PLANT_FLUSH_CUR_ON_STOP = 5
PLANT_POINT_ERROR_ALPHA = 6
PLANT_IGNORE_CONTRIB_GRAD = 7
PLANT_NO_DT0_PREV = 8


def _p(a):
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return a.ctypes.data_as(C.c_void_p)


def _f(x):
    return C.c_float(float(x))


def _u(x):
    return C.c_uint32(int(x))


def _i(x):
    return C.c_int(int(x))


def _sz(x):
    return C.c_size_t(int(x))


def _c(a, dtype):
    if a is None:
        return None
    return np.ascontiguousarray(a, dtype=dtype)


# --------------------------------------------------------------------------
# scalar helpers


def expf(x):
    x = _c(np.atleast_1d(x), np.float32)
    y = np.empty_like(x)
    lib().or_expf_many(_p(x), _p(y), _sz(x.size))
    return y


def logf(x):
    x = _c(np.atleast_1d(x), np.float32)
    y = np.empty_like(x)
    lib().or_logf_many(_p(x), _p(y), _sz(x.size))
    return y


def f32_to_f16_bits(x):
    x = _c(np.atleast_1d(x), np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16_many(_p(x), _p(y), _sz(x.size))
    return y


def exit_face_rows(rows):
    """The walk's exit-face search (tracing_octmap.cu:73-100) on (n, 26)
    float32 rows: site, origin, unit direction, face count (uint32 bits, at
    most 8), 8 half4 face records as 16 words.  Returns (n, 2) uint32: face
    index (0xffffffff = none) and the bits of t1."""
    rows = _c(rows, np.float32)
    assert rows.ndim == 2 and rows.shape[1] == 26
    out = np.empty((rows.shape[0], 2), np.uint32)
    lib().or_exit_face_many(_p(rows), _sz(rows.shape[0]), _p(out))
    return out


def oct_wrap_index(u, v, R):
    return lib().or_oct_wrap_index(int(u), int(v), int(R))


def oct_encode(d, R):
    d = _c(d, np.float32)
    uv = np.empty(2, np.float32)
    lib().or_oct_encode(_p(d), _i(R), _p(uv))
    return uv


def cell_intersection_grad(prim, opp, o, d):
    a = [_c(np.asarray(x), np.float32) for x in (prim, opp, o, d)]
    out = np.empty(3, np.float32)
    lib().or_cell_intersection_grad(*[_p(x) for x in a], _p(out))
    return out


# --------------------------------------------------------------------------
# kernels


def prefetch_adj(points, adjacency, offsets, threads=0):
    points = _c(points, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    out = np.zeros((adjacency.shape[0] + 32, 4), np.float16)
    lib().or_prefetch_adj(_p(points), _u(points.shape[0]), _p(adjacency), _p(offsets), _p(out), _i(threads))
    return out


def trace_infer_f16(points, diffuse4, specular4, diff_res, spec_res, density, adjacency, offsets, adj_diff, rays,
                    start_point, ray_perm=None, weight_threshold=0.001, max_intersections=1024,
                    cell_skip_threshold=0.0, want_stats=False, max_log=0, threads=0):
    """Restates tracing_octmap.cu:552-610.  Returns (rgba f16 [...,4], stats, visit log)."""
    lead = rays.shape[:-1]
    rays = _c(rays, np.float32).reshape(-1, 6)
    nr = rays.shape[0]
    start = _c(start_point, np.uint32).reshape(-1)
    assert start.shape[0] == nr
    perm = None if ray_perm is None or np.size(ray_perm) == 0 else _c(ray_perm, np.int32).view(np.uint32)
    rgba = np.empty((nr, 4), np.float16)
    stats = np.zeros(nr, STATS_DTYPE) if want_stats else None
    log = np.empty((nr, max_log), np.uint32) if max_log else None
    lib().or_trace_infer_f16(
        _p(_c(points, np.float32)), _p(_c(diffuse4, np.float16)), _p(_c(specular4, np.float16)), _i(diff_res),
        _i(spec_res), _p(_c(density, np.float32)), _p(_c(adjacency, np.uint32)), _p(_c(offsets, np.uint32)),
        _p(_c(adj_diff, np.float16)), _p(rays), _u(nr), _p(start), _p(perm), _f(weight_threshold),
        _u(max_intersections), _f(cell_skip_threshold), _p(rgba), _p(stats), _p(log), _u(max_log), _i(threads))
    return rgba.reshape(*lead, 4), stats, log


def trace_infer_q8(points, diffuse_q8, specular_q8, diff_res, spec_res, diff_scale, diff_offset, spec_scale,
                   spec_offset, density, adjacency, offsets, adj_diff, rays, start_point, weight_threshold=0.001,
                   max_intersections=1024, cell_skip_threshold=0.0, want_stats=False, threads=0):
    """Restates tracing_octmap.cu:723-779 with per-channel (3-vector) scale/offset."""
    lead = rays.shape[:-1]
    rays = _c(rays, np.float32).reshape(-1, 6)
    nr = rays.shape[0]
    start = _c(start_point, np.uint32).reshape(-1)

    def v3(x):
        return _c(np.broadcast_to(np.asarray(x, np.float32), (3,)), np.float32)

    ds, do, ss, so = v3(diff_scale), v3(diff_offset), v3(spec_scale), v3(spec_offset)
    rgba = np.empty((nr, 4), np.float16)
    stats = np.zeros(nr, STATS_DTYPE) if want_stats else None
    lib().or_trace_infer_q8(
        _p(_c(points, np.float32)), _p(_c(diffuse_q8, np.uint8)), _p(_c(specular_q8, np.uint8)), _i(diff_res),
        _i(spec_res), _p(ds), _p(do), _p(ss), _p(so), _p(_c(density, np.float32)), _p(_c(adjacency, np.uint32)),
        _p(_c(offsets, np.uint32)), _p(_c(adj_diff, np.float16)), _p(rays), _u(nr), _p(start),
        _f(weight_threshold), _u(max_intersections), _f(cell_skip_threshold), _p(rgba), _p(stats), _i(threads))
    return rgba.reshape(*lead, 4), stats


def trace_fwd(points, diffuse, specular, diff_res, spec_res, density, adjacency, offsets, rays, start_point,
              depth_quantiles=None, weight_threshold=0.001, max_intersections=1024, return_contribution=False,
              want_stats=False, threads=0):
    """Restates the training forward (tracing_octmap.cu:151-230, host :346-546), prefetch included.

    Returns dict with rgba, depth, depth_idx, contribution, n, distortion, W_total, S_total, t_far (+stats).
    """
    f16 = np.asarray(diffuse).dtype == np.float16
    adt = np.float16 if f16 else np.float32
    lead = rays.shape[:-1]
    rays = _c(rays, np.float32).reshape(-1, 6)
    nr = rays.shape[0]
    start = _c(start_point, np.uint32).reshape(-1)
    points = _c(points, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    adj_diff = prefetch_adj(points, adjacency, offsets, threads)
    K = 0
    dq = None
    if depth_quantiles is not None:
        dq = _c(depth_quantiles, np.float32)
        K = dq.shape[-1]
        dq = dq.reshape(nr, K)
    rgba = np.empty((nr, 4), adt)
    depth = np.zeros((nr, K), np.float32) if dq is not None else None
    depth_idx = np.zeros((nr, K), np.uint32) if dq is not None else None
    contrib = np.zeros((points.shape[0], 1), adt) if return_contribution else None
    n = np.empty((nr, 1), np.uint32)
    dist = np.empty((nr, 1), np.float32)
    W = np.empty((nr, 1), np.float32)
    S = np.empty((nr, 1), np.float32)
    tf = np.empty((nr, 1), np.float32)
    stats = np.zeros(nr, STATS_DTYPE) if want_stats else None
    lib().or_trace_fwd(
        _i(1 if f16 else 0), _p(points), _p(_c(diffuse, adt)), _p(_c(specular, adt)), _i(diff_res), _i(spec_res),
        _p(_c(density, np.float32)), _p(adjacency), _p(offsets), _p(adj_diff), _p(rays), _u(nr), _p(start), _u(K),
        _p(dq), _f(weight_threshold), _u(max_intersections), _p(rgba), _p(depth), _p(depth_idx), _p(contrib),
        _p(n), _p(dist), _p(W), _p(S), _p(tf), _p(stats), _i(threads))

    def shp(a, last):
        return None if a is None else a.reshape(*lead, last)

    return dict(rgba=shp(rgba, 4), depth=shp(depth, K), depth_idx=shp(depth_idx, K), contribution=contrib,
                n=shp(n, 1), distortion=shp(dist, 1), W_total=shp(W, 1), S_total=shp(S, 1), t_far=shp(tf, 1),
                stats=stats)


def trace_bwd(points, diffuse, specular, diff_res, spec_res, density, adjacency, offsets, rays, start_point, rgba,
              rgba_grad, depth_quantiles=None, depth_idx=None, depth_grad=None, ray_error=None,
              contribution_alpha_grad=0.0, distortion=None, distortion_grad=None, W_total=None, S_total=None,
              t_far=None, weight_threshold=0.001, max_intersections=1024, want_stats=False, threads=0):
    """Restates the training backward (tracing_octmap.cu:232-340, host :860-1103), prefetch included.

    Returns dict points_grad (N,3), diffuse_grad, specular_grad, density_grad (N,1), point_error.
    """
    f16 = np.asarray(diffuse).dtype == np.float16
    adt = np.float16 if f16 else np.float32
    rays = _c(rays, np.float32).reshape(-1, 6)
    nr = rays.shape[0]
    start = _c(start_point, np.uint32).reshape(-1)
    points = _c(points, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    diffuse = _c(diffuse, adt)
    specular = _c(specular, adt)
    density = _c(density, np.float32)
    adj_diff = prefetch_adj(points, adjacency, offsets, threads)
    K = 0
    dq = di = dg = None
    if depth_quantiles is not None:
        dq = _c(depth_quantiles, np.float32)
        K = dq.shape[-1]
        dq = dq.reshape(nr, K)
        di = _c(depth_idx, np.uint32).reshape(nr, K)
        dg = _c(depth_grad, np.float32).reshape(nr, K)
    N = points.shape[0]
    pg = np.zeros((N, 3), np.float32)
    dgd = np.zeros(diffuse.shape, adt)
    sgd = np.zeros(specular.shape, adt)
    deng = np.zeros((N, 1), np.float32)
    perr = np.zeros((N, 1), adt) if ray_error is not None else None
    stats = np.zeros(nr, STATS_DTYPE) if want_stats else None

    def opt(a, dt):
        return None if a is None else _c(a, dt).reshape(-1)

    lib().or_trace_bwd(
        _i(1 if f16 else 0), _p(points), _p(diffuse), _p(specular), _i(diff_res), _i(spec_res), _p(density),
        _p(adjacency), _p(offsets), _p(adj_diff), _p(rays), _u(nr), _p(start), _p(opt(rgba, adt)),
        _p(opt(rgba_grad, adt)), _u(K), _p(dq), _p(di), _p(dg), _p(opt(ray_error, adt)),
        _f(contribution_alpha_grad), _p(opt(distortion, np.float32)), _p(opt(distortion_grad, np.float32)),
        _p(opt(W_total, np.float32)), _p(opt(S_total, np.float32)), _p(opt(t_far, np.float32)),
        _f(weight_threshold), _u(max_intersections), _p(pg), _p(dgd), _p(sgd), _p(deng), _p(perr), _p(stats),
        _i(threads))
    return dict(points_grad=pg, diffuse_grad=dgd, specular_grad=sgd, density_grad=deng, point_error=perr,
                stats=stats)


def b_alg_infer(stats, tex_bytes=64, perm=False):
    """Algorithmic bytes of the inference walk summed from per-ray stats (8 B/face record)."""
    s = stats
    per_ray = 24 + 4 + 12 + 8 + (4 if perm else 0)
    return int(per_ray * len(s) + 8 * s["visits"].sum(dtype=np.int64) + 8 * s["faces"].sum(dtype=np.int64)
               + 16 * s["exits"].sum(dtype=np.int64) + 4 * s["integrated"].sum(dtype=np.int64)
               + tex_bytes * s["shaded"].sum(dtype=np.int64))


# --------------------------------------------------------------------------
# camera rays


def sincos(x, cos=False):
    x = _c(np.atleast_1d(x), np.float32)
    y = np.empty_like(x)
    lib().or_sincos_many(_i(1 if cos else 0), _p(x), _p(y), _sz(x.size))
    return y


def camera_rays(packed: bytes, num_images: int, H: int, W: int):
    """or_camera_rays over packed vt_camera records (100 bytes each): rays f32
    (num_images, H, W, 6), direction not normalised."""
    assert len(packed) == 100 * num_images
    buf = C.create_string_buffer(packed, len(packed))
    out = np.empty((num_images, H, W, 6), np.float32)
    lib().or_camera_rays(C.cast(buf, C.c_void_p), _u(num_images), _u(H), _u(W), _p(out))
    return out
