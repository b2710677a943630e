"""Operator surface of the reference's ``vorotracing.cuda`` package
(cuda/__init__.py:49-57, _wrapper.py), backed by the HIP library.

``TraceVoroTracing`` is the training autograd Function (_wrapper.py:22-231),
``trace_octmap_infer`` / ``trace_octmap_infer_q8`` / ``prefetch_octmap_adj``
the inference wrappers (_wrapper.py:234-307), ``NNBVH`` /
``nearest_neighbor_bvh`` the start-cell lookup (nn_bvh.h), and
``build_voronoi_adjacency`` the CSR adapter (cuda/__init__.py:16-46) with the
host Delaunay (qhull) standing in for Paragram.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import _C, _lib

NNBVH = _C.NNBVH
nearest_neighbor_bvh = _C.nearest_neighbor_bvh


class ErrorBox:
    def __init__(self):
        self.ray_error = None
        self.point_error = None
        self.cell_distortion_gate = None


class TraceVoroTracing(torch.autograd.Function):
    """_wrapper.py:22-231: forward through _C.trace_vorotracing_fwd, backward
    through _C.trace_vorotracing_bwd, gradients for points, diffuse,
    specular and density (nan_to_num'd)."""

    @staticmethod
    def forward(ctx, _points, _diffuse, _specular, _density, _point_adjacency, _point_adjacency_offsets, rays,
                start_point, depth_quantiles, weight_threshold: float, max_intersections: int,
                return_contribution: bool):
        ctx.rays = rays
        ctx.start_point = start_point
        ctx.depth_quantiles = depth_quantiles
        ctx.weight_threshold = weight_threshold
        ctx.max_intersections = max_intersections
        ctx.points = _points
        ctx.diffuse = _diffuse
        ctx.specular = _specular
        ctx.density = _density
        ctx.point_adjacency = _point_adjacency
        ctx.point_adjacency_offsets = _point_adjacency_offsets
        (rgba, depth, depth_indices, contribution, num_intersections, distortion, W_total, S_total,
         t_far) = _C.trace_vorotracing_fwd(_points, _diffuse, _specular, _density, _point_adjacency,
                                          _point_adjacency_offsets, rays, start_point, depth_quantiles,
                                          weight_threshold, max_intersections, return_contribution)
        ctx.rgba = rgba
        ctx.depth_indices = depth_indices
        ctx.distortion = distortion
        ctx.W_total = W_total
        ctx.S_total = S_total
        ctx.t_far = t_far
        errbox = ErrorBox()
        ctx.errbox = errbox
        return rgba, depth, contribution, num_intersections, errbox, distortion

    @staticmethod
    def backward(ctx, grad_rgba, grad_depth, grad_contribution, grad_num_intersections, errbox_grad,
                 grad_distortion):
        del grad_num_intersections, errbox_grad
        contribution_alpha_grad = 0.0
        if grad_contribution is not None:
            contribution_alpha_grad = float(grad_contribution.detach().abs().max().item())

        def _bwd(grad_rgba_, grad_depth_, ray_error_, contrib_, grad_distortion_):
            return _C.trace_vorotracing_bwd(
                ctx.points, ctx.diffuse, ctx.specular, ctx.density, ctx.point_adjacency,
                ctx.point_adjacency_offsets, ctx.rays, ctx.start_point, ctx.rgba, grad_rgba_, ctx.depth_quantiles,
                ctx.depth_indices, grad_depth_, ray_error_, contrib_, ctx.distortion, grad_distortion_,
                ctx.W_total, ctx.S_total, ctx.t_far, ctx.weight_threshold, ctx.max_intersections)

        if grad_rgba is None:
            grad_rgba = torch.zeros_like(ctx.rgba)
        cell_gate = getattr(ctx.errbox, "cell_distortion_gate", None)
        if cell_gate is not None and grad_distortion is not None:
            res_d = _bwd(torch.zeros_like(grad_rgba), None, None, 0.0, grad_distortion)
            density_grad_dist = res_d[3]
            points_grad, diffuse_grad, specular_grad, density_grad, _ray_grad, point_error = _bwd(
                grad_rgba, grad_depth, ctx.errbox.ray_error, contribution_alpha_grad,
                torch.zeros_like(grad_distortion))
            torch.nan_to_num(density_grad_dist, nan=0.0, posinf=0.0, neginf=0.0, out=density_grad_dist)
            density_grad = density_grad + cell_gate.reshape_as(density_grad) * density_grad_dist
        else:
            points_grad, diffuse_grad, specular_grad, density_grad, _ray_grad, point_error = _bwd(
                grad_rgba, grad_depth, ctx.errbox.ray_error, contribution_alpha_grad, grad_distortion)
        ctx.errbox.point_error = point_error
        for g in (points_grad, diffuse_grad, specular_grad, density_grad):
            torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=0.0, out=g)
        return (points_grad, diffuse_grad, specular_grad, density_grad, None, None, None, None, None, None, None,
                None)


def prefetch_octmap_adj(points, adjacency, offsets):
    return _C.trace_vorotracing_prefetch_adj(points, adjacency, offsets)


def trace_octmap_infer(points, diffuse_fp16, specular_fp16, density, adjacency, offsets, rays, start_point,
                       adjacent_diff, ray_perm, weight_threshold=0.001, max_intersections=1024,
                       cell_skip_threshold=0.0):
    return _C.trace_vorotracing_infer(points, diffuse_fp16, specular_fp16, density, adjacency, offsets, rays,
                                      start_point, adjacent_diff, ray_perm, weight_threshold, max_intersections,
                                      cell_skip_threshold)


def trace_octmap_infer_q8(points, diffuse_q8, specular_q8, density, adjacency, offsets, rays, start_point,
                          adjacent_diff, diff_scale, diff_offset, spec_scale, spec_offset, weight_threshold=0.001,
                          max_intersections=1024, cell_skip_threshold=0.0):
    return _C.trace_vorotracing_infer_q8(points, diffuse_q8, specular_q8, density, adjacency, offsets, rays,
                                         start_point, adjacent_diff, diff_scale, diff_offset, spec_scale,
                                         spec_offset, weight_threshold, max_intersections, cell_skip_threshold)


def build_voronoi_adjacency(points: torch.Tensor, *, debug: bool = False, initial_guesses=None,
                            initial_guesses_offsets=None, chunk_padding: int = 32):
    """cuda/__init__.py:16-46: uint32 CSR (adjacency padded by ``chunk_padding``
    zeros, offsets) and a status tensor, built on the GPU by vt_voronoi_build
    (the reference calls Paragram).  Each neighbour list is ascending; the
    sets are the Delaunay neighbours of the sites.  ``initial_guesses`` are
    accepted for signature compatibility and not needed."""
    del debug, initial_guesses, initial_guesses_offsets
    import ctypes

    pts = points.detach().to(torch.float32).contiguous()
    dev = pts.device
    if dev.type != "cuda":
        raise RuntimeError("build_voronoi_adjacency needs the sites on the GPU")
    n = pts.shape[0]
    lib = _lib.load()
    ws = torch.empty(lib.vt_voronoi_workspace_size(n), dtype=torch.uint8, device=dev)
    offsets = torch.empty(n + 1, dtype=torch.uint32, device=dev)
    m = ctypes.c_uint32(0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    with torch.cuda.device(dev):
        _lib.call("vt_voronoi_build", pts.data_ptr(), n, offsets.data_ptr(), ctypes.addressof(m), ws.data_ptr(),
                  stream)
        adjacency = torch.zeros(m.value + chunk_padding, dtype=torch.uint32, device=dev)
        _lib.call("vt_voronoi_adjacency", n, offsets.data_ptr(), adjacency.data_ptr(), ws.data_ptr(), stream)
    return adjacency, offsets, torch.zeros(1, dtype=torch.int32, device=dev)


__all__ = [
    "TraceVoroTracing",
    "trace_octmap_infer",
    "trace_octmap_infer_q8",
    "prefetch_octmap_adj",
    "build_voronoi_adjacency",
    "NNBVH",
    "nearest_neighbor_bvh",
]
