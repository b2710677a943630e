"""Operator surface of the reference's ``vorotracing.cuda`` package
(cuda/__init__.py:49-57, _wrapper.py), backed by the HIP library.

``TraceVoroTracing`` is the training autograd Function (_wrapper.py:22-231),
``trace_octmap_infer`` / ``trace_octmap_infer_q8`` / ``prefetch_octmap_adj``
the inference wrappers (_wrapper.py:234-307), ``NNBVH`` /
``nearest_neighbor_bvh`` the start-cell lookup (nn_bvh.h), and
``build_voronoi_adjacency`` the CSR adapter (cuda/__init__.py:16-46), built by
the GPU Voronoi builder where the reference calls Paragram.
"""
from __future__ import annotations

import torch

from . import _C, _lib, autograd
from .autograd import ErrorBox

NNBVH = _C.NNBVH
nearest_neighbor_bvh = _C.nearest_neighbor_bvh


class TraceVoroTracing(torch.autograd.Function):
    """Training traversal as an autograd Function (the operator of
    _wrapper.py:22-231): inputs and the six outputs (rgba, depth,
    contribution, n, error box, distortion) as the reference's; gradients
    reach points, diffuse, specular and the activated density, NaN-cleaned.
    The backward planning is ``autograd.scene_gradients``."""

    @staticmethod
    def forward(ctx, points, diffuse, specular, density, adjacency, offsets, rays, start_point, depth_quantiles,
                weight_threshold: float, max_intersections: int, return_contribution: bool):
        outputs, ctx.record = autograd.run_forward((points, diffuse, specular, density, adjacency, offsets), rays,
                                                   start_point, depth_quantiles, weight_threshold, max_intersections,
                                                   return_contribution)
        return outputs

    @staticmethod
    def backward(ctx, grad_rgba, grad_depth, grad_contribution, _grad_n, _grad_box, grad_distortion):
        # the record stays on ctx (as the reference keeps its state), so a graph
        # retained for a second backward gives the same gradients again
        rec = ctx.record
        up = autograd.upstream_of(rec, grad_rgba, grad_depth, grad_contribution, grad_distortion)
        grads = autograd.clean_(autograd.scene_gradients(rec, up))
        return (*grads, None, None, None, None, None, None, None, None)


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


def guess_csr(initial_guesses, initial_guesses_offsets, num_sites: int, device):
    """Checked warm-start CSR for ``build_voronoi_adjacency``: (offsets,
    adjacency) as contiguous uint32 on ``device``, or (None, None).  The
    offsets must have ``num_sites + 1`` non-decreasing entries that end
    within the guess list; ids themselves may be anything (out-of-range ids
    are skipped by the builder)."""
    if (initial_guesses is None) != (initial_guesses_offsets is None):
        raise ValueError("initial_guesses and initial_guesses_offsets are given together or not at all")
    if initial_guesses is None:
        return None, None
    gofs = torch.as_tensor(initial_guesses_offsets, device=device).reshape(-1)
    gadj = torch.as_tensor(initial_guesses, device=device).reshape(-1)
    if gofs.numel() != num_sites + 1:
        raise ValueError(f"initial_guesses_offsets must have {num_sites + 1} entries, got {gofs.numel()}")
    wide = gofs.to(torch.int64)
    if bool((wide < 0).any()) or bool((wide[1:] < wide[:-1]).any()):
        raise ValueError("initial_guesses_offsets must be non-negative and non-decreasing")
    last = int(wide[-1].item())
    if last > gadj.numel():
        raise ValueError(f"initial_guesses has {gadj.numel()} entries, its offsets end at {last}")
    gofs = wide.to(torch.uint32).contiguous() if gofs.dtype != torch.uint32 else gofs.contiguous()
    gadj = gadj.to(torch.int64).to(torch.uint32).contiguous() if gadj.dtype != torch.uint32 else gadj.contiguous()
    return gofs, gadj


def build_voronoi_adjacency(points: torch.Tensor, *, debug: bool = False, initial_guesses=None,
                            initial_guesses_offsets=None, chunk_padding: int = 32):
    """cuda/__init__.py:16-46: uint32 CSR (adjacency padded by ``chunk_padding``
    zeros, offsets) and a status tensor, built on the GPU by the Voronoi
    builder (the reference calls Paragram).  Each neighbour list is
    ascending; the sets are the Delaunay neighbours of the sites.
    ``initial_guesses`` / ``initial_guesses_offsets`` (a CSR over the same
    sites, e.g. the adjacency before the sites moved) warm-start the build;
    the result is the same, found faster when the guesses are close."""
    del debug
    import ctypes

    pts = points.detach().to(torch.float32).contiguous()
    dev = pts.device
    if dev.type != "cuda":
        raise RuntimeError("build_voronoi_adjacency needs the sites on the GPU")
    n = pts.shape[0]
    gofs, gadj = guess_csr(initial_guesses, initial_guesses_offsets, n, dev)
    lib = _lib.load()
    ws = torch.empty(lib.vt_voronoi_workspace_size(n), dtype=torch.uint8, device=dev)
    offsets = torch.empty(n + 1, dtype=torch.uint32, device=dev)
    m = ctypes.c_uint32(0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    with torch.cuda.device(dev):
        _lib.call("vt_voronoi_build_warm", pts.data_ptr(), n, None if gofs is None else gofs.data_ptr(),
                  None if gadj is None else gadj.data_ptr(), 0 if gadj is None else gadj.numel(), offsets.data_ptr(),
                  ctypes.addressof(m), ws.data_ptr(), stream)
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
