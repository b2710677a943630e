"""Autograd plumbing of the training traversal, shared by the two autograd
Functions (``ops.TraceVoroTracing`` on the activated density, and
``train.FusedTraceVoroTracing`` on the raw log-density).

A forward keeps one ``TraceRecord``: the scene tensors, rays, start cells and
the forward outputs the backward kernel re-reads.  A backward turns the
incoming gradients into an ``Upstream`` and asks ``scene_gradients`` for the
four scene gradients; each Function then finishes them its own way (in-place
``nan_to_num``, or the fused epilogue kernel).

Backward semantics kept from the reference (_wrapper.py:95-231, behaviour
only; see the citations per function):
- the contribution output has no true gradient: its upstream gradient
  enters as one scalar, max |dL/dcontribution|, added to every ray's alpha
  gradient (_wrapper.py:113-117, tracing_octmap.cu:281);
- a missing rgba gradient is zero;
- when the caller has set a per-cell ``cell_distortion_gate`` on the error
  box and a distortion gradient arrives, the distortion term's density
  gradient is computed by a backward of its own, NaN-cleaned, weighted per
  cell by the gate and added to the density gradient of a backward that
  carries everything else (_wrapper.py:145-170);
- ``point_error`` is handed back through the error box (_wrapper.py:187).
"""
from __future__ import annotations

import dataclasses
from typing import Iterator, Optional, Tuple

import torch

from . import _C


class ErrorBox:
    """Side channel between a training forward and its backward.  Its
    attribute names are the interface callers of the reference use
    (_wrapper.py:15-19, vorotracing.py:389): before backward a caller may set
    ``ray_error`` (per-ray weights of point_error) and
    ``cell_distortion_gate`` ((N,) or (N, 1) per-cell weights of the
    distortion term's density gradient); backward leaves ``point_error``
    ((N, 1), or None without ray_error)."""

    __slots__ = ("ray_error", "point_error", "cell_distortion_gate")

    def __init__(self):
        self.ray_error = None
        self.point_error = None
        self.cell_distortion_gate = None


@dataclasses.dataclass
class TraceRecord:
    scene: Tuple[torch.Tensor, ...]  # points, diffuse, specular, activated density, adjacency, offsets
    rays: torch.Tensor
    start: torch.Tensor
    quantiles: Optional[torch.Tensor]
    weight_threshold: float
    max_intersections: int
    rgba: torch.Tensor
    depth_idx: Optional[torch.Tensor]
    distortion: torch.Tensor
    totals: Tuple[torch.Tensor, torch.Tensor, torch.Tensor]  # W_total, S_total, t_far
    box: ErrorBox
    perm: Optional[torch.Tensor] = None  # lane order of the forward, reused by the backward
    adj_diff: Optional[torch.Tensor] = None  # the forward's face-offset prefetch, reused by the backward


@dataclasses.dataclass
class Upstream:
    """Incoming gradients in the form one backward launch takes."""
    rgba: torch.Tensor
    depth: Optional[torch.Tensor]
    distortion: Optional[torch.Tensor]
    ray_error: Optional[torch.Tensor]
    alpha_scalar: float


def run_forward(scene, rays, start, quantiles, weight_threshold: float, max_intersections: int,
                want_contribution: bool):
    """One _C.trace_vorotracing_fwd; returns the six autograd outputs
    (rgba, depth, contribution, n, error box, distortion, as
    _wrapper.py:87) and the record a backward needs."""
    perm = _C.default_ray_perm(rays, start, scene[0].shape[0])
    adjacency = scene[4]
    ad = None
    if rays.is_cuda:
        ad = torch.empty((adjacency.shape[0] + 32, 4), dtype=torch.float16, device=rays.device)
    rgba, depth, depth_idx, contribution, n, distortion, w_tot, s_tot, t_far = _C.trace_vorotracing_fwd(
        *scene, rays, start, quantiles, weight_threshold, max_intersections, want_contribution, ray_perm=perm,
        adj_diff_out=ad)
    box = ErrorBox()
    rec = TraceRecord(tuple(scene), rays, start, quantiles, float(weight_threshold), int(max_intersections), rgba,
                      depth_idx, distortion, (w_tot, s_tot, t_far), box, perm, ad)
    return (rgba, depth, contribution, n, box, distortion), rec


def upstream_of(rec: TraceRecord, grad_rgba, grad_depth, grad_contribution, grad_distortion) -> Upstream:
    alpha_scalar = 0.0
    if grad_contribution is not None:
        alpha_scalar = float(grad_contribution.detach().abs().max().item())
    rgba = grad_rgba if grad_rgba is not None else torch.zeros_like(rec.rgba)
    return Upstream(rgba, grad_depth, grad_distortion, rec.box.ray_error, alpha_scalar)


def _launches(rec: TraceRecord, up: Upstream) -> Iterator[Tuple[Upstream, Optional[torch.Tensor]]]:
    """The backward launches for ``up``: (upstream, per-cell weight of the
    launch's density gradient), the first launch's weight None (it gives
    all four gradients and point_error); a gated distortion term gets a
    launch of its own that contributes a weighted density gradient only."""
    gate = rec.box.cell_distortion_gate
    if gate is None or up.distortion is None:
        yield up, None
        return
    yield dataclasses.replace(up, distortion=torch.zeros_like(up.distortion)), None
    yield Upstream(torch.zeros_like(up.rgba), None, up.distortion, None, 0.0), gate


def _launch(rec: TraceRecord, up: Upstream):
    w_tot, s_tot, t_far = rec.totals
    return _C.trace_vorotracing_bwd(*rec.scene, rec.rays, rec.start, rec.rgba, up.rgba, rec.quantiles, rec.depth_idx,
                                    up.depth, up.ray_error, up.alpha_scalar, rec.distortion, up.distortion, w_tot,
                                    s_tot, t_far, rec.weight_threshold, rec.max_intersections, ray_perm=rec.perm,
                                    adj_diff=rec.adj_diff)


def scene_gradients(rec: TraceRecord, up: Upstream):
    """Gradients (points, diffuse, specular, density) of the loss for the
    record's scene, before NaN cleaning; stores point_error in the error box."""
    grads = None
    for u, weight in _launches(rec, up):
        pg, dg, sg, deng, _ray_grad, perr = _launch(rec, u)
        if weight is None:
            grads = [pg, dg, sg, deng]
            rec.box.point_error = perr
        else:
            deng = torch.nan_to_num(deng, nan=0.0, posinf=0.0, neginf=0.0)
            grads[3] = grads[3] + weight.reshape_as(deng) * deng
    return grads


def clean_(grads):
    """NaN and infinities to zero, in place (_wrapper.py:189-198)."""
    for g in grads:
        torch.nan_to_num(g, nan=0.0, posinf=0.0, neginf=0.0, out=g)
    return grads
