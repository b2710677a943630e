"""Fused training-step pieces around the traversal backward.

* ``FusedTraceVoroTracing``: ``TraceVoroTracing`` (_wrapper.py:22-231) taking
  the raw log-density; its backward cleans the four gradients
  (nan_to_num, _wrapper.py:189-198) and applies the activation chain of
  s = a * exp(raw) (vorotracing.py:346-347) in one launch
  (vt_grad_epilogue) instead of five torch passes plus autograd's two.
* ``FusedVoroAdam``: the trainer's optimizer step (trainer.py:233-265): the
  manual specular and diffuse-mean-pull regulariser gradients,
  ``torch.optim.Adam(eps=1e-15)`` over the four parameter groups and the
  log-density clamp, in one launch (vt_adam_voro).  It keeps torch's
  ``param_groups`` (with "name" and "lr") so the trainer's learning-rate
  schedule (trainer.py:547-565) drives it unchanged.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional

import torch

from . import _lib, autograd, native


class FusedTraceVoroTracing(torch.autograd.Function):
    """TraceVoroTracing on the raw log-density: the forward activates it as
    s = a * exp(raw) (vorotracing.py:346-347, the same two torch operations,
    so the kernel sees the same bits), the backward plans its launches with
    ``autograd.scene_gradients`` and finishes all four gradients in one
    launch: NaN cleaning plus d/draw = (dL/ds * a) * exp(raw)."""

    @staticmethod
    def forward(ctx, points, diffuse, specular, density_raw, activation_scale: float, adjacency, offsets, rays,
                start_point, depth_quantiles, weight_threshold: float, max_intersections: int,
                return_contribution: bool):
        e = torch.exp(density_raw)
        density = activation_scale * e
        outputs, ctx.record = autograd.run_forward((points, diffuse, specular, density, adjacency, offsets), rays,
                                                   start_point, depth_quantiles, weight_threshold, max_intersections,
                                                   return_contribution)
        ctx.exp_raw = e
        ctx.activation_scale = float(activation_scale)
        return outputs

    @staticmethod
    def backward(ctx, grad_rgba, grad_depth, grad_contribution, _grad_n, _grad_box, grad_distortion):
        rec, e = ctx.record, ctx.exp_raw  # kept on ctx: a retained graph can run backward again
        up = autograd.upstream_of(rec, grad_rgba, grad_depth, grad_contribution, grad_distortion)
        pg, dg, sg, ds = autograd.scene_gradients(rec, up)
        raw_grad = torch.empty_like(e)
        ds = ds.contiguous()
        _lib.call("vt_grad_epilogue", pg.data_ptr(), pg.numel(), dg.data_ptr(), dg.numel(), sg.data_ptr(),
                  sg.numel(), ds.data_ptr(), e.data_ptr(), ctx.activation_scale, e.numel(), raw_grad.data_ptr(),
                  native._s(e.device))
        return (pg, dg, sg, raw_grad, None, None, None, None, None, None, None, None, None)


def fused_forward(model, rays, start_point=None, depth_quantiles=None, weight_threshold: float = 0.001,
                  max_intersections: int = 1024, return_contribution: bool = False):
    """``VoroTracing.forward`` (vorotracing.py:365-419) through FusedTraceVoroTracing:
    same outputs; the density gradient arrives at ``model.density`` (raw)."""
    return FusedTraceVoroTracing.apply(model.primal_points, model.att_diffuse, model.att_specular, model.density,
                                       model.config.activation_scale, model.point_adjacency,
                                       model.point_adjacency_offsets, rays, model.start_cells(rays, start_point),
                                       depth_quantiles, weight_threshold, max_intersections, return_contribution)


class FusedVoroAdam:
    """Adam over the four VoroTracing parameter groups plus the trainer's
    regulariser gradients and density clamp (trainer.py:233-265, :503-527),
    one HIP launch per ``step()``.  ``param_groups`` mirror torch's (name,
    lr, params); ``state`` holds exp_avg / exp_avg_sq per parameter."""

    GROUPS = ("primal_points", "density", "att_diffuse", "att_specular")

    def __init__(self, model, lr_points: float, lr_density: float, lr_attributes: float, betas=(0.9, 0.999),
                 eps: float = 1e-15, specular_reg_weight: float = 0.0, diffuse_mean_pull_weight: float = 0.0,
                 density_max: Optional[float] = 30.0):
        self.model = model
        self.betas = (float(betas[0]), float(betas[1]))
        self.eps = float(eps)
        self.specular_reg_weight = float(specular_reg_weight)
        self.diffuse_mean_pull_weight = float(diffuse_mean_pull_weight)
        self.density_max = float("inf") if density_max is None else float(density_max)
        lrs = {"primal_points": lr_points, "density": lr_density, "att_diffuse": lr_attributes,
               "att_specular": lr_attributes}
        self.param_groups = [{"name": n, "lr": float(lrs[n]), "params": [getattr(model, n)]} for n in self.GROUPS]
        self.state = {}
        self.step_count = 0

    def zero_grad(self, set_to_none: bool = True):
        for g in self.param_groups:
            p = g["params"][0]
            if set_to_none:
                p.grad = None
            elif p.grad is not None:
                p.grad.zero_()

    def _buffers(self, p):
        st = self.state.get(p)
        if st is None:
            st = self.state[p] = {"exp_avg": torch.zeros_like(p), "exp_avg_sq": torch.zeros_like(p)}
        return st["exp_avg"], st["exp_avg_sq"]

    @torch.no_grad()
    def step(self):
        ps = [g["params"][0] for g in self.param_groups]
        for p in ps:
            if p.grad is None:
                p.grad = torch.zeros_like(p)
        self.step_count += 1
        bufs = [self._buffers(p) for p in ps]
        pts, den, dif, spe = ps
        (pm, pv), (dm, dv), (fm, fv), (sm, sv) = bufs
        res = self.model.config.oct_map_res
        sres = self.model.config.spec_oct_map_res
        lr = (C.c_double * 4)(*[float(g["lr"]) for g in self.param_groups])
        _lib.call("vt_adam_voro", pts.data_ptr(), pts.grad.data_ptr(), pm.data_ptr(), pv.data_ptr(), den.data_ptr(),
                  den.grad.data_ptr(), dm.data_ptr(), dv.data_ptr(), dif.data_ptr(), dif.grad.data_ptr(),
                  fm.data_ptr(), fv.data_ptr(), res, spe.data_ptr(), spe.grad.data_ptr(), sm.data_ptr(),
                  sv.data_ptr(), sres, pts.shape[0], C.cast(lr, C.c_void_p), self.betas[0], self.betas[1], self.eps,
                  self.step_count, self.specular_reg_weight, self.diffuse_mean_pull_weight, self.density_max,
                  native._s(pts.device))
