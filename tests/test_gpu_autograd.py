"""GPU tests of the training autograd Functions (ops.TraceVoroTracing,
train.FusedTraceVoroTracing) against direct _C backward calls, for the
backward semantics of _wrapper.py:95-231: the contribution gradient enters as
the scalar max |dL/dcontribution| on every ray's alpha gradient; a per-cell
distortion gate splits the backward into a distortion-only launch (its density
gradient NaN-cleaned and weighted per cell) and a launch for everything else;
point_error comes back through the error box; absent gradients are zero."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from vorotracing_amd import _C, camera
from vorotracing_amd.model import VoroTracing
from vorotracing_amd.train import fused_forward

pytestmark = pytest.mark.gpu


def _setup(gpu):
    s = H.small_random(900, seed=11, R=4)
    rays = H.to_dev(camera.pinhole_rays(40, 32, eye=(0.2, -3.4, 0.3)), gpu)
    return s, rays


def _direct(model, rays, rgba, dist, W, S, tf, g_rgba, g_dist=None, ray_error=None, cag=0.0):
    sp = model.get_starting_point(rays)
    return _C.trace_vorotracing_bwd(model.primal_points.detach(), model.att_diffuse.detach(),
                                    model.att_specular.detach(), model.activated_density().detach(),
                                    model.point_adjacency, model.point_adjacency_offsets, rays, sp, rgba, g_rgba, None,
                                    None, None, ray_error, cag, dist, g_dist, W, S, tf, 0.001, 1024)


def _fwd_outputs(model, rays):
    sp = model.get_starting_point(rays)
    out = _C.trace_vorotracing_fwd(model.primal_points.detach(), model.att_diffuse.detach(),
                                   model.att_specular.detach(), model.activated_density().detach(),
                                   model.point_adjacency, model.point_adjacency_offsets, rays, sp, None, 0.001, 1024,
                                   True)
    return out[0], out[5], out[6], out[7], out[8]


@pytest.mark.parametrize("fused", [False, True])
def test_contribution_gradient_is_the_max_scalar(gpu, fused):
    s, rays = _setup(gpu)
    model = VoroTracing.from_scene(s, device=gpu)
    rng = np.random.default_rng(3)
    g = torch.from_numpy(rng.normal(size=tuple(rays.shape[:-1]) + (4,)).astype(np.float32)).to(gpu)
    k = torch.from_numpy(rng.normal(size=(s.num_points, 1)).astype(np.float32)).to(gpu)
    run = fused_forward if fused else (lambda m, r, **kw: m(r, **kw))
    rgba, _, contrib, _, box, _ = run(model, rays, return_contribution=True)
    ((rgba * g).sum() + (contrib * k).sum()).backward()
    rgba0, dist, W, S, tf = _fwd_outputs(model, rays)
    want = _direct(model, rays, rgba0, dist, W, S, tf, g, cag=float(k.abs().max()))
    torch.cuda.synchronize()
    H.assert_grad_close(model.primal_points.grad.cpu().numpy(), want[0].cpu().numpy(), "points")
    H.assert_grad_close(model.att_diffuse.grad.cpu().numpy(), want[1].cpu().numpy(), "diffuse")
    dens = model.activated_density().detach()
    H.assert_grad_close(model.density.grad.cpu().numpy(), (want[3] * dens).cpu().numpy(), "raw density")
    assert box.point_error is None


@pytest.mark.parametrize("fused", [False, True])
def test_distortion_gate_splits_the_backward(gpu, fused):
    s, rays = _setup(gpu)
    model = VoroTracing.from_scene(s, device=gpu)
    rng = np.random.default_rng(4)
    lead = tuple(rays.shape[:-1])
    g = torch.from_numpy(rng.normal(size=lead + (4,)).astype(np.float32)).to(gpu)
    gd = torch.from_numpy(rng.uniform(0, 1, size=lead + (1,)).astype(np.float32)).to(gpu)
    err = torch.from_numpy(rng.uniform(0, 1, size=lead).astype(np.float32)).to(gpu)
    gate = torch.from_numpy(rng.uniform(0, 2, size=(s.num_points,)).astype(np.float32)).to(gpu)
    run = fused_forward if fused else (lambda m, r, **kw: m(r, **kw))
    rgba, _, _, _, box, dist_out = run(model, rays)
    box.cell_distortion_gate = gate
    box.ray_error = err
    ((rgba * g).sum() + (dist_out * gd).sum()).backward()
    rgba0, dist, W, S, tf = _fwd_outputs(model, rays)
    main = _direct(model, rays, rgba0, dist, W, S, tf, g, torch.zeros_like(gd), ray_error=err)
    only = _direct(model, rays, rgba0, dist, W, S, tf, torch.zeros_like(g), gd)
    torch.cuda.synchronize()
    want_s = main[3] + gate.reshape(-1, 1) * torch.nan_to_num(only[3], nan=0.0, posinf=0.0, neginf=0.0)
    dens = model.activated_density().detach()
    H.assert_grad_close(model.density.grad.cpu().numpy(), (want_s * dens).cpu().numpy(), "raw density")
    H.assert_grad_close(model.primal_points.grad.cpu().numpy(), main[0].cpu().numpy(), "points")
    H.assert_grad_close(model.att_specular.grad.cpu().numpy(), main[2].cpu().numpy(), "specular")
    H.assert_grad_close(box.point_error.cpu().numpy(), main[5].cpu().numpy(), "point_error")
    # without the gate the distortion gradient goes through the one launch
    ungated = _direct(model, rays, rgba0, dist, W, S, tf, g, gd, ray_error=err)
    torch.cuda.synchronize()
    assert not torch.allclose(ungated[3], want_s, rtol=1e-3, atol=1e-6)


def test_missing_rgba_gradient_is_zero(gpu):
    s, rays = _setup(gpu)
    model = VoroTracing.from_scene(s, device=gpu)
    gd = torch.rand(tuple(rays.shape[:-1]) + (1,), device=gpu)
    _, _, _, _, _, dist_out = model(rays)
    (dist_out * gd).sum().backward()
    rgba0, dist, W, S, tf = _fwd_outputs(model, rays)
    want = _direct(model, rays, rgba0, dist, W, S, tf, torch.zeros_like(rgba0), gd)
    torch.cuda.synchronize()
    H.assert_grad_close(model.primal_points.grad.cpu().numpy(), want[0].cpu().numpy(), "points")
    assert not model.att_diffuse.grad.any()


@pytest.mark.parametrize("fused", [False, True])
def test_retained_graph_backward_twice_doubles(gpu, fused):
    """A graph kept with retain_graph=True runs backward again with the same
    record: every gradient is accumulated twice (the reference keeps its ctx
    state for the same reason, _wrapper.py:39-84)."""
    s, rays = _setup(gpu)
    model = VoroTracing.from_scene(s, device=gpu)
    rng = np.random.default_rng(5)
    g = torch.from_numpy(rng.normal(size=tuple(rays.shape[:-1]) + (4,)).astype(np.float32)).to(gpu)
    run = fused_forward if fused else (lambda m, r, **kw: m(r, **kw))
    rgba, *_ = run(model, rays)
    loss = (rgba * g).sum()
    loss.backward(retain_graph=True)
    once = [p.grad.clone() for p in (model.primal_points, model.att_diffuse, model.att_specular, model.density)]
    loss.backward(retain_graph=True)
    torch.cuda.synchronize()
    for name, p, g1 in zip(("points", "diffuse", "specular", "density"),
                           (model.primal_points, model.att_diffuse, model.att_specular, model.density), once):
        assert g1.abs().max() > 0, name
        H.assert_grad_close(p.grad.cpu().numpy(), (2 * g1).cpu().numpy(), name)
    # torch.autograd.grad through the same retained graph again
    again = torch.autograd.grad(loss, [model.att_diffuse])
    torch.cuda.synchronize()
    H.assert_grad_close(again[0].cpu().numpy(), once[1].cpu().numpy(), "diffuse (autograd.grad)")
