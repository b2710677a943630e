"""GPU parity of the fused training-step pieces (vorotracing_amd/train.py)
against the torch sequence they replace:
- vt_grad_epilogue: nan_to_num of the gradients and autograd's chain through
  s = a * exp(raw), bit for bit;
- FusedTraceVoroTracing: gradients identical to TraceVoroTracing + autograd;
- FusedVoroAdam: torch.optim.Adam (eps 1e-15) with the trainer's regulariser
  gradients and density clamp (trainer.py:233-265), to float tolerance (the
  per-cell mean and Adam's operations round in a different order)."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from vorotracing_amd import _lib, camera, native
from vorotracing_amd.model import VoroTracing, VoroTracingConfig
from vorotracing_amd.train import FusedTraceVoroTracing, FusedVoroAdam, fused_forward

pytestmark = pytest.mark.gpu


def test_grad_epilogue_bit_exact(gpu):
    rng = np.random.default_rng(0)
    n = 5000

    def noisy(shape):
        x = rng.normal(size=shape).astype(np.float32) * 10
        flat = x.reshape(-1)
        k = flat.size // 50
        flat[rng.choice(flat.size, k, replace=False)] = np.nan
        flat[rng.choice(flat.size, k, replace=False)] = np.inf
        flat[rng.choice(flat.size, k, replace=False)] = -np.inf
        flat[rng.choice(flat.size, k, replace=False)] = -0.0
        return torch.from_numpy(x).to(gpu)

    pg, dg, sg, gs = noisy((n, 3)), noisy((n, 48)), noisy((n, 48)), noisy((n, 1))
    raw = torch.from_numpy(rng.normal(size=(n, 1)).astype(np.float32) * 3).to(gpu)
    e = torch.exp(raw)
    for a in (1.0, 0.37):
        want = [torch.nan_to_num(t, nan=0.0, posinf=0.0, neginf=0.0) for t in (pg, dg, sg, gs)]
        want_raw = (want[3] * a) * e
        got = [t.clone() for t in (pg, dg, sg)]
        graw = torch.empty_like(e)
        _lib.call("vt_grad_epilogue", got[0].data_ptr(), got[0].numel(), got[1].data_ptr(), got[1].numel(),
                  got[2].data_ptr(), got[2].numel(), gs.data_ptr(), e.data_ptr(), a, n, graw.data_ptr(),
                  native._s(gpu))
        torch.cuda.synchronize()
        for x, y in zip(got, want[:3]):
            assert torch.equal(x.view(torch.int32), y.view(torch.int32))
        assert torch.equal(graw.view(torch.int32), want_raw.view(torch.int32))


def _small_model(gpu, res=4, sres=4, seed=7):
    s = H.small_random(600, seed=seed, R=res, Rs=sres)
    cfg = VoroTracingConfig(oct_map_res=res, spec_oct_map_res=sres, activation_scale=1.0)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    return VoroTracing(cfg, t(s.points), t(s.diffuse.astype(np.float32)), t(s.specular.astype(np.float32)),
                       t(s.density_raw.astype(np.float32)), t(s.adjacency.view(np.int32)), t(s.offsets.view(np.int32)),
                       device=gpu)


def test_fused_forward_backward_equals_autograd(gpu):
    m1, m2 = _small_model(gpu), _small_model(gpu)
    rays = H.to_dev(camera.pinhole_rays(64, 48, eye=(0.3, -3.5, 0.5)), gpu)
    g = torch.from_numpy(np.random.default_rng(1).normal(size=(48, 64, 4)).astype(np.float32)).to(gpu)
    out1 = m1(rays, weight_threshold=0.001)
    out2 = fused_forward(m2, rays, weight_threshold=0.001)
    assert torch.equal(out1[0], out2[0])
    out1[0].backward(g)
    out2[0].backward(g)
    torch.cuda.synchronize()
    for name in ("primal_points", "att_diffuse", "att_specular", "density"):
        a, b = getattr(m1, name).grad, getattr(m2, name).grad
        assert a.shape == b.shape
        # atomics add in a run-dependent order: compare to the tensor's scale
        assert (a - b).abs().max() <= 1e-5 * max(float(a.abs().max()), 1e-30), name
        assert a.isfinite().all() and b.isfinite().all()


def _reference_step(model, opt, step, spec_w, pull_w, lrs):
    """trainer.py:233-265 with torch's Adam (the regulariser gradients as the trainer writes them)."""
    if spec_w > 0:
        spec = model.att_specular
        spec.grad.add_(spec.data, alpha=2.0 * spec_w / spec.numel())
    if pull_w > 0:
        R = model.config.oct_map_res
        diff = model.att_diffuse.data.reshape(-1, R, R, 3)
        grad = model.att_diffuse.grad.reshape(-1, R, R, 3)
        mean = diff.mean(dim=(1, 2), keepdim=True)
        scale = 2.0 * pull_w / diff.numel()
        grad.add_(diff, alpha=scale)
        grad.add_(mean, alpha=-scale)
    for gr, lr in zip(opt.param_groups, lrs):
        gr["lr"] = lr
    opt.step()
    with torch.no_grad():
        model.density.clamp_(max=30.0)


@pytest.mark.parametrize("res,sres,fused_torch", [(4, 4, False), (8, 4, True)])
def test_fused_adam_matches_torch(gpu, res, sres, fused_torch):
    ref, fus = _small_model(gpu, res, sres), _small_model(gpu, res, sres)
    names = ("primal_points", "density", "att_diffuse", "att_specular")
    lr0 = (2e-4, 1e-1, 2e-2, 2e-2)
    topt = torch.optim.Adam([{"params": getattr(ref, n), "lr": lr, "name": n} for n, lr in zip(names, lr0)],
                            eps=1e-15, fused=fused_torch)
    fopt = FusedVoroAdam(fus, *lr0[:3], specular_reg_weight=1e-2, diffuse_mean_pull_weight=0.5)
    rng = np.random.default_rng(3)
    with torch.no_grad():  # push some log-densities near the clamp
        ref.density[:20] = 29.9
        fus.density[:20] = 29.9
    for step in range(1, 5):
        lrs = [lr * (0.9 ** step) for lr in lr0]
        for n in names:
            g = torch.from_numpy(rng.normal(size=tuple(getattr(ref, n).shape)).astype(np.float32)).to(gpu)
            getattr(ref, n).grad = g.clone()
            getattr(fus, n).grad = g.clone()
        _reference_step(ref, topt, step, 1e-2, 0.5, lrs)
        for gr, lr in zip(fopt.param_groups, lrs):
            gr["lr"] = lr
        fopt.step()
    torch.cuda.synchronize()
    assert float(fus.density.max()) <= 30.0
    for n in names:
        a, b = getattr(ref, n).detach(), getattr(fus, n).detach()
        scale = float(a.abs().max())
        assert (a - b).abs().max() <= 2e-6 * scale, (n, float((a - b).abs().max()), scale)
        st_t, st_f = topt.state[getattr(ref, n)], fopt.state[getattr(fus, n)]
        for k in ("exp_avg", "exp_avg_sq"):
            x, y = st_t[k], st_f[k]
            assert (x - y).abs().max() <= 1e-5 * float(x.abs().max()), (n, k)


def test_fused_adam_argument_errors(gpu):
    m = _small_model(gpu)
    opt = FusedVoroAdam(m, 1e-4, 1e-1, 1e-2)
    m.config.oct_map_res = 5
    with pytest.raises(_lib.VTError, match="diffuse resolution"):
        opt.step()
