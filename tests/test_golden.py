"""Golden fixture tests/golden/scene300.npz (written by
tests/golden/make_golden.py): a 300-site scene, 32x24 rays and the oracle's
fp16 inference, fp32 training forward and backward outputs.

CPU: the oracle (one thread, so atomics add in ray order) reproduces every
array bit for bit.  GPU: the HIP path matches the visit sequences, the
inference alpha and the training forward outputs bit for bit, the inference
RGB within one fp16 ulp (its colour path uses hardware rsq/rcp/exp2), and the
gradients within 1e-3 of each tensor's largest magnitude."""
import os

import numpy as np
import pytest
import torch

from oracle import core, host_ops

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "scene300.npz")


def _load():
    z = np.load(GOLD, allow_pickle=False)
    g = {k: z[k] for k in z.files}
    g["diffuse"] = g["diffuse"].astype(np.float32)
    g["specular"] = g["specular"].astype(np.float32)
    return g


def _oracle(g):
    thr = float(g["thr"])
    d4 = host_ops.pad_3to4(g["diffuse"].astype(np.float16), 4)
    s4 = host_ops.pad_3to4(g["specular"].astype(np.float16), 4)
    ad = core.prefetch_adj(g["points"], g["adjacency"], g["offsets"], threads=1)
    args = (g["points"],)
    rgba16, st, _ = core.trace_infer_f16(g["points"], d4, s4, 4, 4, g["density"], g["adjacency"], g["offsets"], ad,
                                         g["rays"], g["start"], weight_threshold=thr, cell_skip_threshold=1e-3,
                                         want_stats=True, threads=1)
    fw = core.trace_fwd(*args, g["diffuse"], g["specular"], 4, 4, g["density"], g["adjacency"], g["offsets"],
                        g["rays"], g["start"], depth_quantiles=g["quantiles"], weight_threshold=thr,
                        return_contribution=True, threads=1)
    bw = core.trace_bwd(*args, g["diffuse"], g["specular"], 4, 4, g["density"], g["adjacency"], g["offsets"],
                        g["rays"], g["start"], fw["rgba"], g["rgba_grad"], distortion=fw["distortion"],
                        W_total=fw["W_total"], S_total=fw["S_total"], t_far=fw["t_far"], weight_threshold=thr,
                        threads=1)
    return rgba16, st, fw, bw


FWD_KEYS = (("fwd_rgba", "rgba"), ("fwd_n", "n"), ("fwd_depth", "depth"), ("fwd_depth_idx", "depth_idx"),
            ("fwd_distortion", "distortion"), ("fwd_W", "W_total"), ("fwd_S", "S_total"), ("fwd_t_far", "t_far"))
BWD_KEYS = (("bwd_points_grad", "points_grad"), ("bwd_density_grad", "density_grad"),
            ("bwd_diffuse_grad", "diffuse_grad"), ("bwd_specular_grad", "specular_grad"))


def _bits(a):
    a = np.ascontiguousarray(a)
    return a.view(np.uint32) if a.dtype.itemsize == 4 else a.view(np.uint16)


def test_oracle_reproduces_golden():
    g = _load()
    rgba16, st, fw, bw = _oracle(g)
    assert np.array_equal(rgba16.view(np.uint16), g["infer_rgba_bits"])
    assert np.array_equal(st["n"], g["infer_n"])
    assert np.array_equal(st["visits"], g["infer_visits"])
    assert np.array_equal(st["visit_hash"], g["infer_hash"])
    for gk, k in FWD_KEYS:
        assert np.array_equal(_bits(fw[k]), _bits(g[gk])), k
    assert np.array_equal(_bits(fw["contribution"]), _bits(g["fwd_contribution"]))
    for gk, k in BWD_KEYS:
        assert np.array_equal(_bits(bw[k]), _bits(g[gk])), k


def _rel(got, want):
    want = np.asarray(want, np.float64)
    return float(np.abs(np.asarray(got, np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


@pytest.mark.gpu
def test_gpu_matches_golden(gpu):
    from tests import helpers as H
    from vorotracing_amd import _C, native

    g = _load()
    thr = float(g["thr"])
    d = lambda a: H.to_dev(a, gpu)  # noqa: E731
    pts, den, adj, off = d(g["points"]), d(g["density"]), d(g["adjacency"]), d(g["offsets"])
    rays, start = d(g["rays"]), d(g["start"])
    # fp16 inference
    ad = native.prefetch(pts, adj, off)
    d4 = d(host_ops.pad_3to4(g["diffuse"].astype(np.float16), 4))
    s4 = d(host_ops.pad_3to4(g["specular"].astype(np.float16), 4))
    st = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
    got = native.infer_f16(pts, d4, s4, den, adj, off, ad, rays, start, weight_threshold=thr,
                           cell_skip_threshold=1e-3, stats=st)
    torch.cuda.synchronize()
    s = H.stats_np(st)
    H.assert_infer_rgba(got, g["infer_rgba_bits"].view(np.float16))
    assert np.array_equal(s["visit_hash"], g["infer_hash"])
    assert np.array_equal(s["n"], g["infer_n"])
    # fp32 training forward and backward
    dif, spe = d(g["diffuse"]), d(g["specular"])
    rgba, depth, depth_idx, contrib, n, dist, W, S, tf = _C.trace_vorotracing_fwd(
        pts, dif, spe, den.view(-1, 1), adj, off, rays, start, d(g["quantiles"]), thr, 1024, True)
    out = dict(rgba=rgba, n=n, depth=depth, depth_idx=depth_idx, distortion=dist, W_total=W, S_total=S, t_far=tf)
    for gk, k in FWD_KEYS:
        assert np.array_equal(_bits(out[k].cpu().numpy()), _bits(g[gk])), k
    assert _rel(contrib.cpu().numpy(), g["fwd_contribution"]) <= 1e-5
    pg, dgd, sgd, deng, _, _ = _C.trace_vorotracing_bwd(
        pts, dif, spe, den.view(-1, 1), adj, off, rays, start, rgba, d(g["rgba_grad"]), None, None, None, None, 0.0,
        dist, None, W, S, tf, thr, 1024)
    torch.cuda.synchronize()
    for t, gk in ((pg, "bwd_points_grad"), (deng, "bwd_density_grad"), (dgd, "bwd_diffuse_grad"),
                  (sgd, "bwd_specular_grad")):
        assert _rel(t.cpu().numpy(), g[gk]) <= 1e-3, gk
