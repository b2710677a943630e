"""Writes tests/golden/scene300.npz: a small self-contained scene, rays, and
the oracle's outputs on them (fp16 inference, fp32 training forward and
backward).  The fixture freezes the restatement: tests check that the oracle
still reproduces it bit for bit and that the HIP kernels match it.

The reference has no golden vectors of its own for this path (its repository
holds no tests), so these are regression vectors of this build's oracle, made
on seeded synthetic inputs.  Regenerate only after a deliberate change of the
arithmetic convention:

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import core, host_ops  # noqa: E402
from vorotracing_amd import camera, scene  # noqa: E402

PATH = os.path.join(HERE, "scene300.npz")
THR = 0.005


def make():
    s = scene.random_scene(300, seed=11, R=4, extent=2.0)
    # texture logits on the fp16 grid, so the fixture stores them as halves
    s.diffuse = s.diffuse.astype(np.float16).astype(np.float32)
    s.specular = s.specular.astype(np.float16).astype(np.float32)
    rays = camera.pinhole_rays(32, 24, eye=(0.4, -3.5, 0.7)).astype(np.float32)
    start = host_ops.nearest_site(s.points, rays[0, 0, :3][None])[0]
    sp = np.full(rays.shape[:-1], start, np.uint32)
    d4, s4 = (host_ops.pad_3to4(s.diffuse.astype(np.float16), 4), host_ops.pad_3to4(s.specular.astype(np.float16), 4))
    ad = core.prefetch_adj(s.points, s.adjacency, s.offsets, threads=1)
    rgba16, st, _ = core.trace_infer_f16(s.points, d4, s4, 4, 4, s.density, s.adjacency, s.offsets, ad, rays, sp,
                                         weight_threshold=THR, cell_skip_threshold=1e-3, want_stats=True, threads=1)
    q = np.full(rays.shape[:-1] + (2,), [0.7, 0.2], np.float32)
    fw = core.trace_fwd(s.points, s.diffuse, s.specular, 4, 4, s.density, s.adjacency, s.offsets, rays, sp,
                        depth_quantiles=q, weight_threshold=THR, return_contribution=True, threads=1)
    g = np.random.default_rng(12).normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    bw = core.trace_bwd(s.points, s.diffuse, s.specular, 4, 4, s.density, s.adjacency, s.offsets, rays, sp,
                        fw["rgba"], g, distortion=fw["distortion"], W_total=fw["W_total"], S_total=fw["S_total"],
                        t_far=fw["t_far"], weight_threshold=THR, threads=1)
    return dict(
        points=s.points, density=s.density.reshape(-1), diffuse=s.diffuse.astype(np.float16),
        specular=s.specular.astype(np.float16),
        adjacency=s.adjacency, offsets=s.offsets, rays=rays, start=sp, thr=np.float32(THR), quantiles=q,
        rgba_grad=g,
        infer_rgba_bits=rgba16.view(np.uint16), infer_n=st["n"], infer_visits=st["visits"],
        infer_hash=st["visit_hash"],
        fwd_rgba=fw["rgba"], fwd_n=fw["n"], fwd_depth=fw["depth"], fwd_depth_idx=fw["depth_idx"],
        fwd_contribution=fw["contribution"], fwd_distortion=fw["distortion"], fwd_W=fw["W_total"],
        fwd_S=fw["S_total"], fwd_t_far=fw["t_far"],
        bwd_points_grad=bw["points_grad"], bwd_density_grad=bw["density_grad"],
        bwd_diffuse_grad=bw["diffuse_grad"], bwd_specular_grad=bw["specular_grad"])


if __name__ == "__main__":
    data = make()
    np.savez_compressed(PATH, **data)
    print(f"wrote {PATH} ({os.path.getsize(PATH)} bytes)")
