"""Out-of-range indices from a caller (the reference reads out of bounds for
them; these entries do not): start cells at or past num_points give a ray
with no step (rgba 0, n 0, no gradient), the other rays of the launch are
unchanged bit for bit; an adjacency naming a cell past the last makes the walk
layout build refuse the scene, and the fill alone links such a face to its own
cell without reading past its arrays."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from vorotracing_amd import _C, _lib, camera, native
from vorotracing_amd.model import VoroTracing

pytestmark = pytest.mark.gpu


def _bad_starts(start, n):
    bad = start.copy().reshape(-1)
    idx = np.arange(0, bad.size, 7)
    bad[idx[0::2]] = n
    bad[idx[1::2]] = 0xFFFFFFFF
    return bad.reshape(start.shape), np.isin(np.arange(bad.size), idx).reshape(start.shape)


def test_out_of_range_start_cells_infer(gpu):
    s = H.mini_heightfield()
    d4, s4 = H.f16_maps(s)
    dev = dict(points=H.to_dev(s.points, gpu), diffuse4=H.to_dev(d4, gpu), specular4=H.to_dev(s4, gpu),
               density=H.to_dev(s.density.reshape(-1), gpu), adjacency=H.to_dev(s.adjacency, gpu),
               offsets=H.to_dev(s.offsets, gpu))
    adj = native.prefetch(dev["points"], dev["adjacency"], dev["offsets"])
    wl = native.WalkLayout.build(dev["points"], dev["density"], dev["adjacency"], dev["offsets"], adj)
    qm = native.QuadMaps.build(dev["diffuse4"], dev["specular4"])
    rays = camera.orbit_rays(4, 96, 64)
    start = H.start_for(s, rays)
    bad, mask = _bad_starts(start, s.num_points)
    rd = H.to_dev(rays, gpu)
    for tiled, walk, quads in (((8, 8), wl, qm), ((8, 8), None, None), (None, None, None)):
        print(f"case: out-of-range start cells, tiled {tiled}, walk {walk is not None}", flush=True)
        outs = []
        for sp in (start, bad):
            st = native.new_stats(rays.shape[0] * rays.shape[1], gpu)
            out = native.infer_f16(dev["points"], dev["diffuse4"], dev["specular4"], dev["density"],
                                   dev["adjacency"], dev["offsets"], adj, rd, H.to_dev(sp, gpu),
                                   weight_threshold=0.01, cell_skip_threshold=1e-3, stats=st, tiled=tiled,
                                   walk=walk, quads=quads)
            torch.cuda.synchronize()
            outs.append((out.cpu().numpy().view(np.uint16), H.stats_np(st)))
        (good, gst), (got, bst) = outs
        assert not got[mask].any() and (bst["n"][mask.reshape(-1)] == 0).all()
        assert np.array_equal(got[~mask], good[~mask])
        assert np.array_equal(bst["n"][~mask.reshape(-1)], gst["n"][~mask.reshape(-1)])


def test_out_of_range_start_cells_train(gpu):
    s = H.mini_heightfield()
    model = VoroTracing.from_scene(s, device=gpu)
    rays = camera.orbit_rays(6, 64, 48)
    rd = H.to_dev(rays, gpu)
    start = model.get_starting_point(rd).cpu().numpy()
    bad, mask = _bad_starts(start, s.num_points)
    pts = model.primal_points.detach().contiguous()
    dif = model.att_diffuse.detach().contiguous()
    spe = model.att_specular.detach().contiguous()
    den = model.activated_density().detach().reshape(-1).contiguous()
    adj, off = model.point_adjacency, model.point_adjacency_offsets
    fw = {}
    for name, sp in (("good", start), ("bad", bad)):
        print(f"case: training forward, {name} start cells", flush=True)
        fw[name] = _C.trace_vorotracing_fwd(pts, dif, spe, den, adj, off, rd, H.to_dev(sp, gpu), None, 0.001,
                                            1024, False)
    torch.cuda.synchronize()
    rgba_g, n_g = fw["good"][0].cpu().numpy(), fw["good"][4].cpu().numpy()
    rgba_b, n_b = fw["bad"][0].cpu().numpy(), fw["bad"][4].cpu().numpy()
    assert not rgba_b[mask].any() and (n_b[mask] == 0).all()
    assert np.array_equal(rgba_b[~mask].view(np.uint32), rgba_g[~mask].view(np.uint32))
    assert np.array_equal(n_b[~mask], n_g[~mask])
    # backward: a ray with no step adds nothing, as a valid ray with zero upstream gradients
    g = np.random.default_rng(2).normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    g0 = g.copy()
    g0[mask] = 0.0
    grads = {}
    for name, sp, gg in (("bad", bad, g), ("zero", start, g0)):
        print(f"case: training backward, {name}", flush=True)
        f = fw["bad" if name == "bad" else "good"]
        grads[name] = _C.trace_vorotracing_bwd(pts, dif, spe, den, adj, off, rd, H.to_dev(sp, gpu), f[0],
                                               H.to_dev(gg, gpu), None, None, None, None, 0.0, f[5], None, f[6],
                                               f[7], f[8], 0.001, 1024)
    torch.cuda.synchronize()
    for k, name in enumerate(("points_grad", "diffuse_grad", "specular_grad", "density_grad")):
        H.assert_grad_close(grads["bad"][k].cpu().numpy(), grads["zero"][k].cpu().numpy(), name)


def test_walk_layout_refuses_out_of_range_neighbours(gpu):
    s = H.small_random(600, seed=5)
    adjacency = s.adjacency.copy()
    adjacency[37] = s.num_points  # one face of some cell names a cell past the last
    d = dict(points=H.to_dev(s.points, gpu), density=H.to_dev(s.density.reshape(-1), gpu),
             adjacency=H.to_dev(adjacency, gpu), offsets=H.to_dev(s.offsets, gpu))
    adj = native.prefetch(d["points"], H.to_dev(s.adjacency, gpu), d["offsets"])
    with pytest.raises(ValueError, match="neighbour id"):
        native.WalkLayout.build(d["points"], d["density"], d["adjacency"], d["offsets"], adj)
    # the fill alone, past the flag: the face links its own cell
    good = native.WalkLayout.build(d["points"], d["density"], H.to_dev(s.adjacency, gpu), d["offsets"], adj)
    n, total = s.num_points, good.num_chunks
    first = torch.empty(n + 2, dtype=torch.int32, device=gpu)
    ws = torch.empty(max(int(_lib.load().vt_walk_layout_count_workspace_size(n)), 1), dtype=torch.uint8, device=gpu)
    sp = torch.cuda.current_stream().cuda_stream
    _lib.call("vt_walk_layout_count", d["offsets"].data_ptr(), d["adjacency"].data_ptr(), n, first.data_ptr(),
              ws.data_ptr(), sp)
    chunks = torch.zeros((total + 1, 12), dtype=torch.int32, device=gpu)
    links = torch.empty((8 * total, 2), dtype=torch.int32, device=gpu)
    heads = torch.empty((n, 2), dtype=torch.int32, device=gpu)
    cells = torch.empty((n, 4), dtype=torch.float32, device=gpu)
    orig = torch.empty(8 * total, dtype=torch.int16, device=gpu)
    _lib.call("vt_walk_layout_fill", d["points"].data_ptr(), d["density"].data_ptr(), d["adjacency"].data_ptr(),
              d["offsets"].data_ptr(), n, adj.data_ptr(), first.data_ptr(), total, 0, chunks.data_ptr(),
              links.data_ptr(), heads.data_ptr(), cells.data_ptr(), orig.data_ptr(), sp)
    torch.cuda.synchronize()
    flag = int(first[n + 1].item()) & 0xFFFFFFFF
    assert flag >> 31 == 1
    cell = int(np.searchsorted(s.offsets, 37, side="right") - 1)
    slot = 8 * int(first[cell].item()) + (37 - int(s.offsets[cell]))
    assert np.array_equal(links[slot].cpu().numpy(), heads[cell].cpu().numpy())
