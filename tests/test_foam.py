"""The .foam scene format (scripts/export_for_viewer.py:17-43, :146-216):
round trips of V4 and V3 files, the 120-byte header layout, error cases, and
(GPU) rendering a scene reloaded from a file equals rendering the original."""
import struct

import numpy as np
import pytest

from oracle import core, host_ops
from vorotracing_amd import camera, foam, scene


def _arrays(n=300, seed=3):
    s = scene.random_scene(n, seed=seed, R=4)
    dens = core.expf(s.density_raw.reshape(-1).astype(np.float32))
    d4 = host_ops.pad_3to4(s.diffuse.astype(np.float16), 4)
    s4 = host_ops.pad_3to4(s.specular.astype(np.float16), 4)
    poses = np.stack([np.eye(4, dtype=np.float32)[:3], np.eye(4, dtype=np.float32)[:3] * 2])
    return s, dens, d4, s4, poses


def test_v4_round_trip_and_header(tmp_path):
    s, dens, d4, s4, poses = _arrays()
    p = tmp_path / "a.foam"
    foam.write_foam(p, s.points, dens, d4, s4, s.adjacency, s.offsets, poses, 4, 4, 0.01, 1e-3, 512)
    raw = p.read_bytes()
    magic, version, n, npos, adj, ad, rd, rs, w, k, mx = struct.unpack_from("<IIIIIIIIffI", raw, 0)
    assert (magic, version, n, npos, adj, ad, rd, rs, mx) == (0x464F414D, 4, 300, 2, s.adjacency.size, 0, 4, 4, 512)
    assert struct.unpack_from("<I", raw, 116)[0] == 1  # has_specular at byte 116
    n_m = s.adjacency.size
    assert len(raw) == 120 + 300 * 12 + 300 * 4 + 2 * 300 * 48 * 2 + n_m * 4 + 301 * 4 + 2 * 48
    f = foam.read_foam(p)
    assert f.version == 4 and f.adjacent_diff is None
    assert np.array_equal(f.points, s.points) and np.array_equal(f.density, dens)
    # tight RGB: the 4th (zero) channel of the Half4Texel maps is dropped
    assert np.array_equal(f.diffuse.view(np.uint16), d4.reshape(300, 16, 4)[:, :, :3].reshape(300, -1).view(np.uint16))
    assert np.array_equal(f.specular, s4.reshape(300, 16, 4)[:, :, :3].reshape(300, -1))
    assert np.array_equal(f.adjacency, s.adjacency) and np.array_equal(f.offsets, s.offsets)
    assert np.array_equal(f.poses, poses) and np.array_equal(f.default_pose, poses[0])
    assert np.allclose(f.aabb_min, s.points.min(0)) and np.allclose(f.aabb_max, s.points.max(0))
    assert f.weight_threshold == np.float32(0.01) and f.max_intersections == 512


def test_v3_round_trip_without_specular(tmp_path):
    s, dens, d4, s4, poses = _arrays(200, 5)
    ad = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    p = tmp_path / "b.foam"
    foam.write_foam(p, s.points, dens, d4, None, s.adjacency, s.offsets, poses[:1], 4, 4, version=3,
                    adjacent_diff=ad)
    f = foam.read_foam(p, mmap=False)
    assert f.version == 3 and f.specular is None and f.res_spec == 0
    assert np.array_equal(f.diffuse, d4.reshape(200, 16, 4)[:, :, :3].reshape(200, -1))
    assert np.array_equal(f.adjacent_diff.view(np.uint16), ad.view(np.uint16))
    # V3 stores RGBx maps: 4 halves per texel
    assert p.stat().st_size == 120 + 200 * 16 + 200 * 64 * 2 + s.adjacency.size * 4 + 201 * 4 + ad.size * 2 + 48


def test_bad_files(tmp_path):
    s, dens, d4, s4, poses = _arrays(100, 7)
    p = tmp_path / "c.foam"
    foam.write_foam(p, s.points, dens, d4, s4, s.adjacency, s.offsets, poses, 4, 4)
    raw = bytearray(p.read_bytes())
    (tmp_path / "short.foam").write_bytes(raw[:-4])
    with pytest.raises(ValueError, match="does not match its header"):
        foam.read_foam(tmp_path / "short.foam")
    raw[0] ^= 1
    (tmp_path / "magic.foam").write_bytes(raw)
    with pytest.raises(ValueError, match="not a .foam file"):
        foam.read_foam(tmp_path / "magic.foam")
    with pytest.raises(ValueError, match="octmap width"):
        foam.write_foam(p, s.points, dens, d4[:, :40], s4, s.adjacency, s.offsets, poses, 4, 4)


@pytest.mark.gpu
@pytest.mark.parametrize("version", [4, 3])
def test_render_from_foam_equals_original(gpu, tmp_path, version):
    import torch

    from tests import helpers as H
    from vorotracing_amd.infer import VoroTracingInfer
    from vorotracing_amd.model import VoroTracing

    s = H.mini_heightfield()
    inf = VoroTracingInfer(VoroTracing.from_scene(s, device=gpu), sort_morton=True, quantize="fp16")
    rays = H.to_dev(camera.orbit_rays(3, 96, 64), gpu)
    want = inf.render(rays, weight_threshold=0.01, cell_skip_threshold=1e-3)
    p = tmp_path / "s.foam"
    foam.save_infer(p, inf, np.eye(4, dtype=np.float32)[None, :3], weight_threshold=0.01, version=version)
    back = VoroTracingInfer.from_foam(p, device=gpu)
    assert torch.equal(back.adjacent_diff.view(torch.int16), inf.adjacent_diff.view(torch.int16))
    got = back.render(rays, weight_threshold=0.01, cell_skip_threshold=1e-3)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
