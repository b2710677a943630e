"""The first-visited-cells log of the walk statistics (vt_ray_stats.first_cells,
mirrored by the oracle's or_ray_stats), on the CPU: it starts at the ray's start
cell, steps only between adjacent cells, agrees with the oracle's separate
visit log and with the visit count, and is padded with 0xffffffff after a
short walk.  The GPU kernels are compared with it field by field wherever the
parity tests compare walk statistics."""
import numpy as np

from oracle import core
from tests import helpers as H
from vorotracing_amd import camera, native

NONE = np.uint32(0xFFFFFFFF)
LOG = 24


def test_record_layout():
    assert core.STATS_DTYPE.itemsize == 4 * native.STATS_WORDS == 128
    assert core.STATS_DTYPE["first_cells"].shape == (LOG,)


def test_first_cells_follow_the_walk():
    s = H.small_random(4000, seed=5)
    rays = camera.pinhole_rays(24, 16, eye=(0.0, -3.2, 0.4))
    start = H.start_for(s, rays)
    d4, s4 = H.f16_maps(s)
    adj_diff = core.prefetch_adj(s.points, s.adjacency, s.offsets)
    _, st, log = core.trace_infer_f16(s.points, d4, s4, s.diff_res, s.spec_res, s.density, s.adjacency, s.offsets,
                                      adj_diff, rays, start, weight_threshold=1e-4, want_stats=True, max_log=40)
    first = st["first_cells"]
    nvis = st["visits"]
    assert (nvis > LOG).any() and (nvis < LOG).any()  # both long and short walks
    # the oracle's separate visit log
    assert np.array_equal(first, log[:, :LOG])
    # starts at the start cell; entries up to the visit count, padding after
    assert np.array_equal(first[:, 0], start.reshape(-1))
    k = np.arange(LOG)[None, :]
    assert ((first != NONE) == (k < nvis[:, None])).all()
    # consecutive cells are neighbours in the CSR
    off = s.offsets.astype(np.int64)
    for r in range(first.shape[0]):
        m = min(int(nvis[r]), LOG)
        for i in range(m - 1):
            a, b = int(first[r, i]), int(first[r, i + 1])
            assert b in s.adjacency[off[a]:off[a + 1]], (r, i, a, b)
