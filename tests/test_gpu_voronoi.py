"""GPU Voronoi adjacency (vt_voronoi_build) against the host Delaunay
(scipy/qhull): for sites in general position, each cell's neighbour set must
equal qhull's; lists come out ascending, the CSR tail holds the padding."""
import numpy as np
import pytest
import torch

from tests import helpers as H
from vorotracing_amd import ops, scene

pytestmark = pytest.mark.gpu


def _qhull_sets(points):
    adj, off = scene.delaunay_csr(points, pad=0)
    return [np.sort(adj[off[i]:off[i + 1]]) for i in range(points.shape[0])], off


def _check(points, gpu):
    adj, off, status = ops.build_voronoi_adjacency(H.to_dev(points, gpu))
    torch.cuda.synchronize()
    adj, off = adj.cpu().numpy(), off.cpu().numpy()
    want, woff = _qhull_sets(points)
    assert off.shape == (points.shape[0] + 1,)
    assert adj.shape[0] == off[-1] + 32 and not adj[off[-1]:].any()
    bad = [i for i in range(points.shape[0]) if not np.array_equal(adj[off[i]:off[i + 1]], want[i])]
    assert not bad, f"{len(bad)} cells differ from qhull, first {bad[:5]}"
    assert off[-1] == woff[-1]
    assert all(np.all(np.diff(adj[off[i]:off[i + 1]].astype(np.int64)) > 0) for i in range(points.shape[0]))


@pytest.mark.parametrize("n,seed", [(500, 0), (3000, 1)])
def test_random_cube(gpu, n, seed):
    pts = np.random.default_rng(seed).uniform(-2, 2, size=(n, 3)).astype(np.float32)
    _check(pts, gpu)


def test_c1_sites(gpu):
    _check(H.c1_scene().points, gpu)


def test_mini_heightfield_sites(gpu):
    """Config-3 distribution at test size: a thin dense surface layer plus a sparse background."""
    _check(H.mini_heightfield().points, gpu)


def test_heightfield_131k(gpu):
    """C3's site distribution at 131,072 sites: dense surface cells whose lists exceed the
    64-entry slots, background cells next to the surface and the convex-hull cells of the cube."""
    pts = scene._heightfield_sites(np.random.default_rng(3), 131072, 0.8, 4.0, 0.01).astype(np.float32)
    _check(pts, gpu)


def test_ellipsoid_surface(gpu):
    """Every site on a convex surface is a convex-hull site, so every cell is unbounded.  An
    ellipsoid (unlike a sphere) keeps 5 sites off a common sphere: general position."""
    d = np.random.default_rng(5).normal(size=(3000, 3))
    pts = (d / np.linalg.norm(d, axis=1, keepdims=True) * np.array([1.0, 0.7, 0.5])).astype(np.float32)
    _check(pts, gpu)


def test_model_scene_renders_the_same(gpu):
    """A scene whose adjacency comes from the GPU builder renders like the qhull one (same sets,
    ascending order; the walk's choice depends on the order only through exact ties)."""
    from vorotracing_amd import camera
    from vorotracing_amd.model import VoroTracing

    s = H.small_random(800, seed=9)
    rays = H.to_dev(camera.pinhole_rays(48, 32, eye=(0.3, -3.5, 0.5)), gpu)
    m1 = VoroTracing.from_scene(s, device=gpu)
    adj, off, _ = ops.build_voronoi_adjacency(m1.primal_points)
    s_sorted = scene.Scene(s.name, s.points, s.density_raw, s.diffuse, s.specular,
                           adj.cpu().numpy(), off.cpu().numpy(), s.diff_res, s.spec_res, dict(s.params))
    m2 = VoroTracing.from_scene(s_sorted, device=gpu)
    a = m1(rays, weight_threshold=0.001)[0]
    b = m2(rays, weight_threshold=0.001)[0]
    torch.cuda.synchronize()
    assert torch.equal(a, b)


@pytest.mark.parametrize("guess", ["previous", "shuffled", "junk"])
def test_warm_start_equals_cold(gpu, guess):
    """A warm-started build (initial_guesses, cuda/__init__.py:16-37) gives
    the cold build's CSR and qhull's sets, whatever the guesses: the
    adjacency before the sites moved (the training refresh), lists of other
    sites, or ids out of range."""
    rng = np.random.default_rng(17)
    pts0 = scene._heightfield_sites(rng, 40000, 0.8, 4.0, 0.01).astype(np.float32)
    adj0, off0, _ = ops.build_voronoi_adjacency(H.to_dev(pts0, gpu))
    pts = (pts0 + rng.normal(0.0, 2e-3, size=pts0.shape)).astype(np.float32)  # the sites moved
    g_adj, g_off = adj0, off0
    if guess == "shuffled":
        o64 = off0.to(torch.int64)
        g_off = (o64[-1] - o64.flip(0)).to(torch.uint32).contiguous()  # other cells' list lengths and entries
    elif guess == "junk":
        g_adj = torch.full_like(adj0, 0xFFFFFFF0)
        g_adj[::3] = torch.arange(0, g_adj[::3].numel(), device=gpu, dtype=torch.int64).to(torch.uint32)
    pd = H.to_dev(pts, gpu)
    cold = ops.build_voronoi_adjacency(pd)
    warm = ops.build_voronoi_adjacency(pd, initial_guesses=g_adj, initial_guesses_offsets=g_off)
    torch.cuda.synchronize()
    assert torch.equal(warm[1], cold[1]) and torch.equal(warm[0], cold[0])
    if guess == "previous":
        _check(pts, gpu)


def test_model_refresh_warm_start(gpu):
    """VoroTracing.update_triangulation seeds the build with the current
    adjacency; the refreshed CSR equals a cold build's."""
    from vorotracing_amd.model import VoroTracing

    s = H.small_random(3000, seed=21)
    m = VoroTracing.from_scene(s, device=gpu)
    with torch.no_grad():
        m.primal_points.add_(torch.randn_like(m.primal_points) * 1e-3)
    m.update_triangulation()
    adj, off, _ = ops.build_voronoi_adjacency(m.primal_points)
    torch.cuda.synchronize()
    assert torch.equal(m.point_adjacency, adj) and torch.equal(m.point_adjacency_offsets, off)
