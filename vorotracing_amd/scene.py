"""Seeded synthetic Voronoi scenes for the benchmark configurations.

A scene is what the reference's traversal consumes: sites (N,3) f32, raw
log-density (N,1) f32 (activated as ``exp(raw)``, vorotracing.py:346-347),
diffuse/specular octahedral logit maps (N, 3*R*R) f32 in texel-major /
channel-minor order (ray_integrator_octmap.cuh:226-227), and the Voronoi
adjacency in CSR form: ``offsets`` u32 (N+1) and ``adjacency`` u32 with 32
zero padding entries (the layout of cuda/__init__.py:39-46).  The adjacency
comes from the host Delaunay triangulation (scipy/qhull), whose edges are the
Voronoi faces.

Draw order for every config: sites, density, diffuse, specular (numpy PCG64,
``default_rng(seed)``).  Cameras are deterministic (camera.py).
"""
from __future__ import annotations

import dataclasses
import hashlib
import os
import time

import numpy as np

PAD = 32


@dataclasses.dataclass
class Scene:
    name: str
    points: np.ndarray  # (N,3) f32
    density_raw: np.ndarray  # (N,1) f32
    diffuse: np.ndarray  # (N, 3*R*R) f32 logits
    specular: np.ndarray  # (N, 3*Rs*Rs) f32 logits
    adjacency: np.ndarray  # (M+32,) u32
    offsets: np.ndarray  # (N+1,) u32
    diff_res: int
    spec_res: int
    params: dict

    @property
    def num_points(self) -> int:
        return int(self.points.shape[0])

    @property
    def density(self) -> np.ndarray:
        """Activated density s = exp(raw) (activation_scale 1, vorotracing.py:21,346)."""
        return np.exp(self.density_raw.astype(np.float32)).astype(np.float32)

    @property
    def num_faces(self) -> int:
        return int(self.offsets[-1])


def delaunay_csr(points: np.ndarray, pad: int = PAD):
    """Voronoi adjacency of ``points`` as (adjacency u32 (M+pad), offsets u32 (N+1))."""
    from scipy.spatial import Delaunay

    tri = Delaunay(np.asarray(points, np.float64))
    indptr, indices = tri.vertex_neighbor_vertices
    adjacency = np.zeros(indices.shape[0] + pad, np.uint32)
    adjacency[: indices.shape[0]] = indices
    return adjacency, indptr.astype(np.uint32)


def _unit_sphere_shell(rng, n, jitter):
    d = rng.normal(size=(n, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = 1.0 + rng.normal(0.0, jitter, size=(n, 1))
    return d * r


def _torus(rng, n, major, minor, jitter):
    u = rng.uniform(0.0, 2 * np.pi, n)
    v = rng.uniform(0.0, 2 * np.pi, n)
    r = minor + rng.normal(0.0, jitter, n)
    x = (major + r * np.cos(v)) * np.cos(u)
    y = (major + r * np.cos(v)) * np.sin(u)
    z = r * np.sin(v)
    return np.stack([x, y, z], 1)


def height(x, y):
    """Height field of configs 3-5: z = 0.3 sin(3x) cos(2y)."""
    return 0.3 * np.sin(3.0 * x) * np.cos(2.0 * y)


def _heightfield_sites(rng, n, frac_surface, extent, jitter):
    ns = int(round(n * frac_surface))
    x = rng.uniform(-extent, extent, ns)
    y = rng.uniform(-extent, extent, ns)
    z = height(x, y) + rng.normal(0.0, jitter, ns)
    surf = np.stack([x, y, z], 1)
    bg = rng.uniform(-extent, extent, size=(n - ns, 3))
    return np.concatenate([surf, bg], 0)


def _finish(name, pts, raw, diff, spec, R, Rs, params, csr=None):
    pts = np.ascontiguousarray(pts, np.float32)
    if csr is None:
        csr = delaunay_csr(pts)
    adjacency, offsets = csr
    return Scene(name, pts, np.ascontiguousarray(raw, np.float32).reshape(-1, 1),
                 np.ascontiguousarray(diff, np.float32), np.ascontiguousarray(spec, np.float32), adjacency,
                 offsets, R, Rs, params)


def config1(seed: int = 0, n: int = 4096, R: int = 4) -> Scene:
    """C1: unit-sphere shell (70%, radial N(0,0.02)) + U([-2,2]^3) background;
    raw density N(0,1); diffuse U(0,1) logits; specular zero."""
    rng = np.random.default_rng(seed)
    ns = int(round(0.7 * n))
    pts = np.concatenate([_unit_sphere_shell(rng, ns, 0.02), rng.uniform(-2, 2, size=(n - ns, 3))], 0)
    raw = rng.normal(0.0, 1.0, size=(n, 1))
    diff = rng.uniform(0.0, 1.0, size=(n, 3 * R * R))
    spec = np.zeros((n, 3 * R * R))
    return _finish("c1", pts, raw, diff, spec, R, R, dict(config=1, seed=seed, n=n, R=R))


def config2(seed: int = 0, n: int = 262144, R: int = 4) -> Scene:
    """C2: torus (major 1.5, minor 0.5, normal jitter N(0,0.02), 70%) +
    U([-2.5,2.5]^3); raw density N(0,1); diffuse U(0,1); specular N(0,0.1)."""
    rng = np.random.default_rng(seed)
    ns = int(round(0.7 * n))
    pts = np.concatenate([_torus(rng, ns, 1.5, 0.5, 0.02), rng.uniform(-2.5, 2.5, size=(n - ns, 3))], 0)
    raw = rng.normal(0.0, 1.0, size=(n, 1))
    diff = rng.uniform(0.0, 1.0, size=(n, 3 * R * R))
    spec = rng.normal(0.0, 0.1, size=(n, 3 * R * R))
    return _finish("c2", pts, raw, diff, spec, R, R, dict(config=2, seed=seed, n=n, R=R))


def heightfield(seed: int = 0, n: int = 1048576, R: int = 4, extent: float = 4.0, name: str = "c3",
                frac_surface: float = 0.8, csr_fn=None) -> Scene:
    """C3/C4/C5 scene: 80% near z = 0.3 sin(3x) cos(2y) (jitter N(0,0.01)),
    20% U([-4,4]^3); raw density N(3,1) within 0.02 of the surface, N(-4,1)
    elsewhere; diffuse N(0,1) logits; specular N(0,0.1).  ``csr_fn(points)``
    supplies (adjacency, offsets) instead of host qhull (the GPU builder)."""
    rng = np.random.default_rng(seed)
    pts = _heightfield_sites(rng, n, frac_surface, extent, 0.01)
    near = np.abs(pts[:, 2] - height(pts[:, 0], pts[:, 1])) < 0.02
    raw = np.where(near, rng.normal(3.0, 1.0, n), rng.normal(-4.0, 1.0, n)).reshape(n, 1)
    diff = rng.normal(0.0, 1.0, size=(n, 3 * R * R))
    spec = rng.normal(0.0, 0.1, size=(n, 3 * R * R))
    csr = None if csr_fn is None else csr_fn(np.ascontiguousarray(pts, np.float32))
    return _finish(name, pts, raw, diff, spec, R, R, dict(config=name, seed=seed, n=n, R=R, extent=extent), csr)


def config3(seed: int = 0, n: int = 1048576, R: int = 4) -> Scene:
    return heightfield(seed, n, R, name="c3")


def config5(seed: int = 0, n: int = 3145728, R: int = 4) -> Scene:
    return heightfield(seed, n, R, name="c5")


def cubic_lattice(nx: int, ny: int, nz: int, spacing: float = 1.0, raw_density: float = 0.0, R: int = 4,
                  seed: int = 0) -> Scene:
    """Sites on an integer lattice with the exact Voronoi adjacency (the six
    axis neighbours, order -x,+x,-y,+y,-z,+z).  Cells are cubes; offsets are
    exact in fp16, so exit distances have closed forms."""
    rng = np.random.default_rng(seed)
    ii, jj, kk = np.meshgrid(np.arange(nx), np.arange(ny), np.arange(nz), indexing="ij")
    idx = (ii * ny + jj) * nz + kk
    pts = np.stack([ii, jj, kk], -1).reshape(-1, 3).astype(np.float64) * spacing
    n = pts.shape[0]
    flat = idx.reshape(-1)
    lists = []
    coords = np.stack([ii, jj, kk], -1).reshape(-1, 3)
    dims = (nx, ny, nz)
    for c in range(n):
        ijk = coords[c]
        nb = []
        for ax in range(3):
            for s in (-1, 1):
                q = ijk.copy()
                q[ax] += s
                if 0 <= q[ax] < dims[ax]:
                    nb.append(int(flat[(q[0] * ny + q[1]) * nz + q[2]]))
        lists.append(nb)
    offsets = np.zeros(n + 1, np.uint32)
    offsets[1:] = np.cumsum([len(x) for x in lists])
    adjacency = np.zeros(int(offsets[-1]) + PAD, np.uint32)
    adjacency[: offsets[-1]] = np.concatenate(lists)
    raw = np.full((n, 1), raw_density)
    diff = rng.uniform(-1, 1, size=(n, 3 * R * R))
    spec = rng.uniform(-0.5, 0.5, size=(n, 3 * R * R))
    return _finish("lattice", pts, raw, diff, spec, R, R, dict(lattice=(nx, ny, nz), spacing=spacing),
                   csr=(adjacency, offsets))


def random_scene(n: int, seed: int = 0, R: int = 4, Rs: int | None = None, extent: float = 2.0,
                 grid: float | None = None, density_mu: float = 0.0) -> Scene:
    """Uniform random sites in [-extent, extent]^3; with ``grid`` the
    coordinates are snapped to multiples of ``grid`` (e.g. 1/64, so every site
    difference is exact in fp16)."""
    rng = np.random.default_rng(seed)
    Rs = R if Rs is None else Rs
    pts = rng.uniform(-extent, extent, size=(n, 3))
    if grid:
        pts = np.round(pts / grid) * grid
        pts = np.unique(pts, axis=0)
        rng.shuffle(pts)
        n = pts.shape[0]
    raw = rng.normal(density_mu, 1.0, size=(n, 1))
    diff = rng.normal(0.0, 1.0, size=(n, 3 * R * R))
    spec = rng.normal(0.0, 0.3, size=(n, 3 * Rs * Rs))
    return _finish(f"random{n}", pts, raw, diff, spec, R, Rs, dict(n=n, seed=seed, extent=extent, grid=grid))


def cached(builder, *args, cache_dir: str | None = None, **kw) -> Scene:
    """Build a scene once and keep it as an .npz under ``cache_dir`` (default
    $VT_SCENE_CACHE or ~/.cache/vorotracing_amd); qhull at 1M sites takes about
    a minute."""
    cache_dir = cache_dir or os.environ.get("VT_SCENE_CACHE") or os.path.join(
        os.path.expanduser("~"), ".cache", "vorotracing_amd")
    key = hashlib.sha1(repr((builder.__name__, args, sorted(kw.items()))).encode()).hexdigest()[:16]
    path = os.path.join(cache_dir, f"{builder.__name__}_{key}.npz")
    if os.path.exists(path):
        z = np.load(path, allow_pickle=False)
        return Scene(str(z["name"]), z["points"], z["density_raw"], z["diffuse"], z["specular"], z["adjacency"],
                     z["offsets"], int(z["diff_res"]), int(z["spec_res"]), {"cached": path})
    t = time.time()
    s = builder(*args, **kw)
    s.params["build_s"] = round(time.time() - t, 2)
    try:
        os.makedirs(cache_dir, exist_ok=True)
        np.savez(path + ".tmp.npz", name=s.name, points=s.points, density_raw=s.density_raw, diffuse=s.diffuse,
                 specular=s.specular, adjacency=s.adjacency, offsets=s.offsets, diff_res=s.diff_res,
                 spec_res=s.spec_res)
        os.replace(path + ".tmp.npz", path)
    except OSError:
        pass
    return s
