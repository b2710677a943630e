"""The flat ``.foam`` scene format (V4, and the legacy V3) of the reference's
viewer export, scripts/export_for_viewer.py:17-43 (layout) and :146-216
(writer), with a reader that memory-maps the blobs and a loader into
``VoroTracingInfer``.

Layout, all little-endian.  A 120-byte header:
- magic "FOAM", version;
- num_points, num_poses, adjacency_size, adjacent_diff_size;
- res_diff, res_spec;
- weight_threshold, cell_skip_threshold, max_intersections;
- default_pose (3x4 f32), aabb_min, aabb_max, has_specular.

Then the blobs, in order:
- points (N,3) f32, density (N) f32 (activated);
- diffuse (N, R^2*C) f16, specular (optional, same form);
- point_adjacency u32, point_adjacency_offsets (N+1) u32;
- adjacent_diff (V3 only);
- poses (P,3,4) f32.

C is 3 (tight RGB) in V4 and 4 (RGBx) in V3.  V4 drops adjacent_diff, which
the loader recomputes from the adjacency (it is exactly the prefetch output).
"""
from __future__ import annotations

import dataclasses
import struct
from pathlib import Path
from typing import Optional

import numpy as np

MAGIC = 0x464F414D
HEADER = struct.Struct("<IIIIIIIIffI")  # 44 bytes, then pose/aabb/has_specular
HEADER_BYTES = 120


@dataclasses.dataclass
class FoamScene:
    version: int
    points: np.ndarray  # (N,3) f32
    density: np.ndarray  # (N,) f32, activated
    diffuse: np.ndarray  # (N, R^2*3) f16 (V3 maps are returned tight too)
    specular: Optional[np.ndarray]  # (N, Rs^2*3) f16 or None
    adjacency: np.ndarray  # u32, including the 32-entry padding tail
    offsets: np.ndarray  # (N+1,) u32
    poses: np.ndarray  # (P,3,4) f32
    res_diff: int
    res_spec: int
    weight_threshold: float
    cell_skip_threshold: float
    max_intersections: int
    default_pose: np.ndarray  # (3,4) f32
    aabb_min: np.ndarray
    aabb_max: np.ndarray
    adjacent_diff: Optional[np.ndarray] = None  # (M,4) f16, V3 files only


def _tight(maps: np.ndarray, n: int, res: int) -> np.ndarray:
    """(N, R^2*4) RGBx -> (N, R^2*3) RGB (export_for_viewer.py:67-69)."""
    return np.ascontiguousarray(maps.reshape(n, res * res, 4)[:, :, :3].reshape(n, -1))


def _padded(maps: np.ndarray, n: int, res: int) -> np.ndarray:
    """(N, R^2*3) -> (N, R^2*4) with a zero 4th channel (Half4Texel)."""
    out = np.zeros((n, res * res, 4), np.float16)
    out[:, :, :3] = maps.reshape(n, res * res, 3)
    return out.reshape(n, -1)


def write_foam(path, points, density, diffuse, specular, adjacency, offsets, poses, res_diff: int, res_spec: int,
               weight_threshold: float = 0.001, cell_skip_threshold: float = 0.0, max_intersections: int = 1024,
               version: int = 4, adjacent_diff=None, aabb=None) -> None:
    """Writes a scene.  ``diffuse`` / ``specular`` are fp16 maps, tight (N, R^2*3)
    or Half4Texel (N, R^2*4); ``specular=None`` writes has_specular = 0.
    Version 3 additionally needs ``adjacent_diff`` ((M,4) f16)."""
    pts = np.ascontiguousarray(points, np.float32).reshape(-1, 3)
    n = pts.shape[0]
    dens = np.ascontiguousarray(density, np.float32).reshape(-1)
    adj = np.ascontiguousarray(adjacency, np.uint32).reshape(-1)
    off = np.ascontiguousarray(offsets, np.uint32).reshape(-1)
    if dens.shape != (n,) or off.shape != (n + 1,):
        raise ValueError("density must be (N,) and offsets (N+1,)")
    if version not in (3, 4):
        raise ValueError("version must be 3 or 4")
    channels = 3 if version >= 4 else 4

    def maps(m, res):
        m = np.ascontiguousarray(m, np.float16).reshape(n, -1)
        if m.shape[1] == res * res * 4:
            return _tight(m, n, res) if channels == 3 else m
        if m.shape[1] == res * res * 3:
            return m if channels == 3 else _padded(m, n, res)
        raise ValueError(f"octmap width {m.shape[1]} does not match resolution {res}")

    dif = maps(diffuse, res_diff)
    has_spec = specular is not None
    spe = maps(specular, res_spec) if has_spec else None
    poses = np.ascontiguousarray(poses, np.float32).reshape(-1, 3, 4)
    if poses.shape[0] == 0:
        raise ValueError("at least one pose is required (poses[0] is the default view)")
    if version < 4:
        if adjacent_diff is None:
            raise ValueError("version 3 stores adjacent_diff")
        ad = np.ascontiguousarray(adjacent_diff, np.float16).reshape(-1, 4)
    lo, hi = (pts.min(0), pts.max(0)) if aabb is None else (np.asarray(aabb[0]), np.asarray(aabb[1]))
    with open(path, "wb") as f:
        f.write(HEADER.pack(MAGIC, version, n, poses.shape[0], adj.shape[0], 0 if version >= 4 else ad.shape[0],
                            res_diff, res_spec if has_spec else 0, float(weight_threshold),
                            float(cell_skip_threshold), int(max_intersections)))
        f.write(poses[0].tobytes())
        f.write(np.asarray(lo, np.float32).tobytes())
        f.write(np.asarray(hi, np.float32).tobytes())
        f.write(struct.pack("<I", 1 if has_spec else 0))
        for blob in (pts, dens, dif) + ((spe,) if has_spec else ()) + (adj, off):
            f.write(blob.tobytes())
        if version < 4:
            f.write(ad.tobytes())
        f.write(poses.tobytes())


def read_foam(path, mmap: bool = True) -> FoamScene:
    """Reads a V3 or V4 file.  Blobs are memory-mapped (read-only) unless
    ``mmap`` is False; octmaps are returned tight RGB in either version."""
    path = Path(path)
    size = path.stat().st_size
    with open(path, "rb") as f:
        head = f.read(HEADER_BYTES)
    if len(head) < HEADER_BYTES:
        raise ValueError(f"{path}: shorter than the 120-byte header")
    (magic, version, n, n_poses, adj_size, ad_size, rd, rs, wthr, skip, max_int) = HEADER.unpack_from(head, 0)
    if magic != MAGIC:
        raise ValueError(f"{path}: not a .foam file (magic {magic:#x})")
    if version not in (3, 4):
        raise ValueError(f"{path}: unsupported .foam version {version}")
    rest = np.frombuffer(head, np.float32, count=18, offset=HEADER.size)
    default_pose, aabb_min, aabb_max = rest[:12].reshape(3, 4).copy(), rest[12:15].copy(), rest[15:18].copy()
    (has_spec,) = struct.unpack_from("<I", head, HEADER.size + 72)
    channels = 3 if version >= 4 else 4
    specs = [("points", np.float32, (n, 3)), ("density", np.float32, (n,)),
             ("diffuse", np.float16, (n, rd * rd * channels))]
    if has_spec:
        specs.append(("specular", np.float16, (n, rs * rs * channels)))
    specs += [("adjacency", np.uint32, (adj_size,)), ("offsets", np.uint32, (n + 1,))]
    if version < 4:
        specs.append(("adjacent_diff", np.float16, (ad_size, 4)))
    specs.append(("poses", np.float32, (n_poses, 3, 4)))
    need = HEADER_BYTES + sum(int(np.prod(s)) * np.dtype(t).itemsize for _, t, s in specs)
    if need != size:
        raise ValueError(f"{path}: size {size} does not match its header ({need} bytes expected)")
    out = {}
    pos = HEADER_BYTES
    for name, dt, shape in specs:
        count = int(np.prod(shape))
        if mmap:
            a = np.memmap(path, dtype=dt, mode="r", offset=pos, shape=shape)
        else:
            a = np.fromfile(path, dtype=dt, count=count, offset=pos).reshape(shape)
        out[name] = a
        pos += count * np.dtype(dt).itemsize
    dif = out["diffuse"] if channels == 3 else _tight(np.asarray(out["diffuse"]), n, rd)
    spe = out.get("specular")
    if spe is not None and channels == 4:
        spe = _tight(np.asarray(spe), n, rs)
    return FoamScene(version=version, points=out["points"], density=out["density"], diffuse=dif, specular=spe,
                     adjacency=out["adjacency"], offsets=out["offsets"], poses=out["poses"], res_diff=rd,
                     res_spec=rs, weight_threshold=wthr, cell_skip_threshold=skip, max_intersections=max_int,
                     default_pose=default_pose, aabb_min=aabb_min, aabb_max=aabb_max,
                     adjacent_diff=out.get("adjacent_diff"))


def save_infer(path, inf, poses, weight_threshold: float = 0.001, cell_skip_threshold: float = 0.0,
               max_intersections: int = 1024, include_specular: bool = True, version: int = 4) -> None:
    """export_for_viewer.write_foam for a ``VoroTracingInfer`` built with fp16
    attributes (its cells, activated density and Half4Texel maps as stored)."""
    if inf.diffuse_fp16 is None:
        raise ValueError("save_infer needs a VoroTracingInfer with fp16 attributes")
    write_foam(path, inf.primal_points.cpu().numpy(), inf.density.reshape(-1).cpu().numpy(),
               inf.diffuse_fp16.cpu().numpy(), inf.specular_fp16.cpu().numpy() if include_specular else None,
               inf.point_adjacency.cpu().numpy(), inf.point_adjacency_offsets.cpu().numpy(), poses, inf.diff_res,
               inf.spec_res, weight_threshold, cell_skip_threshold, max_intersections, version,
               adjacent_diff=inf.adjacent_diff.cpu().numpy() if version < 4 else None)
