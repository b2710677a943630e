"""numpy restatements of the reference's host-side preparation steps.

TEST INFRASTRUCTURE ONLY -- see oracle/__init__.py.  Each function cites the
reference lines (/root/reference/vorotracing/vorotracing.py) it restates and
the torch-on-CUDA arithmetic it reproduces.
"""
from __future__ import annotations

import numpy as np

from . import core


def morton_keys(points):
    """vorotracing.py:516-530: bbox-normalise, x1023, clamp, truncate, interleave 10 bits/axis.

    torch CUDA computes (p - min) / size with IEEE fp32 division and the
    Python scalar 1023.0 as an fp32 multiply.
    """
    p = np.asarray(points, np.float32)
    lo = p.min(axis=0)
    hi = p.max(axis=0)
    size = np.maximum(hi - lo, np.float32(1e-6)).astype(np.float32)
    norm = ((p - lo) / size).astype(np.float32) * np.float32(1023.0)
    norm = np.clip(norm, np.float32(0.0), np.float32(1023.0)).astype(np.int64)
    key = np.zeros(p.shape[0], np.int64)
    for i in range(10):
        key |= ((norm[:, 0] >> i) & 1) << (3 * i)
        key |= ((norm[:, 1] >> i) & 1) << (3 * i + 1)
        key |= ((norm[:, 2] >> i) & 1) << (3 * i + 2)
    return key


def morton_reorder(points, adjacency, offsets, rows=()):
    """vorotracing.py:514-570.  The reference's argsort is not stable (ties
    unspecified, parity unpinned for them); this restatement fixes a stable
    order.  Returns (perm, points, adjacency, offsets, [rows...]) with the
    adjacency padding tail (32 entries) zero-filled."""
    key = morton_keys(points)
    perm = np.argsort(key, kind="stable")
    n = perm.shape[0]
    inv = np.empty_like(perm)
    inv[perm] = np.arange(n)
    off = np.asarray(offsets, np.int64)
    adj = np.asarray(adjacency, np.int64)
    m = int(off[-1])
    adj_remap = inv[adj[:m]]
    counts = off[1:] - off[:-1]
    new_counts = counts[perm]
    new_off = np.zeros(n + 1, np.int64)
    new_off[1:] = np.cumsum(new_counts)
    new_adj = np.zeros(adj.shape[0], np.int64)
    src = np.repeat(off[:-1][perm], new_counts) + (np.arange(m) - np.repeat(new_off[:-1], new_counts))
    new_adj[:m] = adj_remap[src]
    out_rows = [np.ascontiguousarray(np.asarray(r)[perm]) for r in rows]
    return (perm, np.ascontiguousarray(np.asarray(points)[perm]), new_adj.astype(np.uint32),
            new_off.astype(np.uint32), out_rows)


def tile_perm(H, W, TH=8, TW=8):
    """vorotracing.py:606-625 (reference default TH=4, TW=8; wave64 uses 8x8)."""
    y = np.arange(H).reshape(H, 1).repeat(W, 1)
    x = np.arange(W).reshape(1, W).repeat(H, 0)
    tpr = (W + TW - 1) // TW
    k = ((y // TH) * tpr + (x // TW)).astype(np.int64) * (TH * TW) + ((y % TH) * TW + (x % TW))
    return np.argsort(k.reshape(-1), kind="stable").astype(np.int32)


def quantize_u8(x, per_channel=False):
    """vorotracing.py:495-503 with torch-on-CUDA semantics: scale is the
    float64 (vmax-vmin)/255 rounded to fp32; q = round_half_even((x - vmin)
    * fp32(1/scale)) clamped to [0,255] (PyTorch's CUDA true-division by a CPU
    scalar multiplies by the fp32 reciprocal).  per_channel: one (scale,
    offset) per RGB channel of the (N, 3*R*R) texel-major map."""
    x = np.asarray(x, np.float32)
    if per_channel:
        xv = x.reshape(x.shape[0], -1, 3)
        scales, offs = [], []
        q = np.empty(xv.shape, np.uint8)
        for c in range(3):
            qc, s, o = quantize_u8(xv[:, :, c])
            q[:, :, c] = qc
            scales.append(s)
            offs.append(o)
        return q.reshape(x.shape), np.array(scales, np.float32), np.array(offs, np.float32)
    vmin = float(x.min())
    vmax = float(x.max())
    scale = (vmax - vmin) / 255.0
    inv = np.float32(1.0) / np.float32(scale)
    q = np.rint((x - np.float32(vmin)) * inv)
    q = np.clip(q, 0, 255).astype(np.uint8)
    return q, np.float32(scale), np.float32(vmin)


def pad_3to4(x, R):
    """vorotracing.py:505-512: (N, 3RR) -> (N, 4RR) with a zero 4th channel."""
    x = np.asarray(x)
    n = x.shape[0]
    t = x.reshape(n, R * R, 3)
    out = np.zeros((n, R * R, 4), x.dtype)
    out[:, :, :3] = t
    return out.reshape(n, 4 * R * R)


def nearest_site(points, queries, threads=0):
    """Brute-force exact nearest site (ties -> lowest index), int32."""
    import ctypes as C

    points = np.ascontiguousarray(points, np.float32)
    queries = np.ascontiguousarray(queries, np.float32).reshape(-1, 3)
    out = np.empty(queries.shape[0], np.int32)
    core.lib().or_nearest_site(core._p(points), C.c_uint32(points.shape[0]), core._p(queries),
                               C.c_uint32(queries.shape[0]), core._p(out), C.c_int(threads))
    return out
