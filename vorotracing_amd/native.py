"""Torch-tensor wrappers over the full C ABI (include/vt_abi.h), including
options the reference surface does not expose: per-ray walk statistics,
in-kernel wave tiling, explicit streams.  Used by the callers in infer.py,
the benchmark and the tests.  No validation beyond what the library does:
callers pass contiguous device tensors of the documented dtypes.
"""
from __future__ import annotations

import ctypes as C
import math
import weakref
from typing import Optional, Tuple

import torch

from . import _lib

STATS_WORDS = 32  # vt_ray_stats: 8 counter words and the first 24 visited cells

# Side of the 8x8 wave tiles: leading ray dimensions with at least this many
# rows and columns are traced as images.
IMAGE_MIN = 8


def screen_layout(lead) -> Optional[Tuple[int, int, int]]:
    """(images, rows, columns) of rays whose leading shape ``lead`` holds
    images for the wave tiling, or None for a flat batch.  (..., H, W) with
    H, W >= IMAGE_MIN is a batch of H x W images; (..., H, W, S) with
    S < IMAGE_MIN rays per pixel (the reference's full antialiasing, five per
    pixel, datasets.py:159-176) is a batch of H x (W*S) images, a pixel's rays
    side by side."""
    lead = tuple(int(x) for x in lead)
    n = len(lead)
    if n >= 2 and lead[-2] >= IMAGE_MIN and lead[-1] >= IMAGE_MIN:
        return math.prod(lead[:-2]), lead[-2], lead[-1]
    if n >= 3 and lead[-1] < IMAGE_MIN and lead[-3] >= IMAGE_MIN and lead[-2] >= IMAGE_MIN:
        return math.prod(lead[:-3]), lead[-3], lead[-2] * lead[-1]
    return None


def _p(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _s(device, stream=None) -> int:
    if stream is None:
        stream = torch.cuda.current_stream(device)
    return stream.cuda_stream


def new_stats(num_rays: int, device) -> torch.Tensor:
    return torch.zeros((num_rays, STATS_WORDS), dtype=torch.uint32, device=device)


def map_res(width: int, channels: int) -> int:
    import math

    r = int(round(math.sqrt(width / channels)))
    if r * r * channels != width:
        raise ValueError(f"map width {width} is not {channels}*R*R")
    return r


def math_probe(op: int, x: torch.Tensor) -> torch.Tensor:
    """Elementwise device arithmetic (op 0-4); for op 5 the walk's exit-face
    order on the rows (num, dp, bnum, bdp) of an (n, 4) float32 tensor; for
    op 6 the walk's exit-face search on the rows of an (n, 26) float32 tensor
    (site, origin, direction, face count as int32 bits, 8 half4 records as
    16 words), giving (face index, t1 bits) per row; for op 7 the packed
    walk's search on (n, 30) rows (an op 6 row in slot order, then the slots'
    original indices as 8 u16), giving (original index, t1 bits)."""
    x = x.contiguous()
    if op == 5:
        if x.dim() != 2 or x.size(1) != 4 or x.dtype != torch.float32:
            raise ValueError("op 5 takes an (n, 4) float32 tensor of (num, dp, bnum, bdp)")
        n = x.size(0)
        out = torch.empty(n, dtype=torch.uint32, device=x.device)
    elif op in (6, 7):
        width = 26 if op == 6 else 30
        if x.dim() != 2 or x.size(1) != width or x.dtype != torch.float32:
            raise ValueError(f"op {op} takes an (n, {width}) float32 tensor of exit-face rows")
        n = x.size(0)
        out = torch.empty((n, 2), dtype=torch.uint32, device=x.device)
    else:
        n = x.numel()
        out = torch.empty(x.shape, dtype=torch.uint32, device=x.device)
    _lib.call("vt_math_probe", op, x.data_ptr(), out.data_ptr(), n, _s(x.device))
    return out


def prefetch(points, adjacency, offsets, out=None, stream=None):
    n = points.size(0)
    m = adjacency.size(0)
    if out is None:
        out = torch.empty((m + 32, 4), dtype=torch.float16, device=points.device)
    _lib.call("vt_prefetch_adj", points.data_ptr(), n, adjacency.data_ptr(), m, offsets.data_ptr(), out.data_ptr(),
              _s(points.device, stream))
    return out


def image_dims(rays) -> Tuple[int, int, int]:
    """(images, rows, columns) for the tiled entries: screen_layout of the
    rays, else their last two leading dimensions."""
    lead = rays.shape[:-1]
    lay = screen_layout(lead)
    if lay is None:
        lay = (math.prod(lead[:-2]), int(lead[-2]), int(lead[-1]))
    return lay


def num_tiles(images: int, H: int, W: int, tile_h: int = IMAGE_MIN, tile_w: int = IMAGE_MIN) -> int:
    return int(images) * ((int(H) + tile_h - 1) // tile_h) * ((int(W) + tile_w - 1) // tile_w)


class TileSchedule:
    """Launch order of the screen tiles of a frame rendered again (the same
    rays or cameras on one stream; vt_tile_order): each launch records its
    tiles' costs, and the next render of the same frame launches the tiles
    by decreasing cost, so that it does not end with a few long tiles on an
    otherwise idle GPU (C3, one view rendered repeatedly: 2-7 % per frame).
    A different frame launches in screen order: the costs of the previous
    view mispredict a moved camera's (a 32-pose orbit ran 10 % slower with
    them).  Images are bit-identical in any order.  One schedule per stream:
    a launch reads the costs the previous launch on its stream wrote.

    The walk is deterministic, so every render of unchanged rays records the
    same costs and their sort gives the same order: without a split
    (``split_waves`` 0, the inference entries) the order sorted for a frame
    is kept for its further renders instead of being sorted again.  Each
    render still records its costs."""

    def __init__(self, tiles: int, device, split_waves: int = 0):
        self.tiles = int(tiles)
        # waves the training backward holds at once (the split count of the
        # orders order_for makes; 0: none)
        self.split_waves = int(split_waves)
        self.cost = torch.zeros(self.tiles, dtype=torch.uint32, device=device)
        # the order, then the split count
        self.order = torch.empty(self.tiles + 1, dtype=torch.uint32, device=device)
        self.ws = torch.empty(int(_lib.load().vt_tile_order_workspace_size(self.tiles)), dtype=torch.uint8,
                              device=device)
        self.frame = None  # the frame whose costs self.cost holds
        self.sorted = None  # the frame self.order was sorted for (split_waves 0)

    def _sort(self, stream: int, split_waves: int):
        _lib.call("vt_tile_order", self.cost.data_ptr(), self.tiles, split_waves, self.order.data_ptr(),
                  self.ws.data_ptr(), stream)
        return self.order.data_ptr()

    def launch_args(self, stream: int, frame, split_waves: int = 0):
        """(tile_order, tile_cost) pointers for the next launch on ``stream``
        of ``frame`` (a hashable identity of the launch's rays or cameras).
        ``split_waves``: 0 for the inference entries; the waves the training
        forward holds at once for it, which may then split its costliest
        tiles and record their costs with an atomic max, into costs cleared
        here after the sort has read them."""
        order = None
        if frame is not None and frame == self.frame:
            if split_waves:
                order = self._sort(stream, split_waves)
                self.cost.zero_()
            elif frame == self.sorted:
                order = self.order.data_ptr()
            else:
                order = self._sort(stream, 0)
                self.sorted = frame
        self.frame = frame
        return order, self.cost.data_ptr()

    def order_for(self, stream: int, frame):
        """Launch order from the costs the last launch of ``frame`` recorded
        (the training backward after the forward over the same rays), or
        None when the costs are of another frame."""
        if frame is None or frame != self.frame:
            return None
        self.sorted = None
        return self._sort(stream, self.split_waves)


def frame_key(t: torch.Tensor):
    """Identity of a frame's rays: the tensor object, its storage and its
    in-place version (rays rendered again unchanged keep all three).  The
    schedule only moves work between lanes, so a stale key costs time, not
    correctness."""
    return (id(t), t.data_ptr(), t._version)


def schedule_for(cache: dict, key, tiles: int, device, limit: int = 16, split_waves: int = 0) -> TileSchedule:
    """The TileSchedule of ``key`` in ``cache`` (created on first use; the
    cache keeps the ``limit`` most recent)."""
    sch = cache.pop(key, None)
    if sch is None or sch.tiles != tiles or sch.split_waves != split_waves:
        sch = TileSchedule(tiles, device, split_waves)
    cache[key] = sch
    while len(cache) > limit:
        cache.pop(next(iter(cache)))
    return sch


class SourceKey:
    """Identity of a set of source tensors for data derived from them: the
    tensors themselves (weak references, so a freed source never matches),
    their storage and their in-place version."""

    def __init__(self, *sources):
        self._refs = [weakref.ref(t) for t in sources]
        self._state = [(t.data_ptr(), t._version) for t in sources]

    def matches(self, *sources) -> bool:
        return len(sources) == len(self._refs) and all(
            r() is t and (t.data_ptr(), t._version) == st for r, t, st in zip(self._refs, sources, self._state))


class _WalkLayoutC(C.Structure):
    _fields_ = [("chunks", C.c_void_p), ("links", C.c_void_p), ("heads", C.c_void_p), ("cells", C.c_void_p),
                ("orig", C.c_void_p), ("num_chunks", C.c_uint32)]


class WalkLayout:
    """The packed walk layout of a scene (vt_walk_layout): face records in
    16-byte-aligned chunks of 8 (6 bytes each, no pad half), a link per
    padded face slot carrying the neighbour's chunk range, and a {site,
    density} record per cell.  The inference kernels walk it with fewer
    vector loads per step and render the same images bit for bit.
    ``face_order`` (0: list order; 1, 2, 3: by the x, y or z of the offsets)
    lays out each cell's faces so that the lanes of a wave meet
    forward-facing faces at the same slots (``orig`` keeps the original
    indices for exact ties); 3 suits scenes whose views look up or down.

    ``build`` returns None for a scene beyond the layout's limits (2^24 cells,
    255 chunks per cell); the renders then walk the reference's arrays.
    ``source`` (a SourceKey) tells whether the arrays it was built from are
    still the given tensors, unchanged."""

    MAX_POINTS = 1 << 24
    MAX_CHUNKS_PER_CELL = 255

    def __init__(self, chunks, links, heads, cells, orig, num_chunks: int, face_order: int = 0, sources=()):
        self.chunks, self.links, self.heads, self.cells, self.orig = chunks, links, heads, cells, orig
        self.num_chunks = int(num_chunks)
        self.face_order = int(face_order)
        self.source = SourceKey(*sources)
        self._c = _WalkLayoutC(chunks.data_ptr(), links.data_ptr(), heads.data_ptr(), cells.data_ptr(),
                               orig.data_ptr(), self.num_chunks)

    @property
    def ptr(self) -> int:
        """Address of the vt_walk_layout struct (host memory) for the C ABI."""
        return C.addressof(self._c)


    @classmethod
    def build(cls, points, density, adjacency, offsets, adj_diff, stream=None,
              face_order: int = 3) -> Optional["WalkLayout"]:
        """The layout of a scene (density: f32 per cell, as the renders take
        it; adj_diff from vt_prefetch_adj), or None beyond the limits.  Reads
        two counts back to the host to size the arrays; raises ValueError when
        the adjacency names a cell past the scene's last."""
        n = int(points.shape[0])
        if n >= cls.MAX_POINTS:
            return None
        dev = points.device
        sources = (points, density, adjacency, offsets, adj_diff)
        density = density.reshape(-1)
        sp = _s(dev, stream)
        lib = _lib.load()
        first = torch.empty(n + 2, dtype=torch.int32, device=dev)
        ws = torch.empty(max(int(lib.vt_walk_layout_count_workspace_size(n)), 1), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            _lib.call("vt_walk_layout_count", offsets.data_ptr(), adjacency.data_ptr(), n, first.data_ptr(),
                      ws.data_ptr(), sp)
            torch.cuda.synchronize(dev)
            total, most = (int(v) & 0xFFFFFFFF for v in first[n:].cpu().tolist())
        if most >> 31:
            raise ValueError(f"the adjacency holds a neighbour id of {n} or more (the scene has {n} cells)")
        if most > cls.MAX_CHUNKS_PER_CELL or total >= (1 << 29):
            return None
        # one chunk past the last: the walk loads a cell's first chunk before it knows the list is not empty
        chunks = torch.zeros((total + 1, 12), dtype=torch.int32, device=dev)
        links = torch.empty((max(8 * total, 1), 2), dtype=torch.int32, device=dev)
        heads = torch.empty((max(n, 1), 2), dtype=torch.int32, device=dev)
        cells = torch.empty((max(n, 1), 4), dtype=torch.float32, device=dev)
        orig = torch.empty(max(8 * total, 1), dtype=torch.int16, device=dev)
        with torch.cuda.device(dev):
            _lib.call("vt_walk_layout_fill", points.data_ptr(), density.data_ptr(), adjacency.data_ptr(),
                      offsets.data_ptr(), n, adj_diff.data_ptr(), first.data_ptr(), total, int(face_order),
                      chunks.data_ptr(), links.data_ptr(), heads.data_ptr(), cells.data_ptr(), orig.data_ptr(), sp)
        return cls(chunks, links, heads, cells, orig, total, face_order, sources)


def _walk_ptr(walk: Optional[WalkLayout]):
    return walk.ptr if walk is not None else None


class _QuadMapsC(C.Structure):
    _fields_ = [("diffuse", C.c_void_p), ("specular", C.c_void_p), ("num_points", C.c_uint32),
                ("diff_res", C.c_uint32), ("spec_res", C.c_uint32), ("format", C.c_uint32)]


QUAD_F16, QUAD_Q8 = 0, 1


class QuadMaps:
    """Footprint tables of a scene's octahedral maps (vt_quad_maps): per cell,
    (R + 1)^2 entries, each the four wrapped texels of one bilinear tap, so
    that the inference kernels read a tap with two 16-byte loads (fp16 maps:
    32-byte entries, instead of four 8-byte texels) or one (q8 maps: 16-byte
    entries, instead of twelve bytes) and render the same images bit for bit.
    ``format`` is QUAD_F16 or QUAD_Q8.  ``source`` (a SourceKey) tells whether
    the maps they were built from are still the given tensors, unchanged."""

    def __init__(self, diffuse, specular, num_points: int, diff_res: int, spec_res: int, sources=(),
                 format: int = QUAD_F16):
        self.diffuse, self.specular = diffuse, specular
        self.num_points, self.diff_res, self.spec_res = int(num_points), int(diff_res), int(spec_res)
        self.format = int(format)
        self.source = SourceKey(*sources)
        self._c = _QuadMapsC(diffuse.data_ptr(), specular.data_ptr(), self.num_points, self.diff_res,
                             self.spec_res, self.format)

    @property
    def ptr(self) -> int:
        """Address of the vt_quad_maps struct (host memory) for the C ABI."""
        return C.addressof(self._c)

    @staticmethod
    def table(maps4, stream=None):
        """The footprint table of one Half4Texel map (f16 (N, 4 R^2))."""
        maps4 = maps4.contiguous()
        res = map_res(maps4.shape[-1], 4)
        n = maps4.numel() // (4 * res * res)
        out = torch.empty((max(n, 1), 16 * (res + 1) ** 2), dtype=torch.float16, device=maps4.device)
        with torch.cuda.device(maps4.device):
            _lib.call("vt_quad_maps_f16", maps4.data_ptr(), n, res, out.data_ptr(), _s(maps4.device, stream))
        return out

    @staticmethod
    def table_q8(maps_q8, stream=None):
        """The footprint table of one q8 map (u8 (N, 3 R^2))."""
        maps_q8 = maps_q8.contiguous()
        res = map_res(maps_q8.shape[-1], 3)
        n = maps_q8.numel() // (3 * res * res)
        out = torch.empty((max(n, 1), 16 * (res + 1) ** 2), dtype=torch.uint8, device=maps_q8.device)
        with torch.cuda.device(maps_q8.device):
            _lib.call("vt_quad_maps_q8", maps_q8.data_ptr(), n, res, out.data_ptr(), _s(maps_q8.device, stream))
        return out

    # the share of the device's free memory the tables may take; beyond it
    # build_within returns None and the renders read the maps themselves
    MAX_FREE_SHARE = 0.25

    @staticmethod
    def table_bytes(diffuse, specular) -> int:
        """Bytes of the two tables of these maps."""
        q8 = diffuse.dtype == torch.uint8
        per = 16 if q8 else 32
        rd = map_res(diffuse.shape[-1], 3 if q8 else 4)
        rs = map_res(specular.shape[-1], 3 if q8 else 4)
        return int(diffuse.shape[0]) * per * ((rd + 1) ** 2 + (rs + 1) ** 2)

    @classmethod
    def build_within(cls, diffuse, specular, stream=None) -> Optional["QuadMaps"]:
        """build(), or None when the tables would take more than
        MAX_FREE_SHARE of the device's free memory."""
        free, _ = torch.cuda.mem_get_info(diffuse.device)
        if cls.table_bytes(diffuse, specular) > cls.MAX_FREE_SHARE * free:
            return None
        return cls.build(diffuse, specular, stream)

    @classmethod
    def build(cls, diffuse, specular, stream=None) -> "QuadMaps":
        """The tables of a scene's two maps (one row per cell): Half4Texel f16
        maps give fp16 tables, u8 maps q8 tables."""
        if diffuse.shape[0] != specular.shape[0]:
            raise ValueError(f"the maps have {diffuse.shape[0]} and {specular.shape[0]} rows")
        if diffuse.dtype == torch.uint8:
            return cls(cls.table_q8(diffuse, stream), cls.table_q8(specular, stream), diffuse.shape[0],
                       map_res(diffuse.shape[-1], 3), map_res(specular.shape[-1], 3), (diffuse, specular), QUAD_Q8)
        return cls(cls.table(diffuse, stream), cls.table(specular, stream), diffuse.shape[0],
                   map_res(diffuse.shape[-1], 4), map_res(specular.shape[-1], 4), (diffuse, specular), QUAD_F16)


def _quads_ptr(quads: Optional[QuadMaps]):
    return quads.ptr if quads is not None else None


def infer_f16(points, diffuse4, specular4, density, adjacency, offsets, adj_diff, rays, start_point, ray_perm=None,
              weight_threshold=0.001, max_intersections=1024, cell_skip_threshold=0.0, stats=None, out=None,
              tiled=None, stream=None, schedule: Optional[TileSchedule] = None, walk: Optional[WalkLayout] = None,
              rays_per_start: int = 0, quads: Optional[QuadMaps] = None):
    """fp16 inference.  ``tiled=(tile_h, tile_w)`` uses the in-kernel wave
    tiling over the images of screen_layout (any (..., H, W, 6) when the
    layout finds none), with ``schedule`` (a TileSchedule of this image
    shape and stream) the tiles' launch order, ``walk`` (a WalkLayout of
    the scene) the packed walk, ``rays_per_start`` the rays that share
    each entry of ``start_point`` (0: one per ray), and ``quads`` (the
    QuadMaps of the maps) the footprint tables read in place of the maps."""
    rd = map_res(diffuse4.shape[-1], 4)
    rs = map_res(specular4.shape[-1], 4)
    nr = rays.numel() // 6
    if out is None:
        out = torch.empty(list(rays.shape[:-1]) + [4], dtype=torch.float16, device=rays.device)
    dev = rays.device
    if tiled is not None:
        B, H, W = image_dims(rays)
        sp = _s(dev, stream)
        order, cost = schedule.launch_args(sp, frame_key(rays)) if schedule is not None else (None, None)
        _lib.call("vt_trace_infer_f16_tiled", points.data_ptr(), diffuse4.data_ptr(), specular4.data_ptr(), rd, rs,
                  density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(), points.size(0), adj_diff.data_ptr(),
                  rays.data_ptr(), B, H, W, tiled[0], tiled[1], start_point.data_ptr(), int(rays_per_start),
                  float(weight_threshold),
                  int(max_intersections), float(cell_skip_threshold), out.data_ptr(), order, cost, _p(stats),
                  _walk_ptr(walk), _quads_ptr(quads), sp)
    else:
        if quads is not None:
            raise ValueError("quads (footprint tables) are read by the tiled fp16 renders only")
        _lib.call("vt_trace_infer_f16", points.data_ptr(), diffuse4.data_ptr(), specular4.data_ptr(), rd, rs,
                  density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(), points.size(0), adj_diff.data_ptr(),
                  rays.data_ptr(), nr, start_point.data_ptr(), _p(ray_perm), float(weight_threshold),
                  int(max_intersections), float(cell_skip_threshold), out.data_ptr(), _p(stats), _s(dev, stream))
    return out


def infer_q8(points, diffuse_q8, specular_q8, scales, density, adjacency, offsets, adj_diff, rays, start_point,
             ray_perm=None, weight_threshold=0.001, max_intersections=1024, cell_skip_threshold=0.0, stats=None,
             out=None, stream=None):
    """q8 inference; ``scales`` = (diff_scale[3], diff_offset[3], spec_scale[3], spec_offset[3])."""
    rd = map_res(diffuse_q8.shape[-1], 3)
    rs = map_res(specular_q8.shape[-1], 3)
    nr = rays.numel() // 6
    if out is None:
        out = torch.empty(list(rays.shape[:-1]) + [4], dtype=torch.float16, device=rays.device)
    arrs = [(C.c_float * 3)(*[float(v) for v in torch.as_tensor(x, dtype=torch.float32).reshape(-1).tolist()])
            for x in scales]
    _lib.call("vt_trace_infer_q8", points.data_ptr(), diffuse_q8.data_ptr(), specular_q8.data_ptr(), rd, rs,
              *[C.cast(a, C.c_void_p) for a in arrs], density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(),
              points.size(0), adj_diff.data_ptr(), rays.data_ptr(), nr, start_point.data_ptr(), _p(ray_perm),
              float(weight_threshold), int(max_intersections), float(cell_skip_threshold), out.data_ptr(), _p(stats),
              _s(rays.device, stream))
    return out


def upload_cameras(cameras, device) -> torch.Tensor:
    """The vt_camera records of a batch of ``camera.Camera`` (one image size) as a
    device buffer (u8), the form the camera entries of the C ABI take."""
    from .camera import pack_cameras

    blob = pack_cameras(list(cameras))
    return torch.frombuffer(bytearray(blob), dtype=torch.uint8).to(device)


def camera_rays(cameras, device, out=None, width=None, stream=None, camera_buffer=None):
    """Rays (B, H, W, 6) f32 of a batch of ``camera.Camera`` (one image size),
    generated on the GPU by vt_camera_rays: the rays the camera renders trace.
    ``width=1`` gives each row's origin (start cells of rolling shutters)."""
    cams = list(cameras)
    if camera_buffer is None:
        camera_buffer = upload_cameras(cams, device)
    H, W = cams[0].height, cams[0].width if width is None else width
    if out is None:
        out = torch.empty((len(cams), H, W, 6), dtype=torch.float32, device=device)
    _lib.call("vt_camera_rays", camera_buffer.data_ptr(), len(cams), H, W, out.data_ptr(), _s(device, stream))
    return out
