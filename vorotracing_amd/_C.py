"""The reference's ``_C`` operator module, backed by libvt_hip.so.

Same functions, argument order, return tuples, validation order and error
messages as vorotracing/cuda/csrc/ext.cpp:11-34 (declarations
tracing_octmap.h:11-91, nn_bvh.h:4-16).  Inputs are made contiguous,
outputs are allocated with torch on the input device, and kernels are
enqueued on torch's current stream (the reference uses the legacy default
stream, tracing_octmap.cu:460-461; under default usage the two coincide).
Failed checks raise RuntimeError with the reference's message.
"""
from __future__ import annotations

import math
from typing import Optional, Sequence, Union

import torch

from . import _lib, native

_C10_NAMES = {
    torch.float32: "Float", torch.float64: "Double", torch.float16: "Half", torch.bfloat16: "BFloat16",
    torch.int32: "Int", torch.int64: "Long", torch.int16: "Short", torch.int8: "Char", torch.uint8: "Byte",
    torch.bool: "Bool", torch.uint32: "UInt32", torch.uint16: "UInt16", torch.uint64: "UInt64",
}

MAX_MAP_RES = (4, 8)


def _assert(cond, msg):
    if not cond:
        raise RuntimeError(msg)


def _is_gpu(t: torch.Tensor) -> bool:
    return t.device.type == "cuda"


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def validate_scene_data(points, attributes, point_adjacency, point_adjacency_offsets):
    """validations.h:17-66, same order and messages."""
    if points.size(-1) != 3:
        raise RuntimeError(f"points had dimension {points.size(-1)} along axis -1, expected 3")
    if points.dtype != torch.float32:
        raise RuntimeError(f"points had dtype {_C10_NAMES.get(points.dtype, str(points.dtype))}, expected float32")
    if not _is_gpu(points):
        raise RuntimeError("points must be on CUDA device")
    num_points = points.numel() // 3
    if not _is_gpu(attributes):
        raise RuntimeError("attributes must be on CUDA device")
    if point_adjacency_offsets.dtype != torch.uint32:
        raise RuntimeError("point_adjacency_offsets must have uint32 dtype")
    if not _is_gpu(point_adjacency_offsets):
        raise RuntimeError("point_adjacency_offsets must be on CUDA device")
    if point_adjacency_offsets.numel() != num_points + 1:
        raise RuntimeError("point_adjacency_offsets must have num_points + 1 elements")
    if point_adjacency.dtype != torch.uint32:
        raise RuntimeError("point_adjacency must have uint32 dtype")
    if not _is_gpu(point_adjacency):
        raise RuntimeError("point_adjacency must be on CUDA device")


def _map_res(width: int, channels: int, what: str) -> int:
    r = int(round(math.sqrt(width / channels))) if width > 0 else 0
    if r * r * channels != width or r not in MAX_MAP_RES:
        raise RuntimeError(
            f"{what} width {width} is not {channels}*R*R for a compiled octahedral resolution R in {MAX_MAP_RES}")
    return r


def _u32_view(t: torch.Tensor) -> torch.Tensor:
    """int32 -> uint32 reinterpretation (the reference reads ray_perm int32 as u32)."""
    if t.dtype == torch.int32:
        return t.view(torch.uint32)
    return t


# Explicit ray_perm tensors already checked: id -> (weak reference, _version, num_rays, verdict).
# Callers pass the same cached tensor every frame (the reference's _tile_perm,
# vorotracing.py:606-625), so the device check and its host sync run once per
# tensor and again only after an in-place change.
_PERM_CHECKED: dict = {}


def _remember_perm(t: torch.Tensor, num_rays: int, ok: bool) -> None:
    import weakref

    if len(_PERM_CHECKED) >= 64:
        for k in [k for k, v in _PERM_CHECKED.items() if v[0]() is None]:
            del _PERM_CHECKED[k]
        if len(_PERM_CHECKED) >= 64:
            _PERM_CHECKED.clear()
    _PERM_CHECKED[id(t)] = (weakref.ref(t), t._version, int(num_rays), ok)


def is_permutation(perm: torch.Tensor, num_rays: int) -> bool:
    """Whether ``perm`` (int32 or uint32, read as uint32) holds every index
    0..num_rays-1 exactly once.  With duplicates some rays would never be
    traced (their outputs left unwritten) and lanes sharing a ray would race
    on its outputs, so the entries reject such a ``ray_perm``."""
    hit = _PERM_CHECKED.get(id(perm))
    if hit is not None and hit[0]() is perm and hit[1] == perm._version and hit[2] == num_rays:
        return hit[3]
    flat = perm.reshape(-1)
    if flat.numel() != num_rays or flat.dtype not in (torch.int32, torch.uint32):
        return False
    if num_rays == 0:
        ok = True
    else:
        wide = flat.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
        # entries >= num_rays land in the last bin; n entries fill bins 0..n-1
        # once each only when none is out of range or repeated
        counts = torch.bincount(wide.clamp_(max=num_rays), minlength=num_rays + 1)
        ok = bool(counts[:num_rays].eq(1).all().item())
    _remember_perm(perm, num_rays, ok)
    return ok


# Tile launch schedules of the drop-in inference entries (native.TileSchedule),
# keyed by the caller's ray_perm tensor (the reference caches one per
# resolution, vorotracing.py:606-625), the image shape and the stream.
_SCHEDULES: dict = {}


def _drop_in_schedule(ray_perm_in: torch.Tensor, lay, device) -> "native.TileSchedule":
    key = (id(ray_perm_in), tuple(lay), _stream(device))
    return native.schedule_for(_SCHEDULES, key, native.num_tiles(*lay), device)


# Packed walk layouts (native.WalkLayout) of the scenes the tiled drop-in
# renders walk: built on a scene's first image render and reused while the
# caller's five scene arrays are the same tensors, unchanged (native.SourceKey).
# The layout walks with fewer vector loads per step and renders the same image.
DROP_IN_WALK = True
DROP_IN_FACE_ORDER = 3
_WALK_LAYOUTS: list = []


def _drop_in_walk(srcs_in, srcs) -> Optional["native.WalkLayout"]:
    """The walk layout of the scene whose arrays are ``srcs_in`` (points,
    density, adjacency, offsets, adjacent_diff as the caller passed them),
    built from their contiguous forms ``srcs``; None when off or beyond the
    layout's limits."""
    if not DROP_IN_WALK:
        return None
    for i, (key, wl) in enumerate(_WALK_LAYOUTS):
        if key.matches(*srcs_in) and (wl is None or wl.face_order == DROP_IN_FACE_ORDER):
            _WALK_LAYOUTS.append(_WALK_LAYOUTS.pop(i))
            return wl
    entry = (native.SourceKey(*srcs_in), native.WalkLayout.build(*srcs, face_order=DROP_IN_FACE_ORDER))
    _WALK_LAYOUTS.append(entry)
    del _WALK_LAYOUTS[:-2]
    return entry[1]


# Footprint tables (native.QuadMaps) of the maps the tiled drop-in renders
# read (fp16 or q8): built on a scene's first image render and reused while
# the caller's two map tensors are the same, unchanged.  A bilinear tap then
# reads its four texels with two 16-byte loads (fp16) or one (q8); the image
# is the same.
DROP_IN_QUADS = True
_QUAD_MAPS: list = []


def _drop_in_quads(maps_in, maps) -> Optional["native.QuadMaps"]:
    """The footprint tables of the maps ``maps_in`` (diffuse, specular as the
    caller passed them), built from their contiguous forms ``maps``; None
    when off or when they would take too much of the free memory."""
    if not DROP_IN_QUADS:
        return None
    for i, (key, qm) in enumerate(_QUAD_MAPS):
        if key.matches(*maps_in):
            _QUAD_MAPS.append(_QUAD_MAPS.pop(i))
            return qm
    # None when the tables would take too much of the free memory (native.QuadMaps.MAX_FREE_SHARE)
    entry = (native.SourceKey(*maps_in), native.QuadMaps.build_within(*maps))
    _QUAD_MAPS.append(entry)
    del _QUAD_MAPS[:-2]
    return entry[1]


# Tile launch schedules of the training entries for tiled rays, keyed by the
# image shape and stream: the forward (in screen order) records its tiles'
# costs, and the backward of the same rays (the same tensor, unchanged)
# launches its tiles by decreasing cost.  A single C2 camera has 7,500 tiles
# for 4,096 backward wave slots; in screen order its backward lost about a
# quarter of its time to the tiles that run last (C2 backward 3.95 -> 3.40
# ms).  Both passes also run their costliest tiles as two half-waves each
# (vt_tile_order's split count over the waves the device holds of that
# kernel at once): at C2 each launch otherwise ends with the few costliest
# tiles, started first and still running alone (backward 3.38 -> 2.84 ms).
# The forward takes the previous forward's costs of the same rays, and only
# when it splits (an order alone made it slower, 1.16 -> 1.18 ms; with the
# split 1.15 -> 1.06 ms).  At C5 (25,350 tiles) no tile exceeds the share
# and nothing is split.  TRAIN_SPLIT_WAVES overrides the resident-wave counts
# of both (0: no split; tests use large values to split small frames).
TRAIN_TILE_ORDER = True
TRAIN_SPLIT_WAVES: Optional[int] = None
_TRAIN_SCHEDULES: dict = {}


def _train_schedule(rays_in, img_h: int, img_w: int, num_rays: int, perm, ray_perm_arg, device):
    """(schedule, frame) of a training launch, or (None, None) without tiles.
    Image lanes: screen tiles, one schedule per image shape and stream, the
    frame being the rays tensor.  A ray_perm lane order (a sorted flat
    batch): waves of 64 consecutive ray_perm entries, one schedule per ray
    count and stream, the frame being the rays and the permutation tensors
    (the autograd path hands the forward's permutation to the backward; a
    permutation made inside each entry, "auto", has no frame)."""
    if not TRAIN_TILE_ORDER:
        return None, None
    if perm is not None:
        tiles = (num_rays + 63) // 64
        key = ("perm", tiles, _stream(device))
        frame = ((native.frame_key(rays_in), native.frame_key(ray_perm_arg))
                 if isinstance(ray_perm_arg, torch.Tensor) else None)
    elif img_h:
        images = num_rays // (img_h * img_w)
        tiles = native.num_tiles(images, img_h, img_w)
        key = (images, img_h, img_w, _stream(device))
        frame = native.frame_key(rays_in)
    else:
        return None, None
    return native.schedule_for(_TRAIN_SCHEDULES, key, tiles, device, split_waves=_split_waves("bwd")), frame


def _split_waves(kernel: str) -> int:
    if TRAIN_SPLIT_WAVES is not None:
        return int(TRAIN_SPLIT_WAVES)
    return int(getattr(_lib.load(), f"vt_train_{kernel}_resident_waves")())


def _checked_perm(ray_perm_in: torch.Tensor, num_rays: int) -> torch.Tensor:
    """uint32 view of an explicit lane order that is a permutation of the rays."""
    _assert(ray_perm_in.numel() == num_rays, "ray_perm must be empty or have one entry per ray")
    _assert(ray_perm_in.dtype in (torch.int32, torch.uint32), "ray_perm must have int32 or uint32 dtype")
    _assert(is_permutation(ray_perm_in, num_rays), "ray_perm must be a permutation of the ray indices")
    return _u32_view(ray_perm_in.contiguous())


def trace_vorotracing_prefetch_adj(points_in, point_adjacency_in, point_adjacency_offsets_in):
    """tracing_octmap.cu:612-640: f16 (adjacency_size + 32, 4) per-face site offsets."""
    points = points_in.contiguous()
    adjacency = point_adjacency_in.contiguous()
    offsets = point_adjacency_offsets_in.contiguous()
    num_points = points.size(0)
    adjacency_size = adjacency.size(0)
    adj_diff = torch.empty((adjacency_size + 32, 4), dtype=torch.float16, device=points.device)
    with torch.cuda.device(points.device):
        _lib.call("vt_prefetch_adj", points.data_ptr(), num_points, adjacency.data_ptr(), adjacency_size,
                  offsets.data_ptr(), adj_diff.data_ptr(), _stream(points.device))
    return adj_diff


def _out_shape(rays, last):
    return list(rays.shape[:-1]) + [last]


def trace_vorotracing_infer(points_in, diffuse_in, specular_in, density_in, point_adjacency_in,
                            point_adjacency_offsets_in, rays_in, start_point_in, adjacent_diff_in, ray_perm_in,
                            weight_threshold: float, max_intersections: int, cell_skip_threshold: float):
    """tracing_octmap.cu:642-717 (fp16 Half4Texel inference).  Returns f16 [..., 4]."""
    points = points_in.contiguous()
    diffuse = diffuse_in.contiguous()
    specular = specular_in.contiguous()
    density = density_in.contiguous()
    adjacency = point_adjacency_in.contiguous()
    offsets = point_adjacency_offsets_in.contiguous()
    rays = rays_in.contiguous()
    start_point = start_point_in.contiguous()
    adjacent_diff = adjacent_diff_in.contiguous()
    validate_scene_data(points_in, diffuse_in, point_adjacency_in, point_adjacency_offsets_in)
    num_points = points.size(0)
    num_rays = rays.numel() // 6
    _assert(diffuse.dtype == torch.float16, "inference kernel requires float16 diffuse")
    _assert(specular.dtype == torch.float16, "inference kernel requires float16 specular")
    _assert(density.dtype == torch.float32, "density must have float32 dtype")
    _assert(rays.dtype == torch.float32, "rays must have float32 dtype")
    _assert(start_point.dtype == torch.uint32, "start_point must have uint32 dtype")
    _check_infer_shapes(num_points, num_rays, diffuse, specular, density, start_point, adjacent_diff, adjacency)
    rd = _map_res(diffuse.shape[-1], 4, "diffuse")
    rs = _map_res(specular.shape[-1], 4, "specular")
    ray_perm = _checked_perm(ray_perm_in, num_rays) if ray_perm_in.numel() else None
    out = torch.empty(_out_shape(rays, 4), dtype=torch.float16, device=rays.device)
    if num_rays == 0:
        return out
    # A lane order asks for coherent waves.  For image-shaped rays the kernel
    # tiles the screen itself (8x8 rays per wave64, blocks dealt to the XCDs
    # in turns), and a ray's result does not depend on which lane traces it,
    # so any permutation of an image (the reference's 4x8 warp tiles,
    # vorotracing.py:606-625) renders the same image that way, with no
    # permutation buffer read.
    lay = native.screen_layout(rays.shape[:-1]) if ray_perm is not None else None
    with torch.cuda.device(rays.device):
        if lay is not None:
            order, cost = _drop_in_schedule(ray_perm_in, lay, rays.device).launch_args(
                _stream(rays.device), native.frame_key(rays_in))
            _lib.call("vt_trace_infer_f16_tiled", points.data_ptr(), diffuse.data_ptr(), specular.data_ptr(), rd,
                      rs, density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(), num_points,
                      adjacent_diff.data_ptr(), rays.data_ptr(), lay[0], lay[1], lay[2], native.IMAGE_MIN,
                      native.IMAGE_MIN, start_point.data_ptr(), 0, float(weight_threshold), int(max_intersections),
                      float(cell_skip_threshold), out.data_ptr(), order, cost, None,
                      native._walk_ptr(_drop_in_walk(
                          (points_in, density_in, point_adjacency_in, point_adjacency_offsets_in, adjacent_diff_in),
                          (points, density, adjacency, offsets, adjacent_diff))),
                      native._quads_ptr(_drop_in_quads((diffuse_in, specular_in), (diffuse, specular))),
                      _stream(rays.device))
        else:
            _lib.call("vt_trace_infer_f16", points.data_ptr(), diffuse.data_ptr(), specular.data_ptr(), rd, rs,
                      density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(), num_points,
                      adjacent_diff.data_ptr(), rays.data_ptr(), num_rays, start_point.data_ptr(), _ptr(ray_perm),
                      float(weight_threshold), int(max_intersections), float(cell_skip_threshold), out.data_ptr(),
                      None, _stream(rays.device))
    return out


def _check_infer_shapes(num_points, num_rays, diffuse, specular, density, start_point, adjacent_diff, adjacency):
    # The reference does not check these (Appendix: the infer entries validate
    # dtypes only); out-of-range sizes would read out of bounds, so they are
    # checked here.
    _assert(diffuse.size(0) == num_points and specular.size(0) == num_points and density.numel() == num_points,
            "diffuse, specular, density must each have num_points rows")
    _assert(start_point.numel() == num_rays, "start_point must have the same batch size as rays")
    _assert(adjacent_diff.dim() == 2 and adjacent_diff.size(1) == 4 and adjacent_diff.dtype == torch.float16,
            "adjacent_diff must be float16 (adjacency_size + 32, 4)")
    # The walk reads face records 8 at a time, up to 7 rows past the last
    # list end (offsets[-1] <= adjacency rows); the reference's prefetch
    # allocates adjacency rows + 32 (tracing_octmap.cu:623-624), which covers
    # that reach without a device read of offsets[-1].
    _assert(adjacent_diff.size(0) >= adjacency.size(0) + 32,
            "adjacent_diff must have adjacency_size + 32 rows (the prefetch_adj layout)")


def trace_vorotracing_infer_q8(points_in, diffuse_in, specular_in, density_in, point_adjacency_in,
                               point_adjacency_offsets_in, rays_in, start_point_in, adjacent_diff_in,
                               diff_scale: Union[float, Sequence[float]], diff_offset, spec_scale, spec_offset,
                               weight_threshold: float, max_intersections: int, cell_skip_threshold: float,
                               ray_perm_in: Optional[torch.Tensor] = None):
    """tracing_octmap.cu:781-854 (q8 inference).  Scale/offset may be floats
    (the reference's per-tensor pair) or 3-sequences (per RGB channel).
    ``ray_perm_in`` is an extension (the reference has none); None/empty
    reproduces the reference."""
    points = points_in.contiguous()
    diffuse = diffuse_in.contiguous()
    specular = specular_in.contiguous()
    density = density_in.contiguous()
    adjacency = point_adjacency_in.contiguous()
    offsets = point_adjacency_offsets_in.contiguous()
    rays = rays_in.contiguous()
    start_point = start_point_in.contiguous()
    adjacent_diff = adjacent_diff_in.contiguous()
    validate_scene_data(points_in, diffuse_in, point_adjacency_in, point_adjacency_offsets_in)
    num_points = points.size(0)
    num_rays = rays.numel() // 6
    _assert(diffuse.dtype == torch.uint8, "q8 inference kernel requires uint8 diffuse")
    _assert(specular.dtype == torch.uint8, "q8 inference kernel requires uint8 specular")
    _assert(density.dtype == torch.float32, "density must have float32 dtype")
    _assert(rays.dtype == torch.float32, "rays must have float32 dtype")
    _assert(start_point.dtype == torch.uint32, "start_point must have uint32 dtype")
    _check_infer_shapes(num_points, num_rays, diffuse, specular, density, start_point, adjacent_diff, adjacency)
    rd = _map_res(diffuse.shape[-1], 3, "diffuse")
    rs = _map_res(specular.shape[-1], 3, "specular")
    perm = None
    if ray_perm_in is not None and ray_perm_in.numel():
        perm = _checked_perm(ray_perm_in, num_rays)

    import ctypes as C

    def v3(x):
        vals = [float(v) for v in torch.as_tensor(x, dtype=torch.float64).reshape(-1)]
        _assert(len(vals) in (1, 3), "dequantisation scale/offset must be a float or 3 values")
        return (C.c_float * 3)(*(vals * 3 if len(vals) == 1 else vals))

    ds, do, ss, so = v3(diff_scale), v3(diff_offset), v3(spec_scale), v3(spec_offset)
    out = torch.empty(_out_shape(rays, 4), dtype=torch.float16, device=rays.device)
    if num_rays == 0:
        return out
    scales = [C.cast(v, C.c_void_p) for v in (ds, do, ss, so)]
    lay = native.screen_layout(rays.shape[:-1]) if perm is not None else None
    with torch.cuda.device(rays.device):
        if lay is not None:  # a permuted image: in-kernel tiles, as trace_vorotracing_infer
            order, cost = _drop_in_schedule(ray_perm_in, lay, rays.device).launch_args(
                _stream(rays.device), native.frame_key(rays_in))
            _lib.call("vt_trace_infer_q8_tiled", points.data_ptr(), diffuse.data_ptr(), specular.data_ptr(), rd, rs,
                      *scales, density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(), num_points,
                      adjacent_diff.data_ptr(), rays.data_ptr(), lay[0], lay[1], lay[2], native.IMAGE_MIN,
                      native.IMAGE_MIN, start_point.data_ptr(), 0, float(weight_threshold), int(max_intersections),
                      float(cell_skip_threshold), out.data_ptr(), order, cost, None,
                      native._walk_ptr(_drop_in_walk(
                          (points_in, density_in, point_adjacency_in, point_adjacency_offsets_in, adjacent_diff_in),
                          (points, density, adjacency, offsets, adjacent_diff))),
                      native._quads_ptr(_drop_in_quads((diffuse_in, specular_in), (diffuse, specular))),
                      _stream(rays.device))
        else:
            _lib.call("vt_trace_infer_q8", points.data_ptr(), diffuse.data_ptr(), specular.data_ptr(), rd, rs,
                      *scales, density.data_ptr(), adjacency.data_ptr(), offsets.data_ptr(), num_points,
                      adjacent_diff.data_ptr(), rays.data_ptr(), num_rays, start_point.data_ptr(), _ptr(perm),
                      float(weight_threshold), int(max_intersections), float(cell_skip_threshold), out.data_ptr(),
                      None, _stream(rays.device))
    return out


def _check_train_common(points, diffuse, specular, density, rays, start_point, num_points, num_rays):
    """tracing_octmap.cu:386-398 (fwd) / :903-915 (bwd)."""
    _assert(diffuse.dtype == specular.dtype, "diffuse and specular must have the same dtype")
    _assert(diffuse.size(0) == specular.size(0) and diffuse.size(0) == density.size(0)
            and diffuse.size(0) == num_points, "diffuse, specular, density must each have num_points rows")
    _assert(density.dtype == torch.float32, "density must have float32 dtype")
    _assert(rays.size(-1) == 6, "rays must have 6 as the last dimension")
    _assert(rays.dtype == torch.float32, "rays must have float32 dtype")
    _assert(_is_gpu(rays), "rays must be on CUDA device")
    _assert(start_point.numel() == num_rays, "start_point must have the same batch size as rays")
    _assert(start_point.dtype == torch.uint32, "start_point must have uint32 dtype")
    _assert(_is_gpu(start_point), "start_point must be on CUDA device")


def _image_dims(rays):
    """(H, W) of the images in the rays' leading shape (native.screen_layout)
    for the tiled lane order of the training kernels; (0, 0) for a flat
    batch."""
    lay = native.screen_layout(rays.shape[:-1])
    return (0, 0) if lay is None else (lay[1], lay[2])


# Flat training batches of at least this many rays are traced in the
# ray_order lane order by default; below it the sort's fixed cost (about
# 0.2 ms) outweighs what coherent waves save.
ORDER_MIN_RAYS = 1 << 16


def ray_order(rays_in, start_point_in, num_points: int) -> torch.Tensor:
    """(An extension.)  u32 (num_rays) lane order for a flat training batch:
    the rays sorted by start cell, then by a Morton code of the direction
    (vt_ray_order), so that each wave traces neighbouring rays of one camera.
    The reference traces rays in batch order (tracing_octmap.cu:175-179) and
    its default trainer batches random pixels of random images
    (datasets.py:185-222); pass the result as ``ray_perm``."""
    rays = rays_in.contiguous()
    start_point = start_point_in.contiguous()
    num_rays = rays.numel() // 6
    _assert(rays.size(-1) == 6 and rays.dtype == torch.float32 and _is_gpu(rays),
            "rays must be a float32 (..., 6) CUDA tensor")
    _assert(start_point.dtype == torch.uint32 and start_point.numel() == num_rays and _is_gpu(start_point),
            "start_point must be a uint32 CUDA tensor with one entry per ray")
    perm = torch.empty(num_rays, dtype=torch.uint32, device=rays.device)
    if num_rays == 0:
        return perm
    ws = torch.empty(int(_lib.load().vt_ray_order_workspace_size(num_rays)), dtype=torch.uint8, device=rays.device)
    with torch.cuda.device(rays.device):
        _lib.call("vt_ray_order", rays.data_ptr(), start_point.data_ptr(), num_rays, int(num_points), perm.data_ptr(),
                  ws.data_ptr(), _stream(rays.device))
    _remember_perm(perm, num_rays, True)  # a sort's output order: a permutation by construction
    return perm


def default_ray_perm(rays, start_point, num_points: int) -> Optional[torch.Tensor]:
    """The lane order ``ray_perm="auto"`` picks: ray_order for a flat batch of
    at least ORDER_MIN_RAYS rays, else None (image-shaped rays are traced in
    8x8 screen tiles, small flat batches in batch order)."""
    num_rays = rays.numel() // 6
    if num_rays < ORDER_MIN_RAYS or _image_dims(rays) != (0, 0):
        return None
    if not (rays.size(-1) == 6 and rays.dtype == torch.float32 and _is_gpu(rays)
            and start_point.dtype == torch.uint32 and start_point.numel() == num_rays and _is_gpu(start_point)):
        return None  # the entry's own checks report these with the reference's messages
    return ray_order(rays, start_point, num_points)


def _lane_order(rays, start_point, num_points: int, ray_perm):
    """(image_h, image_w, perm tensor or None) for the training entries."""
    num_rays = rays.numel() // 6
    if isinstance(ray_perm, torch.Tensor):
        _assert(ray_perm.dtype in (torch.int32, torch.uint32) and ray_perm.numel() == num_rays
                and ray_perm.device == rays.device,
                "ray_perm must be a uint32 or int32 tensor with one entry per ray, on the rays' device")
        _assert(is_permutation(ray_perm, num_rays), "ray_perm must be a permutation of the ray indices")
        return 0, 0, _u32_view(ray_perm.contiguous())
    if ray_perm is None:
        h, w = _image_dims(rays)
        return h, w, None
    _assert(isinstance(ray_perm, str) and ray_perm == "auto", "ray_perm must be 'auto', None or a tensor")
    perm = default_ray_perm(rays, start_point, num_points)
    if perm is not None:
        return 0, 0, perm
    h, w = _image_dims(rays)
    return h, w, None


def _attr_code(dtype):
    if dtype == torch.float32:
        return 0
    if dtype == torch.float16:
        return 1
    raise RuntimeError("Unsupported color dtype. Only float32 and float16 are supported.")


def trace_vorotracing_fwd(points_in, diffuse_in, specular_in, density_in, point_adjacency_in,
                          point_adjacency_offsets_in, rays_in, start_point_in, depth_quantiles_in,
                          weight_threshold: float, max_intersections: int, return_contribution: bool,
                          stats: Optional[torch.Tensor] = None, ray_perm: Union[str, torch.Tensor, None] = "auto",
                          adj_diff_out: Optional[torch.Tensor] = None):
    """tracing_octmap.cu:346-546.  Returns (rgba, depth, depth_idx,
    contribution, n, distortion, W_total, S_total, t_far); absent outputs are
    None.  Extensions: ``stats``, None or a u32 (num_rays,
    native.STATS_WORDS) tensor that receives the per-ray walk statistics
    (vt_ray_stats); ``ray_perm``, the lane order: "auto" (default_ray_perm),
    None (screen tiles for image-shaped rays, else batch order) or a
    permutation of the rays (ray_order).  Outputs stay indexed by ray; the
    lane order changes only the order of atomic additions.  ``adj_diff_out``:
    an f16 (adjacency_size + 32, 4) device tensor the call's face-offset
    prefetch goes to (else a temporary), for the backward of the same scene
    to reuse (trace_vorotracing_bwd's ``adj_diff``)."""
    points = points_in.contiguous()
    diffuse = diffuse_in.contiguous()
    specular = specular_in.contiguous()
    density = density_in.contiguous()
    adjacency = point_adjacency_in.contiguous()
    offsets = point_adjacency_offsets_in.contiguous()
    rays = rays_in.contiguous()
    start_point = start_point_in.contiguous()
    validate_scene_data(points_in, diffuse_in, point_adjacency_in, point_adjacency_offsets_in)
    return_depth = depth_quantiles_in is not None
    num_points = points.size(0)
    adjacency_size = adjacency.size(0)
    num_rays = rays.numel() // 6
    K = 0
    _check_train_common(points, diffuse, specular, density, rays, start_point, num_points, num_rays)
    depth_quantiles = None
    if return_depth:
        depth_quantiles = depth_quantiles_in.contiguous()
        K = depth_quantiles.size(-1)
        _assert(depth_quantiles.dtype == torch.float32, "depth_quantiles must have float32 dtype")
        _assert(_is_gpu(depth_quantiles), "depth_quantiles must be on CUDA device")
        _assert(K > 0 and depth_quantiles.numel() // K == num_rays,
                "depth_quantiles must have the same batch size as rays")
    code = _attr_code(diffuse.dtype)
    rd = _map_res(diffuse.shape[-1], 3, "diffuse")
    rs = _map_res(specular.shape[-1], 3, "specular")
    dev = rays.device
    rgba = torch.empty(_out_shape(rays, 4), dtype=diffuse.dtype, device=dev)
    n = torch.empty(_out_shape(rays, 1), dtype=torch.uint32, device=dev)
    contribution = torch.zeros((num_points, 1), dtype=diffuse.dtype, device=dev) if return_contribution else None
    depth = depth_idx = None
    if return_depth:
        depth = torch.zeros(_out_shape(rays, K), dtype=torch.float32, device=dev)
        depth_idx = torch.zeros(_out_shape(rays, K), dtype=torch.uint32, device=dev)
    f1 = _out_shape(rays, 1)
    distortion = torch.empty(f1, dtype=torch.float32, device=dev)
    W_total = torch.empty(f1, dtype=torch.float32, device=dev)
    S_total = torch.empty(f1, dtype=torch.float32, device=dev)
    t_far = torch.empty(f1, dtype=torch.float32, device=dev)
    workspace = _adj_diff_buffer(adj_diff_out, adjacency_size, dev, "adj_diff_out")
    img_h, img_w, perm = _lane_order(rays, start_point, num_points, ray_perm)
    with torch.cuda.device(dev):
        sch, frame = _train_schedule(rays_in, img_h, img_w, num_rays, perm, ray_perm, dev)
        order, cost = (sch.launch_args(_stream(dev), frame, split_waves=_split_waves("fwd"))
                       if sch is not None else (None, None))
        _lib.call("vt_trace_fwd", code, points.data_ptr(), diffuse.data_ptr(), specular.data_ptr(), rd, rs,
                  density.data_ptr(), adjacency.data_ptr(), adjacency_size, offsets.data_ptr(), num_points,
                  rays.data_ptr(), num_rays, img_h, img_w, start_point.data_ptr(), _ptr(perm), K, _ptr(depth_quantiles),
                  float(weight_threshold), int(max_intersections), rgba.data_ptr(), _ptr(depth), _ptr(depth_idx),
                  _ptr(contribution), n.data_ptr(), distortion.data_ptr(), W_total.data_ptr(), S_total.data_ptr(),
                  t_far.data_ptr(), workspace.data_ptr(), order, cost, _stats_ptr(stats, num_rays), _stream(dev))
    return rgba, depth, depth_idx, contribution, n, distortion, W_total, S_total, t_far


def _adj_diff_buffer(given: Optional[torch.Tensor], adjacency_size: int, dev, what: str) -> torch.Tensor:
    """The f16 (adjacency_size + 32, 4) face-offset buffer of a training entry:
    ``given`` (checked), else a new one."""
    if given is None:
        return torch.empty((adjacency_size + 32, 4), dtype=torch.float16, device=dev)
    _assert(given.dtype == torch.float16 and tuple(given.shape) == (adjacency_size + 32, 4) and given.is_contiguous()
            and given.device == dev, f"{what} must be a contiguous float16 (adjacency_size + 32, 4) tensor on the "
                                     "rays' device")
    return given


def _stats_ptr(stats: Optional[torch.Tensor], num_rays: int):
    if stats is None:
        return None
    rec = 4 * native.STATS_WORDS  # sizeof(vt_ray_stats)
    _assert(stats.is_contiguous() and stats.numel() * stats.element_size() == rec * num_rays and _is_gpu(stats),
            f"stats must be a contiguous device tensor of num_rays {rec}-byte records")
    return stats.data_ptr()


def trace_vorotracing_bwd(points_in, diffuse_in, specular_in, density_in, point_adjacency_in,
                          point_adjacency_offsets_in, rays_in, start_point_in, rgb_out, rgb_grad_in,
                          depth_quantiles_in, depth_indices_in, depth_grad_in, ray_error_in,
                          contribution_alpha_grad: float, distortion_in, distortion_grad_in, W_total_in, S_total_in,
                          t_far_in, weight_threshold: float, max_intersections: int,
                          stats: Optional[torch.Tensor] = None, ray_perm: Union[str, torch.Tensor, None] = "auto",
                          adj_diff: Optional[torch.Tensor] = None):
    """tracing_octmap.cu:860-1103.  Returns (points_grad, diffuse_grad,
    specular_grad, density_grad, ray_grad, point_error).  ray_grad is zeros
    (the reference returns it uninitialised and the autograd wrapper drops
    it).  ``stats`` and ``ray_perm`` as for trace_vorotracing_fwd (extensions).
    ``adj_diff`` (an extension): the forward's ``adj_diff_out`` for the same
    points and adjacency, unchanged since; the call then skips its own
    prefetch (the reference prefetches on every call)."""
    points = points_in.contiguous()
    diffuse = diffuse_in.contiguous()
    specular = specular_in.contiguous()
    density = density_in.contiguous()
    adjacency = point_adjacency_in.contiguous()
    offsets = point_adjacency_offsets_in.contiguous()
    rays = rays_in.contiguous()
    start_point = start_point_in.contiguous()
    validate_scene_data(points_in, diffuse_in, point_adjacency_in, point_adjacency_offsets_in)
    return_depth = depth_quantiles_in is not None
    return_error = ray_error_in is not None
    num_points = points.size(0)
    adjacency_size = adjacency.size(0)
    num_rays = rays.numel() // 6
    K = 0
    _check_train_common(points, diffuse, specular, density, rays, start_point, num_points, num_rays)
    rgb_grad = rgb_grad_in.contiguous()
    _assert(rgb_grad.size(-1) == 4, "rgb_grad_in must have 4 as the last dimension")
    _assert(rgb_grad.dtype == diffuse.dtype, "rgb_grad_in must have the same dtype as diffuse/specular")
    _assert(_is_gpu(rgb_grad), "rgb_grad_in must be on CUDA device")
    _assert(rgb_grad.numel() // 4 == num_rays, "rgb_grad_in must have the same batch size as rays")
    rgb_out = rgb_out.contiguous()
    _assert(rgb_out.dtype == diffuse.dtype and rgb_out.numel() == 4 * num_rays,
            "rgb_out must be the forward rgba (same dtype as diffuse, 4 per ray)")
    depth_quantiles = depth_indices = depth_grad = None
    if return_depth:
        depth_quantiles = depth_quantiles_in.contiguous()
        K = depth_quantiles.size(-1)
        _assert(depth_quantiles.dtype == torch.float32, "depth_quantiles must have float32 dtype")
        _assert(_is_gpu(depth_quantiles), "depth_quantiles must be on CUDA device")
        _assert(depth_quantiles.numel() == num_rays * K, "depth_quantiles must have the same batch size as rays")
        _assert(depth_grad_in is not None, "depth_grad must be provided if depth_quantiles is provided")
        _assert(depth_indices_in is not None, "depth_indices must be provided if depth_quantiles is provided")
        depth_indices = depth_indices_in.contiguous()
        _assert(depth_indices.dtype == torch.uint32, "depth_indices must have uint32 dtype")
        _assert(_is_gpu(depth_indices), "depth_indices must be on CUDA device")
        _assert(depth_indices.numel() == num_rays * K, "depth_indices must have the same batch size as rays")
        depth_grad = depth_grad_in.contiguous()
        _assert(depth_grad.size(-1) == K,
                "depth_grad must have the same number of depth quantiles as depth_quantiles")
        _assert(depth_grad.dtype == torch.float32, "depth_grad must have float32 dtype")
        _assert(_is_gpu(depth_grad), "depth_grad must be on CUDA device")
        _assert(depth_grad.numel() == num_rays * K, "depth_grad must have the same batch size as rays")
    ray_error = point_error = None
    dev = rays.device
    if return_error:
        ray_error = ray_error_in.contiguous()
        _assert(ray_error.dtype == diffuse.dtype, "ray_error must have the same dtype as diffuse/specular")
        _assert(_is_gpu(ray_error), "ray_error must be on CUDA device")
        _assert(ray_error.numel() == num_rays, "ray_error must have the same batch size as rays")
        point_error = torch.zeros((num_points, 1), dtype=diffuse.dtype, device=dev)
    W_total = W_total_in.contiguous()
    S_total = S_total_in.contiguous()
    t_far = t_far_in.contiguous()
    distortion = distortion_in.contiguous()
    _assert(W_total.dtype == torch.float32, "W_total must have float32 dtype")
    _assert(S_total.dtype == torch.float32, "S_total must have float32 dtype")
    _assert(t_far.dtype == torch.float32, "t_far must have float32 dtype")
    _assert(distortion.dtype == torch.float32, "distortion must have float32 dtype")
    _assert(W_total.numel() == num_rays, "W_total must have the same batch size as rays")
    _assert(S_total.numel() == num_rays, "S_total must have the same batch size as rays")
    _assert(t_far.numel() == num_rays, "t_far must have the same batch size as rays")
    _assert(distortion.numel() == num_rays, "distortion must have the same batch size as rays")
    distortion_grad = None
    if distortion_grad_in is not None:
        distortion_grad = distortion_grad_in.contiguous()
        _assert(distortion_grad.dtype == torch.float32, "distortion_grad must have float32 dtype")
        _assert(distortion_grad.numel() == num_rays, "distortion_grad must have the same batch size as rays")
    code = _attr_code(diffuse.dtype)
    rd = _map_res(diffuse.shape[-1], 3, "diffuse")
    rs = _map_res(specular.shape[-1], 3, "specular")
    diffuse_grad = torch.zeros_like(diffuse)
    specular_grad = torch.zeros_like(specular)
    density_grad = torch.zeros_like(density, dtype=torch.float32)
    points_grad = torch.zeros((num_points, 3), dtype=rays.dtype, device=dev)
    ray_grad = torch.zeros_like(rays)
    workspace = _adj_diff_buffer(adj_diff, adjacency_size, dev, "adj_diff")
    cell_workspace = torch.empty((num_points, 4), dtype=torch.float32, device=dev)
    img_h, img_w, perm = _lane_order(rays, start_point, num_points, ray_perm)
    with torch.cuda.device(dev):
        sch, frame = _train_schedule(rays_in, img_h, img_w, num_rays, perm, ray_perm, dev)
        order = sch.order_for(_stream(dev), frame) if sch is not None else None
        _lib.call("vt_trace_bwd", code, points.data_ptr(), diffuse.data_ptr(), specular.data_ptr(), rd, rs,
                  density.data_ptr(), adjacency.data_ptr(), adjacency_size, offsets.data_ptr(), num_points,
                  rays.data_ptr(), num_rays, img_h, img_w, start_point.data_ptr(), _ptr(perm), rgb_out.data_ptr(),
                  rgb_grad.data_ptr(), K,
                  _ptr(depth_quantiles), _ptr(depth_indices), _ptr(depth_grad), _ptr(ray_error),
                  float(contribution_alpha_grad), distortion.data_ptr(), _ptr(distortion_grad),
                  W_total.data_ptr(), S_total.data_ptr(), t_far.data_ptr(), float(weight_threshold),
                  int(max_intersections), points_grad.data_ptr(), diffuse_grad.data_ptr(),
                  specular_grad.data_ptr(), density_grad.data_ptr(), _ptr(point_error), workspace.data_ptr(),
                  int(adj_diff is not None), cell_workspace.data_ptr(), order, _stats_ptr(stats, num_rays),
                  _stream(dev))
    return points_grad, diffuse_grad, specular_grad, density_grad, ray_grad, point_error


class NNBVH:
    """nn_bvh.h:4-16 / nn_bvh.cu:43-117: exact nearest-site queries over a
    Morton LBVH built on the GPU (replaces cuBQL).  query returns int32."""

    def __init__(self):
        import ctypes as C

        self._h = C.c_void_p()
        _lib.call("vt_bvh_create", C.byref(self._h))
        self._built = False
        self._n = 0

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            try:
                _lib.load().vt_bvh_destroy(h)
            except Exception:
                pass
            self._h = None

    def build(self, points):
        _assert(points.device.type == "cuda", "points must be on CUDA")
        pts = points.detach().contiguous()
        _assert(pts.dtype == torch.float32 and pts.dim() == 2 and pts.size(1) == 3, "points must be float32 (N, 3)")
        with torch.cuda.device(pts.device):
            _lib.call("vt_bvh_build", self._h, pts.data_ptr(), pts.size(0), _stream(pts.device))
        self._built = True
        self._n = pts.size(0)

    def query(self, points, queries):
        _assert(self._built, "BVH must be built before querying")
        _assert(queries.device.type == "cuda", "queries must be on CUDA")
        pts = points.detach().contiguous()
        q = queries.detach().contiguous()
        _assert(q.dtype == torch.float32, "queries must be float32")
        _assert(pts.size(0) == self._n, "points must be the point set the BVH was built on")
        nq = q.numel() // 3
        out = torch.empty((nq,), dtype=torch.int32, device=q.device)
        if nq == 0:
            return out
        # The scan path's partials come from torch's stream-ordered allocator,
        # not from the handle, so renders on several streams may query at once.
        ws = None
        if nq <= _lib.NN_SCAN_MAX_QUERIES and nq * self._n <= _lib.NN_SCAN_PAIRS:
            ws = torch.empty(_lib.load().vt_nearest_scan_workspace_size(nq), dtype=torch.uint8, device=q.device)
        with torch.cuda.device(q.device):
            _lib.call("vt_bvh_query_ws", self._h, pts.data_ptr(), pts.size(0), q.data_ptr(), nq, out.data_ptr(),
                      None if ws is None else ws.data_ptr(), 0 if ws is None else ws.numel(), _stream(q.device))
        return out


    def start_cells(self, points, rays):
        """u32 nearest site of every ray's origin (rays (..., 6) f32), one
        tree query per run of equal consecutive origins, counted on the GPU
        (vt_start_cells: no wait for the device)."""
        _assert(self._built, "BVH must be built before querying")
        _assert(rays.device.type == "cuda" and rays.dtype == torch.float32 and rays.shape[-1] == 6,
                "rays must be (..., 6) float32 on CUDA")
        pts = points.detach().contiguous()
        _assert(pts.size(0) == self._n, "points must be the point set the BVH was built on")
        r = rays.detach().contiguous()
        n = r.numel() // 6
        out = torch.empty(r.shape[:-1], dtype=torch.uint32, device=r.device)
        if n == 0:
            return out
        ws = torch.empty(int(_lib.load().vt_start_cells_workspace_size(n)), dtype=torch.uint8, device=r.device)
        with torch.cuda.device(r.device):
            _lib.call("vt_start_cells", self._h, pts.data_ptr(), pts.size(0), r.data_ptr(), n, out.data_ptr(),
                      ws.data_ptr(), _stream(r.device))
        return out


def nearest_neighbor_bvh(points, queries):
    """nn_bvh.cu:111-117: one-off build + query."""
    bvh = NNBVH()
    bvh.build(points)
    return bvh.query(points, queries)
