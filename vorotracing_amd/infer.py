"""Inference-side caller of the path: ``VoroTracingInfer``
(vorotracing.py:439-683) with its preparation done by HIP kernels.

Construction: density activation, fp16 Half4Texel padding
(vt_pad_3to4_f16) or q8 quantisation (vt_quantize_u8), Morton reorder of the
cells with CSR rebuild (vt_morton_reorder + vt_permute_rows), LBVH rebuild,
and the per-face offset prefetch.  ``render`` picks start cells and launches
the traversal; full images are rendered with in-kernel 8x8 wave tiling
instead of the reference's 4x8 permutation buffer (the lane assignment never
changes per-ray results).
"""
from __future__ import annotations

from typing import Literal, Optional

import numpy as np
import torch

from . import _C, _lib, camera, native, ops


class VoroTracingInfer:
    """Lightweight inference wrapper (vorotracing.py:439-493).  ``model`` is a
    ``vorotracing_amd.model.VoroTracing`` (or any object with its attributes)."""

    TILE = (8, 8)
    # launch the tiles of a repeated image shape by the previous frame's tile
    # costs (native.TileSchedule; images are bit-identical either way)
    adaptive_tile_order = True
    # walk the packed layout (native.WalkLayout) in the tiled and camera
    # renders, each cell's faces laid out by the z of their offsets
    # (face_order 3; 0 keeps the list order); images are bit-identical either way
    packed_walk = True
    face_order = 3
    # read the maps through their footprint tables (native.QuadMaps: a
    # bilinear tap's four texels in one entry, 32 bytes for fp16 maps, 16 for
    # q8) in the tiled and camera renders; images are bit-identical either way
    quad_maps = True

    def __init__(self, model, sort_morton: bool = True, quantize: Literal["fp16", "q8"] = "fp16",
                 per_channel_q8: bool = False):
        self._setup(model.primal_points.detach().contiguous(),
                    (model.config.activation_scale * torch.exp(model.density)).detach().contiguous(),
                    model.point_adjacency.clone(), model.point_adjacency_offsets, model.bvh,
                    model.att_diffuse.detach(), model.att_specular.detach(), model.config.oct_map_res,
                    model.config.spec_oct_map_res, quantize, per_channel_q8, sort_morton)

    def _setup(self, points, density, adjacency, offsets, bvh, diffuse, specular, diff_res, spec_res, quantize,
               per_channel_q8, sort_morton):
        self.primal_points = points
        self.density = density
        self.point_adjacency = adjacency
        self.point_adjacency_offsets = offsets
        self.bvh = bvh
        self.device = self.primal_points.device
        self.quantize = quantize
        self.diff_res = diff_res
        self.spec_res = spec_res
        self.diffuse_q8 = self.specular_q8 = None
        self.diffuse_fp16 = self.specular_fp16 = None
        if quantize == "q8":
            self.diffuse_q8, self.diff_scale, self.diff_offset = self._quantize_to_uint8(diffuse, per_channel_q8)
            self.specular_q8, self.spec_scale, self.spec_offset = self._quantize_to_uint8(specular, per_channel_q8)
        elif quantize == "fp16":
            self.diffuse_fp16 = self._pad_3to4(diffuse, self.diff_res)
            self.specular_fp16 = self._pad_3to4(specular, self.spec_res)
        else:
            raise ValueError(f"Invalid quantization method: {quantize}")
        if sort_morton:
            self._reorder_by_morton()
        if self.bvh is None:
            self.bvh = ops.NNBVH()
            self.bvh.build(self.primal_points)
        self.adjacent_diff = ops.prefetch_octmap_adj(self.primal_points, self.point_adjacency,
                                                     self.point_adjacency_offsets)
        self._walk_layout = None
        self._quad_maps = None

    def quad_tables(self) -> Optional[native.QuadMaps]:
        """The footprint tables of the maps (fp16 or q8; built on first use,
        and again when the maps have been replaced or changed in place), or
        None when ``quad_maps`` is off or the tables would take more than a
        quarter of the device's free memory (the renders then read the maps)."""
        if not self.quad_maps:
            return None
        src = (self.diffuse_q8, self.specular_q8) if self.quantize == "q8" else (self.diffuse_fp16,
                                                                                  self.specular_fp16)
        entry = self.__dict__.get("_quad_maps")
        if entry is None or not entry[0].matches(*src):
            # None when the tables would take too much of the free memory (QuadMaps.MAX_FREE_SHARE)
            entry = (native.SourceKey(*src), native.QuadMaps.build_within(*src))
            self._quad_maps = entry
        return entry[1]

    def walk_layout(self) -> Optional[native.WalkLayout]:
        """The scene's packed walk layout (built on first use, and again when
        the sites, density, adjacency or face records have been replaced or
        changed in place), or None when ``packed_walk`` is off or the scene
        exceeds the layout's limits."""
        if not self.packed_walk:
            return None
        src = (self.primal_points, self.density, self.point_adjacency, self.point_adjacency_offsets,
               self.adjacent_diff)
        entry = self._walk_layout
        if entry is None or not entry[0].matches(*src) or entry[2] != self.face_order:
            entry = (native.SourceKey(*src), native.WalkLayout.build(*src, face_order=self.face_order),
                     self.face_order)
            self._walk_layout = entry
        return entry[1]

    @classmethod
    def from_foam(cls, path, device=torch.device("cuda"), quantize: Literal["fp16", "q8"] = "fp16",
                  per_channel_q8: bool = False, sort_morton: bool = False):
        """A scene from a ``.foam`` file (V3 or V4; vorotracing_amd.foam, the reference's
        scripts/export_for_viewer.py format).  Cells are used in file order (the exporter writes a
        Morton-sorted VoroTracingInfer); the file's density is already activated; adjacent_diff is
        recomputed by the prefetch kernel.  A file without specular maps renders with zero specular
        logits.  The file's header (thresholds, poses) is kept as ``self.foam``."""
        import numpy as np

        from . import foam

        sc = foam.read_foam(path)
        dev = torch.device(device)
        n = sc.points.shape[0]

        def t(a, dtype=None):
            x = torch.from_numpy(np.ascontiguousarray(a))
            return (x if dtype is None else x.to(dtype)).to(dev)

        rs = sc.res_spec if sc.specular is not None else sc.res_diff
        spec = sc.specular if sc.specular is not None else np.zeros((n, 3 * rs * rs), np.float16)
        self = cls.__new__(cls)
        self._setup(t(sc.points), t(sc.density).reshape(-1, 1), t(sc.adjacency), t(sc.offsets), None,
                    t(sc.diffuse, torch.float32), t(spec, torch.float32), sc.res_diff, rs, quantize, per_channel_q8,
                    sort_morton)
        self.foam = sc
        return self

    # -- preparation (HIP) ----------------------------------------------------

    def _stream(self):
        return torch.cuda.current_stream(self.device).cuda_stream

    def _schedule(self, images: int, H: int, W: int) -> Optional[native.TileSchedule]:
        """The tile launch schedule of this image shape on the current stream."""
        if not self.adaptive_tile_order:
            return None
        cache = self.__dict__.setdefault("_schedules", {})
        return native.schedule_for(cache, (int(images), int(H), int(W), self._stream()),
                                   native.num_tiles(images, H, W, *self.TILE), self.device)

    def _quantize_to_uint8(self, tensor, per_channel=False):
        """vorotracing.py:495-503 -> (q u8, scale, offset); per-channel returns 3-lists."""
        x = tensor.float().contiguous()
        q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
        params = torch.empty(9, dtype=torch.float32, device=x.device)
        ws = torch.empty(_lib.load().vt_quantize_workspace_size(), dtype=torch.uint8, device=x.device)
        rows, cols = x.shape[0], x.numel() // max(x.shape[0], 1)
        with torch.cuda.device(x.device):
            _lib.call("vt_quantize_u8", x.data_ptr(), rows, cols, 1 if per_channel else 0, q.data_ptr(),
                      params.data_ptr(), ws.data_ptr(), self._stream())
        p = params.cpu().tolist()
        if per_channel:
            return q, p[0:3], p[3:6]
        return q, p[0], p[3]

    def _pad_3to4(self, tensor, R):
        """vorotracing.py:505-512 on the .half() map (vorotracing.py:477-482)."""
        x = tensor.float().contiguous()
        n = x.shape[0]
        out = torch.empty((n, 4 * R * R), dtype=torch.float16, device=x.device)
        with torch.cuda.device(x.device):
            _lib.call("vt_pad_3to4_f16", x.data_ptr(), n, R * R, out.data_ptr(), self._stream())
        return out

    def _permute(self, t: torch.Tensor, perm: torch.Tensor) -> torch.Tensor:
        t = t.contiguous()
        out = torch.empty_like(t)
        row_bytes = t[0].numel() * t.element_size() if t.shape[0] else 0
        _lib.call("vt_permute_rows", t.data_ptr(), t.shape[0], row_bytes, perm.data_ptr(), out.data_ptr(),
                  self._stream())
        return out

    def _reorder_by_morton(self):
        """vorotracing.py:514-571 on the GPU; ties in the key keep their index order."""
        pts = self.primal_points
        n = pts.shape[0]
        adj = self.point_adjacency.contiguous()
        off = self.point_adjacency_offsets.contiguous()
        lib = _lib.load()
        ws = torch.empty(lib.vt_morton_workspace_size(n, adj.numel()), dtype=torch.uint8, device=self.device)
        perm = torch.empty(n, dtype=torch.uint32, device=self.device)
        pts_out = torch.empty_like(pts)
        adj_out = torch.empty_like(adj)
        off_out = torch.empty_like(off)
        with torch.cuda.device(self.device):
            _lib.call("vt_morton_reorder", pts.data_ptr(), n, adj.data_ptr(), adj.numel(), off.data_ptr(),
                      perm.data_ptr(), pts_out.data_ptr(), adj_out.data_ptr(), off_out.data_ptr(), ws.data_ptr(),
                      self._stream())
            self.density = self._permute(self.density, perm)
            if self.quantize == "q8":
                self.diffuse_q8 = self._permute(self.diffuse_q8, perm)
                self.specular_q8 = self._permute(self.specular_q8, perm)
            else:
                self.diffuse_fp16 = self._permute(self.diffuse_fp16, perm)
                self.specular_fp16 = self._permute(self.specular_fp16, perm)
        self.morton_perm = perm
        self.primal_points = pts_out
        self.point_adjacency = adj_out
        self.point_adjacency_offsets = off_out
        # The reference rebuilds the model's shared BVH here (vorotracing.py:459,
        # :571), which leaves the model's own start-cell queries running on a tree
        # of the reordered sites; the reordered scene gets its own LBVH instead.
        self.bvh = ops.NNBVH()
        self.bvh.build(self.primal_points)

    @classmethod
    def from_pretrained(cls, pt_path, config, device=torch.device("cuda"), quantize="fp16",
                        sort_morton: bool = True):
        from .model import VoroTracing

        return cls(VoroTracing.from_pretrained(pt_path, config, device=device), quantize=quantize,
                   sort_morton=sort_morton)

    # -- per frame ------------------------------------------------------------

    @torch.no_grad()
    def get_starting_point(self, rays):
        """u32 start cells of a render, one LBVH query per camera: the origin
        of a camera's first ray is every ray's origin for a pinhole image (the
        reference queries the batch's first ray only, vorotracing.py:585-604).
        An image batch (B, H, W, 6) is B cameras, any other shape one."""
        return self.start_cells(rays).expand(rays.shape[:-1]).contiguous()

    def start_cells(self, rays):
        """get_starting_point's cells, one per camera, shaped to broadcast
        over the rays' leading dimensions ((B, 1, 1) or all ones): the form
        ``render`` passes to the tiled kernels without expanding it."""
        lead = rays.shape[:-1]
        cams = lead[0] if rays.dim() == 4 else 1
        first = rays.reshape(cams, -1, 6)[:, 0, :3].contiguous()
        cells = self.bvh.query(self.primal_points, first).view(torch.uint32)
        return cells.reshape((cams,) + (1,) * (len(lead) - 1) if rays.dim() == 4 else (1,) * len(lead))

    @staticmethod
    def _rays_per_start(rays, start_point) -> int:
        """For the tiled kernels: the rays that share one entry of a
        broadcastable ``start_point`` when it holds one cell for all rays or
        one per image of the batch (ray r then starts at r // this); 0 when it
        must be expanded to one cell per ray."""
        lead = tuple(rays.shape[:-1])
        shape = (1,) * (len(lead) - start_point.dim()) + tuple(start_point.shape)
        if len(shape) != len(lead):
            return 0
        B, H, W = native.image_dims(rays)
        if all(x == 1 for x in shape):
            return B * H * W
        if len(lead) == 3 and shape == (lead[0], 1, 1) and B == lead[0]:
            return H * W
        return 0

    def _render_start(self, rays, start_point, image: bool):
        """(start cells, rays per start cell) of a render: for the tiled
        kernels a per-camera (or single) cell array as is, with the rays that
        share each cell; otherwise one cell per ray and 0."""
        if start_point is None:
            start_point = self.start_cells(rays)
        else:
            start_point = torch.as_tensor(start_point, device=rays.device)
        k = self._rays_per_start(rays, start_point) if image else 0
        if k:
            return start_point.reshape(-1).contiguous(), k
        return torch.broadcast_to(start_point, rays.shape[:-1]).contiguous(), 0

    def render_frames(self, frames, in_flight: int = 2, **render_kw):
        """``render`` of a sequence of frames (each a rays tensor as ``render``
        takes, with ``render``'s keyword arguments) with up to ``in_flight``
        frames on the GPU at once: frame k renders on side stream k mod
        in_flight, so the end of one frame, when few waves are left, overlaps
        the start of the next.  Every frame is a whole render (its own
        start-cell query and traversal); outputs come back in order.  On
        return the caller's stream is ordered after every frame, as after
        ``render``.  Side streams keep the default priority.  Frames overlap
        only if their streams get hardware queues of their own: HIP maps
        streams onto GPU_MAX_HW_QUEUES queues (4 by default), so with three
        in flight plus the default stream an earlier stream of the process
        makes two frames share a queue (1.73 instead of 1.62 ms per frame at
        C3); two in flight leave room."""
        cur = torch.cuda.current_stream(self.device)
        streams = self._side_streams(in_flight)
        for s in streams:
            s.wait_stream(cur)
        outs = []
        for k, rays in enumerate(frames):
            with torch.cuda.stream(streams[k % len(streams)]):
                out = self.render(rays, **render_kw)
            out.record_stream(cur)  # allocated on the side stream, used on the caller's
            outs.append(out)
        for s in streams:
            cur.wait_stream(s)
        return outs

    def _side_streams(self, n: int):
        if n < 1:
            raise ValueError("in_flight must be at least 1")
        cache = getattr(self, "_streams", None)
        if cache is None or len(cache) < n:
            cache = self._streams = [torch.cuda.Stream(device=self.device) for _ in range(n)]
        return cache[:n]

    @torch.no_grad()
    def _tile_perm(self, H, W, TH=8, TW=8):
        """vorotracing.py:606-625 (int32, cached), from vt_tile_perm."""
        cache = getattr(self, "_tile_perm_cache", None)
        if cache is None:
            cache = self._tile_perm_cache = {}
        key = (int(H), int(W), TH, TW)
        if key not in cache:
            perm = torch.empty(H * W, dtype=torch.int32, device=self.device)
            _lib.call("vt_tile_perm", H, W, TH, TW, perm.data_ptr(), self._stream())
            cache[key] = perm
        return cache[key]

    def render(self, rays, start_point=None, weight_threshold=0.001, max_intersections=1024,
               cell_skip_threshold=0.0, use_warp_perm: bool = True, stats: Optional[torch.Tensor] = None):
        """vorotracing.py:627-683.  Returns f16 [..., 4]."""
        image = use_warp_perm and rays.shape[-1] == 6 and native.screen_layout(rays.shape[:-1]) is not None
        start_point, rays_per_start = self._render_start(rays, start_point, image)
        if self.quantize == "q8":
            if not image and stats is None:
                return ops.trace_octmap_infer_q8(
                    self.primal_points, self.diffuse_q8, self.specular_q8, self.density, self.point_adjacency,
                    self.point_adjacency_offsets, rays, start_point, self.adjacent_diff, self.diff_scale,
                    self.diff_offset, self.spec_scale, self.spec_offset, weight_threshold, max_intersections,
                    cell_skip_threshold)
            return self._render_q8_native(rays, start_point, weight_threshold, max_intersections,
                                          cell_skip_threshold, image, stats, rays_per_start)
        if not image and stats is None:
            empty = torch.empty(0, dtype=torch.int32, device=self.device)
            return ops.trace_octmap_infer(self.primal_points, self.diffuse_fp16, self.specular_fp16, self.density,
                                          self.point_adjacency, self.point_adjacency_offsets, rays, start_point,
                                          self.adjacent_diff, empty, weight_threshold, max_intersections,
                                          cell_skip_threshold)
        rays = rays.contiguous()
        _check_render_args(self, rays, start_point, self.diffuse_fp16, rays_per_start)
        return native.infer_f16(self.primal_points, self.diffuse_fp16, self.specular_fp16, self.density.reshape(-1),
                                self.point_adjacency, self.point_adjacency_offsets, self.adjacent_diff, rays,
                                start_point, weight_threshold=weight_threshold, max_intersections=max_intersections,
                                cell_skip_threshold=cell_skip_threshold, stats=stats,
                                tiled=self.TILE if image else None,
                                schedule=self._schedule(*native.image_dims(rays)) if image else None,
                                walk=self.walk_layout() if image else None, rays_per_start=rays_per_start,
                                quads=self.quad_tables() if image else None)

    def camera_start_points(self, cameras, camera_buffer=None):
        """Start cells of a camera batch: one LBVH query on each camera's centre, or
        on each row's origin for rolling shutters (vt_camera_rays with one column)."""
        cams = list(cameras)
        with torch.no_grad():
            if any(c.rolling_shutter for c in cams):
                origins = native.camera_rays(cams, self.device, width=1, camera_buffer=camera_buffer)
                origins = origins[..., :3].reshape(-1, 3).contiguous()
                return self.bvh.query(self.primal_points, origins).view(torch.uint32), True
            origins = torch.tensor(np.stack([np.asarray(c.t, np.float32) for c in cams]), device=self.device)
            return self.bvh.query(self.primal_points, origins).view(torch.uint32), False

    def render_cameras(self, cameras, weight_threshold=0.001, max_intersections=1024, cell_skip_threshold=0.0,
                       start_point=None, stats: Optional[torch.Tensor] = None, camera_buffer=None):
        """``render`` of the rays of a batch of ``camera.Camera`` (one image size), with
        the rays generated inside the traversal kernel (vt_trace_infer_*_camera): no
        rays tensor is built or read.  Returns f16 (B, H, W, 4), the image ``render``
        gives for ``native.camera_rays(cameras)``.  ``camera_buffer``: the cameras
        already on the device (``native.upload_cameras``)."""
        import ctypes as C

        cams = list(cameras)
        if camera_buffer is None:
            camera_buffer = native.upload_cameras(cams, self.device)
        B, H, W = len(cams), cams[0].height, cams[0].width
        if start_point is None:
            start_point, per_row = self.camera_start_points(cams, camera_buffer)
        else:
            per_row = start_point.numel() == B * H and any(c.rolling_shutter for c in cams)
        out = torch.empty((B, H, W, 4), dtype=torch.float16, device=self.device)
        sp = native._s(self.device)
        sch = self._schedule(B, H, W)
        frame = camera.pack_cameras(cams)  # host-side records: no device read
        order, cost = sch.launch_args(sp, frame) if sch is not None else (None, None)
        common = (float(weight_threshold), int(max_intersections), float(cell_skip_threshold), out.data_ptr(), order,
                  cost, native._p(stats), native._walk_ptr(self.walk_layout()))
        if self.quantize == "q8":
            def v3(x):
                vals = [float(x)] * 3 if isinstance(x, (int, float)) else [float(v) for v in x]
                return C.cast((C.c_float * 3)(*vals), C.c_void_p)

            keep = [v3(self.diff_scale), v3(self.diff_offset), v3(self.spec_scale), v3(self.spec_offset)]
            rd = native.map_res(self.diffuse_q8.shape[-1], 3)
            rs = native.map_res(self.specular_q8.shape[-1], 3)
            _lib.call("vt_trace_infer_q8_camera", self.primal_points.data_ptr(), self.diffuse_q8.data_ptr(),
                      self.specular_q8.data_ptr(), rd, rs, *keep, self.density.data_ptr(),
                      self.point_adjacency.data_ptr(), self.point_adjacency_offsets.data_ptr(),
                      self.primal_points.shape[0], self.adjacent_diff.data_ptr(), camera_buffer.data_ptr(), B, H, W,
                      self.TILE[0], self.TILE[1], start_point.data_ptr(), int(per_row), *common,
                      native._quads_ptr(self.quad_tables()), sp)
        else:
            rd = native.map_res(self.diffuse_fp16.shape[-1], 4)
            rs = native.map_res(self.specular_fp16.shape[-1], 4)
            _lib.call("vt_trace_infer_f16_camera", self.primal_points.data_ptr(), self.diffuse_fp16.data_ptr(),
                      self.specular_fp16.data_ptr(), rd, rs, self.density.data_ptr(),
                      self.point_adjacency.data_ptr(), self.point_adjacency_offsets.data_ptr(),
                      self.primal_points.shape[0], self.adjacent_diff.data_ptr(), camera_buffer.data_ptr(), B, H, W,
                      self.TILE[0], self.TILE[1], start_point.data_ptr(), int(per_row), *common,
                      native._quads_ptr(self.quad_tables()), sp)
        return out

    def _render_q8_native(self, rays, start_point, thr, max_int, skip, image, stats, rays_per_start=0):
        import ctypes as C

        rays = rays.contiguous()
        _check_render_args(self, rays, start_point, self.diffuse_q8, rays_per_start)

        def v3(x):
            vals = [float(x)] * 3 if isinstance(x, (int, float)) else [float(v) for v in x]
            return C.cast((C.c_float * 3)(*vals), C.c_void_p)

        keep = [v3(self.diff_scale), v3(self.diff_offset), v3(self.spec_scale), v3(self.spec_offset)]
        out = torch.empty(list(rays.shape[:-1]) + [4], dtype=torch.float16, device=rays.device)
        rd = native.map_res(self.diffuse_q8.shape[-1], 3)
        rs = native.map_res(self.specular_q8.shape[-1], 3)
        sp = native._s(rays.device)
        if image:
            B, H, W = native.image_dims(rays)
            sch = self._schedule(B, H, W)
            frame = native.frame_key(rays)
            order, cost = sch.launch_args(sp, frame) if sch is not None else (None, None)
            _lib.call("vt_trace_infer_q8_tiled", self.primal_points.data_ptr(), self.diffuse_q8.data_ptr(),
                      self.specular_q8.data_ptr(), rd, rs, *keep, self.density.data_ptr(),
                      self.point_adjacency.data_ptr(), self.point_adjacency_offsets.data_ptr(),
                      self.primal_points.shape[0], self.adjacent_diff.data_ptr(), rays.data_ptr(), B, H, W,
                      self.TILE[0], self.TILE[1], start_point.data_ptr(), int(rays_per_start), float(thr),
                      int(max_int), float(skip), out.data_ptr(), order, cost, native._p(stats),
                      native._walk_ptr(self.walk_layout()), native._quads_ptr(self.quad_tables()), sp)
        else:
            _lib.call("vt_trace_infer_q8", self.primal_points.data_ptr(), self.diffuse_q8.data_ptr(),
                      self.specular_q8.data_ptr(), rd, rs, *keep, self.density.data_ptr(),
                      self.point_adjacency.data_ptr(), self.point_adjacency_offsets.data_ptr(),
                      self.primal_points.shape[0], self.adjacent_diff.data_ptr(), rays.data_ptr(),
                      rays.numel() // 6, start_point.data_ptr(), None, float(thr), int(max_int), float(skip),
                      out.data_ptr(), native._p(stats), sp)
        return out


def _check_render_args(inf, rays, start_point, diffuse, rays_per_start=0):
    """Shape/dtype checks of the native render paths (same rules as _C).
    With rays_per_start, start_point holds one cell per that many rays."""
    _C.validate_scene_data(inf.primal_points, diffuse, inf.point_adjacency, inf.point_adjacency_offsets)
    if rays.dtype != torch.float32 or rays.shape[-1] != 6:
        raise RuntimeError("rays must have float32 dtype and 6 as the last dimension")
    want = rays.numel() // 6 // rays_per_start if rays_per_start else rays.numel() // 6
    if start_point.dtype != torch.uint32 or start_point.numel() != want:
        raise RuntimeError("start_point must have uint32 dtype and the same batch size as rays")
