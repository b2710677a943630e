"""Training-side caller of the traversal: a Voronoi radiance field whose
forward renders rays through ``ops.TraceVoroTracing``.  It plays the role of
the reference's ``VoroTracing`` module (vorotracing.py:27-436) for the hot
path; trainer, viewer and dataset code are out of scope.

State:
- parameters ``primal_points`` (N, 3) sites, ``density`` (N, 1) raw
  log-density (the kernels take s = a * exp(raw), vorotracing.py:346-347),
  ``att_diffuse`` (N, 3 R^2) and ``att_specular`` (N, 3 Rs^2) octahedral
  logit maps.  These names are what optimiser groups and checkpoints of the
  reference refer to, so they are kept;
- the Voronoi adjacency as a u32 CSR: ``point_adjacency`` (with 32 zero
  padding entries) and ``point_adjacency_offsets`` (N + 1);
- an LBVH over the sites (``bvh``) for start cells.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn as nn

from . import ops


@dataclass
class VoroTracingConfig:
    """The reference's model configuration (vorotracing.py:12-24; same field
    names, so its configs load).  Octahedral map sides 4 and 8 are compiled,
    for diffuse and specular independently."""
    oct_map_res: int = 8
    spec_oct_map_res: int = 8
    activation_scale: float = 1.0
    up_direction: List[float] = field(default_factory=lambda: [0, 0, 0])


def _float_param(value, rows: int, cols: int, device, what: str) -> nn.Parameter:
    """A float32 (rows, cols) parameter holding ``value``, or zeros without one
    (zero logits: grey diffuse, no specular; zero raw density: s = a)."""
    if value is None:
        return nn.Parameter(torch.zeros(rows, cols, dtype=torch.float32, device=device))
    t = torch.as_tensor(value)
    if t.dtype != torch.float32 or tuple(t.shape) != (rows, cols):
        raise ValueError(f"{what}: expected float32 ({rows}, {cols}), got {t.dtype} {tuple(t.shape)}")
    return nn.Parameter(t.to(device).contiguous())


class VoroTracing(nn.Module):
    """Sites, densities and octahedral maps of a Voronoi scene, rendered by
    the HIP traversal.  Without an adjacency the constructor builds it on the
    GPU (``update_triangulation``)."""

    def __init__(self, config: VoroTracingConfig, points, points_diffuse=None, points_specular=None,
                 points_density=None, points_adjacency=None, points_adjacency_offsets=None,
                 device: torch.device = torch.device("cuda")):
        super().__init__()
        sites = torch.as_tensor(points)
        if sites.dim() != 2 or sites.shape[0] == 0:
            raise ValueError(f"sites: expected a non-empty (N, 3) tensor, got shape {tuple(sites.shape)}")
        n = sites.shape[0]
        self.config = config
        self.device = device
        self.primal_points = _float_param(sites, n, 3, device, "sites")
        self.density = _float_param(points_density, n, 1, device, "raw density")
        self.att_diffuse = _float_param(points_diffuse, n, 3 * config.oct_map_res ** 2, device, "diffuse map")
        self.att_specular = _float_param(points_specular, n, 3 * config.spec_oct_map_res ** 2, device, "specular map")
        self.bvh = ops.NNBVH()
        if (points_adjacency is None) != (points_adjacency_offsets is None):
            raise ValueError("the adjacency and its offsets are given together or not at all")
        if points_adjacency is None:
            self.update_triangulation()
        else:
            self.set_adjacency(points_adjacency, points_adjacency_offsets)

    # ---- construction and persistence

    @classmethod
    def from_scene(cls, s, device=torch.device("cuda")) -> "VoroTracing":
        """A model holding a synthetic scene (``vorotracing_amd.scene.Scene``)."""
        cfg = VoroTracingConfig(oct_map_res=s.diff_res, spec_oct_map_res=s.spec_res)
        return cls(cfg, torch.from_numpy(s.points.copy()), torch.from_numpy(s.diffuse.copy()),
                   torch.from_numpy(s.specular.copy()), torch.from_numpy(s.density_raw.copy()),
                   torch.from_numpy(s.adjacency.view("int32").copy()), torch.from_numpy(s.offsets.view("int32").copy()),
                   device=device)

    # checkpoint keys of the reference's files (vorotracing.py:421-436), so checkpoints move both ways
    _CKPT = {"xyz": "primal_points", "density": "density", "color_diffuse": "att_diffuse",
             "color_specular": "att_specular"}

    @classmethod
    def from_pretrained(cls, pt_path, config: VoroTracingConfig, device=torch.device("cuda")) -> "VoroTracing":
        """Load a checkpoint written by ``save_checkpoint`` or by the reference
        (tensors only: ``torch.load(weights_only=True)``)."""
        d = torch.load(pt_path, map_location="cpu", weights_only=True)
        return cls(config, d["xyz"].float(), d["color_diffuse"].float(), d["color_specular"].float(),
                   d["density"].float(), d["adjacency"], d["adjacency_offsets"], device=device)

    def save_checkpoint(self, out_path: str):
        state = {key: getattr(self, attr).detach().float().cpu() for key, attr in self._CKPT.items()}
        state["adjacency"] = self.point_adjacency.cpu().long()
        state["adjacency_offsets"] = self.point_adjacency_offsets.cpu().long()
        torch.save(state, out_path)

    # ---- geometry

    @property
    def num_sites(self) -> int:
        return int(self.primal_points.shape[0])

    def set_adjacency(self, adjacency, offsets):
        """Install a Voronoi CSR (any integer dtype; stored as u32) and build
        the start-cell LBVH over the current sites."""
        off = torch.as_tensor(offsets).reshape(-1)
        if off.numel() != self.num_sites + 1:
            raise ValueError(f"adjacency offsets: expected {self.num_sites + 1} entries, got {off.numel()}")
        self.point_adjacency = torch.as_tensor(adjacency).reshape(-1).to(self.device, dtype=torch.uint32)
        self.point_adjacency_offsets = off.to(self.device, dtype=torch.uint32)
        self.bvh.build(self.primal_points)

    @torch.no_grad()
    def update_triangulation(self, warm_start: bool = True):
        """Rebuild the adjacency after the sites moved, on the GPU Voronoi
        builder (the reference calls Paragram here, vorotracing.py:310-321),
        and the start-cell LBVH.  With ``warm_start`` the current adjacency
        (when it is over the same number of sites) seeds the build: same
        result, found faster after small moves."""
        if not bool(torch.isfinite(self.primal_points).all()):
            raise RuntimeError("update_triangulation: the sites hold NaN or inf")
        guess = {}
        offs = getattr(self, "point_adjacency_offsets", None)
        if warm_start and offs is not None and offs.numel() == self.num_sites + 1:
            guess = dict(initial_guesses=self.point_adjacency, initial_guesses_offsets=offs)
        adjacency, offsets, _ = ops.build_voronoi_adjacency(self.primal_points.detach(), **guess)
        self.set_adjacency(adjacency, offsets)

    @torch.no_grad()
    def sort_morton(self, optimizer=None) -> torch.Tensor:
        """Put the sites in the Morton order of VoroTracingInfer's cells
        (vorotracing.py:514-571, ties by index; vt_morton_reorder): the
        parameters' rows, their gradients, the rows of ``optimizer``'s
        per-parameter state (torch Adam's moments, or FusedVoroAdam's) and
        the CSR are permuted in place, and the LBVH is rebuilt.  Renders are
        the same; neighbouring cells then sit in neighbouring rows, which the
        traversal reads far better for large scenes (C5's 3.1M sites: forward
        7.3 -> 5.2 ms).  Returns the permutation: new row i is old row perm[i]
        (u32)."""
        from . import _lib

        pts = self.primal_points.data.contiguous()
        n = pts.shape[0]
        adj = self.point_adjacency.contiguous()
        off = self.point_adjacency_offsets.contiguous()
        lib = _lib.load()
        dev = pts.device
        stream = torch.cuda.current_stream(dev).cuda_stream
        ws = torch.empty(lib.vt_morton_workspace_size(n, adj.numel()), dtype=torch.uint8, device=dev)
        perm = torch.empty(n, dtype=torch.uint32, device=dev)
        pts_out, adj_out, off_out = torch.empty_like(pts), torch.empty_like(adj), torch.empty_like(off)
        with torch.cuda.device(dev):
            _lib.call("vt_morton_reorder", pts.data_ptr(), n, adj.data_ptr(), adj.numel(), off.data_ptr(),
                      perm.data_ptr(), pts_out.data_ptr(), adj_out.data_ptr(), off_out.data_ptr(), ws.data_ptr(),
                      stream)

            def rows(t):
                t = t.contiguous()
                out = torch.empty_like(t)
                _lib.call("vt_permute_rows", t.data_ptr(), n, t[0].numel() * t.element_size(), perm.data_ptr(),
                          out.data_ptr(), stream)
                return out

            states = []
            if optimizer is not None:
                st = getattr(optimizer, "state", {})
                for p in (self.primal_points, self.density, self.att_diffuse, self.att_specular):
                    for k, v in st.get(p, {}).items():
                        if torch.is_tensor(v) and v.dim() >= 1 and v.shape[0] == n:
                            states.append((st[p], k, v))
            for p in (self.density, self.att_diffuse, self.att_specular):
                p.data = rows(p.data)
                if p.grad is not None:
                    p.grad = rows(p.grad)
            if self.primal_points.grad is not None:
                self.primal_points.grad = rows(self.primal_points.grad)
            self.primal_points.data = pts_out
            for d, k, v in states:
                d[k] = rows(v)
        self.point_adjacency = adj_out
        self.point_adjacency_offsets = off_out
        self.bvh.build(self.primal_points)
        return perm

    @torch.no_grad()
    def get_starting_point(self, rays: torch.Tensor) -> torch.Tensor:
        """u32 start cell of every ray: the nearest site of its origin
        (vorotracing.py:323-344), one LBVH query per run of equal consecutive
        origins, counted on the GPU (NNBVH.start_cells: the call does not wait
        for the device).  Rays of an image share one origin, or one per row
        under a rolling shutter; any order of rays gives the same cells."""
        return self.bvh.start_cells(self.primal_points, rays)

    def start_cells(self, rays: torch.Tensor, start_point: Optional[torch.Tensor] = None) -> torch.Tensor:
        """``start_point`` broadcast over the ray batch, or the nearest sites."""
        if start_point is None:
            return self.get_starting_point(rays)
        return torch.broadcast_to(start_point, rays.shape[:-1])

    # ---- rendering

    def activated_density(self) -> torch.Tensor:
        """The density the kernels take: s = a * exp(raw)."""
        return self.config.activation_scale * torch.exp(self.density)

    def forward(self, rays: torch.Tensor, start_point: Optional[torch.Tensor] = None,
                depth_quantiles: Optional[torch.Tensor] = None, weight_threshold: float = 0.001,
                max_intersections: int = 1024, return_contribution: bool = False):
        """Render ``rays`` (..., 6): (rgba, depth, contribution, n, error box,
        distortion), the outputs of vorotracing.py:365-419; defaults as there."""
        return ops.TraceVoroTracing.apply(self.primal_points, self.att_diffuse, self.att_specular,
                                          self.activated_density(), self.point_adjacency,
                                          self.point_adjacency_offsets, rays, self.start_cells(rays, start_point),
                                          depth_quantiles, weight_threshold, max_intersections, return_contribution)
