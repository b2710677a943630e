"""ctypes loader for libvt_hip.so (the HIP traversal library, include/vt_abi.h).

There is no CPU fallback: if the library is missing or no GPU is visible,
every operator raises.
"""
from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libvt_hip.so")

_lib = None

P = C.c_void_p
U32 = C.c_uint32
F32 = C.c_float
I32 = C.c_int

# name -> argtypes (restype int unless noted); mirrors include/vt_abi.h
SIGNATURES = {
    "vt_last_error": ([], C.c_char_p),
    "vt_abi_version": ([], C.c_int),
    "vt_prefetch_adj": ([P, U32, P, U32, P, P, P], C.c_int),
    "vt_trace_infer_f16": ([P, P, P, U32, U32, P, P, P, U32, P, P, U32, P, P, F32, U32, F32, P, P, P], C.c_int),
    "vt_walk_layout_count_workspace_size": ([U32], C.c_size_t),
    "vt_walk_layout_count": ([P, P, U32, P, P, P], C.c_int),
    "vt_walk_layout_fill": ([P, P, P, P, U32, P, P, U32, I32, P, P, P, P, P, P], C.c_int),
    "vt_quad_maps_f16": ([P, U32, U32, P, P], C.c_int),
    "vt_quad_maps_q8": ([P, U32, U32, P, P], C.c_int),
    "vt_trace_infer_f16_tiled": (
        [P, P, P, U32, U32, P, P, P, U32, P, P, U32, U32, U32, U32, U32, P, U32, F32, U32, F32, P, P, P, P, P, P, P],
        C.c_int),
    "vt_trace_infer_q8": (
        [P, P, P, U32, U32, P, P, P, P, P, P, P, U32, P, P, U32, P, P, F32, U32, F32, P, P, P], C.c_int),
    "vt_trace_infer_q8_tiled": (
        [P, P, P, U32, U32, P, P, P, P, P, P, P, U32, P, P, U32, U32, U32, U32, U32, P, U32, F32, U32, F32, P, P, P, P,
         P, P, P], C.c_int),
    "vt_camera_rays": ([P, U32, U32, U32, P, P], C.c_int),
    "vt_trace_infer_f16_camera": (
        [P, P, P, U32, U32, P, P, P, U32, P, P, U32, U32, U32, U32, U32, P, I32, F32, U32, F32, P, P, P, P, P, P, P],
        C.c_int),
    "vt_trace_infer_q8_camera": (
        [P, P, P, U32, U32, P, P, P, P, P, P, P, U32, P, P, U32, U32, U32, U32, U32, P, I32, F32, U32, F32, P, P, P, P, P,
         P, P], C.c_int),
    "vt_trace_fwd": (
        [I32, P, P, P, U32, U32, P, P, U32, P, U32, P, U32, U32, U32, P, P, U32, P, F32, U32, P, P, P, P, P, P, P, P,
         P, P, P, P, P, P],
        C.c_int),
    "vt_trace_bwd": (
        [I32, P, P, P, U32, U32, P, P, U32, P, U32, P, U32, U32, U32, P, P, P, P, U32, P, P, P, P, F32, P, P, P, P,
         P, F32, U32, P, P, P, P, P, P, I32, P, P, P, P], C.c_int),
    "vt_ray_order_workspace_size": ([U32], C.c_size_t),
    "vt_ray_order": ([P, P, U32, U32, P, P, P], C.c_int),
    "vt_math_probe": ([I32, P, P, U32, P], C.c_int),
    "vt_debug_f16_atomic_add": ([P, U32, P, P, U32, P], C.c_int),
    "vt_grad_epilogue": ([P, C.c_uint64, P, C.c_uint64, P, C.c_uint64, P, P, F32, U32, P, P], C.c_int),
    "vt_adam_voro": ([P, P, P, P, P, P, P, P, P, P, P, P, U32, P, P, P, P, U32, U32, P, C.c_double, C.c_double, F32,
                      U32, F32, F32, F32, P], C.c_int),
    "vt_voronoi_workspace_size": ([U32], C.c_size_t),
    "vt_voronoi_build": ([P, U32, P, P, P, P], C.c_int),
    "vt_voronoi_build_warm": ([P, U32, P, P, U32, P, P, P, P], C.c_int),
    "vt_voronoi_adjacency": ([U32, P, P, P, P], C.c_int),
    "vt_bvh_create": ([P], C.c_int),
    "vt_bvh_destroy": ([P], C.c_int),
    "vt_bvh_build": ([P, P, U32, P], C.c_int),
    "vt_bvh_query": ([P, P, U32, P, U32, P, P], C.c_int),
    "vt_bvh_num_nodes": ([P], C.c_int),
    "vt_nearest_scan_workspace_size": ([U32], C.c_size_t),
    "vt_bvh_query_ws": ([P, P, U32, P, U32, P, P, C.c_size_t, P], C.c_int),
    "vt_start_cells_workspace_size": ([U32], C.c_size_t),
    "vt_start_cells": ([P, P, U32, P, U32, P, P, P], C.c_int),
    "vt_bvh_debug_stack_limit": ([P, U32, I32], C.c_int),
    "vt_nearest_sites_noalloc": ([P, U32, P, U32, P, P], C.c_int),
    "vt_tile_perm": ([U32, U32, U32, U32, P, P], C.c_int),
    "vt_tile_order_workspace_size": ([U32], C.c_size_t),
    "vt_tile_order": ([P, U32, U32, P, P, P], C.c_int),
    "vt_train_fwd_resident_waves": ([], U32),
    "vt_train_bwd_resident_waves": ([], U32),
    "vt_morton_workspace_size": ([U32, U32], C.c_size_t),
    "vt_morton_reorder": ([P, U32, P, U32, P, P, P, P, P, P, P], C.c_int),
    "vt_permute_rows": ([P, U32, U32, P, P, P], C.c_int),
    "vt_quantize_u8": ([P, U32, U32, I32, P, P, P, P], C.c_int),
    "vt_quantize_workspace_size": ([], C.c_size_t),
    "vt_pad_3to4_f16": ([P, U32, U32, P, P], C.c_int),
}


# include/vt_abi.h VT_NN_SCAN_PAIRS / VT_NN_SCAN_MAX_QUERIES: up to this many
# query-site pairs, and this many queries, a start-cell query scans all sites
# (vt_bvh_query_ws then needs its workspace); more queries walk the tree
NN_SCAN_PAIRS = 1 << 26
NN_SCAN_MAX_QUERIES = 64


class VTError(RuntimeError):
    pass


def load():
    """Load libvt_hip.so (once).  Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise VTError(f"{LIB_PATH} not found: build it with vorotracing_amd.build.build() (hipcc, gfx950)")
    lib = C.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue
        fn.argtypes = args
        fn.restype = res
    _lib = lib
    return lib


def exported_symbols():
    lib = load()
    return sorted(n for n in SIGNATURES if getattr(lib, n, None) is not None)


def check(rc: int, what: str):
    if rc != 0:
        msg = load().vt_last_error().decode(errors="replace")
        raise VTError(f"{what} failed (code {rc}): {msg}")


def call(name: str, *args):
    fn = getattr(load(), name)
    check(fn(*args), name)
