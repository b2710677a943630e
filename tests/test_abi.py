"""The C ABI (include/vt_abi.h) without a GPU: libvt_hip.so loads, exports
every function the header declares, the ctypes binding covers each of them
with the header's parameter count, and the host-only entries answer
(version, last error, workspace sizes, argument errors before any launch)."""
import ctypes as C
import os
import re

import pytest

from vorotracing_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "vt_abi.h")


def _declarations():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|size_t|uint32_t|const char \*)\s*(vt_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        decls[m.group(1)] = n
    return decls


def test_header_declarations_parsed():
    d = _declarations()
    assert len(d) == 49, sorted(d)
    for name in ("vt_trace_infer_f16", "vt_trace_fwd", "vt_trace_bwd", "vt_bvh_query", "vt_morton_reorder"):
        assert name in d


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [n for n in _declarations() if getattr(lib, n, None) is None]
    assert not missing, f"declared in vt_abi.h but not exported: {missing}"


def test_binding_matches_header_arity():
    for name, n in _declarations().items():
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"
        assert len(_lib.SIGNATURES[name][0]) == n, f"{name}: header has {n} parameters, binding {len(_lib.SIGNATURES[name][0])}"


def test_host_only_entries():
    lib = _lib.load()
    assert lib.vt_abi_version() == 12
    assert isinstance(lib.vt_last_error(), bytes)
    assert lib.vt_quantize_workspace_size() > 0
    assert lib.vt_morton_workspace_size(1000, 16000) >= lib.vt_morton_workspace_size(10, 160) > 0
    # 24 forward and 16 backward waves per CU; 0 where no device answers
    assert lib.vt_train_fwd_resident_waves() * 2 == lib.vt_train_bwd_resident_waves() * 3
    assert lib.vt_train_bwd_resident_waves() % 16 == 0
    # split_waves is range-checked before any launch; no tiles is no work
    assert lib.vt_tile_order(None, 0, 0, None, None, None) == 0
    assert lib.vt_tile_order(C.c_void_p(16), 10, 1 << 24, C.c_void_p(16), C.c_void_p(16), None) == 1
    assert b"split_waves" in lib.vt_last_error()
    # the walk layout's limits are checked before any launch
    big = 1 << 24
    assert lib.vt_walk_layout_fill(*[C.c_void_p(16)] * 4, big, C.c_void_p(16), C.c_void_p(16), 1, 3,
                                   *[C.c_void_p(16)] * 5, None) == 1
    assert b"below 2^24" in lib.vt_last_error()
    assert lib.vt_walk_layout_fill(*[C.c_void_p(16)] * 4, 10, C.c_void_p(16), C.c_void_p(16), 1, 4,
                                   *[C.c_void_p(16)] * 5, None) == 1
    assert b"face_order" in lib.vt_last_error()
    assert lib.vt_walk_layout_count_workspace_size(10 ** 7) >= lib.vt_walk_layout_count_workspace_size(1000) >= 0


def test_argument_errors_need_no_gpu():
    """Null pointers and bad sizes are rejected on the host, with a message."""
    lib = _lib.load()
    rc = lib.vt_trace_infer_f16_tiled(None, None, None, 4, 4, None, None, None, 10, None, None, 1, 8, 8, 8, 8, None, 0,
                                      0.01, 1024, 0.0, None, None, None, None, None, None, None)
    assert rc == 1
    assert b"null pointer" in lib.vt_last_error()
    with pytest.raises(_lib.VTError, match="null"):
        _lib.check(rc, "vt_trace_infer_f16_tiled")
    # footprint tables: the map resolution and alignment are checked before any launch
    assert lib.vt_quad_maps_f16(C.c_void_p(16), 10, 6, C.c_void_p(16), None) == 1
    assert b"res must be 4 or 8" in lib.vt_last_error()
    assert lib.vt_quad_maps_f16(C.c_void_p(16), 10, 4, C.c_void_p(8), None) == 1
    assert b"16-byte aligned" in lib.vt_last_error()
    # the allocation-free lookup rejects more queries than its scratch holds before touching a device
    rc = lib.vt_nearest_sites_noalloc(None, 1000, None, 65, None, None)
    assert rc == 1
    assert b"exceed its scratch capacity of 64" in lib.vt_last_error()


def test_every_device_kernel_has_its_host_launch_symbol(tmp_path):
    """Each kernel in the library's gfx950 code objects must have a host-side kernel
    symbol of exactly the same name, or its launches cannot find it.  Kernel
    signatures whose types mangle differently in the host and the device
    compilations (an unnamed enum in a template argument, for one) break this."""
    import shutil
    import subprocess

    bundler = "/opt/rocm/llvm/bin/clang-offload-bundler"
    readelf = "/opt/rocm/llvm/bin/llvm-readelf"
    if not (shutil.which("objcopy") and os.path.exists(bundler) and os.path.exists(readelf)):
        pytest.skip("objcopy / clang-offload-bundler / llvm-readelf not available")
    lib = _lib.LIB_PATH
    fat = tmp_path / "fatbin.bin"
    # -O binary with an output file: objcopy never rewrites the library (which this process has mapped)
    subprocess.run(["objcopy", "-O", "binary", "--only-section=.hip_fatbin", lib, str(fat)], check=True)
    data = fat.read_bytes()
    magic = b"__CLANG_OFFLOAD_BUNDLE__"
    starts = []
    i = data.find(magic)
    while i >= 0:
        starts.append(i)
        i = data.find(magic, i + 1)
    assert starts, "no offload bundles in .hip_fatbin"
    device = set()
    for k, a in enumerate(starts):
        part = tmp_path / f"bundle{k}.bin"
        part.write_bytes(data[a:starts[k + 1] if k + 1 < len(starts) else len(data)])
        co = tmp_path / f"co{k}.o"
        subprocess.run([bundler, "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--input={part}",
                        f"--output={co}", "--unbundle"], check=True)
        out = subprocess.run([readelf, "-s", "--wide", str(co)], check=True, capture_output=True, text=True).stdout
        device |= {ln.split()[-1][:-3] for ln in out.splitlines() if ln.strip().endswith(".kd")}
    host = set(subprocess.run(["nm", lib], check=True, capture_output=True, text=True).stdout.split())
    assert len(device) > 40
    missing = sorted(device - host)
    assert not missing, f"{len(missing)} device kernels without a host symbol, e.g. {missing[:2]}"
