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
    for m in re.finditer(r"\b(?:int|size_t|const char \*)\s*(vt_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        params = m.group(2).strip()
        n = 0 if params in ("", "void") else params.count(",") + 1
        decls[m.group(1)] = n
    return decls


def test_header_declarations_parsed():
    d = _declarations()
    assert len(d) == 25, sorted(d)
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
    assert lib.vt_abi_version() == 2
    assert isinstance(lib.vt_last_error(), bytes)
    assert lib.vt_quantize_workspace_size() > 0
    assert lib.vt_morton_workspace_size(1000, 16000) >= lib.vt_morton_workspace_size(10, 160) > 0


def test_argument_errors_need_no_gpu():
    """Null pointers and bad sizes are rejected on the host, with a message."""
    lib = _lib.load()
    rc = lib.vt_trace_infer_f16_tiled(None, None, None, 4, 4, None, None, None, 10, None, None, 1, 8, 8, 8, 8, None,
                                      0.01, 1024, 0.0, None, None, None)
    assert rc == 1
    assert b"null pointer" in lib.vt_last_error()
    with pytest.raises(_lib.VTError, match="null"):
        _lib.check(rc, "vt_trace_infer_f16_tiled")
