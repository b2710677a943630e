"""GPU test of vt_nearest_sites_noalloc, the allocation-free start-cell lookup:
through the C ABI, its answers equal vt_bvh_query's (the existing entry point,
through its LBVH handle) and the brute-force nearest site, bit for bit, on two
calls in a row (the second smaller, so stale partials of the first would show),
with ties to the lowest index across lanes, waves, blocks and strides."""
import ctypes as C

import numpy as np
import pytest
import torch

from oracle import host_ops
from tests import helpers as H
from vorotracing_amd import _lib

pytestmark = pytest.mark.gpu

MAX_QUERIES = 64  # the entry point's stated scratch capacity


def _noalloc(pts_d, q_d):
    nq = q_d.shape[0]
    out = torch.full((nq,), -7, dtype=torch.int32, device=pts_d.device)
    _lib.call("vt_nearest_sites_noalloc", pts_d.data_ptr(), pts_d.shape[0], q_d.data_ptr(), nq, out.data_ptr(),
              torch.cuda.current_stream(pts_d.device).cuda_stream)
    return out


def _bvh_query(pts_d, q_d):
    h = C.c_void_p()
    _lib.call("vt_bvh_create", C.byref(h))
    try:
        s = torch.cuda.current_stream(pts_d.device).cuda_stream
        _lib.call("vt_bvh_build", h, pts_d.data_ptr(), pts_d.shape[0], s)
        out = torch.full((q_d.shape[0],), -7, dtype=torch.int32, device=pts_d.device)
        _lib.call("vt_bvh_query", h, pts_d.data_ptr(), pts_d.shape[0], q_d.data_ptr(), q_d.shape[0], out.data_ptr(), s)
        torch.cuda.synchronize()
    finally:
        _lib.load().vt_bvh_destroy(h)
    return out.cpu().numpy()


def _random_case(n, nq, seed):
    rng = np.random.default_rng(seed)
    pts = rng.normal(size=(n, 3)).astype(np.float32)
    q = np.concatenate([rng.normal(size=(nq - nq // 2, 3)).astype(np.float32) * 1.5,
                        pts[rng.integers(0, n, size=nq // 2)]])  # half exactly on sites
    return pts, q


def test_noalloc_equals_bvh_query_two_calls(gpu):
    print("case: vt_nearest_sites_noalloc, tie set 300000 sites then random 5000 sites", flush=True)
    big_pts, big_q = H.nn_tie_set()                 # 28 queries, every one a tie
    extra = _random_case(300000, 36, 5)[1]          # fill to the 64-query capacity
    big_q = np.concatenate([big_q, extra]).astype(np.float32)
    assert big_q.shape[0] == MAX_QUERIES
    small_pts, small_q = _random_case(5000, 9, 6)
    results = []
    for pts, q in ((big_pts, big_q), (small_pts, small_q)):
        pd, qd = H.to_dev(pts, gpu), H.to_dev(q, gpu)
        got = _noalloc(pd, qd)
        torch.cuda.synchronize()
        got = got.cpu().numpy()
        want_abi = _bvh_query(pd, qd)
        want_bf = host_ops.nearest_site(pts, q)
        assert got.dtype == np.int32
        assert np.array_equal(got, want_abi), f"differs from vt_bvh_query at {np.nonzero(got != want_abi)[0][:8]}"
        assert np.array_equal(got, want_bf), f"differs from brute force at {np.nonzero(got != want_bf)[0][:8]}"
        results.append(got)
    assert results[1].shape == (9,)


def test_noalloc_limits(gpu):
    pts, q = _random_case(1000, 64, 8)
    pd = H.to_dev(pts, gpu)
    q65 = H.to_dev(np.concatenate([q, q[:1]]), gpu)
    out = torch.empty(65, dtype=torch.int32, device=gpu)
    with pytest.raises(_lib.VTError, match="exceed its scratch capacity of 64"):
        _lib.call("vt_nearest_sites_noalloc", pd.data_ptr(), 1000, q65.data_ptr(), 65, out.data_ptr(), None)
    # zero queries: a no-op, nothing dereferenced
    _lib.call("vt_nearest_sites_noalloc", None, 0, None, 0, None, None)
    with pytest.raises(_lib.VTError, match="null pointer"):
        _lib.call("vt_nearest_sites_noalloc", None, 1000, q65.data_ptr(), 3, out.data_ptr(), None)
    # one site: every query answers 0
    one = H.to_dev(pts[:1], gpu)
    got = _noalloc(one, H.to_dev(q[:5], gpu))
    torch.cuda.synchronize()
    assert got.cpu().numpy().tolist() == [0] * 5


def test_noalloc_under_graph_capture(gpu):
    """The entry captured into a graph (its device set up by a zero-query call
    first, buffers allocated before the capture): every replay answers the
    queries the buffer holds at that replay, with eager work and
    synchronisations between replays."""
    print("case: vt_nearest_sites_noalloc captured in a graph, 20000 sites, 48 queries", flush=True)
    pts, q0 = _random_case(20000, 48, 9)
    pd, qd = H.to_dev(pts, gpu), H.to_dev(q0, gpu)
    out = torch.full((48,), -7, dtype=torch.int32, device=gpu)
    _lib.call("vt_nearest_sites_noalloc", None, 0, None, 0, None, None)  # device set-up, no launch
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):  # eager call on the capture stream before capturing (torch's warm-up rule)
        _lib.call("vt_nearest_sites_noalloc", pd.data_ptr(), pd.shape[0], qd.data_ptr(), 48, out.data_ptr(),
                  side.cuda_stream)
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _lib.call("vt_nearest_sites_noalloc", pd.data_ptr(), pd.shape[0], qd.data_ptr(), 48, out.data_ptr(),
                  torch.cuda.current_stream(gpu).cuda_stream)
    for k in range(4):
        q = _random_case(20000, 48, 100 + k)[1]
        qd.copy_(H.to_dev(q, gpu))
        out.fill_(-7)
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        assert np.array_equal(got, host_ops.nearest_site(pts, q)), f"replay {k}"
        # eager work between replays, on the same scratch array
        eager = _noalloc(pd, H.to_dev(q[:5], gpu))
        torch.cuda.synchronize()
        assert np.array_equal(eager.cpu().numpy(), got[:5])
