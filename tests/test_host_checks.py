"""Host-side argument checks that need no GPU: the warm-start guess CSR of
build_voronoi_adjacency (cuda/__init__.py:16-37's initial_guesses) and the
permutation check of explicit ray_perm lane orders (tracing_octmap.cu:642-717
reads ray_perm[t] as the ray of thread t), and the key of the tile launch
order."""
import numpy as np
import pytest
import torch

from vorotracing_amd import _C, ops

from tests import helpers as H


def test_guess_csr_accepts_a_csr():
    adj = torch.tensor([1, 2, 0, 2, 0, 1], dtype=torch.int32)
    offs = torch.tensor([0, 2, 4, 6], dtype=torch.int64)
    gofs, gadj = ops.guess_csr(adj, offs, 3, "cpu")
    assert gofs.dtype == torch.uint32 and gadj.dtype == torch.uint32
    assert gofs.tolist() == [0, 2, 4, 6] and gadj.tolist() == [1, 2, 0, 2, 0, 1]
    assert ops.guess_csr(None, None, 3, "cpu") == (None, None)
    # ids out of range are the builder's to skip, not an error
    gofs, gadj = ops.guess_csr(torch.tensor([7, 99]), torch.tensor([0, 1, 2, 2]), 3, "cpu")
    assert gadj.tolist() == [7, 99]


@pytest.mark.parametrize("offs,msg", [
    ([0, 3, 2, 6], "non-decreasing"),      # gofs[1] > gofs[2]: a reversed range reads past the list
    ([0, 2, 4, 7], "offsets end at 7"),    # beyond the 6 guesses
    ([0, 2, 4], "must have 4 entries"),
    ([-1, 2, 4, 6], "non-negative"),
])
def test_guess_csr_rejects_bad_offsets(offs, msg):
    adj = torch.tensor([1, 2, 0, 2, 0, 1])
    with pytest.raises(ValueError, match=msg):
        ops.guess_csr(adj, torch.tensor(offs), 3, "cpu")
    with pytest.raises(ValueError, match="together"):
        ops.guess_csr(adj, None, 3, "cpu")


def test_is_permutation():
    rng = np.random.default_rng(0)
    p = torch.from_numpy(rng.permutation(5000).astype(np.int32))
    assert _C.is_permutation(p, 5000)
    assert _C.is_permutation(p.view(torch.uint32), 5000)
    assert not _C.is_permutation(p, 4999)  # wrong length
    dup = p.clone()
    dup[10] = dup[11]
    assert not _C.is_permutation(dup, 5000)
    for bad in (5000, -1, 2 ** 31 - 1):
        q = p.clone()
        q[3] = bad
        assert not _C.is_permutation(q, 5000), bad
    assert _C.is_permutation(torch.empty(0, dtype=torch.int32), 0)
    assert not _C.is_permutation(p.to(torch.int64), 5000)


def test_is_permutation_sees_in_place_changes():
    """The verdict is kept per tensor and re-checked after an in-place change."""
    p = torch.arange(100, dtype=torch.int32)
    assert _C.is_permutation(p, 100)
    p[5] = 6
    assert not _C.is_permutation(p, 100)
    p[5] = 5
    assert _C.is_permutation(p, 100)


def test_tile_order_key_buckets():
    """The tile launch order's key: costs below 16 fall in the last bucket, costs
    from 2^20 the first, the key never rises with the cost, and each octave
    [2^k, 2^(k+1)) for k = 4..19 splits into 8 equal buckets."""
    k = H.tile_order_keys
    assert k([0, 1, 15, 16, 31, 1 << 20, 0xFFFFFFFF]).tolist() == [127, 127, 127, 127, 120, 0, 0]
    c = np.arange(1, 1 << 21)
    keys = k(c)
    assert np.all(np.diff(keys) <= 0)
    for e in range(4, 20):
        seg = keys[(1 << e) - 1:(1 << (e + 1)) - 1]
        vals, counts = np.unique(seg, return_counts=True)
        assert len(vals) == 8 and np.all(counts == (1 << e) // 8), e
        assert vals.max() == 127 - 8 * (e - 4) and vals.min() == 120 - 8 * (e - 4), e
    rng = np.random.default_rng(0)
    for x in rng.integers(16, 1 << 20, 2000).tolist() + [16, 17, 23, 24, 1023, 1024]:
        lb = x.bit_length() - 1
        assert k([x])[0] == 127 - (8 * (lb - 4) + ((x >> (lb - 3)) & 7)), x


def test_face_order_key():
    """The walk layout's face-order key orders f16 values numerically, takes
    -0 as +0, and puts NaNs past the infinities of their sign; every bit
    pattern gets a key, so the sort is a total order."""
    vals = np.float16([-np.inf, -65504, -1, -2.0 ** -24, -0.0, 0.0, 2.0 ** -24, 1, 65504, np.inf])
    k = H.face_order_key(vals.view(np.uint16))
    assert k[4] == k[5] and np.all(np.diff(np.delete(k, 4)) > 0)
    nan_pos, nan_neg = H.face_order_key(np.uint16([0x7E00, 0xFE00]))
    assert nan_pos > k[-1] and nan_neg < k[0]
    allk = H.face_order_key(np.arange(1 << 16, dtype=np.uint32))
    assert allk.max() < 1 << 16 and np.unique(allk).size == (1 << 16) - 1  # only -0 and +0 share a key


def test_walk_layout_np_round_trip():
    """The numpy construction of the packed walk layout (the checker of the
    GPU build) decodes back to the CSR it came from, in list order and with
    the faces laid out by their z: every slot's face record and neighbour are
    those of its original index, each cell's original indices are a
    permutation of its list (in z order when the layout sorts), pads are zero
    records with no index, and each link carries its neighbour's own head."""
    rng = np.random.default_rng(2)
    nf = np.array([0, 1, 7, 8, 9, 15, 16, 17, 0, 40, 65], np.int64)
    n = nf.size
    offsets = np.concatenate([[0], np.cumsum(nf)])
    F = int(offsets[-1])
    adjacency = rng.integers(0, n, F + 32)
    adj_diff = rng.integers(1, 1 << 14, (F + 32, 4)).astype(np.uint16)
    adj_diff[3:6, 2] = adj_diff[2, 2]  # equal z values: list order among them
    adj_diff[10:14, 2] = [0x8000, 0x0000, 0x8001, 0x0001]  # -0 and +0 tie; -2^-24 below them, 2^-24 above
    points = rng.standard_normal((n, 3)).astype(np.float32)
    density = rng.random(n).astype(np.float32)
    for order in (0, 3):
        first, chunks, links, heads, cells, orig = H.walk_layout_np(points, density, adjacency, offsets, adj_diff,
                                                                    face_order=order)
        nch = (nf + 7) // 8
        assert first[n] == nch.sum() and first[n + 1] == nch.max() and chunks.shape == (nch.sum(), 12)
        halves = chunks.view(np.uint16).reshape(-1, 8, 3)
        for c in range(n):
            assert heads[c, 0] == (c | nch[c] << 24) and heads[c, 1] == first[c]
            assert np.array_equal(cells[c], np.append(points[c], density[c]))
            seen = []
            for f in range(8 * nch[c]):
                q, j = divmod(f, 8)
                rec = halves[first[c] + q, j]
                lk = links[8 * (first[c] + q) + j]
                og = int(orig[8 * (first[c] + q) + j])
                if f < nf[c]:
                    assert np.array_equal(rec, adj_diff[offsets[c] + og, :3])
                    assert np.array_equal(lk, heads[adjacency[offsets[c] + og]])
                    seen.append(og)
                else:
                    assert not rec.any() and not lk.any() and og == 0xFFFF
            assert sorted(seen) == list(range(nf[c]))
            if order == 0 or nf[c] > 64:
                assert seen == list(range(nf[c]))
            else:
                z = adj_diff[offsets[c] + np.array(seen, np.int64), 2].view(np.float16).astype(np.float32)
                assert np.all(np.diff(z) >= 0)
                ties = np.diff(z) == 0
                assert np.all(np.diff(np.array(seen))[ties] > 0)


def test_quad_table_bytes():
    """The footprint tables' size: (R + 1)^2 entries per map and cell, 32
    bytes for fp16 maps, 16 for q8."""
    from vorotracing_amd import native
    f16 = torch.zeros((10, 4 * 16), dtype=torch.float16)
    f16_8 = torch.zeros((10, 4 * 64), dtype=torch.float16)
    q8 = torch.zeros((10, 3 * 16), dtype=torch.uint8)
    assert native.QuadMaps.table_bytes(f16, f16) == 10 * 32 * 25 * 2
    assert native.QuadMaps.table_bytes(f16_8, f16) == 10 * 32 * (81 + 25)
    assert native.QuadMaps.table_bytes(q8, q8) == 10 * 16 * 25 * 2


def test_quad_maps_reject_mismatched_maps():
    """The footprint tables are built for one scene: maps with different row
    counts are refused on the host, before any launch."""
    from vorotracing_amd import native
    with pytest.raises(ValueError, match="rows"):
        native.QuadMaps.build(torch.zeros((10, 64), dtype=torch.float16), torch.zeros((9, 64), dtype=torch.float16))
