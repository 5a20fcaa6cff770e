"""The adjacency producer without a GPU: the host tetrahedralisation and its
tables (Delaunay empty-sphere property by brute force, orientation, ordering,
neighbour encoding, vert_to_tet, CSR edges) and the oracle's
farthest_neighbor against float64 brute force."""

import numpy as np
import pytest

from oracle import oracle


@pytest.fixture(scope="module")
def small():
    from sdfoam_amd.triangulation import triangulate_host

    rng = np.random.default_rng(7)
    pts = rng.uniform(-1, 1, size=(300, 3)).astype(np.float32)
    return pts, triangulate_host(pts)


def test_empty_circumspheres(small):
    pts, t = small
    p = pts.astype(np.float64)
    tets = t["tets"].astype(np.int64)
    for tet in tets:
        a, b, c, d = p[tet]
        # circumcentre: solve 2 (x_i - a) . o = |x_i|^2 - |a|^2
        A = 2.0 * np.stack([b - a, c - a, d - a])
        rhs = np.array([b @ b - a @ a, c @ c - a @ a, d @ d - a @ a])
        o = np.linalg.solve(A, rhs)
        r2 = (a - o) @ (a - o)
        dist2 = np.sum((p - o) ** 2, axis=1)
        inside = dist2 < r2 * (1 - 1e-9)
        inside[tet] = False
        assert not inside.any()


def test_orientation_order_and_cover(small):
    pts, t = small
    p = pts.astype(np.float64)
    s = t["tets"].astype(np.int64)
    a, b, c, d = (p[s[:, k]] for k in range(4))
    vol = np.einsum("ij,ij->i", np.cross(b - a, c - a), d - a)
    assert np.all(vol > 0)
    # canonical vertex order: ascending but for the last two
    assert np.all((s[:, 0] < s[:, 1]) & (s[:, 1] < s[:, 2]) & (s[:, 1] < s[:, 3]))
    key = np.sort(s, axis=1)
    assert all(tuple(key[i]) < tuple(key[i + 1]) for i in range(len(key) - 1))
    # the tets tile the convex hull
    from scipy.spatial import ConvexHull

    assert abs(vol.sum() / 6.0 - ConvexHull(p).volume) < 1e-9


def test_tet_adjacency_and_vert_to_tet(small):
    pts, t = small
    s = t["tets"].astype(np.int64)
    adj = t["tet_adjacency"].astype(np.int64)
    T = s.shape[0]
    hull = 0
    for i in range(T):
        for j in range(4):
            v = adj[i, j]
            if v == 0xFFFFFFFF:
                hull += 1
                continue
            k, m = v // 4, v % 4
            face_i = set(s[i]) - {s[i, j]}
            face_k = set(s[k]) - {s[k, m]}
            assert face_i == face_k
            assert adj[k, m] == 4 * i + j
    from scipy.spatial import ConvexHull

    assert hull == len(ConvexHull(pts.astype(np.float64)).simplices)
    v2t = t["vert_to_tet"].astype(np.int64)
    for v in range(pts.shape[0]):
        assert v2t[v] == np.min(np.nonzero((s == v).any(axis=1))[0])


def test_point_adjacency_is_the_edge_graph(small):
    from sdfoam_amd.scenes import delaunay_adjacency

    pts, t = small
    adj, offs = delaunay_adjacency(pts)
    assert np.array_equal(adj, t["point_adjacency"]) and np.array_equal(offs, t["point_adjacency_offsets"])
    for i in range(pts.shape[0]):
        row = t["point_adjacency"][t["point_adjacency_offsets"][i]:t["point_adjacency_offsets"][i + 1]]
        assert np.all(np.diff(row.astype(np.int64)) > 0)


def test_failures():
    from sdfoam_amd.triangulation import TriangulationFailedError, triangulate_host

    flat = np.zeros((40, 3), dtype=np.float32)
    flat[:, :2] = np.random.default_rng(0).uniform(size=(40, 2))
    with pytest.raises(TriangulationFailedError):
        triangulate_host(flat)


def test_farthest_neighbor_oracle_against_float64():
    from sdfoam_amd.scenes import delaunay_adjacency

    rng = np.random.default_rng(3)
    pts = rng.normal(size=(500, 3)).astype(np.float32)
    adj, offs = delaunay_adjacency(pts)
    idx, rad = oracle.farthest_neighbor(pts, adj, offs)
    p = pts.astype(np.float64)
    for i in range(500):
        row = adj[offs[i]:offs[i + 1]].astype(np.int64)
        d = np.linalg.norm(p[row] - p[i], axis=1)
        assert idx[i] == row[np.argmax(d)]
        assert abs(rad[i] - 0.5 * d.mean()) <= 1e-6 * max(1.0, d.mean())
    # a point whose neighbours all coincide with it has no farthest neighbour
    pts2 = np.array([[0, 0, 0], [0, 0, 0], [1, 0, 0]], dtype=np.float32)
    i2, r2 = oracle.farthest_neighbor(pts2, np.array([1], dtype=np.uint32),
                                      np.array([0, 1, 1, 1], dtype=np.uint32))
    assert i2[0] == 0xFFFFFFFF and r2[0] == 0.0 and np.isnan(r2[1])


def test_has_coincident_points():
    """The incremental rebuild's duplicate check (exact: equal bit patterns
    after +0 / -0 are made equal), on host tensors: planted duplicates are
    found wherever they sit in the order, points one ulp apart and equal
    coordinates in other rows are not."""
    import torch

    from sdfoam_amd.triangulation import has_coincident_points

    rng = np.random.default_rng(3)
    pts = rng.normal(size=(5000, 3)).astype(np.float32)
    # rows sharing one or two coordinates with another row are not duplicates
    pts[10, :2] = pts[20, :2]
    pts[30, 0] = pts[40, 0]
    assert not has_coincident_points(torch.from_numpy(pts))
    for i, j in [(0, 1), (0, 4999), (1234, 17), (4998, 4999)]:
        q = pts.copy()
        q[i] = q[j]
        assert has_coincident_points(torch.from_numpy(q)), (i, j)
    q = pts.copy()
    q[5] = np.nextafter(q[6], np.float32(np.inf))
    assert not has_coincident_points(torch.from_numpy(q))
    q = pts.copy()
    q[7] = [0.0, 1.5, -2.0]
    q[8] = [-0.0, 1.5, -2.0]
    assert has_coincident_points(torch.from_numpy(q))
    assert not has_coincident_points(torch.from_numpy(pts[:1]))


def test_exhaustive_open_pass_is_bounded():
    """The open points' exhaustive certification grows as the square of
    their number: past _EXHAUSTIVE_MAX of them (and below 32) the open points
    go the Qhull way, before any GPU call."""
    import torch
    from sdfoam_amd import triangulation as T
    assert T._EXHAUSTIVE_MAX == 1 << 16
    for m in (31, T._EXHAUSTIVE_MAX + 1, 211286):
        U = torch.arange(m, dtype=torch.int32)
        assert T._open_candidates_gpu(None, None, U, None, {}) is None


def test_hull_check_finds_missing_tetrahedra():
    """_hull_is_convex, the check the GPU path's merge makes in place of
    Qhull's hull face count: a Delaunay tetrahedralisation passes; removing
    any one tetrahedron (interior, or on the hull: its inner faces are then
    exposed) leaves a face without a neighbour off the hull, which fails;
    and a face on the hull with an open point beyond it (a planted
    inconsistency) fails too."""
    import torch
    from scipy.spatial import Delaunay

    from sdfoam_amd.triangulation import _hull_is_convex

    rng = np.random.default_rng(21)
    pts_np = rng.normal(size=(400, 3)).astype(np.float32)
    d = Delaunay(pts_np.astype(np.float64))
    pts = torch.from_numpy(pts_np)
    tets = torch.from_numpy(d.simplices.astype(np.int32))
    nbr = torch.from_numpy(d.neighbors.astype(np.int32))
    T = tets.shape[0]
    U = torch.arange(pts_np.shape[0], dtype=torch.int32)
    assert _hull_is_convex(pts, tets, nbr, T, U)

    def without(t):
        keep = torch.ones(T, dtype=torch.bool)
        keep[t] = False
        remap = torch.cumsum(keep.int(), 0) - 1
        nb = nbr.clone()
        nb[nb == t] = -1
        nb = torch.where(nb >= 0, remap[nb.clamp(min=0).long()].int(), nb)
        return tets[keep].contiguous(), nb[keep].contiguous()

    hull_tet = int(np.nonzero((d.neighbors < 0).any(1))[0][0])
    inner_tet = int(np.nonzero((d.neighbors >= 0).all(1))[0][0])
    for t in (hull_tet, inner_tet):
        tt, nn = without(t)
        assert not _hull_is_convex(pts, tt, nn, T - 1, U), t
    # a point moved beyond a hull face: the face stays neighbourless but is
    # no longer a hull facet
    f_t, f_j = np.argwhere(d.neighbors < 0)[0]
    face = [d.simplices[f_t][k] for k in range(4) if k != f_j]
    far = d.simplices[f_t][f_j]
    c = pts_np[face].mean(0)
    out = pts_np.copy()
    out[far] = c + 3.0 * (c - pts_np[far])
    assert not _hull_is_convex(torch.from_numpy(out), tets, nbr, T, U)
