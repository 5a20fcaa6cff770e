"""The GPU Delaunay's per-item code (sdfoam_amd/csrc/voronoi_cell.h and
delaunay_grid.h, built for the host by g++ from tests/vcell_host.cpp) against
Qhull: certified cells report exactly the Delaunay tetrahedra of their point,
and [certified tets, each from its lowest certified vertex] + [Qhull of the
open points, kept where the circumsphere is empty] is exactly Qhull's
tetrahedralisation of all points.  This is the same selection the device
merge (sdf_delaunay_merge) makes; the GPU tests compare the device result
with Qhull as well."""

import ctypes as C
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
P = C.c_void_p


@pytest.fixture(scope="module")
def vc(tmp_path_factory):
    out = tmp_path_factory.mktemp("vcell") / "libvcell.so"
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-ffp-contract=off",
                    os.path.join(ROOT, "tests", "vcell_host.cpp"), "-o", str(out)], check=True)
    L = C.CDLL(str(out))
    L.vc_grid.argtypes = [P, C.c_uint32, P]
    L.vc_grid.restype = C.c_int
    L.vc_certify.argtypes = [P, C.c_uint32, P, P, C.c_longlong, P]
    L.vc_certify.restype = C.c_longlong
    L.vc_sphere_empty.argtypes = [P, P, C.c_longlong, P, P]
    L.vc_box_unpaired.restype = C.c_int
    L.vc_insphere.argtypes = [P, P, P, P]
    L.vc_insphere.restype = C.c_int
    L.vc_grid_mismatches.argtypes = [P, C.c_uint32]
    L.vc_grid_mismatches.restype = C.c_longlong
    return L


def _p(a):
    return a.ctypes.data_as(P)


def _delaunay(pts):
    from scipy.spatial import Delaunay

    return Delaunay(np.asarray(pts, dtype=np.float64))


def _tet_set(t):
    return set(map(tuple, np.sort(np.asarray(t), axis=1).tolist()))


def assert_delaunay(pts, tets, hull_volume):
    """tets [T, 4] is a Delaunay tetrahedralisation of pts: every tet has
    positive volume, they tile the convex hull, and no point lies inside a
    circumsphere by more than rounding (cospherical points may sit on it)."""
    from scipy.spatial import cKDTree

    p = np.asarray(pts, dtype=np.float64)
    t = np.asarray(tets, dtype=np.int64)
    a, b, c, d = (p[t[:, k]] for k in range(4))
    vol = np.abs(np.einsum("ij,ij->i", np.cross(b - a, c - a), d - a)) / 6.0
    assert (vol > 0).all()
    assert abs(vol.sum() - hull_volume) <= 1e-9 * hull_volume
    A = 2.0 * np.stack([b - a, c - a, d - a], axis=1)
    rhs = np.stack([(b * b).sum(1) - (a * a).sum(1), (c * c).sum(1) - (a * a).sum(1),
                    (d * d).sum(1) - (a * a).sum(1)], axis=1)
    ctr = np.linalg.solve(A, rhs[..., None])[..., 0]
    r = np.sqrt(((a - ctr) ** 2).sum(1))
    tree = cKDTree(p)
    for k in range(len(t)):
        inside = tree.query_ball_point(ctr[k], r[k] * (1 - 1e-9))
        assert set(inside) <= set(t[k].tolist()), (k, t[k])


def _cells_and_merge(L, pts):
    n = pts.shape[0]
    dims = np.zeros(3, np.uint32)
    assert L.vc_grid(_p(pts), n, _p(dims)) > 0
    status = np.zeros(n, np.uint32)
    cap = 40 * n
    rep = np.zeros((cap, 4), np.uint32)
    co = C.c_longlong()
    rows = L.vc_certify(_p(pts), n, _p(status), _p(rep), cap, C.byref(co))
    assert 0 < rows <= cap and co.value == 0
    rep = rep[:rows]
    cert = status == 0
    U = np.nonzero(~cert)[0]
    lower_cert = ((rep[:, 1:] < rep[:, :1]) & cert[rep[:, 1:]]).any(axis=1)
    kept = rep[~lower_cert]
    cand = np.ascontiguousarray(U[_delaunay(pts[U]).simplices].astype(np.uint32))
    keep = np.zeros(len(cand), np.uint32)
    L.vc_sphere_empty(_p(pts), _p(cand), len(cand), _p(status), _p(keep))
    assert not (keep == 2).any()
    return status, rep, kept, cand[keep == 1]


def _sets():
    rng = np.random.default_rng(5)
    n = 3000
    c = rng.normal(size=(12, 3)) * 3
    s = rng.normal(size=(n, 3))
    s /= np.linalg.norm(s, axis=1, keepdims=True)
    return {
        "uniform": rng.random((n, 3)),
        "gaussian": rng.normal(size=(n, 3)),
        "clustered": c[rng.integers(0, 12, n)] + rng.normal(size=(n, 3)) * 0.05,
        "anisotropic": rng.random((n, 3)) * np.array([10.0, 1.0, 0.1]),
        "shell": np.concatenate([s * (0.5 + 0.02 * rng.normal(size=(n, 1))),
                                 rng.uniform(-1.5, 1.5, size=(n // 4, 3))]),
        # the cube's corners are cospherical: the open points' triangulation
        # decides how each face is split
        "cube_corners": np.concatenate([rng.uniform(-1, 1, size=(n, 3)),
                                        [[x, y, z] for x in (-1, 1) for y in (-1, 1)
                                         for z in (-1, 1)]]),
    }


@pytest.mark.parametrize("name", list(_sets()))
def test_cells_plus_open_points_give_qhull(vc, name):
    from scipy.spatial import ConvexHull

    pts = np.ascontiguousarray(_sets()[name], dtype=np.float32)
    status, rep, kept, cand_kept = _cells_and_merge(vc, pts)
    ref = _tet_set(_delaunay(pts).simplices)
    got = np.concatenate([kept, cand_kept])
    assert len(_tet_set(got)) == len(got)  # each tet once
    if name == "cube_corners":
        # each face of the cube is cospherical: any split of it is Delaunay
        assert_delaunay(pts, got, ConvexHull(pts.astype(np.float64)).volume)
    else:
        assert _tet_set(got) == ref
    # every certified point reports exactly its own Delaunay tets
    full = np.sort(_delaunay(pts).simplices, axis=1)
    for i in np.nonzero(status == 0)[0][:50] if name != "cube_corners" else []:
        assert _tet_set(rep[rep[:, 0] == i]) == _tet_set(full[(full == i).any(axis=1)])
    assert (status == 0).mean() > (0.3 if name in ("anisotropic", "shell") else 0.8)


def test_hull_points_are_never_certified(vc):
    from scipy.spatial import ConvexHull

    pts = np.ascontiguousarray(np.random.default_rng(2).random((2000, 3)), dtype=np.float32)
    status, *_ = _cells_and_merge(vc, pts)
    hull = np.unique(ConvexHull(pts.astype(np.float64)).simplices)
    assert (status[hull] != 0).all()


def test_coincident_points_are_reported(vc):
    pts = np.random.default_rng(3).random((500, 3)).astype(np.float32)
    pts[17] = pts[400]
    dims = np.zeros(3, np.uint32)
    vc.vc_grid(_p(pts), 500, _p(dims))
    status = np.zeros(500, np.uint32)
    rep = np.zeros((40 * 500, 4), np.uint32)
    co = C.c_longlong()
    vc.vc_certify(_p(pts), 500, _p(status), _p(rep), 40 * 500, C.byref(co))
    assert co.value == 2 and status[17] == 2 and status[400] == 2


def test_insphere_signs_and_box_orientation(vc):
    assert vc.vc_box_unpaired() == 0
    a = np.array([1.0, 0, 0])
    b = np.array([0, 1.0, 0])
    c = np.array([0, 0, 1.0])
    # the sphere through 0, a, b, c has centre (0.5, 0.5, 0.5)
    inside = np.array([0.5, 0.5, 0.5])
    outside = np.array([2.0, 2.0, 2.0])
    on = np.array([1.0, 1.0, 0.0])
    assert vc.vc_insphere(_p(a), _p(b), _p(c), _p(inside)) == 1
    assert vc.vc_insphere(_p(a), _p(b), _p(c), _p(outside)) == -1
    assert vc.vc_insphere(_p(a), _p(b), _p(c), _p(on)) == 0
    # orientation does not change the answer
    assert vc.vc_insphere(_p(b), _p(a), _p(c), _p(inside)) == 1


def test_assert_delaunay_rejects_the_other_triangulation():
    """Five points with two tetrahedralisations (2 tets across triangle abc,
    or 3 around edge de): exactly one of them is Delaunay, and a missing tet
    fails the volume check."""
    from scipy.spatial import ConvexHull

    s3 = np.sqrt(3.0) / 2.0
    for dz in (0.6, 2.0):  # d, e near the equator or far out
        pts = np.array([[1, 0, 0.1], [-0.5, s3, 0], [-0.5, -s3, 0], [0.1, 0, dz],
                        [0, 0.1, -dz]], dtype=np.float32)
        two = np.array([[0, 1, 2, 3], [0, 1, 2, 4]])
        three = np.array([[3, 4, 0, 1], [3, 4, 1, 2], [3, 4, 2, 0]])
        vol = ConvexHull(pts.astype(np.float64)).volume
        ok = []
        for t in (two, three):
            try:
                assert_delaunay(pts, t, vol)
                ok.append(True)
            except AssertionError:
                ok.append(False)
        assert sum(ok) == 1, (dz, ok)
        good = two if ok[0] else three
        assert _tet_set(_delaunay(pts).simplices) == _tet_set(good)
        with pytest.raises(AssertionError):
            assert_delaunay(pts, good[1:], vol)


@pytest.mark.parametrize("kind", ["uniform", "shell", "clustered", "flat", "offset"])
def test_one_morton_order_serves_every_level(vc, kind):
    """The grids sort the points once, by the Morton code of their finest
    cell: every level's cell (from a position, as a lookup computes it) is the
    finest cell shifted right by the level, and every level's cells are
    contiguous runs of that one order.  Both table lookups (one slot at a
    time, and 64-byte groups of four) find each point's cell, holding it,
    and agree on the cells beside it.  Includes points on the bounding
    box's far faces (clamped to the last cell) and a flat set (one cell
    across an axis)."""
    rng = np.random.default_rng(11)
    n = 20000
    if kind == "uniform":
        pts = rng.uniform(-1, 1, (n, 3))
    elif kind == "shell":
        v = rng.normal(size=(n, 3))
        pts = v / np.linalg.norm(v, axis=1, keepdims=True) * (1 + 1e-3 * rng.normal(size=(n, 1)))
    elif kind == "clustered":
        c = rng.uniform(-5, 5, (20, 3))
        pts = c[rng.integers(0, 20, n)] + 10.0 ** rng.uniform(-4, -1, (n, 1)) * rng.normal(size=(n, 3))
    elif kind == "flat":
        pts = np.c_[rng.uniform(0, 1, (n, 2)), np.zeros(n)]
    else:
        pts = 1000.0 + rng.uniform(0, 1e-2, (n, 3))
    # points exactly on the box's faces and corners
    pts[:8] = np.array([[a, b, c] for a in (0, 1) for b in (0, 1) for c in (0, 1)]) * (
        pts.max(0) - pts.min(0)) + pts.min(0)
    pts = np.ascontiguousarray(pts, dtype=np.float32)
    dims = np.zeros(3, dtype=np.uint32)
    assert vc.vc_grid(_p(pts), n, _p(dims)) > 0
    assert vc.vc_grid_mismatches(_p(pts), n) == 0
