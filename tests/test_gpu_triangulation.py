"""The adjacency producer on the GPU box: farthest_neighbor bit-exact against
the oracle, and Triangulation driven the way sdfoam_model/scene.py drives it
(construct, permute the points, rebuild incrementally, trace on the
adjacency)."""

import numpy as np
import pytest

from conftest import scene
from oracle import oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _u32(a, dev):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint32).view(np.int32)).to(dev).view(torch.uint32)


def _np(t):
    import torch

    return t.view(torch.int32).cpu().numpy().view(np.uint32)


@pytest.mark.parametrize("cfg", [1, 2])
def test_farthest_neighbor_bitexact(dev, cfg):
    import torch

    import sdfoam_amd

    w = scene(cfg)
    pts = torch.from_numpy(w.points).to(dev)
    idx, rad = sdfoam_amd.farthest_neighbor(pts, _u32(w.adjacency, dev), _u32(w.offsets, dev))
    torch.cuda.synchronize()
    ridx, rrad = oracle.farthest_neighbor(w.points, w.adjacency, w.offsets)
    assert idx.dtype == torch.uint32 and rad.dtype == torch.float32
    assert np.array_equal(_np(idx), ridx)
    assert np.array_equal(rad.cpu().numpy().view(np.uint32), rrad.view(np.uint32))


def test_triangulation_as_scene_uses_it(dev):
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes
    from sdfoam_amd.triangulation import triangulate_host

    rng = np.random.default_rng(21)
    raw = torch.from_numpy(rng.normal(size=(3000, 3)).astype(np.float32) * 0.6).to(dev)
    tri = sdfoam_amd.Triangulation(raw)
    assert tri.last_method == "gpu"
    perm = tri.permutation().to(torch.long)
    assert np.array_equal(perm.cpu().numpy(), scenes.sort_points_order(raw.cpu().numpy()))
    pts = raw[perm]
    host = triangulate_host(pts.cpu().numpy())
    for k in ("tets", "tet_adjacency", "vert_to_tet", "point_adjacency", "point_adjacency_offsets"):
        assert np.array_equal(_np(getattr(tri, k)()).reshape(host[k].shape), host[k]), k
    # moved points, same count: no re-sort, tables of the moved points
    moved = pts + 1e-3 * torch.randn_like(pts)
    assert tri.rebuild(moved, incremental=True) is False
    host2 = triangulate_host(moved.cpu().numpy())
    assert np.array_equal(_np(tri.point_adjacency()), host2["point_adjacency"])
    assert tri.rebuild(moved, incremental=False) is True
    # trace on the triangulation's adjacency: forward parity with the oracle
    pts_np = moved[tri.permutation().to(torch.long)].cpu().numpy()
    tri.rebuild(torch.from_numpy(pts_np).to(dev), incremental=True)
    adj, offs = _np(tri.point_adjacency()), _np(tri.point_adjacency_offsets())
    cam = scenes.look_at([0.0, 0.0, 3.0], [0.0, 0.0, 0.0], [0.0, 1.0, 0.0], 0.8, 32, 32)
    rays = scenes.pinhole_rays(cam)
    start = scenes.start_points_for(pts_np, rays)
    attrs = rng.uniform(0, 1, size=(3000, 4)).astype(np.float32)
    attrs[:, 3] = np.linalg.norm(pts_np, axis=1) - 0.5
    pipe = sdfoam_amd.create_pipeline(0)
    out = pipe.trace_forward(torch.from_numpy(pts_np).to(dev), torch.from_numpy(attrs).to(dev),
                             tri.point_adjacency(), tri.point_adjacency_offsets(),
                             torch.from_numpy(rays).to(dev), _u32(start, dev),
                             alpha_mode="sdfoam", inv_s=5.0)
    torch.cuda.synchronize()
    ref = oracle.trace_forward(0, pts_np, attrs, adj, offs, rays, start, None,
                               alpha_mode="sdfoam", inv_s=5.0)
    assert np.array_equal(_np(out["num_intersections"]).reshape(-1), ref.num_intersections.reshape(-1))
    assert np.max(np.abs(out["rgba"].cpu().numpy() - ref.rgba)) < 1e-5


def test_triangulation_errors(dev):
    import torch

    import sdfoam_amd

    pts = torch.randn(100, 3, device=dev)
    pts[7] = pts[50]
    with pytest.raises(sdfoam_amd.TriangulationFailedError, match="duplicate points"):
        sdfoam_amd.Triangulation(pts)
    with pytest.raises(RuntimeError, match="less than 32 points"):
        sdfoam_amd.Triangulation(torch.randn(20, 3, device=dev))
    with pytest.raises(RuntimeError, match="CUDA device"):
        sdfoam_amd.Triangulation(torch.randn(100, 3))


@pytest.mark.parametrize("n", [33, 1025, 4097, 300_001, 2_500_000])
def test_sort_points_matches_host(dev, n):
    """Every branch of the pass rule: 1024-point blocks, whole-array passes
    and (from more than 1024 segments of more than 1024 points, n > 2^21)
    per-segment passes."""
    import torch

    from sdfoam_amd import scenes
    from sdfoam_amd.triangulation import sort_points

    rng = np.random.default_rng(n)
    pts = rng.normal(size=(n, 3)).astype(np.float32)
    pts[: n // 10, 1] = 0.25  # equal keys: the passes must be stable
    got = _np(sort_points(torch.from_numpy(pts).to(dev)))
    assert np.array_equal(got, scenes.sort_points_order(pts))


@pytest.mark.parametrize("cfg", [1, 2])
def test_device_tables_match_host(dev, cfg):
    """sdf_delaunay_tables against the numpy statement on the same Qhull
    tetrahedra: every table bit-exact."""
    import torch

    from sdfoam_amd.triangulation import device_tables, host_tables, qhull_tetrahedra

    w = scene(cfg)
    simplices, neighbors = qhull_tetrahedra(w.points)
    got = device_tables(torch.from_numpy(w.points).to(dev), simplices, neighbors)
    ref = host_tables(w.points, simplices, neighbors)
    for k, v in ref.items():
        assert np.array_equal(_np(got[k]).reshape(v.shape), v), k
    # the scene's own CSR adjacency is the same edge graph
    assert np.array_equal(_np(got["point_adjacency"]), w.adjacency)
    assert np.array_equal(_np(got["point_adjacency_offsets"]), w.offsets)


def _gpu_sets():
    rng = np.random.default_rng(8)
    n = 60_000
    c = rng.normal(size=(16, 3)) * 3
    sh = rng.normal(size=(n, 3))
    sh /= np.linalg.norm(sh, axis=1, keepdims=True)
    return {
        "C1": lambda: scene(1).points,
        "C2": lambda: scene(2).points,
        "gaussian": lambda: rng.normal(size=(n, 3)).astype(np.float32),
        "clustered": lambda: (c[rng.integers(0, 16, n)] + rng.normal(size=(n, 3)) * 0.05).astype(np.float32),
        "shell": lambda: (sh * (1 + 0.01 * rng.random((n, 1)))).astype(np.float32),
    }


def _face_neighbors(tets):
    """[T, 4]: the tet across the face opposite vertex j (-1 if none), by
    matching sorted vertex triples."""
    T = tets.shape[0]
    faces = np.stack([np.delete(tets, j, axis=1) for j in range(4)], axis=1).reshape(-1, 3)
    key = np.sort(faces.astype(np.int64), axis=1)
    key = (key[:, 0] << 42) | (key[:, 1] << 21) | key[:, 2]
    order = np.argsort(key, kind="stable")
    ks = key[order]
    nbr = np.full(4 * T, -1, dtype=np.int64)
    same = np.nonzero(ks[1:] == ks[:-1])[0]
    assert not np.any(same[1:] == same[:-1] + 1)  # no face of three tets
    a, b = order[same], order[same + 1]
    nbr[a] = b // 4
    nbr[b] = a // 4
    return nbr.reshape(T, 4).astype(np.int32)


@pytest.mark.parametrize("name", list(_gpu_sets()))
def test_gpu_tetrahedra_match_qhull(dev, name):
    """sdf_delaunay_certify + the open points' exhaustive certification
    (sdf_delaunay_certify_exhaustive; Qhull of them where it cannot decide) +
    sdf_delaunay_merge: the same tetrahedra as Qhull on every point, and
    (through sdf_delaunay_tables) every derived table bit-exact."""
    import torch

    from sdfoam_amd.triangulation import device_tables, gpu_tetrahedra, host_tables, qhull_tetrahedra

    from scipy.spatial import ConvexHull

    from test_delaunay_cells import assert_delaunay

    import sdfoam_amd
    from sdfoam_amd.triangulation import _Undecided

    pts = np.ascontiguousarray(_gpu_sets()[name](), dtype=np.float32)
    print(f"gpu_tetrahedra {name} n={pts.shape[0]}", flush=True)
    pd = torch.from_numpy(pts).to(dev)
    if name == "C1":
        # C1 holds the cube's corners: each face of the cube is cospherical.
        # A certified point on such a sphere leaves the split undecided, and
        # Triangulation then runs Qhull on every point.
        try:
            tets, nbr, stats = gpu_tetrahedra(pd)
        except _Undecided:
            tri = sdfoam_amd.Triangulation(pd)
            assert tri.last_method == "qhull"
            return
    else:
        tets, nbr, stats = gpu_tetrahedra(pd)
    tets_np, nbr_np = tets.cpu().numpy(), nbr.cpu().numpy()
    # neighbours by face matching in numpy
    assert np.array_equal(nbr_np, _face_neighbors(tets_np))
    if name == "C1":
        # C1 holds the cube's corners: each face of the cube is cospherical,
        # and either split of it is Delaunay
        assert_delaunay(pts, tets_np, ConvexHull(pts.astype(np.float64)).volume)
        simplices, neighbors = tets_np, nbr_np
    else:
        simplices, neighbors = qhull_tetrahedra(pts)
        got = np.sort(tets_np, axis=1)
        ref = np.sort(simplices, axis=1)
        assert got.shape == ref.shape
        got = got[np.lexsort(got[:, ::-1].T)]
        ref = ref[np.lexsort(ref[:, ::-1].T)]
        assert np.array_equal(got, ref)
        assert stats["tets"] == simplices.shape[0]
    if name not in ("shell",):
        # the hull layer is a larger share of a small set
        assert stats["open"] < (0.2 if pts.shape[0] < 10_000 else 0.12) * pts.shape[0], stats
    print({k: v for k, v in stats.items() if k.startswith("open") and k != "open_ids"}, flush=True)
    if name != "C1":
        # the open points' tetrahedra came from the GPU, not Qhull
        assert stats["open_points_qhull"] == 0 and "open_gpu_retry" not in stats, stats
    mine = device_tables(pd, tets, nbr)
    host = host_tables(pts, simplices, neighbors)
    for k, v in host.items():
        assert np.array_equal(_np(mine[k]).reshape(v.shape), v), k


@pytest.mark.parametrize("name,scale", [("gaussian", 0.0), ("gaussian", 1e-3), ("clustered", 1e-3),
                                        ("shell", 1e-3), ("C2", 3e-4), ("C2", 1e-3)])
def test_incremental_rebuild_matches_qhull(dev, name, scale):
    """rebuild(incremental=True) over moved points (each coordinate moved by
    `scale` times the point's cell radius, N(0, 1)): the old tetrahedra whose
    circumspheres stay empty are kept, the dirty points re-certified, and
    every table equals Qhull's on the moved points."""
    import torch

    import sdfoam_amd
    from sdfoam_amd.triangulation import triangulate_host

    raw = np.ascontiguousarray(_gpu_sets()[name](), dtype=np.float32)
    n = raw.shape[0]
    print(f"incremental {name} n={n} scale={scale}", flush=True)
    tri = sdfoam_amd.Triangulation(torch.from_numpy(raw).to(dev))
    assert tri.last_method == "gpu"
    pts = raw[tri.permutation().view(torch.int32).cpu().numpy()]
    _, radius = sdfoam_amd.farthest_neighbor(torch.from_numpy(pts).to(dev), tri.point_adjacency(),
                                             tri.point_adjacency_offsets())
    r = radius.cpu().numpy()[:, None]
    rng = np.random.default_rng(5)
    moved = (pts + scale * r * rng.normal(size=pts.shape)).astype(np.float32)
    assert tri.rebuild(torch.from_numpy(moved).to(dev), incremental=True) is False
    st = tri.last_stats
    print({k: v for k, v in st.items() if not k.endswith("_s")}, flush=True)
    assert tri.last_method == "gpu" and st.get("incremental"), st
    assert st["verified"] > 0 and st["dirty"] < 0.5 * n, st
    assert st["open_points_qhull"] == 0 and "open_gpu_retry" not in st, st
    host = triangulate_host(moved)
    for k in ("tets", "tet_adjacency", "vert_to_tet", "point_adjacency", "point_adjacency_offsets"):
        assert np.array_equal(_np(getattr(tri, k)()).reshape(host[k].shape), host[k]), k
    # and again from the incremental result
    moved2 = (moved + scale * r * rng.normal(size=pts.shape)).astype(np.float32)
    tri.rebuild(torch.from_numpy(moved2).to(dev), incremental=True)
    assert tri.last_stats.get("incremental"), tri.last_stats
    host2 = triangulate_host(moved2)
    for k in ("tets", "point_adjacency", "point_adjacency_offsets"):
        assert np.array_equal(_np(getattr(tri, k)()).reshape(host2[k].shape), host2[k]), k


def test_incremental_rebuild_falls_back_when_most_points_move(dev):
    """Points moved by about their spacing leave most of them dirty: the
    rebuild is a full one, with the same tables as Qhull's."""
    import torch

    import sdfoam_amd
    from sdfoam_amd.triangulation import triangulate_host

    raw = np.ascontiguousarray(_gpu_sets()["gaussian"](), dtype=np.float32)
    tri = sdfoam_amd.Triangulation(torch.from_numpy(raw).to(dev))
    pts = raw[tri.permutation().view(torch.int32).cpu().numpy()]
    rng = np.random.default_rng(6)
    moved = rng.normal(size=pts.shape).astype(np.float32)
    tri.rebuild(torch.from_numpy(moved).to(dev), incremental=True)
    assert tri.last_method == "gpu" and not tri.last_stats.get("incremental"), tri.last_stats
    host = triangulate_host(moved)
    assert np.array_equal(_np(tri.point_adjacency()), host["point_adjacency"])


@pytest.mark.parametrize("where", ["hull", "interior"])
def test_incremental_rebuild_rejects_coincident_points(dev, where):
    """An incremental rebuild over points where one was moved onto another
    raises TriangulationFailedError, as the reference's does
    (src/delaunay/delaunay.cu:291-294): for two vertices of the old hull
    (which the rebuild sends to the open points without certifying them) and
    for two interior points; the triangulation stays usable afterwards."""
    import torch

    import sdfoam_amd

    raw = np.ascontiguousarray(_gpu_sets()["gaussian"](), dtype=np.float32)
    tri = sdfoam_amd.Triangulation(torch.from_numpy(raw).to(dev))
    pts = raw[tri.permutation().view(torch.int32).cpu().numpy()]
    tets = _np(tri.tets()).reshape(-1, 4)
    adj = _np(tri.tet_adjacency()).reshape(-1, 4)
    on_hull = np.zeros(pts.shape[0], dtype=bool)
    for t, j in zip(*np.nonzero(adj == 0xFFFFFFFF)):
        on_hull[np.delete(tets[t], j)] = True
    pick = np.nonzero(on_hull if where == "hull" else ~on_hull)[0]
    a, b = int(pick[0]), int(pick[len(pick) // 2])
    moved = pts.copy()
    moved[a] = moved[b]
    with pytest.raises(sdfoam_amd.TriangulationFailedError, match="duplicate points"):
        tri.rebuild(torch.from_numpy(moved).to(dev), incremental=True)
    assert tri.rebuild(torch.from_numpy(pts).to(dev), incremental=True) is False
    assert tri.last_method == "gpu"


def test_triangulation_methods_agree(dev):
    import torch

    import sdfoam_amd

    w = scene(2)
    pts = torch.from_numpy(w.points).to(dev)
    a = sdfoam_amd.Triangulation(pts)
    b = sdfoam_amd.Triangulation(pts, method="qhull")
    assert a.last_method == "gpu" and b.last_method == "qhull"
    assert a.last_stats["open"] < 0.05 * w.points.shape[0]
    for k in ("tets", "tet_adjacency", "vert_to_tet", "point_adjacency", "point_adjacency_offsets"):
        assert torch.equal(getattr(a, k)().view(torch.int32), getattr(b, k)().view(torch.int32)), k
    with pytest.raises(ValueError, match="unknown triangulation method"):
        sdfoam_amd.Triangulation(pts, method="cgal")


def test_gpu_delaunay_small_and_degenerate_inputs(dev):
    """32 points (the minimum) on the GPU path; a cubic lattice, where every
    cell is cospherical with its neighbours, still gives a Delaunay
    tetrahedralisation (by whichever path); coplanar points fail as Qhull
    does."""
    import torch
    from scipy.spatial import ConvexHull

    import sdfoam_amd
    from test_delaunay_cells import assert_delaunay

    rng = np.random.default_rng(32)
    pts = rng.normal(size=(32, 3)).astype(np.float32)
    tri = sdfoam_amd.Triangulation(torch.from_numpy(pts).to(dev))
    assert tri.last_method == "gpu"
    perm = tri.permutation().to(torch.long).cpu().numpy()
    tets = _np(tri.tets()).reshape(-1, 4).astype(np.int64)
    assert_delaunay(pts[perm], tets, ConvexHull(pts.astype(np.float64)).volume)
    g = np.arange(8, dtype=np.float32)
    lattice = np.stack(np.meshgrid(g, g, g, indexing="ij"), axis=-1).reshape(-1, 3)
    tri = sdfoam_amd.Triangulation(torch.from_numpy(lattice).to(dev))
    assert tri.last_method in ("gpu", "qhull")
    perm = tri.permutation().to(torch.long).cpu().numpy()
    tets = _np(tri.tets()).reshape(-1, 4).astype(np.int64)
    p = lattice[perm].astype(np.float64)
    a, b, c, d = (p[tets[:, k]] for k in range(4))
    vol = np.einsum("ij,ij->i", np.cross(b - a, c - a), d - a) / 6.0
    # Qhull's triangulated output may hold flat tets on cospherical groups;
    # the rest must tile the cube and have empty circumspheres
    assert (vol >= 0).all() and abs(vol.sum() - 7.0 ** 3) < 1e-9
    solid = vol > 0
    assert_delaunay(lattice[perm], tets[solid], 7.0 ** 3)
    flat = rng.normal(size=(100, 3)).astype(np.float32)
    flat[:, 2] = 0.0
    with pytest.raises(sdfoam_amd.TriangulationFailedError):
        sdfoam_amd.Triangulation(torch.from_numpy(flat).to(dev))


def test_gpu_delaunay_far_from_the_origin(dev):
    """Points at 1000 + [0, 1)^3: the GPU tetrahedralisation works relative to
    each cell's point and stays exactly Delaunay, where Qhull's lifted
    coordinates lose precision (the two may differ here); every GPU tet has
    an empty circumsphere and together they tile the hull."""
    import torch
    from scipy.spatial import ConvexHull

    from sdfoam_amd.triangulation import gpu_tetrahedra
    from test_delaunay_cells import assert_delaunay

    rng = np.random.default_rng(99)
    pts = np.unique((1000.0 + rng.random((20000, 3))).astype(np.float32), axis=0)
    tets, nbr, stats = gpu_tetrahedra(torch.from_numpy(pts).to(dev))
    t = tets.cpu().numpy()
    assert np.array_equal(nbr.cpu().numpy(), _face_neighbors(t))
    # volumes relative to the cloud's corner, in double
    local = (pts.astype(np.float64) - 1000.0).astype(np.float64)
    assert_delaunay(local, t, ConvexHull(local).volume)


@pytest.mark.parametrize("name", ["gaussian", "shell", "C2"])
def test_open_points_by_qhull_when_the_gpu_cannot(dev, name, monkeypatch):
    """The open points' fallback: with the exhaustive certification made to
    give up, Qhull triangulates them (as when a cell is undecided or a face
    without a neighbour is off the hull), and the tetrahedra are the same."""
    import torch

    from sdfoam_amd import triangulation as tr

    pts = np.ascontiguousarray(_gpu_sets()[name](), dtype=np.float32)
    pd = torch.from_numpy(pts).to(dev)
    tets_gpu, _, st_gpu = tr.gpu_tetrahedra(pd)
    monkeypatch.setattr(tr, "_open_candidates_gpu", lambda *a, **k: None)
    tets_q, _, st_q = tr.gpu_tetrahedra(pd)
    assert st_gpu["open_points_qhull"] == 0 and st_q["open_points_qhull"] > 0, (st_gpu, st_q)

    def canon(t):
        t = np.sort(t.cpu().numpy(), axis=1)
        return t[np.lexsort(t[:, ::-1].T)]

    assert np.array_equal(canon(tets_gpu), canon(tets_q))
