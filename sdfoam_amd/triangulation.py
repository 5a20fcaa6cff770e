"""The adjacency producer: ``Triangulation``, ``TriangulationFailedError`` and
``farthest_neighbor`` with the reference's interface
(torch_bindings/triangulation_bindings.cpp:11-115, 183-237;
src/delaunay/delaunay.h:9-44).

``Triangulation(points)`` sorts the points into the reference's
``sort_points`` order (``permutation()``: sorted = points[perm]) and
triangulates them; ``rebuild(points, incremental)`` re-triangulates, sorting
again unless ``incremental`` and the point count is unchanged, and returns
whether it sorted (the caller then permutes its arrays).  An incremental
rebuild starts from the previous tetrahedra: those whose circumspheres stay
empty are kept, and only the points of the others are certified again.  Outputs are CUDA
uint32 tensors indexing the sorted points:

* ``tets()`` [T, 4], ordered by their sorted vertex sets, each listing its
  vertices ascending except that the last two are swapped where that makes
  it positively oriented (det[b - a, c - a, d - a] > 0);
* ``tet_adjacency()`` [T, 4]: across the face opposite vertex j, 4 k + m for
  neighbour tet k and its face m, or 0xffffffff on the hull;
* ``vert_to_tet()`` [N]: the lowest tet index holding each point;
* ``point_adjacency()`` / ``point_adjacency_offsets()``: the Delaunay edges
  as CSR with ascending rows (src/delaunay/delaunay.cu:146-226).

The Delaunay tetrahedralisation is computed on the GPU by certified Voronoi
cells (``gpu_tetrahedra``), with Qhull (scipy) on the host for the few points
whose cells the GPU leaves open; the reference grows it on the GPU by
insertion with exact predicates.  For points in general position both give
the same unique triangulation.  ``method="qhull"`` runs Qhull on every point.
The point order (``sort_points``), the tables derived from the tetrahedra and
``farthest_neighbor`` run in libsdfoam_hip.so; ``host_tables`` is the numpy
statement of the same tables (the check of the device path).
"""

from __future__ import annotations

import ctypes as C
import time

import numpy as np
import torch

from . import _lib
from ._lib import check, ptr

_NONE = np.uint32(0xFFFFFFFF)


class TriangulationFailedError(RuntimeError):
    """src/delaunay/delaunay.h:9-13."""


def _u32_cuda(a: np.ndarray, device) -> torch.Tensor:
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return torch.from_numpy(a.view(np.int32)).to(device).view(torch.uint32)


def qhull_tetrahedra(points: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Delaunay tetrahedra of float32 points [N, 3] (Qhull, in double):
    (simplices [T, 4] int32, neighbors [T, 4] int32, -1 on the hull).  The
    points are centred on their bounding box first: the triangulation does
    not change, and Qhull's lifted coordinates (|x|^2) keep their precision
    for clouds far from the origin."""
    from scipy.spatial import Delaunay
    from scipy.spatial import QhullError

    p = np.asarray(points, dtype=np.float64)
    if p.shape[0] > 0:
        p = p - 0.5 * (p.min(axis=0) + p.max(axis=0))
    try:
        tri = Delaunay(p)
    except QhullError as e:
        raise TriangulationFailedError(f"Qhull failed: {str(e).splitlines()[0]}") from None
    return (np.ascontiguousarray(tri.simplices, dtype=np.int32),
            np.ascontiguousarray(tri.neighbors, dtype=np.int32))


def triangulate_host(points: np.ndarray) -> dict:
    """Delaunay tetrahedralisation of float32 points [N, 3] (already in the
    triangulation's point order) and its derived tables, as numpy uint32."""
    simplices, neighbors = qhull_tetrahedra(points)
    return host_tables(points, simplices, neighbors)


def host_tables(points: np.ndarray, simplices: np.ndarray, neighbors: np.ndarray) -> dict:
    """The tables of sdf_delaunay_tables in numpy (the statement the device
    path is checked against)."""
    p64 = np.asarray(points, dtype=np.float64)
    n = p64.shape[0]
    s = np.asarray(simplices, dtype=np.int64).copy()
    nb = np.asarray(neighbors, dtype=np.int64).copy()
    # canonical vertex order: ascending (neighbour j stays opposite vertex j),
    # then positive orientation by swapping the last two
    o = np.argsort(s, axis=1, kind="stable")
    s = np.take_along_axis(s, o, axis=1)
    nb = np.take_along_axis(nb, o, axis=1)
    a, b, c, d = (p64[s[:, k]] for k in range(4))
    x = np.cross(b - a, c - a)
    w = d - a
    vol = (x[:, 0] * w[:, 0] + x[:, 1] * w[:, 1]) + x[:, 2] * w[:, 2]
    neg = vol < 0
    s[neg, 2], s[neg, 3] = s[neg, 3].copy(), s[neg, 2].copy()
    nb[neg, 2], nb[neg, 3] = nb[neg, 3].copy(), nb[neg, 2].copy()
    # order tets by their sorted vertex sets
    key = np.sort(s, axis=1)
    order = np.lexsort(key[:, ::-1].T)
    rank = np.empty_like(order)
    rank[order] = np.arange(order.size)
    s = s[order]
    nb = nb[order]
    nb = np.where(nb >= 0, rank[np.maximum(nb, 0)], -1)
    T = s.shape[0]
    # face of the neighbour that is shared: the neighbour's vertex not in this tet
    adj_t = np.full((T, 4), _NONE, dtype=np.uint32)
    ii, jj = np.nonzero(nb >= 0)
    kk = nb[ii, jj]
    other = s[kk]  # [M, 4]
    mine = s[ii]
    missing = ~(other[:, :, None] == mine[:, None, :]).any(axis=2)  # [M, 4]
    m = np.argmax(missing, axis=1)
    adj_t[ii, jj] = (4 * kk + m).astype(np.uint32)
    # lowest tet holding each vertex
    v2t = np.full(n, np.iinfo(np.int64).max, dtype=np.int64)
    np.minimum.at(v2t, s.ravel(), np.repeat(np.arange(T), 4))
    v2t = np.where(v2t == np.iinfo(np.int64).max, 0xFFFFFFFF, v2t).astype(np.uint32)
    # CSR point adjacency: unique edges, both directions, ascending rows
    pairs = np.concatenate([s[:, [0, 1]], s[:, [0, 2]], s[:, [0, 3]], s[:, [1, 2]],
                            s[:, [1, 3]], s[:, [2, 3]]])
    lo = np.minimum(pairs[:, 0], pairs[:, 1])
    hi = np.maximum(pairs[:, 0], pairs[:, 1])
    ek = np.unique((lo << 32) | hi)
    lo, hi = ek >> 32, ek & 0xFFFFFFFF
    both = np.concatenate([(lo << 32) | hi, (hi << 32) | lo])
    both.sort()
    rows = both >> 32
    adj = (both & 0xFFFFFFFF).astype(np.uint32)
    offs = np.zeros(n + 1, dtype=np.uint32)
    np.cumsum(np.bincount(rows, minlength=n), out=offs[1:])
    return {"tets": s.astype(np.uint32), "tet_adjacency": adj_t, "vert_to_tet": v2t,
            "point_adjacency": adj, "point_adjacency_offsets": offs}


def sort_points(points: torch.Tensor) -> torch.Tensor:
    """The reference's sort_points order of CUDA float32 points [N, 3], as a
    uint32 permutation (sorted = points[perm]) on the points' device."""
    pts = points.contiguous()
    n = pts.numel() // 3
    perm = torch.empty(n, dtype=torch.int32, device=pts.device)
    if n == 0:
        return perm.view(torch.uint32)
    L = _lib.lib()
    nbytes = int(L.sdf_sort_points_scratch_bytes(n))
    if nbytes == 0:
        raise RuntimeError("sdf_sort_points_scratch_bytes failed")
    scratch = torch.empty(nbytes + 256, dtype=torch.uint8, device=pts.device)
    with torch.cuda.device(pts.device):
        check(L.sdf_sort_points(ptr(pts), n, ptr(perm), (scratch.data_ptr() + 255) & ~255,
                                nbytes, _lib.stream_handle(pts.device)))
    return perm.view(torch.uint32)


def _aligned(nbytes: int, device) -> tuple[torch.Tensor, int]:
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    return buf, (buf.data_ptr() + 255) & ~255


class _Undecided(RuntimeError):
    """The GPU tetrahedralisation met a sign it could not decide."""


def _certify(L, pts: torch.Tensor, gptr: int, gbytes: int, stream, query=None,
             exhaustive: bool = False):
    """sdf_delaunay_certify over CUDA float32 points [n, 3], or with `query`
    (int32 ids) sdf_delaunay_certify_points over those on the grid of an
    sdf_delaunay_check call, or with `exhaustive` sdf_delaunay_certify_exhaustive
    (a small set: hull cells' finite vertices reported too): (reports [nr, 4]
    int32 rows (point, a, b, c), open points [nu] int32 in index order,
    counts).  Raises _Undecided where the GPU cannot decide."""
    dev = pts.device
    n = pts.numel() // 3
    nq = n if query is None else int(query.numel())
    open_pts = torch.empty(max(nq, 1), dtype=torch.int32, device=dev)
    counts = (C.c_uint64 * 5)()
    # report rows: ~27 per certified cell over a whole point set (the mean
    # tetrahedra per vertex); more per cell among the dirty points of an
    # incremental rebuild, where a second pass would double the time
    cap = (28 if query is None else 40) * nq + 4096
    for _ in range(2):
        reports = torch.empty((cap, 4), dtype=torch.int32, device=dev)
        if exhaustive:
            rc = L.sdf_delaunay_certify_exhaustive(ptr(pts), n, ptr(reports), cap, ptr(open_pts),
                                                   counts, gptr, gbytes, stream)
        elif query is None:
            rc = L.sdf_delaunay_certify(ptr(pts), n, ptr(reports), cap, ptr(open_pts), counts,
                                        gptr, gbytes, stream)
        else:
            rc = L.sdf_delaunay_certify_points(ptr(pts), n, ptr(query), nq, ptr(reports), cap,
                                               ptr(open_pts), counts, gptr, gbytes, stream)
        if rc == _lib.SDF_E_INVALID:
            # no volume or non-finite points: Qhull on every point decides
            raise _Undecided(L.sdf_last_error().decode())
        check(rc)
        if counts[0] <= cap:
            break
        cap = int(counts[0])
    if counts[4]:
        raise TriangulationFailedError("duplicate points found")
    nr, nu = int(counts[0]), int(counts[1])
    return reports[:nr], torch.sort(open_pts[:nu])[0], counts


# The open points are certified once more among themselves when there are at
# least 256 of them, and that level's stars are used when it leaves at most
# this share of them open (at C3 it halves them in a few ms; a further level
# would remove another ~12% only, for about the same time again).
_LEVEL_SHRINK = 0.7


# The most open points the exhaustive certification takes (C3 leaves 7,935
# open, C4 11,125; past some 60k, Qhull on those left open after a grid
# level is faster).
_EXHAUSTIVE_MAX = 1 << 16


class _OpenRetry(RuntimeError):
    """The open points' tetrahedra from the GPU left a face without a
    neighbour off the convex hull (a circumcentre beyond the exhaustive
    certification's box, or a fault): they are made again with Qhull."""


def _open_candidates_gpu(L, pts: torch.Tensor, U: torch.Tensor, stream, stats: dict):
    """Candidates [m, 4] for the Delaunay tetrahedra with four open vertices
    from sdf_delaunay_certify_exhaustive over the open points U: every
    Delaunay tetrahedron of the whole set with four vertices in U is one of
    U's own (its circumsphere holds no point at all), which the exhaustive
    certification reports from each of its vertices' cells, hull cells
    included, as long as its circumcentre lies within the 1e8-extent box.
    None when a cell is undecided (Qhull then decides), and for more than
    _EXHAUSTIVE_MAX open points: a cell that the grid search among them
    leaves open is clipped by every one of them, so the pass grows as the
    square of their number (a plane of 300k points leaves 65.8k of them open:
    the rebuild takes 0.78 s that way, 0.59 s with Qhull)."""
    if U.numel() < 32 or U.numel() > _EXHAUSTIVE_MAX:
        return None
    t = time.perf_counter()
    gb = int(L.sdf_delaunay_certify_scratch_bytes(U.numel()))
    if gb == 0:
        return None
    gbuf, gp = _aligned(gb, pts.device)
    try:
        rep, U2, counts = _certify(L, pts[U.long()].contiguous(), gp, gb, stream, exhaustive=True)
    except _Undecided:
        return None
    finally:
        del gbuf
    # a cell over the fixed capacity reports nothing, but each of its
    # tetrahedra comes from its other vertices' cells as well (one whose four
    # vertices all overflow leaves a hole, which the hull check finds); an
    # undecided sign means cospherical points, which Qhull decides
    if counts[2] or rep.shape[0] == 0:
        return None
    cand = U[rep.long()]
    # a tetrahedron comes once from each of its vertices
    cand = torch.unique(torch.sort(cand, dim=1)[0], dim=0)
    stats["open_levels"] = [int(U2.numel())]
    stats["open_points_qhull"] = 0
    stats["open_levels_s"] = time.perf_counter() - t
    stats["open_qhull_s"] = 0.0
    return cand.to(torch.int32).contiguous()


def _hull_is_convex(pts: torch.Tensor, tets: torch.Tensor, nbr: torch.Tensor, T: int,
                    U: torch.Tensor) -> bool:
    """Whether every face of the merged tetrahedra without a neighbour is a
    facet of the convex hull: every point of U (the open points, among which
    are the hull's vertices and the far vertex of any tetrahedron missing
    behind such a face) lies strictly on the face's inner side, the sign of
    each float64 orientation determinant decided against a bound of 1e-14
    times its permanent (Shewchuk's static bound for orient3d is 7.8e-16).
    Then the merged tetrahedra, all Delaunay, cover the hull: no face
    without a neighbour lies inside it."""
    dev = pts.device
    nb = nbr[:T]
    tt, jj = torch.nonzero(nb < 0, as_tuple=True)
    F = int(tt.numel())
    if F == 0:
        return False
    tv = tets[:T][tt].long()
    keep = torch.arange(4, device=dev)[None, :] != jj[:, None]
    fv = tv[keep].view(F, 3)
    far = tv[torch.arange(F, device=dev), jj]
    P = pts.double()
    X = P[U.long()]
    uid = U.long()
    # faces in chunks of up to 2^23 face-point pairs; one host read at the end
    step = max(1, (1 << 23) // max(1, int(uid.numel())))
    ok = torch.ones((), dtype=torch.bool, device=dev)
    for f0 in range(0, F, step):
        f1 = min(F, f0 + step)
        a, b, c, d = P[fv[f0:f1, 0]], P[fv[f0:f1, 1]], P[fv[f0:f1, 2]], P[far[f0:f1]]
        e1, e2 = b - a, c - a
        n = torch.cross(e1, e2, dim=1)
        na = torch.stack([(e1[:, 1] * e2[:, 2]).abs() + (e1[:, 2] * e2[:, 1]).abs(),
                          (e1[:, 2] * e2[:, 0]).abs() + (e1[:, 0] * e2[:, 2]).abs(),
                          (e1[:, 0] * e2[:, 1]).abs() + (e1[:, 1] * e2[:, 0]).abs()], dim=1)
        dd = d - a
        sd = (dd * n).sum(1)
        ok &= (sd.abs() > 1e-14 * (dd.abs() * na).sum(1)).all()
        sx = torch.zeros((f1 - f0, X.shape[0]), dtype=torch.float64, device=dev)
        bx = torch.zeros_like(sx)
        for k in range(3):
            xk = X[None, :, k] - a[:, k:k + 1]
            sx += xk * n[:, k:k + 1]
            bx += xk.abs() * na[:, k:k + 1]
        on_face = (uid[None, :] == fv[f0:f1, 0:1]) | (uid[None, :] == fv[f0:f1, 1:2]) | \
            (uid[None, :] == fv[f0:f1, 2:3])
        inner = (torch.sign(sx) == torch.sign(sd)[:, None]) & (sx.abs() > 1e-14 * bx)
        ok &= (inner | on_face).all()
    return bool(ok.item())


def _open_candidates(L, pts: torch.Tensor, U: torch.Tensor, stream, stats: dict):
    """Candidate tetrahedra [m, 4] (global indices, int32 on the points'
    device) for the Delaunay tetrahedra of `pts` whose four vertices are all
    in the open set U, and the hull's face count.  Such a tetrahedron's
    circumsphere holds no point of U either, so it is one of U's own Delaunay
    tetrahedra: of those, the ones with a vertex whose cell certifies among U
    alone come from that certification, and the rest have four vertices that
    stay open there and come from Qhull on those on the host.  All of these
    are candidates (the merge keeps a candidate only if no point of `pts`
    lies in its circumsphere), and the hull points stay open, so Qhull's
    hull is the whole set's."""
    parts = []
    t = time.perf_counter()
    gb = int(L.sdf_delaunay_certify_scratch_bytes(U.numel())) if U.numel() >= 256 else 0
    if gb:
        gbuf, gp = _aligned(gb, pts.device)
        try:
            rep, U2, _ = _certify(L, pts[U.long()].contiguous(), gp, gb, stream)
        except _Undecided:
            rep = None
        # a TriangulationFailedError (coincident open points) propagates: the
        # points coincide in the whole set too
        del gbuf
        if rep is not None and U2.numel() <= _LEVEL_SHRINK * U.numel():
            if rep.shape[0]:
                parts.append(U[rep.long()])
            stats["open_levels"] = [int(U2.numel())]
            U = U[U2.long()]
    t_levels = time.perf_counter()
    u_np = U.cpu().numpy()
    try:
        simplices, nbr_u = qhull_tetrahedra(pts[U.long()].cpu().numpy())
    except TriangulationFailedError as e:
        # a degenerate open subset: Qhull on every point decides
        raise _Undecided(str(e)) from None
    t_qhull = time.perf_counter()
    stats["open_points_qhull"] = int(u_np.size)
    q = torch.from_numpy(np.ascontiguousarray(u_np[simplices], dtype=np.int32)).to(pts.device)
    if parts:
        # a tetrahedron comes once from each of its certified vertices and
        # possibly from Qhull as well
        cand = torch.cat(parts + [q])
        cand = torch.unique(torch.sort(cand, dim=1)[0], dim=0)
    else:
        cand = q
    stats["open_levels_s"] = t_levels - t
    stats["open_qhull_s"] = t_qhull - t_levels
    return cand.to(torch.int32).contiguous(), int((nbr_u < 0).sum())


def has_coincident_points(pts: torch.Tensor) -> bool:
    """Whether two of the CUDA float32 points [n, 3] are equal (+0 equals
    -0): the coordinates' bit patterns sorted lexicographically by three
    stable sorts, then neighbouring rows compared.  Exact, ~1 ms at 1M
    points."""
    if pts.shape[0] < 2:
        return False
    b = (pts + 0.0).view(torch.int32)  # -0 + 0 = +0
    order = torch.sort(b[:, 2], stable=True)[1]
    order = order[torch.sort(b[order, 1], stable=True)[1]]
    order = order[torch.sort(b[order, 0], stable=True)[1]]
    s = b[order]
    return bool((s[1:] == s[:-1]).all(dim=1).any().item())


def _merge(L, pts: torch.Tensor, gptr: int, gbytes: int, reports, cand, verified,
           hull_faces, stream, tcap: int | None = None, open_ids=None):
    """sdf_delaunay_merge (sdf_delaunay_merge_verified with `verified`
    rows): (tets, neighbors, T); raises _Undecided when a candidate is
    undecided or the union is inconsistent (Qhull on every point decides).
    `tcap`: the tets to make room for (a second merge runs if more come).
    hull_faces None (the candidates came from the GPU, not Qhull): instead
    of Qhull's hull face count, every face without a neighbour must be a
    convex-hull facet (_hull_is_convex over `open_ids`), else _OpenRetry."""
    dev = pts.device
    n = pts.numel() // 3
    nr, m = int(reports.shape[0]), int(cand.shape[0])
    nv = 0 if verified is None else int(verified.shape[0])
    result = (C.c_uint64 * 4)()
    if tcap is None:
        # every certified vertex of a tetrahedron reports it (~4 rows per tet)
        tcap = nr // 3 + m + nv + 4096
    for _ in range(2):
        tets = torch.empty((tcap, 4), dtype=torch.int32, device=dev)
        nbr = torch.empty((tcap, 4), dtype=torch.int32, device=dev)
        mbytes = int(L.sdf_delaunay_merge_scratch_bytes(n, nr, m + nv, tcap))
        if mbytes == 0:
            raise RuntimeError("sdf_delaunay_merge_scratch_bytes failed")
        mbuf, mptr = _aligned(mbytes, dev)
        if verified is None:
            rc = L.sdf_delaunay_merge(ptr(pts), n, gptr, gbytes, ptr(reports), nr, ptr(cand), m,
                                      ptr(tets), ptr(nbr), tcap, result, mptr, mbytes, stream)
        else:
            rc = L.sdf_delaunay_merge_verified(ptr(pts), n, gptr, gbytes, ptr(reports), nr,
                                               ptr(cand), m, ptr(verified), nv, ptr(tets),
                                               ptr(nbr), tcap, result, mptr, mbytes, stream)
        if rc == _lib.SDF_E_INVALID and result[0] > tcap and result[2] == 0:
            tcap = int(result[0])
            continue
        if rc == _lib.SDF_E_INVALID:
            if hull_faces is None:
                raise _OpenRetry(L.sdf_last_error().decode())
            raise _Undecided(L.sdf_last_error().decode())
        check(rc)
        break
    else:
        raise _Undecided("tets did not fit the merge's capacity")
    T = int(result[0])
    if hull_faces is None:
        if not _hull_is_convex(pts, tets, nbr, T, open_ids):
            raise _OpenRetry("a face without a neighbour is not on the convex hull")
    elif int(result[1]) != hull_faces:
        raise _Undecided(f"{int(result[1])} faces without a neighbour, the hull has {hull_faces}")
    return tets, nbr, T


def _open_and_merge(L, pts, U, gptr, gbytes, reports, verified, stream, stats, tcap=None):
    """The open points' candidates (from the GPU's exhaustive certification,
    else Qhull) and the merge: (tets, neighbors, T, candidates)."""
    t = time.perf_counter()
    cand = _open_candidates_gpu(L, pts, U, stream, stats)
    t_open = time.perf_counter()
    if cand is not None:
        try:
            tets, nbr, T = _merge(L, pts, gptr, gbytes, reports, cand, verified, None, stream,
                                  tcap, open_ids=U)
            stats["open_points_qhull_s"] = t_open - t
            stats["merge_s"] = time.perf_counter() - t_open
            return tets, nbr, T, cand
        except _OpenRetry as e:
            stats["open_gpu_retry"] = str(e)
    t = time.perf_counter()
    cand, hull_faces = _open_candidates(L, pts, U, stream, stats)
    t_open = time.perf_counter()
    tets, nbr, T = _merge(L, pts, gptr, gbytes, reports, cand, verified, hull_faces, stream, tcap)
    stats["open_points_qhull_s"] = t_open - t
    stats["merge_s"] = time.perf_counter() - t_open
    return tets, nbr, T, cand


def gpu_tetrahedra(points: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, dict]:
    """Delaunay tetrahedra of CUDA float32 points [N, 3] by certified
    Voronoi cells (sdf_delaunay_certify / sdf_delaunay_merge): the points
    whose cells the GPU cannot certify (the hull and the layer under it) are
    certified again among themselves, exhaustively (hull cells' finite
    vertices included); their tetrahedra are kept where no point lies in the
    circumsphere, and the hull's faces are checked convex.  Where that
    certification cannot decide or the check fails, the open points'
    tetrahedra come from Qhull on the host instead.  Returns (tets [T, 4]
    int32, neighbors [T, 4] int32, -1 on the hull, stats) on the points'
    device."""
    pts = points.contiguous()
    dev = pts.device
    n = pts.numel() // 3
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    gbytes = int(L.sdf_delaunay_certify_scratch_bytes(n))
    if gbytes == 0:
        raise RuntimeError("sdf_delaunay_certify_scratch_bytes failed")
    gbuf, gptr = _aligned(gbytes, dev)
    stats = {}
    t0 = time.perf_counter()
    with torch.cuda.device(dev):
        reports, U, counts = _certify(L, pts, gptr, gbytes, stream)
        nr, nu = int(reports.shape[0]), int(U.numel())
        t1 = time.perf_counter()
        tets, nbr, T, cand = _open_and_merge(L, pts, U, gptr, gbytes, reports, None, stream,
                                             stats)
    stats.update({"open": nu, "reports": nr, "candidates": int(cand.shape[0]), "tets": T,
                  "undecided_cells": int(counts[2]), "overflow_cells": int(counts[3]),
                  "certify_s": t1 - t0, "open_ids": U})
    return tets[:T], nbr[:T], stats


# An incremental rebuild re-certifies the dirty points only; past this share
# of dirty points the full rebuild is used instead (at C3's 1M points the two
# take about as long at ~40% dirty: the check costs ~30 ms, certifying the
# dirty points ~40-50 ms per 100k-300k of them).
_INCREMENTAL_MAX_DIRTY = 0.4


def gpu_tetrahedra_incremental(points: torch.Tensor, tets_old: torch.Tensor,
                               nbr_old: torch.Tensor, open_old: torch.Tensor | None = None):
    """The Delaunay tetrahedra of moved CUDA float32 points [N, 3] from the
    previous tetrahedralisation of the same points (tets_old, nbr_old: int32
    [T, 4] on the points' device, -1 on the hull), in place of
    delete_delaunay_violations and the regrowth from its frontier
    (src/delaunay/delete_violations.cu:7-178, src/delaunay/delaunay.cu:
    288-345).  sdf_delaunay_check keeps the old tetrahedra whose circumsphere
    is still empty and marks the vertices of the others, and of the hull
    faces, dirty; the dirty points alone are certified (the open ones go
    through the open points' path of the full rebuild), and the merge takes
    their reports and candidates and the kept old tetrahedra with a clean
    vertex and no certified one.  A Delaunay tetrahedron of the moved points
    with a clean vertex v is one of v's old ones (those are all kept, so they
    still fill a neighbourhood of v, and Delaunay tetrahedra do not
    overlap); all other Delaunay tetrahedra have four dirty vertices.
    `open_old` (int32 ids on the device, optional): the points the previous
    tetrahedralisation left open; those of them that are dirty join the open
    points without a certification, like the old hull's vertices (their
    cells, next to the hull or to large empty regions, rarely certify and
    take the longest to try: ~20-40 ms for one at C3, against ~0.3 ms for
    the median dirty point).  Any split of the dirty points into certified
    and open ones gives the same tetrahedra.
    Returns (tets, neighbors, stats), stats["open_ids"] the points left open;
    raises _Undecided like gpu_tetrahedra,
    and when more than _INCREMENTAL_MAX_DIRTY of the points are dirty (the
    caller then rebuilds in full)."""
    pts = points.contiguous()
    dev = pts.device
    n = pts.numel() // 3
    T_old = int(tets_old.shape[0])
    L = _lib.lib()
    stream = _lib.stream_handle(dev)
    gbytes = int(L.sdf_delaunay_certify_scratch_bytes(n))
    if gbytes == 0:
        raise RuntimeError("sdf_delaunay_certify_scratch_bytes failed")
    gbuf, gptr = _aligned(gbytes, dev)
    tets_old = tets_old.to(dev, torch.int32).contiguous()
    nbr_old = nbr_old.to(dev, torch.int32).contiguous()
    keep = torch.empty(max(T_old, 1), dtype=torch.int32, device=dev)
    dirty = torch.empty(n, dtype=torch.int32, device=dev)
    stats = {"incremental": True}
    t0 = time.perf_counter()
    with torch.cuda.device(dev):
        rc = L.sdf_delaunay_check(ptr(pts), n, ptr(tets_old), ptr(nbr_old), T_old, ptr(keep),
                                  ptr(dirty), gptr, gbytes, stream)
        if rc == _lib.SDF_E_INVALID:
            raise _Undecided(L.sdf_last_error().decode())
        check(rc)
        # the certification finds a point equal to the one it certifies; the
        # points it does not certify here (clean ones, the old hull's) are
        # checked for coincidence over the whole set, as the reference's
        # incremental rebuild does (src/delaunay/delaunay.cu:291-294)
        if has_coincident_points(pts):
            raise TriangulationFailedError("duplicate points found")
        D = torch.nonzero(dirty).view(-1).to(torch.int32)
        nd = int(D.numel())
        stats.update({"dirty": nd, "kept_old": int(keep[:T_old].sum().item())})
        if nd > _INCREMENTAL_MAX_DIRTY * n:
            raise _Undecided(f"{nd} of {n} points dirty")
        t1 = time.perf_counter()
        # the old hull's vertices (2) go to the open points uncertified: their
        # cells are unbounded, so certifying them would only list them as
        # open (and if one moved inside, its tetrahedra still come from the
        # open points' candidates, the reports and the kept ones); so do the
        # dirty points the previous tetrahedralisation left open
        direct = torch.nonzero(dirty == 2).view(-1).to(torch.int32)
        inner = torch.nonzero(dirty == 1).view(-1).to(torch.int32)
        if open_old is not None and open_old.numel():
            was_open = torch.zeros(n, dtype=torch.bool, device=dev)
            was_open[open_old.to(dev).long()] = True
            again = was_open[inner.long()]
            direct = torch.cat([direct, inner[again]])
            inner = inner[~again]
            stats["open_again"] = int(again.sum().item())
        reports, U, counts = _certify(L, pts, gptr, gbytes, stream, query=inner)
        U = torch.sort(torch.cat([U, direct]))[0]
        nr, nu = int(reports.shape[0]), int(U.numel())
        t2 = time.perf_counter()
        # 0 clean, 1 dirty and certified, 2 dirty and open
        state = torch.zeros(n, dtype=torch.int8, device=dev)
        if nd:
            state[D.long()] = 1
        if nu:
            state[U.long()] = 2
        sv = state[tets_old.long()]
        sel = (keep[:T_old] == 1) & (sv != 1).all(dim=1) & (sv == 0).any(dim=1)
        verified = tets_old[sel].contiguous()
        t_sel = time.perf_counter()
        # about as many tetrahedra as before (a tet may have one certified
        # vertex only, so the reports do not bound them as in a full rebuild),
        # plus the open points' candidates
        tets, nbr, T, cand = _open_and_merge(L, pts, U, gptr, gbytes, reports, verified, stream,
                                             stats, tcap=T_old + T_old // 16 + 8 * nu + 4096)
    stats.update({"open": nu, "reports": nr, "candidates": int(cand.shape[0]),
                  "verified": int(verified.shape[0]), "tets": T,
                  "undecided_cells": int(counts[2]), "overflow_cells": int(counts[3]),
                  "check_s": t1 - t0, "certify_s": t2 - t1, "select_s": t_sel - t2,
                  "open_ids": U})
    return tets[:T], nbr[:T], stats


def device_tables(points: torch.Tensor, simplices, neighbors) -> dict:
    """sdf_delaunay_tables over the tetrahedra of `points` (CUDA float32
    [N, 3]) as Qhull gives them (numpy or device int32 [T, 4]): the tables
    as uint32 tensors on the points' device."""
    pts = points.contiguous()
    dev = pts.device
    n = pts.numel() // 3
    T = int(simplices.shape[0])
    L = _lib.lib()
    if isinstance(simplices, torch.Tensor):
        tets_in = simplices.to(dev, torch.int32).contiguous()
        nbr_in = neighbors.to(dev, torch.int32).contiguous()
    else:
        tets_in = torch.from_numpy(np.ascontiguousarray(simplices, dtype=np.int32)).to(dev)
        nbr_in = torch.from_numpy(np.ascontiguousarray(neighbors, dtype=np.int32)).to(dev)
    tets = torch.empty((T, 4), dtype=torch.int32, device=dev)
    tet_adj = torch.empty((T, 4), dtype=torch.int32, device=dev)
    v2t = torch.empty(n, dtype=torch.int32, device=dev)
    offs = torch.empty(n + 1, dtype=torch.int32, device=dev)
    cap = int(L.sdf_delaunay_adjacency_capacity(n, T))
    adj = torch.empty(cap, dtype=torch.int32, device=dev)
    nbytes = int(L.sdf_delaunay_tables_scratch_bytes(n, T))
    if nbytes == 0:
        raise RuntimeError("sdf_delaunay_tables_scratch_bytes failed")
    scratch = torch.empty(nbytes + 256, dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        check(L.sdf_delaunay_tables(ptr(pts), n, ptr(tets_in), ptr(nbr_in), T, ptr(tets),
                                    ptr(tet_adj), ptr(v2t), ptr(offs), ptr(adj), cap,
                                    (scratch.data_ptr() + 255) & ~255, nbytes,
                                    _lib.stream_handle(dev)))
    num_adj = int(offs[n].item())  # the call synchronised the stream
    return {"tets": tets.view(torch.uint32), "tet_adjacency": tet_adj.view(torch.uint32),
            "vert_to_tet": v2t.view(torch.uint32),
            "point_adjacency": adj[:num_adj].clone().view(torch.uint32),
            "point_adjacency_offsets": offs.view(torch.uint32)}


def _check_points(points: torch.Tensor) -> None:
    if points.size(-1) != 3:
        raise RuntimeError("points must have 3 as the last dimension")
    if points.device.type != "cuda":
        raise RuntimeError("points must be on CUDA device")
    if points.dtype != torch.float32:
        raise RuntimeError("points must have float32 dtype")


class Triangulation:
    """method "gpu": certified Voronoi cells on the GPU with Qhull on the few
    open points (falls back to "qhull" when a sign is undecided); method
    "qhull": Qhull on every point.  Both give the same tetrahedralisation for
    points in general position; ``last_method`` says which one ran."""

    def __init__(self, points: torch.Tensor, method: str = "gpu"):
        _check_points(points)
        if method not in ("gpu", "qhull"):
            raise ValueError(f"unknown triangulation method {method!r}")
        self.method = method
        self.last_method = None
        self.last_stats = None
        self._num_points = 0
        self._perm_t = None
        self._tets_prev = None  # the last tetrahedra (int32 [T, 4] on the device)
        self._nbr_prev = None
        self._open_prev = None  # the points they left open (int32 ids), if from the GPU
        self.rebuild(points, incremental=False)

    def rebuild(self, points: torch.Tensor, incremental: bool = False) -> bool:
        """src/delaunay/delaunay.cu:260-349 (rebuild)."""
        _check_points(points)
        n = points.numel() // 3
        if n < 32:
            raise RuntimeError("Delaunay triangulation does not support less than 32 points")
        pts_dev = points.detach().reshape(n, 3).contiguous()
        if incremental and n == self._num_points:
            sorted_now = False
        else:
            self._perm_t = sort_points(pts_dev)
            pts_dev = pts_dev[self._perm_t.view(torch.int32).long()]
            self._num_points = n
            sorted_now = True
        if self.method == "gpu":
            got = None
            why = None
            if not sorted_now and self._tets_prev is not None:
                try:
                    got = gpu_tetrahedra_incremental(pts_dev, self._tets_prev, self._nbr_prev,
                                                     self._open_prev)
                except _Undecided as e:
                    why = str(e)
            try:
                if got is None:
                    got = gpu_tetrahedra(pts_dev)
                    if why is not None:
                        got[2]["incremental_fallback"] = why
                simplices, neighbors, self.last_stats = got
                self.last_method = "gpu"
                self._keep(simplices, neighbors, self.last_stats["open_ids"])
                self._tables = device_tables(pts_dev, simplices, neighbors)
                return sorted_now
            except _Undecided:
                pass
        pts = pts_dev.cpu().numpy()
        if np.unique(pts, axis=0).shape[0] != n:
            raise TriangulationFailedError("duplicate points found")
        simplices, neighbors = qhull_tetrahedra(pts)
        self.last_method = "qhull"
        self.last_stats = None
        self._keep(simplices, neighbors)
        self._tables = device_tables(pts_dev, simplices, neighbors)
        return sorted_now

    def _keep(self, simplices, neighbors, open_ids=None) -> None:
        """The tetrahedra an incremental rebuild starts from, and the points
        the GPU tetrahedralisation left open (None after Qhull)."""
        dev = self._perm_t.device
        self._open_prev = open_ids
        if isinstance(simplices, torch.Tensor):
            self._tets_prev = simplices.to(dev, torch.int32).contiguous()
            self._nbr_prev = neighbors.to(dev, torch.int32).contiguous()
        else:
            self._tets_prev = torch.from_numpy(np.ascontiguousarray(simplices, np.int32)).to(dev)
            self._nbr_prev = torch.from_numpy(np.ascontiguousarray(neighbors, np.int32)).to(dev)

    def permutation(self) -> torch.Tensor:
        return self._perm_t

    def tets(self) -> torch.Tensor:
        return self._tables["tets"]

    def tet_adjacency(self) -> torch.Tensor:
        return self._tables["tet_adjacency"]

    def point_adjacency(self) -> torch.Tensor:
        return self._tables["point_adjacency"]

    def point_adjacency_offsets(self) -> torch.Tensor:
        return self._tables["point_adjacency_offsets"]

    def vert_to_tet(self) -> torch.Tensor:
        return self._tables["vert_to_tet"]


def farthest_neighbor(points: torch.Tensor, point_adjacency: torch.Tensor,
                      point_adjacency_offsets: torch.Tensor):
    """(indices uint32, cell_radius float32), shaped like points[..., 0]
    (torch_bindings/triangulation_bindings.cpp:183-214)."""
    pts = points.contiguous()
    adj = point_adjacency.contiguous()
    offs = point_adjacency_offsets.contiguous()
    if pts.device.type != "cuda":
        raise RuntimeError("points must be on CUDA device")
    n = pts.size(0)
    shape = tuple(pts.shape[:-1])
    indices = torch.zeros(shape, dtype=torch.uint32, device=pts.device)
    radius = torch.zeros(shape, dtype=torch.float32, device=pts.device)
    with torch.cuda.device(pts.device):
        check(_lib.lib().sdf_farthest_neighbor(ptr(pts), n, adj.numel(), ptr(adj), ptr(offs),
                                               ptr(indices), ptr(radius),
                                               _lib.stream_handle(pts.device)))
    return indices, radius
