"""Invariants and brute-force pins of the oracle on the random scene C1
(4104 points, Qhull adjacency, 64x64 rays).

* Visits form a path in the adjacency graph, never repeat a cell (cells are
  convex and the safe walk's t increases), and n <= max_intersections + 1.
* The transmittance is non-increasing, rgba.a = 1 - T and the weights sum to
  1 - T per ray (checked through the per-point contributions).
* The forward and backward walks of sdfoam mode are the same walk.
* Dense sampling along each ray with a brute-force nearest site per sample
  reproduces the walk's cell sequence (the Voronoi cells the ray crosses),
  away from slivers where the fp16-rounded planes move a crossing.
* nn equals the brute-force fp32 argmin; the AABB tree's nodes are the exact
  bounds of their points.
"""

import numpy as np
import pytest
from scipy.spatial import cKDTree

from conftest import scene


@pytest.fixture(scope="module")
def c1_fwd(oracle_lib):
    w = scene(1)
    f = oracle_lib.trace_forward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                 w.rays, w.extra["start"], w.quantiles, inv_s=w.inv_s, record=64,
                                 threads=4, point_visits=True)
    return w, f


def test_point_visits_count_the_steps(c1_fwd):
    """The oracle's per-point visit counts (the K of the contribution sums'
    tolerance) equal the occurrences of each point in the recorded visit
    sequences, and a point is visited iff its contribution is nonzero or a
    zero-weight step reached it."""
    w, f = c1_fwd
    R = w.num_rays
    steps = f.steps.reshape(R)
    mask = np.arange(64)[None, :] < steps[:, None]
    want = np.bincount(f.cells[mask], minlength=w.num_points)
    assert np.array_equal(f.point_visits, want)
    assert int(f.point_visits.sum()) == int(steps.sum())
    assert np.all(f.contribution.reshape(-1)[f.point_visits == 0] == 0.0)


def test_visits_are_paths(c1_fwd):
    w, f = c1_fwd
    R = w.num_rays
    steps = f.steps.reshape(R)
    assert steps.max() < 64
    rows = [set(w.adjacency[w.offsets[i]:w.offsets[i + 1]].tolist()) for i in range(w.num_points)]
    start = w.extra["start"].reshape(R)
    for r in range(R):
        cells = f.cells[r, : steps[r]].tolist()
        if steps[r]:
            assert cells[0] == start[r]
        assert len(set(cells)) == len(cells), "a cell visited twice"
        for a, b in zip(cells, cells[1:]):
            assert b in rows[a]
    n = f.num_intersections.reshape(R)
    assert np.all(n <= 1024 + 1) and np.all(n >= steps)


def test_transmittance_and_weights(c1_fwd):
    w, f = c1_fwd
    R = w.num_rays
    steps = f.steps.reshape(R)
    a = f.cell_alphas
    T_final = np.ones(R)
    wsum = np.zeros(R)
    for r in range(R):
        al = a[r, : steps[r]].astype(np.float64)
        assert np.all((al >= 0) & (al <= 1))
        T = np.concatenate([[1.0], np.cumprod(1 - al)])
        assert np.all(np.diff(T) <= 0)
        T_final[r] = T[-1]
        wsum[r] = np.sum(T[:-1] * al)
    rgba = f.rgba.reshape(R, 4).astype(np.float64)
    assert np.allclose(rgba[:, 3], 1 - T_final, atol=2e-6)
    assert np.allclose(wsum, 1 - T_final, atol=2e-6)
    # contributions: the per-point sums of the same weights
    assert abs(f.contribution.sum() - wsum.sum()) <= 1e-6 * R


def test_forward_backward_walks_agree(c1_fwd, oracle_lib):
    w, f = c1_fwd
    b = oracle_lib.trace_backward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                  w.rays, w.extra["start"], f.rgba, w.grad_rgba, w.quantiles,
                                  f.depth_indices, w.depth_grad, inv_s=w.inv_s, threads=4)
    assert np.array_equal(b.visit_hash, f.visit_hash)
    assert np.array_equal(b.steps, f.steps)


def test_dense_sampling_matches_walk(oracle_lib):
    """The walk's cells are the Voronoi cells the ray crosses.

    Rays start inside the point cloud (start cell = exact nearest site) and
    are compared while they stay inside [-0.95, 0.95]^3, where every crossing
    is at most a cell diameter from the sites that define its plane.  (Far
    outside the hull the walk runs through the unbounded cells of hull
    points, where the reference's fp16 offsets move a plane by up to
    2^-11 x |offset| x the distance to the sites -- that is the reference's
    own arithmetic, compared against the GPU bit for bit elsewhere.)"""
    w = scene(1)
    rng = np.random.default_rng(0)
    n_rays = 400
    o = rng.uniform(-0.5, 0.5, (n_rays, 3))
    d = rng.normal(size=(n_rays, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    rays = np.concatenate([o, d], axis=1).astype(np.float32)
    start = oracle_lib.nn(w.points, rays[:, :3])
    f = oracle_lib.trace_forward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                 rays, start, inv_s=1e-3, record=128)
    tree = cKDTree(w.points.astype(np.float64))
    o64 = rays[:, :3].astype(np.float64)
    d64 = rays[:, 3:].astype(np.float64)
    d64 /= np.linalg.norm(d64, axis=1, keepdims=True)
    sliver = 1e-3
    exact = robust = 0
    for r in range(n_rays):
        # t at which the ray leaves the box
        with np.errstate(divide="ignore"):
            tb = np.min(np.where(d64[r] > 0, (0.95 - o64[r]) / d64[r], (-0.95 - o64[r]) / d64[r]))
        t = np.linspace(0.0, tb, 60001)
        _, nn = tree.query(o64[r][None, :] + t[:, None] * d64[r][None, :])
        change = np.concatenate([[True], nn[1:] != nn[:-1]])
        seq = nn[change]
        ext = np.diff(np.concatenate([t[change], [tb]]))
        steps = int(f.steps[r])
        t1 = f.t_exit[r, :steps].astype(np.float64)
        keep = t1 < tb  # cells the walk leaves inside the box
        walk = np.array(f.cells[r, :steps])[keep]
        dt = np.diff(np.concatenate([[0.0], t1]))[keep]
        # the last dense cell is the one the ray is in when it leaves the box
        if seq[:-1].tolist() == walk.tolist():
            exact += 1
        # a ray that grazes an edge crosses slivers that the fp16-rounded
        # planes and a finite sampling grid decide differently: drop a cell
        # from both sequences when it is a sliver in either
        slivers = set(walk[dt < sliver].tolist()) | set(seq[:-1][ext[:-1] < sliver].tolist())
        a = [c for c in walk.tolist() if c not in slivers]
        b = [c for c in seq[:-1].tolist() if c not in slivers]
        if a == b:
            robust += 1
    assert exact >= 0.95 * n_rays, f"{exact} of {n_rays} rays match exactly"
    assert robust == n_rays, f"{n_rays - robust} rays differ beyond slivers"


def test_nn_bruteforce(oracle_lib):
    w = scene(1)
    rng = np.random.default_rng(1)
    q = np.concatenate([rng.uniform(-1.5, 1.5, (2000, 3)), w.points[:100]]).astype(np.float32)
    got = oracle_lib.nn(w.points, q, threads=4)
    d = np.linalg.norm(w.points[None, :, :].astype(np.float64) - q[:, None, :].astype(np.float64), axis=-1)
    ref = np.argmin(d, axis=1)
    srt = np.sort(d, axis=1)
    clear = (srt[:, 1] - srt[:, 0]) > 1e-6  # skip near-ties under fp32 rounding
    assert np.array_equal(got[clear], ref[clear])
    assert np.array_equal(got[2000:], np.arange(100))


@pytest.mark.parametrize("n", [32, 33, 1000, 4104, 5000])
def test_aabb_tree_bounds(oracle_lib, n):
    rng = np.random.default_rng(n)
    pts = rng.uniform(-1, 1, (n, 3)).astype(np.float32)
    tree = oracle_lib.build_aabb_tree(pts)
    n2 = tree.shape[0]
    td = n2.bit_length() - 1
    assert n2 == 1 << td and n2 >= n
    padded = np.concatenate([pts, np.repeat(pts[-1:], n2 - n, axis=0)])
    for d in range(td):
        width = 1 << d
        start = n2 - (2 << d)
        span = n2 >> d  # points under one node at depth d
        for i in range(width):
            block = padded[i * span:(i + 1) * span]
            node = tree[start + i]
            assert np.array_equal(node[0], block.min(axis=0)), (d, i)
            assert np.array_equal(node[1], block.max(axis=0)), (d, i)
    assert np.all(tree[n2 - 1] == 0)
