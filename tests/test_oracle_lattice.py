"""Closed-form pins of the oracle's walk, compositing and position gradients.

Sites on a cubic lattice of spacing h = 2^-3 make every fp16 neighbour offset
and every plane crossing exact, so the visit sequence, the segment lengths,
the transmittance chain, rgba and the quantile depth have closed forms that
are evaluated here in float64, independently of the oracle's code.

The position-gradient bookkeeping (src/tracing/pipeline.cu:452-474, with the
reference's quirks: the first cell gets a face against the world origin,
the last two cells are never flushed) is pinned against central finite
differences of a float64 model of the same rendering on a chain of sites."""

import math

import numpy as np
import pytest

H = 0.125
C0 = 0.28209479177387814


def lattice(n, neighbourhood=6):
    nx, ny, nz = n
    idx = np.arange(nx * ny * nz).reshape(nx, ny, nz)
    g = np.stack(np.meshgrid(np.arange(nx), np.arange(ny), np.arange(nz), indexing="ij"), -1)
    pts = ((g - np.array(n) / 2.0) * H).reshape(-1, 3).astype(np.float32)
    if neighbourhood == 6:
        offs = [(1, 0, 0), (-1, 0, 0), (0, 1, 0), (0, -1, 0), (0, 0, 1), (0, 0, -1)]
    else:
        offs = [(a, b, c) for a in (-1, 0, 1) for b in (-1, 0, 1) for c in (-1, 0, 1)
                if (a, b, c) != (0, 0, 0)]
    rows = []
    for i in range(nx):
        for j in range(ny):
            for k in range(nz):
                r = [idx[i + a, j + b, k + c] for a, b, c in offs
                     if 0 <= i + a < nx and 0 <= j + b < ny and 0 <= k + c < nz]
                rows.append(sorted(r))
    offsets = np.zeros(len(rows) + 1, dtype=np.uint32)
    offsets[1:] = np.cumsum([len(r) for r in rows])
    adj = np.array([x for r in rows for x in r], dtype=np.uint32)
    return pts, adj, offsets, idx


def expected(k, sdf, rgb, n_steps, q, thr=1e-7):
    phi = 1.0 / (1.0 + math.exp(k * sdf))
    s = k * phi * (1 - phi)
    T = 1.0
    C = 0.0
    t0 = 0.0
    depth = None
    steps = 0
    for i in range(n_steps):
        dt = 0.75 * H if i == 0 else H
        a = 1 - math.exp(-s * dt)
        Tn = T * (1 - a)
        C += T * a * rgb
        if depth is None and Tn < q:
            frac = min(1.0, max(0.0, (T - q) / (T - Tn)))
            depth = (t0 + frac * dt, i)
        T = Tn
        t0 += dt
        steps += 1
        if not T > thr:
            break
    return C, T, depth, steps


@pytest.mark.parametrize("neigh", [6, 26])
@pytest.mark.parametrize("k,sdf,q", [(math.exp(0.3), 0.0, 0.99), (50.0, 0.02, 0.5), (5.0, -0.1, 0.6)])
def test_axis_walk_closed_form(oracle_lib, neigh, k, sdf, q):
    n = (16, 4, 4)
    pts, adj, offs, idx = lattice(n, neigh)
    N = pts.shape[0]
    v = np.float32(0.37)
    attrs = np.zeros((N, 4), np.float32)
    attrs[:, :3] = v
    attrs[:, 3] = sdf
    c0 = idx[0, 1, 2]
    o = pts[c0] + np.array([-H / 4, H / 8, -3 * H / 16], np.float32)
    rays = np.array([[*o, 1.0, 0.0, 0.0]], np.float32)
    f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays, np.array([c0], np.uint32),
                                 np.array([[q]], np.float32), inv_s=k, record=32)
    rgb = 0.5 + C0 * float(v)
    C, T, depth, steps = expected(k, sdf, rgb, 15, q)
    assert int(f.steps[0]) == steps
    n_loop = 16 if steps == 15 else steps
    assert int(f.num_intersections[0, 0]) == n_loop
    assert list(f.cells[0, :steps]) == [int(idx[i, 1, 2]) for i in range(steps)]
    assert abs(f.rgba[0, 3] - (1 - T)) <= 1e-6
    for c in range(3):
        assert abs(f.rgba[0, c] - C) <= 2e-6 * max(1.0, C)
    if depth is None:
        assert f.depth[0, 0] == -1.0 and f.depth_indices[0, 0] == 0xFFFFFFFF
    else:
        assert abs(f.depth[0, 0] - depth[0]) <= 1e-6
        assert int(f.depth_indices[0, 0]) == int(idx[depth[1], 1, 2])


def test_max_intersections_cap(oracle_lib):
    pts, adj, offs, idx = lattice((16, 4, 4))
    attrs = np.zeros((pts.shape[0], 4), np.float32)
    c0 = idx[0, 1, 2]
    o = pts[c0] + np.array([-H / 4, H / 8, -3 * H / 16], np.float32)
    rays = np.array([[*o, 1.0, 0.0, 0.0]], np.float32)
    for cap in [0, 1, 5, 14, 15, 100]:
        f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays, np.array([c0], np.uint32),
                                     inv_s=1.0, max_intersections=cap)
        assert int(f.steps[0]) == min(cap, 15)
        assert int(f.num_intersections[0, 0]) == (cap + 1 if cap < 16 else 16)


def test_reverse_and_out_of_range_start(oracle_lib):
    pts, adj, offs, idx = lattice((8, 3, 3))
    attrs = np.zeros((pts.shape[0], 4), np.float32)
    c0 = idx[7, 1, 1]
    o = pts[c0] + np.array([H / 4, 0, 0], np.float32)
    rays = np.array([[*o, -2.0, 0.0, 0.0], [*o, -2.0, 0.0, 0.0]], np.float32)
    f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays,
                                 np.array([c0, pts.shape[0] + 5], np.uint32), inv_s=1.0, record=16)
    assert list(f.cells[0, :7]) == [int(idx[i, 1, 1]) for i in range(7, 0, -1)]
    # a start point outside the scene ends the walk before the first step
    assert int(f.num_intersections[1, 0]) == 0 and f.rgba[1, 3] == 0.0


# ---------------------------------------------------------------------------
# position gradients on a chain


def chain(m):
    pts = np.zeros((m, 3), np.float32)
    pts[:, 0] = (np.arange(m) - m / 2) * H
    rows = [[j for j in (i - 1, i + 1) if 0 <= j < m] for i in range(m)]
    offs = np.zeros(m + 1, np.uint32)
    offs[1:] = np.cumsum([len(r) for r in rows])
    adj = np.array([x for r in rows for x in r], np.uint32)
    return pts, adj, offs


def model_loss(P, o, d, attrs, k, g4, m, deltas=None):
    """float64 rendering of the ray through cells 0..m-1 of the chain."""
    T, C = 1.0, np.zeros(3)
    t_prev = 0.0
    for i in range(m - 1):
        p, q = P[i], P[i + 1]
        t = ((p + q) / 2 - o) @ (q - p) / ((q - p) @ d)
        dt = max(t - t_prev, 0.0) if deltas is None else deltas[i]
        phi = 1.0 / (1.0 + math.exp(k * attrs[i, 3]))
        s = k * phi * (1 - phi)
        a = 1 - math.exp(-s * dt)
        rgb = np.maximum(0.0, 0.5 + C0 * attrs[i, :3].astype(np.float64))
        C = C + T * a * rgb
        T *= 1 - a
        t_prev = t
    return g4[:3] @ C + g4[3] * (1 - T)


def test_position_gradient_bookkeeping(oracle_lib):
    m = 9
    pts, adj, offs = chain(m)
    rng = np.random.default_rng(3)
    attrs = np.zeros((m, 4), np.float32)
    attrs[:, :3] = rng.uniform(-1, 1, (m, 3))
    attrs[:, 3] = rng.uniform(-0.2, 0.2, m)
    k = 6.0
    o = (pts[0] + np.array([-H / 4, 0.01, -0.02])).astype(np.float32)
    d = np.array([1.0, 0.03, -0.02])
    d = (d / np.linalg.norm(d)).astype(np.float32)
    rays = np.array([[*o, *d]], np.float32)
    g4 = rng.normal(size=4).astype(np.float32)
    f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays, np.array([0], np.uint32),
                                 inv_s=k, record=16)
    assert list(f.cells[0, : m - 1]) == list(range(m - 1))
    b = oracle_lib.trace_backward(0, pts, attrs, adj, offs, rays, np.array([0], np.uint32),
                                  f.rgba, g4[None, :], inv_s=k)
    P = pts.astype(np.float64)
    o64, d64 = o.astype(np.float64), d.astype(np.float64)
    g64 = g4.astype(np.float64)

    def L(Pp):
        return model_loss(Pp, o64, d64, attrs, k, g64, m)

    eps = 1e-6
    fd = np.zeros((m, 3))
    for i in range(m):
        for c in range(3):
            Pp, Pm = P.copy(), P.copy()
            Pp[i, c] += eps
            Pm[i, c] -= eps
            fd[i, c] = (L(Pp) - L(Pm)) / (2 * eps)
    got = b.points_grad
    scale = np.abs(fd).max()
    # interior cells: the chain rule through both faces of the cell
    for i in range(1, m - 2):
        assert np.allclose(got[i], fd[i], rtol=1e-3, atol=1e-4 * scale), (i, got[i], fd[i])
    # the walk steps through cells 0..m-2; the last stepped cell (m-2) and its
    # exit neighbour (m-1) are never flushed, though both move the last face
    assert np.all(got[m - 2:] == 0.0)
    assert np.abs(fd[m - 2:]).max() > 1e-3 * scale
    # the first cell: true gradient plus dL/dt0 of step 0 times the gradient
    # of a face against the world origin (t0 = 0 there, so the true term is 0)
    t_faces = [((P[i] + P[i + 1]) / 2 - o64) @ (P[i + 1] - P[i]) / ((P[i + 1] - P[i]) @ d64)
               for i in range(m - 1)]
    deltas = np.diff(np.concatenate([[0.0], t_faces]))
    dp, dm = deltas.copy(), deltas.copy()
    dp[0] += eps
    dm[0] -= eps
    dL_ddelta0 = (model_loss(P, o64, d64, attrs, k, g64, m, dp)
                  - model_loss(P, o64, d64, attrs, k, g64, m, dm)) / (2 * eps)
    p0, q0 = P[0], np.zeros(3)
    fn = q0 - p0
    num = ((p0 + q0) / 2 - o64) @ fn
    den = fn @ d64
    G0 = (num * d64 + den * (o64 - p0)) / den ** 2
    expect0 = fd[0] + (-dL_ddelta0) * G0
    assert np.allclose(got[0], expect0, rtol=1e-3, atol=1e-4 * scale), (got[0], expect0, fd[0])


def test_cell_intersection_grad_is_dt_dp(oracle_lib):
    rng = np.random.default_rng(9)
    for _ in range(200):
        p = rng.normal(size=3)
        q = p + rng.normal(size=3) * 0.3
        o = rng.normal(size=3) * 2
        d = rng.normal(size=3)
        d /= np.linalg.norm(d)
        if abs((q - p) @ d) < 0.05:
            continue

        def t(pp):
            return ((pp + q) / 2 - o) @ (q - pp) / ((q - pp) @ d)

        eps = 1e-6
        fd = np.array([(t(p + eps * e) - t(p - eps * e)) / (2 * eps) for e in np.eye(3)])
        got = oracle_lib.cell_intersection_grad(p, q, o, d).astype(np.float64)
        assert np.allclose(got, fd, rtol=2e-3, atol=2e-4 * max(1.0, np.abs(fd).max())), (got, fd)
