"""Hand-derived pins of the oracle's density ("standard") mode: the forward's
analytic quantile depth and colour gate (src/tracing/pipeline.cu:86-101,
217-230) and the density backward's depth and position terms
(src/tracing/pipeline.cu:590-629, 646-760).

On the exact dyadic lattice of test_oracle_lattice the walk, the segment
lengths (3h/4, then h) and the faces are exact, so with a density sigma_i per
cell every quantity of the reference's equations has a closed form, written
here in float64 independently of the oracle's loop:

forward
  alpha_i = 1 - exp(-sigma_i Delta_i), T_{i+1} = T_i (1 - alpha_i); the colour
  of cell i is its SH colour when sigma_i > 1e-6 and 0 otherwise; quantile q is
  crossed in the first segment m with T_{m+1} < q, at depth
  t0_m + log(T_m / q) / sigma_m, with depth index cell m.

backward
  P = sum over the crossed quantiles k of gq_k / sigma_{m_k} (the pending depth
  gradient, taken from the forward's depth indices); for segment i:
    rest  = (C - C_after_i) / (T_i (1 - alpha_i + 1e-6))
    dL/dalpha = T_i (rgb_i - rest) . g_rgb + (1 - A) g_a / (1 - alpha_i + 1e-6)
    dL/dsigma = dL/dalpha Delta_i (1 - alpha_i),  dL/dDelta = dL/dalpha sigma_i (1 - alpha_i)
    for each quantile k crossed in segment i: u = gq_k / sigma_i;
      dL/dt0 += u, dL/dsigma -= u log(T_i / q_k) / sigma_i, P -= u
    while a quantile is still to be crossed after segment i:
      dL/dsigma -= Delta_i P, dL/dDelta -= sigma_i P
    dL/dt0 = units - dL/dDelta, dL/dt1 = dL/dDelta.
  The unit term of the crossing segment is gq / sigma although d depth / d t0 is 1
  (a quirk of the reference, pipeline.cu:709-711): finite differences cannot pin
  it, the closed form does.  Every other depth term is the true derivative of
  t0_m + (-sum_{j<m} sigma_j Delta_j - log q) / sigma_m; test_depth_terms_are_derivatives
  checks that of the closed form by central differences.

The oracle must match these within fp32 rounding; plausible slips (gq instead
of gq/sigma, the unit term on t1, a missing or sign-flipped pending term, a
flipped log) must miss by far more than the tolerance.  Position gradients
with zero depth gradients are also pinned by finite differences of a float64
density rendering of a chain of sites."""

import math

import numpy as np
import pytest

from test_oracle_depth_coupling import position_grads
from test_oracle_lattice import C0, H, chain, lattice

F32_GATE = float(np.float32(1e-6))
# per-cell densities (exact in fp32); cells 2 and 5 sit at or below the colour
# gate and carry a huge SH value, so a wrong gate moves rgba by ~0.03
SIGMA = np.array([2.0, 3.5, 1e-6, 1.25, 5.0, 0.0, 0.75, 4.0, 2.5, 6.0, 1.5, 3.0, 2.0,
                  0.5, 4.5, 1.0], np.float32)
V = np.full(16, 0.37, np.float32)
V[[2, 5]] = 1.0e6


def cell_colour(v):
    return max(0.0, 0.5 + C0 * float(v))


def closed_form(qs, gqs, g4, n, variant=None):
    """The reference's standard-mode forward and density backward on the
    lattice ray, in float64 (see the module docstring).  variant: None (the
    reference), "dg" (unit term gq instead of gq/sigma), "t1" (unit term on t1),
    "nopending" (no pending depth term), "sign" (pending term added with the
    wrong sign), "logsign" (log(q/T) in the crossing's sigma term)."""
    sig = SIGMA[:n].astype(np.float64)
    deltas = np.array([0.75 * H] + [H] * (n - 1))
    alpha = 1.0 - np.exp(-sig * deltas)
    T = np.concatenate([[1.0], np.cumprod(1.0 - alpha)])
    gate = SIGMA[:n] > np.float32(F32_GATE)
    rgb = np.array([cell_colour(V[i]) if gate[i] else 0.0 for i in range(n)])
    w = T[:n] * alpha
    C_after = np.cumsum(w * rgb)
    Cfin = C_after[-1]
    A = 1.0 - T[n]
    t0 = np.concatenate([[0.0], np.cumsum(deltas)])[:n]

    cross, depth, didx = {}, [], []
    for k, q in enumerate(qs):
        hit = np.nonzero(T[1:n + 1] < q)[0]
        if hit.size == 0:
            depth.append(-1.0)
            didx.append(None)
            continue
        m = int(hit[0])
        cross.setdefault(m, []).append(k)
        depth.append(t0[m] + math.log(T[m] / q) / sig[m])
        didx.append(m)
    P = sum(gqs[k] / sig[didx[k]] for k in range(len(qs)) if didx[k] is not None)
    crossed = 0
    dens = np.zeros(n)
    dt0 = np.zeros(n)
    dt1 = np.zeros(n)
    for i in range(n):
        rest = (Cfin - C_after[i]) / (T[i] * (1.0 - alpha[i] + 1e-6))
        dL_da = T[i] * np.sum((rgb[i] - rest) * g4[:3])
        dL_da += (1.0 - A) * g4[3] / (1.0 - alpha[i] + 1e-6)
        dL_ds = dL_da * deltas[i] * (1.0 - alpha[i])
        dL_dD = dL_da * sig[i] * (1.0 - alpha[i])
        units = 0.0
        for k in cross.get(i, []):
            u = gqs[k] / sig[i]
            units += gqs[k] if variant == "dg" else u
            lg = math.log(qs[k] / T[i]) if variant == "logsign" else math.log(T[i] / qs[k])
            dL_ds -= u * lg / sig[i]
            P -= u
            crossed += 1
        if crossed < len(qs) and variant != "nopending":
            sgn = -1.0 if variant == "sign" else 1.0
            dL_ds -= sgn * deltas[i] * P
            dL_dD -= sgn * sig[i] * P
        if variant == "t1":
            dt0[i] = -dL_dD
            dt1[i] = dL_dD + units
        else:
            dt0[i] = units - dL_dD
            dt1[i] = dL_dD
        dens[i] = dL_ds
    sh = np.where(rgb[:, None] > 0.0, C0 * w[:, None] * g4[None, :3], 0.0)
    return dict(T=T, rgb=rgb, w=w, alpha=alpha, C=Cfin, A=A, depth=depth, didx=didx,
                dens=dens, sh=sh, dt0=dt0, dt1=dt1)


def _run(oracle_lib, qs, gqs, g4):
    pts, adj, offs, idx = lattice((16, 4, 4), 26)
    N = pts.shape[0]
    attrs = np.zeros((N, 4), np.float32)
    attrs[:, :3] = 0.37
    attrs[:, 3] = 1.0
    cells = [int(idx[i, 1, 2]) for i in range(16)]
    attrs[cells, :3] = V[:, None]
    attrs[cells, 3] = SIGMA
    o = pts[cells[0]] + np.array([-H / 4, H / 8, -3 * H / 16], np.float32)
    rays = np.array([[*o, 1.0, 0.0, 0.0]], np.float32)
    start = np.array([cells[0]], np.uint32)
    q = np.array([qs], np.float32)
    f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays, start, q, alpha_mode="standard",
                                 record=32)
    n = int(f.steps[0])
    assert n == 15
    assert list(f.cells[0, :n]) == cells[:n]
    b = oracle_lib.trace_backward(0, pts, attrs, adj, offs, rays, start, f.rgba, g4[None, :], q,
                                  f.depth_indices, np.array([gqs], np.float32),
                                  alpha_mode="standard")
    assert int(b.steps[0]) == n
    P = pts[cells].astype(np.float64)
    return f, b, cells, P, o.astype(np.float64), np.array([1.0, 0.0, 0.0]), n


CASES = [
    ([0.6], [1.3]),                 # one quantile
    ([0.45], [-0.8]),               # one quantile, negative upstream gradient
    ([0.7, 0.3], [0.9, -1.1]),      # two quantiles in different segments
    ([0.62, 0.61], [1.5, 0.7]),     # two quantiles crossed in the same segment
    ([0.55, 1e-9], [0.8, 2.0]),     # the second quantile is never reached
    ([0.9, 0.2], [0.6, 0.5]),       # crossed in the first segment, then late
]
G4 = np.array([0.4, -0.7, 0.2, 0.9], np.float32)


def _errors(f, b, cells, P, o, d, n, cf):
    """Each compared quantity's largest error in units of its tolerance."""
    out = {}
    out["rgba"] = max(np.max(np.abs(f.rgba[0, :3] - cf["C"])) / (2e-6 * max(1.0, cf["C"])),
                      abs(f.rgba[0, 3] - cf["A"]) / 1e-6)
    e = 0.0
    for k, dep in enumerate(cf["depth"]):
        if cf["didx"][k] is None:
            e = max(e, 0.0 if (f.depth[0, k] == -1.0 and f.depth_indices[0, k] == 0xFFFFFFFF)
                    else np.inf)
        else:
            e = max(e, abs(f.depth[0, k] - dep) / (2e-6 * max(1.0, abs(dep))))
            e = max(e, 0.0 if int(f.depth_indices[0, k]) == cells[cf["didx"][k]] else np.inf)
    out["depth"] = e
    dens = b.attr_grad[cells[:n], 3]
    sc = np.abs(cf["dens"]).max()
    out["dens"] = np.max(np.abs(dens - cf["dens"]) / (1e-4 * np.abs(cf["dens"]) + 1e-5 * sc))
    sh = b.attr_grad[cells[:n], :3]
    sc = np.abs(cf["sh"]).max()
    out["sh"] = np.max(np.abs(sh - cf["sh"]) / (1e-4 * np.abs(cf["sh"]) + 1e-5 * sc))
    pg = position_grads(cf, P, o, d, n)
    got = b.points_grad[cells[: n + 1]]
    sc = np.abs(pg).max()
    out["pos"] = np.max(np.abs(got - pg) / (1e-4 * np.abs(pg) + 1e-5 * sc))
    return out


@pytest.mark.parametrize("qs,gqs", CASES)
def test_density_mode_closed_form(oracle_lib, qs, gqs):
    f, b, cells, P, o, d, n = _run(oracle_lib, qs, gqs, G4)
    cf = closed_form(qs, gqs, G4.astype(np.float64), n)
    err = _errors(f, b, cells, P, o, d, n, cf)
    assert max(err.values()) <= 1.0, err
    # the gate: cells 2 (sigma = 1e-6) and 5 (sigma = 0) add no colour and get no
    # SH gradient although their SH value is 1e6
    assert np.all(b.attr_grad[[cells[2], cells[5]], :3] == 0.0)
    assert cf["w"][2] > 0.0
    # per-point outputs of the forward
    np.testing.assert_allclose(f.contribution[cells[:n], 0], cf["w"], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(f.alpha[cells[:n], 0], cf["alpha"], rtol=1e-5, atol=1e-7)
    # nothing outside the walk gets a gradient
    others = np.setdiff1d(np.arange(b.points_grad.shape[0]), cells[:n + 1])
    assert np.all(b.points_grad[others] == 0.0) and np.all(b.attr_grad[others] == 0.0)


@pytest.mark.parametrize("variant", ["dg", "t1", "nopending", "sign", "logsign"])
@pytest.mark.parametrize("qs,gqs", [CASES[0], CASES[2], CASES[3]])
def test_density_mode_variants_are_caught(oracle_lib, qs, gqs, variant):
    """Each plausible slip in the density backward's depth terms moves the
    pinned gradients far beyond the tolerance the test above allows."""
    f, b, cells, P, o, d, n = _run(oracle_lib, qs, gqs, G4)
    cf = closed_form(qs, gqs, G4.astype(np.float64), n, variant=variant)
    err = _errors(f, b, cells, P, o, d, n, cf)
    assert max(err["dens"], err["pos"]) > 100.0, (variant, err)


def test_gate_and_depth_variants_are_caught(oracle_lib):
    """A colour gate that lets sigma = 1e-6 through, or a depth anchored on
    t1 or with the log flipped, misses the oracle's forward by far more than
    the tolerance."""
    qs, gqs = CASES[2]
    f, b, cells, P, o, d, n = _run(oracle_lib, qs, gqs, G4)
    cf = closed_form(qs, gqs, G4.astype(np.float64), n)
    # colour through the gate: cell 2's weight times its huge colour
    leak = cf["w"][2] * cell_colour(V[2])
    assert abs((cf["C"] + leak) - f.rgba[0, 0]) > 100 * 2e-6
    for k, m in enumerate(cf["didx"]):
        T, sig = cf["T"], float(SIGMA[m])
        t1 = (0.75 * H + m * H)
        t0 = t1 - (0.75 * H if m == 0 else H)
        anchored_t1 = t1 + math.log(T[m] / qs[k]) / sig
        flipped = t0 - math.log(T[m] / qs[k]) / sig
        for bad in (anchored_t1, flipped):
            assert abs(f.depth[0, k] - bad) > 100 * 2e-6 * max(1.0, abs(bad))


def test_depth_terms_are_derivatives():
    """Apart from the crossing segment's unit term, the closed form's depth
    terms are the derivatives of depth = t0_m + (-sum_{j<m} sigma_j Delta_j -
    log q) / sigma_m with respect to sigma_j and Delta_j (central differences
    in float64, rgba gradients zero)."""
    n = 15
    qs, gqs = [0.7, 0.3], [0.9, -1.1]
    cf = closed_form(qs, gqs, np.zeros(4), n)
    sig0 = SIGMA[:n].astype(np.float64)
    del0 = np.array([0.75 * H] + [H] * (n - 1))

    def depth_sum(sig, dl):
        # crossing segments stay fixed under the small perturbations
        logT = np.concatenate([[0.0], -np.cumsum(sig * dl)])
        t0 = np.concatenate([[0.0], np.cumsum(dl)])
        tot = 0.0
        for k, q in enumerate(qs):
            m = cf["didx"][k]
            tot += gqs[k] * (t0[m] + (logT[m] - math.log(q)) / sig[m])
        return tot

    eps = 1e-7
    for i in range(n):
        if sig0[i] == 0.0:
            continue
        sp, sm = sig0.copy(), sig0.copy()
        sp[i] += eps
        sm[i] -= eps
        fd = (depth_sum(sp, del0) - depth_sum(sm, del0)) / (2 * eps)
        assert abs(cf["dens"][i] - fd) <= 1e-6 * max(1.0, abs(fd)), (i, cf["dens"][i], fd)
    # dL/dDelta_i: the t1 term of the closed form; the t0 side adds the
    # reference's unit term gq / sigma_m on each crossing segment
    for i in range(n):
        dp, dm = del0.copy(), del0.copy()
        dp[i] += eps
        dm[i] -= eps
        fd = (depth_sum(sig0, dp) - depth_sum(sig0, dm)) / (2 * eps)
        # depth moves with t0_m, i.e. with every Delta_j, j < m: d depth/dDelta_j =
        # 1 - sigma_j / sigma_m, whose 1 the walk carries through t0 (face terms)
        unit = sum(gqs[k] for k, m in enumerate(cf["didx"]) if m is not None and m > i)
        assert abs(cf["dt1"][i] + unit - fd) <= 1e-6 * max(1.0, abs(fd)), (i, cf["dt1"][i], fd)
    units = np.zeros(n)
    for k, m in enumerate(cf["didx"]):
        units[m] += gqs[k] / sig0[m]
    np.testing.assert_allclose(cf["dt0"] + cf["dt1"], units, rtol=1e-12, atol=1e-12)


def density_loss(P, o, d, attrs, g4, m):
    """float64 density-mode rendering of the ray through cells 0..m-2 of the chain."""
    T, C = 1.0, np.zeros(3)
    t_prev = 0.0
    for i in range(m - 1):
        p, q = P[i], P[i + 1]
        t = ((p + q) / 2 - o) @ (q - p) / ((q - p) @ d)
        dt = max(t - t_prev, 0.0)
        s = float(attrs[i, 3])
        a = 1 - math.exp(-s * dt)
        rgb = np.maximum(0.0, 0.5 + C0 * attrs[i, :3].astype(np.float64)) if s > F32_GATE \
            else np.zeros(3)
        C = C + T * a * rgb
        T *= 1 - a
        t_prev = t
    return g4[:3] @ C + g4[3] * (1 - T)


def test_density_position_gradients_fd(oracle_lib):
    """With zero depth gradients the density backward's position gradients are
    the derivative of g . rgba: interior cells match central differences; the
    first cell adds the reference's face against the world origin and the last
    two cells are never flushed (as in sdfoam mode)."""
    m = 9
    pts, adj, offs = chain(m)
    rng = np.random.default_rng(11)
    attrs = np.zeros((m, 4), np.float32)
    attrs[:, :3] = rng.uniform(-1, 1, (m, 3))
    attrs[:, 3] = rng.uniform(0.5, 6.0, m)
    o = (pts[0] + np.array([-H / 4, 0.01, -0.02])).astype(np.float32)
    d = np.array([1.0, 0.03, -0.02])
    d = (d / np.linalg.norm(d)).astype(np.float32)
    rays = np.array([[*o, *d]], np.float32)
    g4 = rng.normal(size=4).astype(np.float32)
    qs = np.array([[0.5]], np.float32)
    f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays, np.array([0], np.uint32), qs,
                                 alpha_mode="standard", record=16)
    assert list(f.cells[0, : m - 1]) == list(range(m - 1))
    assert f.depth_indices[0, 0] != 0xFFFFFFFF
    b = oracle_lib.trace_backward(0, pts, attrs, adj, offs, rays, np.array([0], np.uint32),
                                  f.rgba, g4[None, :], qs, f.depth_indices,
                                  np.zeros((1, 1), np.float32), alpha_mode="standard")
    P = pts.astype(np.float64)
    o64, d64, g64 = o.astype(np.float64), d.astype(np.float64), g4.astype(np.float64)
    eps = 1e-6
    fd = np.zeros((m, 3))
    for i in range(m):
        for c in range(3):
            Pp, Pm = P.copy(), P.copy()
            Pp[i, c] += eps
            Pm[i, c] -= eps
            fd[i, c] = (density_loss(Pp, o64, d64, attrs, g64, m)
                        - density_loss(Pm, o64, d64, attrs, g64, m)) / (2 * eps)
    got = b.points_grad
    scale = np.abs(fd).max()
    for i in range(1, m - 2):
        assert np.allclose(got[i], fd[i], rtol=1e-3, atol=1e-4 * scale), (i, got[i], fd[i])
    assert np.all(got[m - 2:] == 0.0)
    assert np.abs(fd[m - 2:]).max() > 1e-3 * scale
    # a sign slip in the face terms would fail the interior cells
    assert not np.allclose(-got[1:m - 2], fd[1:m - 2], rtol=1e-3, atol=1e-4 * scale)
    # density channel: d(g . rgba)/d sigma_i by central differences
    for i in range(m - 1):
        ap, am = attrs.copy(), attrs.copy()
        ap[i, 3] += np.float32(1e-3)
        am[i, 3] -= np.float32(1e-3)
        h2 = float(ap[i, 3]) - float(am[i, 3])
        fds = (density_loss(P, o64, d64, ap, g64, m) - density_loss(P, o64, d64, am, g64, m)) / h2
        assert abs(b.attr_grad[i, 3] - fds) <= 2e-3 * abs(fds) + 2e-4 * scale, (i, fds)
