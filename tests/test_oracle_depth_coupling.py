"""Hand-derived pin of the oracle's sdfoam depth-gradient terms
(src/tracing/pipeline.cu:352-353, 405-482).

These terms are not the derivative of the linearised quantile depth: the
reference adds the quantile's alpha term to dL/dalpha after dL/ds and dL/dDelta
were formed from it (a dead store), and it couples log T0 of a crossing into
the alpha of every *later* segment.  Finite differences therefore cannot check
them.  Instead, on the exact dyadic lattice of test_oracle_lattice (constant
SDF: constant alpha; segment lengths 3h/4 then h; T_i a geometric sequence),
the reference's equations are written out in closed form in float64:

* crossing segment m of quantile q (first m with T_{m+1} < q):
  frac = (T_m - q) / (T_m - T_{m+1}); dL/dt0 gets gq (1 - frac) and dL/dt1
  gets gq frac, i.e. dL/dDelta_m += gq frac and the unit t0 term += gq;
* g_logT = sum of gq Delta_m q / (alpha_m T_m) over the quantiles crossed
  before segment i; every such later segment gets dL/dalpha_i -=
  g_logT / (1 - alpha_i);
* the SDF gradient of cell i is dL/ds_i ds/dd, the sharpness gradient
  sum_i dL/ds_i ds/dsha, and the position gradient of cell i collects the
  four face derivatives of the two segments on either side of it (with the
  reference's face against the world origin for the first cell and the last
  two cells never flushed).

The oracle must match these within fp32 rounding, and variants with the
coupling one segment early or late, with its sign flipped, or without the
frac term must not: each changes the pinned gradients far beyond the
tolerance."""

import math

import numpy as np
import pytest

from test_oracle_lattice import C0, H, lattice

K_SHARP = 5.0
SDF = -0.1
V = 0.37


def _G(p, q, o, d):
    """d t / d p for t = ((p + q) / 2 - o) . (q - p) / ((q - p) . d)
    (src/tracing/tracing_utils.cuh:112-124; pinned by finite differences in
    test_oracle_lattice)."""
    fn = q - p
    num = ((p + q) / 2 - o) @ fn
    den = fn @ d
    return (num * d + den * (o - p)) / den ** 2


def closed_form(qs, gqs, g4, n_steps, variant=None):
    """The reference's sdfoam backward on the lattice ray, in closed form.

    variant: None (the reference), "early" (coupling from the crossing
    segment itself), "late" (from two segments after it), "sign" (coupling
    added with the wrong sign), "nofrac" (no gq frac term on Delta)."""
    k = K_SHARP
    phi = 1.0 / (1.0 + math.exp(k * SDF))
    s = k * phi * (1 - phi)
    deltas = np.array([0.75 * H] + [H] * (n_steps - 1))
    alpha = 1.0 - np.exp(-s * deltas)
    # T_i before segment i: (1 - alpha_0) (1 - alpha)^(i - 1)
    T = np.concatenate([[1.0], np.cumprod(1.0 - alpha)])
    c = max(0.0, 0.5 + C0 * V)
    A = 1.0 - T[n_steps]
    Cfin = c * A
    # accumulated colour after segment i: c (1 - T_{i+1})
    C_after = c * (1.0 - T[1:])

    # crossing segments: first m with T_{m+1} < q (quantiles sorted descending)
    cross = {}
    for q, gq in zip(qs, gqs):
        m = int(np.argmax(T[1:n_steps + 1] < q))
        assert T[m + 1] < q <= T[m]
        cross.setdefault(m, []).append((q, gq))
    # coupling carried into segment i: sum over crossings at m < i
    shift = {"early": 0, "late": 2}.get(variant, 1)
    sign = -1.0 if variant == "sign" else 1.0
    g_logT = np.zeros(n_steps)
    for m, lst in cross.items():
        val = sum(gq * deltas[m] * q / (alpha[m] * T[m]) for q, gq in lst)
        g_logT[m + shift:] += sign * val

    dL_ds = np.zeros(n_steps)
    dL_dt0 = np.zeros(n_steps)
    dL_dt1 = np.zeros(n_steps)
    for i in range(n_steps):
        rest = (np.array([Cfin] * 3) - C_after[i]) / (T[i] * (1 - alpha[i]) + 1e-6)
        dL_da = T[i] * np.sum((c - rest) * g4[:3])
        dL_da += (1.0 - A) * g4[3] / (1.0 - alpha[i] + 1e-6)
        dL_da -= g_logT[i] / max(1.0 - alpha[i], 1e-12)
        dL_ds[i] = dL_da * deltas[i] * (1 - alpha[i])
        dL_dD = dL_da * s * (1 - alpha[i])
        units = 0.0
        for q, gq in cross.get(i, []):
            frac = min(1.0, max(0.0, (T[i] - q) / (T[i] - T[i + 1])))
            units += gq
            if variant != "nofrac":
                dL_dD += gq * frac
        dL_dt0[i] = units - dL_dD
        dL_dt1[i] = dL_dD
    ds_dd = k * (1 - 2 * phi) * (-k * phi * (1 - phi))
    ds_dsha = phi * (1 - phi) * (1 - k * SDF * (1 - 2 * phi))
    return dict(sdf=dL_ds * ds_dd, sharp=float(np.sum(dL_ds * ds_dsha)), dt0=dL_dt0,
                dt1=dL_dt1, T=T)


def position_grads(cf, P, o, d, n_steps):
    """Cell i's position gradient: dL/dt1_{i-1} G(c_i, c_{i-1}) + dL/dt0_i
    G(c_i, c_{i-1}) + dL/dt1_i G(c_i, c_{i+1}) + dL/dt0_{i+1} G(c_i, c_{i+1}),
    with c_{-1} the world origin; cells n-1 and n are never flushed."""
    dt0, dt1 = cf["dt0"], cf["dt1"]
    out = np.zeros((n_steps + 1, 3))
    zero = np.zeros(3)
    for i in range(n_steps - 1):
        prev = P[i - 1] if i > 0 else zero
        g = dt0[i] * _G(P[i], prev, o, d) + dt1[i] * _G(P[i], P[i + 1], o, d)
        g += dt0[i + 1] * _G(P[i], P[i + 1], o, d)
        if i > 0:
            g += dt1[i - 1] * _G(P[i], P[i - 1], o, d)
        out[i] = g
    return out


def _trace(oracle_lib, qs, gqs, g4):
    n = (16, 4, 4)
    pts, adj, offs, idx = lattice(n, 26)
    N = pts.shape[0]
    attrs = np.zeros((N, 4), np.float32)
    attrs[:, :3] = V
    attrs[:, 3] = SDF
    c0 = idx[0, 1, 2]
    o = pts[c0] + np.array([-H / 4, H / 8, -3 * H / 16], np.float32)
    rays = np.array([[*o, 1.0, 0.0, 0.0]], np.float32)
    start = np.array([c0], np.uint32)
    q = np.array([qs], np.float32)
    f = oracle_lib.trace_forward(0, pts, attrs, adj, offs, rays, start, q, inv_s=K_SHARP,
                                 record=32)
    steps = int(f.steps[0])
    assert steps == 15
    cells = [int(idx[i, 1, 2]) for i in range(16)]
    assert list(f.cells[0, :steps]) == cells[:steps]
    b = oracle_lib.trace_backward(0, pts, attrs, adj, offs, rays, start, f.rgba, g4[None, :], q,
                                  f.depth_indices, np.array([gqs], np.float32), inv_s=K_SHARP)
    P = pts[cells].astype(np.float64)
    return b, cells, P, o.astype(np.float64), np.array([1.0, 0.0, 0.0]), steps


CASES = [
    ([0.6], [1.3]),            # one quantile, crossed early
    ([0.45], [-0.8]),          # one quantile, negative upstream gradient
    ([0.7, 0.3], [0.9, -1.1]),  # two quantiles in different segments
    ([0.62, 0.61], [1.5, 0.7]),  # two quantiles crossed in the same segment
]


@pytest.mark.parametrize("qs,gqs", CASES)
def test_depth_coupling_closed_form(oracle_lib, qs, gqs):
    g4 = np.array([0.4, -0.7, 0.2, 0.9], np.float32)
    b, cells, P, o, d, n = _trace(oracle_lib, qs, gqs, g4)
    cf = closed_form(qs, gqs, g4.astype(np.float64), n)
    sdf = b.attr_grad[cells[:n], 3]
    scale_sdf = np.abs(cf["sdf"]).max()
    np.testing.assert_allclose(sdf, cf["sdf"], rtol=1e-4, atol=1e-5 * scale_sdf)
    assert abs(b.sharpness_grad - cf["sharp"]) <= 1e-4 * abs(cf["sharp"]) + 1e-6
    pg = position_grads(cf, P, o, d, n)
    got_pg = b.points_grad[cells[: n + 1]]
    scale_pg = np.abs(pg).max()
    np.testing.assert_allclose(got_pg, pg, rtol=1e-4, atol=1e-5 * scale_pg)
    # no other cell gets a gradient
    others = np.setdiff1d(np.arange(b.points_grad.shape[0]), cells[:n + 1])
    assert np.all(b.points_grad[others] == 0.0)


@pytest.mark.parametrize("variant", ["early", "late", "sign", "nofrac"])
@pytest.mark.parametrize("qs,gqs", CASES[2:])
def test_depth_coupling_variants_are_caught(oracle_lib, qs, gqs, variant):
    """A one-segment slip, a sign slip or a missing term in the coupling moves
    the pinned gradients by far more than the tolerance the test above
    allows, so the closed form tells them apart."""
    g4 = np.array([0.4, -0.7, 0.2, 0.9], np.float32)
    b, cells, P, o, d, n = _trace(oracle_lib, qs, gqs, g4)
    cf = closed_form(qs, gqs, g4.astype(np.float64), n, variant=variant)
    sdf = b.attr_grad[cells[:n], 3]
    scale_sdf = np.abs(sdf).max()
    err_sdf = np.max(np.abs(sdf - cf["sdf"]) / (1e-4 * np.abs(cf["sdf"]) + 1e-5 * scale_sdf))
    pg = position_grads(cf, P, o, d, n)
    got_pg = b.points_grad[cells[: n + 1]]
    err_pg = np.max(np.abs(got_pg - pg) / (1e-4 * np.abs(pg) + 1e-5 * np.abs(got_pg).max()))
    err_sh = abs(b.sharpness_grad - cf["sharp"]) / (1e-4 * abs(cf["sharp"]) + 1e-6)
    assert max(err_sdf, err_pg, err_sh) > 100.0, (variant, err_sdf, err_pg, err_sh)
