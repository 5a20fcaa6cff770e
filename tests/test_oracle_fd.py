"""Finite-difference pins of the oracle's backward passes on scene C1.

Loss L = sum(g . rgba) (+ sum(dg . depth) in density mode), evaluated in
float64 from the oracle's fp32 forward.  Central differences of L with
respect to SH coefficients, the SDF / density channel and the sharpness
must match the oracle's backward.  A perturbation changes only the rays
through the perturbed cell, so the difference carries their fp32 noise only.

Not covered here, and pinned elsewhere: position gradients (the walk uses
fp16 planes, so positions are pinned on an exact lattice,
test_oracle_lattice.py); the depth terms of sdfoam mode, whose coupling
through g_logT follows the reference's code (src/tracing/pipeline.cu:405-469)
and is not the derivative of the linearised depth, so finite differences
cannot pin it: test_oracle_depth_coupling.py restates those equations in
closed form on the exact lattice.
"""

import numpy as np
import pytest

from conftest import scene


def loss(oracle_lib, w, attrs, inv_s, rays, start, g4, mode, q=None, dg=None):
    f = oracle_lib.trace_forward(w.sh_degree, w.points, attrs, w.adjacency, w.offsets, rays, start,
                                 q, alpha_mode=mode, inv_s=inv_s)
    val = np.sum(f.rgba.astype(np.float64) * g4)
    if dg is not None:
        d = f.depth.astype(np.float64)
        val += np.sum(np.where(f.depth_indices != 0xFFFFFFFF, d, 0.0) * dg)
    return val, f


def setup(oracle_lib, mode, n_rays=512):
    w = scene(1, mode=mode)
    rng = np.random.default_rng(4)
    o = rng.uniform(-0.6, 0.6, (n_rays, 3))
    d = rng.normal(size=(n_rays, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    rays = np.concatenate([o, d], 1).astype(np.float32)
    start = oracle_lib.nn(w.points, rays[:, :3])
    g4 = rng.normal(size=(n_rays, 4))
    return w, rays, start, g4


def check(name, got, fd, scale):
    assert abs(got - fd) <= 2e-3 * abs(fd) + 2e-4 * scale, f"{name}: oracle {got} fd {fd}"


def test_sdfoam_attribute_and_sharpness_grads(oracle_lib):
    w, rays, start, g4 = setup(oracle_lib, "sdfoam")
    k = 5.0
    L0, f = loss(oracle_lib, w, w.attributes, k, rays, start, g4, "sdfoam")
    b = oracle_lib.trace_backward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                  rays, start, f.rgba, g4.astype(np.float32), inv_s=k)
    ag = b.attr_grad
    scale = np.abs(ag).max()
    # the most-visited cells, each channel
    order = np.argsort(-b.attr_grad_k[:, 3])[:6]
    for p in order:
        for ch in range(4):
            eps = 1e-2 if ch < 3 else 1e-3
            ap, am = w.attributes.copy(), w.attributes.copy()
            ap[p, ch] += eps
            am[p, ch] -= eps
            fd = (loss(oracle_lib, w, ap, k, rays, start, g4, "sdfoam")[0]
                  - loss(oracle_lib, w, am, k, rays, start, g4, "sdfoam")[0]) / (2 * eps)
            check(f"attr[{p},{ch}]", ag[p, ch], fd, scale)
    # the sharpness moves every ray: larger steps against the fp32 noise of
    # 512 rays, with Richardson extrapolation for the truncation error
    def fd_k(eps):
        return (loss(oracle_lib, w, w.attributes, k + eps, rays, start, g4, "sdfoam")[0]
                - loss(oracle_lib, w, w.attributes, k - eps, rays, start, g4, "sdfoam")[0]) / (2 * eps)

    fd = (4 * fd_k(0.05) - fd_k(0.1)) / 3
    assert abs(b.sharpness_grad - fd) <= 1e-3 * abs(fd) + 1e-4, (b.sharpness_grad, fd)


def test_density_mode_grads_with_depth(oracle_lib):
    w, rays, start, g4 = setup(oracle_lib, "standard")
    rng = np.random.default_rng(8)
    q = np.full((rays.shape[0], 1), 0.7, np.float32)
    dg = rng.normal(size=(rays.shape[0], 1))
    L0, f = loss(oracle_lib, w, w.attributes, 1.0, rays, start, g4, "standard", q, dg)
    b = oracle_lib.trace_backward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                  rays, start, f.rgba, g4.astype(np.float32), q, f.depth_indices,
                                  dg.astype(np.float32), alpha_mode="standard", inv_s=1.0)
    ag = b.attr_grad
    scale = np.abs(ag).max()
    order = np.argsort(-b.attr_grad_k[:, 3])[:6]
    for p in order:
        for ch in range(4):
            eps = 1e-2 if ch < 3 else 1e-3 * max(1.0, abs(float(w.attributes[p, 3])))
            ap, am = w.attributes.copy(), w.attributes.copy()
            ap[p, ch] += eps
            am[p, ch] -= eps
            Lp, fp = loss(oracle_lib, w, ap, 1.0, rays, start, g4, "standard", q, dg)
            Lm, fm = loss(oracle_lib, w, am, 1.0, rays, start, g4, "standard", q, dg)
            if not (np.array_equal(fp.depth_indices, f.depth_indices)
                    and np.array_equal(fm.depth_indices, f.depth_indices)):
                continue  # a quantile moved to another cell: not differentiable there
            check(f"attr[{p},{ch}]", ag[p, ch], (Lp - Lm) / (2 * eps), scale)
