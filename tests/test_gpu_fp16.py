"""fp16 attribute pipelines (create_pipeline(L, "float16"); the reference's
CUDATracingPipeline<__half, L>) against the oracle run on the same
attribute values widened to fp32 (exact).

Arithmetic is fp32 in both, so visit sequences, loop counts and depth
indices stay bit-exact, depths keep the fp32 bars and the render is
bit-exact.  Outputs of the attribute type carry one fp16 rounding
(u_h = 2^-11) and fp16 accumulation: rgba |d| <= 1e-5 + (1e-4 + u_h)|ref|;
contribution and attribute gradients |d| <= 1e-5 + (1e-4 + u_h)|ref| +
gamma_K(u_h) A, with K the element's contribution count and A the sum of
their magnitudes (each fp16 atomic add rounds once).  points_grad and the
sharpness gradient are fp32 and keep the fp32 bars."""

import numpy as np
import pytest

from conftest import scene
from test_gpu_parity import (_threads, assert_close, assert_close_model, gpu_scene, np_u32,
                             sum_depth,
                             to_dev)

pytestmark = pytest.mark.gpu

UH = 2.0 ** -11


def gamma_h(k):
    k = np.maximum(np.asarray(k, dtype=np.float64) - 1.0, 0.0)
    return k * UH / np.maximum(1.0 - k * UH, 1e-3)


def assert_close_h(name, got, ref, abs_sum, k):
    got = np.asarray(got, dtype=np.float64)
    tol = 1e-5 + (1e-4 + UH) * np.abs(ref) + gamma_h(k) * abs_sum
    bad = ~(np.abs(got - ref) <= tol)
    if bad.any():
        i = np.argmax(np.where(bad, np.abs(got - ref) / np.maximum(tol, 1e-30), 0))
        raise AssertionError(f"{name}: {int(bad.sum())} of {bad.size} out of tolerance; worst "
                             f"got {got.ravel()[i]!r} ref {np.ravel(ref)[i]!r} tol {tol.ravel()[i]!r}")


@pytest.fixture(scope="module")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def half_scene(index, mode="sdfoam", **kw):
    import dataclasses

    w = scene(index, mode=mode, **kw)
    return dataclasses.replace(w, attributes=w.attributes.astype(np.float16).astype(np.float32))


def _inputs(w, dev):
    import torch

    g = gpu_scene(w, dev)
    g["attributes"] = g["attributes"].to(torch.float16)
    return g


@pytest.mark.parametrize("cfg,mode,accum,degree", [
    (1, "sdfoam", True, None), (1, "standard", True, None), (2, "sdfoam", True, None),
    (1, "sdfoam", False, None), (2, "sdfoam", False, None), (1, "sdfoam", True, 2),
    (1, "sdfoam", False, 1)])
def test_fp16_forward_backward(dev, oracle_lib, cfg, mode, accum, degree):
    """accum: the backward's fp32 cell rows rounded once into the fp16
    outputs; without: packed fp16 atomics per group into the outputs (odd
    and even attribute counts: degrees 0-3 have 4, 13, 28, 49)."""
    import torch

    import sdfoam_amd

    w = half_scene(cfg, mode) if degree is None else half_scene(cfg, mode, sh_degree=degree)
    g = _inputs(w, dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, "float16")
    q = to_dev(w.quantiles, dev)
    inv_t = torch.tensor([w.inv_s], device=dev)
    rec = 1100 if cfg == 1 else 160
    fwd = pipe.trace_forward(**g, depth_quantiles=q, return_contribution=True, alpha_mode=mode,
                             inv_s=inv_t, record_walk=True)
    assert fwd["rgba"].dtype == torch.float16 and fwd["contribution"].dtype == torch.float16
    assert fwd["depth"].dtype == torch.float32 and fwd["alpha"].dtype == torch.float32
    grad_rgba = w.grad_rgba.astype(np.float16)
    rerr = np.random.default_rng(11).uniform(0, 1, w.rays.shape[:-1]).astype(np.float16)
    bwd = pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=to_dev(grad_rgba, dev),
                              depth_quantiles=q, depth_indices=fwd["depth_indices"],
                              depth_grad_in=to_dev(w.depth_grad, dev),
                              ray_error=to_dev(rerr, dev), alpha_mode=mode, inv_s=inv_t,
                              trace_plan=fwd.get("trace_plan"), grad_accum=accum)
    torch.cuda.synchronize()
    assert bwd["attr_grad"].dtype == torch.float16 and bwd["points_grad"].dtype == torch.float32
    R = w.num_rays
    ref = oracle_lib.trace_forward(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, w.rays, w.extra["start"],
        w.quantiles, alpha_mode=mode, inv_s=w.inv_s, record=rec, threads=_threads())
    assert np.all(ref.steps <= rec)
    ni = np_u32(fwd["num_intersections"]).reshape(R)
    assert np.array_equal(ni, ref.num_intersections.reshape(R))
    assert np.array_equal(np_u32(fwd["depth_indices"]).reshape(R, -1),
                          ref.depth_indices.reshape(R, -1))
    assert_close("depth", fwd["depth"].cpu().numpy().reshape(R, -1), ref.depth.reshape(R, -1))
    rgba = fwd["rgba"].float().cpu().numpy().reshape(R, 4)
    rref = ref.rgba.reshape(R, 4)
    assert_close_h("rgba", rgba, rref, np.zeros_like(rref), 0)
    # contribution: K = visits of the cell (from the full visit record)
    cells = ref.cells[np.arange(rec)[None, :] < ref.steps.reshape(R)[:, None]]
    kc = np.bincount(cells, minlength=w.num_points)
    cref = ref.contribution.reshape(-1)
    assert_close_h("contribution", fwd["contribution"].float().cpu().numpy().reshape(-1), cref,
                   np.abs(cref), kc)

    # backward on the same fp16-rounded inputs the GPU read
    bref = oracle_lib.trace_backward(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets, w.rays, w.extra["start"],
        rgba.reshape(w.rays.shape[:-1] + (4,)), grad_rgba.astype(np.float32), w.quantiles,
        np_u32(fwd["depth_indices"]), w.depth_grad, rerr.astype(np.float32), alpha_mode=mode,
        inv_s=w.inv_s, threads=_threads())
    assert_close_model("points_grad", bwd["points_grad"].cpu().numpy(), bref.points_grad,
                       bref.points_grad_abs, bref.points_grad_k)
    assert_close_h("attr_grad", bwd["attr_grad"].float().cpu().numpy(), bref.attr_grad,
                   bref.attr_grad_abs, bref.attr_grad_k)
    sg = float(bwd["sharpness_grad"].cpu().numpy().reshape(-1)[0])
    assert_close_model("sharpness_grad", np.array([sg]), np.array([bref.sharpness_grad]),
                       np.array([bref.sharpness_abs]),
                       np.array([min(bref.sharpness_k, sum_depth(w, bref))]))
    pe = bwd["point_error"].float().cpu().numpy().reshape(-1)
    pref = bref.point_error.reshape(-1)
    assert_close_h("point_error", pe, pref, np.abs(pref), kc)


def test_fp16_render_bitexact(dev, oracle_lib):
    """benchmark.py's setting: fp16 attributes, the caller's half offset
    table, weight threshold 0.05."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes

    w = half_scene(2)
    cam = scenes.camera_dict(w.extra["camera"], "pinhole", 160, 120)
    pts = to_dev(w.points, dev)
    attrs = to_dev(w.attributes, dev).to(torch.float16)
    g = gpu_scene(w, dev)
    diff = sdfoam_amd.prefetch_adjacent_diff(pts, g["point_adjacency"], g["point_adjacency_offsets"])
    ray0 = np.concatenate([cam["position"], cam["forward"]]).reshape(1, 6).astype(np.float32)
    start = int(scenes.start_points_for(w.points, ray0)[0])
    st = torch.tensor([start], dtype=torch.int32, device=dev).view(torch.uint32)
    out = torch.zeros((120, 160), dtype=torch.uint32, device=dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, "float16")
    pipe.trace_benchmark(pts, attrs, g["point_adjacency"], g["point_adjacency_offsets"], diff,
                         cam, st, out, weight_threshold=0.05, alpha_mode="sdfoam",
                         inv_s=torch.tensor(w.inv_s, device=dev).reshape(()))
    torch.cuda.synchronize()
    got = out.view(torch.int32).cpu().numpy().view(np.uint32)
    ref = oracle_lib.trace_benchmark(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
        diff.view(torch.int16).cpu().numpy().view(np.uint16)[:w.adjacency.size], cam, start,
        alpha_mode="sdfoam", inv_s=w.inv_s, weight_threshold=0.05, threads=_threads())
    assert np.array_equal(got, ref.rgba8)


def test_fp16_trace_rays_autograd(dev):
    import torch

    import sdfoam_amd

    w = half_scene(1)
    g = _inputs(w, dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, "float16")
    pts = g["points"].clone().requires_grad_(True)
    attrs = g["attributes"].clone().requires_grad_(True)
    inv = torch.full((1,), w.inv_s, device=dev, requires_grad=True)
    rgba, depth, contrib, nis, errbox, alpha = sdfoam_amd.TraceRays.apply(
        pipe, pts, attrs, g["point_adjacency"], g["point_adjacency_offsets"], g["rays"],
        g["start_point"], to_dev(w.quantiles, dev), True, True, inv, 1e-6, None)
    loss = (rgba.float() * to_dev(w.grad_rgba, dev)).sum()
    loss.backward()
    assert attrs.grad.dtype == torch.float16 and torch.isfinite(attrs.grad.float()).all()
    assert torch.isfinite(pts.grad).all() and torch.isfinite(inv.grad).all()
    del depth, contrib, nis, errbox, alpha


def test_fp16_dtype_validation(dev):
    import torch

    import sdfoam_amd

    w = half_scene(1)
    g = _inputs(w, dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree, "float16")
    fwd = pipe.trace_forward(**g)
    with pytest.raises(RuntimeError, match="rgb_grad_in had dtype Float, expected float16"):
        pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=fwd["rgba"].float())
    g32 = gpu_scene(w, dev)
    with pytest.raises(RuntimeError, match="expected float16"):
        pipe.trace_forward(**g32)
