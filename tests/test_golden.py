"""Committed C1 fixture (tests/golden/c1.npz, written by gen_golden.py):
the generator reproduces its inputs, the oracle reproduces its outputs bit
for bit, and the GPU path matches it through the C ABI (visits, counts and
depth indices exactly; rgba/depth and gradients to the stated tolerances)."""

import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "c1.npz")
MODES = ("sdfoam", "standard")


@pytest.fixture(scope="module")
def gold():
    return np.load(FIXTURE)


def test_generator_reproduces_inputs(gold):
    from sdfoam_amd import scenes

    w = scenes.make_config(1)
    assert np.array_equal(w.points, gold["points"])
    assert np.array_equal(w.adjacency, gold["adjacency"])
    assert np.array_equal(w.offsets, gold["offsets"])
    assert np.array_equal(w.rays, gold["rays"])
    assert np.array_equal(w.attributes, gold["sdfoam_attributes"])
    assert np.array_equal(scenes.start_points_for(w.points, w.rays), gold["start"])


@pytest.mark.parametrize("mode", MODES)
def test_oracle_reproduces_outputs(gold, oracle_lib, mode):
    g = gold
    inv = float(g["inv_s"])
    attrs = g[f"{mode}_attributes"]
    f = oracle_lib.trace_forward(0, g["points"], attrs, g["adjacency"], g["offsets"], g["rays"],
                                 g["start"], g["quantiles"], alpha_mode=mode, inv_s=inv)
    for k in ("rgba", "depth", "depth_indices", "num_intersections", "visit_hash"):
        assert np.array_equal(getattr(f, k), g[f"{mode}_{k}"]), k
    b = oracle_lib.trace_backward(0, g["points"], attrs, g["adjacency"], g["offsets"], g["rays"],
                                  g["start"], f.rgba, g["grad_rgba"], g["quantiles"],
                                  f.depth_indices, g["depth_grad"], alpha_mode=mode, inv_s=inv)
    assert np.array_equal(b.attr_grad.astype(np.float32), g[f"{mode}_attr_grad"])
    assert np.array_equal(b.points_grad.astype(np.float32), g[f"{mode}_points_grad"])
    assert np.array_equal(b.visit_hash, g[f"{mode}_backward_visit_hash"])


@pytest.mark.gpu
@pytest.mark.parametrize("mode", MODES)
def test_gpu_matches_fixture(gold, oracle_lib, mode):
    import torch

    import sdfoam_amd

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda:0")
    g = gold

    def u32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.uint32).view(np.int32)).to(dev).view(torch.uint32)

    def f32(a):
        return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dev)

    pipe = sdfoam_amd.create_pipeline(0)
    args = (f32(g["points"]), f32(g[f"{mode}_attributes"]), u32(g["adjacency"]), u32(g["offsets"]),
            f32(g["rays"]), u32(g["start"]))
    inv = torch.tensor([float(g["inv_s"])], device=dev)
    q = f32(g["quantiles"])
    out = pipe.trace_forward(*args, depth_quantiles=q, return_contribution=True, alpha_mode=mode,
                             inv_s=inv)
    st = pipe.walk_stats(*args, alpha_mode=mode, inv_s=inv)
    bwd = pipe.trace_backward(*args, out["rgba"], f32(g["grad_rgba"]), q, out["depth_indices"],
                              f32(g["depth_grad"]), alpha_mode=mode, inv_s=inv)
    torch.cuda.synchronize()
    assert np.array_equal(out["num_intersections"].view(torch.int32).cpu().numpy().view(np.uint32),
                          g[f"{mode}_num_intersections"])
    assert np.array_equal(out["depth_indices"].view(torch.int32).cpu().numpy().view(np.uint32),
                          g[f"{mode}_depth_indices"])
    assert np.array_equal(st["visit_hash"].cpu().numpy().view(np.uint64).reshape(64, 64),
                          g[f"{mode}_visit_hash"])
    rgba = out["rgba"].cpu().numpy()
    ref = g[f"{mode}_rgba"]
    assert np.all(np.abs(rgba - ref) <= 1e-5 + 1e-4 * np.abs(ref))
    d = out["depth"].cpu().numpy()
    assert np.all(np.abs(d - g[f"{mode}_depth"]) <= 1e-5 + 1e-4 * np.abs(g[f"{mode}_depth"]))
    # gradients: the fixture's values with the summation bound of the oracle's
    # side buffers (fp32 atomics sum in any order)
    b = oracle_lib.trace_backward(0, g["points"], g[f"{mode}_attributes"], g["adjacency"],
                                  g["offsets"], g["rays"], g["start"], rgba, g["grad_rgba"],
                                  g["quantiles"], g[f"{mode}_depth_indices"], g["depth_grad"],
                                  alpha_mode=mode, inv_s=float(g["inv_s"]))
    u = 2.0 ** -24
    for key, got, A, K in (("attr_grad", bwd["attr_grad"], b.attr_grad_abs, b.attr_grad_k),
                           ("points_grad", bwd["points_grad"], b.points_grad_abs, b.points_grad_k)):
        ref = g[f"{mode}_{key}"].astype(np.float64)
        k = np.maximum(K.astype(np.float64) - 1, 0)
        tol = 1e-5 + 1e-4 * np.abs(ref) + (k * u / (1 - k * u)) * A + 2 * u * np.abs(ref)
        err = np.abs(got.cpu().numpy().astype(np.float64) - ref)
        assert np.all(err <= tol), key
