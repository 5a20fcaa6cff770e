"""The HIP forward and backward on the exact lattice ray, against the float64
closed forms of the reference's equations (tests/test_oracle_density_mode.py
for the standard mode, tests/test_oracle_depth_coupling.py for sdfoam mode),
with and without the walk record, and against the oracle on the same inputs.

References: src/tracing/pipeline.cu:36-264 (forward), :267-550 (backward_sdf),
:553-791 (density backward)."""

import numpy as np
import pytest

import test_oracle_density_mode as dm
import test_oracle_depth_coupling as dc
from test_gpu_parity import np_u32, to_dev, torch_dev, u32  # noqa: F401
from test_oracle_lattice import H, lattice

pytestmark = pytest.mark.gpu


def _gpu_run(dev, pts, attrs, adj, offs, rays, start, qs, gqs, g4, mode, inv_s, record):
    import torch

    import sdfoam_amd

    pipe = sdfoam_amd.create_pipeline(0)
    g = dict(points=to_dev(pts, dev), attributes=to_dev(attrs, dev),
             point_adjacency=u32(adj, dev), point_adjacency_offsets=u32(offs, dev),
             rays=to_dev(rays, dev), start_point=u32(start, dev))
    q = to_dev(np.array([qs], np.float32), dev)
    inv_t = torch.tensor([inv_s], device=dev)
    fwd = pipe.trace_forward(**g, depth_quantiles=q, return_contribution=True, alpha_mode=mode,
                             inv_s=inv_t, record_walk=record)
    bwd = pipe.trace_backward(**g, rgb_out=fwd["rgba"], grad_in=to_dev(g4[None, :], dev),
                              depth_quantiles=q, depth_indices=fwd["depth_indices"],
                              depth_grad_in=to_dev(np.array([gqs], np.float32), dev),
                              alpha_mode=mode, inv_s=inv_t, trace_plan=fwd.get("trace_plan"))
    torch.cuda.synchronize()
    return fwd, bwd


class _F:
    """The GPU outputs under the oracle's field names, for the closed-form checks."""

    def __init__(self, fwd, bwd):
        self.rgba = fwd["rgba"].cpu().numpy().reshape(1, 4)
        self.depth = fwd["depth"].cpu().numpy().reshape(1, -1)
        self.depth_indices = np_u32(fwd["depth_indices"]).reshape(1, -1)
        self.contribution = fwd["contribution"].cpu().numpy().reshape(-1, 1)
        self.alpha = fwd["alpha"].cpu().numpy().reshape(-1, 1)
        self.points_grad = bwd["points_grad"].cpu().numpy()
        self.attr_grad = bwd["attr_grad"].cpu().numpy()
        self.sharpness_grad = float(bwd["sharpness_grad"].cpu().numpy().reshape(-1)[0])


@pytest.mark.parametrize("record", [False, True])
@pytest.mark.parametrize("qs,gqs", dm.CASES)
def test_density_mode_lattice_gpu(torch_dev, oracle_lib, qs, gqs, record):
    pts, adj, offs, idx = lattice((16, 4, 4), 26)
    N = pts.shape[0]
    attrs = np.zeros((N, 4), np.float32)
    attrs[:, :3] = 0.37
    attrs[:, 3] = 1.0
    cells = [int(idx[i, 1, 2]) for i in range(16)]
    attrs[cells, :3] = dm.V[:, None]
    attrs[cells, 3] = dm.SIGMA
    o = pts[cells[0]] + np.array([-H / 4, H / 8, -3 * H / 16], np.float32)
    rays = np.array([[*o, 1.0, 0.0, 0.0]], np.float32)
    start = np.array([cells[0]], np.uint32)
    fwd, bwd = _gpu_run(torch_dev, pts, attrs, adj, offs, rays, start, qs, gqs, dm.G4,
                        "standard", 1.0, record)
    got = _F(fwd, bwd)
    assert int(np_u32(fwd["num_intersections"]).reshape(-1)[0]) == 16
    n = 15
    cf = dm.closed_form(qs, gqs, dm.G4.astype(np.float64), n)
    P = pts[cells].astype(np.float64)
    err = dm._errors(got, got, cells, P, o.astype(np.float64), np.array([1.0, 0.0, 0.0]), n, cf)
    assert max(err.values()) <= 1.0, err
    np.testing.assert_allclose(got.contribution[cells[:n], 0], cf["w"], rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(got.alpha[cells[:n], 0], cf["alpha"], rtol=1e-5, atol=1e-7)
    others = np.setdiff1d(np.arange(N), cells[:n + 1])
    assert np.all(got.points_grad[others] == 0.0) and np.all(got.attr_grad[others] == 0.0)
    # and the oracle on the same inputs
    f, b, *_ = dm._run(oracle_lib, qs, gqs, dm.G4)
    assert np.array_equal(got.depth_indices, f.depth_indices)
    np.testing.assert_allclose(got.rgba, f.rgba, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(got.depth, f.depth, rtol=1e-6, atol=1e-7)
    sc = np.abs(b.points_grad).max()
    np.testing.assert_allclose(got.points_grad, b.points_grad, rtol=1e-5, atol=1e-6 * sc)
    sc = np.abs(b.attr_grad).max()
    np.testing.assert_allclose(got.attr_grad, b.attr_grad, rtol=1e-5, atol=1e-6 * sc)


@pytest.mark.parametrize("record", [False, True])
@pytest.mark.parametrize("qs,gqs", dc.CASES)
def test_sdfoam_depth_coupling_lattice_gpu(torch_dev, oracle_lib, qs, gqs, record):
    pts, adj, offs, idx = lattice((16, 4, 4), 26)
    N = pts.shape[0]
    attrs = np.zeros((N, 4), np.float32)
    attrs[:, :3] = dc.V
    attrs[:, 3] = dc.SDF
    c0 = idx[0, 1, 2]
    cells = [int(idx[i, 1, 2]) for i in range(16)]
    o = pts[c0] + np.array([-H / 4, H / 8, -3 * H / 16], np.float32)
    rays = np.array([[*o, 1.0, 0.0, 0.0]], np.float32)
    g4 = np.array([0.4, -0.7, 0.2, 0.9], np.float32)
    fwd, bwd = _gpu_run(torch_dev, pts, attrs, adj, offs, rays, np.array([c0], np.uint32), qs,
                        gqs, g4, "sdfoam", dc.K_SHARP, record)
    got = _F(fwd, bwd)
    n = 15
    cf = dc.closed_form(qs, gqs, g4.astype(np.float64), n)
    sdf = got.attr_grad[cells[:n], 3]
    np.testing.assert_allclose(sdf, cf["sdf"], rtol=1e-4, atol=1e-5 * np.abs(cf["sdf"]).max())
    assert abs(got.sharpness_grad - cf["sharp"]) <= 1e-4 * abs(cf["sharp"]) + 1e-6
    P = pts[cells].astype(np.float64)
    pg = dc.position_grads(cf, P, o.astype(np.float64), np.array([1.0, 0.0, 0.0]), n)
    np.testing.assert_allclose(got.points_grad[cells[:n + 1]], pg, rtol=1e-4,
                               atol=1e-5 * np.abs(pg).max())
    others = np.setdiff1d(np.arange(N), cells[:n + 1])
    assert np.all(got.points_grad[others] == 0.0)
