"""GPU parity of the inference render (Pipeline.trace_benchmark through
sdf_trace_benchmark) against the host oracle's restatement of the
reference's `benchmark` kernel (src/tracing/pipeline.cu:1067-1199): the
packed RGBA8 image must be bit-exact (camera rays, walk, compositing and
packing all follow the shared fp contract)."""

import numpy as np
import pytest

from conftest import scene

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


def _render_both(w, dev, oracle_lib, cam, mode="sdfoam", bg=None, checker=False,
                 caller_table=False, inv_s=None):
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes

    inv = w.inv_s if inv_s is None else inv_s
    pts = torch.from_numpy(w.points).to(dev)
    attrs = torch.from_numpy(w.attributes).to(dev)
    adj, offs = _u32(w.adjacency, dev), _u32(w.offsets, dev)
    E = w.adjacency.size
    if caller_table:
        # the reference's benchmark.py builds the table itself: (x_adj - x_self)
        # cast to half, one row per adjacency entry, no padding
        self_idx = torch.repeat_interleave(
            torch.arange(w.num_points, device=dev),
            (offs.view(torch.int32)[1:].to(torch.int64) - offs.view(torch.int32)[:-1].to(torch.int64)))
        off3 = pts[adj.view(torch.int32).to(torch.int64)] - pts[self_idx]
        diff = torch.cat([off3, torch.zeros_like(off3[:, :1])], dim=1).to(torch.half).contiguous()
        assert diff.shape == (E, 4)
    else:
        diff = sdfoam_amd.prefetch_adjacent_diff(pts, adj, offs)
    ray0 = np.concatenate([cam["position"], cam["forward"]]).reshape(1, 6).astype(np.float32)
    start = int(scenes.start_points_for(w.points, ray0)[0])
    start_t = _u32([start], dev)
    out = torch.zeros((cam["height"], cam["width"]), dtype=torch.uint32, device=dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    cam_t = dict(cam)
    for k in ("position", "forward", "right", "up"):
        cam_t[k] = torch.from_numpy(np.asarray(cam[k], dtype=np.float32))
    pipe.trace_benchmark(pts, attrs, adj, offs, diff, cam_t, start_t, out, alpha_mode=mode,
                         inv_s=torch.tensor([inv], device=dev), bg_color=bg, checker_bg=checker)
    torch.cuda.synchronize()
    got = out.view(torch.int32).cpu().numpy().view(np.uint32)
    diff_np = diff.view(torch.int16).cpu().numpy().view(np.uint16)[:E]
    ref = oracle_lib.trace_benchmark(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                     diff_np, cam, start, alpha_mode=mode, inv_s=inv,
                                     bg_color=bg, checker_bg=checker, threads=16)
    return got, ref


def _cam(w, model="pinhole", width=None, height=None, fov=None):
    from sdfoam_amd import scenes

    return scenes.camera_dict(w.extra["camera"], model, width, height, fov)


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_render_c1(dev, oracle_lib, mode):
    w = scene(1, mode=mode)
    got, ref = _render_both(w, dev, oracle_lib, _cam(w), mode)
    assert np.array_equal(got, ref.rgba8)
    assert len(np.unique(got)) > 50  # a real image, not a flat background


def test_render_c1_fisheye_masked_checker(dev, oracle_lib):
    """fov 2.6: corner pixels pass phi = pi and take the background colour;
    non-square image whose width is not a multiple of the 16-pixel tile."""
    w = scene(1)
    cam = _cam(w, "fisheye", 70, 45, fov=2.6)
    got, ref = _render_both(w, dev, oracle_lib, cam, bg=[0.1, 0.2, 0.3], checker=True)
    assert np.array_equal(got, ref.rgba8)
    assert got[0, 0] == oracle_lib.make_rgba8(0.1, 0.2, 0.3, 1.0)


def test_render_c2_caller_table(dev, oracle_lib):
    """SH degree 3; the caller's unpadded [E, 4] half table (as the
    reference's benchmark.py builds it) equals the prefetch table and the
    render reads it without over-reading."""
    w = scene(2)
    cam = _cam(w, "pinhole", 200, 150)
    got, ref = _render_both(w, dev, oracle_lib, cam, caller_table=True)
    assert np.array_equal(got, ref.rgba8)
    got2, _ = _render_both(w, dev, oracle_lib, cam, caller_table=False)
    assert np.array_equal(got, got2)


def test_render_c2_sharp_threshold(dev, oracle_lib):
    """inv_s = 50 and the benchmark's weight threshold 0.05: walks end early."""
    import torch

    import sdfoam_amd
    from sdfoam_amd import scenes

    w = scene(2)
    cam = _cam(w, "pinhole", 160, 160)
    pts = torch.from_numpy(w.points).to(dev)
    attrs = torch.from_numpy(w.attributes).to(dev)
    adj, offs = _u32(w.adjacency, dev), _u32(w.offsets, dev)
    diff = sdfoam_amd.prefetch_adjacent_diff(pts, adj, offs)
    ray0 = np.concatenate([cam["position"], cam["forward"]]).reshape(1, 6).astype(np.float32)
    start = int(scenes.start_points_for(w.points, ray0)[0])
    out = torch.zeros((160, 160), dtype=torch.uint32, device=dev)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    pipe.trace_benchmark(pts, attrs, adj, offs, diff, cam, _u32([start], dev), out,
                         weight_threshold=0.05, alpha_mode="sdfoam",
                         inv_s=torch.tensor(50.0, device=dev).reshape(()))
    torch.cuda.synchronize()
    got = out.view(torch.int32).cpu().numpy().view(np.uint32)
    ref = oracle_lib.trace_benchmark(
        w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
        diff.view(torch.int16).cpu().numpy().view(np.uint16)[:w.adjacency.size], cam, start,
        alpha_mode="sdfoam", inv_s=50.0, weight_threshold=0.05, threads=16)
    assert np.array_equal(got, ref.rgba8)


def test_render_validation(dev):
    import torch

    import sdfoam_amd

    w = scene(1)
    pts = torch.from_numpy(w.points).to(dev)
    attrs = torch.from_numpy(w.attributes).to(dev)
    adj, offs = _u32(w.adjacency, dev), _u32(w.offsets, dev)
    diff = sdfoam_amd.prefetch_adjacent_diff(pts, adj, offs)
    cam = _cam(w)
    pipe = sdfoam_amd.create_pipeline(w.sh_degree)
    out = torch.zeros((64, 64), dtype=torch.uint32, device=dev)
    with pytest.raises(RuntimeError, match="start_point must have a single element"):
        pipe.trace_benchmark(pts, attrs, adj, offs, diff, cam, _u32([0, 1], dev), out)
    with pytest.raises(RuntimeError, match="output_rgba must have width"):
        pipe.trace_benchmark(pts, attrs, adj, offs, diff, cam, _u32([0], dev), out[:10])
    bad = dict(cam, model="ortho")
    with pytest.raises(RuntimeError, match="Invalid camera model"):
        pipe.trace_benchmark(pts, attrs, adj, offs, diff, bad, _u32([0], dev), out)
    with pytest.raises(RuntimeError, match="adjacent_diff"):
        pipe.trace_benchmark(pts, attrs, adj, offs, diff[:10], cam, _u32([0], dev), out)
