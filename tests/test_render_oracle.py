"""The inference render's host restatement (oracle.trace_benchmark) and the
shared camera / colour arithmetic, pinned without a GPU:

* sin / cos / atan2 of include/sdfoam_fpmath.h against float64 (a few ulp);
* cast_ray against the camera model in float64 (src/tracing/camera.h:56-85):
  pinhole and fisheye, the centre pixel looks along `forward`, fisheye
  pixels past phi = pi are masked to a zero direction;
* make_rgba8 (src/tracing/tracing_utils.cuh:126-136) on hand-checked values;
* the render equals the traced forward on the same cast rays: the same C and
  T (bit for bit) and loop counts, and the packed pixel is clamp(C + T bg)
  * 255 truncated, stored in row H-1-j.
"""

import math

import numpy as np
import pytest

from conftest import scene

U = 2.0 ** -24


def test_sincos_accuracy(oracle_lib):
    x = np.linspace(-7.0, 7.0, 400001).astype(np.float32)
    s, c = oracle_lib.sincosf(x)
    xd = x.astype(np.float64)
    # absolute error within 2 ulp of 1 (the functions have magnitude <= 1)
    assert np.max(np.abs(s - np.sin(xd))) < 2 * U * 1.0 + 1e-12
    assert np.max(np.abs(c - np.cos(xd))) < 2 * U * 1.0 + 1e-12
    # relative error near the origin (no reduction): 1 ulp
    small = np.abs(xd) < 0.5
    rel = np.abs(s[small] - np.sin(xd[small])) / np.maximum(np.abs(np.sin(xd[small])), 1e-30)
    assert np.max(rel[np.abs(xd[small]) > 1e-6]) < 2 * U
    s0, c0 = oracle_lib.sincosf(np.float32([0.0]))
    assert s0.tolist() == [0.0] and c0.tolist() == [1.0]


def test_atan2_accuracy_and_special_values(oracle_lib):
    rng = np.random.default_rng(1)
    y = np.concatenate([rng.normal(size=100000), rng.uniform(-1, 1, 1000) * 1e-3]).astype(np.float32)
    x = np.concatenate([rng.normal(size=100000), rng.uniform(-1, 1, 1000)]).astype(np.float32)
    a = oracle_lib.atan2f(y, x)
    ref = np.arctan2(y.astype(np.float64), x.astype(np.float64))
    assert np.max(np.abs(a - ref) / np.maximum(np.abs(ref), 1e-30)) < 4 * U
    cases = [((0.0, 0.0), 0.0), ((-0.0, 0.0), -0.0), ((0.0, -0.0), math.pi),
             ((-0.0, -0.0), -math.pi), ((1.0, 0.0), math.pi / 2), ((-1.0, 0.0), -math.pi / 2),
             ((0.0, -1.0), math.pi), ((1.0, 1.0), math.pi / 4), ((-1.0, -1.0), -3 * math.pi / 4)]
    for (yy, xx), want in cases:
        got = float(oracle_lib.atan2f(np.float32([yy]), np.float32([xx]))[0])
        assert got == float(np.float32(want)), (yy, xx, got, want)
        assert math.copysign(1.0, got) == math.copysign(1.0, want)


def _cam(cfg=1, model="pinhole", width=None, height=None, fov=None):
    from sdfoam_amd import scenes

    w = scene(cfg)
    return scenes.camera_dict(w.extra["camera"], model, width, height, fov)


def _cast_f64(cam, i, j):
    W, H = cam["width"], cam["height"]
    f, r, up = (np.asarray(cam[k], dtype=np.float64) for k in ("forward", "right", "up"))
    u = (2.0 * i / W - 1.0) * (W / H)
    v = 1.0 - 2.0 * j / H
    if cam["model"] == "pinhole":
        d = f / math.tan(cam["fov"] / 2) + u * r + v * up
    else:
        th = math.atan2(v, u)
        ph = cam["fov"] * math.hypot(u, v)
        if ph >= math.pi:
            return np.zeros(3)
        d = math.sin(ph) * math.cos(th) * r + math.sin(ph) * math.sin(th) * up + math.cos(ph) * f
    return d / np.linalg.norm(d)


@pytest.mark.parametrize("model", ["pinhole", "fisheye"])
def test_cast_ray_against_float64(oracle_lib, model):
    cam = _cam(2, model, 97, 61, fov=1.1 if model == "pinhole" else 2.6)
    rng = np.random.default_rng(3)
    masked = 0
    for i, j in zip(rng.integers(0, 97, 400), rng.integers(0, 61, 400)):
        got = oracle_lib.cast_ray(cam, int(i), int(j))
        want = _cast_f64(cam, int(i), int(j))
        if not want.any():
            masked += 1
            assert not got.any()
            continue
        assert np.max(np.abs(got - want)) < 2e-6, (i, j, got, want)
    if model == "fisheye":
        assert masked > 0  # fov 2.6 masks the corners


@pytest.mark.parametrize("model", ["pinhole", "fisheye"])
def test_centre_pixel_looks_forward(oracle_lib, model):
    cam = _cam(1, model, 64, 48)
    got = oracle_lib.cast_ray(cam, 32, 24)
    assert np.max(np.abs(got - cam["forward"])) <= 2 * U


def test_make_rgba8_values(oracle_lib):
    m = oracle_lib.make_rgba8
    assert m(0, 0, 0, 1) == 0xFF000000
    assert m(1, 1, 1, 1) == 0xFFFFFFFF
    assert m(2.0, -1.0, 0.5, 1.0) == (255 << 24) | (127 << 16) | (0 << 8) | 255
    assert m(float("nan"), 0, 0, 0) == 255  # min(1, NaN) = 1 as std::min(1.f, NaN)
    assert m(1.0 / 255.0, 0, 0, 0) == 1 and m(0.999, 0, 0, 0) == 254


def _trace_both(oracle_lib, w, cam, mode="sdfoam", bg=None, checker=False):
    from sdfoam_amd import scenes

    W, H = cam["width"], cam["height"]
    diff = oracle_lib.prefetch_adjacent_diff(w.points, w.adjacency, w.offsets)
    ray0 = np.concatenate([cam["position"], cam["forward"]]).reshape(1, 6).astype(np.float32)
    start = scenes.start_points_for(w.points, ray0)[0]
    ren = oracle_lib.trace_benchmark(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                     diff, cam, start, alpha_mode=mode, inv_s=w.inv_s,
                                     bg_color=bg, checker_bg=checker, threads=8)
    rays = np.zeros((H, W, 6), dtype=np.float32)
    rays[..., :3] = cam["position"]
    for j in range(H):
        for i in range(W):
            rays[j, i, 3:] = oracle_lib.cast_ray(cam, i, j)
    starts = np.full((H, W), start, dtype=np.uint32)
    fwd = oracle_lib.trace_forward(w.sh_degree, w.points, w.attributes, w.adjacency, w.offsets,
                                   rays, starts, None, alpha_mode=mode, inv_s=w.inv_s, threads=8)
    return ren, fwd, rays


@pytest.mark.parametrize("mode", ["sdfoam", "standard"])
def test_render_equals_forward_on_cast_rays(oracle_lib, mode):
    w = scene(1, mode=mode)
    cam = _cam(1, "pinhole", 48, 40)
    ren, fwd, _ = _trace_both(oracle_lib, w, cam, mode)
    H, W = 40, 48
    rgbt = ren.rgbt.reshape(H, W, 4)
    assert np.array_equal(rgbt[..., :3].view(np.uint32), fwd.rgba[..., :3].view(np.uint32))
    assert np.array_equal((np.float32(1.0) - rgbt[..., 3]).view(np.uint32),
                          fwd.rgba[..., 3].view(np.uint32))
    assert np.array_equal(ren.num_intersections.reshape(H, W), fwd.num_intersections.reshape(H, W))
    # white background: fma(T, 1, C) = C + T rounded once
    col = rgbt[..., :3] + rgbt[..., 3:4]
    q = (np.clip(col, 0.0, 1.0) * np.float32(255.0)).astype(np.int32).astype(np.uint32)
    packed = (255 << 24) | (q[..., 2] << 16) | (q[..., 1] << 8) | q[..., 0]
    assert np.array_equal(ren.rgba8[::-1], packed)  # row H-1-j holds pixel row j
    assert (ren.num_intersections > 1).mean() > 0.5


def test_render_background_and_checker(oracle_lib):
    """A camera looking away from the cloud from a corner cell leaves it at
    once: T stays 1 and every pixel is the background."""
    from sdfoam_amd import scenes

    w = scene(1)
    cam = scenes.camera_dict(scenes.look_at([0.99, 0.99, 0.99], [3.0, 3.0, 3.0], [0, 0, 1],
                                            0.5, 40, 40))
    ren, _, _ = _trace_both(oracle_lib, w, cam, bg=[0.2, 0.4, 0.6])
    assert np.all(ren.rgbt[:, 3] == 1.0)
    want = oracle_lib.make_rgba8(0.2, 0.4, 0.6, 1.0)
    assert np.all(ren.rgba8 == want)
    ren2, _, _ = _trace_both(oracle_lib, w, cam, checker=True)
    img = ren2.rgba8[::-1]
    g3 = oracle_lib.make_rgba8(0.3, 0.3, 0.3, 1.0)
    g5 = oracle_lib.make_rgba8(0.5, 0.5, 0.5, 1.0)
    assert img[0, 0] == g3 and img[0, 20] == g5 and img[20, 0] == g5 and img[20, 20] == g3
