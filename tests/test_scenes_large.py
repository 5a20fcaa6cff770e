"""Configs C4 (unbounded 360 scene) and C5 (training-step shape), checked at
reduced point counts on the CPU: proportions and geometry of the point sets,
the stale adjacency of C5, cameras, rays and quantiles."""

import math

import numpy as np
import pytest


@pytest.fixture(scope="module")
def c4():
    from sdfoam_amd import scenes

    return scenes.make_config(4, point_scale=0.004, image_scale=0.05)


@pytest.fixture(scope="module")
def c5():
    from sdfoam_amd import scenes

    return scenes.make_config(5, point_scale=0.004, image_scale=0.1)


def test_c4_points_and_cameras(c4):
    p = c4.points.astype(np.float64)
    assert c4.num_points == int(1_800_000 * 0.004) + int(1_200_000 * 0.004)
    r = np.linalg.norm(p, axis=1)
    inner = np.sum(r <= 1.0)
    assert abs(inner - 7200) <= 60  # blobs in the unit ball (+ a few shell points at r ~ 1)
    shell = r[r > 1.0 + 1e-6]
    assert shell.max() <= 16.0 + 1e-4
    # density ~ 1/r^2: r uniform on [1, 16]
    assert abs(np.mean(shell) - 8.5) < 0.5
    cams = c4.extra["cameras"]
    assert len(cams) == 8
    for k, c in enumerate(cams):
        a = 2 * math.pi * k / 8
        assert np.allclose(c.position, [4 * math.cos(a), 4 * math.sin(a), 0.0])
        assert np.allclose(c.forward, -c.position / 4.0)
    assert c4.rays.shape[0] == 8 and c4.rays.shape[-1] == 6
    d = c4.rays[..., 3:].astype(np.float64)
    assert np.allclose(np.linalg.norm(d, axis=-1), 1.0, atol=1e-6)
    # SDF = distance to the nearest blob centre - 0.1
    cen = c4.extra["centres"]
    dist = np.min(np.linalg.norm(p[:50, None, :] - cen[None], axis=-1), axis=1)
    assert np.allclose(c4.attributes[:50, -1], dist - 0.1, atol=1e-6)


def test_c5_stale_adjacency_rays_quantiles(c5):
    from sdfoam_amd import scenes

    # the adjacency is the Delaunay graph of the unperturbed points, so on
    # the perturbed ones it differs from a fresh triangulation
    adj, offs = scenes.delaunay_adjacency(c5.points)
    assert not (np.array_equal(adj, c5.adjacency) and np.array_equal(offs, c5.offsets))
    cams = c5.extra["cameras"]
    assert len(cams) == 64
    pos = np.stack([c.position for c in cams])
    assert np.allclose(np.linalg.norm(pos, axis=1), 4.0)
    assert abs(np.mean(pos[:, 2])) < 1e-9  # Fibonacci sphere: z symmetric
    R = c5.rays.shape[0]
    assert c5.rays.shape == (R, 6) and c5.quantiles.shape == (R, 2)
    assert np.all(c5.quantiles[:, 0] >= c5.quantiles[:, 1])
    # every ray starts at one of the camera centres
    o = c5.rays[:, :3].astype(np.float64)
    dmin = np.min(np.linalg.norm(o[:, None, :] - pos[None].astype(np.float32), axis=-1), axis=1)
    assert dmin.max() < 1e-6
    # step rays are reproducible and differ between steps
    r0, q0 = scenes.c5_step_rays(cams, 0, R)
    r1, _ = scenes.c5_step_rays(cams, 1, R)
    assert np.array_equal(r0, c5.rays) and np.array_equal(q0, c5.quantiles)
    assert not np.array_equal(r0, r1)
