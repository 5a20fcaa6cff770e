"""Synthetic scenes and rays in the reference's data formats.

The tracer consumes a point set in the order the reference's AABB builder
leaves it, a CSR Delaunay adjacency with ascending rows, an AoS attribute
table and pinhole rays.  This module produces all of them on the host with
numpy/scipy, for the bench and the tests:

* ``sort_points_order`` restates the reference's point sort
  (src/aabb_tree/aabb_tree.cu:62-190), including its whole-array passes.
* ``delaunay_adjacency`` builds the CSR ``point_adjacency`` /
  ``point_adjacency_offsets`` pair of src/delaunay/delaunay.cu:146-226 from a
  Qhull triangulation (scipy) instead of the reference's GPU Delaunay.
* ``look_at`` / ``pinhole_rays`` follow src/tracing/camera.h:56-85.
* ``make_config`` builds the workload configurations C1-C3 (seeded).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

SORT_BLOCK_SIZE = 1024  # src/aabb_tree/aabb_tree.cu:15


def pow2_round_up(x: int) -> int:
    """src/utils/typing.h:168-171."""
    return 1 if x <= 1 else 1 << int(x - 1).bit_length()


def _orderable_u32(points: np.ndarray) -> np.ndarray:
    """Float bits mapped to unsigned keys that sort like the floats
    (src/aabb_tree/aabb_tree.cu:85-94)."""
    u = np.ascontiguousarray(points, dtype=np.float32).view(np.uint32).copy()
    neg = (u & np.uint32(0x80000000)) != 0
    u[neg] = ~u[neg]
    u[~neg] ^= np.uint32(0x80000000)
    return u


def sort_points_order(points: np.ndarray) -> np.ndarray:
    """Permutation the reference's ``sort_points`` applies to a point set.

    src/aabb_tree/aabb_tree.cu:100-167: for segment sizes pow2(N), pow2(N)/2,
    ..., 2 it sorts by coordinate (0, 1, 2, 0, ...).  Segments larger than
    1024 with at most 1024 of them get one global radix sort over all points;
    more than 1024 such segments get a segmented sort; segments of at most
    1024 get a sort of each whole 1024-point block.  Radix sorts are stable,
    so each pass is a stable argsort over the stated ranges.
    Returns ``perm`` with ``sorted_points = points[perm]``.
    """
    n = int(points.shape[0])
    keys = _orderable_u32(points)  # [n, 3]
    perm = np.arange(n, dtype=np.int64)
    seg = pow2_round_up(n)
    dim = 0
    while seg > 1:
        nseg = (n + seg - 1) // seg
        k = keys[perm, dim]
        if seg > SORT_BLOCK_SIZE:
            if nseg > 1024:
                order = np.empty(n, dtype=np.int64)
                for s in range(nseg):
                    lo, hi = s * seg, min((s + 1) * seg, n)
                    order[lo:hi] = lo + np.argsort(k[lo:hi], kind="stable")
            else:
                order = np.argsort(k, kind="stable")
        else:
            # each whole 1024-point block sorted on its own (the last block
            # is partial; its padding keys sort after the real ones)
            blk = np.arange(n, dtype=np.uint64) // np.uint64(SORT_BLOCK_SIZE)
            comb = (blk << np.uint64(32)) | k.astype(np.uint64)
            order = np.argsort(comb, kind="stable")
        perm = perm[order]
        seg >>= 1
        dim = (dim + 1) % 3
    return perm


def _scene_blobs_shell(rng, n_blob: int, n_shell: int):
    """32 Gaussian blobs (centres uniform in the unit ball, sigma U(0.05, 0.2),
    samples outside r = 1 redrawn) plus a shell r in [1, 16] with density
    proportional to 1 / r^2 (r uniform) and uniform directions."""
    centres = np.empty((0, 3))
    while centres.shape[0] < 32:
        c = rng.uniform(-1.0, 1.0, size=(64, 3))
        centres = np.concatenate([centres, c[np.linalg.norm(c, axis=1) <= 1.0]])
    centres = centres[:32]
    sigma = rng.uniform(0.05, 0.2, size=32)
    counts = np.full(32, n_blob // 32)
    counts[: n_blob - counts.sum()] += 1
    blobs = []
    for c, sg, k in zip(centres, sigma, counts):
        got = np.empty((0, 3))
        while got.shape[0] < k:
            x = c + rng.normal(0.0, sg, size=(2 * (k - got.shape[0]) + 16, 3))
            got = np.concatenate([got, x[np.linalg.norm(x, axis=1) <= 1.0]])
        blobs.append(got[:k])
    d = rng.normal(size=(n_shell, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = rng.uniform(1.0, 16.0, size=(n_shell, 1))
    pts = np.concatenate(blobs + [d * r]).astype(np.float32)
    return pts, centres


def fibonacci_sphere(n: int, radius: float) -> np.ndarray:
    k = np.arange(n, dtype=np.float64)
    z = 1.0 - 2.0 * (k + 0.5) / n
    rxy = np.sqrt(1.0 - z * z)
    phi = k * math.pi * (3.0 - math.sqrt(5.0))
    return radius * np.stack([rxy * np.cos(phi), rxy * np.sin(phi), z], axis=1)


def delaunay_adjacency(points: np.ndarray, tetrahedra=None) -> tuple[np.ndarray, np.ndarray]:
    """CSR Delaunay adjacency with ascending rows.

    Edges of every tetrahedron, deduplicated, both directions, sorted by
    (row, neighbour): the layout of src/delaunay/delaunay.cu:146-226, where a
    stable sort by row leaves each row ascending.  `tetrahedra(points)` gives
    the tetrahedra [T, 4] (default: Qhull).
    """
    n = int(points.shape[0])
    if tetrahedra is None:
        from scipy.spatial import Delaunay

        s = Delaunay(np.asarray(points, dtype=np.float64)).simplices.astype(np.int64)
    else:
        s = np.asarray(tetrahedra(points), dtype=np.int64)
    pairs = np.concatenate(
        [s[:, [0, 1]], s[:, [0, 2]], s[:, [0, 3]], s[:, [1, 2]], s[:, [1, 3]], s[:, [2, 3]]]
    )
    a = np.minimum(pairs[:, 0], pairs[:, 1])
    b = np.maximum(pairs[:, 0], pairs[:, 1])
    key = np.unique((a << 32) | b)
    a = key >> 32
    b = key & 0xFFFFFFFF
    both = np.concatenate([(a << 32) | b, (b << 32) | a])
    both.sort()
    rows = both >> 32
    adj = (both & 0xFFFFFFFF).astype(np.uint32)
    counts = np.bincount(rows, minlength=n)
    offsets = np.zeros(n + 1, dtype=np.uint32)
    np.cumsum(counts, out=offsets[1:])
    return adj, offsets


@dataclass
class Camera:
    position: np.ndarray
    forward: np.ndarray
    right: np.ndarray
    up: np.ndarray
    fov: float  # vertical field of view, radians
    width: int
    height: int


def _normalize(v: np.ndarray) -> np.ndarray:
    return v / np.linalg.norm(v)


def look_at(position, target, up, fov: float, width: int, height: int) -> Camera:
    """src/tracing/camera.h:34-50."""
    position = np.asarray(position, dtype=np.float64)
    target = np.asarray(target, dtype=np.float64)
    up = np.asarray(up, dtype=np.float64)
    fwd = _normalize(target - position)
    right = _normalize(np.cross(fwd, up))
    cup = _normalize(np.cross(right, fwd))
    return Camera(position, fwd, right, cup, float(fov), int(width), int(height))


def camera_dict(cam: Camera, model: str = "pinhole", width: int | None = None,
                height: int | None = None, fov: float | None = None) -> dict:
    """The camera dict of ``Pipeline.trace_benchmark`` (benchmark.py:63-82 of
    the reference builds the same keys)."""
    return {
        "position": np.asarray(cam.position, dtype=np.float32),
        "forward": np.asarray(cam.forward, dtype=np.float32),
        "right": np.asarray(cam.right, dtype=np.float32),
        "up": np.asarray(cam.up, dtype=np.float32),
        "fov": float(cam.fov if fov is None else fov),
        "width": int(cam.width if width is None else width),
        "height": int(cam.height if height is None else height),
        "model": model,
    }


def default_up(position) -> np.ndarray:
    """World up is +z, or +y for a camera on the z axis."""
    p = np.asarray(position, dtype=np.float64)
    if abs(p[0]) < 1e-12 and abs(p[1]) < 1e-12:
        return np.array([0.0, 1.0, 0.0])
    return np.array([0.0, 0.0, 1.0])


def pinhole_rays(cam: Camera) -> np.ndarray:
    """Rays [H, W, 6] (origin, unit direction) of ``cast_ray`` for pixel
    (i, j) = (column, row), src/tracing/camera.h:56-85 (pinhole model)."""
    w, h = cam.width, cam.height
    aspect = w / h
    x = np.arange(w, dtype=np.float64) / w
    y = np.arange(h, dtype=np.float64) / h
    u = (2.0 * x - 1.0) * aspect
    v = 1.0 - 2.0 * y
    f = 1.0 / math.tan(cam.fov * 0.5)
    d = (
        f * cam.forward[None, None, :]
        + u[None, :, None] * cam.right[None, None, :]
        + v[:, None, None] * cam.up[None, None, :]
    )
    d /= np.linalg.norm(d, axis=-1, keepdims=True)
    rays = np.empty((h, w, 6), dtype=np.float32)
    rays[..., :3] = cam.position.astype(np.float32)
    rays[..., 3:] = d.astype(np.float32)
    return rays


def sh_dim(degree: int) -> int:
    return (degree + 1) ** 2


def attribute_dim(degree: int) -> int:
    """src/tracing/pipeline.cu:1467-1469."""
    return 1 + 3 * sh_dim(degree)


@dataclass
class Workload:
    name: str
    sh_degree: int
    points: np.ndarray  # [N, 3] f32, sort_points order
    attributes: np.ndarray  # [N, D] f32, last channel SDF (or density)
    adjacency: np.ndarray  # [E] u32
    offsets: np.ndarray  # [N+1] u32
    rays: np.ndarray  # [..., 6] f32
    quantiles: np.ndarray | None  # [..., Q] f32
    grad_rgba: np.ndarray | None  # [..., 4] f32
    depth_grad: np.ndarray | None  # [..., Q] f32
    inv_s: float
    alpha_mode: str = "sdfoam"
    extra: dict = field(default_factory=dict)

    @property
    def num_points(self) -> int:
        return int(self.points.shape[0])

    @property
    def num_rays(self) -> int:
        return int(np.prod(self.rays.shape[:-1]))


def _superquadric_F(p, e1, e2, abc):
    x = np.abs(p[:, 0] / abc[0])
    y = np.abs(p[:, 1] / abc[1])
    z = np.abs(p[:, 2] / abc[2])
    return (x ** (2.0 / e2) + y ** (2.0 / e2)) ** (e2 / e1) + z ** (2.0 / e1)


def _spow(w, m):
    return np.sign(w) * np.abs(w) ** m


def _scene_c1(rng):
    pts = rng.uniform(-1.0, 1.0, size=(4096, 3))
    corners = np.array([[sx, sy, sz] for sx in (-1, 1) for sy in (-1, 1) for sz in (-1, 1)], dtype=np.float64)
    return np.concatenate([pts, corners]).astype(np.float32)


def _scene_c2(rng):
    n_shell, n_box = 80_000, 20_000
    d = rng.normal(size=(n_shell, 3))
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    r = 0.5 + rng.normal(0.0, 0.02, size=(n_shell, 1))
    box = rng.uniform(-1.5, 1.5, size=(n_box, 3))
    return np.concatenate([d * r, box]).astype(np.float32)


def _scene_c3(rng):
    e1, e2 = rng.uniform(0.5, 2.0, size=2)
    abc = rng.uniform(0.4, 0.6, size=3)
    n_surf, n_box = 850_000, 150_000
    eta = rng.uniform(-math.pi / 2, math.pi / 2, size=n_surf)
    omega = rng.uniform(-math.pi, math.pi, size=n_surf)
    ce, se = np.cos(eta), np.sin(eta)
    surf = np.stack(
        [
            abc[0] * _spow(ce, e1) * _spow(np.cos(omega), e2),
            abc[1] * _spow(ce, e1) * _spow(np.sin(omega), e2),
            abc[2] * _spow(se, e1),
        ],
        axis=1,
    )
    surf += rng.normal(0.0, 0.01, size=surf.shape)
    box = rng.uniform(-1.0, 1.0, size=(n_box, 3))
    return np.concatenate([surf, box]).astype(np.float32), (e1, e2, abc)


def make_config(index: int, *, mode: str = "sdfoam", inv_s: float | None = None,
                image_scale: float = 1.0, point_scale: float = 1.0,
                sh_degree: int | None = None, tetrahedra=None) -> Workload:
    """Workload configuration C1-C5 (seed = config index).

    ``image_scale`` < 1 shrinks the image (same camera) for quick tests;
    ``point_scale`` < 1 shrinks the point counts of C4 / C5 (same proportions);
    ``sh_degree`` replaces the configuration's SH degree (C1-C3);
    ``tetrahedra(points)`` replaces Qhull for the adjacency (the bench passes the
    GPU tetrahedralisation).
    """
    rng = np.random.default_rng(index if index != 1 else 0)
    inv_s = math.exp(0.3) if inv_s is None else float(inv_s)
    if index == 1:
        pts = _scene_c1(rng)
        degree = 0
        cam_pos = np.array([0.0, 0.0, 3.0])
        fov, w, h = math.radians(50.0), 64, 64
    elif index == 2:
        pts = _scene_c2(rng)
        degree = 3
        th, ph = math.radians(60.0), math.radians(30.0)
        cam_pos = 3.0 * np.array([math.sin(th) * math.cos(ph), math.sin(th) * math.sin(ph), math.cos(th)])
        fov, w, h = math.radians(50.0), 400, 400
    elif index in (4, 5):
        return _make_blob_config(index, rng, mode, inv_s, image_scale, point_scale, tetrahedra)
    elif index == 3:
        pts, sq = _scene_c3(rng)
        degree = 3
        th, ph = math.radians(60.0), math.radians(30.0)
        cam_pos = 2.5 * np.array([math.sin(th) * math.cos(ph), math.sin(th) * math.sin(ph), math.cos(th)])
        fov, w, h = math.radians(40.0), 1600, 1200
    else:
        raise ValueError(f"unknown config {index}")
    if sh_degree is not None:
        degree = int(sh_degree)

    perm = sort_points_order(pts)
    pts = np.ascontiguousarray(pts[perm])
    n = pts.shape[0]
    D = attribute_dim(degree)
    attrs = np.empty((n, D), dtype=np.float32)
    if index == 1:
        attrs[:, : D - 1] = rng.uniform(0.0, 1.0, size=(n, D - 1))
    else:
        attrs[:, : D - 1] = rng.normal(0.0, 0.3, size=(n, D - 1))
    p64 = pts.astype(np.float64)
    radius = np.linalg.norm(p64, axis=1)
    if mode == "sdfoam":
        if index == 1:
            last = radius - 0.5
        elif index == 2:
            last = radius - 0.5 + rng.normal(0.0, 0.005, size=n)
        else:
            e1, e2, abc = sq
            F = _superquadric_F(p64, e1, e2, abc)
            last = radius * (1.0 - F ** (-e1 / 2.0))
    else:
        logit = rng.normal(0.0, 1.0, size=n)
        last = np.logaddexp(0.0, 10.0 * logit) / 10.0  # softplus, beta = 10
    attrs[:, D - 1] = last.astype(np.float32)

    adj, offs = delaunay_adjacency(pts, tetrahedra)

    if image_scale != 1.0:
        w = max(8, int(round(w * image_scale)))
        h = max(8, int(round(h * image_scale)))
    cam = look_at(cam_pos, np.zeros(3), default_up(cam_pos), fov, w, h)
    rays = pinhole_rays(cam)
    q = np.full(rays.shape[:-1] + (1,), 0.5, dtype=np.float32)
    grad_rgba = rng.normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    depth_grad = rng.normal(size=rays.shape[:-1] + (1,)).astype(np.float32)
    return Workload(
        name=f"C{index}",
        sh_degree=degree,
        points=pts,
        attributes=attrs,
        adjacency=adj,
        offsets=offs,
        rays=rays,
        quantiles=q,
        grad_rgba=grad_rgba,
        depth_grad=depth_grad,
        inv_s=inv_s,
        alpha_mode=mode,
        extra={"camera": cam, "permutation": perm},
    )


def _make_blob_config(index: int, rng, mode: str, inv_s: float, image_scale: float,
                      point_scale: float = 1.0, tetrahedra=None) -> Workload:
    """C4 (3M points, 8 ring cameras 1297x840, Q = 1) and C5 (2M points with
    positions perturbed N(0, 0.001) after the adjacency is built, rays of
    step 0: 2^20 (camera, pixel) samples over 64 cameras 960x640, Q = 2
    descending quantiles).  SH degree 3, coefficients N(0, 0.3); SDF =
    distance to the nearest blob centre - 0.1 (density: softplus of a
    N(0, 1) logit)."""
    degree = 3
    n_blob, n_shell = (1_800_000, 1_200_000) if index == 4 else (1_200_000, 800_000)
    pts, centres = _scene_blobs_shell(rng, int(n_blob * point_scale), int(n_shell * point_scale))
    perm = sort_points_order(pts)
    pts = np.ascontiguousarray(pts[perm])
    n = pts.shape[0]
    D = attribute_dim(degree)
    attrs = np.empty((n, D), dtype=np.float32)
    attrs[:, : D - 1] = rng.normal(0.0, 0.3, size=(n, D - 1))
    if mode == "sdfoam":
        from scipy.spatial import cKDTree

        dist, _ = cKDTree(centres).query(pts.astype(np.float64))
        last = dist - 0.1
    else:
        last = np.logaddexp(0.0, 10.0 * rng.normal(0.0, 1.0, size=n)) / 10.0
    attrs[:, D - 1] = last.astype(np.float32)
    adj, offs = delaunay_adjacency(pts, tetrahedra)
    extra = {"permutation": perm, "centres": centres}
    if index == 4:
        w, h = 1297, 840
        if image_scale != 1.0:
            w = max(8, int(round(w * image_scale)))
            h = max(8, int(round(h * image_scale)))
        cams = []
        for k in range(8):
            a = 2.0 * math.pi * k / 8
            pos = 4.0 * np.array([math.cos(a), math.sin(a), 0.0])
            cams.append(look_at(pos, np.zeros(3), default_up(pos), math.radians(50.0), w, h))
        rays = np.stack([pinhole_rays(c) for c in cams])  # [8, H, W, 6]
        q = np.full(rays.shape[:-1] + (1,), 0.5, dtype=np.float32)
        extra["cameras"] = cams
        extra["camera"] = cams[0]
    else:
        # stale adjacency: the training loop moves points between rebuilds
        pts = (pts.astype(np.float64) + rng.normal(0.0, 1e-3, size=pts.shape)).astype(np.float32)
        w, h = 960, 640
        if image_scale != 1.0:
            w = max(8, int(round(w * image_scale)))
            h = max(8, int(round(h * image_scale)))
        cams = [look_at(p, np.zeros(3), default_up(p), math.radians(50.0), w, h)
                for p in fibonacci_sphere(64, 4.0)]
        extra["cameras"] = cams
        extra["camera"] = cams[0]
        rays, q = c5_step_rays(cams, 0, max(1024, int((1 << 20) * point_scale)))
    grad_rgba = rng.normal(size=rays.shape[:-1] + (4,)).astype(np.float32)
    depth_grad = rng.normal(size=rays.shape[:-1] + (q.shape[-1],)).astype(np.float32)
    return Workload(
        name=f"C{index}", sh_degree=degree, points=pts, attributes=attrs, adjacency=adj,
        offsets=offs, rays=rays, quantiles=q, grad_rgba=grad_rgba, depth_grad=depth_grad,
        inv_s=inv_s, alpha_mode=mode, extra=extra)


def c5_step_rays(cams, step: int, num_rays: int) -> tuple[np.ndarray, np.ndarray]:
    """Rays of training step `step`: rng(5000 + step) draws (camera, pixel)
    pairs uniformly with replacement (as src/utils/batch_fetcher.cpp:66-69
    draws random rays), and two quantiles U(0, 1) sorted descending
    (train.py:259-261).  Returns rays [R, 6] and quantiles [R, 2]."""
    rng = np.random.default_rng(5000 + step)
    ncam = len(cams)
    w, h = cams[0].width, cams[0].height
    ci = rng.integers(0, ncam, size=num_rays)
    px = rng.integers(0, w * h, size=num_rays)
    i = (px % w).astype(np.float64)
    j = (px // w).astype(np.float64)
    pos = np.stack([c.position for c in cams])
    fw = np.stack([c.forward for c in cams])
    rt = np.stack([c.right for c in cams])
    up = np.stack([c.up for c in cams])
    f = np.array([1.0 / math.tan(c.fov * 0.5) for c in cams])
    u = (2.0 * i / w - 1.0) * (w / h)
    v = 1.0 - 2.0 * j / h
    d = f[ci, None] * fw[ci] + u[:, None] * rt[ci] + v[:, None] * up[ci]
    d /= np.linalg.norm(d, axis=1, keepdims=True)
    rays = np.empty((num_rays, 6), dtype=np.float32)
    rays[:, :3] = pos[ci]
    rays[:, 3:] = d
    q = -np.sort(-rng.uniform(0.0, 1.0, size=(num_rays, 2)), axis=1)
    return rays, q.astype(np.float32)


def save_workload(w: Workload, path: str) -> None:
    """Write a workload to an .npz file (arrays only; no pickled objects)."""
    cams = w.extra.get("cameras") or ([w.extra["camera"]] if "camera" in w.extra else [])
    cam_arrays = {}
    if cams:
        cam_arrays = dict(
            cam_position=np.stack([c.position for c in cams]),
            cam_forward=np.stack([c.forward for c in cams]),
            cam_right=np.stack([c.right for c in cams]),
            cam_up=np.stack([c.up for c in cams]),
            cam_fov=np.array([c.fov for c in cams]),
            cam_size=np.array([[c.width, c.height] for c in cams]),
        )
    np.savez(
        path, name=np.array(w.name), sh_degree=np.array(w.sh_degree), points=w.points,
        attributes=w.attributes, adjacency=w.adjacency, offsets=w.offsets, rays=w.rays,
        quantiles=w.quantiles, grad_rgba=w.grad_rgba, depth_grad=w.depth_grad,
        inv_s=np.array(w.inv_s), alpha_mode=np.array(w.alpha_mode), **cam_arrays,
    )


def load_workload(path: str) -> Workload:
    """Read a workload written by save_workload (allow_pickle stays off)."""
    z = np.load(path)
    extra = {}
    if "cam_position" in z.files:
        cams = [Camera(z["cam_position"][k], z["cam_forward"][k], z["cam_right"][k],
                       z["cam_up"][k], float(z["cam_fov"][k]), int(z["cam_size"][k][0]),
                       int(z["cam_size"][k][1]))
                for k in range(z["cam_position"].shape[0])]
        extra = {"cameras": cams, "camera": cams[0]}
    return Workload(
        name=str(z["name"]), sh_degree=int(z["sh_degree"]), points=z["points"],
        attributes=z["attributes"], adjacency=z["adjacency"], offsets=z["offsets"],
        rays=z["rays"], quantiles=z["quantiles"], grad_rgba=z["grad_rgba"],
        depth_grad=z["depth_grad"], inv_s=float(z["inv_s"]), alpha_mode=str(z["alpha_mode"]),
        extra=extra,
    )


def nearest_point_bruteforce(points: np.ndarray, queries: np.ndarray) -> np.ndarray:
    """Exact nearest neighbour by float32 distance (host helper for building
    start points; ties go to the smallest index)."""
    p = np.asarray(points, dtype=np.float32)
    out = np.empty(queries.shape[0], dtype=np.uint32)
    for i, q in enumerate(np.asarray(queries, dtype=np.float32)):
        d = p - q
        dist = np.sqrt(d[:, 0] * d[:, 0] + (d[:, 1] * d[:, 1] + d[:, 2] * d[:, 2]))
        out[i] = np.argmin(dist)
    return out


def start_points_for(points: np.ndarray, rays: np.ndarray) -> np.ndarray:
    """Start cell of every ray: the nearest point to its origin, looked up once
    per distinct origin (the scheme of sdfoam_model/scene.py:272-282)."""
    flat = rays.reshape(-1, 6)[:, :3]
    uniq, inv = np.unique(flat, axis=0, return_inverse=True)
    nn = nearest_point_bruteforce(points, uniq)
    return nn[inv.reshape(-1)].reshape(rays.shape[:-1]).astype(np.uint32)
