"""TEST INFRASTRUCTURE -- NOT PART OF THE PRODUCT.

ctypes wrapper around the scalar host oracle (oracle/libsdf_oracle.so).
Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg import
this module, and only as the checker.  The oracle restates the reference's
algorithm (file:line at every function in sdf_oracle.c).
"""

from __future__ import annotations

import ctypes as C
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsdf_oracle.so")

ALPHA_STANDARD = 0
ALPHA_NEUS = 1


def build() -> str:
    """Compile the oracle with its Makefile (gcc)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


class _Settings(C.Structure):
    _fields_ = [
        ("weight_threshold", C.c_float),
        ("max_intersections", C.c_uint32),
        ("alpha_mode", C.c_uint32),
        ("sdf_channel", C.c_int32),
    ]


class _Visits(C.Structure):
    _fields_ = [
        ("hash", C.c_void_p),
        ("cells", C.c_void_p),
        ("alphas", C.c_void_p),
        ("stride", C.c_uint32),
        ("steps", C.c_void_p),
        ("faces", C.c_void_p),
        ("faces_stepped", C.c_void_p),
        ("t_exit", C.c_void_p),
        ("point_visits", C.c_void_p),
    ]


class _Grads(C.Structure):
    _fields_ = [
        ("points_grad", C.c_void_p),
        ("attr_grad", C.c_void_p),
        ("sharpness_grad", C.c_void_p),
        ("point_error", C.c_void_p),
        ("points_grad_abs", C.c_void_p),
        ("attr_grad_abs", C.c_void_p),
        ("sharpness_abs", C.c_void_p),
        ("points_grad_k", C.c_void_p),
        ("attr_grad_k", C.c_void_p),
        ("sharpness_k", C.c_void_p),
    ]


class _Camera(C.Structure):
    _fields_ = [
        ("position", C.c_float * 3),
        ("forward", C.c_float * 3),
        ("right", C.c_float * 3),
        ("up", C.c_float * 3),
        ("fov", C.c_float),
        ("width", C.c_uint32),
        ("height", C.c_uint32),
        ("model", C.c_uint32),
    ]


def make_camera(cam: dict) -> _Camera:
    """camera dict of Pipeline.trace_benchmark (position, forward, right, up,
    fov, width, height, model 'pinhole' | 'fisheye')."""
    model = {"pinhole": 0, "fisheye": 1}[cam.get("model", "pinhole")]
    vec = [np.asarray(cam[k], dtype=np.float32).reshape(3) for k in ("position", "forward", "right", "up")]
    return _Camera(*[(C.c_float * 3)(*v.tolist()) for v in vec], float(cam["fov"]),
                   int(cam["width"]), int(cam["height"]), model)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.oracle_expf.restype = C.c_float
        L.oracle_expf.argtypes = [C.c_float]
        L.oracle_sigmoidf.restype = C.c_float
        L.oracle_sigmoidf.argtypes = [C.c_float]
        L.oracle_f32_to_f16.restype = C.c_uint16
        L.oracle_f32_to_f16.argtypes = [C.c_float]
        L.oracle_f16_to_f32.restype = C.c_float
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_expf_n.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        L.oracle_f32_to_f16_n.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64]
        L.oracle_sh_basis.argtypes = [C.c_uint32, C.c_float, C.c_float, C.c_float, C.c_void_p]
        L.oracle_prefetch_adjacent_diff.argtypes = [
            C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]
        L.oracle_trace_forward.restype = C.c_int
        L.oracle_trace_forward.argtypes = [
            C.POINTER(_Settings), C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
            C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
            C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(_Visits), C.c_int]
        L.oracle_trace_backward.restype = C.c_int
        L.oracle_trace_backward.argtypes = [
            C.POINTER(_Settings), C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
            C.c_uint32, C.c_void_p, C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
            C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
            C.c_void_p, C.c_void_p, C.POINTER(_Grads), C.POINTER(_Visits), C.c_int]
        L.oracle_cell_intersection_grad.argtypes = [C.c_void_p] * 5
        L.oracle_build_aabb_tree.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p]
        L.oracle_nn.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p, C.c_int]
        L.oracle_trace_benchmark.restype = C.c_int
        L.oracle_trace_benchmark.argtypes = [
            C.POINTER(_Settings), C.c_uint32, C.c_uint32, C.c_void_p, C.c_void_p,
            C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.POINTER(_Camera), C.c_uint32,
            C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]
        L.oracle_camera_focal.restype = C.c_float
        L.oracle_camera_focal.argtypes = [C.c_float]
        L.oracle_cast_ray.argtypes = [C.POINTER(_Camera), C.c_uint32, C.c_uint32, C.c_void_p]
        L.oracle_sincosf_n.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64]
        L.oracle_atan2f_n.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64]
        L.oracle_farthest_neighbor.argtypes = [C.c_void_p, C.c_uint32, C.c_void_p, C.c_void_p,
                                               C.c_void_p, C.c_void_p]
        L.oracle_make_rgba8.restype = C.c_uint32
        L.oracle_make_rgba8.argtypes = [C.c_float] * 4
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return None if a is None else np.ascontiguousarray(a, dtype=dtype)


def expf(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    y = np.empty_like(x)
    lib().oracle_expf_n(_p(x), _p(y), x.size)
    return y


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    x = _c(x, np.float32).ravel()
    y = np.empty(x.size, dtype=np.uint16)
    lib().oracle_f32_to_f16_n(_p(x), _p(y), x.size)
    return y


def sh_basis(degree: int, d) -> np.ndarray:
    out = np.zeros(16, dtype=np.float32)
    lib().oracle_sh_basis(degree, float(d[0]), float(d[1]), float(d[2]), _p(out))
    return out


def prefetch_adjacent_diff(points, adjacency, offsets) -> np.ndarray:
    points = _c(points, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    out = np.zeros((adjacency.size, 4), dtype=np.uint16)
    lib().oracle_prefetch_adjacent_diff(_p(points), points.shape[0], adjacency.size,
                                        _p(adjacency), _p(offsets), _p(out))
    return out


def cell_intersection_grad(p, q, o, d) -> np.ndarray:
    args = [np.ascontiguousarray(v, dtype=np.float32) for v in (p, q, o, d)]
    g = np.zeros(3, dtype=np.float32)
    lib().oracle_cell_intersection_grad(*[_p(a) for a in args], _p(g))
    return g


def build_aabb_tree(points) -> np.ndarray:
    from sdfoam_amd.scenes import pow2_round_up

    points = _c(points, np.float32)
    n2 = pow2_round_up(points.shape[0])
    tree = np.zeros((n2, 2, 3), dtype=np.float32)
    lib().oracle_build_aabb_tree(_p(points), points.shape[0], _p(tree))
    return tree


def nn(points, queries, threads: int = 1) -> np.ndarray:
    points = _c(points, np.float32)
    q = _c(queries, np.float32).reshape(-1, 3)
    out = np.zeros(q.shape[0], dtype=np.uint32)
    lib().oracle_nn(_p(points), points.shape[0], _p(q), q.shape[0], _p(out), threads)
    return out.reshape(np.shape(queries)[:-1])


@dataclass
class ForwardResult:
    rgba: np.ndarray
    depth: np.ndarray | None
    depth_indices: np.ndarray | None
    num_intersections: np.ndarray
    contribution: np.ndarray | None
    alpha: np.ndarray
    visit_hash: np.ndarray
    steps: np.ndarray
    faces: np.ndarray
    faces_stepped: np.ndarray
    cells: np.ndarray | None
    cell_alphas: np.ndarray | None
    t_exit: np.ndarray | None
    point_visits: np.ndarray | None = None  # [N] u32: steps into each point


def _settings(alpha_mode, weight_threshold, max_intersections, sdf_channel, D):
    mode = ALPHA_NEUS if str(alpha_mode).lower() in ("sdfoam", "sdf", "alpha_neus") else ALPHA_STANDARD
    if sdf_channel is None:
        sdf_channel = D - 1 if mode == ALPHA_NEUS else -1
    return _Settings(
        1e-7 if weight_threshold is None else float(weight_threshold),
        1024 if max_intersections is None else int(max_intersections),
        mode,
        int(sdf_channel),
    ), mode


def trace_forward(sh_degree, points, attributes, adjacency, offsets, rays, start_point,
                  depth_quantiles=None, *, alpha_mode="sdfoam", inv_s=1.0,
                  weight_threshold=None, max_intersections=None, sdf_channel=None,
                  return_contribution=True, record=0, threads=1,
                  point_visits=False) -> ForwardResult:
    """point_visits=True also counts each point's cell steps over all rays
    (`ForwardResult.point_visits`: the number K of terms of its contribution
    sum, for the summation bound of the parity tests)."""
    points = _c(points, np.float32)
    attributes = _c(attributes, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    lead = rays.shape[:-1]
    rays = _c(rays, np.float32).reshape(-1, 6)
    start = _c(start_point, np.uint32).ravel()
    R = rays.shape[0]
    N = points.shape[0]
    D = attributes.shape[-1]
    st, _ = _settings(alpha_mode, weight_threshold, max_intersections, sdf_channel, D)
    Q = 0 if depth_quantiles is None else int(depth_quantiles.shape[-1])
    quant = None if depth_quantiles is None else _c(depth_quantiles, np.float32).reshape(R, Q)
    sharp = np.array([inv_s], dtype=np.float32).ravel()[:1] if np.ndim(inv_s) == 0 else _c(inv_s, np.float32).ravel()
    rgba = np.zeros((R, 4), dtype=np.float32)
    depth = np.zeros((R, Q), dtype=np.float32) if Q else None
    didx = np.zeros((R, Q), dtype=np.uint32) if Q else None
    nisect = np.zeros(R, dtype=np.uint32)
    contrib = np.zeros(N, dtype=np.float64) if return_contribution else None
    alpha = np.zeros(N, dtype=np.float32)
    vh = np.zeros(R, dtype=np.uint64)
    steps = np.zeros(R, dtype=np.uint32)
    faces = np.zeros(R, dtype=np.uint64)
    faces_st = np.zeros(R, dtype=np.uint64)
    cells = np.zeros((R, record), dtype=np.uint32) if record else None
    calpha = np.zeros((R, record), dtype=np.float32) if record else None
    texit = np.zeros((R, record), dtype=np.float32) if record else None
    pvis = np.zeros(N, dtype=np.uint32) if point_visits else None
    vis = _Visits(_p(vh), _p(cells), _p(calpha), record, _p(steps), _p(faces), _p(faces_st),
                  _p(texit), _p(pvis))
    rc = lib().oracle_trace_forward(
        C.byref(st), sh_degree, N, _p(points), _p(attributes), adjacency.size, _p(adjacency),
        _p(offsets), R, _p(rays), _p(start), Q, _p(quant), _p(sharp), _p(rgba), _p(depth),
        _p(didx), _p(nisect), _p(contrib), _p(alpha), C.byref(vis), threads)
    if rc != 0:
        raise RuntimeError("oracle_trace_forward failed")
    return ForwardResult(
        rgba.reshape(lead + (4,)),
        None if depth is None else depth.reshape(lead + (Q,)),
        None if didx is None else didx.reshape(lead + (Q,)),
        nisect.reshape(lead + (1,)),
        None if contrib is None else contrib.reshape(N, 1),
        alpha.reshape(N, 1),
        vh.reshape(lead), steps.reshape(lead), faces.reshape(lead), faces_st.reshape(lead),
        cells, calpha, texit, pvis)


@dataclass
class BackwardResult:
    points_grad: np.ndarray
    attr_grad: np.ndarray
    sharpness_grad: float
    point_error: np.ndarray | None
    points_grad_abs: np.ndarray
    attr_grad_abs: np.ndarray
    sharpness_abs: float
    points_grad_k: np.ndarray
    attr_grad_k: np.ndarray
    sharpness_k: int
    visit_hash: np.ndarray
    steps: np.ndarray


def trace_backward(sh_degree, points, attributes, adjacency, offsets, rays, start_point,
                   rgba, grad_rgba, depth_quantiles=None, depth_indices=None, depth_grad=None,
                   ray_error=None, *, alpha_mode="sdfoam", inv_s=1.0, weight_threshold=None,
                   max_intersections=None, sdf_channel=None, threads=1,
                   side_buffers=True) -> BackwardResult:
    """side_buffers=False skips the sum|c| / count buffers of the tolerance
    model (the plain algorithm, as timed for the CPU baseline)."""
    points = _c(points, np.float32)
    attributes = _c(attributes, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    lead = rays.shape[:-1]
    rays = _c(rays, np.float32).reshape(-1, 6)
    start = _c(start_point, np.uint32).ravel()
    R = rays.shape[0]
    N = points.shape[0]
    D = attributes.shape[-1]
    st, _ = _settings(alpha_mode, weight_threshold, max_intersections, sdf_channel, D)
    Q = 0 if depth_quantiles is None else int(depth_quantiles.shape[-1])
    quant = None if depth_quantiles is None else _c(depth_quantiles, np.float32).reshape(R, Q)
    didx = None if depth_indices is None else _c(depth_indices, np.uint32).reshape(R, -1)
    dgrad = None if depth_grad is None else _c(depth_grad, np.float32).reshape(R, -1)
    rgba = _c(rgba, np.float32).reshape(R, 4)
    grad_rgba = _c(grad_rgba, np.float32).reshape(R, 4)
    rerr = None if ray_error is None else _c(ray_error, np.float32).ravel()
    sharp = np.array([inv_s], dtype=np.float32).ravel()[:1] if np.ndim(inv_s) == 0 else _c(inv_s, np.float32).ravel()
    pg = np.zeros((N, 3)); ag = np.zeros((N, D)); sg = np.zeros(1)
    pe = np.zeros(N) if rerr is not None else None
    if side_buffers:
        pga = np.zeros((N, 3)); aga = np.zeros((N, D)); sga = np.zeros(1)
        pgk = np.zeros((N, 3), dtype=np.uint32); agk = np.zeros((N, D), dtype=np.uint32)
        sgk = np.zeros(1, dtype=np.uint64)
    else:
        pga = aga = sga = pgk = agk = sgk = None
    g = _Grads(_p(pg), _p(ag), _p(sg), _p(pe), _p(pga), _p(aga), _p(sga), _p(pgk), _p(agk), _p(sgk))
    vh = np.zeros(R, dtype=np.uint64)
    steps = np.zeros(R, dtype=np.uint32)
    vis = _Visits(_p(vh), None, None, 0, _p(steps), None, None, None, None)
    rc = lib().oracle_trace_backward(
        C.byref(st), sh_degree, N, _p(points), _p(attributes), adjacency.size, _p(adjacency),
        _p(offsets), R, _p(rays), _p(start), Q, _p(quant), _p(didx), _p(rgba), _p(grad_rgba),
        _p(dgrad), _p(rerr), _p(sharp), C.byref(g), C.byref(vis), threads)
    if rc != 0:
        raise RuntimeError("oracle_trace_backward failed")
    return BackwardResult(pg, ag, float(sg[0]), None if pe is None else pe.reshape(N, 1),
                          pga, aga, None if sga is None else float(sga[0]), pgk, agk,
                          None if sgk is None else int(sgk[0]),
                          vh.reshape(lead), steps.reshape(lead))


def sincosf(x):
    x = _c(x, np.float32).ravel()
    sn = np.empty_like(x)
    cs = np.empty_like(x)
    lib().oracle_sincosf_n(_p(x), _p(sn), _p(cs), x.size)
    return sn, cs


def atan2f(y, x):
    y = _c(y, np.float32).ravel()
    x = _c(x, np.float32).ravel()
    out = np.empty_like(x)
    lib().oracle_atan2f_n(_p(y), _p(x), _p(out), x.size)
    return out


def make_rgba8(r, g, b, a) -> int:
    return int(lib().oracle_make_rgba8(float(r), float(g), float(b), float(a)))


def cast_ray(cam: dict, i: int, j: int) -> np.ndarray:
    d = np.zeros(3, dtype=np.float32)
    c = make_camera(cam)
    lib().oracle_cast_ray(C.byref(c), i, j, _p(d))
    return d


@dataclass
class RenderResult:
    rgba8: np.ndarray            # [H, W] uint32, row H-1-j holds pixel row j
    rgbt: np.ndarray             # [H*W, 4]: C, T per pixel (j * W + i); -1 where masked
    num_intersections: np.ndarray  # [H*W]


def trace_benchmark(sh_degree, points, attributes, adjacency, offsets, adjacent_diff, camera,
                    start_point, *, alpha_mode="sdfoam", inv_s=1.0, weight_threshold=None,
                    max_intersections=None, sdf_channel=None, bg_color=None, checker_bg=False,
                    threads=1) -> RenderResult:
    points = _c(points, np.float32)
    attributes = _c(attributes, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    diff = _c(adjacent_diff, np.uint16).reshape(-1, 4)
    if diff.shape[0] < adjacency.size:
        raise ValueError("adjacent_diff must have one row per adjacency entry")
    D = attributes.shape[-1]
    st, _ = _settings(alpha_mode, weight_threshold, max_intersections, sdf_channel, D)
    sharp = np.array([inv_s], dtype=np.float32).ravel()[:1] if np.ndim(inv_s) == 0 else _c(inv_s, np.float32).ravel()
    cam = make_camera(camera)
    W, H = cam.width, cam.height
    out = np.zeros((H, W), dtype=np.uint32)
    rgbt = np.zeros((H * W, 4), dtype=np.float32)
    nis = np.zeros(H * W, dtype=np.uint32)
    bg = None if bg_color is None else _c(bg_color, np.float32).ravel()
    rc = lib().oracle_trace_benchmark(
        C.byref(st), sh_degree, points.shape[0], _p(points), _p(attributes), adjacency.size,
        _p(adjacency), _p(offsets), _p(diff), C.byref(cam), int(np.asarray(start_point).ravel()[0]),
        _p(sharp), _p(bg), int(bool(checker_bg)), _p(out), _p(rgbt), _p(nis), threads)
    if rc != 0:
        raise RuntimeError("oracle_trace_benchmark failed")
    return RenderResult(out, rgbt, nis)


# ---------------------------------------------------------------------------
# BatchFetcher row selection (src/utils/batch_fetcher.cpp:63-72 with the RNG
# of src/utils/random.h:11-56), restated with numpy uint32 arithmetic.

def _mix32(x: np.ndarray) -> np.ndarray:
    """The reference's 32-bit integer hash (src/utils/random.h:11-20,
    C. Wellons' hash-prospector "triple32").  Pinned by the inverse that
    hash-prospector publishes beside it (other multipliers: the inverses of
    these modulo 2^32): composed with it the hash gives back every input
    tried, which a multiplier or shift off by one step does not.  The
    reference's header itself cannot be built here (it includes
    cuda_fp16.h)."""
    x = x.astype(np.uint32)
    with np.errstate(over="ignore"):
        x ^= x >> np.uint32(17)
        x *= np.uint32(0xED5AD4BB)
        x ^= x >> np.uint32(11)
        x *= np.uint32(0xAC4C1B51)
        x ^= x >> np.uint32(15)
        x *= np.uint32(0x31848BAB)
        x ^= x >> np.uint32(14)
    return x


def batch_rows(batch_index: int, batch_size: int, num_rows: int, shuffle: bool) -> np.ndarray:
    """Rows of batch `batch_index`: element j uses the first draw of
    make_rng(batch_index * batch_size + j) scaled by randint(rng, 0, n), or
    row (batch_index * batch_size + j) mod n without shuffling."""
    k = np.uint64(batch_index) * np.uint64(batch_size) + np.arange(batch_size, dtype=np.uint64)
    if not shuffle:
        return (k % np.uint64(num_rows)).astype(np.uint32)
    seed = (k & np.uint64(0xFFFFFFFF)).astype(np.uint32)
    draw = _mix32(seed ^ np.uint32(0x2815DB5B))
    diff = np.uint32(num_rows)
    x = draw // (np.uint32(0xFFFFFFFF) // diff)
    return np.minimum(x, diff - np.uint32(1)).astype(np.uint32)


def farthest_neighbor(points, adjacency, offsets):
    points = _c(points, np.float32)
    adjacency = _c(adjacency, np.uint32)
    offsets = _c(offsets, np.uint32)
    n = points.shape[0]
    idx = np.zeros(n, dtype=np.uint32)
    rad = np.zeros(n, dtype=np.float32)
    lib().oracle_farthest_neighbor(_p(points), n, _p(adjacency), _p(offsets), _p(idx), _p(rad))
    return idx, rad
