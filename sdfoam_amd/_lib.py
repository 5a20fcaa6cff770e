"""ctypes binding of libsdfoam_hip.so (the C ABI in include/sdfoam_hip.h).

The library is built in-tree by ``python -m sdfoam_amd.build``.  There is no
fallback: if it is missing, loading raises.
"""

from __future__ import annotations

import ctypes as C
import os

from .build import LIB_PATH

SDF_OK = 0
SDF_E_INVALID = 1
SDF_E_HIP = 2
SDF_ALPHA_STANDARD = 0
SDF_ALPHA_NEUS = 1
SDF_ATTR_F32 = 0
SDF_ATTR_F16 = 1

# every symbol include/sdfoam_hip.h declares
EXPORTS = (
    "sdf_version",
    "sdf_last_error",
    "sdf_attribute_dim",
    "sdf_trace_scratch_bytes",
    "sdf_prefetch_adjacent_diff",
    "sdf_trace_forward",
    "sdf_trace_forward_noalloc",
    "sdf_trace_backward",
    "sdf_trace_benchmark",
    "sdf_walk_record_bytes",
    "sdf_walk_record_pool_bytes",
    "sdf_walk_record_full_chunks",
    "sdf_grad_accum_bytes",
    "sdf_cell_table_bytes",
    "sdf_start_points_scratch_bytes",
    "sdf_start_points",
    "sdf_ray_order_scratch_bytes",
    "sdf_ray_order",
    "sdf_trace_forward_planned",
    "sdf_trace_backward_planned",
    "sdf_batch_fetcher_ring_bytes",
    "sdf_batch_fetcher_create",
    "sdf_batch_fetcher_next",
    "sdf_batch_fetcher_destroy",
    "sdf_batch_rows",
    "sdf_batch_gather",
    "sdf_build_aabb_tree",
    "sdf_farthest_neighbor",
    "sdf_sort_points_scratch_bytes",
    "sdf_sort_points",
    "sdf_delaunay_adjacency_capacity",
    "sdf_delaunay_tables_scratch_bytes",
    "sdf_delaunay_tables",
    "sdf_delaunay_certify_scratch_bytes",
    "sdf_delaunay_certify",
    "sdf_delaunay_certify_exhaustive",
    "sdf_delaunay_merge_scratch_bytes",
    "sdf_delaunay_merge",
    "sdf_delaunay_check",
    "sdf_delaunay_certify_points",
    "sdf_delaunay_merge_verified",
    "sdf_nn",
    "sdf_trace_walk_stats",
    "sdf_debug_fpmath",
    "sdf_set_timing",
    "sdf_timing_collect",
)

KERNEL_NAMES = {0: "prefetch_adjacent_diff", 1: "forward", 2: "backward", 3: "build_aabb_tree", 4: "nn",
                5: "render", 6: "ray_order", 7: "grad_clear", 8: "grad_finalize", 9: "scene_prep"}

SDF_CAMERA_PINHOLE = 0
SDF_CAMERA_FISHEYE = 1


class TraceSettings(C.Structure):
    """sdf_trace_settings (mirrors the fields of the reference's TraceSettings
    that its kernels read, src/tracing/pipeline.h:12-27)."""

    _fields_ = [
        ("weight_threshold", C.c_float),
        ("max_intersections", C.c_uint32),
        ("alpha_mode", C.c_uint32),
        ("sdf_channel", C.c_int32),
        ("ray_image_width", C.c_uint32),
        ("attr_type", C.c_uint32),
    ]


class Camera(C.Structure):
    """sdf_camera (src/tracing/camera.h:17-27)."""

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


class Visualization(C.Structure):
    """sdf_visualization (src/tracing/pipeline.h:50-68)."""

    _fields_ = [("bg_color", C.c_float * 3), ("checker_bg", C.c_int32)]


class TracePlanDesc(C.Structure):
    """sdf_trace_plan: the forward's walk record, the rays' launch order,
    the backward's gradient accumulator and the forward's cell table."""

    _fields_ = [
        ("walk_record", C.c_void_p),
        ("walk_record_bytes", C.c_size_t),
        ("walk_budget", C.c_uint32),
        ("ray_order", C.c_void_p),
        ("grad_accum", C.c_void_p),
        ("grad_accum_bytes", C.c_size_t),
        ("scratch_ready", C.c_uint32),
        ("cell_table", C.c_void_p),
        ("cell_table_bytes", C.c_size_t),
        ("walk_record_chunks", C.c_uint32),
    ]


_lib = None

P = C.c_void_p
U32 = C.c_uint32
SZ = C.c_size_t


class LibraryError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load libsdfoam_hip.so (once)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryError(
            f"{LIB_PATH} is not built; run `python -m sdfoam_amd.build` "
            "(the HIP library is required, there is no CPU fallback)"
        )
    L = C.CDLL(LIB_PATH)
    L.sdf_version.restype = C.c_char_p
    L.sdf_version.argtypes = []
    L.sdf_last_error.restype = C.c_char_p
    L.sdf_last_error.argtypes = []
    L.sdf_attribute_dim.restype = C.c_int
    L.sdf_attribute_dim.argtypes = [C.c_int]
    L.sdf_trace_scratch_bytes.restype = SZ
    L.sdf_trace_scratch_bytes.argtypes = [U32, U32]
    L.sdf_prefetch_adjacent_diff.restype = C.c_int
    L.sdf_prefetch_adjacent_diff.argtypes = [P, U32, U32, P, P, P, P]
    L.sdf_trace_forward.restype = C.c_int
    L.sdf_trace_forward.argtypes = [
        C.c_int, C.POINTER(TraceSettings), U32, P, P, U32, P, P, U32, P, P, U32, P,
        P, P, P, P, P, P, P, P, SZ, P]
    L.sdf_trace_forward_noalloc.restype = C.c_int
    L.sdf_trace_forward_noalloc.argtypes = L.sdf_trace_forward.argtypes[:-3] + [P]
    L.sdf_trace_backward.restype = C.c_int
    L.sdf_trace_backward.argtypes = [
        C.c_int, C.POINTER(TraceSettings), U32, P, P, U32, P, P, U32, P, P, U32, P, P,
        P, P, P, P, P, P, P, P, P, P, SZ, P]
    L.sdf_trace_benchmark.restype = C.c_int
    L.sdf_trace_benchmark.argtypes = [
        C.c_int, C.POINTER(TraceSettings), U32, P, P, U32, P, P, P, SZ, C.POINTER(Camera),
        C.POINTER(Visualization), P, P, P, P]
    L.sdf_walk_record_bytes.restype = SZ
    L.sdf_walk_record_bytes.argtypes = [U32, U32, U32]
    L.sdf_walk_record_pool_bytes.restype = SZ
    L.sdf_walk_record_pool_bytes.argtypes = [U32, U32, U32, U32]
    L.sdf_walk_record_full_chunks.restype = U32
    L.sdf_walk_record_full_chunks.argtypes = [U32, U32, U32]
    L.sdf_grad_accum_bytes.restype = SZ
    L.sdf_grad_accum_bytes.argtypes = [C.c_int, U32]
    L.sdf_start_points_scratch_bytes.restype = SZ
    L.sdf_start_points_scratch_bytes.argtypes = [U32]
    L.sdf_start_points.argtypes = [P, U32, P, U32, P, P, P, SZ, P]
    L.sdf_cell_table_bytes.restype = SZ
    L.sdf_cell_table_bytes.argtypes = [C.c_int, C.c_int, U32]
    L.sdf_ray_order_scratch_bytes.restype = SZ
    L.sdf_ray_order_scratch_bytes.argtypes = [U32, U32]
    L.sdf_ray_order.restype = C.c_int
    L.sdf_ray_order.argtypes = [U32, U32, P, P, P, P, SZ, P]
    L.sdf_trace_forward_planned.restype = C.c_int
    L.sdf_trace_forward_planned.argtypes = [C.POINTER(TracePlanDesc)] + L.sdf_trace_forward.argtypes
    L.sdf_trace_backward_planned.restype = C.c_int
    L.sdf_trace_backward_planned.argtypes = [C.POINTER(TracePlanDesc)] + L.sdf_trace_backward.argtypes
    L.sdf_batch_fetcher_ring_bytes.restype = SZ
    L.sdf_batch_fetcher_ring_bytes.argtypes = [SZ, SZ]
    L.sdf_batch_fetcher_create.restype = C.c_int
    L.sdf_batch_fetcher_create.argtypes = [P, SZ, SZ, SZ, C.c_int, P, SZ, U32, C.POINTER(P)]
    L.sdf_batch_fetcher_next.restype = C.c_int
    L.sdf_batch_fetcher_next.argtypes = [P, P, P]
    L.sdf_batch_fetcher_destroy.restype = C.c_int
    L.sdf_batch_fetcher_destroy.argtypes = [P]
    L.sdf_batch_rows.restype = None
    L.sdf_batch_rows.argtypes = [U32, SZ, SZ, C.c_int, P]
    L.sdf_batch_gather.restype = C.c_int
    L.sdf_batch_gather.argtypes = [P, SZ, SZ, U32, SZ, C.c_int, P, P]
    L.sdf_build_aabb_tree.restype = C.c_int
    L.sdf_build_aabb_tree.argtypes = [P, U32, P, P]
    L.sdf_farthest_neighbor.restype = C.c_int
    L.sdf_farthest_neighbor.argtypes = [P, U32, U32, P, P, P, P, P]
    L.sdf_sort_points_scratch_bytes.restype = SZ
    L.sdf_sort_points_scratch_bytes.argtypes = [U32]
    L.sdf_sort_points.restype = C.c_int
    L.sdf_sort_points.argtypes = [P, U32, P, P, SZ, P]
    L.sdf_delaunay_adjacency_capacity.restype = C.c_uint64
    L.sdf_delaunay_adjacency_capacity.argtypes = [U32, U32]
    L.sdf_delaunay_tables_scratch_bytes.restype = SZ
    L.sdf_delaunay_tables_scratch_bytes.argtypes = [U32, U32]
    L.sdf_delaunay_tables.restype = C.c_int
    L.sdf_delaunay_tables.argtypes = [P, U32, P, P, U32, P, P, P, P, P, C.c_uint64, P, SZ, P]
    L.sdf_delaunay_certify_scratch_bytes.restype = SZ
    L.sdf_delaunay_certify_scratch_bytes.argtypes = [U32]
    L.sdf_delaunay_certify.restype = C.c_int
    L.sdf_delaunay_certify.argtypes = [P, U32, P, C.c_uint64, P, P, P, SZ, P]
    L.sdf_delaunay_certify_exhaustive.restype = C.c_int
    L.sdf_delaunay_certify_exhaustive.argtypes = [P, U32, P, C.c_uint64, P, P, P, SZ, P]
    L.sdf_delaunay_merge_scratch_bytes.restype = SZ
    L.sdf_delaunay_merge_scratch_bytes.argtypes = [U32, C.c_uint64, C.c_uint64, C.c_uint64]
    L.sdf_delaunay_merge.restype = C.c_int
    L.sdf_delaunay_merge.argtypes = [P, U32, P, SZ, P, C.c_uint64, P, C.c_uint64, P, P,
                                     C.c_uint64, P, P, SZ, P]
    L.sdf_delaunay_check.restype = C.c_int
    L.sdf_delaunay_check.argtypes = [P, U32, P, P, C.c_uint64, P, P, P, SZ, P]
    L.sdf_delaunay_certify_points.restype = C.c_int
    L.sdf_delaunay_certify_points.argtypes = [P, U32, P, U32, P, C.c_uint64, P, P, P, SZ, P]
    L.sdf_delaunay_merge_verified.restype = C.c_int
    L.sdf_delaunay_merge_verified.argtypes = [P, U32, P, SZ, P, C.c_uint64, P, C.c_uint64, P,
                                              C.c_uint64, P, P, C.c_uint64, P, P, SZ, P]
    L.sdf_nn.restype = C.c_int
    L.sdf_nn.argtypes = [P, P, P, U32, U32, P, P]
    L.sdf_trace_walk_stats.restype = C.c_int
    L.sdf_trace_walk_stats.argtypes = [
        C.c_int, C.POINTER(TraceSettings), C.c_int, U32, P, P, U32, P, P, U32, P, P, P,
        P, P, P, P, P, U32, P, SZ, P]
    L.sdf_debug_fpmath.restype = C.c_int
    L.sdf_debug_fpmath.argtypes = [C.c_int, P, P, C.c_uint64, P]
    L.sdf_set_timing.restype = C.c_int
    L.sdf_set_timing.argtypes = [C.c_int]
    L.sdf_timing_collect.restype = C.c_int
    L.sdf_timing_collect.argtypes = [P, P, C.c_int, C.POINTER(C.c_int)]
    _lib = L
    return L


def check(rc: int) -> None:
    """Raise RuntimeError with the library's message for a nonzero status."""
    if rc != SDF_OK:
        msg = lib().sdf_last_error()
        raise RuntimeError(msg.decode() if msg else f"sdfoam_hip error {rc}")


def ptr(t) -> int | None:
    """Raw device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()


def stream_handle(device) -> int:
    """hipStream_t of torch's current stream on `device`."""
    import torch

    return torch.cuda.current_stream(device).cuda_stream


def set_timing(enable: bool) -> None:
    """Record HIP events around every kernel launch (see sdf_set_timing)."""
    check(lib().sdf_set_timing(1 if enable else 0))


def collect_timings(max_n: int = 512) -> list[tuple[str, float]]:
    """(kernel name, milliseconds) of every launch recorded since the last
    collect, in launch order."""
    kinds = (C.c_int * max_n)()
    ms = (C.c_float * max_n)()
    n = C.c_int()
    check(lib().sdf_timing_collect(kinds, ms, max_n, C.byref(n)))
    return [(KERNEL_NAMES.get(kinds[i], str(kinds[i])), float(ms[i])) for i in range(n.value)]
