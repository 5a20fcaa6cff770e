"""Start-cell lookup: ``build_aabb_tree``, ``nn`` and ``get_starting_point``.

Same arguments, checks, messages and outputs as the reference's bindings
(torch_bindings/triangulation_bindings.cpp:117-181) and as
``SDFoamScene.get_starting_point`` (sdfoam_model/scene.py:272-282); the work
runs in libsdfoam_hip.so on torch's current stream.
"""

from __future__ import annotations

import torch

from . import _lib
from ._lib import check, ptr
from .pipeline import _c10, _scalar_type


def pow2_round_up(x: int) -> int:
    return 1 if x <= 1 else 1 << int(x - 1).bit_length()


def build_aabb_tree(points: torch.Tensor) -> torch.Tensor:
    """AABB tree [pow2(N), 2, 3] over the points in their given order."""
    if points.size(-1) != 3:
        raise RuntimeError("points must have 3 as the last dimension")
    if points.dim() != 2:
        raise RuntimeError("points must have 2 dimensions")
    if points.device.type != "cuda":
        raise RuntimeError("points must be on CUDA device")
    st = _scalar_type(points.dtype)
    if st != "float32":
        raise RuntimeError("unsupported scalar type")
    p = points.contiguous()
    n = p.numel() // 3
    tree = torch.empty((pow2_round_up(n), 2, 3), dtype=points.dtype, device=points.device)
    with torch.cuda.device(p.device):
        check(_lib.lib().sdf_build_aabb_tree(ptr(p), n, ptr(tree), _lib.stream_handle(p.device)))
    return tree


def nn(points: torch.Tensor, tree: torch.Tensor, queries: torch.Tensor) -> torch.Tensor:
    """Index (uint32) of the nearest point to each query."""
    num_points = points.numel() // 3
    num_queries = queries.numel() // 3
    if points.dtype != queries.dtype:
        raise RuntimeError("points and queries must have the same dtype")
    if points.dtype != tree.dtype:
        raise RuntimeError("points and tree must have the same dtype")
    if points.device.type != "cuda":
        raise RuntimeError("points must be on CUDA device")
    if tree.device.type != "cuda":
        raise RuntimeError("tree must be on CUDA device")
    if queries.device.type != "cuda":
        raise RuntimeError("queries must be on CUDA device")
    indices = torch.zeros(tuple(queries.shape[:-1]), dtype=torch.uint32, device=queries.device)
    if num_points < 32:
        raise RuntimeError("number of points must be at least 32")
    if _scalar_type(points.dtype) != "float32":
        raise RuntimeError("unsupported scalar type")
    p = points.contiguous()
    t = tree.contiguous()
    q = queries.contiguous()
    with torch.cuda.device(q.device):
        check(_lib.lib().sdf_nn(ptr(p), ptr(t), ptr(q), num_points, num_queries, ptr(indices),
                                _lib.stream_handle(q.device)))
    return indices


def get_starting_point(rays: torch.Tensor, points: torch.Tensor, aabb_tree: torch.Tensor):
    """Start cell per ray: the nearest point to each distinct ray origin,
    looked up once per origin (sdfoam_model/scene.py:272-282).  The
    reference deduplicates the origins with torch.unique, which waits for the
    GPU; here sdf_start_points deduplicates them on the GPU, so the call
    queues its work and returns.  The result equals nn over the distinct
    origins for finite points and origins."""
    if rays.size(-1) != 6:
        raise RuntimeError("rays must have 6 as the last dimension")
    if rays.dtype != torch.float32 or points.dtype != torch.float32 or aabb_tree.dtype != torch.float32:
        raise RuntimeError("unsupported scalar type")
    if rays.device.type != "cuda" or points.device.type != "cuda" or aabb_tree.device.type != "cuda":
        raise RuntimeError("rays, points and tree must be on CUDA device")
    num_points = points.numel() // 3
    if num_points < 32:
        raise RuntimeError("number of points must be at least 32")
    r = rays.detach().contiguous()
    num_rays = r.numel() // 6
    start = torch.empty(tuple(r.shape[:-1]), dtype=torch.uint32, device=r.device)
    L = _lib.lib()
    nbytes = int(L.sdf_start_points_scratch_bytes(num_rays))
    scratch = torch.empty(nbytes + 256, dtype=torch.uint8, device=r.device)
    base = (scratch.data_ptr() + 255) & ~255
    with torch.cuda.device(r.device):
        check(L.sdf_start_points(ptr(r), num_rays, ptr(points.detach().contiguous()), num_points,
                                 ptr(aabb_tree.detach().contiguous()), ptr(start), base, nbytes,
                                 _lib.stream_handle(r.device)))
    return start


__all__ = ["build_aabb_tree", "nn", "get_starting_point", "pow2_round_up", "_c10"]
