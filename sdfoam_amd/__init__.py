"""MI355X-native SDFoam Voronoi-foam tracer.

Drop-in for the tracing surface of the reference's ``sdfoam`` module:
``create_pipeline`` -> ``Pipeline.trace_forward`` / ``trace_backward``,
``build_aabb_tree``, ``nn``, plus the ``TraceRays`` autograd Function and
``get_starting_point``, ``BatchFetcher`` (the training loop's batch
prefetcher) and the adjacency producer (``Triangulation``,
``TriangulationFailedError``, ``farthest_neighbor``).  Compute runs in libsdfoam_hip.so (hand-written HIP
for gfx950) through its C ABI; importing this package does not need a GPU,
calling the tracer does.
"""

from .fetch import BatchFetcher
from .pipeline import Pipeline, create_pipeline, prefetch_adjacent_diff, release_trace_plan
from .render import ErrorBox, TraceRays
from .spatial import build_aabb_tree, get_starting_point, nn
from .triangulation import Triangulation, TriangulationFailedError, farthest_neighbor

__all__ = [
    "Pipeline",
    "create_pipeline",
    "prefetch_adjacent_diff",
    "release_trace_plan",
    "TraceRays",
    "ErrorBox",
    "build_aabb_tree",
    "nn",
    "get_starting_point",
    "BatchFetcher",
    "Triangulation",
    "TriangulationFailedError",
    "farthest_neighbor",
]
