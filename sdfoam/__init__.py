"""``import sdfoam`` for callers of the reference's module.

The reference's Python code imports its compiled bindings under this name
(``import sdfoam``: sdfoam_model/scene.py:8, train.py:24, test.py:14,
benchmark.py:14, data_loader/__init__.py:7; the module re-exports
``sdfoam.torch_bindings``, torch_bindings/sdfoam/__init__.py.in:29).  Here
the name is bound to this build: every name those callers use
(``create_pipeline``, ``build_aabb_tree``, ``nn``, ``Triangulation``,
``TriangulationFailedError``, ``farthest_neighbor``, ``BatchFetcher``) is
``sdfoam_amd``'s, so the reference's scene, training and test scripts run
on the MI355X library without an edit.
"""

from sdfoam_amd import *  # noqa: F401,F403
from sdfoam_amd import __all__ as _names


def run_with_viewer(pipeline, callback, total_iterations=None, **options):
    """The reference's OpenGL viewer (torch_bindings/pipeline_bindings.cpp:
    753-797) is not part of this build; training runs without it
    (``train.py`` with ``viewer`` off calls ``train_loop`` directly)."""
    raise RuntimeError("run_with_viewer: the interactive viewer is not part of the MI355X build")


__all__ = list(_names) + ["run_with_viewer"]
