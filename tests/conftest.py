import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


_SCENES = {}


def scene(index: int, **kw):
    """Workload C<index> (seeded; cached per session)."""
    from sdfoam_amd import scenes

    key = (index, tuple(sorted(kw.items())))
    if key not in _SCENES:
        w = scenes.make_config(index, **kw)
        w.extra["start"] = scenes.start_points_for(w.points, w.rays)
        _SCENES[key] = w
    return _SCENES[key]


@pytest.fixture(scope="session")
def oracle_lib():
    from oracle import oracle

    oracle.build()
    return oracle
