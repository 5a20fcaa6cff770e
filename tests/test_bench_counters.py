"""bench.py's use of committed rocprof counter summaries: a summary is used
only while every kernel source it lists has the SHA-256 it was measured on;
otherwise (or without a list) bench reports no rocprof traffic and says why."""

import json
import os

import pytest

import bench


@pytest.fixture
def root(tmp_path, monkeypatch):
    (tmp_path / "profiles").mkdir()
    (tmp_path / "src").mkdir()
    src = tmp_path / "src" / "k.hip"
    src.write_text("kernel v1\n")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    bench.STALE_COUNTERS.clear()
    return tmp_path


def _write(root, sources):
    body = {"hbm_bytes_per_launch": 123.0, "l2_hit": 0.5}
    if sources is not None:
        body["sources"] = sources
    (root / "profiles" / "traffic_x.json").write_text(json.dumps(body))


def test_current_sources_are_used(root):
    _write(root, {"src/k.hip": bench.file_sha256(os.path.join(root, "src", "k.hip"))})
    assert bench.load_traffic("traffic_x.json") == 123.0
    assert "traffic_x.json" not in bench.STALE_COUNTERS


def test_changed_or_missing_sources_are_stale(root):
    _write(root, {"src/k.hip": bench.file_sha256(os.path.join(root, "src", "k.hip"))})
    (root / "src" / "k.hip").write_text("kernel v2\n")
    assert bench.load_traffic("traffic_x.json") is None
    assert "changed" in bench.STALE_COUNTERS["traffic_x.json"]
    _write(root, None)
    assert bench.load_counters("traffic_x.json") is None
    assert bench.STALE_COUNTERS["traffic_x.json"] == "no source hashes"
    _write(root, {"src/gone.hip": "0" * 64})
    assert bench.load_counters("traffic_x.json") is None
    assert bench.load_counters("traffic_missing.json") is None
