"""The committed rocprof traffic summaries (profiles/traffic_*.json) belong to
the kernel sources in the tree: each lists the files it was measured on with
their SHA-256, and every listed file still has that hash.  (bench.py reports
no rocprof traffic for a summary whose sources changed; this test makes the
change visible where it happens.)"""

import glob
import hashlib
import json
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_traffic_summaries_match_the_sources():
    paths = sorted(glob.glob(os.path.join(ROOT, "profiles", "traffic_*.json")))
    assert paths
    for path in paths:
        with open(path) as f:
            c = json.load(f)
        name = os.path.basename(path)
        assert c.get("sources"), f"{name} lists no sources"
        assert c.get("hbm_bytes_per_launch", 0) > 0, name
        for rel, sha in c["sources"].items():
            with open(os.path.join(ROOT, rel), "rb") as f:
                got = hashlib.sha256(f.read()).hexdigest()
            assert got == sha, f"{name}: {rel} changed since it was profiled"
