"""bench.py's contract pieces that need no GPU: the headline metric string is
BASELINE.json's, and more than one GPU is refused with a message (this build
measures one GPU; the sharded design is documented, not run)."""

from __future__ import annotations

import json
import os
import subprocess
import sys

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_headline_metric_is_baselines():
    sys.path.insert(0, REPO)
    import bench
    baseline = json.load(open(os.path.join(REPO, "BASELINE.json")))
    assert bench.METRIC_C5 == baseline["metric"]


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=300, cwd=REPO)
    assert r.returncode != 0
    assert "one GPU" in (r.stdout + r.stderr)
