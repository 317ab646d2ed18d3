"""bench.py's host-side contract, checked without a GPU: more than one GPU is refused with a
message, and the committed HBM-traffic summary parses into the figures bench.py reports."""
from __future__ import annotations

import json
import re
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=300, cwd=ROOT)
    assert r.returncode == 2
    line = json.loads(r.stdout.strip().splitlines()[-1])
    assert "one GPU" in line["error"]


def test_traffic_summary_parses():
    nbytes, digest = bench.read_traffic()
    assert isinstance(nbytes, int) and nbytes > 0
    assert digest is not None and re.fullmatch(r"[0-9a-f]{64}", digest)
    # HBM traffic cannot be below the algorithmic bytes of the headline call by much
    # (the pool and tables are read at least once): 493,994,920 bytes.
    assert nbytes >= 0.99 * 493_994_920


def test_source_digest_covers_the_kernel_sources():
    d1 = bench.source_digest()
    assert re.fullmatch(r"[0-9a-f]{64}", d1)
    assert d1 == bench.source_digest()  # deterministic
