"""The C ABI's in-launch split finishing under concurrency: a fresh process
makes its first calls on eight streams at once (tests/many_streams.py), every
split plan that uses the per-hardware-queue pool, and each result must equal
the same call made alone (bit for bit).  The reference's calls own no memory
and may run on any stream (backend/include/tinyinfer_backend_v2.h:13)."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def test_split_plans_on_eight_streams_equal_lone_calls():
    print("[case] many_streams.py: 7 GEMM plans + split decode and prefill attention on 8 streams, 3 rounds", flush=True)
    res = subprocess.run([sys.executable, str(ROOT / "tests" / "many_streams.py")], cwd=ROOT,
                         capture_output=True, text=True, timeout=110)
    print(res.stdout[-4000:], res.stderr[-4000:], flush=True)
    assert res.returncode == 0, f"many_streams.py exited {res.returncode}"
    report = json.loads(res.stdout.strip().splitlines()[-1])
    assert report["ok"] and report["calls"] == 3 * 8 * 10
