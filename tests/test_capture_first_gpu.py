"""The C ABI allocates nothing, so a process may capture its very first library
calls into a HIP graph (reference contract: the caller owns every buffer and
the stream, backend/include/tinyinfer_backend_v2.h:13; the reference's
ti::v2::gemm is one launch into y, kernels/src/cuda/tc/gemm.cu:147-158).

tests/capture_first.py runs in a fresh interpreter, so no earlier test's calls
can have set anything up: it captures NativeOps.gemm_int8 (M 1/8/64/512, both
configs[1] shapes, configs 0 and 6), ti_amd_pack_w8 + ti_amd_gemm_w8p_fused
(M 1/16/32/64/512, each packed kernel and split plan) and ti_v2_attention_f16
(configs[3]) under
torch.cuda.graph, then checks replays against each other, against eager calls
(also on another stream while a replay runs) and against the CPU oracle."""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def test_first_library_calls_under_graph_capture():
    print("[case] capture_first.py: GEMMs M 1/8/64/512 x configs 0/6 and configs[3] attention, "
          "packed GEMMs at each packed kernel, first calls under torch.cuda.graph", flush=True)
    res = subprocess.run([sys.executable, str(ROOT / "tests" / "capture_first.py")], cwd=ROOT,
                         capture_output=True, text=True, timeout=110)
    print(res.stdout[-4000:], res.stderr[-4000:], flush=True)
    assert res.returncode == 0, f"capture_first.py exited {res.returncode}"
    report = json.loads(res.stdout.strip().splitlines()[-1])
    assert report["ok"]
    assert report["attention_max_err"] <= 1e-4
    assert len(report["gemm_max_err"]) == 16
    assert len(report["packed_max_err"]) == 6
