"""Build the bench-only probe library benchlib/liblimits.so (hipcc, gfx950).

Not a product library: bench.py loads it to measure the machine limits (launch
floor, streaming-read ceilings) that the roofline fractions are read against.
"""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
LIB = HERE / "liblimits.so"


def build() -> None:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [str(ROCM / "bin" / "hipcc"), "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           str(HERE / "limits.hip"), "-o", str(tmp)]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"benchlib build failed: {' '.join(cmd)}\n{res.stdout}")
    os.replace(tmp, LIB)


if __name__ == "__main__":
    build()
