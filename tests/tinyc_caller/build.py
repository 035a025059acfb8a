"""Build the tinyc-style callers of the legacy FP32 ABI (hand_cpu with g++,
hand_gpu with hipcc for gfx950), each linked to the in-tree
libtinyinfer_backend.so as tinyc links TINYC_BACKEND_LIBRARY.  Test programs,
not product code; tests/test_tinyc_hand_path.py runs them."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
PKG = ROOT / "tinyinfer_amd"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _run(cmd):
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines() if "packed-fp32-ops" not in l and "ignoring feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"tinyc caller build failed: {' '.join(map(str, cmd))}\n{out}")


def build_cpu(out_dir):
    """Compiled by the CPU test into its own temporary directory (g++, seconds)."""
    target = Path(out_dir) / "hand_cpu"
    _run(["g++", "-O2", "-std=c++17", "-I", str(ROOT / "include"), str(HERE / "hand_cpu.cpp"), "-o", str(target),
          "-L", str(PKG), "-ltinyinfer_backend", f"-Wl,-rpath,{PKG}"])
    return target


def build_gpu():
    """Built in-tree ahead of the GPU tests (the binary travels with the tree)."""
    target = HERE / "hand_gpu"
    _run([str(ROCM / "bin" / "hipcc"), "--offload-arch=gfx950", "-O2", "-std=c++17",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-I", str(ROOT / "include"),
          str(HERE / "hand_gpu.hip"), "-o", str(target), "-L", str(PKG), "-ltinyinfer_backend",
          "-Wl,-rpath,$ORIGIN/../../tinyinfer_amd"])
    return target


def build():
    build_gpu()


if __name__ == "__main__":
    build()
