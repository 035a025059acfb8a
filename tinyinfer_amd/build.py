"""Build the gfx950 libraries in-tree with hipcc/g++ (no CMake, no JIT cache).

Outputs, next to this file:
  libtinyinfer_backend.so     v2 + legacy C ABI (include/tinyinfer_backend*.h)
  libtinyinfer_llm.so         GPT-2 runtime C ABI (include/tinyinfer_llm.h)
  libtinyinfer_host_codec.so  host INT8 codec (include/tinyinfer_host_codec.h)
  ikernels<ext>               pybind11 module, next to libtinyinfer_backend.so
Usage: python -m tinyinfer_amd.build  (or __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: keep the compiler from emitting v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=fast",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wno-unused-result", "-I", str(ROOT / "include")]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-march=x86-64-v3", "-ffp-contract=fast",
              "-fno-math-errno", "-I", str(ROOT / "include")]

BACKEND_HIP = ["gemm.hip", "attention.hip", "rowops.hip", "backend_v2.hip", "backend_legacy.hip"]
LLM_HIP = ["llm_runtime.hip"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in res.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "ignoring feature" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")


def _hip_obj(src: str) -> Path:
    out = OBJ / (Path(src).stem + ".o")
    _run([HIPCC, *HIP_FLAGS, "-c", str(CSRC / src), "-o", str(out)])
    return out


def _host_obj(src: str, extra: list[str] | None = None) -> Path:
    out = OBJ / (Path(src).stem + ".host.o")
    _run(["g++", *HOST_FLAGS, *(extra or []), "-c", str(CSRC / src), "-o", str(out)])
    return out


def _link(target: Path, objs: list[Path], extra: list[str]) -> None:
    tmp = target.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs), *extra])
    os.replace(tmp, target)


def ikernels_name() -> str:
    return "ikernels" + sysconfig.get_config_var("EXT_SUFFIX")


def build(verbose: bool = True) -> None:
    OBJ.mkdir(exist_ok=True)
    hip_sources = BACKEND_HIP + [s for s in LLM_HIP if (CSRC / s).exists()]
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 4)) as pool:
        hip_jobs = {s: pool.submit(_hip_obj, s) for s in hip_sources}
        cpu_job = pool.submit(_host_obj, "cpu_ops.cpp", ["-fopenmp"])
        codec_job = pool.submit(_host_obj, "host_codec.cpp")
        objs = {s: j.result() for s, j in hip_jobs.items()}
        cpu_obj, codec_obj = cpu_job.result(), codec_job.result()

    rpath = ["-Wl,-rpath,$ORIGIN"]
    _link(PKG / "libtinyinfer_backend.so", [objs[s] for s in BACKEND_HIP] + [cpu_obj],
          ["-lgomp", *rpath])
    _run(["g++", "-shared", "-fPIC", "-o", str(PKG / "libtinyinfer_host_codec.so"), str(codec_obj)])
    if "llm_runtime.hip" in objs:
        _link(PKG / "libtinyinfer_llm.so", [objs["llm_runtime.hip"]],
              ["-L", str(PKG), "-ltinyinfer_backend", *rpath])
    if (CSRC / "ikernels.cpp").exists():
        import pybind11
        inc = sysconfig.get_paths()["include"]
        # Host-only translation unit (no kernels): libgomp's omp.h, linked to the backend.
        _run([HIPCC, "-O2", "-std=c++17", "-fPIC", "-shared", "-x", "c++", "-D__HIP_PLATFORM_AMD__",
              "-I", str(ROCM / "include"), "-I", str(ROOT / "include"), "-I", pybind11.get_include(),
              "-I", inc, "-isystem", "/usr/lib/gcc/x86_64-linux-gnu/11/include",
              str(CSRC / "ikernels.cpp"), "-o", str(PKG / ikernels_name()),
              "-L", str(PKG), "-ltinyinfer_backend", "-L", str(ROCM / "lib"), "-lamdhip64", "-lgomp", *rpath])
    if verbose:
        print("built:", ", ".join(sorted(p.name for p in PKG.glob("*.so"))))


def build_oracle() -> None:
    """Compile oracle/ (the CPU checker) and, where the reference checkout exists,
    oracle/_ref (the reference's own CPU sources)."""
    _run(["make", "-s", "-C", str(ROOT / "oracle"), "all"])
    if Path("/root/reference").is_dir():
        _run(["make", "-s", "-C", str(ROOT / "oracle"), "ref"])


if __name__ == "__main__":
    build()
    if "--no-oracle" not in sys.argv:
        build_oracle()
