"""MI355X-native (gfx950) implementation of tinyinfer's GPT-2 INT8 inference hot path.

The product is a set of C-ABI shared libraries built in-tree by
``tinyinfer_amd.build`` (hipcc/g++):

* ``libtinyinfer_backend.so`` – the v2 kernel ABI (``ti_v2_*``) and the legacy
  FP32 ABI (``ti_cpu_*``/``ti_cuda_*``);
* ``libtinyinfer_llm.so`` – the GPT-2 runtime ABI (``ti_llm_*``);
* ``libtinyinfer_host_codec.so`` – the host INT8 codec (``ti_host_*``);
* ``ikernels`` – the pybind11 module.

``native_ops.NativeOps`` and ``runtime.NativeModel`` are ctypes wrappers with
the reference's Python call signatures.  Nothing here falls back to a CPU or
PyTorch implementation: a missing library raises.
"""
from __future__ import annotations

from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
BACKEND_LIB = PACKAGE_DIR / "libtinyinfer_backend.so"
LLM_LIB = PACKAGE_DIR / "libtinyinfer_llm.so"
CODEC_LIB = PACKAGE_DIR / "libtinyinfer_host_codec.so"


def require(path: Path) -> str:
    """Return the path of a built library or raise with the build command."""
    if not path.is_file():
        raise FileNotFoundError(
            f"{path.name} is not built; run `python -m tinyinfer_amd.build` (hipcc, gfx950) first")
    return str(path)
