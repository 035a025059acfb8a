import sys
from pathlib import Path

import pytest

# torch-ROCm bundles its own libamdhip64.so.7, which shares its SONAME with the
# ROCm runtime the tinyinfer libraries link; whichever loads first serves the
# whole process.  Load torch's first so tests that use torch tensors and the
# native libraries in one process run on one HIP runtime.
try:
    import torch  # noqa: F401
except ImportError:
    pass

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); runs the gfx950 kernels")


@pytest.fixture(scope="session")
def golden():
    import json
    return json.loads((GOLDEN / "known_answers.json").read_text())


@pytest.fixture(scope="session")
def ops():
    """NativeOps over the in-tree libtinyinfer_backend.so (raises if it is not built)."""
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a HIP device")
    from tinyinfer_amd.native_ops import NativeOps
    return NativeOps()
