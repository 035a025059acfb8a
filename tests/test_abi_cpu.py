"""CPU-side checks of the C-ABI libraries: they load, export every symbol the
include/*.h headers declare, report the reference's version numbers and catalog,
and their host-only entry points (INT8 codec, ti_cpu_*) match the reference's
outputs.  No GPU compute is launched here."""
import ctypes as C
import json
import re

import numpy as np
import pytest

import oracle
from tests.conftest import GOLDEN, ROOT
from tinyinfer_amd import BACKEND_LIB, CODEC_LIB, LLM_LIB

HEADERS = {"tinyinfer_backend_v2.h": BACKEND_LIB, "tinyinfer_backend.h": BACKEND_LIB,
           "tinyinfer_amd_ext.h": BACKEND_LIB,
           "tinyinfer_host_codec.h": CODEC_LIB, "tinyinfer_llm.h": LLM_LIB}


def declared(header):
    text = (ROOT / "include" / header).read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tia?_[a-z0-9_]+)\s*\(", text)))


@pytest.mark.parametrize("header", sorted(HEADERS))
def test_library_exports_every_declared_symbol(header):
    lib = C.CDLL(str(HEADERS[header]))
    names = declared(header)
    assert names
    for name in names:
        assert hasattr(lib, name), f"{HEADERS[header].name} lacks {name}"


def test_v2_versions_and_catalog():
    from tinyinfer_amd.native_ops import GEMM_CATALOG, NativeOps
    lib = C.CDLL(str(BACKEND_LIB))
    lib.ti_v2_gemm_catalog_json.restype = C.c_char_p
    catalog = json.loads(lib.ti_v2_gemm_catalog_json())
    assert catalog["schema_version"] == 1 and catalog["only_config"] == -1
    assert [dict(e, tile=tuple(e["tile"])) for e in catalog["configs"]] == list(GEMM_CATALOG)
    assert lib.ti_v2_abi_version() == 2
    ops = NativeOps()  # constructor checks version and catalog without touching a GPU
    assert ops.catalog == catalog


def test_native_ops_rejects_host_tensors_before_any_call():
    torch = pytest.importorskip("torch")
    from tinyinfer_amd.native_ops import NativeOps
    ops = NativeOps()
    a = torch.ones((2, 3), dtype=torch.float16)
    with pytest.raises(TypeError):
        ops.gemm(a, a.t().contiguous())
    with pytest.raises(TypeError):
        ops.layernorm(a, a[0], a[0])


# ---------------------------------------------------------------- host codec
def _codec():
    from tinyinfer_amd.artifact import HostCodec
    return HostCodec()


@pytest.mark.parametrize("key", ["all_half", "fixed0", "fixed1", "fixed2", "fixed3", "random"])
def test_product_codec_matches_reference_bytes(key):
    v = np.load(GOLDEN / "codec_vectors.npz")
    q, s = _codec().quantize(v[key + "_in"])
    assert np.array_equal(q, v[key + "_q"])
    assert np.array_equal(s.view(np.uint32), v[key + "_s"].view(np.uint32))


def test_product_codec_known_answers_and_dequant(golden):
    codec = _codec()
    case = golden["quantize_output_axis"]
    q, s = codec.quantize(np.asarray(case["rows"], np.float16).view(np.uint16))
    assert q.tolist() == case["q"] and s.tolist() == case["scales"]
    deq = codec.dequantize(q, s).view(np.float16).astype(np.float64)
    assert deq.tolist() == case["dequant"]
    v = np.load(GOLDEN / "codec_vectors.npz")
    assert np.array_equal(codec.dequantize(v["deq_q"], v["deq_s"]), v["deq_out"])


def test_numpy_quantizer_agrees_with_product_codec():
    from tinyinfer_amd.artifact import quantize_numpy
    v = np.load(GOLDEN / "codec_vectors.npz")
    for key in ("all_half", "random", "fixed3"):
        q, s = quantize_numpy(v[key + "_in"])
        assert np.array_equal(q, v[key + "_q"]) and np.array_equal(s, v[key + "_s"])


def test_product_codec_rejections_leave_outputs_untouched(golden):
    lib = _codec().lib
    src = (C.c_uint16 * 2)(0x3C00, 0x7C00)
    out = (C.c_int8 * 2)(17, 19)
    sc = (C.c_float * 1)(23.0)
    before = bytes(out), bytes(sc)
    assert lib.ti_host_quantize_f16(src, 2, 1, out, 2, sc, 1) == 1  # non-finite input
    assert (bytes(out), bytes(sc)) == before
    src = (C.c_uint16 * 2)(0x3C00, 0x4000)
    assert lib.ti_host_quantize_f16(src, 2, 1, out, 1, sc, 1) == 1  # extent mismatch
    assert lib.ti_host_quantize_f16(src, 2, 1, C.cast(src, C.c_void_p), 2, sc, 1) == 1  # overlap
    assert (bytes(out), bytes(sc)) == before
    for qv, sv in golden["invalid_dequantize"]["cases"]:
        qq = (C.c_int8 * 1)(qv[0])
        ss = (C.c_float * 1)(float(sv[0]))
        yy = (C.c_uint16 * 1)(0x1234)
        assert lib.ti_host_dequantize_i8(qq, 1, 1, ss, 1, yy, 1) == 1 and yy[0] == 0x1234
    # a valid prefix is not written before a later invalid value is found
    qq = (C.c_int8 * 2)(1, -128)
    ss = (C.c_float * 2)(1.0, 1.0)
    yy = (C.c_uint16 * 2)(0x1234, 0x5678)
    assert lib.ti_host_dequantize_i8(qq, 2, 2, ss, 2, yy, 2) == 1 and list(yy) == [0x1234, 0x5678]


# ---------------------------------------------------------------- legacy CPU entry points
def _cpu_lib():
    lib = C.CDLL(str(BACKEND_LIB))
    p, i = C.c_void_p, C.c_int
    lib.ti_cpu_gemm.argtypes = [p, p, p, i, i, i]
    lib.ti_cpu_softmax.argtypes = [p, p, i, i]
    lib.ti_cpu_layernorm.argtypes = [p, p, p, p, i, i, C.c_float]
    return lib


def ptr(a):
    return a.ctypes.data_as(C.c_void_p)


@pytest.mark.parametrize("shape", [(1, 1, 1), (7, 13, 5), (33, 65, 70)])
def test_ti_cpu_gemm_matches_reference(shape):
    m, n, k = shape
    v = np.load(GOLDEN / "cpu_kernel_vectors.npz")
    a, b, y = v[f"mm{m}_{n}_{k}_a"], v[f"mm{m}_{n}_{k}_b"], v[f"mm{m}_{n}_{k}_y"]
    out = np.empty((m, n), np.float32)
    _cpu_lib().ti_cpu_gemm(ptr(a), ptr(b), ptr(out), m, k, n)  # legacy (m, k, n) order
    assert np.allclose(out, y, atol=1e-5 * k + 1e-5)


@pytest.mark.parametrize("cols", [2, 64, 768, 1024, 4099])
def test_ti_cpu_layernorm_matches_reference(cols):
    v = np.load(GOLDEN / "cpu_kernel_vectors.npz")
    x, g, b, y = (v[f"ln{cols}_{s}"] for s in "xgby")
    out = np.empty_like(x)
    _cpu_lib().ti_cpu_layernorm(ptr(x), ptr(g), ptr(b), ptr(out), x.shape[0], cols, C.c_float(1e-5))
    assert np.allclose(out, oracle.layernorm_f32_exact(x, g, b), atol=1e-4)
    assert np.allclose(out, y, atol=1e-4)


@pytest.mark.parametrize("cols", [1, 31, 128, 1000, 4097])
def test_ti_cpu_softmax_matches_reference(cols):
    v = np.load(GOLDEN / "cpu_kernel_vectors.npz")
    x, y = v[f"sm{cols}_x"], v[f"sm{cols}_y"]
    out = np.empty_like(x)
    _cpu_lib().ti_cpu_softmax(ptr(x), ptr(out), x.shape[0], cols)
    assert np.allclose(out, y, atol=1e-6)
    assert np.allclose(out.sum(1), 1, atol=1e-4)
