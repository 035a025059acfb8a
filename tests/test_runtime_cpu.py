"""Host-side contract of the GPT-2 runtime ABI (no GPU compute): struct layouts,
row packing, import hygiene, artifact reader (SHA-256, strict JSON, schema and
identity checks) and create-time validation, mirroring reference
llm/tests/test_contracts.py:140-149 and llm/tests/test_artifact.cpp:6-17."""
import ctypes as C
import json
import shutil
import subprocess
import sys

import pytest

from tests.conftest import ROOT
from tinyinfer_amd import LLM_LIB
from tinyinfer_amd.runtime import Options, Trace, _rows


def test_struct_sizes_and_row_packing(golden):
    sizes = golden["struct_sizes"]
    assert C.sizeof(Options) == sizes["options"] and C.sizeof(Trace) == sizes["trace"]
    case = golden["rows_packing"]
    ids, lengths, stride = _rows(case["rows"])
    assert (list(ids), list(lengths), stride) == (case["flat"], case["lengths"], case["stride"])
    for rows in case["invalid"]:
        with pytest.raises(ValueError):
            _rows(rows)


def test_runtime_wrapper_imports_no_heavy_modules():
    code = ("import sys, tinyinfer_amd.runtime; "
            "bad=[m for m in ('torch','numpy','transformers','datasets') if m in sys.modules]; "
            "assert not bad, bad")
    subprocess.run([sys.executable, "-c", code], check=True, cwd=ROOT)


def _lib():
    lib = C.CDLL(str(LLM_LIB))
    lib.tia_llm_sha256_hex.argtypes = [C.c_void_p, C.c_size_t, C.c_char_p]
    lib.tia_llm_json_accepts.argtypes = [C.c_char_p]
    lib.ti_llm_create.argtypes = [C.c_char_p, C.POINTER(Options), C.POINTER(C.c_void_p)]
    lib.ti_llm_last_error.restype = C.c_char_p
    return lib


def test_sha256_vectors(golden):
    lib = _lib()
    for text, digest in golden["sha256"]["vectors"]:
        data = b"a" * 1000000 if text == "a*1000000" else text.encode()
        out = C.create_string_buffer(65)
        lib.tia_llm_sha256_hex(data, len(data), out)
        assert out.value.decode() == digest


def test_json_reader_strictness(golden):
    lib = _lib()
    case = golden["json_parser"]
    assert lib.tia_llm_json_accepts(case["valid"].encode()) == 1
    for bad in case["invalid"]:
        assert lib.tia_llm_json_accepts(bad.encode()) == 0, bad
    assert lib.tia_llm_json_accepts(b"18446744073709551616") == 1  # number syntax is fine...


TINY = {"layers": 2, "heads": 2, "hidden": 128, "vocab": 300, "capacity": 64, "gelu": "gelu_new",
        "layer_norm_eps": 1e-5}


@pytest.fixture(scope="module")
def tiny(tmp_path_factory):
    from tinyinfer_amd.artifact import write_synthetic
    return write_synthetic(tmp_path_factory.mktemp("tiny_rt"), TINY, seed=5)


def _create(lib, manifest, **kw):
    o = Options(C.sizeof(Options), 0, 2, 4, 64, 0, 0)
    for k, v in kw.items():
        setattr(o, k, v)
    model = C.c_void_p()
    st = lib.ti_llm_create(str(manifest).encode(), C.byref(o), C.byref(model))
    return st, lib.ti_llm_last_error().decode()


@pytest.mark.parametrize("field,value", [("struct_size", 27), ("max_batch", 0), ("max_batch", 33),
                                         ("cache_slots", 1), ("capacity", 1), ("capacity", 1025),
                                         ("gemm_config", 12), ("attention_config", 2), ("device", -1)])
def test_create_rejects_invalid_options(tiny, field, value):
    st, msg = _create(_lib(), tiny, **{field: value})
    assert st == 1 and "invalid options" in msg


def test_create_rejects_bad_artifacts(tiny, tmp_path):
    lib = _lib()
    st, _ = _create(lib, tmp_path / "missing" / "manifest.json")
    assert st == 2  # TI_LLM_IO
    bad = tmp_path / "bad"
    shutil.copytree(tiny.parent, bad)
    weights = bytearray((bad / "weights.bin").read_bytes())
    weights[1000] ^= 1
    (bad / "weights.bin").write_bytes(bytes(weights))
    st, msg = _create(lib, bad / "manifest.json")
    assert st == 1 and "SHA-256" in msg
    manifest = json.loads(tiny.read_text())
    for key, value in (("model_id", "someone/else"), ("schema_version", 2), ("alignment", 128)):
        other = tmp_path / f"m_{key}"
        shutil.copytree(tiny.parent, other)
        m = dict(manifest, **{key: value})
        (other / "manifest.json").write_text(json.dumps(m))
        st, msg = _create(lib, other / "manifest.json")
        assert st == 1, (key, msg)
    dup = tmp_path / "dup"
    shutil.copytree(tiny.parent, dup)
    text = (dup / "manifest.json").read_text()
    (dup / "manifest.json").write_text(text.replace('{"schema_version": 1,', '{"schema_version": 1, "schema_version": 1,', 1)
                                       if text.startswith('{"schema_version": 1,') else
                                       text.replace('"schema_version": 1,', '"schema_version": 1, "schema_version": 1,', 1))
    st, msg = _create(lib, dup / "manifest.json")
    assert st == 1 and "duplicate" in msg
