"""The artifact reader of libtinyinfer_llm (tinyinfer_amd/csrc/artifact.hpp: strict
JSON, SHA-256, schema checks of reference llm/src/artifact.hpp:148-204) built on
the host with AddressSanitizer and UBSan and run over a small valid synthetic
artifact, every structural defect the schema must reject, and a seeded set of
truncated and byte-flipped manifests: each input is accepted or rejected with
Invalid / IOError, with no sanitizer report."""
import hashlib
import json
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent
TINY = {"layers": 1, "heads": 1, "hidden": 64, "vocab": 256, "capacity": 16,
        "gelu": "gelu_new", "layer_norm_eps": 1e-5}


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ is not available")
    exe = tmp_path_factory.mktemp("asan") / "artifact_fuzz"
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined",
           "-fno-omit-frame-pointer", str(HERE / "asan" / "artifact_fuzz.cpp"), "-o", str(exe)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0 and "sanitize" in res.stderr:
        pytest.skip("the host compiler lacks the sanitizer runtimes")
    assert res.returncode == 0, res.stderr
    return exe


def run(driver, mode, paths):
    res = subprocess.run([str(driver), mode, *map(str, paths)], capture_output=True, text=True,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=1", "UBSAN_OPTIONS": "print_stacktrace=1"})
    assert res.returncode == 0, res.stderr[-4000:]
    accepted, rejected = map(int, res.stdout.strip().splitlines()[-1].split())
    return accepted, rejected, res.stdout


@pytest.fixture(scope="module")
def valid(tmp_path_factory):
    from tinyinfer_amd.artifact import write_synthetic
    d = tmp_path_factory.mktemp("tiny")
    path = write_synthetic(d, TINY, seed=5)
    return d, json.loads(path.read_text(encoding="ascii")), (d / "weights.bin").read_bytes()


def write_case(root, name, manifest, binary):
    d = root / name
    d.mkdir()
    text = manifest if isinstance(manifest, str) else json.dumps(manifest)
    (d / "manifest.json").write_text(text, encoding="latin-1")
    if binary is not None:
        (d / "weights.bin").write_bytes(binary)
    return d / "manifest.json"


def resigned(manifest, binary, name):
    """The manifest with tensor `name`'s SHA and the binary's SHA recomputed."""
    m = json.loads(json.dumps(manifest))
    for e in m["tensors"]:
        if e["name"] == name:
            e["sha256"] = hashlib.sha256(binary[e["offset"]:e["offset"] + e["nbytes"]]).hexdigest()
    m["binary_sha256"] = hashlib.sha256(binary).hexdigest()
    return m


def defects(manifest, binary):
    """(name, manifest, binary) for every structural defect the reader must reject."""
    def edit(fn):
        m = json.loads(json.dumps(manifest))
        fn(m)
        return m

    t0, t1 = manifest["tensors"][0], manifest["tensors"][1]
    f16 = next(e for e in manifest["tensors"] if e["dtype"] == "float16")
    f32 = next(e for e in manifest["tensors"] if e["dtype"] == "float32")
    i8 = next(e for e in manifest["tensors"] if e["dtype"] == "int8")
    out = [
        ("not_object", "[]", binary),
        ("missing_sha", edit(lambda m: m.pop("binary_sha256")), binary),
        ("schema_2", edit(lambda m: m.update(schema_version=2)), binary),
        ("alignment_128", edit(lambda m: m.update(alignment=128)), binary),
        ("unknown_identity", edit(lambda m: m.update(model_id="someone/else")), binary),
        ("hidden_not_heads_x64", edit(lambda m: m["architecture"].update(hidden=65)), binary),
        ("zero_layers", edit(lambda m: m["architecture"].update(layers=0)), binary),
        ("precision_int4", edit(lambda m: m.update(precision="int4")), binary),
        ("binary_bytes_plus_one", edit(lambda m: m.update(binary_bytes=m["binary_bytes"] + 1)), binary),
        ("binary_sha_wrong", edit(lambda m: m.update(binary_sha256="0" * 64)), binary),
        ("tensors_not_array", edit(lambda m: m.update(tensors={})), binary),
        ("rank_0", edit(lambda m: m["tensors"][0].update(shape=[])), binary),
        ("rank_3", edit(lambda m: m["tensors"][0].update(shape=[1, 1, t0["nbytes"] // 2])), binary),
        ("zero_dim", edit(lambda m: m["tensors"][0].update(shape=[0, 64])), binary),
        ("huge_dim", edit(lambda m: m["tensors"][0].update(shape=[1 << 21, 1 << 21])), binary),
        ("negative_dim", edit(lambda m: m["tensors"][0].update(shape=[-1, 64])), binary),
        ("float_dim", edit(lambda m: m["tensors"][0].update(shape=[1.5, 64])), binary),
        ("dtype_bf16", edit(lambda m: m["tensors"][0].update(dtype="bfloat16")), binary),
        ("unaligned_offset", edit(lambda m: m["tensors"][1].update(offset=t1["offset"] + 2)), binary),
        ("offset_past_end", edit(lambda m: m["tensors"][1].update(offset=len(binary) + 256)), binary),
        ("offset_2_64", edit(lambda m: m["tensors"][1].update(offset=1 << 64)), binary),
        ("nbytes_mismatch", edit(lambda m: m["tensors"][0].update(nbytes=t0["nbytes"] - 2)), binary),
        ("tensor_sha_wrong", edit(lambda m: m["tensors"][0].update(sha256="f" * 64)), binary),
        ("duplicate_name", edit(lambda m: m["tensors"][1].update(name=t0["name"])), binary),
        ("overlap", edit(lambda m: m["tensors"].append(dict(m["tensors"][0], name="copy"))), binary),
        ("missing_binary", manifest, None),
        ("truncated_binary", manifest, binary[:-1]),
    ]
    for tag, entry, value in (("inf_fp16", f16, b"\x00\x7c"), ("zero_scale", f32, b"\x00\x00\x00\x00"),
                              ("int8_minus_128", i8, b"\x80")):
        b = bytearray(binary)
        b[entry["offset"]:entry["offset"] + len(value)] = value
        out.append((tag, resigned(manifest, bytes(b), entry["name"]), bytes(b)))
    return out


def test_valid_artifact_loads_and_every_defect_is_rejected(driver, valid, tmp_path):
    _, manifest, binary = valid
    good = write_case(tmp_path, "valid", manifest, binary)
    accepted, rejected, _ = run(driver, "manifest", [good])
    assert (accepted, rejected) == (1, 0)
    cases = defects(manifest, binary)
    paths = [write_case(tmp_path, name, m, b) for name, m, b in cases]
    accepted, rejected, out = run(driver, "manifest", paths)
    assert (accepted, rejected) == (0, len(cases)), out


def test_malformed_json_never_crashes(driver, valid, tmp_path):
    _, manifest, _ = valid
    text = json.dumps(manifest).encode("ascii")
    rng = np.random.default_rng(9)
    # Invalid in any strict JSON reader (empty, unclosed, nested deeper than
    # the reader's limit of 33 levels, malformed numbers and literals, a raw
    # control character in a string, non-ASCII bytes):
    invalid = [b"", b"{", b"[" * 40 + b"]" * 40, b"[" * 34 + b"]" * 34, b"-", b"01", b"1e", b'"\x01"', b"nul",
               b"\xff\xfe"]
    paths = []
    for i, data in enumerate(invalid):
        p = tmp_path / f"invalid{i}.json"
        p.write_bytes(data)
        paths.append(p)
    accepted, rejected, out = run(driver, "json", paths)
    assert (accepted, rejected) == (0, len(invalid)), out
    # Edge cases whose verdict is the reader's choice, then truncations and
    # byte flips of a real manifest: no expectation but a clean verdict.
    inputs = [b'{"a":1e999999}', b'"\\ud800"', b'"\\u0000"', b'{"a":1,"a":2}', b"[" * 33 + b"]" * 33]
    for n in rng.integers(0, len(text), 60):
        inputs.append(text[:n])
    for _ in range(120):
        b = bytearray(text)
        for i in rng.integers(0, len(b), int(rng.integers(1, 6))):
            b[i] = int(rng.integers(0, 256))
        inputs.append(bytes(b))
    paths = []
    for i, data in enumerate(inputs):
        p = tmp_path / f"case{i}.json"
        p.write_bytes(data)
        paths.append(p)
    accepted, rejected, _ = run(driver, "json", paths)
    assert accepted + rejected == len(paths)
