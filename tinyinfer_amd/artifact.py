"""GPT-2 weight artifacts: ``manifest.json`` + 256-byte-aligned ``weights.bin``.

The format is the reference's (writer reference llm/export_weights.py:140-208,
reader reference llm/src/artifact.hpp:148-204): Conv1D ``[in, out]`` weight
orientation, fp16 embeddings / LayerNorm parameters / biases, per-output-channel
INT8 linears with fp32 ``.scales``, and a tied head stored as the (quantized)
transpose of the fp16 token embedding.  Every tensor carries its SHA-256.

The reference pins the artifact identity to the official GPT-2 file
(artifact.hpp:156-158).  Random-init artifacts (no checkpoint is available
offline) carry a second, verifiable identity instead: ``model_id``
``tinyinfer-amd/gpt2-synthetic``, a ``synthetic`` block with the generator
parameters, and ``source_sha256`` = SHA-256 of that block's canonical JSON.  The
native loader accepts exactly these two identities.
"""
from __future__ import annotations

import collections
import concurrent.futures as cf
import ctypes
import hashlib
import json
import math
import os
from pathlib import Path

import numpy as np

from . import CODEC_LIB, require

ALIGNMENT = 256
SYNTHETIC_ID = "tinyinfer-amd/gpt2-synthetic"
GPT2_SMALL = {"layers": 12, "heads": 12, "hidden": 768, "vocab": 50257, "capacity": 1024,
              "gelu": "gelu_new", "layer_norm_eps": 1e-5}
GPT2_XL = {"layers": 48, "heads": 25, "hidden": 1600, "vocab": 50257, "capacity": 1024,
           "gelu": "gelu_new", "layer_norm_eps": 1e-5}
LINEARS = (("attn.c_attn", 1, 3), ("attn.c_proj", 1, 1), ("mlp.c_fc", 1, 4), ("mlp.c_proj", 4, 1))


def canonical_hash(value) -> str:
    return hashlib.sha256(json.dumps(value, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def tensor_shapes(arch):
    """Ordered tensor list of the artifact (reference llm/export_weights.py:32-45)."""
    h, v, L = arch["hidden"], arch["vocab"], arch["layers"]
    shapes = {"transformer.wte.weight": [v, h], "transformer.wpe.weight": [arch["capacity"], h],
              "transformer.ln_f.weight": [h], "transformer.ln_f.bias": [h]}
    for l in range(L):
        p = f"transformer.h.{l}."
        for ln in ("ln_1", "ln_2"):
            shapes[p + ln + ".weight"] = [h]
            shapes[p + ln + ".bias"] = [h]
        for name, kin, kout in LINEARS:
            shapes[p + name + ".weight"] = [kin * h, kout * h]
            shapes[p + name + ".bias"] = [kout * h]
    return shapes


# -- INT8 codec --------------------------------------------------------------------
class HostCodec:
    """ctypes access to libtinyinfer_host_codec.so (include/tinyinfer_host_codec.h)."""

    def __init__(self, path=None):
        self.lib = ctypes.CDLL(require(CODEC_LIB) if path is None else str(path))
        p, s = ctypes.c_void_p, ctypes.c_size_t
        self.lib.ti_host_quantize_f16.argtypes = [p, s, s, p, s, p, s]
        self.lib.ti_host_dequantize_i8.argtypes = [p, s, s, p, s, p, s]
        if self.lib.ti_host_codec_abi_version() != 1:
            raise RuntimeError("host codec ABI mismatch")

    def quantize(self, w_bits: np.ndarray):
        w = np.ascontiguousarray(w_bits, np.uint16)
        k, n = w.shape
        q = np.empty((k, n), np.int8)
        sc = np.empty(n, np.float32)
        if self.lib.ti_host_quantize_f16(w.ctypes.data, w.size, n, q.ctypes.data, q.size, sc.ctypes.data, n):
            raise ValueError("ti_host_quantize_f16 rejected the input")
        return q, sc

    def dequantize(self, q: np.ndarray, scales: np.ndarray):
        q = np.ascontiguousarray(q, np.int8)
        sc = np.ascontiguousarray(scales, np.float32)
        out = np.empty(q.shape, np.uint16)
        if self.lib.ti_host_dequantize_i8(q.ctypes.data, q.size, q.shape[1], sc.ctypes.data, sc.size,
                                          out.ctypes.data, out.size):
            raise ValueError("ti_host_dequantize_i8 rejected the input")
        return out


def quantize_numpy(w_bits: np.ndarray):
    """Independent vectorized quantizer (the exporter's second implementation,
    reference llm/export_weights.py:126-137): scale = fp32(max|w| / 127) or 1,
    q = clip(rint(w / scale), -127, 127) in binary64 (rint rounds half to even)."""
    w = np.ascontiguousarray(w_bits, np.uint16).view(np.float16).astype(np.float64)
    mx = np.abs(w).max(axis=0)
    scales = np.where(mx > 0, (mx / 127.0).astype(np.float32), np.float32(1.0)).astype(np.float32)
    r = np.rint(w / scales.astype(np.float64))
    return np.clip(r, -127, 127, out=r).astype(np.int8), scales


# -- synthetic weights -------------------------------------------------------------
def _normal_f16(rng, shape, mean, std):
    return (rng.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean)).astype(np.float16)


def _quantized(codec, name, bits):
    """INT8 bytes and scales of fp16 `bits` [K, N]; the native codec and the
    numpy quantizer must agree byte for byte (reference export_weights.py:146-151)."""
    q, sc = codec.quantize(bits)
    q2, sc2 = quantize_numpy(bits)
    if not (np.array_equal(q, q2) and np.array_equal(sc.view(np.uint32), sc2.view(np.uint32))):
        raise ValueError(f"native/numpy INT8 bytes differ for {name}")
    return q, sc


def _record(name, dtype, arr):
    raw = np.ascontiguousarray(arr)
    return name, dtype, list(arr.shape), raw, hashlib.sha256(memoryview(raw).cast("B")).hexdigest()


def _writer_threads():
    # Generation, quantization and hashing release the GIL; a GPU box gives a
    # process 16 cores whatever os.cpu_count() reports.
    return max(1, min(16, os.cpu_count() or 1))


def write_synthetic(dest, arch=None, seed=42, precision="int8", std=0.02, progress=None):
    """Write a random-init GPT-2 artifact: every weight matrix, embedding and bias
    ~ N(0, std), LayerNorm gamma ~ N(1, std), beta ~ N(0, std), stored fp16;
    linears and the tied head INT8-quantized (``precision="int8"``) or kept fp16
    (``"fp16"``, the format's two precisions, reference export_weights.py:142).  Tensor i of the manifest order draws from its own numpy
    PCG64 stream, ``SeedSequence(seed).spawn(count)[i]``, so worker threads build
    tensors concurrently and the bytes do not depend on their scheduling.
    Returns the manifest path.  ``progress``, if given, is called with each
    tensor name as it is written."""
    arch = dict(GPT2_SMALL if arch is None else arch)
    if precision not in ("int8", "fp16"):
        raise ValueError("precision must be 'int8' or 'fp16'")
    dest = Path(dest)
    dest.mkdir(parents=True, exist_ok=True)
    codec = HostCodec() if precision == "int8" else None
    shapes = list(tensor_shapes(arch).items())
    streams = np.random.SeedSequence(seed).spawn(len(shapes))
    spec = {"generator": "numpy.PCG64, tensor i from SeedSequence(seed).spawn(count)[i] in manifest order",
            "seed": seed, "std": std, "precision": precision,
            "distribution": "matrices/embeddings/biases N(0,std); ln gamma N(1,std); ln beta N(0,std)",
            "architecture": arch}

    def build(index):
        name, shape = shapes[index]
        mean = 1.0 if (".ln_" in name or "ln_f" in name) and name.endswith(".weight") else 0.0
        vals = _normal_f16(np.random.Generator(np.random.PCG64(streams[index])), shape, mean, std)
        bits = vals.view(np.uint16)
        if precision == "int8" and len(shape) == 2 and ".h." in name and name.endswith(".weight"):
            q, sc = _quantized(codec, name, bits)
            return [_record(name, "int8", q), _record(name + ".scales", "float32", sc)], None
        return [_record(name, "float16", bits)], (bits if name == "transformer.wte.weight" else None)

    # The tied head is the transposed fp16 wte [hidden, vocab].  Quantization is
    # per output column, so column blocks are quantized as independent jobs.
    head_block_cols = 8192

    def head_block(wte_bits, c0):
        t = np.ascontiguousarray(wte_bits[c0:c0 + head_block_cols].T)
        return _quantized(codec, "lm_head.weight", t) if precision == "int8" else (t, None)

    def head_records(blocks):
        mat = np.concatenate([b[0] for b in blocks], axis=1)
        if precision == "int8":
            scales = np.concatenate([b[1] for b in blocks])
            return [_record("lm_head.weight", "int8", mat), _record("lm_head.weight.scales", "float32", scales)]
        return [_record("lm_head.weight", "float16", mat)]

    entries = []
    binary = dest / "weights.bin"
    digest = hashlib.sha256()
    with binary.open("wb") as f, cf.ThreadPoolExecutor(_writer_threads()) as pool:
        def emit(records):
            for name, dtype, shape, raw, sha in records:
                pad = (-f.tell()) % ALIGNMENT
                if pad:
                    f.write(bytes(pad))
                    digest.update(bytes(pad))
                off = f.tell()
                view = memoryview(raw).cast("B")
                f.write(view)
                digest.update(view)
                entries.append({"name": name, "dtype": dtype, "shape": shape, "offset": off,
                                "nbytes": raw.nbytes, "sha256": sha})
                if progress:
                    progress(name)

        window = 2 * _writer_threads()
        pending = collections.deque()
        head_jobs = []
        for index in range(len(shapes)):
            pending.append(pool.submit(build, index))
            while len(pending) > window or (index == len(shapes) - 1 and pending):
                records, wte_bits = pending.popleft().result()
                if wte_bits is not None:
                    head_jobs = [pool.submit(head_block, wte_bits, c0)
                                 for c0 in range(0, wte_bits.shape[0], head_block_cols)]
                emit(records)
        emit(head_records([job.result() for job in head_jobs]))
    manifest = {"schema_version": 1, "model_id": SYNTHETIC_ID, "revision": f"seed-{seed}",
                "source_sha256": canonical_hash(spec), "synthetic": spec, "precision": precision,
                "architecture": arch, "binary": "weights.bin", "binary_bytes": binary.stat().st_size,
                "binary_sha256": digest.hexdigest(), "alignment": ALIGNMENT,
                "quantization": {"axis": "output", "range": [-127, 127], "rounding": "ties_to_even",
                                 "zero_channel_scale": 1, "reference": "fp16",
                                 "dequantize": "fp32_then_fp16"},
                "tied_head": "transpose_of_fp16_transformer.wte.weight_then_optional_quantization",
                "tensors": entries}
    path = dest / "manifest.json"
    path.write_text(json.dumps(manifest, indent=1, allow_nan=False) + "\n", encoding="ascii")
    return path


def load_tensors(manifest_path):
    """Map tensor name -> numpy view (memory-mapped) of an artifact; fp16 tensors
    are returned as uint16 bit patterns."""
    manifest_path = Path(manifest_path)
    manifest = json.loads(manifest_path.read_text(encoding="ascii"))
    raw = np.memmap(manifest_path.parent / manifest["binary"], dtype=np.uint8, mode="r")
    dtypes = {"float16": np.uint16, "float32": np.float32, "int8": np.int8}
    out = {}
    for e in manifest["tensors"]:
        dt = dtypes[e["dtype"]]
        out[e["name"]] = np.frombuffer(raw, dtype=dt, count=math.prod(e["shape"]),
                                       offset=e["offset"]).reshape(e["shape"])
    return manifest, out
