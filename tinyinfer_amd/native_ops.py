"""ctypes wrapper of the v2 kernel ABI with the reference's Python signatures.

Mirrors reference llm/native_ops.py:33-210 (class ``NativeOps``): the same
method names, argument meaning, tensor checks (CUDA/HIP device, dtype,
contiguity, no grad, rank, extents), catalog check, ``record_stream`` on every
tensor before the call, the current torch stream and device index appended to
every native call, and ``RuntimeError`` carrying ``ti_v2_last_error()`` when a
call returns a nonzero status.  Inference only; no CPU fallback exists.
"""
from __future__ import annotations

import ctypes
import json
import math
from pathlib import Path

from . import BACKEND_LIB, require

_I32_MAX = 2**31 - 1
_TILES = ((32, 32, 16, 4), (64, 32, 32, 8), (64, 64, 32, 8))
# The 12-entry allow-list the library must report (reference llm/native_ops.py:14-16).
GEMM_CATALOG = tuple({"id": i, "tile": _TILES[i % 3],
                      "stages": 1 if (3 <= i < 6 or i >= 9) else 2,
                      "epilogue": "separate" if i >= 6 else "fused"} for i in range(12))


def _dim(value, name):
    if type(value) is not int or value <= 0 or value > _I32_MAX:
        raise ValueError(f"{name} must be an integer in [1, INT32_MAX]")
    return value


def _metadata(value, batch, default, maximum, name):
    """Host-side per-request metadata: None, one int, or `batch` ints in [0, maximum]."""
    if value is None:
        values = [default] * batch
    elif type(value) is int:
        values = [value] * batch
    else:
        values = list(value)
    if len(values) != batch or any(type(x) is not int or not 0 <= x <= maximum for x in values):
        raise ValueError(f"{name} must contain {batch} integers in [0,{maximum}]")
    return values


class NativeOps:
    def __init__(self, library_path=None):
        import torch
        self.torch = torch
        path = require(BACKEND_LIB) if library_path is None else library_path
        self.library_path = str(Path(path).expanduser().resolve(strict=True))
        self.lib = ctypes.CDLL(self.library_path)
        p, i, u = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
        table = {
            "ti_v2_gemm_f16": [p, p, p, p, i, i, i, i, i, u, i],
            "ti_v2_gemm_i8": [p, p, p, p, p, i, i, i, i, i, u, i],
            "ti_v2_gemm_ex_f16": [p, p, p, p, p, i, i, i, i, i, u, i],
            "ti_v2_gemm_ex_i8": [p, p, p, p, p, p, i, i, i, i, i, u, i],
            "ti_v2_legacy_gemm_f32": [p, p, p, i, i, i, u, i],
            "ti_v2_attention_f16": [p, p, p, p, p, p, p, i, i, i, i, i, i, i, u, i],
            "ti_v2_layernorm_f16": [p, p, p, p, i, i, ctypes.c_float, u, i],
            "ti_v2_gelu_new_f16": [p, p, ctypes.c_int64, u, i],
            "ti_v2_softmax_f16": [p, p, i, i, u, i],
        }
        self.lib.ti_v2_abi_version.argtypes, self.lib.ti_v2_abi_version.restype = [], i
        self.lib.ti_v2_last_error.argtypes, self.lib.ti_v2_last_error.restype = [], ctypes.c_char_p
        if self.lib.ti_v2_abi_version() != 2:
            raise RuntimeError("native v2 ABI version mismatch")
        self.lib.ti_v2_gemm_catalog_json.argtypes = []
        self.lib.ti_v2_gemm_catalog_json.restype = ctypes.c_char_p
        self.catalog = json.loads(self.lib.ti_v2_gemm_catalog_json())
        reported = [dict(entry, tile=tuple(entry["tile"])) for entry in self.catalog["configs"]]
        if reported != list(GEMM_CATALOG):
            raise RuntimeError("native GEMM catalog does not match wrapper allow-list")
        for name, args in table.items():
            fn = getattr(self.lib, name)
            fn.argtypes, fn.restype = args, i

    # -- checks ---------------------------------------------------------------
    def _tensor(self, tensor, dtype, name, ndim=None, device=None):
        t = self.torch
        if not isinstance(tensor, t.Tensor) or tensor.device.type != "cuda":
            raise TypeError(f"{name} must be a CUDA Tensor")
        if tensor.dtype != dtype or not tensor.is_contiguous():
            raise TypeError(f"{name} must have dtype={dtype} and contiguous row-major storage")
        if tensor.requires_grad:
            raise ValueError(f"{name} requires_grad is unsupported by inference-only native ops")
        if ndim is not None and tensor.ndim != ndim:
            raise ValueError(f"{name} must have rank {ndim}")
        if tensor.ndim == 0 or tensor.numel() == 0:
            raise ValueError(f"{name} must have at least one nonempty dimension")
        for axis, size in enumerate(tensor.shape):
            _dim(size, f"{name}.shape[{axis}]")
        if tensor.numel() > (2**63 - 1) // tensor.element_size():
            raise ValueError(f"{name} byte extent exceeds signed 64-bit indexing")
        if device is not None and tensor.device != device:
            raise ValueError(f"{name} must be on {device}")
        return tensor

    @staticmethod
    def _ptr(tensor):
        return None if tensor is None else tensor.data_ptr()

    def _call(self, name, tensors, args):
        device = tensors[0].device
        with self.torch.cuda.device(device):
            stream = self.torch.cuda.current_stream(device)
            for tensor in tensors:
                if tensor is not None:
                    tensor.record_stream(stream)
            status = getattr(self.lib, name)(*args, stream.cuda_stream, device.index)
            if status:
                reason = self.lib.ti_v2_last_error().decode("utf-8", errors="replace")
                raise RuntimeError(f"{name} failed ({status}): {reason}")

    def _gemm_args(self, a, b, bias, config, output_dtype, weight_dtype):
        t = self.torch
        self._tensor(a, t.float16, "a", 2)
        self._tensor(b, weight_dtype, "b", 2, a.device)
        m, k = a.shape
        if b.shape[0] != k:
            raise ValueError("GEMM a[M,K] and b[K,N] inner dimensions differ")
        n = b.shape[1]
        if type(config) is not int or not 0 <= config < len(GEMM_CATALOG):
            raise ValueError("GEMM config must be allow-listed ID0..11")
        only = getattr(self, "catalog", {}).get("only_config", -1)
        if only != -1 and config != only:
            raise ValueError("GEMM config is unavailable in this single-candidate build")
        if (m - 1) // GEMM_CATALOG[config]["tile"][0] + 1 > 65535:
            raise ValueError("GEMM M exceeds grid-y limit")
        if bias is not None:
            self._tensor(bias, t.float16, "bias", 1, a.device)
            if bias.shape != (n,):
                raise ValueError("bias must have shape [N]")
        dtype = t.float16 if output_dtype is None else output_dtype
        if dtype not in (t.float16, t.float32):
            raise TypeError("output_dtype must be torch.float16 or torch.float32")
        out = t.empty((m, n), dtype=dtype, device=a.device)
        return out, (m, n, k, int(dtype == t.float32), config)

    # -- ops --------------------------------------------------------------------
    def gemm(self, a, b, *, bias=None, config=0, output_dtype=None):
        out, dims = self._gemm_args(a, b, bias, config, output_dtype, self.torch.float16)
        ws = self.torch.empty(out.shape, dtype=self.torch.float32, device=out.device) if config >= 6 else None
        tensors = (a, b, bias, out, ws)
        self._call("ti_v2_gemm_ex_f16", tensors, tuple(map(self._ptr, tensors)) + dims)
        return out

    def gemm_int8(self, a, b, scales, *, bias=None, config=0, output_dtype=None):
        self._tensor(a, self.torch.float16, "a", 2)
        self._tensor(b, self.torch.int8, "b", 2, a.device)
        self._tensor(scales, self.torch.float32, "scales", 1, a.device)
        if scales.shape != (b.shape[1],):
            raise ValueError("scales must have shape [N], one scale per output channel")
        out, dims = self._gemm_args(a, b, bias, config, output_dtype, self.torch.int8)
        ws = self.torch.empty(out.shape, dtype=self.torch.float32, device=out.device) if config >= 6 else None
        tensors = (a, b, scales, bias, out, ws)
        self._call("ti_v2_gemm_ex_i8", tensors, tuple(map(self._ptr, tensors)) + dims)
        return out

    def legacy_gemm(self, a, b):
        self._tensor(a, self.torch.float32, "a", 2)
        self._tensor(b, self.torch.float32, "b", 2, a.device)
        if a.shape[1] != b.shape[0] or (a.shape[0] - 1) // 64 + 1 > 65535:
            raise ValueError("invalid FP32 GEMM dimensions")
        out = self.torch.empty((a.shape[0], b.shape[1]), dtype=a.dtype, device=a.device)
        tensors = (a, b, out)
        self._call("ti_v2_legacy_gemm_f32", tensors,
                   tuple(map(self._ptr, tensors)) + (a.shape[0], b.shape[1], a.shape[1]))
        return out

    def layernorm(self, x, gamma, beta, *, eps=1e-5):
        t = self.torch
        self._tensor(x, t.float16, "x")
        self._tensor(gamma, t.float16, "gamma", 1, x.device)
        self._tensor(beta, t.float16, "beta", 1, x.device)
        cols = x.shape[-1]
        rows = _dim(x.numel() // cols, "rows")
        if gamma.shape != (cols,) or beta.shape != (cols,) or not math.isfinite(eps) or eps <= 0:
            raise ValueError("LayerNorm gamma/beta shape or eps invalid")
        out = t.empty_like(x)
        tensors = (x, gamma, beta, out)
        self._call("ti_v2_layernorm_f16", tensors, tuple(map(self._ptr, tensors)) + (rows, cols, eps))
        return out

    def gelu_new(self, x):
        self._tensor(x, self.torch.float16, "x")
        out = self.torch.empty_like(x)
        self._call("ti_v2_gelu_new_f16", (x, out), (x.data_ptr(), out.data_ptr(), x.numel()))
        return out

    def softmax(self, x):
        self._tensor(x, self.torch.float16, "x")
        cols = x.shape[-1]
        rows = _dim(x.numel() // cols, "rows")
        out = self.torch.empty_like(x)
        self._call("ti_v2_softmax_f16", (x, out), (x.data_ptr(), out.data_ptr(), rows, cols))
        return out

    def attention(self, q, k, v, *, q_lengths=None, kv_lengths=None, query_offsets=None,
                  causal=True, config=0):
        t = self.torch
        self._tensor(q, t.float16, "q", 4)
        self._tensor(k, t.float16, "k", 4, q.device)
        self._tensor(v, t.float16, "v", 4, q.device)
        batch, heads, nq, d = q.shape
        nk = k.shape[2]
        if k.shape != v.shape or k.shape[:2] != q.shape[:2] or k.shape[3] != d or d not in (64, 128):
            raise ValueError("attention expects q[B,H,Q,D], k/v[B,H,K,D], D64/128")
        if (batch > 65535 or heads > 65535 or type(causal) is not bool or type(config) is not int
                or config not in (0, 1)):
            raise ValueError("invalid attention grid, causal flag or config")
        ql = _metadata(q_lengths, batch, nq, nq, "q_lengths")
        kl = _metadata(kv_lengths, batch, nk, nk, "kv_lengths")
        offsets = _metadata(query_offsets, batch, 0, _I32_MAX - nq, "query_offsets")
        with t.cuda.device(q.device):
            meta = tuple(t.tensor(vals, dtype=t.int32, device=q.device) for vals in (ql, kl, offsets))
            out = t.empty_like(q)
            tensors = (q, k, v, out) + meta
            self._call("ti_v2_attention_f16", tensors,
                       tuple(map(self._ptr, tensors)) + (batch, heads, nq, nk, d, int(causal), config))
        return out
