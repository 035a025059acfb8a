"""Torch-facing ctypes binding of the v2 kernel ABI (libtinyinfer_backend.so).

The public surface is the one reference llm/native_ops.py:33-210 gives its
callers: ``NativeOps`` with ``gemm``, ``gemm_int8``, ``legacy_gemm``,
``layernorm``, ``gelu_new``, ``softmax`` and ``attention``; the module constant
``GEMM_CATALOG`` (reference :14-16) that the library's catalog JSON must equal;
and the exception contract -- ``TypeError`` for an operand that is not a
contiguous device tensor of the right dtype, ``ValueError`` for a bad rank,
extent, device, integer argument or a tensor that requires grad,
``RuntimeError`` carrying ``ti_v2_last_error()`` for a nonzero native status.

How it is built here: every native symbol is described by a string of
parameter codes (``_ABI``); each call goes through a ``_Call`` that validates
the operands in argument order, allocates outputs on the operands' device,
records every tensor on the current torch stream (the caller's allocator must
not recycle them while the queued kernels run), and appends that stream and the
device index as the ABI's last two arguments.  There is no CPU path: the
library must be built, and the operands must already live on the GPU.
"""
from __future__ import annotations

import ctypes
import json
import math
from pathlib import Path

from . import BACKEND_LIB, require

INT32_MAX = 2**31 - 1
INT64_MAX = 2**63 - 1

# The 12 GEMM configurations the library must report, in order (the reference
# catalog, kernels/src/cuda/tc/catalog.cuh:8-15): three CUDA tile hints, one or
# two stages, fused bias epilogue for ids 0-5, a caller FP32 workspace for 6-11.
_TILE_HINTS = ((32, 32, 16, 4), (64, 32, 32, 8), (64, 64, 32, 8))
GEMM_CATALOG = tuple(
    {"id": cid, "tile": _TILE_HINTS[cid % 3],
     "stages": 2 if (cid % 6) < 3 else 1,
     "epilogue": "fused" if cid < 6 else "separate"}
    for cid in range(12))

# Parameter codes of each entry point, before the implicit (stream, device)
# trailer: p = pointer, i = int, f = float, q = int64.
_ABI = {
    "ti_v2_gemm_f16": "ppppiiiii",
    "ti_v2_gemm_i8": "pppppiiiii",
    "ti_v2_gemm_ex_f16": "pppppiiiii",
    "ti_v2_gemm_ex_i8": "ppppppiiiii",
    "ti_v2_legacy_gemm_f32": "pppiii",
    "ti_v2_attention_f16": "pppppppiiiiiii",
    "ti_v2_layernorm_f16": "ppppiif",
    "ti_v2_gelu_new_f16": "ppq",
    "ti_v2_softmax_f16": "ppii",
}
_CTYPE = {"p": ctypes.c_void_p, "i": ctypes.c_int, "f": ctypes.c_float, "q": ctypes.c_int64}
_TRAILER = [ctypes.c_size_t, ctypes.c_int]   # hipStream_t as uintptr_t, device ordinal


def _count(value, name, low=1, high=INT32_MAX):
    """An exact int (bool excluded) in [low, high], else ValueError."""
    if type(value) is not int or value < low or value > high:
        raise ValueError(f"{name} must be an integer in [{low}, {high}]")
    return value


def _per_request(value, batch, default, upper, name):
    """Host metadata for each of `batch` requests: None (every request gets
    `default`), a single int for all, or a sequence of `batch` ints in [0, upper]."""
    if value is None:
        return [default] * batch
    seq = [value] * batch if type(value) is int else list(value)
    if len(seq) != batch:
        raise ValueError(f"{name} must hold {batch} entries, got {len(seq)}")
    for item in seq:
        _count(item, name, 0, upper)
    return seq


class _Call:
    """One native call being assembled: operands are checked and their
    pointers appended in the ABI's argument order."""

    def __init__(self, ops, symbol):
        self.ops, self.symbol = ops, symbol
        self.args, self.held = [], []
        self.device = None

    def operand(self, x, dtype, name, rank=None, shape=None):
        torch = self.ops.torch
        if not isinstance(x, torch.Tensor) or x.device.type != "cuda":
            raise TypeError(f"{name}: a GPU (torch 'cuda' device) tensor is required")
        if x.dtype != dtype:
            raise TypeError(f"{name}: dtype {x.dtype} given, {dtype} required")
        if not x.is_contiguous():
            raise TypeError(f"{name}: contiguous row-major storage required")
        if x.requires_grad:
            raise ValueError(f"{name}: tensors that require grad are not accepted (inference only)")
        if rank is not None and x.dim() != rank:
            raise ValueError(f"{name}: rank {rank} required, got {x.dim()}")
        if x.dim() == 0 or x.numel() == 0:
            raise ValueError(f"{name}: an empty or zero-rank tensor is not accepted")
        for axis, extent in enumerate(x.shape):
            _count(extent, f"{name}.shape[{axis}]")
        if x.numel() * x.element_size() > INT64_MAX:
            raise ValueError(f"{name}: byte extent beyond signed 64-bit indexing")
        if self.device is None:
            self.device = x.device
        elif x.device != self.device:
            raise ValueError(f"{name}: on {x.device}, the call's operands are on {self.device}")
        if shape is not None and tuple(x.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {tuple(shape)} required, got {tuple(x.shape)}")
        self.held.append(x)
        self.args.append(x.data_ptr())
        return x

    def optional(self, x, dtype, name, shape):
        if x is None:
            self.args.append(None)
            return None
        return self.operand(x, dtype, name, shape=shape)

    def output(self, shape, dtype):
        y = self.ops.torch.empty(shape, dtype=dtype, device=self.device)
        self.held.append(y)
        self.args.append(y.data_ptr())
        return y

    def workspace(self, shape, needed):
        if not needed:
            self.args.append(None)
            return None
        return self.output(shape, self.ops.torch.float32)

    def scalars(self, *values):
        self.args.extend(values)

    def run(self):
        torch = self.ops.torch
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device)
            for x in self.held:
                x.record_stream(stream)
            status = getattr(self.ops.lib, self.symbol)(*self.args, stream.cuda_stream, self.device.index)
        if status != 0:
            detail = self.ops.lib.ti_v2_last_error().decode("utf-8", errors="replace")
            raise RuntimeError(f"{self.symbol} failed ({status}): {detail}")


class NativeOps:
    """Inference-only device ops over the v2 ABI; operands are torch GPU tensors,
    work is queued on the current torch stream of their device."""

    def __init__(self, library_path=None):
        import torch
        self.torch = torch
        where = require(BACKEND_LIB) if library_path is None else library_path
        self.library_path = str(Path(where).expanduser().resolve(strict=True))
        self.lib = ctypes.CDLL(self.library_path)
        self._declare("ti_v2_abi_version", [], ctypes.c_int)
        self._declare("ti_v2_last_error", [], ctypes.c_char_p)
        self._declare("ti_v2_gemm_catalog_json", [], ctypes.c_char_p)
        for symbol, codes in _ABI.items():
            self._declare(symbol, [_CTYPE[c] for c in codes] + _TRAILER, ctypes.c_int)
        if self.lib.ti_v2_abi_version() != 2:
            raise RuntimeError("native v2 ABI version mismatch: version 2 required")
        self.catalog = json.loads(self.lib.ti_v2_gemm_catalog_json())
        listed = tuple({**entry, "tile": tuple(entry["tile"])} for entry in self.catalog["configs"])
        if listed != GEMM_CATALOG:
            raise RuntimeError("native GEMM catalog differs from the wrapper's GEMM_CATALOG")

    def _declare(self, symbol, argtypes, restype):
        fn = getattr(self.lib, symbol)
        fn.argtypes, fn.restype = argtypes, restype

    # -- GEMMs --------------------------------------------------------------
    def _linear(self, symbol, a, weight, weight_dtype, scales, bias, config, output_dtype):
        torch = self.torch
        call = _Call(self, symbol)
        call.operand(a, torch.float16, "a", rank=2)
        call.operand(weight, weight_dtype, "b", rank=2)
        if scales is not None:
            call.operand(scales, torch.float32, "scales", rank=1)
            if scales.shape[0] != weight.shape[1]:
                raise ValueError("scales must have shape [N], one scale per output column")
        m, k = a.shape
        if weight.shape[0] != k:
            raise ValueError(f"a is [{m}, {k}] but b has {weight.shape[0]} rows")
        n = weight.shape[1]
        if type(config) is not int or config not in range(len(GEMM_CATALOG)):
            raise ValueError(f"GEMM config must be one of the catalog ids 0..{len(GEMM_CATALOG) - 1}")
        only = self.catalog.get("only_config", -1)
        if only not in (-1, config):
            raise ValueError(f"this build compiles only GEMM config {only}")
        rows_per_tile = GEMM_CATALOG[config]["tile"][0]
        if (m + rows_per_tile - 1) // rows_per_tile > 65535:
            raise ValueError("M needs more than 65535 row tiles")
        call.optional(bias, torch.float16, "bias", shape=(n,))
        out_dtype = torch.float16 if output_dtype is None else output_dtype
        if out_dtype not in (torch.float16, torch.float32):
            raise TypeError("output_dtype must be torch.float16 or torch.float32")
        y = call.output((m, n), out_dtype)
        call.workspace((m, n), GEMM_CATALOG[config]["epilogue"] == "separate")
        call.scalars(m, n, k, 1 if out_dtype == torch.float32 else 0, config)
        call.run()
        return y

    def gemm(self, a, b, *, bias=None, config=0, output_dtype=None):
        """y = a[M,K] @ b[K,N] (+ bias), fp16 weights, fp32 accumulation."""
        return self._linear("ti_v2_gemm_ex_f16", a, b, self.torch.float16, None, bias, config, output_dtype)

    def gemm_int8(self, a, b, scales, *, bias=None, config=0, output_dtype=None):
        """W8A16: b int8 [K,N] with one fp32 scale per output column."""
        if scales is None:
            raise TypeError("scales: a GPU (torch 'cuda' device) tensor is required")
        return self._linear("ti_v2_gemm_ex_i8", a, b, self.torch.int8, scales, bias, config, output_dtype)

    def legacy_gemm(self, a, b):
        """FP32 y = a @ b through ti_v2_legacy_gemm_f32."""
        torch = self.torch
        call = _Call(self, "ti_v2_legacy_gemm_f32")
        call.operand(a, torch.float32, "a", rank=2)
        call.operand(b, torch.float32, "b", rank=2)
        (m, k), n = a.shape, b.shape[1]
        if b.shape[0] != k or (m + 63) // 64 > 65535:
            raise ValueError(f"FP32 GEMM: a [{m}, {k}] and b {list(b.shape)} do not multiply within the grid limit")
        y = call.output((m, n), torch.float32)
        call.scalars(m, n, k)
        call.run()
        return y

    # -- row ops -------------------------------------------------------------
    def _rows(self, x):
        cols = x.shape[-1]
        return _count(x.numel() // cols, "rows"), cols

    def layernorm(self, x, gamma, beta, *, eps=1e-5):
        """fp16 LayerNorm over the last axis, gamma/beta fp16 [cols]."""
        torch = self.torch
        call = _Call(self, "ti_v2_layernorm_f16")
        call.operand(x, torch.float16, "x")
        rows, cols = self._rows(x)
        call.operand(gamma, torch.float16, "gamma", rank=1)
        call.operand(beta, torch.float16, "beta", rank=1)
        if gamma.shape[0] != cols or beta.shape[0] != cols:
            raise ValueError(f"gamma and beta must have shape [{cols}]")
        if not (isinstance(eps, (int, float)) and math.isfinite(eps) and eps > 0):
            raise ValueError("eps must be finite and positive")
        y = call.output(tuple(x.shape), torch.float16)
        call.scalars(rows, cols, float(eps))
        call.run()
        return y

    def gelu_new(self, x):
        """fp16 tanh-approximation GELU, elementwise."""
        call = _Call(self, "ti_v2_gelu_new_f16")
        call.operand(x, self.torch.float16, "x")
        y = call.output(tuple(x.shape), self.torch.float16)
        call.scalars(x.numel())
        call.run()
        return y

    def softmax(self, x):
        """fp16 softmax over the last axis."""
        call = _Call(self, "ti_v2_softmax_f16")
        call.operand(x, self.torch.float16, "x")
        rows, cols = self._rows(x)
        y = call.output(tuple(x.shape), self.torch.float16)
        call.scalars(rows, cols)
        call.run()
        return y

    # -- attention -------------------------------------------------------------
    def attention(self, q, k, v, *, q_lengths=None, kv_lengths=None, query_offsets=None,
                  causal=True, config=0):
        """q [B,H,Q,D], k/v [B,H,K,D] fp16, D in {64, 128}; per-request query
        and key counts and absolute query offsets for the causal mask."""
        torch = self.torch
        call = _Call(self, "ti_v2_attention_f16")
        call.operand(q, torch.float16, "q", rank=4)
        batch, heads, nq, dim = q.shape
        call.operand(k, torch.float16, "k", rank=4)
        call.operand(v, torch.float16, "v", rank=4)
        nk = k.shape[2]
        if (tuple(v.shape) != tuple(k.shape) or tuple(k.shape[:2]) != (batch, heads)
                or k.shape[3] != dim or dim not in (64, 128)):
            raise ValueError("attention takes q [B,H,Q,D] and k, v [B,H,K,D] with D 64 or 128")
        if batch > 65535 or heads > 65535:
            raise ValueError("batch and heads must each be at most 65535")
        if type(causal) is not bool or type(config) is not int or config not in (0, 1):
            raise ValueError("causal must be a bool and config 0 or 1")
        meta = (_per_request(q_lengths, batch, nq, nq, "q_lengths"),
                _per_request(kv_lengths, batch, nk, nk, "kv_lengths"),
                _per_request(query_offsets, batch, 0, INT32_MAX - nq, "query_offsets"))
        with torch.cuda.device(q.device):
            y = call.output(tuple(q.shape), torch.float16)
            for values in meta:
                call.held.append(torch.tensor(values, dtype=torch.int32, device=q.device))
                call.args.append(call.held[-1].data_ptr())
        call.scalars(batch, heads, nq, nk, dim, int(causal), config)
        call.run()
        return y
