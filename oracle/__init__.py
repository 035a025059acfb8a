"""ORACLE — test infrastructure, not product code.

numpy/ctypes access to ``liboracle.so`` (oracle/oracle.cpp), the CPU
restatement of the reference tinyinfer arithmetic, and to ``_ref/libref_cpu.so``,
the reference's own CPU kernels and INT8 codec compiled from
/root/reference by oracle/Makefile.  Only tests/, ``__graft_entry__.smoke()``
and the ``cpu_baseline`` leg of bench.py may import this package, and only as
the checker or as the timed CPU baseline; the product libraries never call it.

Every function here names the reference file:line it restates in
oracle/oracle.cpp; tests/test_oracle.py pins each one against the reference's
golden vectors, the compiled reference (where it builds) and closed forms.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libref_cpu.so"

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)
        _lib = C.CDLL(str(LIB_PATH))
    return _lib


def ref_lib():
    """The reference's own CPU code, or None where it was not built."""
    global _ref
    if _ref is None and REF_PATH.is_file():
        _ref = C.CDLL(str(REF_PATH))
    return _ref


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# -- fp16 -------------------------------------------------------------------------
def f32_to_f16_bits(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_f16(_p(x), _p(out), C.c_int64(x.size))
    return out


def f16_bits_to_f32(x):
    x = _c(x, np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().or_f16_to_f32(_p(x), _p(out), C.c_int64(x.size))
    return out


# -- codec --------------------------------------------------------------------------
def quantize(w_bits):
    """fp16 bits [K,N] -> (int8 q [K,N], fp32 scales [N])."""
    w = _c(w_bits, np.uint16)
    k, n = w.shape
    q = np.empty((k, n), np.int8)
    s = np.empty(n, np.float32)
    if lib().or_quantize(_p(w), C.c_int64(k), C.c_int64(n), _p(q), _p(s)):
        raise ValueError("non-finite fp16 input")
    return q, s


def dequantize(q, scales):
    q = _c(q, np.int8)
    s = _c(scales, np.float32)
    out = np.empty(q.shape, np.uint16)
    lib().or_dequantize(_p(q), _p(s), C.c_int64(q.shape[0]), C.c_int64(q.shape[1]), _p(out))
    return out


# -- linear ---------------------------------------------------------------------------
def linear(a_bits, *, q=None, scales=None, w_bits=None, bias_bits=None, out_dtype="f16",
           gelu=False):
    """y = A @ W (+ bias) with fp32 accumulation; W given as int8+scales or fp16 bits.
    Returns fp16 bits (out_dtype 'f16') or float32."""
    a = _c(a_bits, np.uint16)
    m, k = a.shape
    if w_bits is not None:
        w = _c(w_bits, np.uint16)
        n = w.shape[1]
        qq = ss = None
    else:
        qq, ss, w = _c(q, np.int8), _c(scales, np.float32), None
        n = qq.shape[1]
    bias = None if bias_bits is None else _c(bias_bits, np.uint16)
    dt = 1 if out_dtype == "f32" else 0
    out = np.empty((m, n), np.float32 if dt else np.uint16)
    lib().or_linear(_p(a), _p(qq), _p(ss), _p(w), _p(bias), C.c_int(m), C.c_int(n), C.c_int(k),
                    C.c_int(dt), C.c_int(1 if gelu else 0), _p(out))
    return out


def matmul_blocked(a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty((a.shape[0], b.shape[1]), np.float32)
    lib().or_matmul_blocked(_p(a), _p(b), _p(out), C.c_int(a.shape[0]), C.c_int(b.shape[1]),
                            C.c_int(a.shape[1]))
    return out


# -- row ops ---------------------------------------------------------------------------
def layernorm_f16(x_bits, g_bits, b_bits, eps=1e-5):
    x = _c(x_bits, np.uint16)
    cols = x.shape[-1]
    rows = x.size // cols
    out = np.empty(x.shape, np.uint16)
    lib().or_layernorm_f16(_p(x), _p(_c(g_bits, np.uint16)), _p(_c(b_bits, np.uint16)), _p(out),
                           C.c_int(rows), C.c_int(cols), C.c_float(eps))
    return out


def softmax_f16(x_bits):
    x = _c(x_bits, np.uint16)
    cols = x.shape[-1]
    out = np.empty(x.shape, np.uint16)
    lib().or_softmax_f16(_p(x), _p(out), C.c_int(x.size // cols), C.c_int(cols))
    return out


def gelu_f16(x_bits):
    x = _c(x_bits, np.uint16)
    out = np.empty(x.shape, np.uint16)
    lib().or_gelu_f16(_p(x), _p(out), C.c_int64(x.size))
    return out


def _rowop32(name, x, *extra):
    x = _c(x, np.float32)
    cols = x.shape[-1]
    out = np.empty(x.shape, np.float32)
    args = [_p(x)]
    if extra:
        args += [_p(_c(extra[0], np.float32)), _p(_c(extra[1], np.float32))]
    args += [_p(out), C.c_int(x.size // cols), C.c_int(cols)]
    if extra:
        args.append(C.c_float(extra[2]))
    getattr(lib(), name)(*args)
    return out


def layernorm_f32_exact(x, g, b, eps=1e-5):
    return _rowop32("or_layernorm_f32_exact", x, g, b, eps)


def layernorm_f32_fused(x, g, b, eps=1e-5):
    return _rowop32("or_layernorm_f32_fused", x, g, b, eps)


def softmax_f32_exact(x):
    return _rowop32("or_softmax_f32_exact", x)


def softmax_f32_fused(x):
    return _rowop32("or_softmax_f32_fused", x)


# -- attention -----------------------------------------------------------------------
def attention_f16(q_bits, k_bits, v_bits, q_lengths, kv_lengths, offsets, causal=True):
    q, k, v = (_c(t, np.uint16) for t in (q_bits, k_bits, v_bits))
    b, h, nq, d = q.shape
    nk = k.shape[2]
    ql, kl, off = (_c(t, np.int32) for t in (q_lengths, kv_lengths, offsets))
    out = np.empty(q.shape, np.uint16)
    lib().or_attention_f16(_p(q), _p(k), _p(v), _p(out), _p(ql), _p(kl), _p(off), C.c_int(b),
                           C.c_int(h), C.c_int(nq), C.c_int(nk), C.c_int(d), C.c_int(int(causal)))
    return out


def num_threads():
    return lib().or_num_threads()


# -- GPT-2 -----------------------------------------------------------------------------
class _Weights(C.Structure):
    _fields_ = [("layers", C.c_int), ("heads", C.c_int), ("hidden", C.c_int), ("vocab", C.c_int),
                ("ctx", C.c_int), ("wte", C.c_void_p), ("wpe", C.c_void_p), ("lnf_g", C.c_void_p),
                ("lnf_b", C.c_void_p), ("ln1_g", C.c_void_p), ("ln1_b", C.c_void_p),
                ("ln2_g", C.c_void_p), ("ln2_b", C.c_void_p), ("w", C.c_void_p * 4),
                ("s", C.c_void_p * 4), ("bias", C.c_void_p * 4), ("head_q", C.c_void_p),
                ("head_s", C.c_void_p), ("w16", C.c_void_p * 4), ("head16", C.c_void_p)]


_LINEARS = ("attn.c_attn", "attn.c_proj", "mlp.c_fc", "mlp.c_proj")


class Gpt2:
    """CPU GPT-2 restating reference llm/src/runtime.cu, fed from a dict of numpy
    arrays keyed by the artifact's tensor names: INT8 weight-only linears
    (dequantised fp16_rn(q * scale)) or, for fp16-precision artifacts, fp16
    linears used as stored (reference runtime.cu:97-113)."""

    def __init__(self, tensors, arch, slots, capacity):
        L = arch["layers"]
        keep = []

        def ptr(name, dtype):
            arr = np.ascontiguousarray(tensors[name], dtype=dtype)
            keep.append(arr)
            return arr.ctypes.data

        def table(ptrs):
            arr = (C.c_void_p * len(ptrs))(*ptrs)
            keep.append(arr)
            return C.cast(arr, C.c_void_p)

        w = _Weights()
        w.layers, w.heads, w.hidden = L, arch["heads"], arch["hidden"]
        w.vocab, w.ctx = arch["vocab"], arch["capacity"]
        w.wte = ptr("transformer.wte.weight", np.uint16)
        w.wpe = ptr("transformer.wpe.weight", np.uint16)
        w.lnf_g = ptr("transformer.ln_f.weight", np.uint16)
        w.lnf_b = ptr("transformer.ln_f.bias", np.uint16)
        for field, ln, part in (("ln1_g", "ln_1", "weight"), ("ln1_b", "ln_1", "bias"),
                                ("ln2_g", "ln_2", "weight"), ("ln2_b", "ln_2", "bias")):
            setattr(w, field, table([ptr(f"transformer.h.{l}.{ln}.{part}", np.uint16) for l in range(L)]))
        # fp16-precision artifacts keep the linears and the head as fp16 bits.
        fp16 = tensors["lm_head.weight"].dtype == np.uint16
        for i, lin in enumerate(_LINEARS):
            if fp16:
                w.w16[i] = table([ptr(f"transformer.h.{l}.{lin}.weight", np.uint16) for l in range(L)])
            else:
                w.w[i] = table([ptr(f"transformer.h.{l}.{lin}.weight", np.int8) for l in range(L)])
                w.s[i] = table([ptr(f"transformer.h.{l}.{lin}.weight.scales", np.float32) for l in range(L)])
            w.bias[i] = table([ptr(f"transformer.h.{l}.{lin}.bias", np.uint16) for l in range(L)])
        if fp16:
            w.head16 = ptr("lm_head.weight", np.uint16)
        else:
            w.head_q = ptr("lm_head.weight", np.int8)
            w.head_s = ptr("lm_head.weight.scales", np.float32)
        lib().or_gpt2_create.restype = C.c_void_p
        self._h = C.c_void_p(lib().or_gpt2_create(C.byref(w), C.c_int(slots), C.c_int(capacity)))
        self.vocab = arch["vocab"]
        del keep  # the model copied what it needs

    def close(self):
        if self._h:
            lib().or_gpt2_destroy(self._h)
            self._h = C.c_void_p()

    __del__ = close

    def reset(self, slot):
        lib().or_gpt2_reset(self._h, C.c_int(slot))

    def length(self, slot):
        return lib().or_gpt2_length(self._h, C.c_int(slot))

    def forward(self, slots, rows, *, logits=True):
        b = len(rows)
        stride = max(len(r) for r in rows)
        toks = np.zeros((b, stride), np.int32)
        for i, r in enumerate(rows):
            toks[i, :len(r)] = r
        lens = np.array([len(r) for r in rows], np.int32)
        ss = np.array(slots, np.int32)
        out = np.empty((b, self.vocab), np.float32) if logits else None
        nxt = np.empty(b, np.int32)
        lib().or_gpt2_forward(self._h, _p(ss), _p(toks), _p(lens), C.c_int(b), C.c_int(stride),
                              _p(out), _p(nxt))
        return out, nxt

    def greedy(self, slots, prompts, max_new):
        b = len(prompts)
        stride = max(len(r) for r in prompts)
        toks = np.zeros((b, stride), np.int32)
        for i, r in enumerate(prompts):
            toks[i, :len(r)] = r
        lens = np.array([len(r) for r in prompts], np.int32)
        req = np.array([max_new] * b if isinstance(max_new, int) else max_new, np.int32)
        out_stride = int(req.max())
        out = np.empty((b, out_stride), np.int32)
        lib().or_gpt2_greedy(self._h, _p(np.array(slots, np.int32)), _p(toks), _p(lens), _p(req),
                             C.c_int(b), C.c_int(stride), _p(out), C.c_int(out_stride))
        return [list(out[i, :req[i]]) for i in range(b)]
