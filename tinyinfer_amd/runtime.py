"""Standard-library ctypes binding of the GPT-2 runtime ABI (libtinyinfer_llm.so).

Interface kept from reference llm/runtime.py:10-165 so its callers run
unchanged: the ``Options`` (28 bytes) and ``Trace`` (96 bytes) structures with
their field order, ``_rows`` (ragged token rows -> zero-padded int32 [B, stride],
lengths, stride), and ``NativeModel(library, manifest, *, device, max_batch,
cache_slots, capacity, gemm_config, attention_config)`` with ``forward``,
``greedy``, ``score``, ``lengths``, ``trace``, ``reset``, ``reset_all``,
``close`` and context-manager use, returning the same dictionaries.  Bad
integer arguments raise ``ValueError``; a nonzero native status raises
``RuntimeError`` with ``ti_llm_last_error()``.

Importing this module imports neither torch nor numpy: token rows are packed
with ``array('i')`` buffers that ctypes views without copying, and every native
call is synchronous (the library owns the device, stream and buffers).  The
vocabulary comes from the manifest's architecture block when it has one (GPT-2
XL artifacts), else GPT-2's 50257.
"""
from __future__ import annotations

import ctypes as C
import json
from array import array
from pathlib import Path

VOCAB = 50257


class Options(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("device", C.c_int32), ("max_batch", C.c_int32),
                ("cache_slots", C.c_int32), ("capacity", C.c_int32), ("gemm_config", C.c_int32),
                ("attention_config", C.c_int32)]


class Trace(C.Structure):
    _fields_ = [(field, C.c_uint64) for field in (
        "forward_calls", "embedding", "gemm_fp16", "gemm_int8", "layernorm", "gelu", "attention",
        "residual", "kv_scatter_gather", "lm_head", "argmax", "nll")]


_P, _I = C.c_void_p, C.c_int32
# Argument and result types of each ti_llm_* entry point.
_LLM_ABI = {
    "ti_llm_abi_version": ([], C.c_int),
    "ti_llm_last_error": ([], C.c_char_p),
    "ti_llm_create": ([C.c_char_p, C.POINTER(Options), C.POINTER(_P)], C.c_int),
    "ti_llm_destroy": ([_P], C.c_int),
    "ti_llm_reset": ([_P, _I], C.c_int),
    "ti_llm_lengths": ([_P, _P, _I], C.c_int),
    "ti_llm_get_trace": ([_P, C.POINTER(Trace)], C.c_int),
    "ti_llm_forward_batch": ([_P, _P, _P, _P, _I, _I, _P, _P], C.c_int),
    "ti_llm_greedy_batch": ([_P, _P, _P, _P, _P, _I, _I, _P, _I, _P, _P, _P], C.c_int),
    "ti_llm_score_window": ([_P, _P, _P, _I, _P, _P, _P], C.c_int),
}


def _bounded(value, name, low, high):
    """An exact int (bool excluded) in [low, high], else ValueError."""
    if type(value) is not int or value < low or value > high:
        raise ValueError(f"{name} must be an integer in [{low},{high}]")
    return value


def _int32(values):
    """A ctypes int32 view over an array('i') of `values` (no per-item ctypes objects)."""
    buf = array("i", values)
    return (C.c_int32 * len(buf)).from_buffer(buf)


def _rows(rows, vocab=VOCAB):
    """Ragged token rows -> (int32 [B * stride] zero-padded, int32 lengths [B], stride)."""
    if not rows:
        raise ValueError("token batch is empty")
    lengths = [len(row) for row in rows]
    if min(lengths) == 0:
        raise ValueError(f"token row {lengths.index(0)} is empty")
    stride = max(lengths)
    flat = array("i", bytes(4 * stride * len(rows)))
    for b, row in enumerate(rows):
        base = b * stride
        for j, token in enumerate(row):
            flat[base + j] = _bounded(token, "token", 0, vocab - 1)
    return (C.c_int32 * len(flat)).from_buffer(flat), _int32(lengths), stride


class NativeModel:
    """One GPT-2 context of libtinyinfer_llm: weights, KV slots and a stream on
    one device.  Calls are synchronous; callers serialise calls on one model."""

    def __init__(self, library, manifest, *, device=0, max_batch=32, cache_slots=32, capacity=1024,
                 gemm_config=0, attention_config=0):
        _bounded(max_batch, "max_batch", 1, 32)
        self.options = Options(
            C.sizeof(Options), _bounded(device, "device", 0, 1024), max_batch,
            _bounded(cache_slots, "cache_slots", max_batch, 1024), _bounded(capacity, "capacity", 2, 1024),
            _bounded(gemm_config, "gemm_config", 0, 11), _bounded(attention_config, "attention_config", 0, 1))
        self.library_path = str(Path(library).resolve())
        self.manifest_path = str(Path(manifest).resolve())
        self.manifest = json.loads(Path(self.manifest_path).read_text(encoding="ascii"))
        self.vocab = int(self.manifest.get("architecture", {}).get("vocab", VOCAB))
        self.lib = C.CDLL(self.library_path)
        for symbol, (argtypes, restype) in _LLM_ABI.items():
            fn = getattr(self.lib, symbol)
            fn.argtypes, fn.restype = argtypes, restype
        if self.lib.ti_llm_abi_version() != 1:
            raise RuntimeError("libtinyinfer_llm reports an ABI version other than 1")
        self._model = C.c_void_p()
        self._status(self.lib.ti_llm_create(self.manifest_path.encode(), C.byref(self.options),
                                            C.byref(self._model)))

    # -- plumbing ------------------------------------------------------------
    def _status(self, code):
        if code != 0:
            why = self.lib.ti_llm_last_error().decode("utf-8", errors="replace")
            raise RuntimeError(f"ti_llm status {code}: {why}")

    def _invoke(self, symbol, *args):
        if not self._model:
            raise RuntimeError("model is closed")
        self._status(getattr(self.lib, symbol)(self._model, *args))

    def _slot_ids(self, slots):
        top = self.options.cache_slots - 1
        return _int32([_bounded(s, "slot", 0, top) for s in slots])

    # -- lifetime --------------------------------------------------------------
    def close(self):
        if self._model:
            handle, self._model = self._model, C.c_void_p()
            self._status(self.lib.ti_llm_destroy(handle))

    def __enter__(self):
        return self

    def __exit__(self, *_exc):
        self.close()

    # -- cache state -------------------------------------------------------------
    def reset(self, slot):
        self._invoke("ti_llm_reset", _bounded(slot, "slot", 0, self.options.cache_slots - 1))

    def reset_all(self):
        for slot in range(self.options.cache_slots):
            self.reset(slot)

    def lengths(self):
        out = _int32([0] * self.options.cache_slots)
        self._invoke("ti_llm_lengths", out, len(out))
        return list(out)

    def trace(self):
        counters = Trace()
        self._invoke("ti_llm_get_trace", C.byref(counters))
        return {field: getattr(counters, field) for field, _ in Trace._fields_}

    # -- inference -----------------------------------------------------------------
    def forward(self, slots, rows, *, return_logits=True, return_next=True):
        """Append each row to its slot's cache; last-position logits (flat
        float32 ctypes buffer, shape [B, vocab]) and greedy next ids."""
        batch = len(rows)
        if len(slots) != batch or batch > self.options.max_batch:
            raise ValueError("slots and rows must have one entry per request, at most max_batch")
        slot_ids = self._slot_ids(slots)
        tokens, lengths, stride = _rows(rows, self.vocab)
        logits = (C.c_float * (batch * self.vocab))() if return_logits else None
        next_ids = _int32([0] * batch) if return_next else None
        self._invoke("ti_llm_forward_batch", slot_ids, tokens, lengths, batch, stride, logits, next_ids)
        return {"logits": logits, "shape": [batch, self.vocab],
                "next_tokens": None if next_ids is None else list(next_ids)}

    def greedy(self, prompts, max_new_tokens, *, slots=None):
        """Prefill each prompt into its slot, then greedy-decode max_new_tokens
        (an int, or one count per request) tokens per request."""
        batch = len(prompts)
        if batch == 0 or batch > self.options.max_batch:
            raise ValueError("greedy takes 1..max_batch prompts")
        slot_list = list(range(batch)) if slots is None else list(slots)
        counts = [max_new_tokens] * batch if type(max_new_tokens) is int else list(max_new_tokens)
        if len(slot_list) != batch or len(counts) != batch:
            raise ValueError("slots and max_new_tokens must have one entry per prompt")
        counts = [_bounded(n, "max_new_tokens", 1, self.options.capacity) for n in counts]
        slot_ids = self._slot_ids(slot_list)
        tokens, lengths, stride = _rows(prompts, self.vocab)
        width = max(counts)
        out = _int32([-1] * (batch * width))
        produced = _int32([0] * batch)
        ttft, total = (C.c_double * batch)(), (C.c_double * batch)()
        self._invoke("ti_llm_greedy_batch", slot_ids, tokens, lengths, _int32(counts), batch, stride,
                     out, width, produced, ttft, total)
        return {"tokens": [list(out[b * width:b * width + produced[b]]) for b in range(batch)],
                "output_lengths": list(produced), "ttft_ms": list(ttft), "total_ms": list(total)}

    def score(self, tokens, mask, *, positions=False):
        """Teacher-forced NLL of a window in the internal scoring slot:
        sum over masked targets, their count, optionally per position."""
        length = len(tokens)
        if len(mask) != length or not 2 <= length <= self.options.capacity:
            raise ValueError("tokens and mask must have equal length in [2, capacity]")
        ids = _int32([_bounded(t, "token", 0, self.vocab - 1) for t in tokens])
        flags = (C.c_uint8 * length)(*[_bounded(m, "mask", 0, 1) for m in mask])
        total, count = C.c_double(), C.c_uint64()
        per_position = (C.c_double * length)() if positions else None
        self._invoke("ti_llm_score_window", ids, flags, length, C.byref(total), C.byref(count), per_position)
        return {"sum_nll": total.value, "target_count": count.value,
                "position_nll": None if per_position is None else list(per_position)}
