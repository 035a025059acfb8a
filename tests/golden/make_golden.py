"""Write the golden fixtures under tests/golden/ from the reference's own code.

Run in the build container (where /root/reference exists) after
`make -C oracle ref`, which compiles the reference's CPU kernels and INT8 host
codec from their sources (oracle/_ref/libref_cpu.so).  The fixtures are data:
inputs and the outputs the reference code produced for them.

  codec_vectors.npz  reference backend/host_codec.cpp: every finite fp16 bit
                     pattern as a [1984, 32] matrix, the fixed matrices of
                     reference fuzz/check_codec.py:21-25 and the exporter rows of
                     reference llm/tests/test_contracts.py:36, each quantized;
                     the dequantization case of check_codec.py:30-34.
  cpu_kernel_vectors.npz  reference kernels/src/cpu/{layernorm,softmax,matmul}.cpp
                     on seeded inputs at the shapes of reference
                     kernels/tests/test_cpu.cpp:33-71 (fewer rows).
"""
from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
import oracle  # noqa: E402


def p(a):
    return a.ctypes.data_as(C.c_void_p)


def ref_quantize(ref, bits, cols):
    bits = np.ascontiguousarray(bits, np.uint16)
    q = np.empty(bits.size, np.int8)
    s = np.empty(cols, np.float32)
    st = ref.ti_host_quantize_f16(p(bits), C.c_size_t(bits.size), C.c_size_t(cols), p(q),
                                  C.c_size_t(bits.size), p(s), C.c_size_t(cols))
    assert st == 0, st
    return q.reshape(-1, cols), s


def main():
    ref = oracle.ref_lib()
    if ref is None:
        raise SystemExit("oracle/_ref/libref_cpu.so is missing: run `make -C oracle ref` first")
    out = {}
    finite = np.array([i for i in range(65536) if (i & 0x7C00) != 0x7C00], np.uint16)
    out["all_half_in"] = finite.reshape(-1, 32)
    out["all_half_q"], out["all_half_s"] = ref_quantize(ref, finite, 32)
    fixed = [
        (np.array([0., -0., 1., -1., 127., -127., 0.5, -0.5, 1.5, -1.5], np.float16), 1),
        (np.array([0., 2**-24, 65504., -0., -2**-24, -65504.], np.float16), 3),
        (np.array([127., 127., 0.5, 1.5, 2.5, -2.5], np.float16), 2),
        (np.array([.12, 0, -3.25, 1.5, 0, 7.75, -2.0, 0, .125], np.float16), 3),
    ]
    for i, (vals, cols) in enumerate(fixed):
        bits = vals.view(np.uint16)
        out[f"fixed{i}_in"] = bits.reshape(-1, cols)
        out[f"fixed{i}_q"], out[f"fixed{i}_s"] = ref_quantize(ref, bits, cols)
    rng = np.random.default_rng(20261101)
    w = (rng.standard_normal((64, 48)) * 0.02).astype(np.float16)
    w[:, 5] = 0
    out["random_in"] = w.view(np.uint16)
    out["random_q"], out["random_s"] = ref_quantize(ref, w.view(np.uint16), 48)
    dq = np.array([[-127, -3, -1, 0, 1, 3, 127], [1, 2, 3, 4, 5, 6, 7]], np.int8)
    ds = np.array([2**-24, 0.5, 1., 1., 1., 2., np.float32(65504 / 127)], np.float32)
    half = np.empty(dq.size, np.uint16)
    assert ref.ti_host_dequantize_i8(p(dq), C.c_size_t(dq.size), C.c_size_t(7), p(ds), C.c_size_t(7),
                                     p(half), C.c_size_t(dq.size)) == 0
    out["deq_q"], out["deq_s"], out["deq_out"] = dq, ds, half.reshape(dq.shape)
    np.savez_compressed(HERE / "codec_vectors.npz", **out)

    k = {}
    for cols in (2, 64, 768, 1024, 4099):
        x = rng.uniform(-3, 5, (3, cols)).astype(np.float32)
        g = rng.uniform(0.5, 1.5, cols).astype(np.float32)
        b = rng.uniform(-1, 1, cols).astype(np.float32)
        y = np.empty_like(x)
        ref.ref_layernorm_fused(p(x), p(g), p(b), p(y), C.c_int(3), C.c_int(cols), C.c_float(1e-5))
        k[f"ln{cols}_x"], k[f"ln{cols}_g"], k[f"ln{cols}_b"], k[f"ln{cols}_y"] = x, g, b, y
    for cols in (1, 31, 128, 1000, 4097):
        x = rng.uniform(-8, 8, (3, cols)).astype(np.float32)
        y = np.empty_like(x)
        ref.ref_softmax_fused(p(x), p(y), C.c_int(3), C.c_int(cols))
        k[f"sm{cols}_x"], k[f"sm{cols}_y"] = x, y
    for m, n, kk in ((1, 1, 1), (7, 13, 5), (33, 65, 70)):
        a = rng.uniform(-1, 1, (m, kk)).astype(np.float32)
        bm = rng.uniform(-1, 1, (kk, n)).astype(np.float32)
        y = np.empty((m, n), np.float32)
        ref.ref_matmul_blocked(p(a), p(bm), p(y), C.c_int(m), C.c_int(n), C.c_int(kk))
        k[f"mm{m}_{n}_{kk}_a"], k[f"mm{m}_{n}_{kk}_b"], k[f"mm{m}_{n}_{kk}_y"] = a, bm, y
    np.savez_compressed(HERE / "cpu_kernel_vectors.npz", **k)
    print("wrote", ", ".join(sorted(f.name for f in HERE.glob("*.npz"))))


if __name__ == "__main__":
    main()
