"""GPU parity of the gfx950 kernels, called through the C ABI (NativeOps mirror of
reference llm/native_ops.py and ctypes), against the CPU oracle on identical
seeded inputs.

Tolerances (stated per north star): fp16 linear and attention outputs within
rtol 1e-2 / atol 2e-2 of the oracle's fp32-accumulate result; FP32 LayerNorm and
Softmax within 1e-4 relative; fp16 row ops within 1e-2/2e-2 (the reference's own
kernel gate, reference bench/v2/kernels/correctness.py:6).  Each test prints the
case it runs before launching, so a failing GPU run names its case.
"""
import ctypes as C
import gc

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-2, 2e-2


def torch():
    import torch as t
    return t


def dev(a, dtype=None):
    t = torch()
    x = t.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        x = x.view(dtype)
    return x.cuda()


def host(x):
    torch().cuda.synchronize()
    return x.cpu().numpy()


def hbits(x):
    return host(x.view(torch().int16)).view(np.uint16)


def f16(a):
    return np.asarray(a, np.float16).view(np.uint16)


def h(bits):
    return np.asarray(bits, np.uint16).view(np.float16).astype(np.float64)


def say(*args):
    print("[case]", *args, flush=True)


def close(actual, expected, rtol=RTOL, atol=ATOL):
    actual, expected = np.asarray(actual, np.float64), np.asarray(expected, np.float64)
    assert np.all(np.isfinite(actual))
    err = np.abs(actual - expected)
    bad = err > atol + rtol * np.abs(expected)
    assert not bad.any(), f"max abs err {err.max():.3g} at {np.argwhere(bad)[:3].tolist()}"
    return float(err.max())


# ---------------------------------------------------------------- GEMM
def gemm_case(ops, m, n, k, config, int8, seed=0):
    t = torch()
    rng = np.random.default_rng(seed + 1000 * m + n + 7 * k + config)
    a = f16(rng.standard_normal((m, k)) * 0.25)
    w = f16(rng.standard_normal((k, n)) * 0.25)
    bias = f16(rng.standard_normal(n) * 0.1)
    if int8:
        wv = w.copy()
        wv[:, 0] = 0  # zero channel: scale 1, q 0 (reference correctness.py:202)
        q, s = oracle.quantize(wv)
        ref32 = oracle.linear(a, q=q, scales=s, bias_bits=bias, out_dtype="f32")
        ref16 = oracle.linear(a, q=q, scales=s, bias_bits=bias)
        out32 = ops.gemm_int8(dev(a, t.float16), dev(q), dev(s), bias=dev(bias, t.float16), config=config,
                              output_dtype=t.float32)
        out16 = ops.gemm_int8(dev(a, t.float16), dev(q), dev(s), bias=dev(bias, t.float16), config=config)
    else:
        ref32 = oracle.linear(a, w_bits=w, bias_bits=bias, out_dtype="f32")
        ref16 = oracle.linear(a, w_bits=w, bias_bits=bias)
        out32 = ops.gemm(dev(a, t.float16), dev(w, t.float16), bias=dev(bias, t.float16), config=config,
                         output_dtype=t.float32)
        out16 = ops.gemm(dev(a, t.float16), dev(w, t.float16), bias=dev(bias, t.float16), config=config)
    close(host(out32), ref32)
    # fp32 output: only the summation order differs from the oracle
    close(host(out32), ref32, rtol=1e-4, atol=1e-4 * max(1.0, np.abs(ref32).max()))
    close(h(hbits(out16)), h(ref16))


@pytest.mark.parametrize("int8", [True, False])
@pytest.mark.parametrize("config", list(range(12)))
def test_gemm_reference_gate_shapes(ops, golden, config, int8):
    for m, n, k in golden["gemm_shapes"]["shapes"]:
        say("gemm", m, n, k, "config", config, "int8", int8)
        gemm_case(ops, m, n, k, config, int8)


@pytest.mark.parametrize("m,n,k", [(1, 768, 3072), (3, 100, 1000), (8, 3072, 768), (20, 2304, 768),
                                   (32, 768, 3072), (33, 70, 129), (64, 3072, 768), (100, 50, 40),
                                   (2, 50257, 768), (64, 768, 3072), (512, 768, 3072), (40, 130, 2000),
                                   (40, 1000, 776), (100, 1000, 1000), (700, 264, 1000), (1024, 768, 768)])
def test_gemm_split_k_and_tiled_paths(ops, m, n, k):
    say("gemm paths", m, n, k)
    gemm_case(ops, m, n, k, 0, True, seed=1)


@pytest.mark.parametrize("m,n,k", [(1, 768, 3072), (2, 3072, 768), (3, 1040, 1000), (5, 16, 17), (8, 2048, 4096),
                                   (8, 48, 40)])
@pytest.mark.parametrize("config", [0, 6])
def test_gemm_rowmajor_gemv_shapes(ops, m, n, k, config):
    """Row-major int8 W at M <= 8 through the reference ABI (fused config 0 and
    separate-workspace config 6): the row GEMV where rows and weight rows are
    4/8-element aligned (K not a multiple of 32: a ragged last step; N across
    several 64-column tiles with a part-filled last one; N = 48, one tile;
    K = 4096), the skinny split-K kernel where they are not (N = 16, K = 17)."""
    say("gemm row-major gemv", m, n, k, "config", config)
    gemm_case(ops, m, n, k, config, True, seed=3)


@pytest.mark.parametrize("m,n,k", [(16, 3072, 768), (17, 768, 3072), (64, 1000, 1000), (65, 3072, 768),
                                   (130, 768, 3072)])
@pytest.mark.parametrize("config", [0, 6])
def test_gemm_rowmajor_row_blocks(ops, m, n, k, config):
    """Row-major int8 W through the reference ABI across the row GEMV / GEMM
    boundaries: 16 rows (one block, the row GEMV), 17 (two 16-row blocks, the
    second one row), 64 with ragged N and K, 65 (three 32-row blocks, the last
    one row), 130; fused (config 0) and caller-workspace fp32 (config 6)."""
    say("gemm row-major row blocks", m, n, k, "config", config)
    gemm_case(ops, m, n, k, config, True, seed=5)


@pytest.mark.parametrize("config", [0, 6])
def test_gemm_tiled_split_k_fp16_weights(ops, config):
    """Row-major fp16 W over few tiles (M = 64, 3072 -> 768): K split over the
    library scratch, fused bias (config 0) or the fp32 workspace + bias pass (6)."""
    say("gemm tiled split fp16", config)
    gemm_case(ops, 64, 768, 3072, config, False, seed=2)


def test_gemm_repeat_calls_are_identical(ops):
    """The split-K arrival counters reset themselves: back-to-back launches agree."""
    t = torch()
    rng = np.random.default_rng(3)
    a = dev(f16(rng.standard_normal((4, 3072))), t.float16)
    q = dev(rng.integers(-127, 128, (3072, 768)).astype(np.int8))
    s = dev(rng.uniform(1e-3, 1e-2, 768).astype(np.float32))
    say("gemm repeat")
    outs = [hbits(ops.gemm_int8(a, q, s)) for _ in range(4)]
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])


def _fused(ops_lib, a, q, s, bias, y, res, m, n, k, epi):
    t = torch()
    fn = ops_lib.ti_amd_gemm_i8_fused
    fn.argtypes = [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    stream = t.cuda.current_stream()
    ptr = lambda x: None if x is None else x.data_ptr()
    st = fn(ptr(a), ptr(q), ptr(s), ptr(bias), ptr(y), ptr(res), m, n, k, epi, stream.cuda_stream, 0)
    assert st == 0, ops_lib.ti_v2_last_error()


@pytest.mark.parametrize("m", [1, 8, 64, 512, 1024])
@pytest.mark.parametrize("k,n", [(768, 3072), (3072, 768)])
def test_w8a16_sweep_fused_bias_gelu(ops, m, k, n):
    """A ~ N(0,1) fp16, q ~ U[-127,127], scales U[1e-3,1e-2] drawn
    as fp16 and widened to fp32, bias N(0,0.02), fused bias+GELU, fp16 output
    (and M = 1024, the row GEMM's largest M)."""
    t = torch()
    rng = np.random.default_rng(20261101 + m + n)
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("sweep gelu", m, k, n)
    y = t.empty((m, n), dtype=t.float16, device="cuda")
    _fused(ops.lib, dev(a, t.float16), dev(q), dev(s), dev(bias, t.float16), y, None, m, n, k, 1)
    ref = oracle.linear(a, q=q, scales=s, bias_bits=bias, gelu=True)
    close(h(hbits(y)), h(ref))
    # residual epilogue, in place (y = y + proj)
    res = dev(f16(rng.standard_normal((m, n))), t.float16)
    expect = h(hbits(res)) + h(oracle.linear(a, q=q, scales=s, bias_bits=bias))
    _fused(ops.lib, dev(a, t.float16), dev(q), dev(s), dev(bias, t.float16), res, res, m, n, k, 2)
    close(h(hbits(res)), expect.astype(np.float16).astype(np.float64))


def _pack_gpu(lib, q_dev, k, n):
    t = torch()
    lib.ti_amd_packed_w8_bytes.restype = C.c_int64
    lib.ti_amd_packed_w8_bytes.argtypes = [C.c_int, C.c_int]
    lib.ti_amd_pack_w8.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_size_t, C.c_int]
    size = lib.ti_amd_packed_w8_bytes(k, n)
    out = t.empty(size, dtype=t.uint8, device="cuda")
    st = lib.ti_amd_pack_w8(q_dev.data_ptr(), k, n, out.data_ptr(), t.cuda.current_stream().cuda_stream, 0)
    assert st == 0, lib.ti_v2_last_error()
    return out


def _packed(lib, a, packed, s, bias, y, res, m, n, k, epi):
    t = torch()
    fn = lib.ti_amd_gemm_w8p_fused
    fn.argtypes = [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    ptr = lambda x: None if x is None else x.data_ptr()
    st = fn(ptr(a), ptr(packed), ptr(s), ptr(bias), ptr(y), ptr(res), m, n, k, epi,
            t.cuda.current_stream().cuda_stream, 0)
    assert st == 0, lib.ti_v2_last_error()


@pytest.mark.parametrize("k,n", [(768, 3072), (3072, 768), (128, 100), (1600, 48)])
def test_pack_w8_layout_bit_exact(ops, k, n):
    """The device packer writes exactly the panel layout of the numpy restatement."""
    from tests.test_packed_layout import pack_w8_numpy
    rng = np.random.default_rng(k + n)
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    say("pack_w8", k, n)
    got = host(_pack_gpu(ops.lib, dev(q), k, n))
    assert np.array_equal(got.view(np.int8), pack_w8_numpy(q))


@pytest.mark.parametrize("m", [1, 8, 17, 32])
@pytest.mark.parametrize("k,n", [(768, 3072), (3072, 768), (768, 2304), (128, 100), (64, 50257), (768, 50257),
                                 (1024, 16400), (1600, 6400), (1600, 1600), (2048, 1000), (6400, 1600)])
def test_packed_gemv_against_oracle(ops, m, k, n):
    """Decode GEMV over panel-packed weights: bias, bias+GELU and in-place residual
    epilogues against the oracle's fp32-accumulate linear.  Through the C ABI,
    fewer than 128 column blocks over a long K (3072 -> 768 at M > 8, 6400 ->
    1600) split K and finish in the launch."""
    t = torch()
    rng = np.random.default_rng(7 * m + k + n)
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("packed gemv", m, k, n)
    packed = _pack_gpu(ops.lib, dev(q), k, n)
    ad, sd, bd = dev(a, t.float16), dev(s), dev(bias, t.float16)
    y = t.empty((m, n), dtype=t.float16, device="cuda")
    _packed(ops.lib, ad, packed, sd, bd, y, None, m, n, k, 0)
    ref = oracle.linear(a, q=q, scales=s, bias_bits=bias)
    close(h(hbits(y)), h(ref))
    _packed(ops.lib, ad, packed, sd, bd, y, None, m, n, k, 1)
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, bias_bits=bias, gelu=True)))
    res = dev(f16(rng.standard_normal((m, n))), t.float16)
    expect = (h(hbits(res)) + h(ref)).astype(np.float16).astype(np.float64)
    _packed(ops.lib, ad, packed, sd, bd, res, res, m, n, k, 2)
    close(h(hbits(res)), expect)


@pytest.mark.parametrize("k,n", [(768, 768), (1600, 1600), (6400, 1600), (192, 2040), (64, 8), (3072, 2048)])
def test_packed_gemv_single_row_parts(ops, k, n):
    """M = 1 over at most 2048 columns (the 8-column part-block kernel): odd and
    multi-round chunk counts (K = 1600 -> 25, 6400 -> 100), a ragged last block
    (2040, 8 columns), bias / no bias + GELU / in-place residual epilogues."""
    t = torch()
    rng = np.random.default_rng(5 * k + n)
    a = f16(rng.standard_normal((1, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("packed gemv single row", k, n)
    packed = _pack_gpu(ops.lib, dev(q), k, n)
    ad, sd, bd = dev(a, t.float16), dev(s), dev(bias, t.float16)
    y = t.empty((1, n), dtype=t.float16, device="cuda")
    _packed(ops.lib, ad, packed, sd, bd, y, None, 1, n, k, 0)
    ref = oracle.linear(a, q=q, scales=s, bias_bits=bias)
    close(h(hbits(y)), h(ref))
    _packed(ops.lib, ad, packed, sd, None, y, None, 1, n, k, 1)
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, gelu=True)))
    res = dev(f16(rng.standard_normal((1, n))), t.float16)
    expect = (h(hbits(res)) + h(ref)).astype(np.float16).astype(np.float64)
    _packed(ops.lib, ad, packed, sd, bd, res, res, 1, n, k, 2)
    close(h(hbits(res)), expect)


@pytest.mark.parametrize("m,k,n", [(1024, 768, 768), (512, 768, 3072)])
def test_panel_and_f16_record_gemm_agree_bitwise(ops, m, k, n):
    """Unsplit, the int8 panel GEMM and the fp16-record GEMM run the same MFMA
    sequence over the same weight values: their outputs are equal bit for bit
    (the runtime's batch-invariant prefill takes either, by shape)."""
    t = torch()
    rng = np.random.default_rng(m + k + n)
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("panel vs f16 records", m, k, n)
    ad, qd, sd, bd = dev(a, t.float16), dev(q), dev(s), dev(bias, t.float16)
    packed, packed16 = _pack_gpu(ops.lib, qd, k, n), _pack16_gpu(ops.lib, qd, sd, k, n)
    y8 = t.empty((m, n), dtype=t.float16, device="cuda")
    y16 = t.empty((m, n), dtype=t.float16, device="cuda")
    _packed(ops.lib, ad, packed, sd, bd, y8, None, m, n, k, 1)
    assert _w16(ops.lib, ad, packed16, bd, y16, None, m, n, k, 1) == 0
    assert np.array_equal(hbits(y8), hbits(y16))


@pytest.mark.parametrize("m,k,n", [(32, 1600, 8192), (24, 768, 50257), (32, 3072, 2048), (32, 6400, 1600), (20, 1600, 4800)])
def test_packed_gemv_column_block_groups(ops, m, k, n):
    """M in (16, 32] over a wide matrix: four column blocks share each A fragment,
    including a split longer than one round of loads (K = 1600 -> 25 chunks)."""
    t = torch()
    rng = np.random.default_rng(m + k + n)
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("packed gemv column groups", m, k, n)
    packed = _pack_gpu(ops.lib, dev(q), k, n)
    y = t.empty((m, n), dtype=t.float16, device="cuda")
    _packed(ops.lib, dev(a, t.float16), packed, dev(s), dev(bias, t.float16), y, None, m, n, k, 1)
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, bias_bits=bias, gelu=True)))


@pytest.mark.parametrize("m,k,n", [(33, 768, 3072), (64, 3072, 768), (130, 128, 100), (512, 64, 2000),
                                   (512, 768, 3072), (512, 3072, 768), (2048, 768, 2304), (4100, 1600, 6400),
                                   (2050, 64, 8200), (48, 1600, 6400), (64, 6400, 1600), (40, 64, 8200),
                                   (64, 768, 3072), (57, 768, 50257), (65, 768, 1000), (100, 3072, 768),
                                   (128, 768, 3072)])
def test_packed_prefill_gemm_against_oracle(ops, m, k, n):
    """Prefill (M > 32) GEMM over panel-packed weights: ragged row and column tiles,
    bias and bias+GELU epilogues against the oracle; fp32-accumulate tolerance.
    33..128 rows over at most 192 column blocks and K <= 3072 run the packed GEMV
    over row blocks of 16 up to 64 rows (the last one partly filled at M = 33,
    40, 57) and of 32 above (M = 65: a one-row last block; 100, 128); the
    in-place residual epilogue at M <= 128."""
    t = torch()
    rng = np.random.default_rng(11 * m + k + n)
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("packed prefill gemm", m, k, n)
    packed = _pack_gpu(ops.lib, dev(q), k, n)
    ad, sd, bd = dev(a, t.float16), dev(s), dev(bias, t.float16)
    y = t.empty((m, n), dtype=t.float16, device="cuda")
    _packed(ops.lib, ad, packed, sd, bd, y, None, m, n, k, 0)
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, bias_bits=bias)))
    _packed(ops.lib, ad, packed, sd, None, y, None, m, n, k, 1)
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, gelu=True)))
    if m <= 128:
        ref = oracle.linear(a, q=q, scales=s, bias_bits=bias)
        res = dev(f16(rng.standard_normal((m, n))), t.float16)
        expect = (h(hbits(res)) + h(ref)).astype(np.float16).astype(np.float64)
        _packed(ops.lib, ad, packed, sd, bd, res, res, m, n, k, 2)
        close(h(hbits(res)), expect)


def _pack16_gpu(lib, q_dev, s_dev, k, n):
    t = torch()
    lib.ti_amd_packed_w16_bytes.restype = C.c_int64
    lib.ti_amd_packed_w16_bytes.argtypes = [C.c_int, C.c_int]
    lib.ti_amd_pack_w16.argtypes = [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_size_t, C.c_int]
    out = t.empty(lib.ti_amd_packed_w16_bytes(k, n), dtype=t.uint8, device="cuda")
    st = lib.ti_amd_pack_w16(q_dev.data_ptr(), s_dev.data_ptr(), k, n, out.data_ptr(),
                             t.cuda.current_stream().cuda_stream, 0)
    assert st == 0, lib.ti_v2_last_error()
    return out


def _w16(lib, a, packed, bias, y, res, m, n, k, epi):
    t = torch()
    fn = lib.ti_amd_gemm_w16p_fused
    fn.argtypes = [C.c_void_p] * 5 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    ptr = lambda x: None if x is None else x.data_ptr()
    return fn(ptr(a), ptr(packed), ptr(bias), ptr(y), ptr(res), m, n, k, epi, t.cuda.current_stream().cuda_stream, 0)


@pytest.mark.parametrize("k,n", [(768, 3072), (200, 40), (1600, 48)])
def test_pack_w16_layout_bit_exact(ops, k, n):
    """The device dequantise-and-pack writes exactly the numpy restatement (the
    int8 kernels' fp16_rn(float(q) * scale) values in MFMA B order)."""
    from tests.test_packed_layout import pack_w16_numpy
    rng = np.random.default_rng(k + 3 * n)
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    say("pack_w16", k, n)
    got = host(_pack16_gpu(ops.lib, dev(q), dev(s), k, n)).view(np.uint16)
    assert np.array_equal(got, pack_w16_numpy(q, s).view(np.uint16))


@pytest.mark.parametrize("m,k,n", [(33, 768, 3072), (64, 3072, 768), (130, 128, 100), (512, 64, 2000),
                                   (512, 768, 3072), (1024, 768, 2304), (2048, 3072, 768), (4100, 1600, 6400),
                                   (70, 224, 40), (2100, 1632, 1700), (3000, 800, 4000), (3000, 4096, 4000),
                                   (8200, 256, 4000)])
def test_f16_packed_prefill_gemm_against_oracle(ops, m, k, n):
    """Prefill GEMM over the pre-dequantised fp16 weights: ragged row and column
    tiles, K a multiple of 32 but not of 64, the 256 x 256 tiles (K >= 4096,
    192 of them) and the 256 x 128 tiles (1056 of them), bias / bias+GELU /
    in-place residual epilogues against the oracle's int8 linear (the same
    weight values)."""
    t = torch()
    rng = np.random.default_rng(13 * m + k + n)
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("f16-packed prefill gemm", m, k, n)
    packed = _pack16_gpu(ops.lib, dev(q), dev(s), k, n)
    ad, bd = dev(a, t.float16), dev(bias, t.float16)
    y = t.empty((m, n), dtype=t.float16, device="cuda")
    assert _w16(ops.lib, ad, packed, bd, y, None, m, n, k, 0) == 0, ops.lib.ti_v2_last_error()
    ref = oracle.linear(a, q=q, scales=s, bias_bits=bias)
    close(h(hbits(y)), h(ref))
    assert _w16(ops.lib, ad, packed, None, y, None, m, n, k, 1) == 0
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, gelu=True)))
    res = dev(f16(rng.standard_normal((m, n))), t.float16)
    expect = (h(hbits(res)) + h(ref)).astype(np.float16).astype(np.float64)
    assert _w16(ops.lib, ad, packed, bd, res, res, m, n, k, 2) == 0
    close(h(hbits(res)), expect)


@pytest.mark.parametrize("layout", ["row_major", "panel", "f16"])
@pytest.mark.parametrize("n,off", [(1000, 0), (1000, 1), (998, 0)])
def test_gemm_tile_epilogue_ragged_and_unaligned(ops, layout, n, off):
    """The M > 32 GEMMs finish from an LDS tile, 4 columns per thread, with one
    8-byte store per group when the output allows it.  N = 1000 at offset 0
    takes the vector stores (a part-filled last tile); the same output one
    element into its buffer (2-byte aligned) and N = 998 (rows not a multiple
    of 4 elements, a 2-column group at the edge) take the per-element path.
    Bias, bias+GELU and in-place residual epilogues of the row-major,
    int8-panel and fp16-record kernels against the oracle, and nothing
    written outside the output."""
    t = torch()
    m, k = 65, 128
    rng = np.random.default_rng(n + 7 * off + len(layout))
    a = f16(rng.standard_normal((m, k)))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("gemm tile epilogue", layout, n, "offset", off)
    ad, sd, bd = dev(a, t.float16), dev(s), dev(bias, t.float16)
    if layout == "panel":
        w = _pack_gpu(ops.lib, dev(q), k, n)
        run = lambda b_, y_, r_, epi: _packed(ops.lib, ad, w, sd, b_, y_, r_, m, n, k, epi)
    elif layout == "f16":
        w = _pack16_gpu(ops.lib, dev(q), sd, k, n)
        run = lambda b_, y_, r_, epi: _w16(ops.lib, ad, w, b_, y_, r_, m, n, k, epi) == 0 or pytest.fail(
            ops.lib.ti_v2_last_error())
    else:
        qd = dev(q)
        run = lambda b_, y_, r_, epi: _fused(ops.lib, ad, qd, sd, b_, y_, r_, m, n, k, epi)
    buf = t.zeros(m * n + 8, dtype=t.float16, device="cuda")
    y = buf[off:off + m * n].view(m, n)
    ref = oracle.linear(a, q=q, scales=s, bias_bits=bias)
    run(bd, y, None, 0)
    close(h(hbits(y)), h(ref))
    run(None, y, None, 1)
    close(h(hbits(y)), h(oracle.linear(a, q=q, scales=s, gelu=True)))
    r0 = f16(rng.standard_normal((m, n)))
    y.copy_(dev(r0, t.float16))
    run(bd, y, y, 2)
    close(h(hbits(y)), (h(r0) + h(ref)).astype(np.float16).astype(np.float64))
    # Nothing outside the output was written.
    rest = hbits(buf).astype(np.int64)
    assert not rest[:off].any() and not rest[off + m * n:].any()


def test_f16_packed_gemm_rejects_unsupported_shapes(ops):
    t = torch()
    a = t.zeros((64, 96), dtype=t.float16, device="cuda")
    packed = t.zeros(1 << 16, dtype=t.uint8, device="cuda")
    y = t.empty((64, 16), dtype=t.float16, device="cuda")
    say("f16-packed gemm invalid")
    assert _w16(ops.lib, a, packed, None, y, None, 64, 16, 80, 0) == 1   # K % 32 != 0
    assert _w16(ops.lib, a, packed, None, y, None, 32, 16, 96, 0) == 1   # M <= 32: the decode GEMV's shapes
    assert _w16(ops.lib, a, packed, None, y, None, 64, 16, 96, 3) == 1   # unknown epilogue


def test_packed_gemv_rejects_unsupported_shapes(ops):
    t = torch()
    a = t.zeros((33, 64), dtype=t.float16, device="cuda")
    q = t.zeros((64, 16), dtype=t.int8, device="cuda")
    packed = _pack_gpu(ops.lib, q, 64, 16)
    s = t.ones(16, dtype=t.float32, device="cuda")
    y = t.empty((33, 16), dtype=t.float16, device="cuda")
    fn = ops.lib.ti_amd_gemm_w8p_fused
    fn.argtypes = [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    say("packed gemv invalid")
    assert fn(a.data_ptr(), packed.data_ptr(), s.data_ptr(), None, y.data_ptr(), None, 1, 16, 63, 0, 0, 0) == 1
    assert fn(a.data_ptr() + 2, packed.data_ptr(), s.data_ptr(), None, y.data_ptr(), None, 1, 16, 64, 0, 0, 0) == 1
    assert fn(a.data_ptr(), packed.data_ptr(), s.data_ptr(), None, y.data_ptr(), None, 0, 16, 64, 0, 0, 0) == 1


def _ln_packed(lib, a, g, b, eps, packed, s, bias, y, res, m, n, k, epi):
    t = torch()
    fn = lib.ti_amd_gemm_w8p_ln_fused
    fn.argtypes = [C.c_void_p] * 3 + [C.c_float] + [C.c_void_p] * 5 + [C.c_int] * 4 + [C.c_size_t, C.c_int]
    ptr = lambda x: None if x is None else x.data_ptr()
    return fn(ptr(a), ptr(g), ptr(b), eps, ptr(packed), ptr(s), ptr(bias), ptr(y), ptr(res), m, n, k, epi,
              t.cuda.current_stream().cuda_stream, 0)


@pytest.mark.parametrize("m", [1, 7, 32])
@pytest.mark.parametrize("k,n", [(768, 2304), (768, 3072), (768, 50257), (1600, 6400), (64, 100), (2048, 64)])
def test_layernorm_prologue_gemv_against_oracle(ops, m, k, n):
    """Decode GEMV with the LayerNorm of its A rows computed in the prologue:
    epilogue(LN(A) @ W + bias) against the oracle's layernorm_f16 followed by its
    linear.  Rows carry offsets up to 50 (the two-pass variance matters) and
    the head shape at M = 32 takes the four-column-block variant."""
    t = torch()
    rng = np.random.default_rng(3 * m + k + n)
    a = f16(rng.standard_normal((m, k)) * rng.uniform(0.5, 4, (m, 1)) + rng.uniform(-50, 50, (m, 1)))
    gam = f16(1 + 0.2 * rng.standard_normal(k))
    bet = f16(0.1 * rng.standard_normal(k))
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    s = rng.uniform(1e-3, 1e-2, n).astype(np.float16).astype(np.float32)
    bias = f16(rng.standard_normal(n) * 0.02)
    say("layernorm-prologue gemv", m, k, n)
    packed = _pack_gpu(ops.lib, dev(q), k, n)
    ad, gd, bd = dev(a, t.float16), dev(gam, t.float16), dev(bet, t.float16)
    sd, biasd = dev(s), dev(bias, t.float16)
    normed = oracle.layernorm_f16(a, gam, bet, 1e-5)
    y = t.empty((m, n), dtype=t.float16, device="cuda")
    assert _ln_packed(ops.lib, ad, gd, bd, 1e-5, packed, sd, biasd, y, None, m, n, k, 0) == 0, \
        ops.lib.ti_v2_last_error()
    ref = oracle.linear(normed, q=q, scales=s, bias_bits=bias)
    close(h(hbits(y)), h(ref))
    assert _ln_packed(ops.lib, ad, gd, bd, 1e-5, packed, sd, biasd, y, None, m, n, k, 1) == 0
    close(h(hbits(y)), h(oracle.linear(normed, q=q, scales=s, bias_bits=bias, gelu=True)))
    res = dev(f16(rng.standard_normal((m, n))), t.float16)
    expect = (h(hbits(res)) + h(ref)).astype(np.float16).astype(np.float64)
    assert _ln_packed(ops.lib, ad, gd, bd, 1e-5, packed, sd, biasd, res, res, m, n, k, 2) == 0
    close(h(hbits(res)), expect)


def test_layernorm_prologue_gemv_rejects_unsupported_shapes(ops):
    t = torch()
    a = t.zeros((33, 2112), dtype=t.float16, device="cuda")
    g = t.ones(2112, dtype=t.float16, device="cuda")
    q = t.zeros((2112, 16), dtype=t.int8, device="cuda")
    packed = _pack_gpu(ops.lib, q, 2112, 16)
    s = t.ones(16, dtype=t.float32, device="cuda")
    y = t.empty((33, 16), dtype=t.float16, device="cuda")
    say("layernorm-prologue gemv invalid")
    args = lambda m, k, eps=1e-5: (ops.lib, a, g, g, eps, packed, s, None, y, None, m, 16, k, 0)
    assert _ln_packed(*args(33, 64)) == 1        # M > 32
    assert _ln_packed(*args(1, 2112)) == 1       # K / 64 > 32
    assert _ln_packed(*args(1, 100)) == 1        # K % 64 != 0
    assert _ln_packed(*args(1, 64, eps=0.0)) == 1
    assert _ln_packed(*args(0, 64)) == 1


def test_legacy_fp32_gemm(ops):
    t = torch()
    rng = np.random.default_rng(4)
    for m, n, k in ((1, 1, 1), (7, 13, 5), (65, 257, 300), (128, 96, 513)):
        say("legacy gemm", m, n, k)
        a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
        b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
        out = host(ops.legacy_gemm(dev(a), dev(b)))
        assert np.allclose(out, a.astype(np.float64) @ b, atol=1e-5 * k + 1e-5)


# ---------------------------------------------------------------- attention
@pytest.mark.parametrize("config", [0, 1])
@pytest.mark.parametrize("d", [64, 128])
def test_attention_reference_cases(ops, golden, d, config):
    t = torch()
    rng = np.random.default_rng(d + config)
    for nq, nk, ql, kl, off, causal in golden["attention_cases"]["cases"]:
        say("attention", d, config, nq, nk, ql, kl, off, causal)
        q = f16(rng.standard_normal((2, 2, nq, d)) * 0.5)
        k = f16(rng.standard_normal((2, 2, nk, d)) * 0.5)
        v = f16(rng.standard_normal((2, 2, nk, d)))
        out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                            kv_lengths=kl, query_offsets=off, causal=causal, config=config)
        got = h(hbits(out))
        ref = oracle.attention_f16(q, k, v, ql, kl, off, causal)
        close(got, h(ref))
        zero_rows = h(ref) == 0
        rows_zero = np.all(zero_rows, axis=-1)
        assert np.all(got[rows_zero] == 0), "all-masked output must be exactly zero"


def test_decode_attention_config3(ops):
    """B=32, H=12, D=64, one query per request, ragged
    context lengths U[128,1024], Q/K/V ~ N(0,1)/8, FP32 softmax."""
    t = torch()
    rng = np.random.default_rng(20261101)
    B, H, D = 32, 12, 64
    L = rng.integers(128, 1025, B)
    K = int(L.max())
    q = f16(rng.standard_normal((B, H, 1, D)) / 8)
    k = f16(rng.standard_normal((B, H, K, D)) / 8)
    v = f16(rng.standard_normal((B, H, K, D)) / 8)
    say("decode attention", B, H, D, K)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=[1] * B,
                        kv_lengths=L.tolist(), query_offsets=(L - 1).tolist(), causal=True)
    got = h(hbits(out))
    ref = h(oracle.attention_f16(q, k, v, [1] * B, L, L - 1, True))
    close(got, ref)
    # At this distribution the outputs are means of ~L values of sd 1/8 (sd about
    # 4e-3 .. 1.1e-2), so the linear tolerance alone is wider than the signal.
    # Bound the error at the signal's scale: 1e-4 is ~13 fp16 ulps at 0.01.
    SIGNAL_ATOL = 1e-4
    assert np.abs(got - ref).max() <= SIGNAL_ATOL, np.abs(got - ref).max()
    # The bound has teeth: an oracle without the 1/sqrt(D) score scale (q * 8 is
    # exact in fp16, so it reproduces scores q.k unscaled) and an oracle that
    # drops each request's newest key both land outside it.
    unscaled = h(oracle.attention_f16(f16(h(q) * 8), k, v, [1] * B, L, L - 1, True))
    short = h(oracle.attention_f16(q, k, v, [1] * B, L - 1, L - 2, True))
    assert np.abs(got - unscaled).max() > 5 * SIGNAL_ATOL
    assert np.abs(got - short).max() > 2 * SIGNAL_ATOL


def poison_past_lengths(k, v, kv_lengths):
    """fp16 NaN in every K and V entry at or past a request's length: keys a
    request does not see must not reach its output, whatever the cache holds
    there (the oracle never reads them)."""
    for b, n in enumerate(kv_lengths):
        k[b, :, int(n):] = 0x7E00
        v[b, :, int(n):] = 0x7E00


@pytest.mark.parametrize("d,nk", [(64, 1024), (64, 1500), (128, 512), (128, 1100)])
@pytest.mark.parametrize("causal", [0, 1])
def test_split_decode_attention_ragged(ops, d, nk, causal):
    """Single-query attention over a long cache runs split over key chunks plus a
    merge pass: ragged lengths including 0 and 1 visible keys, a request with no
    query (its output row is zero), offsets that hide the tail when causal."""
    t = torch()
    rng = np.random.default_rng(d + nk + causal)
    B, H = 6, 3
    kl = [nk, 1, 0, nk - 37, 255, min(513, nk)]
    ql = [1, 1, 1, 1, 0, 1]
    off = [nk - 1, 0, 0, nk // 3, 0, 200]
    q = f16(rng.standard_normal((B, H, 1, d)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, d)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, d)))
    poison_past_lengths(k, v, kl)
    say("split decode attention", d, nk, causal)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                        kv_lengths=kl, query_offsets=off, causal=bool(causal))
    got = h(hbits(out))
    close(got, h(oracle.attention_f16(q, k, v, ql, kl, off, bool(causal))))
    assert not got[2].any() and not got[4].any()


def test_split_decode_attention_large_batch(ops):
    """The key-split kernel plus its merge pass over a large batch (260
    requests, 520 (b, h) rows): ragged lengths, ties, empty rows and a request
    with no query, against the oracle."""
    t = torch()
    rng = np.random.default_rng(260)
    B, H, D, nk = 260, 2, 64, 600
    kl = rng.integers(0, nk + 1, B)
    kl[:8] = [nk, nk, 1, 0, 517, 517, 512, 128]
    ql = np.ones(B, np.int64)
    ql[9] = 0
    off = np.maximum(kl - 1, 0)
    q = f16(rng.standard_normal((B, H, 1, D)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, D)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, D)))
    say("split decode attention, batch", B)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql.tolist(),
                        kv_lengths=kl.tolist(), query_offsets=off.tolist(), causal=True)
    got = h(hbits(out))
    close(got, h(oracle.attention_f16(q, k, v, ql, kl, off, True)))
    assert not got[3].any() and not got[9].any()


@pytest.mark.parametrize("d,nk", [(64, 384), (64, 4200), (128, 2100)])
def test_decode_attention_outside_split_range(ops, d, nk):
    """Single-query attention whose cache is too short (fewer than 4 chunks of
    128 / 64 keys) or too long (more than 32 chunks) for the key split: one
    workgroup per (b, h) whose waves split the keys and merge in LDS, with
    ragged lengths, a row of 0 keys and a causal offset that hides the tail."""
    t = torch()
    rng = np.random.default_rng(7 * d + nk)
    B, H = 4, 2
    kl = [nk, 0, nk - 45, 1]
    ql = [1, 1, 1, 1]
    off = [nk // 2, 0, nk - 46, 0]
    q = f16(rng.standard_normal((B, H, 1, d)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, d)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, d)))
    poison_past_lengths(k, v, kl)
    say("decode attention outside the split range", d, nk)
    for causal in (False, True):
        out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                            kv_lengths=kl, query_offsets=off, causal=causal)
        got = h(hbits(out))
        close(got, h(oracle.attention_f16(q, k, v, ql, kl, off, causal)))
        assert not got[1].any()


@pytest.mark.parametrize("nq,nk", [(64, 64), (300, 300), (1, 2000), (3, 700)])
def test_attention_prefill_and_long(ops, nq, nk):
    t = torch()
    rng = np.random.default_rng(nq + nk)
    B, H, D = 2, 3, 64
    ql = [nq, max(1, nq // 2)]
    kl = [nk, max(1, nk - 5)]
    off = [nk - nq, max(0, kl[1] - ql[1])]
    q = f16(rng.standard_normal((B, H, nq, D)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, D)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, D)))
    say("attention prefill", nq, nk)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                        kv_lengths=kl, query_offsets=off, causal=True)
    close(h(hbits(out)), h(oracle.attention_f16(q, k, v, ql, kl, off, True)))


@pytest.mark.parametrize("causal", [0, 1])
def test_attention_prefill_many_tiles(ops, causal):
    """More than 512 query tiles (8 x 12 x 6 = 576 workgroups) take the 4-wave
    prefill kernel, fewer the 8-wave key-split one (covered above); ragged
    per-request lengths, offsets and a request with no query."""
    t = torch()
    rng = np.random.default_rng(21 + causal)
    B, H, D, nq, nk = 8, 12, 64, 384, 420
    ql = [384, 300, 1, 0, 129, 384, 64, 250]
    kl = [420, 310, 5, 17, 129, 384, 400, 251]
    off = [max(0, kv - qv) for qv, kv in zip(ql, kl)]
    q = f16(rng.standard_normal((B, H, nq, D)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, D)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, D)))
    say("attention prefill many tiles", causal)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                        kv_lengths=kl, query_offsets=off, causal=bool(causal))
    close(h(hbits(out)), h(oracle.attention_f16(q, k, v, ql, kl, off, bool(causal))))


@pytest.mark.parametrize("causal", [0, 1])
def test_attention_prefill_four_key_groups(ops, causal):
    """At most 256 workgroups of 64 queries (2 x 4 x 17): the 16-wave kernel with
    four key groups, each taking every fourth key tile, merged at the end;
    ragged lengths and offsets, and queries past a request's length zero."""
    t = torch()
    rng = np.random.default_rng(41 + causal)
    B, H, D, nq, nk = 2, 4, 64, 1088, 1200
    ql = [1088, 701]
    kl = [1200, 760]
    off = [kv - qv for qv, kv in zip(ql, kl)]
    q = f16(rng.standard_normal((B, H, nq, D)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, D)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, D)))
    say("attention prefill four key groups", causal)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                        kv_lengths=kl, query_offsets=off, causal=bool(causal))
    got = h(hbits(out))
    close(got, h(oracle.attention_f16(q, k, v, ql, kl, off, bool(causal))))
    assert not got[1, :, 701:].any()


@pytest.mark.parametrize("causal", [0, 1])
def test_attention_prefill_two_query_blocks(ops, causal):
    """At least 768 workgroups of 128 queries (4 x 12 x 16): the 4-wave kernel
    with two 16-query blocks per wave.  Ragged lengths put a block boundary
    inside a wave (a request of 17 queries, one of 130), a request with no
    query, and queries past a request's length that must come out zero."""
    t = torch()
    rng = np.random.default_rng(31 + causal)
    B, H, D, nq, nk = 16, 12, 64, 512, 530
    ql = [512, 17, 130, 0, 511, 128, 1, 300, 512, 64, 96, 200, 255, 257, 33, 480]
    kl = [530, 17, 140, 9, 520, 128, 1, 310, 512, 100, 96, 210, 255, 300, 40, 500]
    off = [max(0, kv - qv) for qv, kv in zip(ql, kl)]
    q = f16(rng.standard_normal((B, H, nq, D)) * 0.5)
    k = f16(rng.standard_normal((B, H, nk, D)) * 0.5)
    v = f16(rng.standard_normal((B, H, nk, D)))
    say("attention prefill two query blocks", causal)
    out = ops.attention(dev(q, t.float16), dev(k, t.float16), dev(v, t.float16), q_lengths=ql,
                        kv_lengths=kl, query_offsets=off, causal=bool(causal))
    got = h(hbits(out))
    close(got, h(oracle.attention_f16(q, k, v, ql, kl, off, bool(causal))))
    assert not got[3].any() and not got[1, :, 17:].any()


# ---------------------------------------------------------------- row ops fp16
@pytest.mark.parametrize("cols", [1, 7, 257, 768, 3072, 5000])
def test_layernorm_gelu_softmax_f16(ops, cols):
    t = torch()
    rng = np.random.default_rng(cols)
    x = f16(rng.standard_normal((3, cols)))
    g, b = f16(rng.standard_normal(cols)), f16(rng.standard_normal(cols))
    say("fp16 rowops", cols)
    xd = dev(x, t.float16)
    close(h(hbits(ops.layernorm(xd, dev(g, t.float16), dev(b, t.float16)))), h(oracle.layernorm_f16(x, g, b)))
    close(h(hbits(ops.gelu_new(xd))), h(oracle.gelu_f16(x)))
    close(h(hbits(ops.softmax(xd))), h(oracle.softmax_f16(x)))


def test_rowops_f16_tight_against_oracle(ops):
    """GPT-2 shapes: LN over 768 and GELU over 3072 land within one fp16 ulp."""
    t = torch()
    rng = np.random.default_rng(5)
    x = f16(rng.standard_normal((64, 768)))
    g, b = f16(1 + 0.02 * rng.standard_normal(768)), f16(0.02 * rng.standard_normal(768))
    say("fp16 LN tight")
    got = hbits(ops.layernorm(dev(x, t.float16), dev(g, t.float16), dev(b, t.float16)))
    ref = oracle.layernorm_f16(x, g, b)
    ulp = np.abs(got.astype(np.int32) - ref.astype(np.int32))
    assert ulp.max() <= 1
    y = f16(rng.standard_normal((16, 3072)) * 2)
    got = hbits(ops.gelu_new(dev(y, t.float16)))
    want = oracle.gelu_f16(y)
    zero = (got & 0x7FFF == 0) & (want & 0x7FFF == 0)  # +0 and -0 are the same value
    assert np.abs(got.astype(np.int32) - want.astype(np.int32))[~zero].max() <= 1


def test_gelu_f16_every_input_against_oracle(ops):
    """All 65 536 fp16 patterns through ti_v2_gelu_new_f16 (the same gelu_tanh the
    GEMM epilogues use) against the oracle's std::tanh form: NaN stays NaN, the
    infinities and +-0 match, and finite inputs differ by at most one fp16 ulp
    in at most 16 values (5 measured on MI355X)."""
    t = torch()
    x = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    say("gelu every fp16")
    got = hbits(ops.gelu_new(dev(x, t.float16)))
    want = oracle.gelu_f16(x)
    gf, wf = got.view(np.float16).astype(np.float32), want.view(np.float16).astype(np.float32)
    assert np.array_equal(np.isnan(gf), np.isnan(wf))
    ok = np.isnan(wf) | (gf == wf)  # +0 == -0
    d = np.abs(got.astype(np.int32) - want.astype(np.int32))
    assert d[~ok].max(initial=0) <= 1 and int((~ok).sum()) <= 16, int((~ok).sum())


# ---------------------------------------------------------------- row ops fp32 (legacy ABI)
def _legacy():
    from tinyinfer_amd import BACKEND_LIB
    lib = C.CDLL(str(BACKEND_LIB))
    p, i = C.c_void_p, C.c_int
    lib.ti_cuda_softmax.argtypes = [p, p, i, i]
    lib.ti_cuda_layernorm.argtypes = [p, p, p, p, i, i, C.c_float]
    lib.ti_cuda_gemm.argtypes = [p, p, p, i, i, i]
    return lib


@pytest.mark.parametrize("rows,cols", [(4096, 768), (7, 4099), (3, 1), (33, 1000)])
def test_fp32_layernorm_config2(rows, cols):
    """LayerNorm [4096,768], eps 1e-5, gamma N(1,0.1), beta N(0,0.1),
    x N(0,1); 1e-4 relative against the float64 reference."""
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    dx, dg, db = dev(x), dev(g), dev(b)
    y = torch().empty_like(dx)
    say("fp32 layernorm", rows, cols)
    _legacy().ti_cuda_layernorm(dx.data_ptr(), dg.data_ptr(), db.data_ptr(), y.data_ptr(), rows, cols, 1e-5)
    ref = oracle.layernorm_f32_exact(x, g, b)
    close(host(y), ref, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("rows,cols", [(4096, 1024), (17, 4097), (5, 31)])
def test_fp32_softmax_config2(rows, cols):
    rng = np.random.default_rng(rows * cols)
    x = (3 * rng.standard_normal((rows, cols))).astype(np.float32)
    x[0, ::5] = -np.inf
    dx = dev(x)
    y = torch().empty_like(dx)
    say("fp32 softmax", rows, cols)
    _legacy().ti_cuda_softmax(dx.data_ptr(), y.data_ptr(), rows, cols)
    out = host(y)
    ref = oracle.softmax_f32_exact(x)
    close(out, ref, rtol=1e-4, atol=1e-8)
    assert np.all(out[0, ::5] == 0)


def test_fp32_layernorm_then_softmax_config2():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((4096, 768)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(768)).astype(np.float32)
    b = (0.1 * rng.standard_normal(768)).astype(np.float32)
    dx, dg, db = dev(x), dev(g), dev(b)
    mid = torch().empty_like(dx)
    y = torch().empty_like(dx)
    lib = _legacy()
    say("fp32 LN->softmax")
    lib.ti_cuda_layernorm(dx.data_ptr(), dg.data_ptr(), db.data_ptr(), mid.data_ptr(), 4096, 768, 1e-5)
    lib.ti_cuda_softmax(mid.data_ptr(), y.data_ptr(), 4096, 768)
    ref = oracle.softmax_f32_exact(oracle.layernorm_f32_exact(x, g, b))
    close(host(y), ref, rtol=1e-4, atol=1e-8)


@pytest.mark.parametrize("rows,cols", [(4096, 768), (9, 4096), (5, 100), (3, 2048), (6, 4098), (2, 1)])
def test_fp32_fused_layernorm_softmax(rows, cols):
    """ti_amd_layernorm_softmax_f32 (one pass per row) returns exactly what the two
    calls ti_cuda_layernorm then ti_cuda_softmax return (same values, maxima and
    sums in the same lane order; widths past 4096 or not a multiple of 4 take those
    two kernels), and 1e-4 relative of the float64 reference."""
    rng = np.random.default_rng(rows + 3 * cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    g = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    b = (0.1 * rng.standard_normal(cols)).astype(np.float32)
    dx, dg, db = dev(x), dev(g), dev(b)
    mid, y2, y = (torch().empty_like(dx) for _ in range(3))
    lib = _legacy()
    say("fp32 fused LN->softmax", rows, cols)
    lib.ti_cuda_layernorm(dx.data_ptr(), dg.data_ptr(), db.data_ptr(), mid.data_ptr(), rows, cols, 1e-5)
    lib.ti_cuda_softmax(mid.data_ptr(), y2.data_ptr(), rows, cols)
    fn = lib.ti_amd_layernorm_softmax_f32
    fn.argtypes = [C.c_void_p] * 4 + [C.c_int, C.c_int, C.c_float, C.c_size_t, C.c_int]
    st = fn(dx.data_ptr(), dg.data_ptr(), db.data_ptr(), y.data_ptr(), rows, cols, 1e-5,
            torch().cuda.current_stream().cuda_stream, 0)
    assert st == 0
    got = host(y)
    assert np.array_equal(got.view(np.uint32), host(y2).view(np.uint32))
    close(got, oracle.softmax_f32_exact(oracle.layernorm_f32_exact(x, g, b)), rtol=1e-4, atol=1e-8)
    # an output that overlaps the input is rejected before anything is queued
    assert fn(dx.data_ptr(), dg.data_ptr(), db.data_ptr(), dx.data_ptr(), rows, cols, 1e-5,
              torch().cuda.current_stream().cuda_stream, 0) == 1


def test_ti_cuda_gemm_legacy_order():
    rng = np.random.default_rng(12)
    m, k, n = 37, 70, 45
    a = rng.uniform(-1, 1, (m, k)).astype(np.float32)
    b = rng.uniform(-1, 1, (k, n)).astype(np.float32)
    da, db = dev(a), dev(b)
    y = torch().empty((m, n), dtype=torch().float32, device="cuda")
    say("ti_cuda_gemm")
    _legacy().ti_cuda_gemm(da.data_ptr(), db.data_ptr(), y.data_ptr(), m, k, n)
    assert np.allclose(host(y), a.astype(np.float64) @ b, atol=1e-5 * k + 1e-5)


# ---------------------------------------------------------------- contracts
def test_invalid_contracts(ops):
    """Wrapper-level rejections of reference correctness.py:286-302 and the native
    status codes of reference tinyinfer_host_validation.hpp."""
    t = torch()
    a = t.ones((2, 3), device="cuda", dtype=t.float16)
    b = t.ones((3, 4), device="cuda", dtype=t.float16)
    for fn in (lambda: ops.gemm(a.cpu(), b), lambda: ops.gemm(a.float(), b), lambda: ops.gemm(a.t(), b),
               lambda: ops.gemm(a, b, config=True), lambda: ops.gemm(a, b, config=12),
               lambda: ops.gemm(a, b, bias=t.zeros(3, device=a.device, dtype=a.dtype)),
               lambda: ops.gemm(a.clone().requires_grad_(), b)):
        with pytest.raises((ValueError, TypeError)):
            fn()
    q = t.ones((1, 1, 1, 64), device="cuda", dtype=t.float16)
    for fn in (lambda: ops.attention(q, q, q, q_lengths=[2]), lambda: ops.attention(q, q, q, query_offsets=[-1]),
               lambda: ops.attention(q, q, q, kv_lengths=[True]), lambda: ops.attention(q, q, q, causal=1)):
        with pytest.raises((ValueError, TypeError)):
            fn()
    lib = ops.lib
    s = t.cuda.current_stream().cuda_stream
    y = t.empty((2, 4), device="cuda", dtype=t.float16)
    assert lib.ti_v2_gemm_ex_f16(a.data_ptr(), b.data_ptr(), None, y.data_ptr(), None, 2, 4, 3, 0, 12, s, 0) == 3
    assert lib.ti_v2_gemm_ex_f16(a.data_ptr(), b.data_ptr(), None, y.data_ptr(), None, 2, 4, 3, 0, 6, s, 0) == 1
    assert lib.ti_v2_gemm_ex_f16(a.data_ptr() + 1, b.data_ptr(), None, y.data_ptr(), None, 2, 4, 3, 0, 0, s, 0) == 1
    assert lib.ti_v2_gemm_ex_f16(a.data_ptr(), b.data_ptr(), None, y.data_ptr(), None, 2, 4, 3, 2, 0, s, 0) == 1
    assert lib.ti_v2_gemm_ex_f16(a.data_ptr(), b.data_ptr(), None, y.data_ptr(), None, 2, 4, 3, 0, 0, s, -1) == 1
    assert lib.ti_v2_gemm_ex_f16(a.data_ptr(), b.data_ptr(), None, y.data_ptr(), None, 2, 4, 3, 0, 0, s, 7) == 2
    assert b"device" in lib.ti_v2_last_error()
    assert lib.ti_v2_layernorm_f16(a.data_ptr(), a.data_ptr(), a.data_ptr(), y.data_ptr(), 2, 3,
                                   C.c_float(0.0), s, 0) == 1
    assert lib.ti_v2_gelu_new_f16(a.data_ptr(), y.data_ptr(), 0, s, 0) == 1
    m = t.zeros(1, dtype=t.int32, device="cuda")
    assert lib.ti_v2_attention_f16(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), m.data_ptr(),
                                   m.data_ptr(), m.data_ptr(), 1, 1, 1, 1, 64, 1, 2, s, 0) == 3
    assert lib.ti_v2_attention_f16(q.data_ptr(), q.data_ptr(), q.data_ptr(), q.data_ptr(), m.data_ptr(),
                                   m.data_ptr(), m.data_ptr(), 1, 1, 1, 1, 96, 1, 0, s, 0) == 1
    assert lib.ti_v2_last_error() == b"invalid attention arguments"
    t.cuda.synchronize()


def test_non_default_stream_and_input_lifetime(ops):
    """reference correctness.py:263-284: inputs allocated on the default stream,
    consumed on a side stream behind queued work, then freed; record_stream keeps
    their storage from being reused before the kernel ran."""
    t = torch()
    default = t.cuda.current_stream()
    stream = t.cuda.Stream()
    rng = np.random.default_rng(13)
    an = f16(rng.standard_normal((33, 19)))
    bn = f16(rng.standard_normal((19, 67)))
    a, b = dev(an, t.float16), dev(bn, t.float16)
    expected = h(an) @ h(bn)
    stream.wait_stream(default)
    say("stream lifetime")
    with t.cuda.stream(stream):
        blocker = t.ones((256, 256), device="cuda", dtype=t.float32) * 0.001
        for _ in range(8):
            blocker = blocker @ blocker
        actual = ops.gemm(a, b, config=0, output_dtype=t.float32)
    del a, b
    gc.collect()
    for _ in range(32):
        tmp = t.empty((33, 19), device="cuda", dtype=t.float16)
        tmp.fill_(123)
        tmp2 = t.empty((19, 67), device="cuda", dtype=t.float16)
        tmp2.fill_(124)
    del tmp, tmp2, blocker
    default.wait_stream(stream)
    close(host(actual), expected)
