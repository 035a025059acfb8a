"""The panel-packed int8 weight layout of the decode GEMV (CPU).

pack_w8_numpy restates the layout declared in include/tinyinfer_amd_ext.h with
array reshapes; it is pinned here against a loop over the definition (record
(cb, kc) at (cb * KC + kc) * 1024 bytes, lane l = column cb*16 + (l & 15), byte
b < 8 = row kc*64 + 8*(l >> 4) + b, byte b >= 8 = row kc*64 + 32 + 8*(l >> 4) +
b - 8, zero past K or N), and the GPU tests compare the device packer with it
byte for byte.  The layout only moves bytes, so parity is bit-exact.
"""
import ctypes as C

import numpy as np
import pytest

from tinyinfer_amd import BACKEND_LIB


def pack_w8_numpy(q):
    """q int8 [K, N] -> packed int8 [ceil(N/16) * ceil(K/64) * 1024]."""
    k, n = q.shape
    kc, nb = -(-k // 64), -(-n // 16)
    qp = np.zeros((kc * 64, nb * 16), np.int8)
    qp[:k, :n] = q
    # row = kc*64 + s*32 + g*8 + r, col = cb*16 + j  ->  [cb][kc][g][j][s][r]
    t = qp.reshape(kc, 2, 4, 8, nb, 16).transpose(4, 0, 2, 5, 1, 3)
    return np.ascontiguousarray(t).reshape(-1)


def pack_w16_numpy(q, scales):
    """q int8 [K, N], scales fp32 [N] -> fp16 records [ceil(N/16) * ceil(K/32) * 512]
    of fp16_rn(float32(q) * scale) (the dequantisation of reference
    kernels/src/cuda/tc/gemm.cu:21,24: an fp32 product, then fp16 rounding)."""
    k, n = q.shape
    kk, nb = -(-k // 32), -(-n // 16)
    deq = (q.astype(np.float32) * scales.astype(np.float32)[None, :]).astype(np.float16)
    dp = np.zeros((kk * 32, nb * 16), np.float16)
    dp[:k, :n] = deq
    # row = kk*32 + g*8 + r, col = cb*16 + j  ->  [cb][kk][g][j][r]
    t = dp.reshape(kk, 4, 8, nb, 16).transpose(3, 0, 1, 4, 2)
    return np.ascontiguousarray(t).reshape(-1)


def pack_w16_loops(q, scales):
    k, n = q.shape
    kk, nb = -(-k // 32), -(-n // 16)
    out = np.zeros(nb * kk * 512, np.float16)
    for cb in range(nb):
        for c in range(kk):
            for lane in range(64):
                col, g = cb * 16 + (lane & 15), lane >> 4
                for r in range(8):
                    row = c * 32 + 8 * g + r
                    if row < k and col < n:
                        out[(cb * kk + c) * 512 + lane * 8 + r] = np.float16(np.float32(q[row, col]) *
                                                                           np.float32(scales[col]))
    return out


def test_pack_w16_numpy_matches_loop_definition():
    rng = np.random.default_rng(4)
    for k, n in ((64, 16), (100, 40), (40, 33)):
        q = rng.integers(-127, 128, (k, n)).astype(np.int8)
        s = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
        assert np.array_equal(pack_w16_numpy(q, s).view(np.uint16), pack_w16_loops(q, s).view(np.uint16))


def pack_w8_loops(q):
    k, n = q.shape
    kc, nb = -(-k // 64), -(-n // 16)
    out = np.zeros(nb * kc * 1024, np.int8)
    for cb in range(nb):
        for c in range(kc):
            for lane in range(64):
                col, g = cb * 16 + (lane & 15), lane >> 4
                for b in range(16):
                    row = c * 64 + (b // 8) * 32 + 8 * g + (b % 8)
                    if row < k and col < n:
                        out[(cb * kc + c) * 1024 + lane * 16 + b] = q[row, col]
    return out


@pytest.mark.parametrize("k,n", [(64, 16), (128, 48), (100, 37), (64, 50), (1, 1), (130, 17)])
def test_numpy_packer_matches_definition(k, n):
    rng = np.random.default_rng(k * 131 + n)
    q = rng.integers(-127, 128, (k, n)).astype(np.int8)
    assert np.array_equal(pack_w8_numpy(q), pack_w8_loops(q))


def test_packed_record_feeds_mfma_operands():
    """Closed form: with q[k, n] = (k + 3n) mod 251 - 125, lane l of record (cb, kc)
    holds column cb*16 + (l & 15) at 8 consecutive rows starting 8*(l >> 4) and
    32 + 8*(l >> 4) -- the B operand layout of v_mfma_f32_16x16x32_f16."""
    k, n = 192, 48
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    q = ((kk + 3 * nn) % 251 - 125).astype(np.int8)
    p = pack_w8_numpy(q).reshape(n // 16, k // 64, 64, 16)
    cb, c, lane = 2, 1, 37
    col, g = cb * 16 + (lane & 15), lane >> 4
    rows = [c * 64 + 8 * g + r for r in range(8)] + [c * 64 + 32 + 8 * g + r for r in range(8)]
    assert p[cb, c, lane].tolist() == [int(q[r, col]) for r in rows]


def test_packed_size_export():
    lib = C.CDLL(str(BACKEND_LIB))
    lib.ti_amd_packed_w8_bytes.restype = C.c_int64
    lib.ti_amd_packed_w8_bytes.argtypes = [C.c_int, C.c_int]
    assert lib.ti_amd_packed_w8_bytes(768, 3072) == 768 * 3072
    assert lib.ti_amd_packed_w8_bytes(768, 50257) == 12 * 3142 * 1024
    assert lib.ti_amd_packed_w8_bytes(100, 17) == 2 * 2 * 1024
    assert lib.ti_amd_packed_w8_bytes(0, 5) == 0
    assert lib.ti_amd_packed_w8_bytes(5, -1) == 0
