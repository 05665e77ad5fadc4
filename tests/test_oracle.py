"""Pins the CPU oracle before it is trusted as the parity checker (CPU only).

- value_at vs an independent numpy decoder, bit-exact, every type;
- special cases: d = 0, Q8_0 code -128, every scale_min_k4 pattern, all f16/bf16
  bit patterns;
- the reference's own unit tests (src/quant.rs:973-1063), with their libm
  known-answer inputs;
- scalar dots vs a float64 brute force; AVX2 restatement vs scalar;
- matvec thread-count invariance (src/backend.rs:143-162).
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

import ggml_numpy
from oracle_ffi import AVX2, SCALAR

ALL_TYPES = [0, 1, 30, 2, 3, 6, 7, 8, 12, 13, 14]
_libm = ctypes.CDLL("libm.so.6")
_libm.sinf.restype = _libm.cosf.restype = ctypes.c_float
_libm.sinf.argtypes = _libm.cosf.argtypes = [ctypes.c_float]


def sinf(v):
    return _libm.sinf(ctypes.c_float(v).value)


def cosf(v):
    return _libm.cosf(ctypes.c_float(v).value)


def f32(v):
    return float(np.float32(v))


def seq(n, fn):
    """Rust `(0..n).map(|i| fn(i as f32)).collect::<Vec<f32>>()` with glibc libm."""
    return np.array([fn(float(i)) for i in range(n)], dtype=np.float32)


@pytest.mark.parametrize("ty", ALL_TYPES)
def test_value_at_matches_independent_decoder(llrs, oracle, ty):
    cols = 768 if ty in (12, 13, 14) else 160
    rows = 5
    data = llrs.blocks.random_tensor_bytes(ty, rows, cols, seed=100 + ty)
    want = ggml_numpy.dequantize(data, ty, rows, cols)
    for r in range(rows):
        got = oracle.dequant_row(data, ty, r, cols)
        np.testing.assert_array_equal(got.view(np.uint32), want[r].view(np.uint32))


@pytest.mark.parametrize("ty", [2, 3, 6, 7, 8, 12, 13, 14])
def test_zero_scale_blocks_decode_to_zero(llrs, oracle, ty):
    qt = llrs.QuantType(ty)
    cols = qt.block_size()
    raw = np.frombuffer(llrs.blocks.random_tensor_bytes(ty, 1, cols, seed=7), np.uint8).copy()
    for off in {2: [0], 3: [0, 2], 6: [0], 7: [0, 2], 8: [0], 12: [0, 2], 13: [0, 2],
                14: [208]}[ty]:
        raw[off:off + 2] = 0
    out = oracle.dequant_row(raw.tobytes(), ty, 0, cols)
    assert np.all(out == 0.0)


def test_q8_0_code_minus_128(oracle):
    block = np.zeros(34, np.uint8)
    block[0:2] = np.array([0.5], np.float16).view(np.uint8)
    block[2:] = 0x80
    out = oracle.dequant_row(block.tobytes(), 8, 0, 32)
    assert np.all(out == -64.0)


def test_every_scale_min_k4_pattern(oracle):
    """Q4_K with d = 1, dmin = 0 and all codes 1 decodes to the 6-bit scale of each
    sub-block; with codes 0 and dmin = -1 it decodes to the 6-bit min."""
    rng = np.random.default_rng(3)
    for trial in range(64):
        scales = rng.integers(0, 256, 12, dtype=np.uint8)
        if trial < 2:
            scales[:] = 0 if trial == 0 else 255
        for use_min in (False, True):
            blk = np.zeros(144, np.uint8)
            blk[0:2] = np.array([0.0 if use_min else 1.0], np.float16).view(np.uint8)
            blk[2:4] = np.array([-1.0 if use_min else 0.0], np.float16).view(np.uint8)
            blk[4:16] = scales
            blk[16:] = 0x00 if use_min else 0x11
            out = oracle.dequant_row(blk.tobytes(), 12, 0, 256)
            sc, mn = ggml_numpy._scale_min_k4(scales[None, :])
            want = (mn if use_min else sc)[0]
            np.testing.assert_array_equal(out.reshape(8, 32), np.repeat(want[:, None], 32, 1))


def test_f16_and_bf16_widening_all_patterns(oracle):
    bits = np.arange(65536, dtype=np.uint32)
    f16 = np.array([oracle.lib.oq_f16_to_f32(int(b)) for b in bits], np.float32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    ok = np.isnan(want)
    assert np.array_equal(np.isnan(f16), ok)
    np.testing.assert_array_equal(f16[~ok].view(np.uint32), want[~ok].view(np.uint32))
    bf = np.array([oracle.lib.oq_bf16_to_f32(int(b)) for b in bits[::97]], np.float32)
    wbf = (bits[::97] << 16).view(np.float32)
    nan = np.isnan(wbf)
    np.testing.assert_array_equal(bf[~nan].view(np.uint32), wbf[~nan].view(np.uint32))
    assert np.all(np.isnan(bf[nan]))


@pytest.mark.parametrize("ty", ALL_TYPES)
def test_scalar_dot_vs_float64_brute_force(llrs, oracle, ty):
    cols = 1024 if ty in (12, 13, 14) else 992
    rows = 6
    data = llrs.blocks.random_tensor_bytes(ty, rows, cols, seed=200 + ty)
    x = llrs.blocks.random_activation(cols, seed=300 + ty)
    w = ggml_numpy.dequantize(data, ty, rows, cols).astype(np.float64)
    rb = oracle.row_bytes(ty, cols)
    for r in range(rows):
        want = float(w[r] @ x.astype(np.float64))
        got = oracle.dot(data[r * rb:(r + 1) * rb], ty, x)
        bound = 2 * cols * 2.0 ** -24 * float(np.abs(w[r] * x).sum())  # sequential-sum error
        assert abs(got - want) <= bound, (r, got, want, bound)


@pytest.mark.parametrize("ty", ALL_TYPES)
def test_avx2_restatement_matches_scalar(llrs, oracle, ty):
    if not oracle.has_avx2():
        pytest.skip("CPU lacks AVX2+FMA")
    cols = 512 if ty in (12, 13, 14) else 480
    data = llrs.blocks.random_tensor_bytes(ty, 4, cols, seed=400 + ty)
    x = llrs.blocks.random_activation(cols, seed=500 + ty)
    rb = oracle.row_bytes(ty, cols)
    for r in range(4):
        row = data[r * rb:(r + 1) * rb]
        s, v = oracle.dot(row, ty, x, SCALAR), oracle.dot(row, ty, x, AVX2)
        assert abs(s - v) <= 2e-4 * max(abs(s), 1.0)
        if ty in (1, 30):  # src/simd.rs:296: F16/BF16 use the scalar kernel
            assert s == v


def test_matvec_is_thread_count_invariant(llrs, oracle):
    rows, cols = 1024, 512
    data = llrs.blocks.random_tensor_bytes(12, rows, cols, seed=9)
    x = llrs.blocks.random_activation(cols, seed=10)
    for kernel in (SCALAR, AVX2):
        y1 = oracle.matvec(data, 12, rows, cols, x, kernel, threads=1)
        y8 = oracle.matvec(data, 12, rows, cols, x, kernel, threads=8, threshold=0)
        np.testing.assert_array_equal(y1.view(np.uint32), y8.view(np.uint32))
    rb = oracle.row_bytes(12, cols)
    assert y1[5] == np.float32(oracle.dot(data[5 * rb:6 * rb], 12, x, AVX2))


# ------------------------- the reference's own unit tests (src/quant.rs:969-1063)

def test_reference_q4k_roundtrip_and_dot_are_consistent(llrs, oracle):
    values = seq(512, lambda i: f32(f32(sinf(f32(i * f32(0.17))) + cosf(f32(i * f32(0.03)))) * f32(0.3)))
    t = llrs.QuantTensor.quantize(llrs.QuantType.Q4K, values, 2, 256)
    assert t.quant_type == llrs.QuantType.Q4K
    row = oracle.dequant_row(t.data, 12, 1, 256)
    mae = float(np.abs(row - values[256:]).sum(dtype=np.float32) / np.float32(256))
    assert mae < 0.06, mae
    x = seq(256, lambda i: cosf(f32(i * f32(0.11))))
    expected = float(np.float32(sum(np.float32(a) * np.float32(b) for a, b in zip(row, x))))
    for kernel in (SCALAR, AVX2):
        out = oracle.matvec(t.data, 12, 2, 256, x, kernel)
        assert abs(out[1] - expected) < 1e-4


def test_reference_q4k_shape_falls_back_like_llama_cpp(llrs):
    t = llrs.QuantTensor.quantize(llrs.QuantType.Q4K, np.zeros(896, np.float32), 1, 896)
    assert t.quant_type == llrs.QuantType.Q5_0


def _reference_q5k_block():
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.array([0.003], np.float16).view(np.uint8)
    blk[2:4] = np.array([0.001], np.float16).view(np.uint8)
    blk[4:] = (np.arange(172, dtype=np.uint32) * 73 + 19).astype(np.uint8)
    return blk.tobytes()


def test_reference_avx2_quant_kernels_match_scalar(llrs, oracle):
    if not oracle.has_avx2():
        pytest.skip("CPU lacks AVX2+FMA")
    x = seq(256, lambda i: sinf(f32(i * f32(0.037))))
    values = seq(256, lambda i: f32(f32(sinf(f32(i * f32(0.071))) - cosf(f32(i * f32(0.19)))) * f32(0.2)))
    QT = llrs.QuantType
    tensors = [llrs.QuantTensor.quantize(q, values, 1, 256) for q in (QT.Q4K, QT.Q5_0, QT.Q6K, QT.Q8_0)]
    tensors.append(llrs.QuantTensor.from_owned(_reference_q5k_block(), (1, 256), QT.Q5K))
    assert [t.quant_type for t in tensors] == [QT.Q4K, QT.Q5_0, QT.Q6K, QT.Q8_0, QT.Q5K]
    for t in tensors:
        s = oracle.dot(t.data, int(t.quant_type), x, SCALAR)
        v = oracle.dot(t.data, int(t.quant_type), x, AVX2)
        assert abs(s - v) <= 2e-4 * max(abs(s), 1.0), (t.quant_type, s, v)


def test_reference_q6k_and_q8_roundtrip(llrs, oracle):
    values = seq(512, lambda i: f32(f32(sinf(f32(i * f32(0.071))) - cosf(f32(i * f32(0.19)))) * f32(0.2)))
    QT = llrs.QuantType
    for q, max_mae in ((QT.Q6K, 0.008), (QT.Q8_0, 0.003)):
        t = llrs.QuantTensor.quantize(q, values, 2, 256)
        assert t.quant_type == q
        dec = np.concatenate([oracle.dequant_row(t.data, int(q), r, 256) for r in range(2)])
        mae = float(np.abs(dec - values).sum(dtype=np.float32) / np.float32(512))
        assert mae < max_mae, (q, mae)
        x = seq(256, lambda i: sinf(f32(i * f32(0.13))))
        expected = float(np.float32(sum(np.float32(a) * np.float32(b) for a, b in zip(dec[:256], x))))
        out = oracle.matvec(t.data, int(q), 2, 256, x, AVX2)
        assert abs(out[0] - expected) < 1e-4


def test_quantizer_fallbacks(llrs):
    QT = llrs.QuantType
    z = np.zeros(3 * 96, np.float32)
    assert llrs.QuantTensor.quantize(QT.Q4K, z, 3, 96).quant_type == QT.Q5_0
    assert llrs.QuantTensor.quantize(QT.Q6K, z, 3, 96).quant_type == QT.Q8_0
    assert llrs.QuantTensor.quantize(QT.Q5_0, np.zeros(30, np.float32), 3, 10).quant_type == QT.F32
    t = llrs.QuantTensor.quantize(QT.Q6K, np.zeros(256, np.float32), 1, 256)
    assert t.quant_type == QT.Q6K and t.data == bytes(210)  # all-zero block (src/quant.rs:682-685)


def _total_cmp_key(a: np.ndarray) -> np.ndarray:
    """f32::total_cmp as a signed integer order (IEEE 754 totalOrder):
    -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN."""
    b = a.astype(np.float32).view(np.int32).astype(np.int64)
    return np.where(b < 0, b ^ 0x7FFFFFFF, b)


def test_argmax_total_cmp_last_index_wins(oracle):
    """argmax_current_logits (src/engine.rs:233-241): Iterator::max_by with
    total_cmp keeps the LAST of equal maxima; NaNs order by sign."""
    f32p = ctypes.POINTER(ctypes.c_float)

    def am(v):
        v = np.ascontiguousarray(v, np.float32)
        return int(oracle.lib.oq_argmax(v.ctypes.data_as(f32p), v.size))

    nan, inf = np.float32(np.nan), np.float32(np.inf)
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    assert am([1, 3, 3, 2]) == 2
    assert am([-0.0, 0.0]) == 1 and am([0.0, -0.0]) == 0
    assert am([1, nan, 5]) == 1
    assert am([neg_nan, -inf]) == 1
    assert am([inf, inf, 1]) == 1
    rng = np.random.default_rng(12)
    pool = np.array([-inf, -1.5, -0.0, 0.0, 0.25, 7.0, inf, nan, neg_nan], np.float32)
    for _ in range(200):
        v = pool[rng.integers(0, pool.size, rng.integers(1, 40))]
        k = _total_cmp_key(v)
        want = int(np.flatnonzero(k == k.max())[-1])
        assert am(v) == want, v
