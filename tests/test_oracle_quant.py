"""Pins the oracle's quantizers and dequantizers (src/models/quantization.rs:7-122).

- the reference's own deterministic test (cpu_engine.rs:3501-3647): inputs
  w[i] = 0.5 cos(0.17 i), h[i] = sin(0.31 i), h_block[i] = sin(0.23 i), 64x128, block 4,
  bounds |w - deq| <= s/2 + 1e-5 and quantized == dequantized GEMV/GEMM within 1e-4;
- bit-exact agreement with an independent numpy restatement (tests/ref64.py);
- the closed-form edge cases (all-zero row, +-maxabs, nibble order, NaN).
"""
import numpy as np
import pytest

import oracle
import ref64


def reference_test_inputs():
    out_f, in_f = 64, 128
    i = np.arange(out_f * in_f, dtype=np.float32)
    w = (np.cos(i * np.float32(0.17)) * np.float32(0.5)).astype(np.float32).reshape(out_f, in_f)
    h = np.sin(np.arange(in_f, dtype=np.float32) * np.float32(0.31)).astype(np.float32)
    hb = np.sin(np.arange(4 * in_f, dtype=np.float32) * np.float32(0.23)).astype(np.float32).reshape(4, in_f)
    return w, h, hb


def test_reference_int8_bounds_and_gemv():
    w, h, hb = reference_test_inputs()
    q, s = oracle.quantize_int8(w)
    deq = oracle.dequantize_int8(q, s)
    assert np.all(np.abs(w - deq) <= s[:, None] * 0.5 + 1e-5)
    rf = oracle.matvec_mul(oracle.F32, h, deq, None, 64)
    rq = oracle.matvec_mul(oracle.Q8_ROW, h, q, s, 64)
    assert np.max(np.abs(rf - rq)) < 1e-4
    gf = oracle.gemm_cpu(oracle.F32, hb, deq, None, 64)
    gq = oracle.gemm_cpu(oracle.Q8_ROW, hb, q, s, 64)
    assert np.max(np.abs(gf - gq)) < 1e-4


def test_reference_int4_bounds_and_gemv():
    w, h, hb = reference_test_inputs()
    q, s = oracle.quantize_int4(w)
    deq = oracle.dequantize_int4(q, s, 128)
    assert np.all(np.abs(w - deq) <= s[:, None] * 0.5 + 1e-5)
    rf = oracle.matvec_mul(oracle.F32, h, deq, None, 64)
    rq = oracle.matvec_mul(oracle.Q4_ROW, h, q, s, 64)
    assert np.max(np.abs(rf - rq)) < 1e-4
    gf = oracle.gemm_cpu(oracle.F32, hb, deq, None, 64)
    gq = oracle.gemm_cpu(oracle.Q4_ROW, hb, q, s, 64)
    assert np.max(np.abs(gf - gq)) < 1e-4
    # the decode GEMV (4 partial sums) against the same bound
    rq2 = oracle.matvec_mul_into(oracle.Q4_ROW, h, q, s, 64)
    assert np.max(np.abs(rf - rq2)) < 1e-4


def _weights(seed, n, k, zero_rows=(), ties=False):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    for r in zero_rows:
        w[r] = 0
    if ties:  # exact .5 quotients: x/s lands on k + 0.5
        w[1, :] = 0
        w[1, 0] = 7.0
        w[1, 1:8] = np.float32(2.5)
        w[1, 8:16] = np.float32(-3.5)
    return w


@pytest.mark.parametrize("n,k", [(64, 128), (37, 96), (8, 4864)])
def test_quantizers_bit_exact_numpy(n, k):
    w = _weights(n * k, n, k, zero_rows=(3,), ties=True)
    q8, s8 = oracle.quantize_int8(w)
    r8, rs8 = ref64.quant_int8(w)
    assert np.array_equal(q8, r8) and np.array_equal(s8.view(np.uint32), rs8.view(np.uint32))
    q4, s4 = oracle.quantize_int4(w)
    r4, rs4 = ref64.quant_int4(w)
    assert np.array_equal(q4, r4) and np.array_equal(s4.view(np.uint32), rs4.view(np.uint32))
    g4, gs = oracle.quantize_q4g32(w)
    rg4, rgs = ref64.quant_q4g32(w)
    assert np.array_equal(g4, rg4) and np.array_equal(gs, rgs)


@pytest.mark.parametrize("n,k", [(64, 128), (37, 96)])
def test_dequantizers_bit_exact_numpy(n, k):
    w = _weights(7, n, k, zero_rows=(0,))
    q8, s8 = oracle.quantize_int8(w)
    assert np.array_equal(oracle.dequantize_int8(q8, s8).view(np.uint32), ref64.deq_int8(q8, s8).view(np.uint32))
    q4, s4 = oracle.quantize_int4(w)
    assert np.array_equal(oracle.dequantize_int4(q4, s4, k).view(np.uint32), ref64.deq_int4(q4, s4).view(np.uint32))
    g4, gs = oracle.quantize_q4g32(w)
    assert np.array_equal(oracle.dequantize_q4g32(g4, gs, k).view(np.uint32), ref64.deq_q4g32(g4, gs).view(np.uint32))


def test_edge_cases():
    w = np.zeros((3, 32), np.float32)
    w[1, 5] = 0.7   # +maxabs
    w[2, 6] = -0.7  # -maxabs
    q4, s4 = oracle.quantize_int4(w)
    assert s4[0] == 1.0 and np.all(q4[0] == 0x88)  # all-zero row: scale 1, q = 8
    nib = ref64.unpack4(q4)
    assert nib[1, 5] == 15 and nib[2, 6] == 1 and np.all(np.delete(nib[1], 5) == 8)
    q8, s8 = oracle.quantize_int8(w)
    assert s8[0] == 1.0 and q8[1, 5] == 127 and q8[2, 6] == -127
    # high nibble is the even element
    w2 = np.zeros((1, 2), np.float32)
    w2[0, 0], w2[0, 1] = 1.0, -1.0
    q, s = oracle.quantize_int4(w2)
    assert q[0, 0] == (15 << 4) | 1
    # nibble 0 decodes to -8 * scale
    d = oracle.dequantize_int4(np.array([[0x0F]], np.uint8), np.array([2.0], np.float32), 2)
    assert d[0, 0] == -16.0 and d[0, 1] == 14.0
    # NaN quantizes to 0 (saturating cast), not to garbage
    w3 = np.array([[np.nan, 1.0]], np.float32)
    q, s = oracle.quantize_int8(w3)
    assert q[0, 0] == 0 and q[0, 1] == 127
    with pytest.raises(ValueError):
        oracle.quantize_int4(np.zeros((1, 3), np.float32))


def test_half_conversion_exhaustive():
    hs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = hs.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(h) for h in hs], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    rng = np.random.default_rng(3)
    xs = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * np.float32(0.02),
        (rng.standard_normal(2000) * 1e-6).astype(np.float32),  # subnormal halves
        np.array([65504, 65519.99, 65520, 1e-8, -0.0, 0.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26], np.float32),
    ])
    with np.errstate(over="ignore"):
        want16 = xs.astype(np.float16).view(np.uint16)
    got16 = np.array([oracle.float_to_half(x) for x in xs], np.uint16)
    assert np.array_equal(got16, want16)


def test_q4g32_error_bound():
    w = _weights(11, 48, 256)
    q, s = oracle.quantize_q4g32(w)
    deq = oracle.dequantize_q4g32(q, s, 256)
    sf = np.repeat(s.view(np.float16).astype(np.float32), 32, axis=1)
    # |w - deq| <= s/2 where |w| <= 7 s; the fp16 rounding of s can push the group max past
    # 7 s by at most one fp16 ulp, which the clamp absorbs into a slightly larger error.
    assert np.all(np.abs(w - deq) <= sf * 0.5 + np.abs(w) * 2.0 ** -10 + 1e-7)
