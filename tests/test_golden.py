"""Committed fixtures (tests/golden/reference_vectors.npz, written by tests/golden/make_golden.py
from the reference's own deterministic test inputs) against the oracle on the CPU and the device
kernels on the GPU: quantized bytes and scales bit-exact, dequantized weights bit-exact, GEMV and
GEMM within f32 accumulation error of the float64 products, and the reference's bounds
(cpu_engine.rs:3501-3647: |w - deq| <= s/2 + 1e-5; wgpu_backend.rs:1747-1780: |y - y_cpu| < 1e-4)."""
import os

import numpy as np
import pytest

import oracle

G = np.load(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_vectors.npz"))


def _close(got, want, x, deq):
    bound = 2e-6 * (np.abs(x).astype(np.float64) @ np.abs(deq).astype(np.float64).T) + 1e-7
    assert np.all(np.abs(got - want) <= bound)


def test_oracle_quantizers_match_fixtures():
    w = G["w"]
    q8, s8 = oracle.quantize_int8(w)
    q4, s4 = oracle.quantize_int4(w)
    g4, gs = oracle.quantize_q4g32(w)
    for a, b in ((q8, "q8"), (s8, "s8"), (q4, "q4"), (s4, "s4"), (g4, "g4"), (gs, "gs")):
        assert np.array_equal(np.asarray(a).view(np.uint8), G[b].view(np.uint8)), b
    for deq, s, name in ((oracle.dequantize_int8(q8, s8), s8, "deq8"), (oracle.dequantize_int4(q4, s4, 128), s4, "deq4")):
        assert np.array_equal(deq.view(np.uint32), G[name].view(np.uint32)), name
        assert np.all(np.abs(w - deq) <= s[:, None] * 0.5 + 1e-5)
    assert np.array_equal(oracle.dequantize_q4g32(g4, gs, 128).view(np.uint32), G["deqg"].view(np.uint32))


def test_oracle_gemv_matches_fixtures():
    h, hb = G["h"], G["h_block"]
    for fmt, q, s, name in ((oracle.Q8_ROW, G["q8"], G["s8"], "deq8"), (oracle.Q4_ROW, G["q4"], G["s4"], "deq4")):
        _close(oracle.matvec_mul_into(fmt, h, q, s, 64), G[name + "_h"], h[None], G[name])
        _close(oracle.gemm_cpu(fmt, hb, q, s, 64), G[name + "_hb"], hb, G[name])
    y = oracle.matvec_mul_into(oracle.F32, G["wgpu_h"], G["wgpu_w"], None, 64)
    assert np.max(np.abs(y - G["wgpu_y"])) < 1e-4


@pytest.mark.gpu
def test_device_matches_fixtures(plane):
    from bramha_amd import BH_Q4_G32, BH_Q4_ROW, BH_Q8_ROW, ops

    h, hb = G["h"], G["h_block"]
    for fmt, q, s, name in ((BH_Q8_ROW, "q8", "s8", "deq8"), (BH_Q4_ROW, "q4", "s4", "deq4"), (BH_Q4_G32, "g4", "gs", "deqg")):
        dw = ops.DeviceWeight(plane, fmt, 64, 128, G[q], G[s])
        assert np.array_equal(dw.dequant().numpy().view(np.uint32), G[name].view(np.uint32)), name
        for x, want in ((h[None], G[name + "_h"][None]), (hb, G[name + "_hb"])):
            y = dw.gemv(ops.DeviceArray.from_numpy(plane, x)).numpy()
            _close(y, want, x, G[name])
    yw = plane.matvec_mul(G["wgpu_h"], G["wgpu_w"].ravel(), 64)
    assert np.max(np.abs(np.asarray(yw) - G["wgpu_y"])) < 1e-4
