"""Writes tests/golden/reference_vectors.npz: the reference's own deterministic test inputs and
the outputs an independent float64 / numpy restatement (tests/ref64.py, not the oracle) gives
for them.

Inputs (the reference's tests):
- test_quantization_correctness (src/inference/cpu_engine.rs:3501-3647): 64 x 128 weights
  w[i] = 0.5 cos(0.17 i), h[i] = sin(0.31 i), a 4-row block h_block[i] = sin(0.23 i);
- test_wgpu_gemv_vs_cpu (src/compute/wgpu_backend.rs:1747-1780): 128 -> 64, h[i] = 0.01 i,
  w[i] = 1e-4 i.
Outputs: int8 / int4 / group-32 quantization (bytes and scales), their dequantized f32 weights,
and float64 products of the dequantized weights with h and h_block.

Run from the repository root: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import ref64  # noqa: E402


def main():
    out_f, in_f = 64, 128
    i = np.arange(out_f * in_f, dtype=np.float32)
    w = (np.cos(i * np.float32(0.17)) * np.float32(0.5)).astype(np.float32).reshape(out_f, in_f)
    h = np.sin(np.arange(in_f, dtype=np.float32) * np.float32(0.31)).astype(np.float32)
    hb = np.sin(np.arange(4 * in_f, dtype=np.float32) * np.float32(0.23)).astype(np.float32).reshape(4, in_f)
    d = {"w": w, "h": h, "h_block": hb}
    q8, s8 = ref64.quant_int8(w)
    q4, s4 = ref64.quant_int4(w)
    g4, gs = ref64.quant_q4g32(w)
    d.update(q8=q8, s8=s8, deq8=ref64.deq_int8(q8, s8), q4=q4, s4=s4, deq4=ref64.deq_int4(q4, s4),
             g4=g4, gs=gs, deqg=ref64.deq_q4g32(g4, gs))
    for name in ("deq8", "deq4", "deqg"):
        m = d[name].astype(np.float64)
        d[name + "_h"] = m @ h.astype(np.float64)
        d[name + "_hb"] = hb.astype(np.float64) @ m.T
    wh = (np.arange(128, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    ww = (np.arange(128 * 64, dtype=np.float32) * np.float32(0.0001)).astype(np.float32).reshape(64, 128)
    d.update(wgpu_h=wh, wgpu_w=ww, wgpu_y=ww.astype(np.float64) @ wh.astype(np.float64))
    np.savez_compressed(os.path.join(HERE, "reference_vectors.npz"), **d)


if __name__ == "__main__":
    main()
