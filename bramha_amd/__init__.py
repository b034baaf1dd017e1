"""bramha_amd — MI355X (gfx950) compute backend for Bramha's quantized decode path.

The product is libbramha_hip.so (C ABI: include/bramha_hip.h): hand-written HIP
kernels plus the C++ host runtime. This package is its Python binding:

  plane.HipComputePlane   mirror of the reference's WgpuComputePlane GEMV seam
  ops                     single device operators (GEMV, dequant, norm, RoPE, attention)
  model.HipDecoder        the device decoder (prefill, graph-replayed greedy decode)
"""
from . import _lib
from ._lib import BH_F32, BH_Q4_G32, BH_Q4_ROW, BH_Q8_ROW, BhError
from .model import QWEN2_0_5B, QWEN2_7B, DecoderConfig, HipDecoder, synth_weights
from .plane import HipComputePlane, get_hip_plane, is_cpu_only, route_op

__all__ = [
    "BH_F32", "BH_Q8_ROW", "BH_Q4_ROW", "BH_Q4_G32", "BhError", "DecoderConfig", "HipDecoder", "HipComputePlane",
    "QWEN2_0_5B", "QWEN2_7B", "get_hip_plane", "is_cpu_only", "route_op", "synth_weights",
]
