"""HipComputePlane: the host-side mirror of the reference's WgpuComputePlane.

Reference: src/compute/wgpu_backend.rs:100-1257 (struct, matvec_mul, matvec_mul_int8,
matvec_mul_int4, get_or_create_op, clear_persistent_buffers) and the global getter
get_wgpu_plane (:1707-1728), which returns None in CPU-only mode or when the device
cannot be initialised, after which the caller stays on its CPU path.

Methods take host numpy vectors and return a new host vector, like the reference's
Result<Vec<f32>, String>; an Err is raised as BhError.
"""
import ctypes
import os
import threading

import numpy as np

from . import _lib
from ._lib import BhError, check, lib, ptr


def is_cpu_only():
    """inference::is_cpu_only (src/inference/mod.rs:31-35): BRAMHA_CPU set => CPU only."""
    return "BRAMHA_CPU" in os.environ


def _name(s):
    return s.encode() if isinstance(s, str) else s


class HipComputePlane:
    """One gfx950 device: a stream plus a registry of device-resident weights keyed
    "model:layer", evicted least-recently-used under a byte cap."""

    def __init__(self, device=0):
        h = ctypes.c_void_p()
        st = lib.bh_init(device, ctypes.byref(h))
        if st != _lib.BH_OK:
            raise BhError(st, "device %d" % device)
        self._ctx = h.value
        self.device = device

    @property
    def ctx(self):
        return self._ctx

    def close(self):
        if self._ctx:
            lib.bh_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- WgpuComputePlane::matvec_mul / _int8 / _int4 -------------------------
    def matvec_mul(self, h, weight, out_features, model_name=None, layer_name=None):
        h = np.ascontiguousarray(h, dtype=np.float32)
        w = np.ascontiguousarray(weight, dtype=np.float32).reshape(-1)
        out = np.empty(out_features, dtype=np.float32)
        st = lib.bh_matvec_mul(self._ctx, ptr(h), h.size, ptr(w), w.size, out_features, _name(model_name),
                               _name(layer_name), ptr(out))
        check(st, self._ctx)
        return out

    def matvec_mul_int8(self, h, q_weight, scales, out_features, model_name=None, layer_name=None):
        h = np.ascontiguousarray(h, dtype=np.float32)
        q = np.ascontiguousarray(q_weight, dtype=np.int8).reshape(-1)
        s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        out = np.empty(out_features, dtype=np.float32)
        st = lib.bh_matvec_mul_int8(self._ctx, ptr(h), h.size, ptr(q), q.size, ptr(s), s.size, out_features,
                                    _name(model_name), _name(layer_name), ptr(out))
        check(st, self._ctx)
        return out

    def matvec_mul_int4(self, h, q_weight, scales, out_features, model_name=None, layer_name=None):
        h = np.ascontiguousarray(h, dtype=np.float32)
        q = np.ascontiguousarray(q_weight, dtype=np.uint8).reshape(-1)
        s = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        out = np.empty(out_features, dtype=np.float32)
        st = lib.bh_matvec_mul_int4(self._ctx, ptr(h), h.size, ptr(q), q.size, ptr(s), s.size, out_features,
                                    _name(model_name), _name(layer_name), ptr(out))
        check(st, self._ctx)
        return out

    def clear_persistent_buffers(self):
        check(lib.bh_clear_persistent_buffers(self._ctx), self._ctx)

    # -- registry / policy ----------------------------------------------------
    def set_vram_cap(self, nbytes):
        check(lib.bh_set_vram_cap(self._ctx, nbytes), self._ctx)

    def registry_stats(self):
        n = ctypes.c_size_t()
        b = ctypes.c_size_t()
        check(lib.bh_registry_stats(self._ctx, ctypes.byref(n), ctypes.byref(b)), self._ctx)
        return n.value, b.value

    def inject_fault(self, op=_lib.BH_OP_ANY, status=_lib.BH_ERR_INJECTED, count=1):
        check(lib.bh_debug_inject_fault(self._ctx, op, status, count), self._ctx)


_PLANE = None
_PLANE_LOCK = threading.Lock()
_PLANE_INIT = False


def get_hip_plane():
    """get_wgpu_plane (wgpu_backend.rs:1710-1728): None in CPU-only mode; otherwise the
    process-wide plane, initialised once; None forever if initialisation failed."""
    global _PLANE, _PLANE_INIT
    if is_cpu_only():
        return None
    with _PLANE_LOCK:
        if not _PLANE_INIT:
            _PLANE_INIT = True
            try:
                _PLANE = HipComputePlane(0)
            except BhError:
                _PLANE = None
        return _PLANE


# HeterogeneousScheduler::route_op (src/planner/scheduler.rs:31-62)
CPU, GPU = "cpu", "gpu"


def route_op(size, op_type, gpu_available=None, force_cpu=None):
    if force_cpu is None:
        force_cpu = is_cpu_only()
    if gpu_available is None:
        gpu_available = get_hip_plane() is not None
    if force_cpu or not gpu_available:
        return CPU
    if op_type in ("embedding", "sampling"):
        return CPU
    if op_type == "gemv":
        return CPU if size < 131072 else GPU
    if op_type == "gemm":
        return GPU if size >= 262144 else CPU
    return GPU


def try_gpu_matvec(h, weight_kind, weight, scales, out_features, name=None, layer_name=None, plane=None):
    """The device branch of cpu_engine.rs:matvec_mul (:380-454) without the CPU part:
    returns the device result, or None when the op is routed to the CPU or the device
    call failed; the caller then runs its own CPU GEMV (:430-446). weight_kind is
    "f32", "int8" or "int4"."""
    in_features = int(np.asarray(h).size)
    plane = plane if plane is not None else get_hip_plane()
    if route_op(in_features * out_features, "gemv", gpu_available=plane is not None) != GPU:
        return None
    try:
        if weight_kind == "f32":
            return plane.matvec_mul(h, weight, out_features, name, layer_name)
        if weight_kind == "int8":
            return plane.matvec_mul_int8(h, weight, scales, out_features, name, layer_name)
        if weight_kind == "int4":
            return plane.matvec_mul_int4(h, weight, scales, out_features, name, layer_name)
    except BhError:
        return None
    return None
