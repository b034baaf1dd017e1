"""Device-pointer operators of the C ABI (bh_gemv, bh_dequant, bh_rmsnorm, bh_rope,
bh_silu_mul, bh_attn_decode). Arguments are torch tensors on the device (torch is
used only for device memory and streams) and work is ordered on the current torch
stream."""
import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib, ptr


def _stream():
    import torch

    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _host_bytes(a):
    a = np.ascontiguousarray(a)
    return a, a.nbytes


class DeviceWeight:
    """A weight uploaded once from its reference layout (bh_weight_upload)."""

    def __init__(self, plane, fmt, n, k, q, scales=None):
        self.plane = plane
        self.fmt, self.n, self.k = fmt, n, k
        q, qb = _host_bytes(q)
        s, sb = (None, 0) if scales is None else _host_bytes(scales)
        h = ctypes.c_void_p()
        check(lib.bh_weight_upload(plane.ctx, fmt, n, k, ptr(q), qb, ptr(s), sb, ctypes.byref(h)), plane.ctx)
        self.handle = h.value

    def free(self):
        if self.handle:
            lib.bh_weight_free(self.plane.ctx, self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass

    def gemv(self, x, y=None):
        import torch

        assert x.is_cuda and x.dtype == torch.float32 and x.is_contiguous() and x.shape[-1] == self.k
        batch = x.numel() // self.k
        if y is None:
            y = torch.empty(batch, self.n, device=x.device, dtype=torch.float32)
        check(lib.bh_gemv(self.plane.ctx, self.handle, ptr(x), ptr(y), batch, _stream()), self.plane.ctx)
        return y

    def dequant(self):
        import torch

        out = torch.empty(self.n, self.k, device="cuda", dtype=torch.float32)
        check(lib.bh_dequant(self.plane.ctx, self.handle, ptr(out), _stream()), self.plane.ctx)
        return out


def rmsnorm(plane, x, w, eps):
    import torch

    rows, n = x.shape
    out = torch.empty_like(x)
    check(lib.bh_rmsnorm(plane.ctx, ptr(x), ptr(w), eps, ptr(out), rows, n, _stream()), plane.ctx)
    return out


def rope_(plane, v, pos, n_heads, head_dim, theta, max_pos):
    rows = pos.numel()
    check(lib.bh_rope(plane.ctx, ptr(v), ptr(pos), rows, n_heads, head_dim, theta, max_pos, _stream()), plane.ctx)
    return v


def silu_mul(plane, g, u):
    import torch

    out = torch.empty_like(g)
    check(lib.bh_silu_mul(plane.ctx, ptr(g), ptr(u), ptr(out), g.numel(), _stream()), plane.ctx)
    return out


def attn_decode(plane, q, k, v, seq_off, seq_len, n_q, n_kv, head_dim, max_len):
    """q: [B, n_q*hd] f32; k, v: [n_kv, rows, hd] (f16 or f32); seq_off int64 [B];
    seq_len int32 [B]."""
    import torch

    batch = q.shape[0]
    out = torch.empty_like(q)
    kv_f16 = 1 if k.dtype == torch.float16 else 0
    check(lib.bh_attn_decode(plane.ctx, ptr(q), ptr(k), ptr(v), kv_f16, k.shape[1], ptr(seq_off), ptr(seq_len),
                             batch, n_q, n_kv, head_dim, max_len, ptr(out), _stream()), plane.ctx)
    return out
