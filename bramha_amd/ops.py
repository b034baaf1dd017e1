"""Device buffers and single device operators of the C ABI (bh_dev_*, bh_gemv,
bh_dequant, bh_rmsnorm, bh_rope, bh_silu_mul, bh_attn_decode).

Buffers are allocated through the library itself, so no other GPU runtime shares the
process; all work is ordered on the context's stream and every copy back to the host
waits for it."""
import ctypes

import numpy as np

from ._lib import check, lib, ptr


class DeviceArray:
    """A device buffer with a numpy shape and dtype."""

    def __init__(self, plane, shape, dtype):
        self.plane = plane
        self.shape = tuple(int(s) for s in np.atleast_1d(shape))
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        h = ctypes.c_void_p()
        check(lib.bh_dev_alloc(plane.ctx, self.nbytes, ctypes.byref(h)), plane.ctx)
        self.ptr = h.value

    @classmethod
    def from_numpy(cls, plane, a):
        a = np.ascontiguousarray(a)
        d = cls(plane, a.shape, a.dtype)
        check(lib.bh_memcpy_h2d(plane.ctx, d.ptr, ptr(a), a.nbytes), plane.ctx)
        return d

    def numpy(self):
        out = np.empty(self.shape, self.dtype)
        check(lib.bh_memcpy_d2h(self.plane.ctx, ptr(out), self.ptr, self.nbytes), self.plane.ctx)
        return out

    def data_ptr(self):
        return self.ptr

    def free(self):
        if self.ptr and self.plane.ctx:
            lib.bh_dev_free(self.plane.ctx, self.ptr)
        self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class DeviceWeight:
    """A weight uploaded once from its reference layout (bh_weight_upload)."""

    def __init__(self, plane, fmt, n, k, q, scales=None):
        self.plane = plane
        self.fmt, self.n, self.k = fmt, n, k
        q = np.ascontiguousarray(q)
        s = None if scales is None else np.ascontiguousarray(scales)
        h = ctypes.c_void_p()
        check(lib.bh_weight_upload(plane.ctx, fmt, n, k, ptr(q), q.nbytes, ptr(s), 0 if s is None else s.nbytes,
                                   ctypes.byref(h)), plane.ctx)
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

    def gemv(self, x):
        """x: DeviceArray f32 [batch, k] -> DeviceArray f32 [batch, n]."""
        assert x.dtype == np.float32 and x.shape[-1] == self.k
        batch = int(np.prod(x.shape)) // self.k
        y = DeviceArray(self.plane, (batch, self.n), np.float32)
        check(lib.bh_gemv(self.plane.ctx, self.handle, x.ptr, y.ptr, batch, None), self.plane.ctx)
        return y

    def dequant(self):
        out = DeviceArray(self.plane, (self.n, self.k), np.float32)
        check(lib.bh_dequant(self.plane.ctx, self.handle, out.ptr, None), self.plane.ctx)
        return out

    def time_gemv(self, x, y, iters=64, rotate_bytes=1 << 30):
        """Mean microseconds of one bh_gemv launch over x -> y (bh_time_gemv): a graph of
        `iters` launches rotating over device copies of this weight totalling rotate_bytes."""
        batch = int(np.prod(x.shape)) // self.k
        us = ctypes.c_double()
        check(lib.bh_time_gemv(self.plane.ctx, self.handle, x.ptr, y.ptr, batch, iters, rotate_bytes,
                               ctypes.byref(us)), self.plane.ctx)
        return us.value


def rmsnorm(plane, x, w, eps):
    rows, n = x.shape
    out = DeviceArray(plane, x.shape, np.float32)
    check(lib.bh_rmsnorm(plane.ctx, x.ptr, w.ptr, eps, out.ptr, rows, n, None), plane.ctx)
    return out


def rope_(plane, v, pos, n_heads, head_dim, theta, max_pos):
    check(lib.bh_rope(plane.ctx, v.ptr, pos.ptr, pos.shape[0], n_heads, head_dim, theta, max_pos, None), plane.ctx)
    return v


def silu_mul(plane, g, u):
    out = DeviceArray(plane, g.shape, np.float32)
    check(lib.bh_silu_mul(plane.ctx, g.ptr, u.ptr, out.ptr, int(np.prod(g.shape)), None), plane.ctx)
    return out


def kv_tile_index(rows, hd):
    """Element offsets (within one head's region) of the fp16 cache's MFMA-tile layout for a
    [rows][hd] block: (k_idx, v_idx), each [rows][hd] int64 (bh_attn_decode's kv_k_off /
    kv_v_off). rows must be a multiple of 64."""
    tr = 64 if hd == 64 else 32
    t = np.arange(rows, dtype=np.int64)[:, None]
    d = np.arange(hd, dtype=np.int64)[None, :]
    r, base = t % tr, (t // tr) * tr * hd
    blk, lr = 2 * (r // 32) + (r % 8) // 4, 4 * ((r % 32) // 8) + r % 4
    k_idx = base + ((blk * (hd // 32) + d // 32) * 64 + lr + 16 * ((d % 32) // 8)) * 8 + d % 8
    v_idx = base + (((r // 32) * (hd // 16) + d // 16) * 64 + d % 16 + 16 * ((r % 32) // 8)) * 8 + r % 8
    return k_idx, v_idx


def pack_kv_f16(k, v):
    """Row-major K, V [n_kv, rows, hd] (rows a multiple of 64) -> the fp16 cache layout of
    bh_attn_decode, two fp16 arrays [n_kv, rows * hd]."""
    nkv, rows, hd = k.shape
    ki, vi = kv_tile_index(rows, hd)
    kp = np.empty((nkv, rows * hd), np.float16)
    vp = np.empty((nkv, rows * hd), np.float16)
    for h in range(nkv):
        kp[h, ki.ravel()] = k[h].astype(np.float16).ravel()
        vp[h, vi.ravel()] = v[h].astype(np.float16).ravel()
    return kp, vp


def attn_decode(plane, q, k, v, seq_off, seq_len, n_q, n_kv, head_dim, max_len):
    """q: [B, n_q*hd] f32; k, v: [n_kv, rows, hd] row-major f32, or [n_kv, rows*hd] fp16 in the
    tile layout (pack_kv_f16); seq_off int64 [B]; seq_len int32 [B] (all DeviceArrays)."""
    out = DeviceArray(plane, q.shape, np.float32)
    kv_f16 = 1 if k.dtype == np.float16 else 0
    rows = k.shape[1] // head_dim if kv_f16 else k.shape[1]
    check(lib.bh_attn_decode(plane.ctx, q.ptr, k.ptr, v.ptr, kv_f16, rows, seq_off.ptr, seq_len.ptr,
                             q.shape[0], n_q, n_kv, head_dim, max_len, out.ptr, None), plane.ctx)
    return out


def time_attn(plane, q, k, v, seq_off, seq_len, n_q, n_kv, head_dim, max_len, iters=64, rotate_bytes=1 << 30):
    """Mean microseconds of one bh_attn_decode launch (bh_time_attn), K/V rotated over device
    copies totalling rotate_bytes."""
    out = DeviceArray(plane, q.shape, np.float32)
    kv_f16 = 1 if k.dtype == np.float16 else 0
    rows = k.shape[1] // head_dim if kv_f16 else k.shape[1]
    us = ctypes.c_double()
    check(lib.bh_time_attn(plane.ctx, q.ptr, k.ptr, v.ptr, kv_f16, rows, seq_off.ptr, seq_len.ptr,
                           q.shape[0], n_q, n_kv, head_dim, max_len, out.ptr, iters, rotate_bytes,
                           ctypes.byref(us)), plane.ctx)
    out.free()
    return us.value


def synchronize(plane):
    check(lib.bh_synchronize(plane.ctx), plane.ctx)


def time_probe(plane, copy, nbytes, wgs, unroll, iters=20):
    """Mean microseconds of one probe launch (bh_time_probe): copy = False streams nbytes with
    16-byte non-temporal loads, True copies them into a second buffer, 2 is one link of a chain of
    dependent launches over nbytes / 4 floats, 3 one grid-barrier phase of a resident grid (the
    time per phase)."""
    us = ctypes.c_double()
    mode = copy if copy in (2, 3) else (1 if copy else 0)
    check(lib.bh_time_probe(plane.ctx, mode, nbytes, wgs, unroll, iters, ctypes.byref(us)), plane.ctx)
    return us.value
