"""The oracle: a CPU restatement of the reference's quantized decode path.

TEST INFRASTRUCTURE ONLY. It is what the HIP backend is compared against;
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import it.
The restatement is oracle/oracle.cpp (built by oracle/Makefile into liboracle.so);
every function there cites the reference file:line it follows.

Pinning (what checks each part independently of the restatement itself) is listed
per function in tests/test_oracle_*.py: the reference's own deterministic test
vectors, closed forms, float64 brute force, and a float64 numpy decoder.
"""
import ctypes
import os
import subprocess
from ctypes import POINTER, c_float, c_int, c_int32, c_int64, c_uint16, c_uint32, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

F32, Q8_ROW, Q4_ROW, Q4_G32 = 0, 1, 2, 3


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


if not os.path.exists(LIB_PATH):
    build()

_lib = ctypes.CDLL(LIB_PATH)
_P = c_void_p


class orc_config(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32), ("hidden", c_int32), ("n_heads", c_int32), ("n_kv_heads", c_int32),
        ("head_dim", c_int32), ("ffn", c_int32), ("vocab", c_int32), ("rope_theta", c_float),
        ("rms_eps", c_float), ("attn_bias", c_int32), ("o_bias", c_int32), ("wfmt", c_int32),
        ("head_fmt", c_int32), ("max_context", c_int32), ("sink_tokens", c_int32),
    ]


_PROTOS = {
    "orc_quantize_int8": (None, [_P, c_int64, c_int64, _P, _P]),
    "orc_quantize_int4": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "orc_dequantize_int8": (None, [_P, _P, c_int64, c_int64, _P]),
    "orc_dequantize_int4": (None, [_P, _P, c_int64, c_int64, _P]),
    "orc_quantize_q4g32": (c_int, [_P, c_int64, c_int64, _P, _P]),
    "orc_dequantize_q4g32": (None, [_P, _P, c_int64, c_int64, _P]),
    "orc_half_to_float": (c_float, [c_uint16]),
    "orc_float_to_half": (c_uint16, [c_float]),
    "orc_matvec_mul_into": (None, [c_int32, _P, c_int64, _P, _P, c_int64, _P]),
    "orc_matvec_mul": (None, [c_int32, _P, c_int64, _P, _P, c_int64, _P]),
    "orc_gemm_cpu": (None, [c_int32, _P, c_int64, c_int64, _P, _P, c_int64, _P]),
    "orc_rms_norm": (None, [_P, _P, c_float, c_int64, _P]),
    "orc_rope_thetas": (None, [c_int64, c_float, _P]),
    "orc_apply_rope": (None, [_P, c_int64, c_int64, c_int64, c_float]),
    "orc_attn_decode": (None, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, _P]),
    "orc_attn_prefill": (None, [_P, _P, _P, c_int64, c_int64, c_int64, c_int64, c_int64, _P]),
    "orc_silu_mul": (None, [_P, _P, c_int64, _P]),
    "orc_penalize_argmax": (c_int64, [_P, c_int64, _P, c_int64]),
    "orc_sample_topk": (c_int64, [_P, c_int64, c_float, c_int, c_float]),
    "orc_model_create": (c_void_p, [POINTER(orc_config)]),
    "orc_model_destroy": (None, [_P]),
    "orc_model_set": (c_int, [_P, ctypes.c_char_p, _P, _P]),
    "orc_generate": (c_int64, [_P, _P, c_int64, c_int64, _P, _P]),
    "orc_generate_ex": (c_int64, [_P, _P, c_int64, c_int64, _P, _P, c_int64, _P, _P, _P, _P, _P]),
    "orc_num_threads": (c_int, []),
    "orc_set_threads": (None, [c_int]),
    "orc_set_fast": (None, [c_int]),
}
for _n, (_r, _a) in _PROTOS.items():
    _f = getattr(_lib, _n)
    _f.restype = _r
    _f.argtypes = _a


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- quantization (src/models/quantization.rs) ----
def quantize_int8(w):
    w = _f32(w)
    n, k = w.shape
    q, s = np.empty((n, k), np.int8), np.empty(n, np.float32)
    _lib.orc_quantize_int8(_p(w), n, k, _p(q), _p(s))
    return q, s


def quantize_int4(w):
    w = _f32(w)
    n, k = w.shape
    q, s = np.empty((n, k // 2), np.uint8), np.empty(n, np.float32)
    if _lib.orc_quantize_int4(_p(w), n, k, _p(q), _p(s)) != 0:
        raise ValueError("in_features must be a multiple of 2 for INT4 packing")
    return q, s


def dequantize_int8(q, s):
    q = np.ascontiguousarray(q, np.int8)
    n, k = q.shape
    out = np.empty((n, k), np.float32)
    _lib.orc_dequantize_int8(_p(q), _p(_f32(s)), n, k, _p(out))
    return out


def dequantize_int4(q, s, k):
    q = np.ascontiguousarray(q, np.uint8)
    n = q.shape[0]
    out = np.empty((n, k), np.float32)
    _lib.orc_dequantize_int4(_p(q), _p(_f32(s)), n, k, _p(out))
    return out


def quantize_q4g32(w):
    w = _f32(w)
    n, k = w.shape
    q, s = np.empty((n, k // 2), np.uint8), np.empty((n, k // 32), np.uint16)
    if _lib.orc_quantize_q4g32(_p(w), n, k, _p(q), _p(s)) != 0:
        raise ValueError("in_features must be a multiple of 32")
    return q, s


def dequantize_q4g32(q, s, k):
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.uint16)
    n = q.shape[0]
    out = np.empty((n, k), np.float32)
    _lib.orc_dequantize_q4g32(_p(q), _p(s), n, k, _p(out))
    return out


def half_to_float(h):
    return _lib.orc_half_to_float(int(h))


def float_to_half(f):
    return _lib.orc_float_to_half(float(f))


# ---- GEMV / GEMM orders ----
def _wargs(fmt, w, s):
    if fmt == F32:
        return _f32(w), None
    if fmt == Q8_ROW:
        return np.ascontiguousarray(w, np.int8), _f32(s)
    return np.ascontiguousarray(w, np.uint8), _f32(s)


def matvec_mul_into(fmt, h, w, s, out_features):
    """cpu_engine.rs:1307-1444 (decode GEMV, 4 partial sums)."""
    h = _f32(h)
    w, s = _wargs(fmt, w, s)
    out = np.empty(out_features, np.float32)
    _lib.orc_matvec_mul_into(fmt, _p(h), h.size, _p(w), _p(s), out_features, _p(out))
    return out


def matvec_mul(fmt, h, w, s, out_features):
    """cpu_engine.rs:355-562 (single running sum)."""
    h = _f32(h)
    w, s = _wargs(fmt, w, s)
    out = np.empty(out_features, np.float32)
    _lib.orc_matvec_mul(fmt, _p(h), h.size, _p(w), _p(s), out_features, _p(out))
    return out


def gemm_cpu(fmt, hb, w, s, out_features):
    """cpu_engine.rs:565-708 (prefill GEMM)."""
    hb = _f32(hb)
    bs, k = hb.shape
    w, s = _wargs(fmt, w, s)
    out = np.empty((bs, out_features), np.float32)
    _lib.orc_gemm_cpu(fmt, _p(hb), bs, k, _p(w), _p(s), out_features, _p(out))
    return out


def rms_norm(x, w, eps):
    x = _f32(x)
    out = np.empty_like(x)
    _lib.orc_rms_norm(_p(x), _p(_f32(w)), eps, x.size, _p(out))
    return out


def rope_thetas(hd, theta):
    out = np.empty(hd // 2, np.float32)
    _lib.orc_rope_thetas(hd, theta, _p(out))
    return out


def apply_rope(v, pos, n_heads, hd, theta):
    v = _f32(v).copy()
    _lib.orc_apply_rope(_p(v), pos, n_heads, hd, theta)
    return v


def attn_decode(q, kc, vc, kv_len, nq, nkv, hd):
    """flash_attention_single_into: q [nq*hd], caches [T][nkv][hd] f32."""
    q, kc, vc = _f32(q), _f32(kc), _f32(vc)
    out = np.empty(nq * hd, np.float32)
    _lib.orc_attn_decode(_p(q), _p(kc), _p(vc), kv_len, nq, nkv, hd, _p(out))
    return out


def attn_prefill(qb, kc, vc, start_pos, nq, nkv, hd):
    qb, kc, vc = _f32(qb), _f32(kc), _f32(vc)
    bs = qb.size // (nq * hd)
    out = np.empty(bs * nq * hd, np.float32)
    _lib.orc_attn_prefill(_p(qb), _p(kc), _p(vc), bs, start_pos, nq, nkv, hd, _p(out))
    return out.reshape(bs, nq * hd)


def silu_mul(g, u):
    g, u = _f32(g), _f32(u)
    out = np.empty_like(g)
    _lib.orc_silu_mul(_p(g), _p(u), g.size, _p(out))
    return out


def penalize_argmax(logits, generated):
    """Returns (argmax id, penalized logits copy)."""
    lg = _f32(logits).copy()
    g = np.ascontiguousarray(generated, np.uint32)
    idx = _lib.orc_penalize_argmax(_p(lg), lg.size, _p(g), g.size)
    return int(idx), lg


def sample_topk(penalized, temperature, top_k, r):
    """The reference's temperature / top-k choice over penalized logits for a given draw r."""
    lg = _f32(penalized)
    return int(_lib.orc_sample_topk(_p(lg), lg.size, float(temperature), int(top_k), float(r)))


def num_threads():
    return _lib.orc_num_threads()


def set_threads(n):
    """OpenMP thread count of the following oracle calls."""
    _lib.orc_set_threads(int(n))


def set_fast(on):
    """True (default): the token-blocked / parallel loops; False: the scalar loops in the
    reference's order that they are pinned against (bit-identical results)."""
    _lib.orc_set_fast(1 if on else 0)


class OracleModel:
    """The reference decode loop (generate_cpu_inner_logits, CPU-only, temperature 0)."""

    def __init__(self, cfg):
        c = orc_config()
        for f, _ in orc_config._fields_:
            v = getattr(cfg, f)
            setattr(c, f, int(v) if isinstance(v, bool) else v)
        self.cfg = cfg
        self._c = c
        self.m = _lib.orc_model_create(ctypes.byref(c))
        self._keep = []

    def close(self):
        if self.m:
            _lib.orc_model_destroy(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set(self, name, data, scales=None):
        d = np.ascontiguousarray(data)
        s = None if scales is None else np.ascontiguousarray(scales)
        if _lib.orc_model_set(self.m, name.encode(), _p(d), _p(s)) != 0:
            raise KeyError(name)

    def load(self, weights):
        for name, data, scales in weights:
            self.set(name, data, scales)

    def generate(self, prompt, max_new, want_logits=False):
        p = np.ascontiguousarray(prompt, np.uint32)
        ids = np.empty(max(max_new, 1), np.uint32)
        lg = np.empty((max(max_new, 1), self.cfg.vocab), np.float32) if want_logits else None
        n = _lib.orc_generate(self.m, _p(p), p.size, max_new, _p(ids), _p(lg))
        if n < 0:
            raise ValueError("prefill past max_context with eviction (the reference's prefill attention "
                             "indexes evicted rows and panics)")
        return (ids[:n].copy(), lg[:n].copy()) if want_logits else ids[:n].copy()

    def generate_ex(self, prompt, max_new, want_logits=False, kv_in=None, want_kv=False):
        """generate with a prefix-cache hit and/or the caches after the prefill.
        kv_in: (k, v) arrays [n_layers][prefix_len][n_kv*head_dim] f32 holding the prompt's first
        prefix_len rows (the prefill then starts at prefix_len). Returns (ids, logits or None,
        (k, v) after the prefill or None)."""
        c = self.cfg
        kd = c.n_kv_heads * c.head_dim
        p = np.ascontiguousarray(prompt, np.uint32)
        ids = np.empty(max(max_new, 1), np.uint32)
        lg = np.empty((max(max_new, 1), c.vocab), np.float32) if want_logits else None
        plen, kin, vin = 0, None, None
        if kv_in is not None:
            kin = np.ascontiguousarray(kv_in[0], np.float32)
            vin = np.ascontiguousarray(kv_in[1], np.float32)
            plen = kin.shape[1]
            assert kin.shape == vin.shape == (c.n_layers, plen, kd)
        rows_cap = max(p.size - 1, 0)
        if c.max_context > 0:
            rows_cap = min(rows_cap, c.max_context)
        rows_cap = max(rows_cap, plen)
        # the library writes [n_layers][rows][kd] contiguously for the row count it reports
        kout = np.empty(c.n_layers * rows_cap * kd, np.float32) if want_kv else None
        vout = np.empty_like(kout) if want_kv else None
        rows = c_int64(0)
        n = _lib.orc_generate_ex(self.m, _p(p), p.size, max_new, _p(ids), _p(lg), plen, _p(kin), _p(vin),
                                 _p(kout), _p(vout), ctypes.byref(rows))
        if n < 0:
            raise ValueError("prefill past max_context with eviction (the reference's prefill attention "
                             "indexes evicted rows and panics)")
        r = rows.value
        assert r <= rows_cap
        kv = (kout[:c.n_layers * r * kd].reshape(c.n_layers, r, kd).copy(),
              vout[:c.n_layers * r * kd].reshape(c.n_layers, r, kd).copy()) if want_kv else None
        return ids[:n].copy(), (lg[:n].copy() if want_logits else None), kv
