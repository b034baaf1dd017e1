"""ctypes binding of libbramha_hip.so (the C ABI in include/bramha_hip.h).

The library is built in-tree by bramha_amd/build.py. Importing this module without
it raises ImportError: there is no CPU fallback inside the package.
"""
import ctypes
import os
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_uint32, c_uint64, c_void_p

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbramha_hip.so")

if not os.path.exists(LIB_PATH):
    raise ImportError(
        "bramha_amd: %s is missing; build it with `python bramha_amd/build.py` "
        "(or __graft_entry__.build())" % LIB_PATH
    )

lib = ctypes.CDLL(LIB_PATH)

# status codes (bh_status)
BH_OK = 0
BH_ERR_INVALID = -1
BH_ERR_NO_DEVICE = -2
BH_ERR_HIP = -3
BH_ERR_OOM = -4
BH_ERR_NOT_FOUND = -5
BH_ERR_INJECTED = -6
BH_ERR_UNSUPPORTED = -7
BH_ERR_CAPACITY = -8

# weight formats (bh_qfmt)
BH_F32, BH_Q8_ROW, BH_Q4_ROW, BH_Q4_G32 = 0, 1, 2, 3

# fault-injection op ids
BH_OP_ANY, BH_OP_MATVEC, BH_OP_UPLOAD, BH_OP_GEMV, BH_OP_DECODE = 0, 1, 2, 3, 4

# kernel classes for per-kernel timing
KCLASSES = ["gemv_qkv", "attention", "gemv_o", "gemv_gate_up", "gemv_down", "lm_head", "rmsnorm", "other",
            "attn_o"]
BH_K_COUNT = len(KCLASSES)


class bh_model_config(ctypes.Structure):
    _fields_ = [
        ("n_layers", c_int32),
        ("hidden", c_int32),
        ("n_heads", c_int32),
        ("n_kv_heads", c_int32),
        ("head_dim", c_int32),
        ("ffn", c_int32),
        ("vocab", c_int32),
        ("rope_theta", c_float),
        ("rms_eps", c_float),
        ("attn_bias", c_int32),
        ("o_bias", c_int32),
        ("wfmt", c_int32),
        ("head_fmt", c_int32),
        ("max_context", c_int32),
        ("sink_tokens", c_int32),
        ("kv_f16", c_int32),
        ("max_seqs", c_int32),
        ("kv_rows", c_int64),
        ("max_tokens", c_int32),
    ]


_P = c_void_p
_PROTOS = {
    "bh_init": (c_int, [c_int, POINTER(c_void_p)]),
    "bh_destroy": (None, [_P]),
    "bh_last_error": (c_char_p, [_P]),
    "bh_status_str": (c_char_p, [c_int]),
    "bh_set_vram_cap": (c_int, [_P, c_size_t]),
    "bh_registry_stats": (c_int, [_P, POINTER(c_size_t), POINTER(c_size_t)]),
    "bh_debug_inject_fault": (c_int, [_P, c_int, c_int, c_int]),
    "bh_dev_alloc": (c_int, [_P, c_size_t, POINTER(c_void_p)]),
    "bh_dev_free": (c_int, [_P, _P]),
    "bh_memcpy_h2d": (c_int, [_P, _P, _P, c_size_t]),
    "bh_memcpy_d2h": (c_int, [_P, _P, _P, c_size_t]),
    "bh_synchronize": (c_int, [_P]),
    "bh_matvec_mul": (c_int, [_P, _P, c_size_t, _P, c_size_t, c_size_t, c_char_p, c_char_p, _P]),
    "bh_matvec_mul_int8": (c_int, [_P, _P, c_size_t, _P, c_size_t, _P, c_size_t, c_size_t, c_char_p, c_char_p, _P]),
    "bh_matvec_mul_int4": (c_int, [_P, _P, c_size_t, _P, c_size_t, _P, c_size_t, c_size_t, c_char_p, c_char_p, _P]),
    "bh_clear_persistent_buffers": (c_int, [_P]),
    "bh_weight_upload": (c_int, [_P, c_int, c_int64, c_int64, _P, c_size_t, _P, c_size_t, POINTER(c_void_p)]),
    "bh_weight_free": (None, [_P, _P]),
    "bh_gemv": (c_int, [_P, _P, _P, _P, c_int, _P]),
    "bh_dequant": (c_int, [_P, _P, _P, _P]),
    "bh_rmsnorm": (c_int, [_P, _P, _P, c_float, _P, c_int, c_int, _P]),
    "bh_rope": (c_int, [_P, _P, _P, c_int, c_int, c_int, c_float, c_int, _P]),
    "bh_silu_mul": (c_int, [_P, _P, _P, _P, c_int64, _P]),
    "bh_attn_decode": (c_int, [_P, _P, _P, _P, c_int, c_int64, _P, _P, c_int, c_int, c_int, c_int, c_int, _P, _P]),
    "bh_attn_decode_noalloc": (c_int, [_P, _P, _P, _P, c_int, c_int64, _P, _P, c_int, c_int, c_int, c_int, c_int, _P,
                                       _P]),
    "bh_time_gemv": (c_int, [_P, _P, _P, _P, c_int, c_int, c_size_t, POINTER(c_double)]),
    "bh_time_attn": (c_int, [_P, _P, _P, _P, c_int, c_int64, _P, _P, c_int, c_int, c_int, c_int, c_int, _P, c_int,
                             c_size_t, POINTER(c_double)]),
    "bh_time_probe": (c_int, [_P, c_int, c_size_t, c_int, c_int, c_int, POINTER(c_double)]),
    "bh_model_create": (c_int, [_P, POINTER(bh_model_config), POINTER(c_void_p)]),
    "bh_model_load_dir": (c_int, [_P, c_char_p, POINTER(c_int)]),
    "bh_model_kv_read": (c_int, [_P, c_int, c_int64, c_int64, _P, _P]),
    "bh_model_kv_write": (c_int, [_P, c_int, c_int64, c_int64, _P, _P]),
    "bh_model_seq_len": (c_int, [_P, c_int, POINTER(c_int64)]),
    "bh_model_set_sampling": (c_int, [_P, c_float, c_int, c_uint64]),
    "bh_sample_uniform": (c_float, [c_uint64, c_int, c_int]),
    "bh_model_destroy": (None, [_P]),
    "bh_model_set_weight": (c_int, [_P, c_char_p, _P, c_size_t, _P, c_size_t]),
    "bh_model_missing": (c_int, [_P, POINTER(c_int)]),
    "bh_model_seq_open": (c_int, [_P, c_int, c_int64]),
    "bh_model_prefill": (c_int, [_P, c_int, _P, c_int]),
    "bh_model_prefill_batch": (c_int, [_P, c_int, _P, _P, _P]),
    "bh_model_decode_setup": (c_int, [_P, c_int, _P, _P]),
    "bh_model_decode_replace": (c_int, [_P, c_int, c_int, c_uint32]),
    "bh_model_decode": (c_int, [_P, c_int, _P, _P]),
    "bh_model_generate": (c_int, [_P, c_int, _P, c_int, c_int, _P, POINTER(c_int), _P]),
    "bh_model_stream": (c_void_p, [_P]),
    "bh_model_time_kernels": (c_int, [_P, c_int, POINTER(c_double), POINTER(c_int64)]),
    "bh_model_kernel_bytes": (c_int, [_P, c_int, POINTER(c_double)]),
    "bh_synth_normal": (c_int, [c_uint64, c_char_p, c_float, c_int64, _P]),
    "bh_synth_tokens": (c_int, [c_uint64, c_char_p, c_int64, c_uint32, _P]),
    "bh_quantize": (c_int, [c_int, _P, c_int64, c_int64, _P, _P]),
}

for _name, (_res, _args) in _PROTOS.items():
    _f = getattr(lib, _name)
    _f.restype = _res
    _f.argtypes = _args


class BhError(RuntimeError):
    """A non-zero bh_status: the Err(String) of the reference's Result."""

    def __init__(self, status, message):
        super().__init__("%s (%d): %s" % (lib.bh_status_str(status).decode(), status, message))
        self.status = status
        self.message = message


def check(status, ctx=None):
    if status != BH_OK:
        msg = lib.bh_last_error(ctx).decode(errors="replace") if ctx else ""
        raise BhError(status, msg)


def ptr(a):
    """Address of a numpy array, a torch tensor or an int (None -> NULL)."""
    if a is None:
        return None
    if isinstance(a, int):
        return a
    if hasattr(a, "data_ptr"):
        return a.data_ptr()
    return a.ctypes.data
