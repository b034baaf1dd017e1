"""Decoder configuration, synthetic weights and the device decoder (bh_model_*).

Config fields mirror what generate_cpu_inner_logits reads from config.json
(src/inference/cpu_engine.rs:2361-2381) plus the device-side choices (weight format,
KV element type, slots and KV rows).
"""
import ctypes
import os
from dataclasses import asdict, dataclass

import numpy as np

from . import _lib
from ._lib import BH_F32, BH_Q4_G32, BH_Q4_ROW, BH_Q8_ROW, check, lib, ptr

EOS_IDS = (2, 151645, 151643)  # cpu_engine.rs:3060

QWEN2_0_5B = dict(n_layers=24, hidden=896, n_heads=14, n_kv_heads=2, head_dim=64, ffn=4864, vocab=151936,
                  rope_theta=1e6, rms_eps=1e-6, attn_bias=True)
QWEN2_7B = dict(n_layers=28, hidden=3584, n_heads=28, n_kv_heads=4, head_dim=128, ffn=18944, vocab=152064,
                rope_theta=1e6, rms_eps=1e-6, attn_bias=True)


@dataclass
class DecoderConfig:
    n_layers: int
    hidden: int
    n_heads: int
    n_kv_heads: int
    head_dim: int
    ffn: int
    vocab: int
    rope_theta: float = 1e6
    rms_eps: float = 1e-6
    attn_bias: bool = True
    o_bias: bool = False
    wfmt: int = BH_Q4_G32
    head_fmt: int = BH_Q4_G32
    max_context: int = 0
    sink_tokens: int = 4
    kv_f16: bool = True
    max_seqs: int = 1
    kv_rows: int = 4096
    max_tokens: int = 64
    tied: bool = True  # False: a separate "lm_head.weight" (host-side only: the C config has no field)

    @property
    def q_dim(self):
        return self.n_heads * self.head_dim

    @property
    def kv_dim(self):
        return self.n_kv_heads * self.head_dim

    def to_c(self):
        c = _lib.bh_model_config()
        for k, v in asdict(self).items():
            if k != "tied":
                setattr(c, k, int(v) if isinstance(v, bool) else v)
        return c


def tensor_shapes(cfg):
    """(name, shape) of every tensor, Hugging Face names (tied LM head)."""
    H, I, V = cfg.hidden, cfg.ffn, cfg.vocab
    out = [("model.embed_tokens.weight", (V, H)), ("model.norm.weight", (H,))]
    if not cfg.tied:
        out.append(("lm_head.weight", (V, H)))
    for l in range(cfg.n_layers):
        p = "model.layers.%d." % l
        out += [
            (p + "input_layernorm.weight", (H,)),
            (p + "post_attention_layernorm.weight", (H,)),
            (p + "self_attn.q_proj.weight", (cfg.q_dim, H)),
            (p + "self_attn.k_proj.weight", (cfg.kv_dim, H)),
            (p + "self_attn.v_proj.weight", (cfg.kv_dim, H)),
            (p + "self_attn.o_proj.weight", (H, cfg.q_dim)),
            (p + "mlp.gate_proj.weight", (I, H)),
            (p + "mlp.up_proj.weight", (I, H)),
            (p + "mlp.down_proj.weight", (H, I)),
        ]
        if cfg.attn_bias:
            out += [(p + "self_attn.q_proj.bias", (cfg.q_dim,)), (p + "self_attn.k_proj.bias", (cfg.kv_dim,)),
                    (p + "self_attn.v_proj.bias", (cfg.kv_dim,))]
        if cfg.o_bias:
            out.append((p + "self_attn.o_proj.bias", (H,)))
    return out


def synth_normal(seed, name, n, sigma):
    out = np.empty(n, dtype=np.float32)
    check(lib.bh_synth_normal(seed, name.encode(), sigma, n, ptr(out)))
    return out


def synth_tokens(seed, name, n, vocab):
    out = np.empty(n, dtype=np.uint32)
    check(lib.bh_synth_tokens(seed, name.encode(), n, vocab, ptr(out)))
    return out


def quantize(fmt, w):
    """Reference-layout quantization: (q, scales) for BH_Q8_ROW / BH_Q4_ROW / BH_Q4_G32."""
    w = np.ascontiguousarray(w, dtype=np.float32)
    n, k = w.shape
    if fmt == BH_Q8_ROW:
        q, s = np.empty((n, k), np.int8), np.empty(n, np.float32)
    elif fmt == BH_Q4_ROW:
        q, s = np.empty((n, k // 2), np.uint8), np.empty(n, np.float32)
    elif fmt == BH_Q4_G32:
        q, s = np.empty((n, k // 2), np.uint8), np.empty((n, k // 32), np.uint16)
    else:
        raise ValueError("not a quantized format: %r" % fmt)
    check(lib.bh_quantize(fmt, ptr(w), n, k, ptr(q), ptr(s)))
    return q, s


def ragged_contexts(seed=0, n_seq=32, lo=128, hi=8192):
    """Context lengths of the ragged batched-decode workload: n_seq draws uniform in [lo, hi]."""
    return np.random.default_rng(seed).integers(lo, hi + 1, size=n_seq)


def synth_weights(cfg, seed=0, sigma=0.02):
    """Random-init weights: matrices and biases N(0, sigma) from the named streams, norms 1.0.
    Yields (name, data, scales) in the formats the config names (scales None for f32)."""
    for name, shape in tensor_shapes(cfg):
        n = int(np.prod(shape))
        if name.endswith("norm.weight"):
            yield name, np.ones(shape, np.float32), None
            continue
        w = synth_normal(seed, name, n, sigma).reshape(shape)
        if len(shape) == 1:
            yield name, w, None
            continue
        fmt = cfg.head_fmt if name in ("model.embed_tokens.weight", "lm_head.weight") else cfg.wfmt
        if fmt == BH_F32:
            yield name, w, None
        else:
            q, s = quantize(fmt, w)
            yield name, q, s


class HipDecoder:
    """The device decoder: bh_model_create / set_weight / seq_open / prefill / decode."""

    def __init__(self, plane, cfg):
        self.plane, self.cfg = plane, cfg
        self._c = cfg.to_c()
        h = ctypes.c_void_p()
        check(lib.bh_model_create(plane.ctx, ctypes.byref(self._c), ctypes.byref(h)), plane.ctx)
        self.m = h.value

    def close(self):
        if self.m:
            lib.bh_model_destroy(self.m)
            self.m = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st):
        check(st, self.plane.ctx)

    def set_weight(self, name, data, scales=None):
        d = np.ascontiguousarray(data)
        s = None if scales is None else np.ascontiguousarray(scales)
        self._check(lib.bh_model_set_weight(self.m, name.encode(), ptr(d), d.nbytes, ptr(s),
                                            0 if s is None else s.nbytes))

    def load(self, weights):
        for name, data, scales in weights:
            self.set_weight(name, data, scales)
        n = ctypes.c_int()
        self._check(lib.bh_model_missing(self.m, ctypes.byref(n)))
        if n.value:
            raise ValueError("%d tensors missing" % n.value)

    def load_dir(self, path):
        """Load a model directory in the reference's on-disk format (bh_model_load_dir); returns
        the number of tensors uploaded."""
        n = ctypes.c_int()
        self._check(lib.bh_model_load_dir(self.m, os.fsencode(path), ctypes.byref(n)))
        return n.value

    def kv_read(self, slot, row0, n):
        """KV rows [row0, row0 + n) of a slot -> (k, v) f32 [n_layers, n, n_kv * head_dim]."""
        c = self.cfg
        k = np.empty((c.n_layers, n, c.kv_dim), np.float32)
        v = np.empty_like(k)
        self._check(lib.bh_model_kv_read(self.m, slot, row0, n, ptr(k), ptr(v)))
        return k, v

    def kv_write(self, slot, row0, k, v):
        """Write KV rows starting at row0 (k, v f32 [n_layers, n, n_kv * head_dim]); the slot's
        length becomes row0 + n."""
        k = np.ascontiguousarray(k, dtype=np.float32)
        v = np.ascontiguousarray(v, dtype=np.float32)
        assert k.shape == v.shape and k.shape[0] == self.cfg.n_layers and k.shape[2] == self.cfg.kv_dim
        self._check(lib.bh_model_kv_write(self.m, slot, row0, k.shape[1], ptr(k), ptr(v)))

    def set_sampling(self, temperature, top_k=40, seed=0):
        """temperature 0: greedy (default); > 0: top-k sampling on the device
        (bh_model_set_sampling)."""
        self._check(lib.bh_model_set_sampling(self.m, float(temperature), int(top_k), int(seed)))

    def seq_len(self, slot):
        n = ctypes.c_int64()
        self._check(lib.bh_model_seq_len(self.m, slot, ctypes.byref(n)))
        return n.value

    def seq_open(self, slot, capacity):
        self._check(lib.bh_model_seq_open(self.m, slot, capacity))

    def prefill(self, slot, tokens):
        t = np.ascontiguousarray(tokens, dtype=np.uint32)
        self._check(lib.bh_model_prefill(self.m, slot, ptr(t), t.size))

    def prefill_batch(self, slots, token_lists):
        """Prefill token_lists[i] into slots[i] for every i in one pass (bh_model_prefill_batch)."""
        s = np.ascontiguousarray(slots, dtype=np.int32)
        counts = np.array([len(t) for t in token_lists], dtype=np.int32)
        toks = np.ascontiguousarray(np.concatenate([np.asarray(t, dtype=np.uint32) for t in token_lists])
                                    if len(token_lists) else np.zeros(0, np.uint32), dtype=np.uint32)
        self._check(lib.bh_model_prefill_batch(self.m, s.size, ptr(s), ptr(toks), ptr(counts)))

    def decode_setup(self, slots, first_tokens):
        s = np.ascontiguousarray(slots, dtype=np.int32)
        t = np.ascontiguousarray(first_tokens, dtype=np.uint32)
        self.batch = s.size
        self._check(lib.bh_model_decode_setup(self.m, s.size, ptr(s), ptr(t)))

    def decode_replace(self, b, slot, first_token):
        self._check(lib.bh_model_decode_replace(self.m, b, slot, int(first_token)))

    def decode(self, n_steps, want_logits=False):
        ids = np.empty((n_steps, self.batch), np.uint32)
        lg = np.empty((n_steps, self.batch, self.cfg.vocab), np.float32) if want_logits else None
        self._check(lib.bh_model_decode(self.m, n_steps, ptr(ids), ptr(lg)))
        return (ids, lg) if want_logits else ids

    def generate(self, prompt, max_new, slot=0, want_logits=False):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        ids = np.empty(max(max_new, 1), np.uint32)
        lg = np.empty((max(max_new, 1), self.cfg.vocab), np.float32) if want_logits else None
        n = ctypes.c_int()
        self._check(lib.bh_model_generate(self.m, slot, ptr(p), p.size, max_new, ptr(ids), ctypes.byref(n), ptr(lg)))
        k = n.value
        return (ids[:k].copy(), lg[:k].copy()) if want_logits else ids[:k].copy()

    def stream(self):
        return lib.bh_model_stream(self.m)

    def time_kernels(self, n_steps):
        mean = (ctypes.c_double * _lib.BH_K_COUNT)()
        cnt = (ctypes.c_int64 * _lib.BH_K_COUNT)()
        self._check(lib.bh_model_time_kernels(self.m, n_steps, mean, cnt))
        return {k: (mean[i], cnt[i]) for i, k in enumerate(_lib.KCLASSES)}

    def kernel_bytes(self, kclass):
        b = ctypes.c_double()
        self._check(lib.bh_model_kernel_bytes(self.m, _lib.KCLASSES.index(kclass), ctypes.byref(b)))
        return b.value
