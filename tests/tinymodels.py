"""Small decoder configurations and weights shared by the oracle and GPU tests."""
import numpy as np

import oracle
import ref64
from bramha_amd.model import DecoderConfig, tensor_shapes

F32, Q8_ROW, Q4_ROW, Q4_G32 = 0, 1, 2, 3


def tiny_cfg(wfmt=F32, head_fmt=F32, gqa7=False, **kw):
    if gqa7:  # 7 query heads per KV head, like Qwen2-0.5B and -7B
        base = dict(n_layers=2, hidden=256, n_heads=7, n_kv_heads=1, head_dim=64, ffn=512, vocab=1024)
    else:
        base = dict(n_layers=2, hidden=128, n_heads=2, n_kv_heads=1, head_dim=64, ffn=256, vocab=512)
    base.update(dict(rope_theta=1e6, rms_eps=1e-6, attn_bias=True, wfmt=wfmt, head_fmt=head_fmt,
                     max_seqs=4, kv_rows=4096, max_tokens=64, kv_f16=False))
    base.update(kw)
    return DecoderConfig(**base)


def tiny_weights(cfg, seed=0, sigma=0.05, norm_jitter=True):
    """(list of (name, data, scales) in the config's formats, dict name -> dequantized f32).
    Quantized with the oracle's quantizers."""
    rng = np.random.default_rng(seed)
    out, deq = [], {}
    for name, shape in tensor_shapes(cfg):
        if name.endswith("norm.weight"):
            w = (1.0 + (rng.standard_normal(shape) * 0.1 if norm_jitter else 0)).astype(np.float32)
            out.append((name, w, None))
            deq[name] = w
            continue
        w = (rng.standard_normal(shape) * sigma).astype(np.float32)
        if len(shape) == 1:
            out.append((name, w, None))
            deq[name] = w
            continue
        fmt = cfg.head_fmt if name in ("model.embed_tokens.weight", "lm_head.weight") else cfg.wfmt
        if fmt == F32:
            out.append((name, w, None))
            deq[name] = w
        elif fmt == Q8_ROW:
            q, s = oracle.quantize_int8(w)
            out.append((name, q, s))
            deq[name] = ref64.deq_int8(q, s)
        elif fmt == Q4_ROW:
            q, s = oracle.quantize_int4(w)
            out.append((name, q, s))
            deq[name] = ref64.deq_int4(q, s)
        else:
            q, s = oracle.quantize_q4g32(w)
            out.append((name, q, s))
            deq[name] = ref64.deq_q4g32(q, s)
    return out, deq


def prompt(n, vocab, seed=1):
    return np.random.default_rng(seed).integers(0, vocab, size=n).astype(np.uint32)


def rel_l2(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))
