"""Independent numpy restatements used to pin the oracle.

Nothing here calls the oracle or the product. Quantizers are restated in numpy f32
arithmetic (bit-exact pins); the math ops and the decoder are textbook float64
(tolerance pins), so a dropped term, a wrong sign or index, or a transposed operand
in the oracle shows up as a mismatch.
"""
import numpy as np

EOS = (2, 151645, 151643)


def round_half_away(v):
    """Rust f32::round on f32 values (exact in float64)."""
    v = np.asarray(v, np.float64)
    return np.sign(v) * np.floor(np.abs(v) + 0.5)


def quant_int8(w):
    w = np.asarray(w, np.float32)
    mx = np.abs(w).max(axis=1)
    s = np.where(mx == 0, np.float32(1.0), (mx / np.float32(127.0)).astype(np.float32)).astype(np.float32)
    v = (w / s[:, None]).astype(np.float32)
    q = np.clip(round_half_away(v), -127, 127).astype(np.int8)
    return q, s


def quant_int4(w):
    w = np.asarray(w, np.float32)
    mx = np.abs(w).max(axis=1)
    s = np.where(mx == 0, np.float32(1.0), (mx / np.float32(7.0)).astype(np.float32)).astype(np.float32)
    v = (w / s[:, None]).astype(np.float32)
    q = (np.clip(round_half_away(v), -7, 7) + 8).astype(np.uint8)
    return ((q[:, 0::2] << 4) | (q[:, 1::2] & 0x0F)).astype(np.uint8), s


def quant_q4g32(w):
    w = np.asarray(w, np.float32)
    n, k = w.shape
    g = w.reshape(n, k // 32, 32)
    mx = np.abs(g).max(axis=2)
    s16 = (mx / np.float32(7.0)).astype(np.float32).astype(np.float16)
    s16 = np.where(mx == 0, np.float16(1.0), s16)
    s16 = np.where(s16 == 0, np.float16(2.0 ** -24), s16).astype(np.float16)
    sf = s16.astype(np.float32)
    v = (g / sf[:, :, None]).astype(np.float32)
    q = (np.clip(round_half_away(v), -7, 7) + 8).astype(np.uint8).reshape(n, k)
    return ((q[:, 0::2] << 4) | (q[:, 1::2] & 0x0F)).astype(np.uint8), s16.view(np.uint16)


def unpack4(q):
    """[n][k/2] bytes -> [n][k] nibble values (high nibble = even element)."""
    q = np.asarray(q, np.uint8)
    out = np.empty((q.shape[0], q.shape[1] * 2), np.uint8)
    out[:, 0::2] = q >> 4
    out[:, 1::2] = q & 0x0F
    return out


def deq_int4(q, s):
    return ((unpack4(q).astype(np.float32) - np.float32(8)) * np.asarray(s, np.float32)[:, None]).astype(np.float32)


def deq_int8(q, s):
    return (np.asarray(q).astype(np.float32) * np.asarray(s, np.float32)[:, None]).astype(np.float32)


def deq_q4g32(q, s16):
    nib = unpack4(q).astype(np.float32) - np.float32(8)
    sf = np.asarray(s16, np.uint16).view(np.float16).astype(np.float32)
    return (nib * np.repeat(sf, 32, axis=1)).astype(np.float32)


def rms_norm(x, w, eps):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def rope(v, pos, nh, hd, theta, ang=None):
    """Rotate-half RoPE in float64. `ang` overrides the per-pair angles (the reference
    forms them in f32 as (pos as f32) * theta_i, which drifts from the exact angle by
    ~pos * 2^-23 rad)."""
    v = np.asarray(v, np.float64).reshape(nh, hd).copy()
    half = hd // 2
    i = np.arange(half, dtype=np.float64)
    if ang is None:
        ang = pos * theta ** (-2.0 * i / hd)
    ang = np.asarray(ang, np.float64)
    c, s = np.cos(ang), np.sin(ang)
    x1, x2 = v[:, :half].copy(), v[:, half:].copy()
    v[:, :half] = x1 * c - x2 * s
    v[:, half:] = x2 * c + x1 * s
    return v.reshape(-1)


def attention(q, kc, vc, kv_len, nq, nkv, hd):
    """softmax(q k^T / sqrt(hd)) v per head, kv head = head // (nq // nkv); caches [T][nkv][hd]."""
    q = np.asarray(q, np.float64).reshape(nq, hd)
    k = np.asarray(kc, np.float64).reshape(-1, nkv, hd)[:kv_len]
    v = np.asarray(vc, np.float64).reshape(-1, nkv, hd)[:kv_len]
    out = np.empty((nq, hd))
    for h in range(nq):
        kh = h // (nq // nkv)
        sc = k[:, kh, :] @ q[h] / np.sqrt(hd)
        p = np.exp(sc - sc.max())
        out[h] = (p / p.sum()) @ v[:, kh, :]
    return out.reshape(-1)


def silu_mul(g, u):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


class Decoder64:
    """Textbook Qwen2 decoder in float64 with the reference's generation rules:
    prefill all prompt tokens but the last, rep penalty 1.15 per generated occurrence,
    first-max argmax, stop after an EOS id, sink eviction of the KV rows."""

    def __init__(self, cfg, tensors):
        self.cfg = cfg
        self.t = {k: np.asarray(v, np.float64) for k, v in tensors.items()}

    def _layer(self, l, x, pos, kv):
        c, t = self.cfg, self.t
        p = "model.layers.%d." % l
        h = rms_norm(x, t[p + "input_layernorm.weight"], c.rms_eps)
        q = t[p + "self_attn.q_proj.weight"] @ h
        k = t[p + "self_attn.k_proj.weight"] @ h
        v = t[p + "self_attn.v_proj.weight"] @ h
        if c.attn_bias:
            q = q + t[p + "self_attn.q_proj.bias"]
            k = k + t[p + "self_attn.k_proj.bias"]
            v = v + t[p + "self_attn.v_proj.bias"]
        q = rope(q, pos, c.n_heads, c.head_dim, c.rope_theta)
        k = rope(k, pos, c.n_kv_heads, c.head_dim, c.rope_theta)
        kv[l][0].append(k)
        kv[l][1].append(v)
        if c.max_context > 0 and len(kv[l][0]) > c.max_context:
            ex = len(kv[l][0]) - c.max_context
            for side in (0, 1):
                del kv[l][side][c.sink_tokens:c.sink_tokens + ex]
        kc, vc = np.array(kv[l][0]), np.array(kv[l][1])
        a = attention(q, kc, vc, len(kc), c.n_heads, c.n_kv_heads, c.head_dim)
        o = t[p + "self_attn.o_proj.weight"] @ a
        if c.o_bias:
            o = o + t[p + "self_attn.o_proj.bias"]
        x = x + o
        h2 = rms_norm(x, t[p + "post_attention_layernorm.weight"], c.rms_eps)
        m = silu_mul(t[p + "mlp.gate_proj.weight"] @ h2, t[p + "mlp.up_proj.weight"] @ h2)
        return x + t[p + "mlp.down_proj.weight"] @ m

    def _forward(self, tok, pos, kv):
        x = self.t["model.embed_tokens.weight"][tok % self.cfg.vocab].copy()
        for l in range(self.cfg.n_layers):
            x = self._layer(l, x, pos, kv)
        return x

    def generate(self, prompt, max_new):
        c = self.cfg
        toks = list(int(t) for t in prompt) or [1]
        kv = [([], []) for _ in range(c.n_layers)]
        for i in range(len(toks) - 1):
            self._forward(toks[i], i, kv)
        gen, logits = [], []
        while len(gen) < max_new:
            x = self._forward(toks[-1], len(toks) - 1, kv)
            head = self.t.get("lm_head.weight", self.t["model.embed_tokens.weight"])  # cpu_engine.rs:2449-2451
            lg = head @ rms_norm(x, self.t["model.norm.weight"], c.rms_eps)
            logits.append(lg.copy())
            for g in gen:
                lg[g] = lg[g] / 1.15 if lg[g] > 0 else lg[g] * 1.15
            nid = int(np.argmax(lg))
            gen.append(nid)
            toks.append(nid)
            if nid in EOS:
                break
        return np.array(gen, np.uint32), np.array(logits)


def synth_normal_np(seed, name, n, sigma):
    """Independent numpy restatement of bh_synth_normal (SplitMix64 + Box-Muller)."""
    m64 = np.uint64(0xFFFFFFFFFFFFFFFF)

    def mix(z):
        z = np.asarray(z, np.uint64)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))

    h = 0xCBF29CE484222325
    for ch in name.encode():
        h ^= ch
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    with np.errstate(over="ignore"):
        key = mix(np.uint64(seed) ^ np.uint64(h))
        pairs = (n + 1) // 2
        i = np.arange(2 * pairs, dtype=np.uint64)
        bits = mix(key + (i + np.uint64(1)) * np.uint64(0x9E3779B97F4A7C15))
    del m64
    u = (bits >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    u1, u2 = 1.0 - u[0::2], u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    ang = 6.283185307179586 * u2
    out = np.empty(2 * pairs, np.float32)
    sig = float(np.float32(sigma))
    out[0::2] = (sig * (r * np.cos(ang))).astype(np.float32)
    out[1::2] = (sig * (r * np.sin(ang))).astype(np.float32)
    return out[:n]
