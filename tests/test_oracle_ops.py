"""Pins the oracle's GEMV orders, RMSNorm, RoPE, attention, SiLU and sampling
against closed forms, the reference's own GEMV test vectors, float64 brute force and
small pure-Python emulations of each accumulation order."""
import numpy as np
import pytest

import oracle
import ref64


def _mats(seed, n, k):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    h = rng.standard_normal(k).astype(np.float32)
    return w, h


@pytest.mark.parametrize("fmt", [oracle.F32, oracle.Q8_ROW, oracle.Q4_ROW])
@pytest.mark.parametrize("n,k", [(64, 128), (300, 96), (128, 4864)])
def test_gemv_orders_vs_float64(fmt, n, k):
    w, h = _mats(n + k + fmt, n, k)
    if fmt == oracle.F32:
        q, s, deq = w, None, w
    elif fmt == oracle.Q8_ROW:
        q, s = oracle.quantize_int8(w)
        deq = ref64.deq_int8(q, s)
    else:
        q, s = oracle.quantize_int4(w)
        deq = ref64.deq_int4(q, s)
    want = deq.astype(np.float64) @ h.astype(np.float64)
    tol = 1e-5 * np.sqrt(k) * (np.abs(deq) @ np.abs(h)).max() / np.sqrt(k) + 1e-6
    for f in (oracle.matvec_mul_into, oracle.matvec_mul):
        assert np.max(np.abs(f(fmt, h, q, s, n) - want)) < tol
    hb = np.stack([h, -h, 0.5 * h])
    g = oracle.gemm_cpu(fmt, hb, q, s, n)
    assert np.max(np.abs(g - np.stack([want, -want, 0.5 * want]))) < tol


def test_reference_wgpu_gemv_vectors():
    # test_wgpu_gemv_vs_cpu (wgpu_backend.rs:1747-1780): h[i] = 0.01 i, w[i] = 1e-4 i, 128 -> 64
    h = (np.arange(128, dtype=np.float32) * np.float32(0.01)).astype(np.float32)
    w = (np.arange(128 * 64, dtype=np.float32) * np.float32(0.0001)).astype(np.float32).reshape(64, 128)
    want = w.astype(np.float64) @ h.astype(np.float64)
    for f in (oracle.matvec_mul_into, oracle.matvec_mul):
        assert np.max(np.abs(f(oracle.F32, h, w, None, 64) - want)) < 1e-4


def test_integer_gemv_exact():
    rng = np.random.default_rng(5)
    q = rng.integers(-127, 128, size=(40, 64)).astype(np.int8)
    s = np.ones(40, np.float32)
    h = np.ones(64, np.float32)
    want = q.astype(np.int64).sum(axis=1).astype(np.float32)
    for f in (oracle.matvec_mul_into, oracle.matvec_mul):
        assert np.array_equal(f(oracle.Q8_ROW, h, q, s, 40), want)


def _f32_loop_4sum(h, w):
    s = [np.float32(0)] * 4
    k = len(h)
    for i in range(k // 4):
        for j in range(4):
            s[j] = np.float32(s[j] + np.float32(h[4 * i + j] * w[4 * i + j]))
    for i in range(k // 4 * 4, k):
        s[0] = np.float32(s[0] + np.float32(h[i] * w[i]))
    return np.float32(np.float32(np.float32(s[0] + s[1]) + s[2]) + s[3])


def _f32_loop_1sum(h, w):
    s = np.float32(0)
    for i in range(len(h)):
        s = np.float32(s + np.float32(h[i] * w[i]))
    return s


def test_accumulation_order_is_the_reference_one():
    # values where the order changes the f32 result: the 4-partial-sum decode GEMV
    # (matvec_mul_into, cpu_engine.rs:1311-1334) and the single sum (matvec_mul, :456-464)
    h = np.array([1e8, 1, 1, 1, -1e8, 1, 1, 1, 3, 7e7, -7e7, 1, 1, 1, 1, 1, 5], np.float32)
    w = np.ones((1, h.size), np.float32)
    a = oracle.matvec_mul_into(oracle.F32, h, w, None, 1)[0]
    b = oracle.matvec_mul(oracle.F32, h, w, None, 1)[0]
    assert a == _f32_loop_4sum(h, w[0]) and b == _f32_loop_1sum(h, w[0]) and a != b


def test_rms_norm_closed_form_and_random():
    w = np.linspace(0.5, 1.5, 96).astype(np.float32)
    x = np.full(96, 3.0, np.float32)
    got = oracle.rms_norm(x, w, 1e-6)
    assert np.allclose(got, 3.0 / np.sqrt(9.0 + 1e-6) * w, rtol=1e-6)
    rng = np.random.default_rng(1)
    x = rng.standard_normal(896).astype(np.float32) * 4
    assert np.allclose(oracle.rms_norm(x, w[:1].repeat(896), 1e-6), ref64.rms_norm(x, w[:1].repeat(896), 1e-6),
                       rtol=2e-6, atol=1e-6)


def test_rope():
    th = oracle.rope_thetas(64, 1e6)
    i = np.arange(32)
    assert np.allclose(th, 1e6 ** (-2.0 * i / 64), rtol=2e-7)
    rng = np.random.default_rng(2)
    v = rng.standard_normal(14 * 64).astype(np.float32)
    assert np.array_equal(oracle.apply_rope(v, 0, 14, 64, 1e6), v)  # pos 0: identity
    for pos in (1, 17, 4095):
        got = oracle.apply_rope(v, pos, 14, 64, 1e6)
        assert np.allclose(got, ref64.rope(v, pos, 14, 64, 1e6), atol=2e-5 + pos * 2e-7)
        ang32 = (np.float32(pos) * th).astype(np.float32)  # the reference's f32 angle
        assert np.allclose(got, ref64.rope(v, pos, 14, 64, 1e6, ang=ang32), atol=3e-6)
        a, b = got.reshape(14, 2, 32), v.reshape(14, 2, 32)
        assert np.allclose(a[:, 0] ** 2 + a[:, 1] ** 2, b[:, 0] ** 2 + b[:, 1] ** 2, rtol=1e-5)


def test_attention_decode():
    rng = np.random.default_rng(4)
    nq, nkv, hd, T = 14, 2, 64, 37
    q = rng.standard_normal(nq * hd).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    got = oracle.attn_decode(q, k, v, T, nq, nkv, hd)
    assert np.allclose(got, ref64.attention(q, k, v, T, nq, nkv, hd), atol=2e-5)
    # kv_len 1: each head returns its KV head's value row
    got1 = oracle.attn_decode(q, k, v, 1, nq, nkv, hd).reshape(nq, hd)
    for h in range(nq):
        assert np.array_equal(got1[h], v[0, h // 7])
    # identical keys: mean of V
    k2 = np.repeat(k[:1], T, axis=0)
    got2 = oracle.attn_decode(q, k2, v, T, nq, nkv, hd).reshape(nq, hd)
    assert np.allclose(got2[0], v[:, 0].mean(axis=0), atol=1e-5)
    assert np.allclose(got2[13], v[:, 1].mean(axis=0), atol=1e-5)


def test_attention_prefill_causal():
    rng = np.random.default_rng(6)
    nq, nkv, hd, start, bs = 4, 2, 64, 5, 6
    T = start + bs
    q = rng.standard_normal((bs, nq * hd)).astype(np.float32)
    k = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    v = rng.standard_normal((T, nkv, hd)).astype(np.float32)
    got = oracle.attn_prefill(q, k, v, start, nq, nkv, hd)
    for b in range(bs):
        assert np.allclose(got[b], ref64.attention(q[b], k, v, start + b + 1, nq, nkv, hd), atol=2e-5)


def test_silu_mul():
    rng = np.random.default_rng(8)
    g = (rng.standard_normal(4864) * 3).astype(np.float32)
    u = rng.standard_normal(4864).astype(np.float32)
    assert np.allclose(oracle.silu_mul(g, u), ref64.silu_mul(g, u), rtol=2e-6, atol=1e-7)
    assert oracle.silu_mul(np.zeros(1, np.float32), np.ones(1, np.float32))[0] == 0.0


def test_penalty_and_argmax():
    lg = np.array([1.0, 3.0, 3.0, -2.0, 0.5], np.float32)
    idx, _ = oracle.penalize_argmax(lg, [])
    assert idx == 1  # first max wins ties
    idx, pl = oracle.penalize_argmax(lg, [1])
    assert idx == 2 and pl[1] == np.float32(3.0) / np.float32(1.15)
    idx, pl = oracle.penalize_argmax(lg, [3, 3, 1, 2, 2])  # compounding; negatives multiplied
    assert pl[3] == np.float32(np.float32(-2.0 * np.float32(1.15)) * np.float32(1.15))
    assert pl[2] == np.float32(np.float32(np.float32(3.0) / np.float32(1.15)) / np.float32(1.15))
    assert idx == 1
    idx, _ = oracle.penalize_argmax(np.array([np.nan, -1.0, np.nan], np.float32), [])
    assert idx == 1  # NaN never compares greater
    idx, _ = oracle.penalize_argmax(np.full(4, -np.inf, np.float32), [])
    assert idx == 0
    idx, pl = oracle.penalize_argmax(lg, [99])  # ids past the vocab are ignored
    assert idx == 1 and np.array_equal(pl, lg)


def test_sample_topk_reference_rules():
    """The temperature branch (cpu_engine.rs:2998-3022) for a given draw r: top_k = 1 is the
    argmax; r = 0 the most likely id; ties keep index order; sweeping r over [0, 1) visits the
    top-k ids with their renormalised probabilities."""
    rng = np.random.default_rng(7)
    lg = (rng.standard_normal(300) * 2).astype(np.float32)
    order = np.argsort(-lg, kind="stable")
    assert oracle.sample_topk(lg, 0.7, 1, 0.99) == int(order[0])
    assert oracle.sample_topk(lg, 0.7, 40, 0.0) == int(order[0])
    tie = np.zeros(50, np.float32)
    assert [oracle.sample_topk(tie, 1.0, 5, r) for r in (0.0, 0.25, 0.45, 0.65, 0.85)] == [0, 1, 2, 3, 4]
    T, k = 0.8, 6
    p = np.exp(lg[order[:k]].astype(np.float64) / T - lg[order[0]] / T)
    p /= p.sum()
    draws = (np.arange(20000) + 0.5) / 20000
    got = np.array([oracle.sample_topk(lg, T, k, r) for r in draws])
    for i in range(k):
        assert abs(np.mean(got == order[i]) - p[i]) < 2e-3
    assert set(got) <= set(order[:k].tolist())
