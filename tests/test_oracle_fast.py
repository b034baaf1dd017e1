"""The oracle's token-blocked / parallel loops against its scalar loops in the reference's order.

The fast forms (the default) only place independent chains side by side (tokens in SIMD lanes,
rows and heads on threads); every output keeps the reference's summation order. These tests
pin that claim bit for bit: gemm_cpu, prefill and decode attention and the whole decoder give
identical results with orc_set_fast(0) and (1), and for 1 and several OpenMP threads.
"""
import numpy as np
import pytest

import oracle
from tinymodels import F32, Q4_G32, Q4_ROW, Q8_ROW, prompt, tiny_cfg, tiny_weights


@pytest.fixture
def scalar_then_fast():
    yield
    oracle.set_fast(True)


def _both(fn):
    oracle.set_fast(False)
    a = fn()
    oracle.set_fast(True)
    b = fn()
    return a, b


def _weight(fmt, n, k, rng):
    w = (rng.standard_normal((n, k)) * 0.1).astype(np.float32)
    if fmt == F32:
        return w, None
    if fmt == Q8_ROW:
        return oracle.quantize_int8(w)
    return oracle.quantize_int4(w)


@pytest.mark.parametrize("fmt", [F32, Q8_ROW, Q4_ROW])
@pytest.mark.parametrize("bs,k", [(1, 36), (5, 50), (17, 64), (64, 130), (33, 896)])
def test_gemm_cpu_fast_equals_scalar(scalar_then_fast, fmt, bs, k):
    rng = np.random.default_rng(bs * 1000 + k + fmt)
    n = 37
    w, s = _weight(fmt, n, k, rng)
    hb = rng.standard_normal((bs, k)).astype(np.float32)
    a, b = _both(lambda: oracle.gemm_cpu(fmt, hb, w, s, n))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("nq,nkv,hd", [(14, 2, 64), (4, 2, 128), (8, 8, 64), (8, 1, 64)])
@pytest.mark.parametrize("kv_len", [1, 7, 8, 9, 131])
def test_attention_fast_equals_scalar(scalar_then_fast, nq, nkv, hd, kv_len):
    rng = np.random.default_rng(kv_len * 10 + nq)
    kc = rng.standard_normal((kv_len + 20, nkv * hd)).astype(np.float32)
    vc = rng.standard_normal((kv_len + 20, nkv * hd)).astype(np.float32)
    q = rng.standard_normal(nq * hd).astype(np.float32) * 2
    a, b = _both(lambda: oracle.attn_decode(q, kc[:kv_len], vc[:kv_len], kv_len, nq, nkv, hd))
    assert np.array_equal(a, b)
    bs, start = 13, max(kv_len - 1, 0)
    qb = rng.standard_normal((bs, nq * hd)).astype(np.float32)
    a, b = _both(lambda: oracle.attn_prefill(qb, kc[:start + bs], vc[:start + bs], start, nq, nkv, hd))
    assert np.array_equal(a, b)


@pytest.mark.parametrize("wfmt,head_fmt,kw", [
    (F32, F32, {}), (Q8_ROW, F32, {"gqa7": True}), (Q4_ROW, F32, {"gqa7": True}), (Q4_G32, Q4_G32, {"gqa7": True}),
    (Q4_G32, Q4_G32, {"hidden": 512, "n_heads": 4, "n_kv_heads": 2, "head_dim": 128, "ffn": 768}),
    (F32, F32, {"max_context": 90, "sink_tokens": 4})])
def test_decoder_fast_equals_scalar_and_thread_invariant(scalar_then_fast, wfmt, head_fmt, kw):
    cfg = tiny_cfg(wfmt, head_fmt, **kw)
    w, _ = tiny_weights(cfg, seed=3)
    om = oracle.OracleModel(cfg)
    om.load(w)
    p = prompt(83, cfg.vocab, seed=4)  # 82 prefill tokens: chunks of 64 + 18 (then rows pass 90)
    (ia, la), (ib, lb) = _both(lambda: om.generate(p, 10, want_logits=True))
    assert np.array_equal(ia, ib) and np.array_equal(la, lb)
    n0 = oracle.num_threads()
    try:
        oracle.set_threads(1)
        ic, lc = om.generate(p, 10, want_logits=True)
    finally:
        oracle.set_threads(n0)
    assert np.array_equal(ia, ic) and np.array_equal(la, lc)


@pytest.mark.parametrize("plen", [16, 48, 82])
def test_generate_with_cached_prefix_equals_uncached(plen):
    """A prefix-cache hit (the caches start as the cached rows, the prefill continues at
    prefix_len: cpu_engine.rs:2577-2606) reproduces the uncached run bit for bit, and the rows
    after the prefill are what save_prefix would store."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True)
    w, _ = tiny_weights(cfg, seed=5)
    om = oracle.OracleModel(cfg)
    om.load(w)
    p = prompt(83, cfg.vocab, seed=6)
    ids, lg, (k, v) = om.generate_ex(p, 8, want_logits=True, want_kv=True)
    assert k.shape == (cfg.n_layers, 82, cfg.n_kv_heads * cfg.head_dim)
    ids0, lg0 = om.generate(p, 8, want_logits=True)
    assert np.array_equal(ids, ids0) and np.array_equal(lg, lg0)
    ids2, lg2, (k2, v2) = om.generate_ex(p, 8, want_logits=True, kv_in=(k[:, :plen], v[:, :plen]), want_kv=True)
    assert np.array_equal(ids2, ids) and np.array_equal(lg2, lg)
    assert np.array_equal(k2, k) and np.array_equal(v2, v)
    # a wrong cached row changes the continuation
    kb = k[:, :plen].copy()
    kb[:, 3] += 1.0
    ids3, lg3, _ = om.generate_ex(p, 8, want_logits=True, kv_in=(kb, v[:, :plen]))
    assert np.max(np.abs(lg3[0] - lg[0])) > 1e-4


def test_prefill_past_eviction_limit_is_refused():
    """The reference panics there (its prefill attention reads evicted rows by absolute
    position); the oracle refuses, as the device decoder does."""
    cfg = tiny_cfg(F32, F32, max_context=40, sink_tokens=4)
    w, _ = tiny_weights(cfg, seed=3)
    om = oracle.OracleModel(cfg)
    om.load(w)
    with pytest.raises(ValueError):
        om.generate(prompt(60, cfg.vocab, seed=4), 4)
