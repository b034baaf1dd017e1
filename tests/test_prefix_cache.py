"""Prefix KV cache file format and lookup (src/inference/paged_kv/prefix_cache.rs): the
reference's own test scenario (test_rolling_prefix_matching_saving_eviction, :190-230), the
token hash test (:175-185), bincode standard-configuration vectors, and, on the GPU, a prefill
that takes its prefix from the cache giving the same decode as a full prefill."""
import os

import numpy as np
import pytest

from bramha_amd import prefix_cache as pc


def test_tokens_hash():
    assert pc.compute_tokens_hash([1, 2, 3, 4]) == pc.compute_tokens_hash([1, 2, 3, 4])
    assert pc.compute_tokens_hash([1, 2, 3, 4]) != pc.compute_tokens_hash([1, 2, 3, 5])
    # SHA-256 of the little-endian u32 bytes 01000000 02000000
    import hashlib
    assert pc.compute_tokens_hash([1, 2]) == hashlib.sha256(bytes([1, 0, 0, 0, 2, 0, 0, 0])).hexdigest()


def test_bincode_layout():
    # varint markers: < 251 one byte; 251 + u16; 252 + u32; 253 + u64 (all little-endian)
    b = pc.encode_entry([5, 300, 70000], [np.array([1.0], np.float32)], [np.zeros(0, np.float32)], 2 ** 40)
    assert b[:1] == bytes([3]) and b[1:2] == bytes([5])
    assert b[2:5] == bytes([251, 0x2C, 0x01]) and b[5:10] == bytes([252, 0x70, 0x11, 0x01, 0x00])
    assert b[10:12] == bytes([1, 1]) and b[12:16] == np.float32(1.0).tobytes()
    assert b[16:18] == bytes([1, 0]) and b[18:] == bytes([253]) + (2 ** 40).to_bytes(8, "little")
    toks, k, v, last = pc.decode_entry(b)
    assert list(toks) == [5, 300, 70000] and k[0].tolist() == [1.0] and v[0].size == 0 and last == 2 ** 40


def test_reference_rolling_prefix_scenario(tmp_path, monkeypatch):
    monkeypatch.setenv("BRAMHA_KV_TRIM_N", "0")
    base = str(tmp_path)
    tokens = np.arange(1, 36, dtype=np.uint32)
    keys = [np.full(35 * 2, 0.5, np.float32), np.full(35 * 2, 0.7, np.float32)]
    values = [np.full(35 * 2, 1.5, np.float32), np.full(35 * 2, 1.7, np.float32)]
    assert pc.find_longest_prefix(base, tokens) is None
    pc.save_prefix(base, tokens, keys, values)  # prefixes of 16 and 32
    assert os.path.isdir(os.path.join(base, pc.CACHE_DIR))
    assert len(os.listdir(os.path.join(base, pc.CACHE_DIR))) == 2
    plen, (toks, k, v, _) = pc.find_longest_prefix(base, tokens)
    assert plen == 32 and list(toks) == list(tokens[:32]) and len(k) == 2 and k[0].size == 64
    assert np.all(k[0] == 0.5) and np.all(v[1] == 1.7)
    plen, (toks, _, _, _) = pc.find_longest_prefix(base, np.arange(1, 21, dtype=np.uint32))
    assert plen == 16 and list(toks) == list(tokens[:16])
    # 6. a sequence sharing no prefix misses (prefix_cache.rs:221-229)
    assert pc.find_longest_prefix(base, np.arange(99, 117, dtype=np.uint32)) is None
    # 7. eviction bounded to one file (:231-242)
    pc.enforce_limit(base, 1)
    assert len([e for e in os.scandir(os.path.join(base, pc.CACHE_DIR)) if e.is_file()]) == 1
    monkeypatch.setenv("BRAMHA_PREFIX_CACHE", "false")
    assert pc.find_longest_prefix(base, tokens) is None


def test_save_keeps_the_20_newest_entries(tmp_path, monkeypatch):
    """save_prefix ends with enforce_limit(base, 20) (prefix_cache.rs:162): the oldest entries
    by modification time go first."""
    monkeypatch.setenv("BRAMHA_KV_TRIM_N", "0")
    base = str(tmp_path)
    cache = os.path.join(base, pc.CACHE_DIR)
    keys = [np.ones(32 * 2, np.float32)]
    made = []
    for i in range(25):
        toks = np.arange(1000 * i, 1000 * i + 16, dtype=np.uint32)
        pc.save_prefix(base, toks, keys, keys)
        path = os.path.join(cache, pc.compute_tokens_hash(toks) + ".bin")
        if os.path.exists(path):
            os.utime(path, ns=(10 ** 18 + i * 10 ** 9, 10 ** 18 + i * 10 ** 9))  # distinct, increasing mtimes
        made.append(path)
    left = sorted(e.path for e in os.scandir(cache) if e.is_file())
    assert len(left) == 20
    assert left == sorted(made[-20:])
    assert pc.enforce_limit(base, 20) == 0 and pc.enforce_limit(str(tmp_path / "none"), 1) == 0


@pytest.mark.parametrize("val,want", [("", 4), ("0", 0), ("7", 7), ("+3", 3), ("-1", 4), (" 2", 4), ("1_0", 4),
                                      ("x", 4), (str(2 ** 64), 4)])
def test_trim_n_parses_like_rust_usize(monkeypatch, val, want):
    monkeypatch.setenv("BRAMHA_KV_TRIM_N", val)
    assert pc._trim_n() == want


@pytest.mark.gpu
@pytest.mark.parametrize("kv_f16", [False, True])
def test_prefill_through_prefix_cache(plane, tmp_path, kv_f16):
    from bramha_amd.model import HipDecoder
    from tinymodels import Q4_G32, prompt, tiny_cfg, tiny_weights

    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=kv_f16)
    w, _ = tiny_weights(cfg, seed=61)
    p = prompt(40, cfg.vocab, seed=62)
    a, b = HipDecoder(plane, cfg), HipDecoder(plane, cfg)
    a.load(w)
    b.load(w)
    base = str(tmp_path)
    a.seq_open(0, 128)
    assert pc.prefill_cached(a, 0, p[:-1], base) == 0  # cold: full prefill, prefixes saved
    b.seq_open(0, 128)
    assert pc.prefill_cached(b, 0, p[:-1], base) == 32  # warm: 32 rows from the cache
    assert a.seq_len(0) == b.seq_len(0) == 39
    ka, va = a.kv_read(0, 0, 39)
    kb, vb = b.kv_read(0, 0, 39)
    # the cached rows are the cold run's own rows; the 7 rows after them were computed by a
    # 7-token pass instead of inside the 39-token one (another kernel, another summation order)
    assert np.array_equal(ka[:, :32], kb[:, :32]) and np.array_equal(va[:, :32], vb[:, :32])
    tol = (2e-3 if kv_f16 else 1e-5) * max(1.0, np.abs(ka).max(), np.abs(va).max())
    assert np.abs(ka - kb).max() <= tol and np.abs(va - vb).max() <= tol
    ia, la = a.decode_setup([0], [p[-1]]) or a.decode(8, want_logits=True)
    ib, lb = b.decode_setup([0], [p[-1]]) or b.decode(8, want_logits=True)
    assert np.array_equal(ia, ib)
    assert np.abs(la - lb).max() <= 1e-3 * max(1.0, np.abs(la).max())


@pytest.mark.gpu
@pytest.mark.parametrize("kv_f16", [False, True])
def test_kv_import_export_against_oracle(plane, kv_f16):
    """The prefix-cache flow against the oracle: the oracle's per-layer KV after a 40-token
    prefill (the rows save_prefix stores, cpu_engine.rs:2746-2756) written to the device with
    bh_model_kv_write reads back unchanged (f32 cache) or fp16-rounded (fp16 cache); the device
    decode continuing from those rows (a cache hit: the remaining prompt tokens prefilled, then
    greedy steps) matches the oracle's decode after the same hit (:2577-2606); and the device's
    own prefill rows are the oracle's within f32 tolerance."""
    import oracle
    from bramha_amd.model import HipDecoder
    from test_gpu_model import agreement
    from tinymodels import Q4_G32, prompt, rel_l2, tiny_cfg, tiny_weights

    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=kv_f16)
    w, _ = tiny_weights(cfg, seed=63)
    om = oracle.OracleModel(cfg)
    om.load(w)
    p = prompt(53, cfg.vocab, seed=64)
    _, _, (k, v) = om.generate_ex(p[:41], 0, want_kv=True)  # rows of the first 40 tokens
    assert k.shape == (cfg.n_layers, 40, cfg.kv_dim)
    plen = 32
    oids, olg, _ = om.generate_ex(p, 12, want_logits=True, kv_in=(k[:, :plen], v[:, :plen]))
    gm = HipDecoder(plane, cfg)
    gm.load(w)
    gm.seq_open(0, 128)
    gm.kv_write(0, 0, k[:, :plen], v[:, :plen])
    assert gm.seq_len(0) == plen
    kr, vr = gm.kv_read(0, 0, plen)
    if kv_f16:
        assert np.array_equal(kr, k[:, :plen].astype(np.float16).astype(np.float32))
        assert np.array_equal(vr, v[:, :plen].astype(np.float16).astype(np.float32))
    else:
        assert np.array_equal(kr, k[:, :plen]) and np.array_equal(vr, v[:, :plen])
    gm.prefill(0, p[plen:-1])
    gm.decode_setup([0], [p[-1]])
    gids, glg = gm.decode(12, want_logits=True)
    n = agreement(oids, gids[:, 0], olg, glg[:, 0])
    assert n == len(oids) == 12
    tol = 2e-2 if kv_f16 else 1e-4 * max(1.0, np.abs(olg).max())
    assert np.max(np.abs(glg[:n, 0] - olg[:n])) <= tol
    assert max(rel_l2(glg[t, 0], olg[t]) for t in range(n)) < 1e-3
    # the device's own prefill rows against the oracle's
    gm.seq_open(1, 128)
    gm.prefill(1, p[:40])
    kd, vd = gm.kv_read(1, 0, 40)
    ref_k = k.astype(np.float16).astype(np.float32) if kv_f16 else k
    ref_v = v.astype(np.float16).astype(np.float32) if kv_f16 else v
    scale = max(1.0, np.abs(k).max(), np.abs(v).max())
    bound = (2e-3 if kv_f16 else 1e-4) * scale
    assert np.abs(kd - ref_k).max() <= bound and np.abs(vd - ref_v).max() <= bound
    gm.close()
