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
    monkeypatch.setenv("BRAMHA_PREFIX_CACHE", "false")
    assert pc.find_longest_prefix(base, tokens) is None


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
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    ia, la = a.decode_setup([0], [p[-1]]) or a.decode(8, want_logits=True)
    ib, lb = b.decode_setup([0], [p[-1]]) or b.decode(8, want_logits=True)
    assert np.array_equal(ia, ib) and np.array_equal(la, lb)
