"""Prefix KV cache files (src/inference/paged_kv/prefix_cache.rs:37-160) for the device decoder.

An entry is the bincode (2.x, standard configuration) encoding of
`PrefixCacheEntry { tokens: Vec<u32>, keys: Vec<Vec<f32>>, values: Vec<Vec<f32>>,
last_accessed: u64 }`, stored as `<base>/prefix_kv_cache_data/<sha256(tokens as LE u32)>.bin`
for every prefix whose length is a multiple of 16 tokens; keys[layer] / values[layer] are the
flat LayerKvCache rows [tokens][n_kv * head_dim] f32. Lookups try the longest page-aligned
prefix first. `BRAMHA_PREFIX_CACHE=false` disables both directions and `BRAMHA_KV_TRIM_N`
(default 4) trailing tokens are left out of what is saved, as in the reference. After each save
the directory keeps its 20 most recently modified entries (PrefixCacheDb::enforce_limit,
src/storage/cache_db.rs:9-34, called at prefix_cache.rs:162).

The device side moves rows with bh_model_kv_read / bh_model_kv_write
(HipDecoder.kv_read / kv_write); `prefill_cached` is the prefill flow of
generate_cpu_inner_logits with the cache (cpu_engine.rs:2518-2534, 2746-2756).
"""
import hashlib
import os
import re
import struct
import time

import numpy as np

PAGE_SIZE = 16  # prefix_cache.rs:44
CACHE_DIR = "prefix_kv_cache_data"
MAX_ENTRIES = 20  # prefix_cache.rs:162
_USIZE_MAX = (1 << 64) - 1


# ---- bincode standard configuration: little-endian, variable-length integers ----
def _put_varint(out, v):
    if v < 251:
        out.append(v)
    elif v < 1 << 16:
        out += b"\xfb" + struct.pack("<H", v)
    elif v < 1 << 32:
        out += b"\xfc" + struct.pack("<I", v)
    else:
        out += b"\xfd" + struct.pack("<Q", v)


def _get_varint(buf, i):
    b = buf[i]
    if b < 251:
        return b, i + 1
    if b == 251:
        return struct.unpack_from("<H", buf, i + 1)[0], i + 3
    if b == 252:
        return struct.unpack_from("<I", buf, i + 1)[0], i + 5
    if b == 253:
        return struct.unpack_from("<Q", buf, i + 1)[0], i + 9
    raise ValueError("unsupported integer width marker %d" % b)


def encode_entry(tokens, keys, values, last_accessed):
    out = bytearray()
    _put_varint(out, len(tokens))
    for t in tokens:
        _put_varint(out, int(t))
    for mats in (keys, values):
        _put_varint(out, len(mats))
        for m in mats:
            m = np.ascontiguousarray(m, dtype="<f4").ravel()
            _put_varint(out, m.size)
            out += m.tobytes()
    _put_varint(out, int(last_accessed))
    return bytes(out)


def decode_entry(buf):
    """-> (tokens u32 array, keys list of f32 arrays, values list, last_accessed)."""
    i = 0
    n, i = _get_varint(buf, i)
    toks = np.empty(n, np.uint32)
    for j in range(n):
        toks[j], i = _get_varint(buf, i)
    mats = []
    for _ in range(2):
        n_layers, i = _get_varint(buf, i)
        layer = []
        for _ in range(n_layers):
            m, i = _get_varint(buf, i)
            layer.append(np.frombuffer(buf, dtype="<f4", count=m, offset=i).astype(np.float32))
            i += 4 * m
        mats.append(layer)
    last, i = _get_varint(buf, i)
    if i != len(buf):
        raise ValueError("trailing bytes in a prefix cache entry")
    return toks, mats[0], mats[1], last


def compute_tokens_hash(tokens):
    """SHA-256 of the tokens as little-endian u32 (prefix_cache.rs:16-22), hex."""
    return hashlib.sha256(np.ascontiguousarray(tokens, dtype="<u4").tobytes()).hexdigest()


def _enabled():
    return os.environ.get("BRAMHA_PREFIX_CACHE", "") != "false"


def _now_ms():
    return int(time.time() * 1000)


def _trim_n():
    """BRAMHA_KV_TRIM_N as Rust's `parse::<usize>()` reads it (digits with an optional leading
    '+', no sign, spaces or underscores, at most usize::MAX), else 4 (prefix_cache.rs:99-102)."""
    v = os.environ.get("BRAMHA_KV_TRIM_N", "")
    if not re.fullmatch(r"\+?[0-9]+", v):
        return 4
    n = int(v)
    return n if n <= _USIZE_MAX else 4


def enforce_limit(base_path, max_entries):
    """Keep the max_entries most recently modified files of the cache directory and delete the
    rest, oldest first (PrefixCacheDb::enforce_limit, cache_db.rs:9-34). Returns the number
    deleted."""
    cache_dir = os.path.join(base_path, CACHE_DIR)
    if not os.path.isdir(cache_dir):
        return 0
    entries = []
    for e in os.scandir(cache_dir):
        if e.is_file():
            entries.append((e.stat().st_mtime_ns, e.path))
    if len(entries) <= max_entries:
        return 0
    entries.sort(key=lambda x: x[0])  # a stable sort by modification time, oldest first
    gone = 0
    for _, path in entries[:len(entries) - max_entries]:
        try:
            os.remove(path)
            gone += 1
        except OSError:
            pass
    return gone


def find_longest_prefix(base_path, tokens):
    """(prefix_len, (tokens, keys, values, last_accessed)) of the longest cached page-aligned
    prefix of `tokens`, or None (prefix_cache.rs:37-80). A hit refreshes last_accessed."""
    if not _enabled():
        return None
    tokens = np.asarray(tokens, dtype=np.uint32)
    cache_dir = os.path.join(base_path, CACHE_DIR)
    if not os.path.isdir(cache_dir):
        return None
    for pages in range(len(tokens) // PAGE_SIZE, 0, -1):
        plen = pages * PAGE_SIZE
        path = os.path.join(cache_dir, compute_tokens_hash(tokens[:plen]) + ".bin")
        if not os.path.exists(path):
            continue
        try:
            with open(path, "rb") as f:
                toks, keys, values, _ = decode_entry(f.read())
        except (OSError, ValueError, IndexError, struct.error):
            continue
        if np.array_equal(toks, tokens[:plen]):
            with open(path, "wb") as f:
                f.write(encode_entry(toks, keys, values, _now_ms()))
            return plen, (toks, keys, values, _now_ms())
    return None


def save_prefix(base_path, tokens, keys, values):
    """Save every page-aligned prefix of `tokens` not yet on disk (prefix_cache.rs:90-160);
    keys / values: per layer, flat [len(tokens)][dim] f32."""
    if not _enabled():
        return
    tokens = np.asarray(tokens, dtype=np.uint32)
    n = len(tokens)
    trim = _trim_n()
    if n <= trim:
        return
    active = n - trim
    if active < PAGE_SIZE or not keys or np.asarray(keys[0]).size == 0:
        return
    cache_dir = os.path.join(base_path, CACHE_DIR)
    os.makedirs(cache_dir, exist_ok=True)
    dim = np.asarray(keys[0]).size // n
    if dim == 0:
        return
    for pages in range(1, active // PAGE_SIZE + 1):
        plen = pages * PAGE_SIZE
        path = os.path.join(cache_dir, compute_tokens_hash(tokens[:plen]) + ".bin")
        if os.path.exists(path):
            continue
        sl = plen * dim
        pk, pv = [], []
        for k, v in zip(keys, values):
            k, v = np.asarray(k).ravel(), np.asarray(v).ravel()
            if k.size < sl or v.size < sl:
                raise ValueError("KV length is shorter than sliced prefix length")
            pk.append(k[:sl])
            pv.append(v[:sl])
        with open(path, "wb") as f:
            f.write(encode_entry(tokens[:plen], pk, pv, _now_ms()))
    enforce_limit(base_path, MAX_ENTRIES)


def prefill_cached(model, slot, tokens, base_path):
    """Prefill `tokens` into an open slot through the prefix cache: rows of the longest cached
    prefix are written to the device cache instead of computed, the rest is prefilled, and the
    prefilled state is saved back. Returns the number of tokens taken from the cache."""
    tokens = np.asarray(tokens, dtype=np.uint32)
    hit = find_longest_prefix(base_path, tokens)
    plen = 0
    if hit is not None:
        plen, (_, keys, values, _) = hit
        model.kv_write(slot, 0, np.stack(keys).reshape(len(keys), plen, -1),
                       np.stack(values).reshape(len(values), plen, -1))
    if plen < len(tokens):
        model.prefill(slot, tokens[plen:])
    if len(tokens):
        k, v = model.kv_read(slot, 0, len(tokens))
        save_prefix(base_path, tokens, list(k.reshape(k.shape[0], -1)), list(v.reshape(v.shape[0], -1)))
    return plen
