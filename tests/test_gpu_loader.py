"""The on-disk loader (bh_model_load_dir) against the reference's directory format: a model
written the way src/bin/quantize_model.rs writes it loads to the same device model as one set
tensor by tensor, and generates the oracle's ids; checksum mismatches and formats outside this
path are errors."""
import json
import os

import numpy as np
import pytest

import oracle
from bramha_amd import BhError
from bramha_amd.model import HipDecoder
from refformat import write_reference_dir
from tinymodels import F32, Q4_ROW, Q8_ROW, prompt, tiny_cfg, tiny_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("wfmt", [Q4_ROW, Q8_ROW])
def test_load_reference_dir(plane, tmp_path, wfmt):
    cfg = tiny_cfg(wfmt, F32, gqa7=True)
    w, _ = tiny_weights(cfg, seed=51)
    write_reference_dir(str(tmp_path), cfg, w)
    a = HipDecoder(plane, cfg)
    n = a.load_dir(str(tmp_path))
    assert n == len(w)
    b = HipDecoder(plane, cfg)
    b.load(w)
    p = prompt(9, cfg.vocab, seed=52)
    ia, la = a.generate(p, 10, want_logits=True)
    ib, lb = b.generate(p, 10, want_logits=True)
    assert np.array_equal(ia, ib) and np.array_equal(la, lb)
    om = oracle.OracleModel(cfg)
    om.load(w)
    io, lo = om.generate(p, 10, want_logits=True)
    assert np.array_equal(ia, io)
    assert np.max(np.abs(la - lo)) <= 1e-4 * max(1.0, np.abs(lo).max())


def test_load_reference_dir_errors(plane, tmp_path):
    cfg = tiny_cfg(Q4_ROW, F32)
    w, _ = tiny_weights(cfg, seed=53)
    write_reference_dir(str(tmp_path), cfg, w)
    man = json.load(open(tmp_path / "manifest.json"))
    # a corrupted shard: the SHA-256 no longer matches its manifest entry
    name = "model.layers.0.mlp.down_proj.weight"
    f = tmp_path / (name.replace(".", "_") + "_u4.bin")
    raw = bytearray(f.read_bytes())
    raw[0] ^= 0xFF
    f.write_bytes(bytes(raw))
    with pytest.raises(BhError, match="checksum mismatch"):
        HipDecoder(plane, cfg).load_dir(str(tmp_path))
    # a layer stored in a format outside this path
    man["layers"][name]["compression_format"] = "Svd"
    man["layers"][name]["checksum"] = ""
    json.dump(man, open(tmp_path / "manifest.json", "w"))
    with pytest.raises(BhError, match="not supported"):
        HipDecoder(plane, cfg).load_dir(str(tmp_path))
    with pytest.raises(BhError):
        HipDecoder(plane, cfg).load_dir(str(tmp_path / "missing"))
