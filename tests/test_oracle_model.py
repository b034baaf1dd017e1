"""Pins the oracle's whole decode loop (generate_cpu_inner_logits, cpu_engine.rs:2290-3064)
against an independent float64 numpy decoder on tiny configurations: per-step raw logits
within f32 tolerance and identical greedy ids, for every weight format, GQA 7:1, a
prompt longer than one 64-token prefill chunk, sink eviction, and the EOS stop."""
import numpy as np
import pytest

import oracle
import ref64
from tinymodels import F32, Q4_G32, Q4_ROW, Q8_ROW, prompt, tiny_cfg, tiny_weights


def _run(cfg, n_prompt, max_new, seed=0):
    w, deq = tiny_weights(cfg, seed)
    om = oracle.OracleModel(cfg)
    om.load(w)
    p = prompt(n_prompt, cfg.vocab, seed + 1)
    ids, lg = om.generate(p, max_new, want_logits=True)
    rids, rlg = ref64.Decoder64(cfg, deq).generate(p, max_new)
    return ids, lg, rids, rlg


@pytest.mark.parametrize("wfmt,head_fmt", [(F32, F32), (Q8_ROW, F32), (Q4_ROW, F32), (Q4_G32, Q4_G32)])
def test_oracle_decoder_vs_float64(wfmt, head_fmt):
    cfg = tiny_cfg(wfmt, head_fmt)
    ids, lg, rids, rlg = _run(cfg, 9, 12)
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(lg - rlg)) < 2e-4 * max(1.0, np.abs(rlg).max())


@pytest.mark.parametrize("head_fmt", [F32, Q4_G32])
def test_oracle_untied_lm_head(head_fmt):
    """lm_head.weight present: logits come from it, not the embedding (cpu_engine.rs:2449-2451)."""
    cfg = tiny_cfg(Q4_G32, head_fmt, tied=False)
    ids, lg, rids, rlg = _run(cfg, 9, 10, seed=7)
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(lg - rlg)) < 2e-4 * max(1.0, np.abs(rlg).max())
    # the tied model (same seed, same other tensors) gives different logits
    _, lg2, _, _ = _run(tiny_cfg(Q4_G32, head_fmt), 9, 10, seed=7)
    assert np.max(np.abs(lg2[0] - lg[0])) > 1e-3


def test_oracle_gqa7_and_two_prefill_chunks():
    cfg = tiny_cfg(Q8_ROW, F32, gqa7=True)
    ids, lg, rids, rlg = _run(cfg, 70, 6, seed=3)  # 69 prefill tokens: chunks of 64 + 5
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(lg - rlg)) < 2e-4 * max(1.0, np.abs(rlg).max())


def test_oracle_sink_eviction():
    cfg = tiny_cfg(F32, F32, max_context=8, sink_tokens=4)
    ids, lg, rids, rlg = _run(cfg, 6, 14, seed=5)  # rows exceed 8 after the 3rd step
    assert np.array_equal(ids, rids)
    assert np.max(np.abs(lg - rlg)) < 2e-4 * max(1.0, np.abs(rlg).max())
    # eviction changes the result: without it the logits differ
    cfg2 = tiny_cfg(F32, F32)
    _, lg2, _, _ = _run(cfg2, 6, 14, seed=5)
    assert np.max(np.abs(lg2[-1] - lg[-1])) > 1e-4


def test_oracle_stops_after_eos():
    # vocab 4 keeps id 2 (an EOS id) within reach; the penalty rotates the argmax
    cfg = tiny_cfg(F32, F32, vocab=4)
    for seed in range(6):
        ids, lg, rids, rlg = _run(cfg, 3, 40, seed=seed)
        assert np.array_equal(ids, rids)
        if 2 in ids.tolist():
            assert ids[-1] == 2 and ids.tolist().count(2) == 1 and len(ids) < 40
            return
    pytest.fail("no seed produced the EOS id")
