"""GPU parity at the full sizes of the two heavy workloads.

Ragged batched decode (Qwen2-0.5B shape, 4-bit g32, fp16 KV): 32 sequences with contexts drawn
uniformly from [128, 8192] by seed and prefilled at prefix-sum offsets of one packed KV buffer,
128 decode steps with one sequence replaced halfway by a new 64-token prompt.
  - every sequence's ids equal its own batch-1 decode on the device (numerical ties excepted,
    judged on the batch-1 run's penalized logits), logits at the checkpoint steps within
    2e-2 max-abs / 1e-3 relative L2 of the batch-1 run, everything finite;
  - the refilled sequence against the oracle (64 ids, logits);
  - the reference's sink eviction at this shape (max_context 4096, 4 sinks,
    cpu_engine.rs:1728-1754): a 4080-row context decoded 40 steps past 4096 rows, against the
    oracle.

Qwen2-7B widths (hidden 3584, 28/4 heads of 128, FFN 18944, vocab 152064, untied LM head,
4-bit g32, fp16 KV) with 2 of the 28 layers: a 2048-token prompt (2047 prefilled through the
tiled MFMA GEMM and causal attention), then 16 decode steps at batch 1 against the oracle, and
at batch 16 (16 such prompts) against each sequence's batch-1 decode.

The oracle runs the reference's CPU loops (strict f32 in its summation order; tokens and rows
of the prefill spread over threads without changing any sum).
"""
import numpy as np
import pytest

import oracle
from bramha_amd import BH_Q4_G32
from bramha_amd.model import (QWEN2_0_5B, QWEN2_7B, DecoderConfig, HipDecoder, ragged_contexts, synth_tokens,
                              synth_weights)
from test_gpu_model import agreement, penalized
from tinymodels import rel_l2

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def _tie_ok(ref_raw, ref_ids, t, err):
    """Step t of a run whose ids differ from ref_ids[t] is a numerical tie of the reference run."""
    top2 = np.sort(penalized(ref_raw, ref_ids[:t]))[-2:]
    return top2[1] - top2[0] <= 10 * err


def _batch1(gm, slot, prompt, n_steps):
    """Decode of one sequence alone at batch 1 in `slot`: ids and raw logits of every step."""
    gm.seq_open(slot, len(prompt) + n_steps + 16)
    gm.prefill(slot, prompt[:-1])
    gm.decode_setup([slot], [prompt[-1]])
    ids, lg = gm.decode(n_steps, want_logits=True)
    return ids[:, 0], lg[:, 0]


@pytest.mark.timeout(900)
def test_ragged_32_sequences_with_refill_and_eviction(plane):
    seed, n_seq, steps, half = 0, 32, 128, 64
    ctx = ragged_contexts(seed, n_seq)
    caps = [int(c) + steps + 16 for c in ctx]
    new_len, refill_b = 64, 5
    rows = 2 * (sum(caps) + new_len + steps + 16) + 64 * 2 * (n_seq + 1)
    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=2 * n_seq + 2,
                        kv_rows=rows, max_tokens=2048)
    say("contexts", int(ctx.min()), "..", int(ctx.max()), "sum", int(ctx.sum()))
    w = list(synth_weights(cfg, seed=seed))
    gm = HipDecoder(plane, cfg)
    gm.load(w)
    prompts = [synth_tokens(seed, "ragged.%d" % s, int(ctx[s]), cfg.vocab) for s in range(n_seq)]
    newp = synth_tokens(seed, "ragged.new.%d" % n_seq, new_len, cfg.vocab)
    for s, p in enumerate(prompts):
        gm.seq_open(s, caps[s])
        gm.prefill(s, p[:-1])
    say("prefilled")
    # the batched run: ids of every step, raw logits at the checkpoint steps
    gm.decode_setup(list(range(n_seq)), [p[-1] for p in prompts])
    ids = np.zeros((steps, n_seq), np.uint32)
    ck = {}
    for t0, t1, want in ((0, 1, True), (1, half - 1, False), (half - 1, half, True)):
        out = gm.decode(t1 - t0, want_logits=want)
        ids[t0:t1] = out[0] if want else out
        if want:
            ck[t0] = out[1][0].copy()
    gm.seq_open(n_seq, new_len + steps)
    gm.prefill(n_seq, newp[:-1])
    gm.decode_replace(refill_b, n_seq, newp[-1])
    for t0, t1, want in ((half, half + 1, True), (half + 1, steps - 1, False), (steps - 1, steps, True)):
        out = gm.decode(t1 - t0, want_logits=want)
        ids[t0:t1] = out[0] if want else out
        if want:
            ck[t0] = out[1][0].copy()
    for t, a in ck.items():
        assert np.isfinite(a).all(), t
    say("batched run done")

    # each sequence alone at batch 1 (its own slot), compared step by step
    seqs = [(s, prompts[s], 0, steps if s != refill_b else half) for s in range(n_seq)]
    seqs.append((refill_b, newp, half, steps - half))  # the refilled entry: column refill_b from step 64
    diverged = 0
    b1_refill = None
    for i, (b, p, t0, n) in enumerate(seqs):
        rids, rlg = _batch1(gm, n_seq + 1 + i, p, n)
        assert np.isfinite(rlg).all(), i
        got = ids[t0:t0 + n, b]
        errs = [np.abs(ck[t][b] - rlg[t - t0]).max() for t in ck if t0 <= t < t0 + n]
        err = max(errs + [1e-5])
        m = n
        for t in range(n):
            if got[t] != rids[t]:
                assert _tie_ok(rlg[t], rids, t, err), (i, t, err)
                say("sequence", i, "numerical tie at step", t)
                m = t
                diverged += 1
                break
        for t in ck:
            if t0 <= t < t0 + m:
                assert np.abs(ck[t][b] - rlg[t - t0]).max() <= 2e-2, (i, t)
                assert rel_l2(ck[t][b], rlg[t - t0]) <= 1e-3, (i, t)
        if i == n_seq:
            b1_refill = (rids, rlg)
    assert diverged <= 3
    say("batch-1 comparisons done,", diverged, "numerical ties")
    gm.close()

    # the refilled sequence against the oracle
    om = oracle.OracleModel(cfg)
    om.load(w)
    oids, olg = om.generate(newp, steps - half, want_logits=True)
    n = agreement(oids, b1_refill[0], olg, b1_refill[1])
    assert n == len(oids)
    for t in range(n):
        assert np.max(np.abs(b1_refill[1][t] - olg[t])) <= 2e-2 and rel_l2(b1_refill[1][t], olg[t]) <= 1e-3, t
    say("refilled sequence matches the oracle")

    # the reference eviction at this shape: 4080 prefilled rows, 40 steps crossing 4096
    cfg_e = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=1, kv_rows=4096,
                          max_tokens=2048, max_context=4096, sink_tokens=4)
    ge = HipDecoder(plane, cfg_e)
    ge.load(w)
    pe = synth_tokens(seed, "ragged.evict", 4081, cfg.vocab)
    gids, glg = ge.generate(pe, 40, want_logits=True)
    ge.close()
    om.close()
    oe = oracle.OracleModel(cfg_e)
    oe.load(w)
    del w
    oids, olg = oe.generate(pe, 40, want_logits=True)
    oe.close()
    n = agreement(oids, gids, olg, glg)
    say("eviction: ids equal for", n, "of", len(oids), "steps")
    assert n == len(oids) == 40
    for t in range(n):
        assert np.max(np.abs(glg[t] - olg[t])) <= 2e-2 and rel_l2(glg[t], olg[t]) <= 1e-3, t


@pytest.mark.timeout(900)
def test_qwen2_7b_widths_prefill_2048_decode_b1_b16(plane):
    seed, plen, steps, nb = 0, 2048, 16, 16
    shape = dict(QWEN2_7B, n_layers=2)
    cfg = DecoderConfig(**shape, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=2 * nb + 1,
                        kv_rows=(2 * nb + 1) * (plen + steps + 64), max_tokens=plen, tied=False)
    w = list(synth_weights(cfg, seed=seed))
    gm = HipDecoder(plane, cfg)
    gm.load(w)
    prompts = [synth_tokens(seed, "7b.prompt.%d" % s, plen, cfg.vocab) for s in range(nb)]
    # batch 16
    for s, p in enumerate(prompts):
        gm.seq_open(s, plen + steps + 16)
        gm.prefill(s, p[:-1])
    gm.decode_setup(list(range(nb)), [p[-1] for p in prompts])
    ids, lg = gm.decode(steps, want_logits=True)
    assert np.isfinite(lg).all()
    say("batch 16 done")
    diverged = 0
    b1 = None
    for s, p in enumerate(prompts):
        rids, rlg = _batch1(gm, nb + s, p, steps)
        if s == 0:
            b1 = (rids, rlg)
        m = steps
        for t in range(steps):
            if ids[t, s] != rids[t]:
                assert _tie_ok(rlg[t], rids, t, max(np.abs(lg[t, s] - rlg[t]).max(), 1e-5)), (s, t)
                m = t
                diverged += 1
                break
        for t in range(m):
            assert np.abs(lg[t, s] - rlg[t]).max() <= 2e-2 and rel_l2(lg[t, s], rlg[t]) <= 1e-3, (s, t)
    assert diverged <= 2
    say("batch-1 comparisons done,", diverged, "numerical ties")
    gm.close()
    # batch 1 against the oracle
    om = oracle.OracleModel(cfg)
    om.load(w)
    del w
    oids, olg = om.generate(prompts[0], steps, want_logits=True)
    om.close()
    n = agreement(oids, b1[0], olg, b1[1])
    say("7B widths batch 1: ids equal for", n, "of", len(oids), "steps")
    assert n == len(oids) == steps
    for t in range(n):
        assert np.max(np.abs(b1[1][t] - olg[t])) <= 2e-2 and rel_l2(b1[1][t], olg[t]) <= 1e-3, t
