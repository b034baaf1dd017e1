"""GPU decoder parity against the oracle's decode loop.

Bars: greedy ids equal; per-step raw logits within 2e-2 max-abs and 1e-3
relative L2. The tiny configurations with f32 KV are held to a much tighter 1e-4
relative bound so that indexing mistakes cannot hide inside the tolerance.
With an fp16 KV cache the device sees rounded K/V rows that the f32 oracle does not;
greedy ids are then required to agree wherever the oracle's top-2 logit margin exceeds
ten times the measured logit error (a smaller margin is a numerical tie)."""
import numpy as np
import pytest

import oracle
from bramha_amd import BH_F32, BH_Q4_G32, BH_Q8_ROW
from bramha_amd.model import QWEN2_0_5B, DecoderConfig, HipDecoder, synth_tokens, synth_weights
from tinymodels import F32, Q4_G32, Q4_ROW, Q8_ROW, prompt, rel_l2, tiny_cfg, tiny_weights

pytestmark = pytest.mark.gpu


def _pair(plane, cfg, seed=0):
    w, _ = tiny_weights(cfg, seed)
    om = oracle.OracleModel(cfg)
    om.load(w)
    gm = HipDecoder(plane, cfg)
    gm.load(w)
    return om, gm


def penalized(raw, gen):
    """The step's logits after the reference's repetition penalty over the ids generated before
    it (cpu_engine.rs:2984-2992): each occurrence divides a positive logit by 1.15 or multiplies
    a negative one."""
    lg = np.array(raw, np.float32, copy=True)
    for g in gen:
        lg[g] = lg[g] / np.float32(1.15) if lg[g] > 0 else lg[g] * np.float32(1.15)
    return lg


def agreement(oids, gids, olg, glg):
    """Number of leading steps whose greedy ids agree. Where they first differ, the choice must
    be a numerical tie: the oracle's top-2 margin over the PENALIZED logits (what the argmax
    sees) at most ten times that step's largest logit difference."""
    n = min(len(oids), len(gids))
    for t in range(n):
        if oids[t] != gids[t]:
            top2 = np.sort(penalized(olg[t], oids[:t]))[-2:]
            err = np.abs(olg[t] - glg[t]).max()
            assert top2[1] - top2[0] <= 10 * err, (t, top2, err)
            print("numerical tie at step", t, "margin", top2[1] - top2[0], "logit error", err, flush=True)
            return t
    return n


@pytest.mark.parametrize("wfmt,head_fmt,gqa7", [
    (F32, F32, False), (Q8_ROW, F32, False), (Q4_ROW, F32, True), (Q4_G32, Q4_G32, True), (Q8_ROW, Q4_G32, True)])
def test_tiny_generate_parity(plane, wfmt, head_fmt, gqa7):
    cfg = tiny_cfg(wfmt, head_fmt, gqa7=gqa7)
    om, gm = _pair(plane, cfg, seed=wfmt)
    p = prompt(9, cfg.vocab, seed=11)
    oids, olg = om.generate(p, 16, want_logits=True)
    gids, glg = gm.generate(p, 16, want_logits=True)
    assert np.array_equal(oids, gids)
    assert np.max(np.abs(olg - glg)) <= 1e-4 * max(1.0, np.abs(olg).max())


def test_tiny_long_prompt_crosses_prefill_chunks(plane):
    cfg = tiny_cfg(Q8_ROW, F32, gqa7=True)
    om, gm = _pair(plane, cfg, seed=3)
    p = prompt(70, cfg.vocab, seed=4)  # 69 prefill tokens: 64 + 5
    oids, olg = om.generate(p, 8, want_logits=True)
    gids, glg = gm.generate(p, 8, want_logits=True)
    assert np.array_equal(oids, gids)
    assert np.max(np.abs(olg - glg)) <= 1e-4 * max(1.0, np.abs(olg).max())


@pytest.mark.parametrize("plen", [70, 41, 12])
@pytest.mark.parametrize("wfmt", [Q4_G32, Q4_ROW])
def test_tiny_4bit_prefill_mfma(plane, wfmt, plen):
    # 69 prefill tokens: a 64-token tiled MFMA chunk, then a 5-token VALU pass; 40 and 11 tokens:
    # one tiled MFMA launch per projection over a partial token tile
    cfg = tiny_cfg(wfmt, Q4_G32 if wfmt == Q4_G32 else F32, gqa7=True)
    om, gm = _pair(plane, cfg, seed=21)
    p = prompt(plen, cfg.vocab, seed=22)
    oids, olg = om.generate(p, 8, want_logits=True)
    gids, glg = gm.generate(p, 8, want_logits=True)
    assert np.array_equal(oids, gids)
    assert np.max(np.abs(olg - glg)) <= 1e-4 * max(1.0, np.abs(olg).max())


def test_batch20_decode_mfma(plane):
    # 20 sequences decoded together: MFMA pass of 16 + VALU pass of 4 in every projection
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, max_seqs=20, kv_rows=20 * 64)
    om, gm = _pair(plane, cfg, seed=23)
    prompts = [prompt(3 + (s * 7) % 30, cfg.vocab, seed=100 + s) for s in range(20)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, 64)
        gm.prefill(s, p[:-1])
    gm.decode_setup(list(range(20)), [p[-1] for p in prompts])
    ids, lg = gm.decode(6, want_logits=True)
    for s, p in enumerate(prompts):
        want, wl = om.generate(p, 6, want_logits=True)
        n = len(want)
        assert np.array_equal(ids[:n, s], want), s
        assert np.max(np.abs(lg[:n, s] - wl)) <= 1e-4 * max(1.0, np.abs(wl).max()), s


@pytest.mark.parametrize("nseq", [16, 32])
def test_batch_decode_large_vocab(plane, nseq):
    # a 40000-id vocabulary: the LM head's MFMA pass has 626 row tiles (the 4-wave variant that
    # requests the penalty counts at kernel start), every step's ids and logits as the oracle's
    cfg = tiny_cfg(Q4_G32, Q4_G32, max_seqs=nseq, kv_rows=nseq * 64, vocab=40000)
    om, gm = _pair(plane, cfg, seed=29)
    prompts = [prompt(3 + (s * 5) % 20, cfg.vocab, seed=200 + s) for s in range(nseq)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, 64)
        gm.prefill(s, p[:-1])
    gm.decode_setup(list(range(nseq)), [p[-1] for p in prompts])
    ids, lg = gm.decode(6, want_logits=True)
    for s, p in enumerate(prompts):
        want, wl = om.generate(p, 6, want_logits=True)
        n = len(want)
        assert np.array_equal(ids[:n, s], want), s
        assert np.max(np.abs(lg[:n, s] - wl)) <= 1e-4 * max(1.0, np.abs(wl).max()), s


def test_batch32_token_groups_with_k_split(plane):
    """32 sequences decoded together: every 32-token MFMA pass runs as two 16-token workgroup
    groups; the down projection (FFN 2048: 64 chunks of K) also splits K over 4 workgroups per
    row tile, each group with its own partial-sum and arrival-counter region. An O bias takes the
    batched residual epilogue's prefetched bias."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, ffn=2048, max_seqs=32, kv_rows=32 * 64, o_bias=True)
    om, gm = _pair(plane, cfg, seed=51)
    prompts = [prompt(2 + (s * 3) % 17, cfg.vocab, seed=300 + s) for s in range(32)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, 64)
        gm.prefill(s, p[:-1])
    gm.decode_setup(list(range(32)), [p[-1] for p in prompts])
    ids, lg = gm.decode(6, want_logits=True)
    for s, p in enumerate(prompts):
        want, wl = om.generate(p, 6, want_logits=True)
        n = len(want)
        assert np.array_equal(ids[:n, s], want), s
        assert np.max(np.abs(lg[:n, s] - wl)) <= 1e-4 * max(1.0, np.abs(wl).max()), s


def test_batch32_fp16_kv_ragged_regions_vs_oracle(plane):
    """The batch-32 headline path at model level, against the oracle per sequence: an fp16 KV
    cache written in MFMA tiles by the QKV epilogue of the 32-token MFMA passes (two 16-token
    workgroup groups), attention through the MFMA kernel with the entries' region offsets as
    launch arguments, over slot regions of unequal capacity (offsets 64, 128 and 192 rows
    apart), prompts of 2 to 150 tokens (prefills through the tiled MFMA GEMM past 64 tokens)."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True, ffn=2048, max_seqs=32, kv_rows=32 * 320)
    om, gm = _pair(plane, cfg, seed=53)
    prompts = [prompt(2 + (s * 37) % 149, cfg.vocab, seed=400 + s) for s in range(32)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, len(p) + 8 + 64 * (s % 3))
        gm.prefill(s, p[:-1])
    gm.decode_setup(list(range(32)), [p[-1] for p in prompts])
    steps = 8
    ids, lg = gm.decode(steps, want_logits=True)
    assert np.isfinite(lg).all()
    ties = 0
    for s, p in enumerate(prompts):
        want, wl = om.generate(p, steps, want_logits=True)
        n = agreement(want, ids[:, s], wl, lg[:, s])
        ties += n < len(want)
        assert np.max(np.abs(lg[:n, s] - wl[:n])) < 2e-2, s
        assert max(rel_l2(lg[t, s], wl[t]) for t in range(n)) < 1e-3, s
    assert ties <= 2


def test_tiny_sink_eviction(plane):
    cfg = tiny_cfg(F32, F32, max_context=16, sink_tokens=4)
    om, gm = _pair(plane, cfg, seed=5)
    p = prompt(6, cfg.vocab, seed=6)
    oids, olg = om.generate(p, 30, want_logits=True)  # rows pass 16 at step 11
    gids, glg = gm.generate(p, 30, want_logits=True)
    assert np.array_equal(oids, gids)
    assert np.max(np.abs(olg - glg)) <= 1e-4 * max(1.0, np.abs(olg).max())


def test_batch16_fp16_kv_sink_eviction(plane):
    """Sixteen sequences decoded together past a 16-row context with 4 sink rows: the KV rows of
    the 16-token MFMA passes' QKV epilogue land in the ring (positions 4 + (p - 4) % 12), and the
    batched attention reads each sequence's ring, against the oracle's eviction per sequence.
    Prompts of 3 to 12 tokens (the reference's prefill stays below the limit), 24 steps."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True, max_context=16, sink_tokens=4, max_seqs=16,
                   kv_rows=16 * 64)
    om, gm = _pair(plane, cfg, seed=71)
    prompts = [prompt(3 + (s * 5) % 10, cfg.vocab, seed=500 + s) for s in range(16)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, 64)
        gm.prefill(s, p[:-1])
    steps = 24
    gm.decode_setup(list(range(16)), [int(p[-1]) for p in prompts])
    ids, lg = gm.decode(steps, want_logits=True)
    assert np.isfinite(lg).all()
    for s, p in enumerate(prompts):
        oids, olg = om.generate(p, steps, want_logits=True)
        n = agreement(oids, ids[:, s], olg, lg[:, s])
        assert n >= 12, (s, n)  # well past the first eviction (step 16 - len(p) + 1 at most)
        assert np.max(np.abs(olg[:n] - lg[:n, s])) < 2e-2, s
        assert max(rel_l2(lg[t, s], olg[t]) for t in range(n)) < 1e-3, s


def test_tiny_fp16_kv_sink_eviction_o_bias(plane):
    """Batch-1 decode over an fp16 cache (attention, O projection and residual add in one
    launch) with sink eviction (a 16-row ring after 4 sink rows) and an O bias."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True, max_context=16, sink_tokens=4, o_bias=True)
    om, gm = _pair(plane, cfg, seed=45)
    p = prompt(6, cfg.vocab, seed=46)
    oids, olg = om.generate(p, 30, want_logits=True)  # rows pass 16 at step 11
    gids, glg = gm.generate(p, 30, want_logits=True)
    n = agreement(oids, gids, olg, glg)
    assert n == len(oids) == 30
    assert np.max(np.abs(olg[:n] - glg[:n])) < 2e-2 and max(rel_l2(glg[t], olg[t]) for t in range(n)) < 1e-3


def test_tiny_fp16_kv(plane):
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True)
    om, gm = _pair(plane, cfg, seed=7)
    p = prompt(12, cfg.vocab, seed=8)
    oids, olg = om.generate(p, 16, want_logits=True)
    gids, glg = gm.generate(p, 16, want_logits=True)
    n = agreement(oids, gids, olg, glg)
    assert n == len(oids) == 16
    assert np.max(np.abs(olg[:n] - glg[:n])) < 2e-2 and max(rel_l2(glg[t], olg[t]) for t in range(n)) < 1e-3


@pytest.mark.parametrize("hd128", [False, True])
@pytest.mark.parametrize("batch", [1, 2])
def test_fp16_kv_rows_past_the_length_are_never_used(plane, hd128, batch):
    """Every row of the slots' KV regions is NaN before the prefill, and the rows past each
    sequence's length stay NaN until the decode writes them. The prefill attention, the batch-1
    attention + O launch and the batched decode attention load whole KV tiles, rows past the
    length included: the logits must equal, bit for bit, those of the same model over a
    zero-filled cache (and agree with the oracle). Prompts of 45 and 29 rows and 21 decode steps
    end inside tiles."""
    if hd128:
        cfg = tiny_cfg(Q4_G32, Q4_G32, kv_f16=True, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=768)
    else:
        cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True)
    w, _ = tiny_weights(cfg, 61 + hd128)
    om = oracle.OracleModel(cfg)
    om.load(w)
    prompts = [prompt(45, cfg.vocab, seed=62), prompt(29, cfg.vocab, seed=63)][:batch]
    steps, cap = 21, 128
    runs = []
    for fill in (np.nan, 0.0):
        gm = HipDecoder(plane, cfg)
        gm.load(w)
        rows = np.full((cfg.n_layers, cap, cfg.kv_dim), fill, np.float32)
        for s in range(batch):
            gm.seq_open(s, cap)
            gm.kv_write(s, 0, rows, rows)
            assert gm.seq_len(s) == cap
            gm.seq_open(s, cap)  # the same region, length 0
            gm.prefill(s, prompts[s][:-1])
        gm.decode_setup(list(range(batch)), [int(p[-1]) for p in prompts])
        runs.append(gm.decode(steps, want_logits=True))
        gm.close()
    (gids, glg), (zids, zlg) = runs
    assert np.all(np.isfinite(glg))
    assert np.array_equal(gids, zids) and np.array_equal(glg.view(np.uint32), zlg.view(np.uint32))
    for s in range(batch):
        oids, olg = om.generate(prompts[s], steps, want_logits=True)
        n = agreement(oids, gids[:, s], olg, glg[:, s])
        assert n >= 8, (s, n)
        assert np.max(np.abs(olg[:n] - glg[:n, s])) < 2e-2
        assert max(rel_l2(glg[t, s], olg[t]) for t in range(n)) < 1e-3


@pytest.mark.parametrize("hd128", [False, True])
def test_tiny_prefill_tiled_fp16_kv(plane, hd128):
    """A 199-token prefill chunk: tiled MFMA projections over all tokens (QKV with RoPE and KV
    append, O and down with the residual add, gate/up with SiLU) and the causal prefill
    attention over the fp16 cache; then decode. head_dim 128 also takes the two-group QKV
    tiles and the 128-wide attention of the decode steps."""
    if hd128:
        cfg = tiny_cfg(Q4_G32, Q4_G32, kv_f16=True, max_tokens=256, hidden=512, n_heads=4, n_kv_heads=2,
                       head_dim=128, ffn=768)
    else:
        cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True, max_tokens=256)
    om, gm = _pair(plane, cfg, seed=31 + hd128)
    p = prompt(200, cfg.vocab, seed=32)
    oids, olg = om.generate(p, 12, want_logits=True)
    gids, glg = gm.generate(p, 12, want_logits=True)
    n = agreement(oids, gids, olg, glg)
    assert n == len(oids) == 12
    assert np.max(np.abs(olg[:n] - glg[:n])) < 2e-2 and max(rel_l2(glg[t], olg[t]) for t in range(n)) < 1e-3


@pytest.mark.parametrize("hd128,plen", [(False, 800), (True, 420)])
def test_tiny_long_prompt_attention_runs(plane, hd128, plen):
    """Prompts long enough that each wave of the causal prefill attention walks three or more
    whole KV tiles (the run whose next tile is requested unconditionally), prefilled in 256-token
    chunks, then decode steps over the same rows: against the oracle."""
    if hd128:
        cfg = tiny_cfg(Q4_G32, Q4_G32, kv_f16=True, max_tokens=256, hidden=512, n_heads=4, n_kv_heads=2,
                       head_dim=128, ffn=768)
    else:
        cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True, max_tokens=256)
    om, gm = _pair(plane, cfg, seed=81 + hd128)
    p = prompt(plen, cfg.vocab, seed=82)
    oids, olg = om.generate(p, 8, want_logits=True)
    gids, glg = gm.generate(p, 8, want_logits=True)
    assert np.all(np.isfinite(glg))
    n = agreement(oids, gids, olg, glg)
    assert n >= 4, n
    assert np.max(np.abs(olg[:n] - glg[:n])) < 2e-2 and max(rel_l2(glg[t], olg[t]) for t in range(n)) < 1e-3


def test_tiny_untied_lm_head(plane):
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, tied=False)
    om, gm = _pair(plane, cfg, seed=41)
    p = prompt(9, cfg.vocab, seed=42)
    oids, olg = om.generate(p, 12, want_logits=True)
    gids, glg = gm.generate(p, 12, want_logits=True)
    assert np.array_equal(oids, gids)
    assert np.max(np.abs(olg - glg)) <= 1e-4 * max(1.0, np.abs(olg).max())


def test_ragged_batch_and_refill(plane):
    cfg = tiny_cfg(Q8_ROW, F32, gqa7=True, max_seqs=6)
    om, gm = _pair(plane, cfg, seed=9)
    prompts = [prompt(n, cfg.vocab, seed=20 + n) for n in (3, 9, 17, 40)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, 64)
        gm.prefill(s, p[:-1])
    gm.decode_setup([0, 1, 2, 3], [p[-1] for p in prompts])
    ids_a = gm.decode(6)
    # refill entry 2 with a new sequence in slot 5, keep decoding everyone
    newp = prompt(11, cfg.vocab, seed=99)
    gm.seq_open(5, 64)
    gm.prefill(5, newp[:-1])
    gm.decode_replace(2, 5, newp[-1])
    ids_b = gm.decode(6)
    for b, p in enumerate(prompts):
        want = om.generate(p, 12 if b != 2 else 6)
        got = np.concatenate([ids_a[:, b], ids_b[:, b]]) if b != 2 else ids_a[:, b]
        n = len(want)  # the oracle stops at an EOS id; the batch keeps decoding
        assert np.array_equal(got[:n], want), b
    want = om.generate(newp, 6)
    assert np.array_equal(ids_b[:len(want), 2], want)


@pytest.mark.parametrize("kv_f16", [False, True])
def test_refill_reopening_the_finished_slot(plane, kv_f16):
    """A finished entry's own slot reopened for a new sequence (same region, so the captured decode
    step with its static region offsets stays valid) and swapped in with decode_replace; decoding
    without replacing it first is refused. Every sequence against the oracle."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, max_seqs=4, kv_f16=kv_f16, kv_rows=4 * 128)
    om, gm = _pair(plane, cfg, seed=17)
    prompts = [prompt(n, cfg.vocab, seed=30 + n) for n in (5, 12, 30)]
    for s, p in enumerate(prompts):
        gm.seq_open(s, 96)
        gm.prefill(s, p[:-1])
    gm.decode_setup([0, 1, 2], [p[-1] for p in prompts])
    ids_a, lg_a = gm.decode(6, want_logits=True)
    newp = prompt(20, cfg.vocab, seed=99)
    gm.seq_open(1, 96)  # entry 1's slot, same capacity: same region
    with pytest.raises(Exception):
        gm.decode(1)
    gm.prefill(1, newp[:-1])
    gm.decode_replace(1, 1, newp[-1])
    ids_b, lg_b = gm.decode(8, want_logits=True)
    for b, p in enumerate(prompts):
        n_steps = 14 if b != 1 else 6
        want, wl = om.generate(p, n_steps, want_logits=True)
        got = np.concatenate([ids_a[:, b], ids_b[:, b]])[:n_steps] if b != 1 else ids_a[:, b]
        glg = np.concatenate([lg_a[:, b], lg_b[:, b]])[:n_steps] if b != 1 else lg_a[:, b]
        n = agreement(want, got[:len(want)], wl, glg[:len(want)])
        assert n == len(want), b
    want, wl = om.generate(newp, 8, want_logits=True)
    n = agreement(want, ids_b[:len(want), 1], wl, lg_b[:len(want), 1])
    assert n == len(want)
    assert np.max(np.abs(lg_b[:n, 1] - wl[:n])) < 2e-2


def test_graph_replay_matches_single_steps(plane):
    cfg = tiny_cfg(Q4_G32, Q4_G32)
    _, gm = _pair(plane, cfg, seed=12)
    p = prompt(5, cfg.vocab, seed=13)
    for slot in (0, 1):
        gm.seq_open(slot, 64)
        gm.prefill(slot, p[:-1])
    gm.decode_setup([0], [p[-1]])
    a, la = gm.decode(8, want_logits=True)
    gm.decode_setup([1], [p[-1]])
    parts = [gm.decode(1, want_logits=True) for _ in range(8)]
    b = np.concatenate([x[0] for x in parts])
    lb = np.concatenate([x[1] for x in parts])
    assert np.array_equal(a, b) and np.array_equal(la, lb)


@pytest.mark.parametrize("shape,plen", [("gqa7", 20), ("gqa7", 100), ("gqa7", 300), ("hd128", 40), ("hd128", 200),
                                        ("g1", 40), ("g4", 100), ("g8", 40)])
def test_batch1_attention_o_launch_matches_batched_path(plane, shape, plen):
    """Batch-1 decode over an fp16 cache computes attention, the O projection and the residual
    add in one launch; a batch of two runs them as separate kernels. The same prompt decoded
    both ways gives the same ids and logits to 1e-4 (the launches differ only in summation
    order). Context bounds of 64, 128 and 512 rows (one tile per attention wave at 1, 2 and 8
    waves per KV head); head_dim 128 with two KV heads at bounds of 64 (2 waves of one tile)
    and 256 rows (4 waves of two tiles); 1, 4 and 8 query heads per KV head."""
    if shape == "hd128":
        cfg = tiny_cfg(Q4_G32, Q4_G32, kv_f16=True, hidden=512, n_heads=4, n_kv_heads=2, head_dim=128, ffn=768)
    elif shape in ("g1", "g4", "g8"):
        heads = {"g1": (4, 4), "g4": (4, 1), "g8": (8, 1)}[shape]
        cfg = tiny_cfg(Q4_G32, Q4_G32, kv_f16=True, hidden=64 * heads[0], n_heads=heads[0], n_kv_heads=heads[1],
                       head_dim=64, ffn=512, vocab=1024)
    else:
        cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, kv_f16=True)
    _, gm = _pair(plane, cfg, seed=41)
    p = prompt(plen, cfg.vocab, seed=42)
    q = prompt(plen // 2 + 3, cfg.vocab, seed=43)
    for slot, pp in ((0, p), (1, p), (2, q)):
        gm.seq_open(slot, (plen + 64) // 64 * 64 + 64)
        gm.prefill(slot, pp[:-1])
    gm.decode_setup([0], [p[-1]])
    a, la = gm.decode(8, want_logits=True)
    gm.decode_setup([1, 2], [p[-1], q[-1]])
    b, lb = gm.decode(8, want_logits=True)
    assert np.array_equal(a[:, 0], b[:, 0])
    assert np.max(np.abs(la[:, 0] - lb[:, 0])) <= 1e-4 * max(1.0, np.abs(lb[:, 0]).max())


def _full_model(cfg, seed):
    return list(synth_weights(cfg, seed=seed))


@pytest.mark.timeout(900)
def test_qwen2_0_5b_reference_format_64_tokens(plane):
    """The reference-format workload: Qwen2-0.5B shape, int8 per-row projections, f32 tied
    embedding / LM head, f32 KV, 32 seeded prompt ids, 64 greedy steps."""
    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q8_ROW, head_fmt=BH_F32, kv_f16=False, max_seqs=1, kv_rows=256,
                        max_tokens=64)
    w = _full_model(cfg, seed=0)
    p = synth_tokens(0, "prompt", 32, cfg.vocab)
    print("weights ready", flush=True)
    gm = HipDecoder(plane, cfg)
    gm.load(w)
    gids, glg = gm.generate(p, 64, want_logits=True)
    print("gpu done", flush=True)
    om = oracle.OracleModel(cfg)
    om.load(w)
    del w
    oids, olg = om.generate(p, 64, want_logits=True)
    print("oracle done", len(oids), flush=True)
    assert np.array_equal(gids, oids)
    for t in range(len(oids)):
        assert np.max(np.abs(glg[t] - olg[t])) <= 2e-2, t
        assert rel_l2(glg[t], olg[t]) <= 1e-3, t


@pytest.mark.timeout(900)
def test_qwen2_0_5b_4bit_parity(plane):
    """The 4-bit throughput workload's model (Q4 g32 projections and tied head, fp16 KV)."""
    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=1, kv_rows=256,
                        max_tokens=64)
    w = _full_model(cfg, seed=1)
    p = synth_tokens(1, "prompt", 32, cfg.vocab)
    gm = HipDecoder(plane, cfg)
    gm.load(w)
    gids, glg = gm.generate(p, 64, want_logits=True)
    om = oracle.OracleModel(cfg)
    om.load(w)
    del w
    oids, olg = om.generate(p, 64, want_logits=True)
    n = agreement(oids, gids, olg, glg)
    print("greedy ids equal for", n, "of", len(oids), "steps", flush=True)
    assert n == len(oids) == 64
    for t in range(n):
        assert np.max(np.abs(glg[t] - olg[t])) <= 2e-2, t
        assert rel_l2(glg[t], olg[t]) <= 1e-3, t


@pytest.mark.parametrize("temperature,top_k", [(0.8, 40), (1.5, 5)])
def test_device_sampling_matches_reference_rule(plane, temperature, top_k):
    """Top-k temperature sampling on the device: at every step the chosen id is the oracle's
    choice (the reference rule, cpu_engine.rs:2998-3022) over the same step's penalized logits
    and the same draw r = bh_sample_uniform(seed, slot, position); steps whose r lies within
    1e-5 of a cumulative boundary are numerical ties and not compared."""
    from bramha_amd import _lib

    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True)
    _, gm = _pair(plane, cfg, seed=71)
    seed = 1234
    gm.set_sampling(temperature, top_k, seed)
    p = prompt(7, cfg.vocab, seed=72)
    ids, lg = gm.generate(p, 24, want_logits=True)
    assert len(ids) >= 1
    gen = []
    checked = 0
    for t in range(len(ids)):
        pen = lg[t].copy()
        for g in gen:
            pen[g] = pen[g] / 1.15 if pen[g] > 0 else pen[g] * 1.15
        r = _lib.lib.bh_sample_uniform(seed, 0, len(p) - 1 + t)
        want = oracle.sample_topk(pen, temperature, top_k, r)
        near = any(abs(oracle.sample_topk(pen, temperature, top_k, r + d) - want) > 0 for d in (-1e-5, 1e-5))
        if not near:
            assert ids[t] == want, (t, ids[t], want, r)
            checked += 1
        gen.append(int(ids[t]))
    assert checked >= len(ids) - 2
    # back to greedy: the default decode again
    gm.set_sampling(0.0)
    g1 = gm.generate(p, 8)
    om, _ = _pair(plane, cfg, seed=71)
    assert np.array_equal(g1, om.generate(p, 8))


@pytest.mark.parametrize("kv_f16,max_tokens", [(False, 64), (True, 64), (True, 48), (False, 16)])
def test_batch_prefill_vs_oracle(plane, kv_f16, max_tokens):
    """Several prompts prefilled in one pass (bh_model_prefill_batch: with an fp16 cache every
    sequence padded to whole 16-row groups with pad rows that write no KV row; chunks of at most
    max_tokens rows cutting through sequences), then decoded together: every sequence's ids and
    logits as the oracle's own prefill + decode of it (f32 cache: the 1e-4 bar; fp16 cache: the
    fp16 bars with the tie rule). Prompt lengths 1 (nothing to prefill), 6, 21, 40 and 17."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, gqa7=True, max_seqs=5, kv_rows=5 * 128, kv_f16=kv_f16, max_tokens=max_tokens)
    om, gm = _pair(plane, cfg, seed=61)
    lens = [1, 6, 21, 40, 17]
    prompts = [prompt(n, cfg.vocab, seed=400 + s) for s, n in enumerate(lens)]
    slots = [3, 0, 4, 1, 2]
    for s in slots:
        gm.seq_open(s, 128)
    gm.prefill_batch(slots, [p[:-1] for p in prompts])
    gm.decode_setup(slots, [p[-1] for p in prompts])
    ids, lg = gm.decode(8, want_logits=True)
    for b, p in enumerate(prompts):
        want, wl = om.generate(p, 8, want_logits=True)
        n = len(want)
        if not kv_f16:
            assert np.array_equal(ids[:n, b], want), b
            assert np.max(np.abs(lg[:n, b] - wl)) <= 1e-4 * max(1.0, np.abs(wl).max()), b
        else:
            k = agreement(want, list(ids[:n, b]), wl, lg[:n, b])
            assert k == n, b
            assert np.max(np.abs(wl[:k] - lg[:k, b])) < 2e-2 and max(rel_l2(lg[t, b], wl[t]) for t in range(k)) < 1e-3, b


def test_batch_prefill_errors(plane):
    """A slot twice in one batch, a closed slot and a prompt past the slot's capacity are refused
    with nothing prefilled; an empty batch is a no-op."""
    cfg = tiny_cfg(Q4_G32, Q4_G32, max_seqs=3, kv_rows=3 * 64)
    _, gm = _pair(plane, cfg, seed=3)
    gm.seq_open(0, 32)
    gm.seq_open(1, 32)
    from bramha_amd._lib import BhError
    for slots, toks in (([0, 0], [[1, 2], [3]]), ([0, 2], [[1], [2]]), ([1], [list(range(40))])):
        with pytest.raises(BhError):
            gm.prefill_batch(slots, toks)
    assert gm.seq_len(0) == 0 and gm.seq_len(1) == 0
    gm.prefill_batch([], [])
