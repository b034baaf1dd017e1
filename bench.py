#!/usr/bin/env python3
"""Decode throughput of the Qwen2-0.5B-shaped 4-bit model on one MI355X.

Workload: 24 layers, hidden 896, 14/2 heads of 64, FFN 4864, vocab 151936, tied
embedding; projections and LM head 4-bit with one fp16 scale per 32 weights, weights
N(0, 0.02) from a seeded generator, norms 1.0, q/k/v biases N(0, 0.02), fp16 KV cache,
RoPE theta 1e6. Each sequence gets a 32-token random prompt (prefilled), then greedy
decode steps (embedding, 24 layers, LM head, repetition penalty, argmax) are replayed
from a HIP graph. `value` is decode tokens/s at batch 1; the same line carries batch 32.

A step is one decode step of the batch (one token per sequence). Inputs and weights are
resident in HBM before the timed region. Defaults: 8 warm-up steps, then 64 timed steps (the
64 greedy tokens after a 32-token prompt of the reference's CPU run).

The same line also carries the other workloads, each with its own roofline: the HBM read and
copy ceilings measured on this GPU, the isolated 4-bit GEMV sweep (the Qwen2-0.5B projection
shapes and the Qwen2-7B ones), the GQA decode attention sweep, the ragged 32-sequence decode
with refills, the Qwen2-7B prefill + decode at batch 1 and 16, and the CPU baseline.
"""
import argparse
import json
import os
import sys
import time

METRIC = "decode tok/s @ bs1 & bs32 (Qwen2-0.5B, 4-bit); achieved HBM GB/s vs peak"
HBM_PEAK = 8.0e12


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def build_model(plane, batch, prompt_len, steps_total, seed=0):
    import numpy as np

    from bramha_amd import BH_Q4_G32
    from bramha_amd.model import QWEN2_0_5B, DecoderConfig, HipDecoder, synth_tokens, synth_weights

    cap = prompt_len + steps_total + 8
    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=batch,
                        kv_rows=cap * batch, max_tokens=max(64, batch))
    m = HipDecoder(plane, cfg)
    m.load(synth_weights(cfg, seed=seed))
    firsts = []
    for s in range(batch):
        p = synth_tokens(seed, "prompt.%d" % s, prompt_len, cfg.vocab)
        m.seq_open(s, cap)
        m.prefill(s, p[:-1])
        firsts.append(int(p[-1]))
    m.decode_setup(np.arange(batch, dtype=np.int32), np.array(firsts, np.uint32))
    return m, cfg


def timed_decode(m, steps, warmup):
    from bramha_amd import ops

    m.decode(warmup)
    ops.synchronize(m.plane)
    t0 = time.perf_counter()
    m.decode(steps)
    ops.synchronize(m.plane)
    return time.perf_counter() - t0


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def pmc_traffic(kclass, batch):
    """HBM bytes per launch of a kernel class at this batch, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary of that batch (scaled by its copy probe); None when not
    measured."""
    path = os.path.join(PROFILES, "pmc_traffic_decode_qwen2_0.5b_q4g32_bs%d.md" % batch)
    try:
        for line in open(path):
            if line.startswith("traffic:"):
                vals = dict(kv.split("=") for kv in line.split()[1:])
                return float(vals[kclass]) if kclass in vals else None
    except OSError:
        return None
    return None


def launch_floor(plane, n=896, iters=200):
    """Time per launch of a graph-replayed chain of dependent kernels whose workgroups each read
    the n floats the previous launch wrote (bh_time_probe's chain mode): the floor under every
    dependent kernel of the decode step, at 14, 36 and 256 workgroups."""
    from bramha_amd import ops

    out = {}
    for wgs in (14, 36, 256):
        out[str(wgs)] = round(ops.time_probe(plane, 2, n * 4, wgs, 4, iters=iters), 3)
    log("dependent-launch floor (us per launch at 14 / 36 / 256 workgroups): %s" % out)
    return out


def grid_barrier(plane, iters=20):
    """Time per phase of a persistent grid of 14 to 256 resident workgroups whose phases (the
    chain link's work) are separated by a grid-wide barrier with release/acquire ordering
    (bh_time_probe mode 3): what fusing the decode step's dependent launches into one persistent
    kernel would pay per boundary instead of the dependent-launch floor."""
    from bramha_amd import ops

    out = {}
    for wgs in (14, 36, 112, 256):
        out[str(wgs)] = round(ops.time_probe(plane, 3, 4096, wgs, 4, iters=iters), 3)
    log("grid barrier (us per phase at 14 / 36 / 112 / 256 resident workgroups): %s" % out)
    return out


def above_floor(roof, floor):
    """Per kernel class: mean launch time minus the dependent-launch floor, and the step's
    launch count times that floor (the floor of the 256-workgroup chain, the largest of the
    three)."""
    f = max(floor.values())
    cls = {k: round(v - f, 3) for k, v in roof["per_class_us"].items() if roof["launches_per_step"].get(k)}
    n = sum(roof["launches_per_step"].values())
    tot = sum(roof["per_class_us"][k] * c for k, c in roof["launches_per_step"].items())
    return {"floor_us": f, "chain_us_by_workgroups": floor, "above_floor_us": cls, "launches_per_step": n,
            "step_kernel_us": round(tot, 1), "step_floor_us": round(n * f, 1), "step_above_floor_us": round(tot - n * f, 1)}


def roofline(m, n_steps=16, batch=1):
    """Per-kernel-class mean launch durations over eager decode steps (HIP events on the
    model's stream) and the algorithmic bytes of one launch; the dominant class is the one
    with the largest total time per step."""
    t = m.time_kernels(n_steps)
    best, best_tot = None, -1.0
    for k, (mean_us, cnt) in t.items():
        tot = mean_us * cnt / n_steps
        if k != "other" and tot > best_tot:
            best, best_tot = k, tot
    mean_us = t[best][0]
    nbytes = m.kernel_bytes(best)
    achieved = nbytes / (mean_us * 1e-6)
    # the step's weight-streaming launch (the LM head), measured the same way, for comparison
    lm_us = t["lm_head"][0]
    lm_bytes = m.kernel_bytes("lm_head")
    stream = {"kernel": "lm_head", "mean_us": lm_us, "bytes_per_launch": lm_bytes,
              "achieved": lm_bytes / (lm_us * 1e-6) / 1e9 if lm_us else None,
              "frac": lm_bytes / (lm_us * 1e-6) / HBM_PEAK if lm_us else None}
    return best, {"bound": "hbm", "achieved": achieved / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                  "frac": achieved / HBM_PEAK, "traffic": pmc_traffic(best, batch), "kernel": best,
                  "bytes_per_launch": nbytes,
                  "mean_us": mean_us,
                  "weight_stream": stream,
                  "per_class_us": {k: round(v[0], 3) for k, v in t.items()},
                  "launches_per_step": {k: v[1] // n_steps for k, v in t.items()}}


# (out_features, in_features) of the Qwen2-0.5B projections: q/o, k/v, gate/up, down, LM head;
# then the Qwen2-7B ones: q/o, k/v, gate/up, down, LM head.
GEMV_SHAPES = ((896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896))
GEMV_BATCHES = (1, 4, 16, 32)
GEMV_SHAPES_7B = ((3584, 3584), (512, 3584), (18944, 3584), (3584, 18944), (152064, 3584))
GEMV_BATCHES_7B = (1, 16)


def gemv_sweep(plane, rotate=1 << 30, iters=64, shapes=GEMV_SHAPES, batches=GEMV_BATCHES):
    """Isolated 4-bit GEMV/GEMM: one fp16 scale per 32 weights, weights N(0, 0.02) before
    quantization, activations N(0, 1). Each launch streams its weight from HBM (graph of
    launches rotating over >= 1 GiB of weight copies). Bytes = packed nibbles + scales +
    activations in + outputs."""
    import numpy as np

    from bramha_amd import BH_Q4_G32, ops
    from bramha_amd.model import quantize, synth_normal

    out = []
    for n, k in shapes:
        w = synth_normal(0, "sweep.%dx%d" % (n, k), n * k, 0.02).reshape(n, k)
        q, sc = quantize(BH_Q4_G32, w)
        del w
        dw = ops.DeviceWeight(plane, BH_Q4_G32, n, k, q, sc)
        for b in batches:
            x = ops.DeviceArray.from_numpy(plane, synth_normal(0, "sweep.x", b * k, 1.0).reshape(b, k))
            y = ops.DeviceArray(plane, (b, n), np.float32)
            us = dw.time_gemv(x, y, iters=iters, rotate_bytes=rotate)
            nbytes = n * k * 0.5 + n * k / 32 * 2 + b * k * 4 + b * n * 4
            r = {"n": n, "k": k, "batch": b, "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
                 "hbm_frac": round(nbytes / (us * 1e-6) / HBM_PEAK, 4),
                 "TFLOPs": round(2.0 * n * k * b / us / 1e6, 2)}
            log("gemv %6dx%-5d B=%-2d %8.2f us %7.1f GB/s (%.1f%% HBM)" %
                (n, k, b, us, r["GBps"], 100 * r["hbm_frac"]))
            out.append(r)
            x.free()
            y.free()
        dw.free()
    return out


def hbm_probe(plane, nbytes=1 << 30):
    """Achievable HBM bandwidth on this GPU: a 1 GiB buffer (4x the Infinity Cache) streamed with
    16-byte non-temporal loads (read), or copied into a second buffer (copy: read + write bytes),
    best over grid sizes and loads in flight per thread."""
    from bramha_amd import ops

    best = {"read": (0.0, None), "copy": (0.0, None)}
    for copy in (False, True):
        for wgs in (2048, 4096, 8192):
            for unroll in (4, 8, 16):
                us = ops.time_probe(plane, copy, nbytes, wgs, unroll, iters=10)
                gbps = (2 if copy else 1) * nbytes / us / 1e3
                key = "copy" if copy else "read"
                if gbps > best[key][0]:
                    best[key] = (gbps, {"workgroups": wgs, "loads_in_flight": unroll, "us": round(us, 1)})
    r = {"read_GBps": round(best["read"][0], 1), "read_frac": round(best["read"][0] * 1e9 / HBM_PEAK, 4),
         "read_shape": best["read"][1], "copy_GBps": round(best["copy"][0], 1),
         "copy_frac": round(best["copy"][0] * 1e9 / HBM_PEAK, 4), "copy_shape": best["copy"][1],
         "bytes": nbytes}
    log("HBM probe: read %.0f GB/s (%.1f%% of 8 TB/s), copy %.0f GB/s" %
        (r["read_GBps"], 100 * r["read_frac"], r["copy_GBps"]))
    return r


def attn_sweep(plane, rotate=1 << 30, iters=32, seed=0, nq=14, nkv=2, hd=64, contexts=(512, 4096, 32768),
               batches=(1, 8)):
    """GQA decode attention alone: 14 query heads over 2 KV heads of 64, fp16 K/V N(0, 1) in the
    decoder's MFMA-tile layout, one query token per sequence at the end of its context, softmax
    in f32.
    Bytes = K + V rows read + queries + outputs."""
    import numpy as np

    from bramha_amd import ops

    rng = np.random.default_rng(seed)
    out = []
    for T in contexts:
        for B in batches:
            rows = T * B
            k = rng.standard_normal((nkv, rows, hd), dtype=np.float32).astype(np.float16)
            v = rng.standard_normal((nkv, rows, hd), dtype=np.float32).astype(np.float16)
            k, v = ops.pack_kv_f16(k, v)  # the decoder's fp16 cache layout
            q = rng.standard_normal((B, nq * hd), dtype=np.float32)
            dk, dv, dq = (ops.DeviceArray.from_numpy(plane, a) for a in (k, v, q))
            off = ops.DeviceArray.from_numpy(plane, np.arange(B, dtype=np.int64) * T)
            ln = ops.DeviceArray.from_numpy(plane, np.full(B, T, np.int32))
            us = ops.time_attn(plane, dq, dk, dv, off, ln, nq, nkv, hd, T, iters=iters, rotate_bytes=rotate)
            nbytes = 2.0 * rows * nkv * hd * 2 + 2 * B * nq * hd * 4
            r = {"context": T, "batch": B, "us": round(us, 3), "GBps": round(nbytes / us / 1e3, 1),
                 "hbm_frac": round(nbytes / (us * 1e-6) / HBM_PEAK, 4)}
            log("attn T=%-6d B=%d %8.2f us %7.1f GB/s (%.1f%% HBM)" % (T, B, us, r["GBps"], 100 * r["hbm_frac"]))
            out.append(r)
            for a in (dk, dv, dq, off, ln):
                a.free()
    return out


def ragged_decode(plane, n_seq=32, lo=128, hi=8192, steps=128, new_prompt=64, max_chunk=16, seed=0):
    """Ragged batched decode, Qwen2-0.5B shape, 4-bit: n_seq sequences whose contexts are drawn
    uniformly from [lo, hi] by seed (random prompt tokens, prefilled into one packed KV buffer at
    prefix-sum offsets), then `steps` decode steps of the whole batch. A sequence ends at an EOS
    id or at its own output length, drawn uniformly from [16, steps] by seed (requests of unequal
    length); an ended sequence is replaced in its batch entry by a new one with a
    `new_prompt`-token random prompt, prefilled inside the timed loop into the ended sequence's
    KV region (its slot reopened), so the captured decode step stays valid; the prompts of the
    entries that end at the same step are prefilled together (one multi-sequence pass). Only tokens of live
    sequences count. No sink eviction: the reference's prefill cannot pass its 4096-row eviction
    limit (its prefill attention reads evicted rows by absolute position and panics,
    cpu_engine.rs:1166-1170, 1728-1754), so every sequence keeps its whole context."""
    import numpy as np

    from bramha_amd import BH_Q4_G32, ops
    from bramha_amd.model import (EOS_IDS, QWEN2_0_5B, DecoderConfig, HipDecoder, ragged_contexts, synth_tokens,
                                  synth_weights)

    ctx = ragged_contexts(seed, n_seq, lo, hi)
    rng = np.random.default_rng(seed + 1)
    caps = [int(c) + steps + 16 for c in ctx]
    kv_rows = sum((c + 63) // 64 * 64 for c in caps)
    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=n_seq,
                        kv_rows=kv_rows, max_tokens=2048)
    m = HipDecoder(plane, cfg)
    m.load(synth_weights(cfg, seed=seed))
    firsts = []
    ops.synchronize(plane)
    t0 = time.perf_counter()
    for s in range(n_seq):
        p = synth_tokens(seed, "ragged.%d" % s, int(ctx[s]), cfg.vocab)
        m.seq_open(s, caps[s])
        m.prefill(s, p[:-1])
        firsts.append(int(p[-1]))
    ops.synchronize(plane)
    t_pf = time.perf_counter() - t0
    pf_tokens = int(ctx.sum()) - n_seq
    log("ragged: prefilled %d tokens of %d sequences in %.2f s (%.0f tok/s)" % (pf_tokens, n_seq, t_pf, pf_tokens / t_pf))
    m.decode_setup(np.arange(n_seq, dtype=np.int32), np.array(firsts, np.uint32))
    m.decode(1)  # graph capture and a first replay, untimed
    ops.synchronize(plane)
    left = rng.integers(16, steps + 1, size=n_seq)  # output tokens still to come per entry
    left[:] = np.maximum(left - 1, 1)
    ctx_len = ctx.astype(np.int64) + 1  # rows attended by each entry's next step
    replaced = valid = 0
    kv_rows_steps = 0  # sum over timed steps of the rows attended
    t_decode = 0.0
    t0 = time.perf_counter()
    done = 0
    while done < steps:
        k = int(min(max_chunk, steps - done, left.min()))
        kv_rows_steps += int(sum(ctx_len)) * k + n_seq * k * (k - 1) // 2
        td = time.perf_counter()
        ids = m.decode(k)
        t_decode += time.perf_counter() - td
        refill = []
        for b in range(n_seq):
            hit = np.nonzero(np.isin(ids[:, b], EOS_IDS))[0]
            n_ok = min(int(hit[0]) + 1 if hit.size else k, int(left[b]))
            valid += n_ok
            left[b] -= k
            ctx_len[b] += k
            if (hit.size or left[b] <= 0) and done + k < steps:
                refill.append((b, synth_tokens(seed, "ragged.new.%d" % replaced, new_prompt, cfg.vocab)))
                replaced += 1
                left[b] = rng.integers(16, steps + 1)
                ctx_len[b] = new_prompt
        if refill:
            # the prompts of the entries that ended together are prefilled in one pass, each into
            # its entry's own slot reopened (same KV region: the captured step stays valid)
            for b, _ in refill:
                m.seq_open(b, new_prompt + steps + 16)
            m.prefill_batch([b for b, _ in refill], [p[:-1] for _, p in refill])
            for b, p in refill:
                m.decode_replace(b, b, int(p[-1]))
        done += k
    ops.synchronize(plane)
    dt = time.perf_counter() - t0
    m.close()
    weights = 277853184 + 175616 + 110592  # 4-bit layers + LM head, norms, biases
    kv_per_row = cfg.n_layers * 2 * cfg.kv_dim * 2  # fp16 K and V of one context row, all layers
    step_bytes = weights + kv_per_row * kv_rows_steps / steps
    r = {"value": valid / dt, "unit": "tok/s", "batch": n_seq, "steps": steps, "ms_per_step": dt * 1e3 / steps,
         "decode_ms_per_step": t_decode * 1e3 / steps,
         "contexts": {"min": int(ctx.min()), "max": int(ctx.max()), "mean": float(ctx.mean())},
         "replaced": replaced, "eviction": "none (every sequence keeps its whole context)",
         "end_rule": "EOS or a per-sequence output length uniform in [16, %d]" % steps,
         "prefill_tok_s": pf_tokens / t_pf, "prefill_tokens": pf_tokens,
         "roofline": {"bound": "hbm", "bytes_per_step": step_bytes,
                      "achieved": step_bytes / (t_decode / steps) / 1e9, "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                      "frac": step_bytes / (t_decode / steps) / HBM_PEAK,
                      "note": "weights + fp16 K/V rows attended, per decode step (refill prefills excluded)"}}
    log("ragged: %.1f tok/s (%.3f ms/step, decode %.3f ms/step = %.0f GB/s), %d replaced" %
        (r["value"], r["ms_per_step"], r["decode_ms_per_step"], r["roofline"]["achieved"], replaced))
    return r


def qwen7b(plane, prompt_len=2048, steps=256, warmup=8, batches=(1, 16), seed=0):
    """Qwen2-7B shape, 4-bit g32 (untied LM head), fp16 KV: a prefill of `prompt_len` random
    tokens (one chunk), then `steps` greedy decode steps at each batch size (each sequence with
    its own prefilled prompt)."""
    import numpy as np

    from bramha_amd import BH_Q4_G32, ops
    from bramha_amd.model import QWEN2_7B, DecoderConfig, HipDecoder, synth_tokens, synth_weights

    nb = max(batches)
    cap = prompt_len + warmup + steps + 16
    cfg = DecoderConfig(**QWEN2_7B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=1 + nb,
                        kv_rows=(1 + nb) * ((cap + 7) // 8 * 8), max_tokens=prompt_len, tied=False)
    m = HipDecoder(plane, cfg)
    t0 = time.perf_counter()

    def progress(ws):
        for i, w in enumerate(ws):
            if i % 40 == 0:
                log("7b: tensor %d (%s) at %.1f s" % (i, w[0], time.perf_counter() - t0))
            yield w

    m.load(progress(synth_weights(cfg, seed=seed)))
    log("7b: weights ready in %.1f s" % (time.perf_counter() - t0))
    H, I, L, V = cfg.hidden, cfg.ffn, cfg.n_layers, cfg.vocab
    params = L * (H * (cfg.q_dim + 2 * cfg.kv_dim) + cfg.q_dim * H + 3 * H * I)
    out = {"params_per_token": params}
    slot = 0
    firsts = {}
    for B in batches:
        slots = list(range(slot, slot + B))
        tp = 0.0
        for s in slots:
            p = synth_tokens(seed, "7b.prompt.%d" % s, prompt_len, V)
            m.seq_open(s, cap)
            ops.synchronize(plane)
            t0 = time.perf_counter()
            m.prefill(s, p[:-1])
            ops.synchronize(plane)
            tp += time.perf_counter() - t0
            firsts[s] = int(p[-1])
        if B == batches[0]:
            n = prompt_len - 1
            flops = 2.0 * params * n + 4.0 * L * cfg.n_heads * cfg.head_dim * n * (n + 1) / 2
            out["prefill"] = {"tokens": n, "seconds": tp / B, "tok_s": n * B / tp, "TFLOPs": flops * B / tp / 1e12,
                              "roofline": {"bound": "mfma", "achieved": flops * B / tp / 1e12, "peak": 2500.0,
                                           "unit": "TFLOP/s", "frac": flops * B / tp / 2.5e15,
                                           "note": "algorithmic flops (2 per weight per token + causal attention) "
                                                   "over the dense fp16 MFMA peak; the projections issue each "
                                                   "product twice (fp16 hi + lo activation halves)"}}
            log("7b prefill: %d tokens in %.3f s (%.0f tok/s, %.1f TFLOP/s algorithmic)" %
                (n, tp / B, n * B / tp, flops * B / tp / 1e12))
        if steps <= 0:  # prefill only (counter collection)
            slot += B
            continue
        m.decode_setup(np.array(slots, np.int32), np.array([firsts[s] for s in slots], np.uint32))
        dt = timed_decode(m, steps, warmup)
        t = m.time_kernels(8)
        wbytes = (params + V * H) * 0.5625
        out["decode_bs%d" % B] = {"tok_s": B * steps / dt, "ms_per_step": dt * 1e3 / steps,
                                  "roofline": {"bound": "hbm", "bytes_per_step": wbytes,
                                               "achieved": wbytes / (dt / steps) / 1e9, "peak": HBM_PEAK / 1e9,
                                               "unit": "GB/s", "frac": wbytes / (dt / steps) / HBM_PEAK,
                                               "note": "4-bit g32 weights read once per step"},
                                  "per_class_us": {k: round(v[0], 2) for k, v in t.items()}}
        log("7b bs%d per-kernel us: %s" % (B, out["decode_bs%d" % B]["per_class_us"]))
        log("7b decode bs%d: %.1f tok/s (%.3f ms/step)" % (B, B * steps / dt, dt * 1e3 / steps))
        slot += B
    m.close()
    return out


def _cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s=15.0, prompt_len=32, max_steps=64):
    """The reference CPU path (the oracle's restatement of generate_cpu with CPU-only mode) on
    the headline workload: Qwen2-0.5B shape, the same 4-bit g32 projections and tied LM head
    (computed as the reference's Float GEMVs over the dequantized weights, the only form its CPU
    path has for them), a 32-token prompt (31 prefilled, as the reference prefills all but the
    last) and 64 greedy steps, on this host's cores; the run is repeated until about two thirds of
    the budget is timed. Also one run of the reference's own 4-bit format (per-row 4-bit
    projections with LUT dequant and the f32 tied LM head it keeps, cpu_engine.rs:2449-2455)."""
    import oracle
    from bramha_amd import BH_F32, BH_Q4_G32, BH_Q4_ROW
    from bramha_amd.model import QWEN2_0_5B, DecoderConfig, synth_tokens, synth_weights

    def run(cfg, runs_min, budget):
        """Decode steps and seconds of decode (each run's time minus that of its prefill alone)."""
        om = oracle.OracleModel(cfg)
        om.load(synth_weights(cfg, seed=0))
        p = synth_tokens(0, "prompt.0", prompt_len, cfg.vocab)
        om.generate(p[:2], 1)  # warm caches
        t0 = time.perf_counter()
        om.generate(p, 0)  # the prefill alone
        t_pre = time.perf_counter() - t0
        n = runs = 0
        dt = 0.0
        while runs < runs_min or dt < budget:
            t0 = time.perf_counter()
            n += len(om.generate(p, max_steps))
            dt += time.perf_counter() - t0 - t_pre
            runs += 1
        om.close()
        return n, runs, dt

    n, runs, dt = run(DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32), 1, budget_s * 2 / 3)
    n2, _, dt2 = run(DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_ROW, head_fmt=BH_F32), 1, 0.0)
    return {"value": n / dt, "unit": "tok/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": "%d runs of a %d-token prompt (%d prefilled) + %d greedy decode steps at batch 1 on the "
                      "headline model (4-bit g32 projections and tied LM head as f32 GEMVs over the dequantized "
                      "weights); decode steps over decode time (each run less its prefill), %.1f s"
                      % (runs, prompt_len, prompt_len - 1, max_steps, dt),
            "cpu_model": _cpu_model(), "nproc": os.cpu_count(),
            "threads_env": os.environ.get("OMP_NUM_THREADS"),
            "reference_format": {"value": n2 / dt2, "unit": "tok/s",
                                 "sample": "one run of the same prompt and steps with the reference's own 4-bit "
                                           "format: per-row 4-bit projections (LUT dequant) + f32 tied LM head, "
                                           "%.1f s of decode" % dt2}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--quick", action="store_true",
                    help="only the batch-1 and batch-32 decode (no probe, sweeps, other workloads or CPU baseline)")
    ap.add_argument("--only-bs1", action="store_true",
                    help="for kernel traces: only the batch-1 decode, printed as its own JSON object")
    ap.add_argument("--only-bs32", action="store_true",
                    help="for kernel traces: only the batch-32 decode, printed as its own JSON object")
    ap.add_argument("--only-workloads", action="store_true",
                    help="only the ragged 32-sequence decode and the Qwen2-7B prefill + decode")
    ap.add_argument("--profile-eager", type=int, default=0, metavar="BATCH",
                    help="for counter collection: only eager (non-graph) decode steps at this batch, kernel by kernel")
    ap.add_argument("--profile-7b", type=int, default=0, metavar="BATCH",
                    help="eager decode steps of a 2-layer model at Qwen2-7B widths (with its 152064-row LM "
                         "head) at this batch, for counter profiles of the 7B kernels")
    ap.add_argument("--profile-prefill", action="store_true",
                    help="for counter collection: only a 2047-token prefill of the Qwen2-7B shape")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="for counter scaling: 4 launches of the device copy probe over MB megabytes")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X "
              "(--gpus %d requested); sharding across GPUs is not implemented." % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    from bramha_amd.plane import HipComputePlane

    plane = HipComputePlane(0)
    if args.copy_probe:
        from bramha_amd import ops

        nbytes = args.copy_probe << 20
        us = ops.time_probe(plane, True, nbytes, 4096, 8, iters=1)
        print(json.dumps({"copy_probe_bytes": nbytes, "launches": 4, "us": us}), flush=True)
        plane.close()
        return
    if args.profile_eager:
        m, _ = build_model(plane, args.profile_eager, args.prompt, 64)
        t = m.time_kernels(8)
        print(json.dumps({k: v[0] for k, v in t.items()}), flush=True)
        m.close()
        plane.close()
        return
    if args.profile_7b:
        from bramha_amd import BH_Q4_G32
        from bramha_amd.model import QWEN2_7B, DecoderConfig, HipDecoder, synth_tokens, synth_weights

        b = args.profile_7b
        cfg = DecoderConfig(**dict(QWEN2_7B, n_layers=2), wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True,
                            max_seqs=b, kv_rows=b * 1024, max_tokens=64, tied=False)
        m = HipDecoder(plane, cfg)
        m.load(synth_weights(cfg, seed=0))
        for s_ in range(b):
            m.seq_open(s_, 1024)
            m.prefill(s_, synth_tokens(0, "7b.profile.%d" % s_, 8, cfg.vocab))
        m.decode_setup(list(range(b)), [1] * b)
        t = m.time_kernels(8)
        print(json.dumps({k: v[0] for k, v in t.items()}), flush=True)
        m.close()
        plane.close()
        return
    if args.profile_prefill:
        print(json.dumps({"qwen2_7b": qwen7b(plane, steps=0, batches=(1,))}), flush=True)
        plane.close()
        return
    if args.only_workloads:
        print(json.dumps({"ragged32": ragged_decode(plane), "qwen2_7b": qwen7b(plane)}), flush=True)
        plane.close()
        return
    total = args.warmup + args.steps
    if args.only_bs1 or args.only_bs32:
        b = 1 if args.only_bs1 else 32
        m, _ = build_model(plane, b, args.prompt, total + 32)
        dt = timed_decode(m, args.steps, args.warmup)
        kern, roof = roofline(m, batch=b)
        print(json.dumps({"bs%d" % b: {"value": b * args.steps / dt, "unit": "tok/s",
                                       "ms_per_step": dt * 1e3 / args.steps, "roofline": roof}}), flush=True)
        m.close()
        plane.close()
        return
    log("building bs1 model")
    floor = launch_floor(plane)
    m1, cfg = build_model(plane, 1, args.prompt, total + 32)
    dt1 = timed_decode(m1, args.steps, args.warmup)
    tok1 = args.steps / dt1
    log("bs1: %.1f tok/s (%.3f ms/step)" % (tok1, dt1 * 1e3 / args.steps))
    kern, roof = roofline(m1, batch=1)
    roof["floor"] = above_floor(roof, floor)
    roof["floor"]["grid_barrier_us_by_workgroups"] = grid_barrier(plane)
    log("dominant kernel %s: %.1f GB/s (%.1f%% of HBM peak)" % (kern, roof["achieved"], 100 * roof["frac"]))
    log("bs1 time above the dependent-launch floor: %s" % roof["floor"])
    m1.close()
    log("building bs32 model")
    m32, _ = build_model(plane, 32, args.prompt, total + 32)
    dt32 = timed_decode(m32, args.steps, args.warmup)
    kern32, roof32 = roofline(m32, batch=32)
    roof32["floor"] = above_floor(roof32, floor)
    bs32 = {"value": 32 * args.steps / dt32, "unit": "tok/s", "ms_per_step": dt32 * 1e3 / args.steps,
            "batch": 32, "roofline": roof32}
    log("bs32: %.1f tok/s (%.3f ms/step); dominant kernel %s: %.1f GB/s" %
        (bs32["value"], bs32["ms_per_step"], kern32, roof32["achieved"]))
    m32.close()
    probe = gsweep = gsweep7 = asweep = work = cpu = None
    if not args.quick:
        probe = hbm_probe(plane)
        log("isolated GEMV sweep")
        gsweep = gemv_sweep(plane)
        gsweep7 = gemv_sweep(plane, shapes=GEMV_SHAPES_7B, batches=GEMV_BATCHES_7B)
        log("isolated attention sweep")
        asweep = attn_sweep(plane)
        work = {"ragged32": ragged_decode(plane), "qwen2_7b": qwen7b(plane)}
        if not args.no_cpu_baseline:
            log("timing the CPU baseline")
            cpu = cpu_baseline()
            log("cpu baseline: %.2f tok/s on %d threads (%s)" % (cpu["value"], cpu["cores"], cpu["cpu_model"]))
    line = {
        "metric": METRIC,
        "value": tok1,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": dt1 * 1e3 / args.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "qwen2-0.5b-shape greedy decode, batch 1, 4-bit g32 fp16-scale projections and "
                               "tied LM head, fp16 KV, 32-token prompt, random-init weights N(0,0.02)",
                   "batch": 1, "prompt_len": args.prompt, "context_at_end": args.prompt + total,
                   "layers": cfg.n_layers, "hidden": cfg.hidden, "vocab": cfg.vocab},
        "bs32": bs32,
        "roofline": roof,
        "cpu_baseline": cpu,
        "hbm_probe": probe,
        "gemv_sweep": gsweep,
        "gemv_sweep_7b": gsweep7,
        "attn_sweep": asweep,
        "workloads": work,
    }
    print(json.dumps(line), flush=True)
    plane.close()


if __name__ == "__main__":
    main()
