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


TRAFFIC_PROFILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                               "pmc_traffic_decode_qwen2_0.5b_q4g32_bs1.md")


def pmc_traffic(kclass):
    """HBM bytes per launch of a kernel class at batch 1, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE summary (scaled by its copy probe); None when not measured."""
    try:
        for line in open(TRAFFIC_PROFILE):
            if line.startswith("traffic:"):
                vals = dict(kv.split("=") for kv in line.split()[1:])
                return float(vals[kclass]) if kclass in vals else None
    except OSError:
        return None
    return None


def roofline(m, n_steps=16, traffic=False):
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
                  "frac": achieved / HBM_PEAK, "traffic": pmc_traffic(best) if traffic else None, "kernel": best,
                  "bytes_per_launch": nbytes,
                  "mean_us": mean_us,
                  "weight_stream": stream,
                  "per_class_us": {k: round(v[0], 3) for k, v in t.items()},
                  "launches_per_step": {k: v[1] // n_steps for k, v in t.items()}}


# (out_features, in_features) of the Qwen2-0.5B projections: q/o, k/v, gate/up, down, LM head.
GEMV_SHAPES = ((896, 896), (128, 896), (4864, 896), (896, 4864), (151936, 896))
GEMV_BATCHES = (1, 4, 16, 32)


def gemv_sweep(plane, rotate=1 << 30, iters=64):
    """Isolated 4-bit GEMV/GEMM: one fp16 scale per 32 weights, weights N(0, 0.02) before
    quantization, activations N(0, 1). Each launch streams its weight from HBM (graph of
    launches rotating over >= 1 GiB of weight copies). Bytes = packed nibbles + scales +
    activations in + outputs."""
    import numpy as np

    from bramha_amd import BH_Q4_G32, ops
    from bramha_amd.model import quantize, synth_normal

    out = []
    for n, k in GEMV_SHAPES:
        w = synth_normal(0, "sweep.%dx%d" % (n, k), n * k, 0.02).reshape(n, k)
        q, sc = quantize(BH_Q4_G32, w)
        del w
        dw = ops.DeviceWeight(plane, BH_Q4_G32, n, k, q, sc)
        for b in GEMV_BATCHES:
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


def ragged_decode(plane, n_seq=32, lo=128, hi=8192, steps=128, new_prompt=64, chunk=16, seed=0):
    """Ragged batched decode, Qwen2-0.5B shape, 4-bit: n_seq sequences whose contexts are drawn
    uniformly from [lo, hi] by seed (random prompt tokens, prefilled into one packed KV buffer at
    prefix-sum offsets), then `steps` decode steps of the whole batch; a sequence that emits an
    EOS id is replaced by a new one with a `new_prompt`-token random prompt (prefilled inside
    the timed loop). Tokens after an EOS within a chunk of steps are not counted."""
    import numpy as np

    from bramha_amd import BH_Q4_G32, ops
    from bramha_amd.model import EOS_IDS, QWEN2_0_5B, DecoderConfig, HipDecoder, synth_tokens, synth_weights

    rng = np.random.default_rng(seed)
    ctx = rng.integers(lo, hi + 1, size=n_seq)
    caps = [int(c) + steps + 16 for c in ctx]
    rep_cap = new_prompt + steps + 16
    kv_rows = sum((c + 7) // 8 * 8 for c in caps) + n_seq * ((rep_cap + 7) // 8 * 8)
    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_G32, head_fmt=BH_Q4_G32, kv_f16=True, max_seqs=2 * n_seq,
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
    m.decode(2)  # graph capture and first replays, untimed
    ops.synchronize(plane)
    next_slot, replaced, valid = n_seq, 0, 0
    t0 = time.perf_counter()
    done = 0
    while done < steps:
        k = min(chunk, steps - done)
        ids = m.decode(k)
        for b in range(n_seq):
            col = ids[:, b]
            hit = np.nonzero(np.isin(col, EOS_IDS))[0]
            if hit.size and next_slot < cfg.max_seqs:
                valid += int(hit[0]) + 1
                p = synth_tokens(seed, "ragged.new.%d" % next_slot, new_prompt, cfg.vocab)
                m.seq_open(next_slot, rep_cap)
                m.prefill(next_slot, p[:-1])
                m.decode_replace(b, next_slot, int(p[-1]))
                next_slot += 1
                replaced += 1
            else:
                valid += k
        done += k
    ops.synchronize(plane)
    dt = time.perf_counter() - t0
    m.close()
    r = {"value": valid / dt, "unit": "tok/s", "batch": n_seq, "steps": steps, "ms_per_step": dt * 1e3 / steps,
         "contexts": {"min": int(ctx.min()), "max": int(ctx.max()), "mean": float(ctx.mean())},
         "replaced": replaced, "prefill_tok_s": pf_tokens / t_pf, "prefill_tokens": pf_tokens}
    log("ragged: %.1f tok/s decode (%.3f ms/step), %d replaced" % (r["value"], r["ms_per_step"], replaced))
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
                              "mfma_frac": flops * B / tp / 2.5e15}
            log("7b prefill: %d tokens in %.3f s (%.0f tok/s, %.1f TFLOP/s algorithmic)" %
                (n, tp / B, n * B / tp, flops * B / tp / 1e12))
        m.decode_setup(np.array(slots, np.int32), np.array([firsts[s] for s in slots], np.uint32))
        dt = timed_decode(m, steps, warmup)
        t = m.time_kernels(8)
        out["decode_bs%d" % B] = {"tok_s": B * steps / dt, "ms_per_step": dt * 1e3 / steps,
                                  "weight_GBps": (params + V * H) * 0.5625 / (dt / steps) / 1e9,
                                  "per_class_us": {k: round(v[0], 2) for k, v in t.items()}}
        log("7b bs%d per-kernel us: %s" % (B, out["decode_bs%d" % B]["per_class_us"]))
        log("7b decode bs%d: %.1f tok/s (%.3f ms/step)" % (B, B * steps / dt, dt * 1e3 / steps))
        slot += B
    m.close()
    return out


def cpu_baseline(budget_s=15.0, max_steps=64):
    """The reference CPU path (the oracle's restatement of generate_cpu with CPU-only mode):
    Qwen2-0.5B shape, 4-bit per-row projections (the reference's U4 format) and the f32 tied
    LM head the reference keeps (cpu_engine.rs:2449-2455), on this host's cores."""
    import numpy as np

    import oracle
    from bramha_amd import BH_F32, BH_Q4_ROW
    from bramha_amd.model import QWEN2_0_5B, DecoderConfig, synth_tokens, synth_weights

    cfg = DecoderConfig(**QWEN2_0_5B, wfmt=BH_Q4_ROW, head_fmt=BH_F32)
    om = oracle.OracleModel(cfg)
    om.load(synth_weights(cfg, seed=0))
    p = synth_tokens(0, "prompt.0", 2, cfg.vocab)
    om.generate(p, 1)  # warm caches
    # the same run repeated until about two thirds of the budget (~10 s) of CPU work is timed
    n = runs = 0
    dt = 0.0
    while runs == 0 or dt < budget_s * 2 / 3:
        t0 = time.perf_counter()
        n += len(om.generate(p, max_steps))
        dt += time.perf_counter() - t0
        runs += 1
    return {"value": n / dt, "unit": "tok/s", "cores": oracle.num_threads(), "kind": "port",
            "sample": "%d runs of %d greedy decode steps at batch 1 after a 1-token prefill, 4-bit per-row "
                      "projections + f32 tied LM head (the reference's CPU 4-bit path), %.1f s"
                      % (runs, max_steps, dt)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only-bs1", action="store_true")
    ap.add_argument("--only-bs32", action="store_true",
                    help="for kernel traces: only the batch-32 decode, printed as its own JSON object")
    ap.add_argument("--no-sweeps", action="store_true", help="skip the isolated GEMV and attention sweeps")
    ap.add_argument("--full", action="store_true",
                    help="also run the ragged 32-sequence decode and the Qwen2-7B prefill + decode workloads")
    ap.add_argument("--only-full", action="store_true", help="run only the --full workloads")
    ap.add_argument("--profile-eager", action="store_true",
                    help="for counter collection: only eager (non-graph) bs1 decode steps, kernel by kernel")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MB",
                    help="for counter scaling: a plain device copy of MB megabytes (torch), 4 times")
    args = ap.parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the decode path runs on a single MI355X "
              "(--gpus %d requested); sharding across GPUs is not implemented." % args.gpus,
              file=sys.stderr)
        sys.exit(2)

    if args.copy_probe:
        import torch

        src = torch.ones(args.copy_probe << 18, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": src.numel() * 4, "launches": 4}), flush=True)
        return

    from bramha_amd.plane import HipComputePlane

    plane = HipComputePlane(0)
    if args.profile_eager:
        m1, _ = build_model(plane, 1, args.prompt, 64)
        t = m1.time_kernels(8)
        print(json.dumps({k: v[0] for k, v in t.items()}), flush=True)
        m1.close()
        plane.close()
        return
    if args.only_full:
        print(json.dumps({"ragged32": ragged_decode(plane), "qwen2_7b": qwen7b(plane)}), flush=True)
        plane.close()
        return
    total = args.warmup + args.steps
    if args.only_bs32:
        m32, _ = build_model(plane, 32, args.prompt, total + 32)
        dt32 = timed_decode(m32, args.steps, args.warmup)
        kern32, roof32 = roofline(m32)
        print(json.dumps({"bs32": {"value": 32 * args.steps / dt32, "unit": "tok/s",
                                   "ms_per_step": dt32 * 1e3 / args.steps, "roofline": roof32}}), flush=True)
        m32.close()
        plane.close()
        return
    log("building bs1 model")
    m1, cfg = build_model(plane, 1, args.prompt, total + 32)
    dt1 = timed_decode(m1, args.steps, args.warmup)
    tok1 = args.steps / dt1
    log("bs1: %.1f tok/s (%.3f ms/step)" % (tok1, dt1 * 1e3 / args.steps))
    kern, roof = roofline(m1, traffic=True)
    log("dominant kernel %s: %.1f GB/s (%.1f%% of HBM peak)" % (kern, roof["achieved"], 100 * roof["frac"]))
    m1.close()
    bs32 = None
    if not args.only_bs1:
        log("building bs32 model")
        m32, _ = build_model(plane, 32, args.prompt, total + 32)
        dt32 = timed_decode(m32, args.steps, args.warmup)
        kern32, roof32 = roofline(m32)
        bs32 = {"value": 32 * args.steps / dt32, "unit": "tok/s", "ms_per_step": dt32 * 1e3 / args.steps,
                "batch": 32, "roofline": roof32}
        log("bs32: %.1f tok/s (%.3f ms/step); dominant kernel %s: %.1f GB/s" %
            (bs32["value"], bs32["ms_per_step"], kern32, roof32["achieved"]))
        m32.close()
    gsweep = asweep = None
    if not args.no_sweeps:
        log("isolated GEMV sweep")
        gsweep = gemv_sweep(plane)
        log("isolated attention sweep")
        asweep = attn_sweep(plane)
    full = None
    if args.full:
        full = {"ragged32": ragged_decode(plane), "qwen2_7b": qwen7b(plane)}
    cpu = None
    if not args.no_cpu_baseline:
        log("timing the CPU baseline")
        cpu = cpu_baseline()
        log("cpu baseline: %.2f tok/s on %d threads" % (cpu["value"], cpu["cores"]))
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
        "gemv_sweep": gsweep,
        "attn_sweep": asweep,
        "full": full,
    }
    print(json.dumps(line), flush=True)
    plane.close()


if __name__ == "__main__":
    main()
