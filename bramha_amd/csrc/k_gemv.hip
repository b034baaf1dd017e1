// k_gemv.hip — weight-streaming GEMV for decode (batch <= 8 per pass) on gfx950.
//
// Reference semantics: matvec_mul_into (src/inference/cpu_engine.rs:1307-1444):
// y[j] = scale[j] * sum_i h[i] * q[j][i] for the row formats, plain dot for F32.
// The Q4_G32 format applies its fp16 scale per group of 32 (one 16-byte chunk).
//
// Design (HBM-bound, no MFMA): one lane per output row streaming the K-major 16-byte chunks
// with SGPR activations (k_stream.h). The first stage of weight loads is requested before
// anything else the kernel loads, so the weight latency overlaps the per-token norm factors and
// epilogue operands. Waves of a workgroup split K and combine in LDS in a fixed order, so
// results are deterministic without atomics.
// Epilogues fuse the RMSNorm factor, bias, residual add (with the next norm's inputs),
// SiLU gate, RoPE + KV-cache append, and the LM-head repetition penalty + argmax.
// Batch-1 group-32 passes whose activations come as int4 limb records (k_xl.h) take each chunk as
// 24 integer dots (v_dot8_i32_i4) instead of 32 converts and 32 FMAs.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include <atomic>

#include "k_epilogue.h"
#include "k_stream.h"

namespace bh {
namespace {

template <int FMT, int B, int EPI, int RW, int U, int CP, bool XL>
__global__ void __launch_bounds__(1024) k_gemv(const GemvArgs a) {
    extern __shared__ float smem[];
    float* rn = smem;          // [32] per-token norm factors
    float* comb = smem + 32;   // K-split combine area, then epilogue scratch
    constexpr int E = Fmt<FMT>::E;
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    // U: chunks per pipeline stage (two stages in flight), sized to the wave's chunk count
    constexpr int TOT = NACC * B * ROWS;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nwaves = blockDim.x >> 6;
    const int ksplit = nwaves / RW;
    const int rw = wave % RW, kw = wave / RW;
    const int r = rw * 64 + lane;
    const int ksw = a.ksw;
    const int tiles = gridDim.x / ksw;
    const int tile = blockIdx.x % tiles, kws = blockIdx.x / tiles;
    const int64_t n = (int64_t)tile * ROWS + r;
    // this workgroup's chunk range, then this wave's share of it
    const int per_wg = (a.C + ksw - 1) / ksw;
    const int wc0 = kws * per_wg, wc1 = min(a.C, wc0 + per_wg);
    const int per = (max(wc1 - wc0, 0) + ksplit - 1) / ksplit;
    const int c0 = wc0 + kw * per;
    const int c1 = min(wc1, c0 + per);
    const bool row_ok = n < a.n_pad;

    // Loads use a clamped row so they are unconditional and in bounds; rows past n_pad (RW = 2
    // tiles) compute values the epilogue never stores.
    const int64_t nl = row_ok ? n : (int64_t)a.n_pad - 1;
    EpiPre<EPI> pre;

    {
        float acc[NACC][B];
        float touch[TOUCH_ROWS];
        RnormLanes<B, (B <= 4 ? RN_U : 8)> rq;
        stream_chunks<FMT, B, NACC, U, CP, XL>(a, nl, c0, c1, acc, [&] {
            // the activation touch (bs1 decode step: 1232 -> 1291 tok/s), the norm factors and the
            // batch-1 epilogue operands load while the first weight stage is in flight
            if constexpr (XL) touch_xl(a, wc0, wc1, touch);
            else touch_activations<B, E>(a, wc0, wc1, touch);
            rq.request(a);
            if constexpr (B == 1) pre.load(a, (int64_t)tile * ROWS, ROWS);
        });
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int b = 0; b < B; ++b) comb[kw * TOT + (j * B + b) * ROWS + r] = acc[j][b];
        rq.finish(a, rn);
        touch_sink<B>(touch);
    }

    if constexpr (B == 1 && RW == 1 && (EPI == EPI_RESNORM || EPI == EPI_QKV)) {
        // batch 1: wave 0 (lane = row, holding the row's epilogue operands) sums the waves'
        // partials in order, reduces a residual producer's K split and finishes the tile in
        // registers; the other waves are done. (The gate/up pair stays on the shared path: one
        // wave summing both halves ran 0.5 % slower per step than two waves and a barrier.)
        if (EPI == EPI_RESNORM || ksw == 1) {
            __syncthreads();
            if (wave != 0) return;
            float sum = comb[lane];
            for (int w = 1; w < ksplit; ++w) sum += comb[w * TOT + lane];
            if constexpr (EPI == EPI_RESNORM) {
                if (ksw > 1 && !split_reduce_wave(a, sum, tile, kws)) return;
                resnorm_wave<FMT>(a, sum, (int64_t)tile * ROWS, pre);
            } else {
                qkv_wave<FMT>(a, sum, rn[0], (int64_t)tile * ROWS, pre);
            }
            return;
        }
    }

    // ---- combine the K-split partial sums in a fixed order ----
    __syncthreads();
    for (int i = threadIdx.x; i < TOT; i += blockDim.x) {
        float sum = comb[i];
        for (int w = 1; w < ksplit; ++w) sum += comb[w * TOT + i];
        comb[i] = sum;
    }
    if (ksw > 1 && !split_reduce<TOT>(a, comb, tile, kws)) return;
    __syncthreads();
    run_epilogue<FMT, B, EPI, ROWS>(a, comb, comb + TOT, rn, (int64_t)tile * ROWS, B == 1 ? &pre : nullptr);
}

template <int FMT, int B, int EPI, int RW, int U, bool XL = false>
hipError_t launch_one(const GemvArgs& a, int ksplit, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    const int tiles = (a.n_pad + ROWS - 1) / ROWS * a.ksw;
    size_t shm = (size_t)ksplit * NACC * B * ROWS * sizeof(float);
    if (EPI == EPI_LMHEAD || EPI == EPI_RESNORM) shm = std::max(shm, (size_t)(NACC * B * ROWS + B * ROWS) * sizeof(float));
    shm += 32 * sizeof(float);
    // non-temporal weight loads pay off on weights far larger than the caches (LM head: 20 us
    // instead of 22) and cost latency-bound small ones ~0.2 us
    if (FMT == BH_Q4_G32 && (size_t)a.C * a.n_pad * 16 >= STREAM_BYTES)
        launch_kernel((k_gemv<FMT, B, EPI, RW, U, FMT == BH_Q4_G32 ? CPOL_STREAM : 0, XL>), dim3(tiles),
                      dim3(64 * RW * ksplit), shm, st, a);
    else
        launch_kernel((k_gemv<FMT, B, EPI, RW, U, 0, XL>), dim3(tiles), dim3(64 * RW * ksplit), shm, st, a);
    return hipGetLastError();
}

// The batch-1 group-32 pass with limb activations (a.xl set). With the integer dots the loop
// waits on loads, not on arithmetic, and shallow stages keep more wavefronts resident: stages of
// 2 chunks, 1 for the gate/up pair and QKV (measured in the Qwen2-7B-width decode step: LM head
// 57 -> 50 us with 8 waves per tile, gate/up 22.2 -> 19.1, down 12.1 -> 10.8, QKV 8.0 -> 7.7;
// Qwen2-0.5B LM head 17.6 -> 15.9, gate/up 5.2 -> 4.8, QKV 4.8 -> 4.5).
template <int EPI, int RW>
hipError_t launch_xl(const GemvArgs& a, int ksplit, int cpw, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    if (cpw <= 1 || NACC == 2 || EPI == EPI_QKV) return launch_one<BH_Q4_G32, 1, EPI, RW, 1, true>(a, ksplit, st);
    return launch_one<BH_Q4_G32, 1, EPI, RW, 2, true>(a, ksplit, st);
}

// Stage depth from the chunks each wave streams (cpw): a single stage covers short ranges,
// deep stages keep long ones in flight. NACC == 2 doubles the loads per chunk.
template <int FMT, int EPI, int RW>
hipError_t launch_b(const GemvArgs& a, int B, int ksplit, int cpw, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    if constexpr (FMT == BH_Q4_G32)
        if (B == 1 && a.xl) return launch_xl<EPI, RW>(a, ksplit, cpw, st);
    if (B <= 2) {
        const bool b1 = B == 1;
        if (cpw <= 2) return b1 ? launch_one<FMT, 1, EPI, RW, 2>(a, ksplit, st) : launch_one<FMT, 2, EPI, RW, 2>(a, ksplit, st);
        if (cpw <= 12 || NACC == 2)
            return b1 ? launch_one<FMT, 1, EPI, RW, 4>(a, ksplit, st) : launch_one<FMT, 2, EPI, RW, 4>(a, ksplit, st);
        return b1 ? launch_one<FMT, 1, EPI, RW, 8 / NACC>(a, ksplit, st)
                  : launch_one<FMT, 2, EPI, RW, 8 / NACC>(a, ksplit, st);
    }
    if (B == 4) return launch_one<FMT, 4, EPI, RW, 4 / NACC>(a, ksplit, st);
    return launch_one<FMT, 8, EPI, RW, 4 / NACC>(a, ksplit, st);
}

template <int FMT>
hipError_t launch_fmt(int epi, const GemvArgs& a, int B, int rw, int ksplit, int cpw, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: return launch_b<FMT, EPI_STORE, 1>(a, B, ksplit, cpw, st);
        case EPI_RESNORM: return launch_b<FMT, EPI_RESNORM, 1>(a, B, ksplit, cpw, st);
        case EPI_SILU: return launch_b<FMT, EPI_SILU, 1>(a, B, ksplit, cpw, st);
        case EPI_QKV:
            return rw == 2 ? launch_b<FMT, EPI_QKV, 2>(a, B, ksplit, cpw, st)
                           : launch_b<FMT, EPI_QKV, 1>(a, B, ksplit, cpw, st);
        default:
            if constexpr (FMT == BH_F32 || FMT == BH_Q4_G32) return launch_b<FMT, EPI_LMHEAD, 1>(a, B, ksplit, cpw, st);
            return hipErrorInvalidValue;
    }
}

// Limb records (k_xl.h) of one activation row of n elements: a wavefront per 64 elements
// (elements past n count as zero), records of chunks [0, ceil(n / 32)).
__global__ void __launch_bounds__(256) k_xl_pack(const float* x, int n, uint32_t* rec) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t base = i & ~(int64_t)63;
    if (base >= n) return;  // whole wavefronts
    const float v = i < n ? x[i] : 0.f;
    xl_pack64(v, rec, base / 32, (n + 31) / 32);
}

}  // namespace

hipError_t launch_xl_pack(const float* x, int n, uint32_t* rec, hipStream_t st) {
    if (n <= 0) return hipSuccess;
    launch_kernel(k_xl_pack, dim3((n + 255) / 256), dim3(256), 0, st, x, n, rec);
    return hipGetLastError();
}

// Waves per workgroup along K: aim for ~32 waves per CU and >= 2 chunks per wave; the combine
// area stays under 60 KB. (Measured on the 151936 x 896 LM head: 4 waves per row tile stream
// 3.5 TB/s where 1 wave per tile streams 2.8.)
static int waves_per_tile(int tiles, int rw, int C, int nacc, int B) {
    int ks = (8192 + tiles * rw - 1) / (tiles * rw);
    // at most 12 waves per tile (8 for the gate/up pair, whose kernel holds fewer waves per CU) on
    // matrices with many row tiles, so that every workgroup of the launch stays resident (18944 x
    // 3584 streams 2.8 TB/s instead of 2.3 with 16; the 7B gate/up pair 25 us instead of 31);
    // 16 on small ones (latency-bound: 16 waves per tile are fastest on 4864 x 896)
    // (a K-split launch of at most 256 workgroups keeps 16: 3584 x 18944 at 4 splits, 13.3 us
    // instead of 14.8 with 12)
    ks = std::max(1, std::min({ks, (tiles > 256 ? (nacc == 2 ? 8 : 12) : 16) / rw, std::max(1, C / 2)}));
    while (ks > 1 && (size_t)ks * nacc * B * 64 * rw * 4 > 60 * 1024) --ks;
    return ks;
}

// Workgroups per row tile for a K-split GEMV: about `target` workgroups in all, each streaming
// at least `min_chunks` chunks, at most MAX_KSW.
int gemv_splits(int tiles, int C, int min_chunks, int target) {
    const int ksw = target / std::max(tiles, 1);
    return std::max(1, std::min({ksw, MAX_KSW, std::max(1, C / std::max(min_chunks, 1))}));
}

// K splits of one pass when the caller left the choice to the launcher (ksw == 0) and provided
// split scratch: VALU passes split long-K matrices with few row tiles, and at batch 1 also long-K
// matrices with many (16 chunks per workgroup); MFMA passes split whenever the row tiles leave
// CUs idle. Bounded by the scratch (SPLIT_PART_FLOATS floats of sums, SPLIT_TILES_MAX arrival
// counters).
static int auto_splits(const GemvArgs& a, int epi, bool mfma, int rows_per_tile, int tot) {
    if (a.ksw > 0) return a.ksw;
    if (!a.part || !a.tile_cnt || tot > SPLIT_TOT_MAX) return 1;
    const int tiles = (a.n_pad + rows_per_tile - 1) / rows_per_tile;
    if (tiles > SPLIT_TILES_MAX) return 1;
    int ksw;
    // splits pay for their ordered reduction only on long-K matrices (measured: the 896-wide
    // projections are fastest unsplit at 1 and at 32 tokens; the 3584- and 18944-wide ones of a
    // 7B model stream 1.3-2x faster split to fill the CUs); MFMA passes aim at two workgroups
    // per CU, VALU passes at one. A batch-1 pass over many row tiles and a long K (the 7B
    // 18944 x 3584 gate/up pair: 25.2 us unsplit, 23.2 at 7 splits, 24.4 at 2, 26.9 at 14) takes
    // 16-chunk splits; not the LM head, whose split would add a reduction to its argmax epilogue.
    if (!(a.C >= 64)) ksw = 1;
    // (MFMA passes over 256+ row tiles and a long K aim at ~1200 workgroups: the 7B gate/up pair
    // at 16 tokens 67.7 us unsplit, 57.2 / 52.2 / 50.0 / 55.1 us at 2 / 3 / 4 / 6 splits)
    else if (mfma) ksw = tiles < 256 ? gemv_splits(tiles, a.C, 16, 512) : (epi == EPI_LMHEAD ? 1 : gemv_splits(tiles, a.C, 16, 1200));
    else if (tiles < 128) ksw = std::min(gemv_splits(tiles, a.C, 16, 256), 8);
    else ksw = (a.batch == 1 && a.C >= 100 && epi != EPI_LMHEAD) ? std::min(a.C / 16, 8) : 1;
    while (ksw > 1 && (int64_t)tiles * ksw * tot > (int64_t)SPLIT_PART_FLOATS) --ksw;
    return ksw;
}

// Compute units of the current device (queried once per device).
static int device_cus() {
    static std::atomic<int> cus[64];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cus[dev].load(std::memory_order_relaxed);
    if (v <= 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cus[dev].store(v, std::memory_order_relaxed);
    }
    return v;
}

// Splits the batch into passes: MFMA passes of 32 or 16 rows for 4-bit weights (k_gemm.hip),
// VALU passes of at most 8 rows otherwise.
hipError_t launch_gemv(int fmt, int epi, const GemvArgs& a0, hipStream_t st) {
    const int rw = (epi == EPI_QKV && a0.hd > 64) ? a0.hd / 64 : 1;
    if (rw > 2) return hipErrorInvalidValue;
    if (a0.ssq_in && a0.batch > 0 && (a0.ssq_tiles <= 0 || a0.norm_n <= 0.f)) return hipErrorInvalidValue;
    if (epi == EPI_RESNORM && (!a0.xw_out || !a0.wnext || !a0.ssq_out || a0.ssq_tiles != a0.n_pad / 64))
        return hipErrorInvalidValue;
    if (a0.ksw < 0 || a0.ksw > MAX_KSW || (a0.ksw > 1 && (!a0.part || !a0.tile_cnt))) return hipErrorInvalidValue;
    const int nacc = epi == EPI_SILU ? 2 : 1;
    int b0 = 0;
    while (b0 < a0.batch) {
        const int rem = a0.batch - b0;
        const bool q4 = fmt == BH_Q4_G32 || fmt == BH_Q4_ROW;
        if (q4 && rem >= PF_MIN_TOKENS && epi != EPI_LMHEAD) {
            // prefill chunk: every remaining token in one tiled launch, or, where its 128-row x
            // 64/128-token tiles would not give every CU a workgroup (narrow matrices, chunks of a
            // few hundred tokens: a batch of refill prompts), one launch of 16-token MFMA groups
            // (a 384-token chunk of the 896-wide projections: QKV 85 -> ~15 us)
            GemvArgs a = gemv_tokens(a0, b0, rem);
            a.ksw = 1;
            const int mt = epi == EPI_SILU ? 64 : 128;
            const int64_t pf_grid = (int64_t)((rem + mt - 1) / mt) * ((a0.n_pad + 127) / 128);
            if (rem <= MF_GROUPED_MAX && pf_grid < device_cus()) {
                const int B = (rem + 15) / 16 * 16;
                a.ksw = auto_splits(a0, epi, true, 64 * rw, nacc * 16 * 64 * rw);
                if (a.ksw > 1) {  // every group's split scratch must fit
                    const int64_t gt = (int64_t)(B / 16) * ((a0.n_pad + 64 * rw - 1) / (64 * rw));
                    if (gt > SPLIT_TILES_MAX || gt * a.ksw * nacc * 16 * 64 * rw > SPLIT_PART_FLOATS) a.ksw = 1;
                }
                return launch_gemm_mf(fmt, epi, a, B, rw, st);
            }
            return launch_gemm_pf(fmt, epi, a, st);
        }
        // MFMA passes of 16 or 32 token columns; the last pass of more than 8 tokens takes the
        // next column count up with only its tokens valid (activations past them read as zero,
        // nothing of theirs is stored), so a pass of 9..31 tokens is one launch
        const bool mf = q4 && rem > 8;
        int B = mf ? (rem > 16 ? 32 : 16) : (rem >= 8 ? 8 : (rem >= 4 ? 4 : (rem >= 2 ? 2 : 1)));
        // 33..63 tokens (below the tiled prefill GEMM): one launch of 16-token groups instead of
        // two 32-token passes (a 63-token refill prompt: one dependent launch per projection)
        if (mf && rem > 32 && epi != EPI_LMHEAD) B = (rem + 15) / 16 * 16;
        GemvArgs a = gemv_tokens(a0, b0, mf ? std::min(B, rem) : B);
        hipError_t e;
        if (B == 1 && !mf && fmt == BH_Q4_G32) {
            if (b0 > 0) a.xl = nullptr;  // a producer's records describe token 0
            if (!a.xl && a.xl_tmp) {     // the caller has x only: its records first
                e = launch_xl_pack(a.x, a.C * 32, a.xl_tmp, st);
                if (e != hipSuccess) return e;
                a.xl = a.xl_tmp;
            }
        } else {
            a.xl = nullptr;
        }
        if (mf && epi == EPI_LMHEAD && fmt == BH_Q4_G32 && lmhead_mf_fits(a, device_cus())) {
            e = launch_lmhead_mf(a, device_cus(), st);
        } else if (mf) {
            a.ksw = auto_splits(a0, epi, true, 64 * rw, nacc * std::min(B, 32) * 64 * rw);
            if (B > 32 && a.ksw > 1) {  // the groups' split scratch must fit too
                const int64_t gt = (int64_t)(B / 16) * ((a0.n_pad + 64 * rw - 1) / (64 * rw));
                if (gt > SPLIT_TILES_MAX || gt * a.ksw * nacc * 16 * 64 * rw > SPLIT_PART_FLOATS) a.ksw = 1;
            }
            e = launch_gemm_mf(fmt, epi, a, B, rw, st);
        } else {
            a.ksw = auto_splits(a0, epi, false, 64 * rw, nacc * B * 64 * rw);
            const int tiles = (a0.n_pad + 64 * rw - 1) / (64 * rw);
            int ks = waves_per_tile(tiles * a.ksw, rw, (a0.C + a.ksw - 1) / a.ksw, nacc, B);
            if (B == 1 && a.xl) {  // limb passes (launch_xl): LM heads ~14 chunks per wave, QKV <= 8 waves
                if (epi == EPI_LMHEAD) ks = std::max(4, std::min(a0.C / 14, 12));
                else if (epi == EPI_QKV) ks = std::min(ks, 8);
            }
            const int cpw = ((a0.C + a.ksw - 1) / a.ksw + ks - 1) / ks;  // chunks per wave
            switch (fmt) {
                case BH_F32: e = launch_fmt<BH_F32>(epi, a, B, rw, ks, cpw, st); break;
                case BH_Q8_ROW: e = launch_fmt<BH_Q8_ROW>(epi, a, B, rw, ks, cpw, st); break;
                case BH_Q4_ROW: e = launch_fmt<BH_Q4_ROW>(epi, a, B, rw, ks, cpw, st); break;
                case BH_Q4_G32: e = launch_fmt<BH_Q4_G32>(epi, a, B, rw, ks, cpw, st); break;
                default: return hipErrorInvalidValue;
            }
        }
        if (e != hipSuccess) return e;
        b0 += B;
    }
    return hipSuccess;
}

}  // namespace bh
