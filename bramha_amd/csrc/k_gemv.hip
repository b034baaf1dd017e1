// k_gemv.hip — weight-streaming GEMV for decode (batch <= 8 per pass) on gfx950.
//
// Reference semantics: matvec_mul_into (src/inference/cpu_engine.rs:1307-1444):
// y[j] = scale[j] * sum_i h[i] * q[j][i] for the row formats, plain dot for F32.
// The Q4_G32 format applies its fp16 scale per group of 32 (one 16-byte chunk).
//
// Design (HBM-bound, no MFMA): the weight is stored K-major in 16-byte chunks
// (bh_internal.h, "KM16"), so each lane owns one output row and a wavefront
// streams 1 KiB of contiguous weight bytes per chunk step with one
// global_load_dwordx4 per lane. The activations of a chunk are identical for all
// 64 lanes, so they arrive through scalar loads (s_load_dwordx16) and enter the
// FMAs as SGPR operands: no LDS traffic and no cross-lane reduction in the main loop.
// Nibbles are decoded as signed int4 (q ^ 8 == q - 8 in two's complement) shifted
// into the top of a byte and converted with the SDWA sign-extending byte convert:
// one VALU op per element plus three bit ops per 8 elements; the factor 16 is
// folded into the scale. The chunk loop is software-pipelined (the next batch of
// chunks is in flight while the current one is converted), and the first batch is
// requested before anything else the kernel loads, so the weight latency overlaps the
// per-token norm factors and epilogue operands. Waves of a workgroup split K and combine
// in LDS in a fixed order, so results are deterministic without atomics.
// Epilogues fuse the RMSNorm factor, bias, residual add (with the next norm's inputs),
// SiLU gate, RoPE + KV-cache append, and the LM-head repetition penalty + argmax.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_epilogue.h"

namespace bh {
namespace {

// Signed byte SEL of v converted to f32 (v_cvt_f32_i32 with SDWA sign extension).
template <int SEL>
__device__ __forceinline__ float sb2f(uint32_t v) {
    float r;
    if constexpr (SEL == 0)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_0" : "=v"(r) : "v"(v));
    else if constexpr (SEL == 1)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_1" : "=v"(r) : "v"(v));
    else if constexpr (SEL == 2)
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_2" : "=v"(r) : "v"(v));
    else
        asm("v_cvt_f32_i32_sdwa %0, sext(%1) dst_sel:DWORD dst_unused:UNUSED_PAD src0_sel:BYTE_3" : "=v"(r) : "v"(v));
    return r;
}

template <int FMT>
struct Fmt {
    static constexpr int E = (FMT == BH_Q4_ROW || FMT == BH_Q4_G32) ? 32 : (FMT == BH_Q8_ROW ? 16 : 4);
};

// Decode one 16-byte chunk into E values. Q4 values come out as 16*(q-8),
// Q8 values as q, F32 as is.
template <int FMT>
__device__ __forceinline__ void decode(const uint4 q, float* v) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    if constexpr (FMT == BH_Q4_ROW || FMT == BH_Q4_G32) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t hi = (w[d] & 0xF0F0F0F0u) ^ 0x80808080u;         // even elements
            const uint32_t lo = ((w[d] << 4) & 0xF0F0F0F0u) ^ 0x80808080u;  // odd elements
            v[8 * d + 0] = sb2f<0>(hi);
            v[8 * d + 1] = sb2f<0>(lo);
            v[8 * d + 2] = sb2f<1>(hi);
            v[8 * d + 3] = sb2f<1>(lo);
            v[8 * d + 4] = sb2f<2>(hi);
            v[8 * d + 5] = sb2f<2>(lo);
            v[8 * d + 6] = sb2f<3>(hi);
            v[8 * d + 7] = sb2f<3>(lo);
        }
    } else if constexpr (FMT == BH_Q8_ROW) {
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            v[4 * d + 0] = sb2f<0>(w[d]);
            v[4 * d + 1] = sb2f<1>(w[d]);
            v[4 * d + 2] = sb2f<2>(w[d]);
            v[4 * d + 3] = sb2f<3>(w[d]);
        }
    } else {
#pragma unroll
        for (int d = 0; d < 4; ++d) v[d] = __uint_as_float(w[d]);
    }
}

template <int FMT, int B, int EPI, int RW, int U, int CP>
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
        // Weight and scale loads are raw buffer loads: an SGPR resource per matrix, the lane's row
        // as the VGPR offset and the chunk as the (uniform) SGPR offset, so a stage costs no
        // per-load address arithmetic. Every load of a stage is unconditional (chunk index
        // clamped to the wave's last chunk, scale kept as raw fp16 bits) so all of a stage's
        // loads are in flight before the first of them is waited on.
        __amdgpu_buffer_rsrc_t rW[NACC], rS[NACC];
        rW[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.C * a.n_pad * 16, 0x00020000);
        rS[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S, (short)0, a.C * a.n_pad * 2, 0x00020000);
        if constexpr (NACC == 2) {
            rW[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W2, (short)0, a.C * a.n_pad * 16, 0x00020000);
            rS[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S2, (short)0, a.C * a.n_pad * 2, 0x00020000);
        }
        const int vo_w = (int)nl * 16, vo_s = (int)nl * 2;
        uint4 q0[NACC][U], q1[NACC][U];
        uint16_t s0[NACC][U], s1[NACC][U];
        auto fetch = [&](int c, uint4 (&q)[NACC][U], uint16_t (&s)[NACC][U]) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int cc = min(c + u, c1 - 1);
#pragma unroll
                for (int j = 0; j < NACC; ++j) {
                    q[j][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rW[j], vo_w, cc * a.n_pad * 16, CP));
                    if constexpr (FMT == BH_Q4_G32) s[j][u] = __builtin_amdgcn_raw_buffer_load_b16(rS[j], vo_s, cc * a.n_pad * 2, CP);
                }
            }
        };
        if (c0 < c1) fetch(c0, q0, s0);
        // The activations reach the FMAs through scalar loads issued chunk by chunk; they were
        // just written by the previous kernel (often on another XCD), so a first touch here, one
        // vector load per 128-byte line of the workgroup's range, brings them into L2 while the
        // first weight stage is in flight (bs1 decode step: 1232 -> 1291 tok/s). The value is
        // consumed only after the main loop, so nothing waits on it early.
        float touch = 0.f;
        {
            const int nx = (wc1 - wc0) * E;
            for (int bb = 0; bb < B; ++bb)
                for (int i2 = threadIdx.x * 32; i2 < nx; i2 += blockDim.x * 32)
                    touch += a.x[(int64_t)bb * a.ldx + wc0 * E + i2];
        }
        load_rnorm<B>(a, rn);
        if constexpr (B == 1)
            if (threadIdx.x < ROWS) pre.load(a, (int64_t)tile * ROWS);

        float acc[NACC][B];
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int b = 0; b < B; ++b) acc[j][b] = 0.f;

        // Chunks past c1 (clamped re-reads of the last one) are skipped by a uniform branch that
        // holds no vector loads, so the loads' wait counts are unaffected by it.
        auto consume = [&](int c, const uint4 (&q)[NACC][U], const uint16_t (&s)[NACC][U]) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (c + u < c1) {
                    const int kb = (c + u) * E;
#pragma unroll
                    for (int j = 0; j < NACC; ++j) {
                        float v[E];
                        decode<FMT>(q[j][u], v);
#pragma unroll
                        for (int b = 0; b < B; ++b) {
                            const float* xb = a.x + (int64_t)b * a.ldx + kb;
                            float p = 0.f;
#pragma unroll
                            for (int e = 0; e < E; ++e) p = fmaf(xb[e], v[e], p);
                            if constexpr (FMT == BH_Q4_G32)
                                acc[j][b] = fmaf(p, __half2float(__ushort_as_half(s[j][u])) * 0.0625f, acc[j][b]);
                            else
                                acc[j][b] += p;
                        }
                    }
                }
            }
        };
        if (c0 < c1) {
            for (int c = c0;; c += 2 * U) {
                fetch(c + U, q1, s1);
                consume(c, q0, s0);
                if (c + U >= c1) break;
                fetch(c + 2 * U, q0, s0);
                consume(c + U, q1, s1);
                if (c + 2 * U >= c1) break;
            }
        }
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int b = 0; b < B; ++b) comb[kw * TOT + (j * B + b) * ROWS + r] = acc[j][b];
        asm volatile("" ::"v"(touch));
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

template <int FMT, int B, int EPI, int RW, int U>
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
        launch_kernel((k_gemv<FMT, B, EPI, RW, U, FMT == BH_Q4_G32 ? CPOL_STREAM : 0>), dim3(tiles), dim3(64 * RW * ksplit),
                      shm, st, a);
    else
        launch_kernel((k_gemv<FMT, B, EPI, RW, U, 0>), dim3(tiles), dim3(64 * RW * ksplit), shm, st, a);
    return hipGetLastError();
}

// Stage depth from the chunks each wave streams (cpw): a single stage covers short ranges,
// deep stages keep long ones in flight. NACC == 2 doubles the loads per chunk.
template <int FMT, int EPI, int RW>
hipError_t launch_b(const GemvArgs& a, int B, int ksplit, int cpw, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
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

}  // namespace

// Waves per workgroup along K: aim for ~32 waves per CU and >= 2 chunks per wave; the combine
// area stays under 60 KB. (Measured on the 151936 x 896 LM head: 4 waves per row tile stream
// 3.5 TB/s where 1 wave per tile streams 2.8.)
static int waves_per_tile(int tiles, int rw, int C, int nacc, int B) {
    int ks = (8192 + tiles * rw - 1) / (tiles * rw);
    // at most 12 waves per tile (8 for the gate/up pair, whose kernel holds fewer waves per CU) on
    // matrices with many row tiles, so that every workgroup of the launch stays resident (18944 x
    // 3584 streams 2.8 TB/s instead of 2.3 with 16; the 7B gate/up pair 25 us instead of 31);
    // 16 on small ones (latency-bound: 16 waves per tile are fastest on 4864 x 896)
    ks = std::max(1, std::min({ks, (tiles > 128 ? (nacc == 2 ? 8 : 12) : 16) / rw, std::max(1, C / 2)}));
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
// split scratch: VALU passes split only long-K matrices with few row tiles; MFMA passes split
// whenever the row tiles leave CUs idle. Bounded by the scratch (SPLIT_WG_MAX workgroups of
// SPLIT_TOT_MAX floats).
static int auto_splits(const GemvArgs& a, bool mfma, int rows_per_tile, int tot) {
    if (a.ksw > 0) return a.ksw;
    if (!a.part || !a.tile_cnt || tot > SPLIT_TOT_MAX) return 1;
    const int tiles = (a.n_pad + rows_per_tile - 1) / rows_per_tile;
    int ksw;
    // splits pay for their ordered reduction only on long-K matrices (measured: the 896-wide
    // projections are fastest unsplit at 1 and at 32 tokens; the 3584- and 18944-wide ones of a
    // 7B model stream 1.3-2x faster split to fill the CUs); MFMA passes aim at two workgroups
    // per CU, VALU passes at one
    ksw = !(a.C >= 64) ? 1
          : mfma ? (tiles < 256 ? gemv_splits(tiles, a.C, 16, 512) : 1)
                 : (tiles < 128 ? std::min(gemv_splits(tiles, a.C, 16, 256), 8) : 1);
    while (ksw > 1 && tiles * ksw > SPLIT_WG_MAX) --ksw;
    return ksw;
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
            // prefill chunk: every remaining token in one tiled launch
            GemvArgs a = gemv_tokens(a0, b0, rem);
            a.ksw = 1;
            return launch_gemm_pf(fmt, epi, a, st);
        }
        const bool mf = q4 && rem >= 16;
        const int B = mf ? (rem >= 32 ? 32 : 16) : (rem >= 8 ? 8 : (rem >= 4 ? 4 : (rem >= 2 ? 2 : 1)));
        GemvArgs a = gemv_tokens(a0, b0, B);
        hipError_t e;
        if (mf) {
            a.ksw = auto_splits(a0, true, 64 * rw, nacc * B * 64 * rw);
            e = launch_gemm_mf(fmt, epi, a, B, rw, st);
        } else {
            a.ksw = auto_splits(a0, false, 64 * rw, nacc * B * 64 * rw);
            const int tiles = (a0.n_pad + 64 * rw - 1) / (64 * rw);
            const int ks = waves_per_tile(tiles * a.ksw, rw, (a0.C + a.ksw - 1) / a.ksw, nacc, B);
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
