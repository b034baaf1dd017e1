// k_gemm.hip — MFMA GEMM for passes of 16 or 32 tokens over 4-bit weights (batched decode
// and prefill) on gfx950.
//
// Reference semantics: gemm_cpu / fused_qkv_gemm (src/inference/cpu_engine.rs:565-912,
// 3325-3339) and, per token, matvec_mul_into (:1307-1444): Y[b][n] = sum_k W[n][k] X[b][k].
//
// Design: a workgroup owns a tile of 64 * RW weight rows and a K range; K splits further over
// the workgroup's KW wavefronts per 64-row group (their sums meet in an LDS tree, halving in a
// fixed order) and, for matrices with few row tiles, over workgroups (the ordered split
// reduction of k_epilogue.h).
// Each wavefront runs v_mfma_f32_16x16x32_f16 over its 64 rows as four 16-row A blocks — one
// 16-byte load of a row's chunk per lane, transposed across the lane groups into one dword of
// 8 nibbles per lane per block (rows_to_a), decoded to exact fp16 (q - 8) — with the tokens as the
// B operand: f32 activations split into fp16 hi + lo (hi + lo carries ~22 bits), so each product
// takes two MFMAs and the B operand of a chunk is shared by the four row blocks. All loads are
// raw buffer loads (SGPR resource, per-lane VGPR offset, per-chunk SGPR offset) issued
// unconditionally (clamped in range) a stage ahead of their use; group-32 fp16 scales multiply
// each chunk's MFMA result per row; per-row scales are applied in the epilogue.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_epilogue.h"
#include "k_mfma.h"

namespace bh {
namespace {

template <int NACC, int TB, int S>
struct MfStage {
    uint32_t w[S][NACC][4];  // [chunk][matrix]: the chunk of row n0 + lane (rows_to_a makes it A operands)
    uint4 s[S][NACC][2];     // fp16 group scales of rows rb * 16 + 4 lg .. + 3, rb = 0 .. 3 (sc_pos order)
    uint4 x[S][TB][2];       // f32 activations of token tb * 16 + lr, k = 8 lg .. + 7
};

// blockIdx.y: token group, tokens blockIdx.y * B .. + B - 1 of the launch's arguments (a pass
// of 32 tokens can run as two groups of 16: twice the workgroups, nothing shared between them),
// each group with its own region of the split scratch.
template <int FMT, int B, int EPI, int RW, int KW, int S, bool ONE_ROUND>
__global__ void __launch_bounds__(64 * KW * RW) k_gemm_mf(const GemvArgs a0) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    constexpr int TB = B / 16;
    constexpr int TOT = NACC * B * ROWS;
    // a pass's last group may hold fewer than B valid tokens (a.batch): their activations read as
    // zero through the buffer resource and the epilogues store only tokens below a.batch
    GemvArgs a = gemv_tokens(a0, (int)blockIdx.y * B, max(1, min(B, a0.batch - (int)blockIdx.y * B)));
    if (a0.part) a.part = a0.part + (int64_t)blockIdx.y * gridDim.x * TOT;
    if (a0.tile_cnt) a.tile_cnt = a0.tile_cnt + blockIdx.y * (gridDim.x / a0.ksw);
    // S: chunks per pipeline stage (two stages in flight)
    extern __shared__ float smem[];
    float* rn = smem;          // [32] per-token norm factors
    float* comb = smem + 32;   // [NACC][B][ROWS] sums, then epilogue scratch [B][ROWS]
    float* tree = comb + TOT;  // [KW or KW / 2][B][ROWS + 4] wave-sum exchange (before the epilogue)

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lr = lane & 15, lg = lane >> 4;
    const int rw = wave % RW, kw = wave / RW;  // 64-row group, K-split index (0 .. KW - 1)
    const int ksw = a.ksw;
    const int tiles = gridDim.x / ksw;
    // workgroup b runs on XCD b % 8; with a K split over fewer than 256 row tiles, each XCD takes
    // a contiguous range of the (K range, tile) items in K-range-major order, so the row tiles
    // that read one K range of the activations share an XCD's L2 instead of fetching it into all
    // eight (0.5B down at 32 tokens: 12.7 -> 9.3 MB fetched per launch, time unchanged). Not for
    // the 7B-width passes over more tiles (the gate/up pair at 16 tokens: 39.6 -> 43.8 us).
    int item = blockIdx.x;
    if (ksw > 1 && tiles < 256) {
        const int g = (int)gridDim.x, xcd = (int)blockIdx.x & 7, per = g >> 3, rem = g & 7;
        item = xcd * per + min(xcd, rem) + ((int)blockIdx.x >> 3);
    }
    const int tile = item % tiles, kws = item / tiles;
    const int per_wg = (a.C + ksw - 1) / ksw;
    const int wc0 = kws * per_wg, wc1 = min(a.C, wc0 + per_wg);
    const int per = (max(wc1 - wc0, 0) + KW - 1) / KW;
    const int c0 = wc0 + kw * per, c1 = min(wc1, c0 + per);

    // the group's 64 rows; a group past the padded matrix re-reads the last one (never stored)
    const int n0 = min(tile * ROWS + rw * 64, a.n_pad - 64);
    __amdgpu_buffer_rsrc_t rW[NACC], rS[NACC];
    rW[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.C * a.n_pad * 16, 0x00020000);
    if constexpr (NACC == 2) rW[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W2, (short)0, a.C * a.n_pad * 16, 0x00020000);
    if constexpr (FMT == BH_Q4_G32) {
        rS[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S, (short)0, a.C * a.n_pad * 2, 0x00020000);
        if constexpr (NACC == 2)
            rS[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S2, (short)0, a.C * a.n_pad * 2, 0x00020000);
    }
    const __amdgpu_buffer_rsrc_t rX =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)(a.batch * a.ldx * 4), 0x00020000);
    const int vo_x = ((int)((lr) * a.ldx) + 8 * lg) * 4;  // token lr (+ tb * 16 rows), k 8 lg

    auto fetch = [&](int c, MfStage<NACC, TB, S>& st) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            const int cc = min(c + u, c1 - 1);
#pragma unroll
            for (int j = 0; j < NACC; ++j) {
                const uint4 q = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rW[j], (n0 + lane) * 16,
                                                                                               cc * a.n_pad * 16, 0));
                st.w[u][j][0] = q.x;
                st.w[u][j][1] = q.y;
                st.w[u][j][2] = q.z;
                st.w[u][j][3] = q.w;
                if constexpr (FMT == BH_Q4_G32) {
                    // n0 is a multiple of 64: sc_pos puts this lane group's 16 rows at n0 + 16 lg
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        st.s[u][j][h] = __builtin_bit_cast(
                            uint4, __builtin_amdgcn_raw_buffer_load_b128(rS[j], (n0 + 16 * lg) * 2 + 16 * h, cc * a.n_pad * 2, 0));
                }
            }
#pragma unroll
            for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                for (int h = 0; h < 2; ++h)
                    st.x[u][tb][h] = __builtin_bit_cast(
                        uint4, __builtin_amdgcn_raw_buffer_load_b128(rX, vo_x + (int)(tb * 16 * a.ldx * 4) + h * 16, cc * 128, 0));
        }
    };

    f32x4 acc[NACC][4][TB];
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) acc[j][rb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    const Dec8K mg = dec8_consts();
    auto consume = [&](int c, const MfStage<NACC, TB, S>& st) {
#pragma unroll
        for (int u = 0; u < S; ++u) {
            if (c + u < c1) {
                half8 bh[TB], bl[TB];
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
                    split8(__builtin_bit_cast(float4, st.x[u][tb][0]), __builtin_bit_cast(float4, st.x[u][tb][1]), bh[tb],
                           bl[tb]);
#pragma unroll
                for (int j = 0; j < NACC; ++j) {
                    uint32_t wa[4] = {st.w[u][j][0], st.w[u][j][1], st.w[u][j][2], st.w[u][j][3]};
                    rows_to_a(wa);
#pragma unroll
                    for (int rb = 0; rb < 4; ++rb) {
                        const half8 av = dec8(wa[rb], mg);
                        if constexpr (FMT == BH_Q4_G32) {
                            const __half2* s2 = (const __half2*)&st.s[u][j][0] + 2 * rb;
                            const float2 sa = __half22float2(s2[0]), sb = __half22float2(s2[1]);
#pragma unroll
                            for (int tb = 0; tb < TB; ++tb) {
                                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[tb], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[tb], t, 0, 0, 0);
                                acc[j][rb][tb][0] = fmaf(sa.x, t[0], acc[j][rb][tb][0]);
                                acc[j][rb][tb][1] = fmaf(sa.y, t[1], acc[j][rb][tb][1]);
                                acc[j][rb][tb][2] = fmaf(sb.x, t[2], acc[j][rb][tb][2]);
                                acc[j][rb][tb][3] = fmaf(sb.y, t[3], acc[j][rb][tb][3]);
                            }
                        } else {
#pragma unroll
                            for (int tb = 0; tb < TB; ++tb) {
                                acc[j][rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[tb], acc[j][rb][tb], 0, 0, 0);
                                acc[j][rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[tb], acc[j][rb][tb], 0, 0, 0);
                            }
                        }
                    }
                }
            }
        }
    };

    MfStage<NACC, TB, S> s0, s1;
    if (c0 < c1) fetch(c0, s0);
    RnormReq<B> rq;
    rq.request(a);
    constexpr int NT = 64 * KW * RW;
    PenPre<B, ROWS, NT> pp;  // LM head: penalty counts, in flight with the weight stream
    if constexpr (EPI == EPI_LMHEAD) pp.load(a, (int64_t)tile * ROWS);
    ResPre<B, ROWS, NT> rp;  // residual producers: residual, norm weight, bias, likewise
    if constexpr (EPI == EPI_RESNORM) rp.load(a, (int64_t)tile * ROWS);
    QkvPre<B, ROWS, NT> qp;  // QKV: the tokens' positions and KV offsets (scalar loads)
    if constexpr (EPI == EPI_QKV) qp.request(a);
    if (c0 < c1) {
        for (int c = c0;; c += 2 * S) {
            fetch(c + S, s1);
            consume(c, s0);
            if (c + S >= c1) break;
            // the 8-wave (latency-bound) launches skip the clamped re-read past their last chunk:
            // 896 x 896 at 32 tokens 11.1 -> 10.1 us; the 4-wave LM head is faster with it
            if (KW == 4 || c + 2 * S < c1) fetch(c + 2 * S, s0);
            consume(c + S, s1);
            if (c + 2 * S >= c1) break;
        }
    }

    rq.finish(a, rn);  // read by the epilogue, after the barriers below
    if constexpr (EPI == EPI_QKV) qp.rope(a, (int64_t)tile * ROWS);  // in flight through the reduction
    // D layout: lane holds token tb * 16 + lr, rows 4 * lg + v of each 16-row block. In the
    // exchange buffers a token's rows are TS = ROWS + 4 floats apart and row 4 lg + v of a block
    // sits at 4 v + lg, so the 64 lanes of one D element fall in 64 distinct banks (4 lr + lg);
    // with rows in natural order at stride ROWS the 16 lr lanes shared a bank (16-way conflicts:
    // 94K conflict cycles of 420K busy on 896 x 896 at 32 tokens).
    constexpr float FIN = FMT == BH_Q4_ROW ? 16.0f : 1.0f;  // row formats: the epilogue scales by s/16
    constexpr int TS = ROWS + 4;
    auto at = [&](int rb, int tb, int v) { return (tb * 16 + lr) * TS + rw * 64 + rb * 16 + 4 * v + lg; };
    if constexpr (ONE_ROUND) {
        // every K-split wave stores its sums in its own buffer, one barrier, then each thread adds
        // the KW partials of its comb elements in wave order (2 barriers per matrix instead of
        // the 2 log2(KW) + 2 of the halving tree)
#pragma unroll
        for (int j = 0; j < NACC; ++j) {
            float* buf = tree + kw * B * TS;
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                    for (int v = 0; v < 4; ++v) buf[at(rb, tb, v)] = acc[j][rb][tb][v];
            lds_barrier();
            // to [b][row]: row r of a 16-row block is at (r & 3) * 4 + (r >> 2) & 3
            for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
                const int b = i / ROWS, r = i % ROWS;
                const float* p = tree + b * TS + (r & ~15) + ((r & 3) << 2) + ((r >> 2) & 3);
                float t = p[0];
#pragma unroll
                for (int w = 1; w < KW; ++w) t += p[w * B * TS];
                comb[j * B * ROWS + i] = t * FIN;
            }
            lds_barrier();
        }
    } else
#pragma unroll
    for (int j = 0; j < NACC; ++j) {
        // waves [h, 2h) hand their sums to waves [0, h); wave 0 ends with the group's total
#pragma unroll
        for (int h = KW / 2; h >= 1; h >>= 1) {
            if (kw >= h && kw < 2 * h) {
                float* buf = tree + (kw - h) * B * TS;
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                        for (int v = 0; v < 4; ++v) buf[at(rb, tb, v)] = acc[j][rb][tb][v];
            }
            __syncthreads();
            if (kw < h) {
                const float* buf = tree + kw * B * TS;
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[j][rb][tb][v] += buf[at(rb, tb, v)];
            }
            __syncthreads();
        }
        if (kw == 0) {
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                    for (int v = 0; v < 4; ++v) tree[at(rb, tb, v)] = acc[j][rb][tb][v] * FIN;
        }
        __syncthreads();
        // to [b][row]: row r of a 16-row block is at (r & 3) * 4 + (r >> 2) & 3
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, r = i % ROWS;
            comb[j * B * ROWS + i] = tree[b * TS + (r & ~15) + ((r & 3) << 2) + ((r >> 2) & 3)];
        }
        __syncthreads();
    }
    if (ksw > 1 && !split_reduce<TOT>(a, comb, tile, kws)) return;
    __syncthreads();
    if constexpr (EPI == EPI_LMHEAD)
        run_lmhead_pre<FMT, B, ROWS, NT>(a, comb, comb + TOT, rn, (int64_t)tile * ROWS, pp);
    else if constexpr (EPI == EPI_RESNORM)
        run_resnorm_pre<FMT, B, ROWS, NT>(a, comb, comb + TOT, (int64_t)tile * ROWS, rp);
    else if constexpr (EPI == EPI_QKV)
        run_qkv_pre<FMT, B, ROWS, NT>(a, comb, rn, (int64_t)tile * ROWS, qp);
    else
        run_epilogue<FMT, B, EPI, ROWS>(a, comb, comb + TOT, rn, (int64_t)tile * ROWS);
}

// Waves per row group: 8 for passes of at most 512 workgroups, whose time is the chain of loads
// each wave walks (896 x 4864 at 32 tokens: 17.7 -> 13.8 us; 896-wide K unchanged), 4 for larger
// ones, where occupancy decides (the 151936-row LM head at 32 tokens: 66 us with 4, 103 with 8).
template <int FMT, int B, int EPI, int RW, int KW>
hipError_t launch_k(const GemvArgs& a, int groups, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    const int tiles = (a.n_pad + ROWS - 1) / ROWS;
    // the one-round wave-sum exchange where its KW buffers fit 64 KiB, else the halving tree
    const size_t base = (32 + (size_t)NACC * B * ROWS) * sizeof(float);
    constexpr bool ONE = (32 + (size_t)NACC * B * ROWS + (size_t)KW * B * (ROWS + 4)) * sizeof(float) <= 64 * 1024;
    const size_t shm = base + (size_t)(ONE ? KW : std::max(1, KW / 2)) * B * (ROWS + 4) * sizeof(float);
    if (shm > 64 * 1024) return hipErrorInvalidValue;
    // 8-wave launches without a K split over workgroups take two chunks per stage (all of a
    // 3.5-chunk wave's loads in flight at once: 896-wide K at 32 tokens, QKV 10.4 -> 10.0 us, O
    // 9.4 -> 8.7, gate/up 13.1 -> 12.6); split launches keep one (down 11.5 -> 11.9 with two)
    // (not the 32-token gate/up pair, whose two-chunk stages do not fit the registers)
    constexpr bool S2 = KW == 8 && !(NACC == 2 && B == 32);
    if (S2 && a.ksw == 1)
        launch_kernel((k_gemm_mf<FMT, B, EPI, RW, KW, S2 ? 2 : 1, ONE>), dim3(tiles * a.ksw, groups), dim3(64 * KW * RW), shm, st, a);
    else
        launch_kernel((k_gemm_mf<FMT, B, EPI, RW, KW, 1, ONE>), dim3(tiles * a.ksw, groups), dim3(64 * KW * RW), shm, st, a);
    return hipGetLastError();
}

template <int FMT, int B, int EPI, int RW>
hipError_t launch_t(const GemvArgs& a, int groups, hipStream_t st) {
    if constexpr (RW == 1)
        if ((a.n_pad + 63) / 64 * a.ksw * groups <= 512) return launch_k<FMT, B, EPI, RW, 8>(a, groups, st);
    return launch_k<FMT, B, EPI, RW, 4>(a, groups, st);
}

template <int FMT, int EPI, int RW>
hipError_t launch_b(const GemvArgs& a, int B, int groups, hipStream_t st) {
    return B == 32 ? launch_t<FMT, 32, EPI, RW>(a, groups, st) : launch_t<FMT, 16, EPI, RW>(a, groups, st);
}

template <int FMT>
hipError_t launch_e(int epi, const GemvArgs& a, int B, int groups, int rw, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: return launch_b<FMT, EPI_STORE, 1>(a, B, groups, st);
        case EPI_RESNORM: return launch_b<FMT, EPI_RESNORM, 1>(a, B, groups, st);
        case EPI_SILU: return launch_b<FMT, EPI_SILU, 1>(a, B, groups, st);
        case EPI_QKV:
            return rw == 2 ? launch_b<FMT, EPI_QKV, 2>(a, B, groups, st) : launch_b<FMT, EPI_QKV, 1>(a, B, groups, st);
        case EPI_LMHEAD:
            if constexpr (FMT == BH_Q4_G32) return launch_b<FMT, EPI_LMHEAD, 1>(a, B, groups, st);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemm_mf(int fmt, int epi, const GemvArgs& a, int B, int rw, hipStream_t st) {
    if (B < 16 || B % 16 || B > MF_GROUPED_MAX || a.batch < 1 || a.batch > B || a.ksw < 1 || a.n_pad % 64 ||
        rw < 1 || rw > 2 || (B > 32 && (epi == EPI_LMHEAD || a.batch <= B - 16)))
        return hipErrorInvalidValue;
    if (B > 32) {
        // 33..MF_GROUPED_MAX tokens (a short prefill chunk: a refill's prompt, or a few of them):
        // B / 16 groups of 16 tokens in one launch, each group its own split scratch region, every
        // group holding a token
        const int groups = B / 16;
        const int tiles = (a.n_pad + 64 * rw - 1) / (64 * rw);
        const int tot16 = (epi == EPI_SILU ? 2 : 1) * 16 * 64 * rw;
        if (a.ksw > 1 && (groups * tiles > SPLIT_TILES_MAX || (int64_t)groups * tiles * a.ksw * tot16 > SPLIT_PART_FLOATS))
            return hipErrorInvalidValue;
        if (fmt == BH_Q4_G32) return launch_e<BH_Q4_G32>(epi, a, 16, groups, rw, st);
        if (fmt == BH_Q4_ROW) return launch_e<BH_Q4_ROW>(epi, a, 16, groups, rw, st);
        return hipErrorInvalidValue;
    }
    // A 32-token pass whose launch leaves most CUs idle runs as two 16-token groups: twice the
    // workgroups with no reduction between them (a 16-token pass of 896 x 896 takes 7.7 us, a
    // 32-token one 10.2). Not for the LM head, whose row tiles fill the chip and whose weights
    // the second group would stream again. Each group takes its own split scratch region.
    int groups = 1;
    const int tiles = (a.n_pad + 64 * rw - 1) / (64 * rw);
    const int tot16 = (epi == EPI_SILU ? 2 : 1) * 16 * 64 * rw;
    if (B == 32 && a.batch > 16 && epi != EPI_LMHEAD && 2 * tiles * a.ksw <= 512 &&
        (a.ksw == 1 || (2 * tiles <= SPLIT_TILES_MAX && (int64_t)2 * tiles * a.ksw * tot16 <= SPLIT_PART_FLOATS))) {
        groups = 2;
        B = 16;
    }
    if (fmt == BH_Q4_G32) return launch_e<BH_Q4_G32>(epi, a, B, groups, rw, st);
    if (fmt == BH_Q4_ROW) return launch_e<BH_Q4_ROW>(epi, a, B, groups, rw, st);
    return hipErrorInvalidValue;
}

}  // namespace bh
