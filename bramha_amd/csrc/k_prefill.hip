// k_prefill.hip — tiled MFMA GEMM over 4-bit weights for prefill chunks on gfx950.
//
// Reference semantics: gemm_cpu / fused_qkv_gemm (src/inference/cpu_engine.rs:565-912,
// 3325-3339), the prefill projections: Y[m][n] = sum_k W[n][k] X[m][k] for every token m of a
// chunk, here with the chunk's epilogue (RMSNorm factor, bias, RoPE + KV append, SiLU gate,
// residual add + next norm inputs) fused.
//
// Design: a workgroup of 4 wavefronts owns a 128-row by 128-token output tile (64 tokens when
// it carries both gate and up accumulators) and walks all of K; wavefront (wn, wm) owns rows
// 64 wn .. 64 wn + 63 and one half of the tokens, as 4 x TBW blocks of 16 x 16. Per 32-wide K
// chunk a wavefront decodes its 4 row blocks from one dword of nibbles per lane (exact fp16
// q - 8), splits each token block's f32 activations into fp16 hi + lo once, and runs
// 2 * 4 * TBW v_mfma_f32_16x16x32_f16 — each weight operand serves TBW token blocks and each
// activation operand 4 row blocks, so the decode and split costs are amortised over the tile.
// The group-32 fp16 scale multiplies each chunk's MFMA result per row (exactly the reference's
// dequantized weight (q - 8) * s, with the product formed in f32). Operands come straight from
// global memory with raw buffer loads one chunk ahead (no LDS staging: a chunk's weight tile is
// 2 KiB and its activation tile 16 KiB, both re-read by the sibling wavefronts through L1/L2).
// The epilogue runs in phases of 32 tokens through LDS with the decode kernels' epilogues.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_epilogue.h"
#include "k_mfma.h"

namespace bh {
namespace {

constexpr int PF_ROWS = 128;

template <int NACC, int TBW>
struct PfStage {
    uint32_t w[NACC][4];  // [matrix][row block]: dword lg of row rb * 16 + lr
    uint2 s[NACC][4];     // fp16 group scales of rows rb * 16 + 4 lg .. + 3
    uint4 x[TBW][2];      // token tb * 16 + lr, k = 8 lg .. + 7: f32, or (PRE) fp16 hi and lo
};

// The activations of a prefill pass split once into the MFMA B operands: for token m and chunk c,
// 64 fp16 at (m * C + c) * 64: hi of k = 8 lg + kperm(s) at 8 lg + s, lo at 32 + 8 lg + s (split8,
// the values every workgroup would compute). One thread per 8 elements.
__global__ void __launch_bounds__(256) k_split_act(const float* __restrict__ x, int64_t ldx, int M, int C,
                                                   uint16_t* __restrict__ xhl) {
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;  // (m, c, lg)
    if (g >= (int64_t)M * C * 4) return;
    const int lg = (int)(g & 3);
    const int64_t mc = g >> 2;
    const int64_t m = mc / C, c = mc % C;
    const float4* src = (const float4*)(x + m * ldx + c * 32 + lg * 8);
    half8 hi, lo;
    split8(src[0], src[1], hi, lo);
    uint4* dst = (uint4*)(xhl + mc * 64 + lg * 8);
    dst[0] = __builtin_bit_cast(uint4, hi);
    dst[4] = __builtin_bit_cast(uint4, lo);
}

template <int FMT, int EPI, bool PRE>
__global__ void __launch_bounds__(256) k_gemm_pf(const GemvArgs a) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int TBW = NACC == 2 ? 2 : 4;  // 16-token blocks per wavefront
    constexpr int MT = 2 * TBW * 16;        // tokens per workgroup
    constexpr int ROWS = PF_ROWS;
    constexpr int PH = 32;                  // tokens per epilogue phase
    __shared__ float rn[MT];
    __shared__ float comb[NACC * PH * ROWS];
    __shared__ float scratch[PH * ROWS];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lr = lane & 15, lg = lane >> 4;
    const int wn = wave & 1, wm = wave >> 1;
    const int mtiles = (a.batch + MT - 1) / MT;
    const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const int tok0 = mt * MT;                      // first token of the workgroup
    const int wtok0 = tok0 + wm * TBW * 16;        // first token of this wavefront
    // this wavefront's 64 rows; a group past the padded matrix re-reads the last one (never stored)
    const int n0 = min(nt * ROWS + wn * 64, a.n_pad - 64);

    __amdgpu_buffer_rsrc_t rW[NACC], rS[NACC];
    rW[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.C * a.n_pad * 16, 0x00020000);
    if constexpr (NACC == 2) rW[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W2, (short)0, a.C * a.n_pad * 16, 0x00020000);
    if constexpr (FMT == BH_Q4_G32) {
        rS[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S, (short)0, a.C * a.n_pad * 2, 0x00020000);
        if constexpr (NACC == 2)
            rS[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S2, (short)0, a.C * a.n_pad * 2, 0x00020000);
    }
    // f32 rows of ldx floats, or (PRE) rows of C * 64 fp16; either way 128 bytes per chunk
    const __amdgpu_buffer_rsrc_t rX =
        PRE ? __builtin_amdgcn_make_buffer_rsrc((void*)a.xhl, (short)0, (int)((int64_t)a.batch * a.C * 128), 0x00020000)
            : __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, (int)((int64_t)a.batch * a.ldx * 4), 0x00020000);
    // token of block tb for this lane, clamped into the chunk (rows past it are never stored)
    int vo_x[TBW];
#pragma unroll
    for (int tb = 0; tb < TBW; ++tb) {
        const int tok = min(wtok0 + tb * 16 + lr, a.batch - 1);
        vo_x[tb] = PRE ? tok * a.C * 128 + 16 * lg : (tok * (int)a.ldx + 8 * lg) * 4;
    }

    auto fetch = [&](int c, PfStage<NACC, TBW>& st) {
        const int cc = min(c, a.C - 1);
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                st.w[j][rb] = __builtin_amdgcn_raw_buffer_load_b32(rW[j], (n0 + rb * 16 + lr) * 16 + 4 * lg,
                                                                   cc * a.n_pad * 16, 0);
                if constexpr (FMT == BH_Q4_G32)
                    st.s[j][rb] = __builtin_bit_cast(
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(rS[j], (n0 + rb * 16 + 4 * lg) * 2, cc * a.n_pad * 2, 0));
            }
#pragma unroll
        for (int tb = 0; tb < TBW; ++tb)
#pragma unroll
            for (int h = 0; h < 2; ++h)  // f32: the two halves of 8 values; PRE: hi at +0, lo at +64 bytes
                st.x[tb][h] = __builtin_bit_cast(
                    uint4, __builtin_amdgcn_raw_buffer_load_b128(rX, vo_x[tb] + h * (PRE ? 64 : 16), cc * 128, 0));
    };

    f32x4 acc[NACC][4][TBW];
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int tb = 0; tb < TBW; ++tb) acc[j][rb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](const PfStage<NACC, TBW>& st) {
        half8 bh[TBW], bl[TBW];
#pragma unroll
        for (int tb = 0; tb < TBW; ++tb) {
            if constexpr (PRE) {
                bh[tb] = __builtin_bit_cast(half8, st.x[tb][0]);
                bl[tb] = __builtin_bit_cast(half8, st.x[tb][1]);
            } else {
                split8(__builtin_bit_cast(float4, st.x[tb][0]), __builtin_bit_cast(float4, st.x[tb][1]), bh[tb], bl[tb]);
            }
        }
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const half8 av = dec8(st.w[j][rb]);
                if constexpr (FMT == BH_Q4_G32) {
                    const __half2* s2 = (const __half2*)&st.s[j][rb];
                    const float2 sa = __half22float2(s2[0]), sb = __half22float2(s2[1]);
#pragma unroll
                    for (int tb = 0; tb < TBW; ++tb) {
                        f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[tb], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[tb], t, 0, 0, 0);
                        acc[j][rb][tb][0] = fmaf(sa.x, t[0], acc[j][rb][tb][0]);
                        acc[j][rb][tb][1] = fmaf(sa.y, t[1], acc[j][rb][tb][1]);
                        acc[j][rb][tb][2] = fmaf(sb.x, t[2], acc[j][rb][tb][2]);
                        acc[j][rb][tb][3] = fmaf(sb.y, t[3], acc[j][rb][tb][3]);
                    }
                } else {
#pragma unroll
                    for (int tb = 0; tb < TBW; ++tb) {
                        acc[j][rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[tb], acc[j][rb][tb], 0, 0, 0);
                        acc[j][rb][tb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[tb], acc[j][rb][tb], 0, 0, 0);
                    }
                }
            }
    };

    {
        PfStage<NACC, TBW> s0, s1;
        fetch(0, s0);
        // per-token norm factors of the workgroup's tokens
        const GemvArgs at = gemv_tokens(a, tok0, min(MT, a.batch - tok0));
        if (threadIdx.x < MT) rn[threadIdx.x] = (at.ssq_in && (int)threadIdx.x < at.batch) ? stream_rnorm(at, threadIdx.x) : 1.0f;
        for (int c = 0;; c += 2) {
            fetch(c + 1, s1);
            consume(s0);
            if (c + 1 >= a.C) break;
            fetch(c + 2, s0);
            consume(s1);
            if (c + 2 >= a.C) break;
        }
    }

    // Epilogue in phases of 32 tokens: the wavefronts holding them write their sums into LDS
    // (D layout: lane holds token tb * 16 + lr, rows 4 lg + v of each 16-row block).
    constexpr float FIN = FMT == BH_Q4_ROW ? 16.0f : 1.0f;  // row formats: the epilogue scales by s/16
    for (int ph = 0; ph < MT / PH; ++ph) {
        __syncthreads();  // the previous phase's epilogue has finished with comb/scratch
#pragma unroll
        for (int tb = 0; tb < TBW; ++tb) {
            const int t = wm * TBW * 16 + tb * 16;  // workgroup-relative first token of the block
            if (t / PH != ph) continue;
#pragma unroll
            for (int j = 0; j < NACC; ++j)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        comb[(j * PH + (t % PH) + lr) * ROWS + wn * 64 + rb * 16 + 4 * lg + v] = acc[j][rb][tb][v] * FIN;
        }
        __syncthreads();
        const int b0 = tok0 + ph * PH;
        if (b0 >= a.batch) break;  // uniform
        const GemvArgs ap = gemv_tokens(a, b0, min(PH, a.batch - b0));
        run_epilogue<FMT, PH, EPI, ROWS>(ap, comb, scratch, rn + ph * PH, (int64_t)nt * ROWS);
    }
}

template <int FMT, int EPI>
hipError_t launch_t(const GemvArgs& a, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int MT = NACC == 2 ? 64 : 128;
    const int mtiles = (a.batch + MT - 1) / MT;
    const int ntiles = (a.n_pad + PF_ROWS - 1) / PF_ROWS;
    if (a.xhl) {
        // split the activations once (the VALU work of the in-kernel split, ~half of the inner
        // loop's, is otherwise repeated by every row tile)
        const int64_t groups = (int64_t)a.batch * a.C * 4;
        launch_kernel(k_split_act, dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, a.x, a.ldx, a.batch, a.C,
                      a.xhl);
        launch_kernel((k_gemm_pf<FMT, EPI, true>), dim3(mtiles * ntiles), dim3(256), 0, st, a);
    } else {
        launch_kernel((k_gemm_pf<FMT, EPI, false>), dim3(mtiles * ntiles), dim3(256), 0, st, a);
    }
    return hipGetLastError();
}

template <int FMT>
hipError_t launch_e(int epi, const GemvArgs& a, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: return launch_t<FMT, EPI_STORE>(a, st);
        case EPI_RESNORM: return launch_t<FMT, EPI_RESNORM>(a, st);
        case EPI_SILU: return launch_t<FMT, EPI_SILU>(a, st);
        case EPI_QKV: return launch_t<FMT, EPI_QKV>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t launch_gemm_pf(int fmt, int epi, const GemvArgs& a, hipStream_t st) {
    if (a.batch <= 0 || a.n_pad % 64 || a.C <= 0 || a.ksw > 1) return hipErrorInvalidValue;
    // byte offsets of the buffer loads are 32-bit
    if ((int64_t)a.C * a.n_pad * 16 >= (1ll << 31) || (int64_t)a.batch * a.ldx * 4 >= (1ll << 31) ||
        (int64_t)a.batch * a.C * 128 >= (1ll << 31))
        return hipErrorInvalidValue;
    if (a.xhl && a.ldx % 4) return hipErrorInvalidValue;  // the split pass loads 16 bytes at a time
    if (epi == EPI_QKV) {
        // a 128-row tile holds whole heads: hd 64, or hd 128 with 128-aligned sections
        if (!(a.hd == 64 || (a.hd == 128 && a.qd % 128 == 0 && a.kd % 128 == 0))) return hipErrorInvalidValue;
    }
    if (fmt == BH_Q4_G32) return launch_e<BH_Q4_G32>(epi, a, st);
    if (fmt == BH_Q4_ROW) return launch_e<BH_Q4_ROW>(epi, a, st);
    return hipErrorInvalidValue;
}

}  // namespace bh
