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
                        uint2, __builtin_amdgcn_raw_buffer_load_b64(rS[j], (int)sc_pos(n0 + rb * 16 + 4 * lg) * 2, cc * a.n_pad * 2, 0));
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

// LDS-staged variant for activations split once (a.xhl): per 32-wide K chunk the workgroup's 256
// threads load the chunk's activation hi + lo of its MT tokens and its 128 weight rows, decode the
// weights once to exact fp16 (q - 8) and store both, with the rows' fp16 group scales as f32, in
// one of two LDS stages; every wave then reads its MFMA operands from LDS. Loads are requested
// D chunks ahead into registers. Row strides are padded (80 B per weight row, 144 B per token) so
// that the lanes of one 16-byte operand read fall in distinct banks. Arithmetic and accumulation
// order are those of k_gemm_pf; the epilogue is the same.
template <int FMT, int EPI>
__global__ void __launch_bounds__(256, 2) k_gemm_pfl(const GemvArgs a) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int TBW = NACC == 2 ? 2 : 4;  // 16-token blocks per wavefront
    constexpr int MT = 2 * TBW * 16;        // tokens per workgroup
    constexpr int ROWS = PF_ROWS;
    constexpr int PH = 32;                  // tokens per epilogue phase
    constexpr int AS = 80, BS = 144;        // LDS bytes per weight row (64 + pad), per token (128 + pad)
    constexpr int A_BYTES = NACC * ROWS * AS, S_BYTES = NACC * ROWS * 4, B_BYTES = MT * BS;
    constexpr int STAGE = A_BYTES + S_BYTES + B_BYTES;
    constexpr int KB = MT * 8 / 256;        // 16-byte activation pieces per thread per chunk
    constexpr int D = NACC == 2 ? 3 : 2;    // chunks in flight in registers (as many as fit 256 VGPRs)
    static_assert((NACC * PH * ROWS + PH * ROWS) * 4 <= 2 * STAGE, "epilogue buffers fit the stages");
    __shared__ __attribute__((aligned(16))) unsigned char lds[2 * STAGE];
    __shared__ float rn[MT];
    float* comb = (float*)lds;              // after the main loop: [NACC][PH][ROWS] sums
    float* scratch = comb + NACC * PH * ROWS;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int lr = lane & 15, lg = lane >> 4;
    const int wn = wave & 1, wm = wave >> 1;
    const int mtiles = (a.batch + MT - 1) / MT;
    const int mt = blockIdx.x % mtiles, nt = blockIdx.x / mtiles;
    const int tok0 = mt * MT;
    const int C = a.C;

    // loader roles: activation pieces q = tid + k * 256 (token q / 8, 16-byte part q % 8); weight
    // row tid % 128 of matrix tid / 128 (threads below NACC * 128); clamped rows / tokens are never stored
    const __amdgpu_buffer_rsrc_t rX =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.xhl, (short)0, (int)((int64_t)a.batch * C * 128), 0x00020000);
    int vo_b[KB];
#pragma unroll
    for (int k = 0; k < KB; ++k) {
        const int q = threadIdx.x + k * 256;
        vo_b[k] = min(tok0 + q / 8, a.batch - 1) * C * 128 + (q % 8) * 16;
    }
    const bool aload = (int)threadIdx.x < NACC * ROWS;
    const int aj = NACC == 2 ? (int)threadIdx.x / ROWS : 0, arow = (int)threadIdx.x % ROWS;
    const int grow = min(nt * ROWS + arow, a.n_pad - 1);
    const __amdgpu_buffer_rsrc_t rW = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(aj == 0 ? a.W : a.W2), (short)0, C * a.n_pad * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t rS = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(aj == 0 ? a.S : a.S2), (short)0, C * a.n_pad * 2, 0x00020000);

    struct Regs {
        uint4 b[KB];
        uint4 w;
        uint32_t s;
    };
    Regs R[D];
    auto request = [&](int c, Regs& r) {
        const int cc = min(c, C - 1);
#pragma unroll
        for (int k = 0; k < KB; ++k)
            r.b[k] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rX, vo_b[k], cc * 128, 0));
        if (aload) {
            r.w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rW, grow * 16, cc * a.n_pad * 16, 0));
            if constexpr (FMT == BH_Q4_G32) r.s = __builtin_amdgcn_raw_buffer_load_b16(rS, (int)sc_pos(grow) * 2, cc * a.n_pad * 2, 0);
        }
    };
    auto store = [&](const Regs& r, int stage) {
        unsigned char* st = lds + stage * STAGE;
#pragma unroll
        for (int k = 0; k < KB; ++k) {
            const int q = threadIdx.x + k * 256;
            *(uint4*)(st + A_BYTES + S_BYTES + (q / 8) * BS + (q % 8) * 16) = r.b[k];
        }
        if (aload) {
            half8* dst = (half8*)(st + (aj * ROWS + arow) * AS);
            dst[0] = dec8(r.w.x);
            dst[1] = dec8(r.w.y);
            dst[2] = dec8(r.w.z);
            dst[3] = dec8(r.w.w);
            if constexpr (FMT == BH_Q4_G32)
                ((float*)(st + A_BYTES))[aj * ROWS + arow] = __half2float(__ushort_as_half((uint16_t)r.s));
        }
    };

    f32x4 acc[NACC][4][TBW];
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
#pragma unroll
            for (int tb = 0; tb < TBW; ++tb) acc[j][rb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto compute = [&](int stage) {
        const unsigned char* st = lds + stage * STAGE;
        half8 bh[TBW], bl[TBW];
#pragma unroll
        for (int tb = 0; tb < TBW; ++tb) {
            const unsigned char* bp = st + A_BYTES + S_BYTES + (wm * TBW * 16 + tb * 16 + lr) * BS + lg * 16;
            bh[tb] = *(const half8*)bp;
            bl[tb] = *(const half8*)(bp + 64);
        }
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) {
                const half8 av = *(const half8*)(st + (j * ROWS + wn * 64 + rb * 16 + lr) * AS + lg * 16);
                if constexpr (FMT == BH_Q4_G32) {
                    const float4 sc = *(const float4*)(st + A_BYTES + (j * ROWS + wn * 64 + rb * 16 + 4 * lg) * 4);
#pragma unroll
                    for (int tb = 0; tb < TBW; ++tb) {
                        f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[tb], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[tb], t, 0, 0, 0);
                        acc[j][rb][tb][0] = fmaf(sc.x, t[0], acc[j][rb][tb][0]);
                        acc[j][rb][tb][1] = fmaf(sc.y, t[1], acc[j][rb][tb][1]);
                        acc[j][rb][tb][2] = fmaf(sc.z, t[2], acc[j][rb][tb][2]);
                        acc[j][rb][tb][3] = fmaf(sc.w, t[3], acc[j][rb][tb][3]);
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

    // chunk c is in LDS stage c & 1 at the top of its iteration; chunks c + 1 .. c + D - 1 are in
    // flight in register slots (c + 1) % D ..; slot c % D takes chunk c + D
#pragma unroll
    for (int u = 0; u < D; ++u) request(u, R[u]);
    {
        const GemvArgs at = gemv_tokens(a, tok0, min(MT, a.batch - tok0));
        if (threadIdx.x < MT) rn[threadIdx.x] = (at.ssq_in && (int)threadIdx.x < at.batch) ? stream_rnorm(at, threadIdx.x) : 1.0f;
    }
    store(R[0], 0);
    __syncthreads();
    for (int c0 = 0; c0 < C; c0 += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const int c = c0 + u;
            if (c >= C) break;  // uniform
            request(c + D, R[u]);
            compute(c & 1);
            if (c + 1 < C) store(R[(u + 1) % D], (c + 1) & 1);
            __syncthreads();
        }
    }

    // Epilogue in phases of 32 tokens, as k_gemm_pf (comb / scratch now over the stages).
    constexpr float FIN = FMT == BH_Q4_ROW ? 16.0f : 1.0f;
    for (int ph = 0; ph < MT / PH; ++ph) {
        __syncthreads();
#pragma unroll
        for (int tb = 0; tb < TBW; ++tb) {
            const int t = wm * TBW * 16 + tb * 16;
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
        launch_kernel((k_gemm_pfl<FMT, EPI>), dim3(mtiles * ntiles), dim3(256), 0, st, a);
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
