// k_lmhead.hip — the LM head of a decode batch of 9 to 32 tokens over a 4-bit g32 vocabulary
// matrix on gfx950, as one launch of about one workgroup per CU.
//
// Reference semantics: the logits of the decode loop (matvec_mul_into over the output matrix,
// src/inference/cpu_engine.rs:1307-1444, after the final RMSNorm), the repetition penalty
// (:2984-2992) and the first-max argmax (:2993-2997), per token of the batch. Outputs are those of
// the other LM-head launches: raw logits (when y is set) and one (max, index) partial per token and
// 64-row tile for the sample kernel.
//
// Design: the vocabulary's 64-row tiles are divided evenly over the workgroups, one contiguous
// range each. A workgroup first splits its tokens' activations into the MFMA B operands — fp16
// hi + lo, in LDS, in the lane order of v_mfma_f32_16x16x32_f16 — so the activations cross the
// memory hierarchy once per workgroup instead of once per row tile; its 8 wavefronts divide the
// range's 16-row blocks (a few each per sweep) and each walks all of K for its blocks with
// LH_S chunks of weight loads in flight, so no wavefront's sums leave its registers and there is no
// cross-wave reduction. The first stages of weight loads are requested before the activations are
// staged. The epilogue scales by the norm factor, stores raw logits, applies the penalty and folds
// each token's candidates into its 64-row tile's slot in LDS with a 64-bit atomic max over an
// order-preserving key (value, then lower index): exact, and independent of the order in which the
// wavefronts arrive, so the partials equal a sequential first-max scan of the same logits.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_epilogue.h"
#include "k_mfma.h"

namespace bh {
namespace {

constexpr int LH_RBMAX = 5;    // 16-row blocks per wavefront and sweep (at most)
constexpr int LH_NW = 8;       // wavefronts per workgroup (2 per SIMD)
constexpr int LH_RBM = 5;      // blocks per sweep of the launched kernels
constexpr int LH_S = 4;        // chunks of weight loads in flight per wavefront
constexpr int LH_TMAX = 32;    // 64-row tiles per workgroup
constexpr int LH_XBYTES = 112 * 1024;

// Order-preserving key of a candidate: larger value first, then lower index. -0 is taken as +0
// so that equal floats give equal keys (the scan compares with `>`); values are never NaN here.
__device__ __forceinline__ unsigned long long lh_key(float v, int idx) {
    uint32_t u = __float_as_uint(v == 0.f ? 0.f : v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (uint32_t)(0xFFFFFFFFu - (uint32_t)idx);
}
__device__ __forceinline__ void lh_unkey(unsigned long long k, float& v, int& idx) {
    const uint32_t u = (uint32_t)(k >> 32);
    v = __uint_as_float((u & 0x80000000u) ? (u & 0x7FFFFFFFu) : ~u);
    idx = (int)(0xFFFFFFFFu - (uint32_t)k);
}

struct LhStage {
    uint32_t w[LH_RBMAX];  // dword lg of row rb * 16 + lr
    uint2 s[LH_RBMAX];     // fp16 group scales of rows rb * 16 + 4 lg .. + 3 (contiguous at sc_pos)
};

struct LhCtx {
    __amdgpu_buffer_rsrc_t rW, rS;
    int lr, lg, n_pad, C;
};

// Chunk c of blocks 0 .. RB - 1 of the rows from n0, chunk and rows clamped into the matrix (a
// block past it is never used).
template <int RB>
__device__ __forceinline__ void lh_fetch(const LhCtx& k, int n0, int c, LhStage& st) {
    c = min(c, k.C - 1);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
        const int nb = min(n0 + rb * 16, k.n_pad - 16);
        st.w[rb] = __builtin_amdgcn_raw_buffer_load_b32(k.rW, (nb + k.lr) * 16 + 4 * k.lg, c * k.n_pad * 16, CPOL_STREAM);
        st.s[rb] = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(k.rS, (int)sc_pos(nb + 4 * k.lg) * 2, c * k.n_pad * 2, CPOL_STREAM));
    }
}

// Offset past every buffer resource of this kernel: a raw buffer load there returns zero.
constexpr int LH_OOB = 0x7FFFFF00;

// One sweep of a wavefront over RB blocks from row n0 (a multiple of 16; tile t0 is the
// workgroup's first): all of K, then the epilogue. st holds chunks 0 .. LH_S - 2 on entry.
// Every load is unconditional (out-of-range lanes read zero through the buffer resources), so
// the only waits are the data dependencies themselves.
template <int TB, int RB>
__device__ __forceinline__ void lh_sweep(const GemvArgs& a, const LhCtx& k, const uint8_t* xs, const float* rn,
                                         unsigned long long* keys, int t0, int n0, LhStage (&st)[LH_S],
                                         const int (&slot)[TB]) {
    const int lane = threadIdx.x & 63;
    lh_fetch<RB>(k, n0, LH_S - 1, st[LH_S - 1]);
    // penalty counts of this lane's tokens and rows (4 consecutive rows: one 8-byte load); tokens
    // past the batch read zero. Requested when the last LH_S chunks start, whose stages are not
    // refilled: the registers come free as the weight stream ends, and the epilogue is still a
    // few chunks of work away.
    const __amdgpu_buffer_rsrc_t rP =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.pen, (short)0, a.n_slots * a.vocab * 2, 0x00020000);
    uint2 cnt[RB][TB];
    auto request_counts = [&]() {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                const int row = n0 + rb * 16 + 4 * k.lg;
                const int off = tb * 16 + k.lr < a.batch ? (slot[tb] * a.vocab + row) * 2 : LH_OOB;
                cnt[rb][tb] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rP, off, 0, 0));
            }
    };

    static_assert(RB <= 5, "a sweep spans at most two 64-row tiles");
    const Dec8K mg = dec8_consts();
    f32x4 acc[RB][TB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) acc[rb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};

    auto consume = [&](int c, const LhStage& sg) {
        half8 bh[TB], bl[TB];
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const uint8_t* b = xs + ((size_t)(c * TB + tb) * 2 * 64 + lane) * 16;
            bh[tb] = *(const half8*)b;
            bl[tb] = *(const half8*)(b + 64 * 16);
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const half8 av = dec8(sg.w[rb], mg);
            const __half2* s2 = (const __half2*)&sg.s[rb];
            const float2 sa = __half22float2(s2[0]), sb = __half22float2(s2[1]);
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bh[tb], f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                t = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bl[tb], t, 0, 0, 0);
                acc[rb][tb][0] = fmaf(sa.x, t[0], acc[rb][tb][0]);
                acc[rb][tb][1] = fmaf(sa.y, t[1], acc[rb][tb][1]);
                acc[rb][tb][2] = fmaf(sb.x, t[2], acc[rb][tb][2]);
                acc[rb][tb][3] = fmaf(sb.y, t[3], acc[rb][tb][3]);
            }
        }
    };
    // each stage is refilled with the chunk LH_S ahead right after it is consumed; the last
    // LH_S chunks are consumed without refills
    int cb = 0;
    for (; cb + LH_S < k.C; cb += LH_S) {
#pragma unroll
        for (int u = 0; u < LH_S; ++u) {
            consume(cb + u, st[u]);
            lh_fetch<RB>(k, n0, cb + u + LH_S, st[u]);
        }
    }
    request_counts();
#pragma unroll
    for (int u = 0; u < LH_S; ++u)
        if (cb + u < k.C) consume(cb + u, st[u]);

    // epilogue: lane (lr, lg) holds, per block rb and token block tb, rows n0 + rb * 16 + 4 lg + j
    // of token tb * 16 + lr. The RB <= 5 blocks span at most two 64-row tiles: each lane folds its
    // candidates per tile in registers, then one LDS max per token and tile.
    const int o = (n0 / 16) & 3;  // block offset of n0 within its tile
    const int lt0 = n0 / 64 - t0;
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        const int tok = tb * 16 + k.lr;
        if (tok >= a.batch) continue;
        const float r = rn[tok];
        unsigned long long best0 = 0, best1 = 0;
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const int row = n0 + rb * 16 + 4 * k.lg;
            float v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = acc[rb][tb][j] * r;
            if (a.y) {
                float* y = a.y + (int64_t)tok * a.ldy + row;
                if ((a.ldy & 3) == 0 && row + 3 < a.N) {
                    *(float4*)y = float4{v[0], v[1], v[2], v[3]};
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (row + j < a.N) y[j] = v[j];
                }
            }
            const uint32_t c4[4] = {cnt[rb][tb].x & 0xFFFFu, cnt[rb][tb].x >> 16, cnt[rb][tb].y & 0xFFFFu,
                                    cnt[rb][tb].y >> 16};
            unsigned long long best = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                float p = v[j];
                for (uint32_t t = 0; t < c4[j]; ++t) p = p > 0.f ? p / 1.15f : p * 1.15f;
                const bool ok = row + j < a.N && p > -INFINITY;  // NaN and -inf never win
                const unsigned long long key = ok ? lh_key(p, row + j) : lh_key(-INFINITY, 0x7fffffff);
                best = key > best ? key : best;
            }
            if (o + rb < 4) best0 = best > best0 ? best : best0;
            else best1 = best > best1 ? best : best1;
        }
        __hip_atomic_fetch_max(&keys[tok * LH_TMAX + lt0], best0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (o + RB > 4)
            __hip_atomic_fetch_max(&keys[tok * LH_TMAX + lt0 + 1], best1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
}

// NW wavefronts of at most RBM blocks per sweep; PRE: the activations come split in x_hl.
template <int TB, int NW, int RBM, bool PRE>
__global__ void __launch_bounds__(64 * NW) k_lmhead_mf(const GemvArgs a) {
    static_assert(RBM >= 1 && RBM <= LH_RBMAX, "blocks per sweep");
    constexpr int NTOK = 16 * TB;
    __shared__ __attribute__((aligned(16))) uint8_t xs[LH_XBYTES];
    __shared__ unsigned long long keys[NTOK * LH_TMAX];
    __shared__ float rn[32];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    LhCtx k;
    k.lr = lane & 15;
    k.lg = lane >> 4;
    k.n_pad = a.n_pad;
    k.C = a.C;
    k.rW = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.C * a.n_pad * 16, 0x00020000);
    k.rS = __builtin_amdgcn_make_buffer_rsrc((void*)a.S, (short)0, a.C * a.n_pad * 2, 0x00020000);

    // Activations first (the staging waits on them), as MFMA B operands: chunk c, token block tb,
    // hi (h = 0) or lo (h = 1) is 64 lanes of 16 bytes at ((c * TB + tb) * 2 + h) * 1 KiB, lane
    // 16 lg + lr holding token tb * 16 + lr, k = c * 32 + 8 lg .. + 7 in the kperm order of dec8.
    // Wavefront w stages chunks w, w + NW, ...; tokens past the batch read zero.
    // With the split already in x_hl (token-major, from the producer's epilogue) each 1 KiB
    // block is one load straight into LDS, lane l's 16 bytes landing at l * 16.
    constexpr int XR = (LH_XBYTES / (TB * 2048) + NW - 1) / NW;  // chunk rounds per wavefront
    float4 xv[PRE ? 1 : XR][TB][2];
    if constexpr (PRE) {
        const __amdgpu_buffer_rsrc_t rH =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.x_hl, (short)0, a.batch * a.C * 128, 0x00020000);
#pragma unroll
        for (int r = 0; r < XR; ++r)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                const int c = wave + r * NW;
                if (c < a.C) {
#pragma unroll
                    for (int h = 0; h < 2; ++h)
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            rH, (__attribute__((address_space(3))) void*)(xs + (size_t)((c * TB + tb) * 2 + h) * 1024), 16,
                            ((tb * 16 + k.lr) * a.C + c) * 128 + (k.lg * 8 + h * 32) * 2, 0, 0, 0);
                }
            }
    } else {
        const __amdgpu_buffer_rsrc_t rX =
            __builtin_amdgcn_make_buffer_rsrc((void*)a.x, (short)0, a.batch * (int)a.ldx * 4, 0x00020000);
#pragma unroll
        for (int r = 0; r < XR; ++r)
#pragma unroll
            for (int tb = 0; tb < TB; ++tb) {
                const int c = wave + r * NW;
                const int off = c < a.C ? ((tb * 16 + k.lr) * (int)a.ldx + c * 32 + k.lg * 8) * 4 : LH_OOB;
                xv[PRE ? 0 : r][tb][0] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rX, off, 0, 0));
                xv[PRE ? 0 : r][tb][1] =
                    __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rX, off + 16, 0, 0));
            }
    }
    RnormReq<32> rq;
    rq.request(a);

    // this workgroup's 64-row tiles [t0, t1) and this wavefront's 16-row blocks [b0, b1) of them
    const int T = a.n_pad / 64, G = gridDim.x;
    const int t0 = (int)((int64_t)blockIdx.x * T / G), t1 = (int)((int64_t)(blockIdx.x + 1) * T / G);
    const int R = (t1 - t0) * 4;
    const int b0 = wave * R / NW, b1 = (wave + 1) * R / NW;
    const int n0 = t0 * 64 + b0 * 16;

    // first stages of the first sweep (RBM blocks: a sweep of fewer leaves the last ones unused)
    LhStage st[LH_S];
#pragma unroll
    for (int u = 0; u < LH_S - 1; ++u) lh_fetch<RBM>(k, n0, u, st[u]);
    // slots of this lane's tokens
    const __amdgpu_buffer_rsrc_t rQ = __builtin_amdgcn_make_buffer_rsrc((void*)a.slot, (short)0, a.batch * 4, 0x00020000);
    int slot[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) slot[tb] = (int)__builtin_amdgcn_raw_buffer_load_b32(rQ, (tb * 16 + k.lr) * 4, 0, 0);

    if constexpr (PRE) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's loads into LDS have landed
    } else {
#pragma unroll
    for (int r = 0; r < XR; ++r)
#pragma unroll
        for (int tb = 0; tb < TB; ++tb) {
            const int c = wave + r * NW;
            if (c < a.C) {
                half8 hi, lo;
                split8(xv[PRE ? 0 : r][tb][0], xv[PRE ? 0 : r][tb][1], hi, lo);
                uint8_t* d = xs + ((size_t)(c * TB + tb) * 2 * 64 + lane) * 16;
                *(half8*)d = hi;
                *(half8*)(d + 64 * 16) = lo;
            }
        }
    }
    for (int i = threadIdx.x; i < NTOK * LH_TMAX; i += blockDim.x) keys[i] = 0ull;
    rq.finish(a, rn);
    lds_barrier();  // the weight loads stay in flight

    for (int s0 = b0; s0 < b1; s0 += RBM) {
        const int nb = min(RBM, b1 - s0);
        const int ns = t0 * 64 + s0 * 16;
        if (s0 != b0) {
#pragma unroll
            for (int u = 0; u < LH_S - 1; ++u) lh_fetch<RBM>(k, ns, u, st[u]);
        }
        if (nb == RBM) lh_sweep<TB, RBM>(a, k, xs, rn, keys, t0, ns, st, slot);
        else if (RBM > 1 && nb == RBM - 1) lh_sweep<TB, (RBM > 1 ? RBM - 1 : 1)>(a, k, xs, rn, keys, t0, ns, st, slot);
        else if (nb == 1) lh_sweep<TB, 1>(a, k, xs, rn, keys, t0, ns, st, slot);
        else if (nb == 2) lh_sweep<TB, 2>(a, k, xs, rn, keys, t0, ns, st, slot);
        else if (nb == 3) lh_sweep<TB, 3>(a, k, xs, rn, keys, t0, ns, st, slot);
        else lh_sweep<TB, 4>(a, k, xs, rn, keys, t0, ns, st, slot);
    }
    lds_barrier();  // the keys are complete; logit stores need not be

    // one partial per token and tile
    const int nt = t1 - t0;
    for (int i = threadIdx.x; i < NTOK * nt; i += blockDim.x) {
        const int m = i / nt, lt = i % nt;
        if (m >= a.batch) continue;
        float v;
        int idx;
        lh_unkey(keys[m * LH_TMAX + lt], v, idx);
        a.part_val[(int64_t)m * T + t0 + lt] = v;
        a.part_idx[(int64_t)m * T + t0 + lt] = idx;
    }
}

}  // namespace

bool lmhead_mf_fits(const GemvArgs& a, int n_cu) {
    const int T = a.n_pad / 64;
    const int G = std::max(std::min(n_cu, T), (T + LH_TMAX - 1) / LH_TMAX);
    const int tb = a.batch > 16 ? 2 : 1;
    return a.batch >= 1 && a.batch <= 32 && a.n_pad % 64 == 0 && a.n_pad >= LH_RBMAX * 16 && a.C >= 1 &&
           (size_t)a.C * tb * 2 * 1024 <= (size_t)LH_XBYTES && (T + G - 1) / G <= LH_TMAX && a.ldx % 4 == 0 &&
           a.vocab % 4 == 0 && a.part_val && a.part_idx && a.slot && a.pen && a.n_slots > 0 &&
           (int64_t)a.n_slots * a.vocab * 2 < LH_OOB && (int64_t)a.batch * a.ldx * 4 < LH_OOB &&
           (int64_t)a.C * a.n_pad * 16 < LH_OOB && (!a.x_hl || (int64_t)a.batch * a.C * 128 < LH_OOB);
}

hipError_t launch_lmhead_mf(const GemvArgs& a, int n_cu, hipStream_t st) {
    if (!lmhead_mf_fits(a, n_cu)) return hipErrorInvalidValue;
    const int T = a.n_pad / 64;
    const int G = std::max(std::min(n_cu, T), (T + LH_TMAX - 1) / LH_TMAX);
    const dim3 g(G), b(64 * LH_NW);
    if (a.batch > 16) {
        if (a.x_hl) launch_kernel(k_lmhead_mf<2, LH_NW, LH_RBM, true>, g, b, 0, st, a);
        else launch_kernel(k_lmhead_mf<2, LH_NW, LH_RBM, false>, g, b, 0, st, a);
    } else {
        if (a.x_hl) launch_kernel(k_lmhead_mf<1, LH_NW, LH_RBM, true>, g, b, 0, st, a);
        else launch_kernel(k_lmhead_mf<1, LH_NW, LH_RBM, false>, g, b, 0, st, a);
    }
    return hipGetLastError();
}

}  // namespace bh
