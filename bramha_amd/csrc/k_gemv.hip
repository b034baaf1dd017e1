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

// ---- MFMA path (16 or 32 tokens per pass, 4-bit weights) ----
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One dword of a Q4 chunk (8 weights) -> 8 exact fp16 values q - 8 for the A operand of
// v_mfma_f32_16x16x32_f16. Register pair j holds (nibble j, nibble j + 4): 1024 + q is
// formed in the fp16 mantissa and 1032 subtracted. Nibble t is element t ^ 1 of the 8
// (the high nibble of a byte is the even element), so K slot s of the lane holds element
// kperm(s) = {1, 5, 0, 4, 3, 7, 2, 6}[s]; the activations use the same permutation (the MFMA
// sum over K is order-free). A function, not a table, so that every index folds at compile time.
__host__ __device__ constexpr int kperm(int s) { return ((s >> 1) ^ 1) + 4 * (s & 1); }

__device__ __forceinline__ half8 dec8(uint32_t w) {
    const half2v off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    half8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t p = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        const half2v h = __builtin_bit_cast(half2v, p) + off;
        r[2 * j] = h.x;
        r[2 * j + 1] = h.y;
    }
    return r;
}

// f32 activations -> fp16 hi + lo (hi + lo carries ~22 bits of the f32 mantissa).
__device__ __forceinline__ void split8(const float4& x0, const float4& x1, half8& hi, half8& lo) {
    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const float f = xv[kperm(s)];
        const _Float16 h = (_Float16)f;
        hi[s] = h;
        lo[s] = (_Float16)(f - (float)h);
    }
}

// One pipeline stage of the MFMA loop: a chunk's weight dwords, group scales and activations.
template <int NACC, int TB>
struct MfStage {
    uint32_t aw[NACC][4];
    uint2 sw[NACC][4];
    float4 xv[TB][2];
};

template <int FMT, int NACC, int TB>
__device__ __forceinline__ void mf_fetch(const GemvArgs& a, const uint32_t* const (&Wd)[NACC],
                                         const __half* const (&Sh)[NACC], int c, int64_t n0, int lr, int lg,
                                         MfStage<NACC, TB>& st) {
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            st.aw[j][rb] = Wd[j][((int64_t)c * a.n_pad + n0 + rb * 16 + lr) * 4 + lg];
            if constexpr (FMT == BH_Q4_G32)
                st.sw[j][rb] = *(const uint2*)(Sh[j] + (int64_t)c * a.n_pad + n0 + rb * 16 + 4 * lg);
        }
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) {
        // rows past the batch read the last row (in bounds) and are zeroed by value selects,
        // which keeps the stage in registers (a pointer select would move it to scratch)
        const int m = tb * 16 + lr;
        const bool ok = m < a.batch;
        const float4* xp = (const float4*)(a.x + (int64_t)(ok ? m : a.batch - 1) * a.ldx + c * 32 + 8 * lg);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const float4 v = xp[h];
            st.xv[tb][h] = make_float4(ok ? v.x : 0.f, ok ? v.y : 0.f, ok ? v.z : 0.f, ok ? v.w : 0.f);
        }
    }
}

template <int FMT, int NACC, int TB>
__device__ __forceinline__ void mf_consume(const MfStage<NACC, TB>& st, f32x4 (&acc)[NACC][4][TB]) {
    half8 bh[TB], bl[TB];
#pragma unroll
    for (int tb = 0; tb < TB; ++tb) split8(st.xv[tb][0], st.xv[tb][1], bh[tb], bl[tb]);
#pragma unroll
    for (int j = 0; j < NACC; ++j) {
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            const half8 av = dec8(st.aw[j][rb]);
            if constexpr (FMT == BH_Q4_G32) {
                const __half2* s2 = (const __half2*)&st.sw[j][rb];
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

// Per-token RMSNorm factors of a normalized residual-stream input (1 without one), into LDS.
template <int B>
__device__ __forceinline__ void load_rnorm(const GemvArgs& a, float* rn) {
    if (threadIdx.x < B) rn[threadIdx.x] = (a.ssq_in && (int)threadIdx.x < a.batch) ? stream_rnorm(a, threadIdx.x) : 1.0f;
}

template <int FMT, int B, int EPI, int RW, int U>
__global__ void __launch_bounds__(B >= 16 ? 256 : 1024) k_gemv(const GemvArgs a) {
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
    const uint4* Wp[NACC];
    const uint16_t* Sp[NACC];
    Wp[0] = (const uint4*)a.W + nl;
    Sp[0] = (const uint16_t*)a.S + nl;
    if constexpr (NACC == 2) {
        Wp[1] = (const uint4*)a.W2 + nl;
        Sp[1] = (const uint16_t*)a.S2 + nl;
    }

    if constexpr (B >= 16) {
        static_assert(FMT == BH_Q4_G32 || FMT == BH_Q4_ROW, "MFMA path is for 4-bit weights");
        constexpr int TB = B / 16;
        const int lr = lane & 15, lg = lane >> 4;
        const int64_t n0 = (int64_t)tile * ROWS + rw * 64;
        f32x4 acc[NACC][4][TB];
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int tb = 0; tb < TB; ++tb) acc[j][rb][tb] = f32x4{0.f, 0.f, 0.f, 0.f};
        const uint32_t* Wd[NACC];
        Wd[0] = (const uint32_t*)a.W;
        if constexpr (NACC == 2) Wd[1] = (const uint32_t*)a.W2;
        const __half* Sh[NACC];
        Sh[0] = (const __half*)a.S;
        if constexpr (NACC == 2) Sh[1] = (const __half*)a.S2;
        const bool work = n0 < a.n_pad && c0 < c1;
        // two stages in flight; the refetch past the end re-reads the last chunk (in bounds, unused)
        MfStage<NACC, TB> s0, s1;
        if (work) mf_fetch<FMT>(a, Wd, Sh, c0, n0, lr, lg, s0);
        load_rnorm<B>(a, rn);
        if (work) {
            int c = c0;
            for (; c + 1 < c1; c += 2) {
                mf_fetch<FMT>(a, Wd, Sh, c + 1, n0, lr, lg, s1);
                mf_consume<FMT>(s0, acc);
                mf_fetch<FMT>(a, Wd, Sh, min(c + 2, c1 - 1), n0, lr, lg, s0);
                mf_consume<FMT>(s1, acc);
            }
            if (c < c1) mf_consume<FMT>(s0, acc);
        }
        // D layout of 16x16 MFMA: lane holds column lr (token), rows 4*lg + v
        constexpr float FIN = FMT == BH_Q4_ROW ? 16.0f : 1.0f;  // row formats: the epilogue scales by s/16
#pragma unroll
        for (int j = 0; j < NACC; ++j)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb)
#pragma unroll
                for (int tb = 0; tb < TB; ++tb)
#pragma unroll
                    for (int v = 0; v < 4; ++v)
                        comb[kw * TOT + (j * B + tb * 16 + lr) * ROWS + rw * 64 + rb * 16 + 4 * lg + v] =
                            acc[j][rb][tb][v] * FIN;
    } else {
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
                    q[j][u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rW[j], vo_w, cc * a.n_pad * 16, 0));
                    if constexpr (FMT == BH_Q4_G32) s[j][u] = __builtin_amdgcn_raw_buffer_load_b16(rS[j], vo_s, cc * a.n_pad * 2, 0);
                }
            }
        };
        if (c0 < c1) fetch(c0, q0, s0);
        load_rnorm<B>(a, rn);

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
    }

    // ---- combine the K-split partial sums in a fixed order ----
    __syncthreads();
    for (int i = threadIdx.x; i < TOT; i += blockDim.x) {
        float sum = comb[i];
        for (int w = 1; w < ksplit; ++w) sum += comb[w * TOT + i];
        comb[i] = sum;
    }
    if (ksw > 1) {
        // K split over workgroups: publish this split's sums, and let the tile's last workgroup
        // add all splits in split order and run the epilogue. The sums are published with
        // agent-scope atomic exchanges and read back with agent-scope atomic loads, which are
        // performed at the device-coherent level; the exchanges have returned (the barrier's wait)
        // before the arrival count is taken, so the last arrival reads every split's sums without
        // a cache-wide writeback or invalidate.
        __shared__ int s_last;
        float* mine = a.part + (int64_t)(tile * ksw + kws) * TOT;
        float sink = 0.f;
        for (int i = threadIdx.x; i < TOT; i += blockDim.x)
            sink += __hip_atomic_exchange(&mine[i], comb[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("" ::"v"(sink));  // the returned values are consumed: the exchanges have completed
        __syncthreads();
        if (threadIdx.x == 0)
            s_last = __hip_atomic_fetch_add(&a.tile_cnt[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ksw - 1;
        __syncthreads();
        if (!s_last) return;
        const float* all = a.part + (int64_t)tile * ksw * TOT;
        for (int i = threadIdx.x; i < TOT; i += blockDim.x) {
            // all splits' loads in flight at once (index clamped in bounds), added in split order
            float v[MAX_KSW];
#pragma unroll
            for (int k = 0; k < MAX_KSW; ++k)
                v[k] = __hip_atomic_load(&all[(int64_t)min(k, ksw - 1) * TOT + i], __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
            float sum = 0.f;
#pragma unroll
            for (int k = 0; k < MAX_KSW; ++k) sum += k < ksw ? v[k] : 0.f;
            comb[i] = sum;
        }
        if (threadIdx.x == 0) __hip_atomic_store(&a.tile_cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    run_epilogue<FMT, B, EPI, ROWS>(a, comb, comb + TOT, rn, (int64_t)tile * ROWS);
}

template <int FMT, int B, int EPI, int RW, int U>
hipError_t launch_one(const GemvArgs& a, int ksplit, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    const int tiles = (a.n_pad + ROWS - 1) / ROWS * a.ksw;
    size_t shm = (size_t)ksplit * NACC * B * ROWS * sizeof(float);
    if (EPI == EPI_LMHEAD || EPI == EPI_RESNORM) shm = std::max(shm, (size_t)(NACC * B * ROWS + B * ROWS) * sizeof(float));
    shm += 32 * sizeof(float);
    launch_kernel((k_gemv<FMT, B, EPI, RW, U>), dim3(tiles), dim3(64 * RW * ksplit), shm, st, a);
    return hipGetLastError();
}

// Stage depth from the chunks each wave streams (cpw): a single stage covers short ranges,
// deep stages keep long ones in flight. NACC == 2 doubles the loads per chunk.
template <int FMT, int EPI, int RW>
hipError_t launch_b(const GemvArgs& a, int B, int ksplit, int cpw, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    if constexpr (FMT == BH_Q4_G32 || FMT == BH_Q4_ROW) {
        if (B == 32) return launch_one<FMT, 32, EPI, RW, 1>(a, ksplit, st);
        if (B == 16) return launch_one<FMT, 16, EPI, RW, 1>(a, ksplit, st);
    }
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

// Waves per workgroup along K: aim for ~8 waves per CU and >= 2 chunks per wave
// (MFMA passes: at most 256 threads per workgroup); the combine area stays under 60 KB.
static int waves_per_tile(int tiles, int rw, int C, int nacc, int B) {
    int ks = ((B >= 16 ? 4096 : 2048) + tiles * rw - 1) / (tiles * rw);
    ks = std::max(1, std::min({ks, (B >= 16 ? 4 : 16) / rw, std::max(1, C / 2)}));
    while (ks > 1 && (size_t)ks * nacc * B * 64 * rw * 4 > 60 * 1024) --ks;
    return ks;
}

// Workgroups per row tile for a K-split GEMV: enough for about one workgroup per CU (256),
// each streaming at least `min_chunks` chunks, at most MAX_KSW.
int gemv_splits(int tiles, int C, int min_chunks) {
    const int ksw = 256 / std::max(tiles, 1);
    return std::max(1, std::min({ksw, MAX_KSW, std::max(1, C / std::max(min_chunks, 1))}));
}

// Splits the batch into passes: MFMA passes of 32 or 16 rows for 4-bit weights, VALU passes
// of at most 8 rows otherwise.
hipError_t launch_gemv(int fmt, int epi, const GemvArgs& a0, hipStream_t st) {
    const int rw = (epi == EPI_QKV && a0.hd > 64) ? a0.hd / 64 : 1;
    if (rw > 2) return hipErrorInvalidValue;
    if (a0.ssq_in && a0.batch > 0 && (a0.ssq_tiles <= 0 || a0.norm_n <= 0.f)) return hipErrorInvalidValue;
    if (epi == EPI_RESNORM && (!a0.xw_out || !a0.wnext || !a0.ssq_out || a0.ssq_tiles != a0.n_pad / 64))
        return hipErrorInvalidValue;
    if (a0.ksw < 1 || a0.ksw > MAX_KSW || (a0.ksw > 1 && (!a0.part || !a0.tile_cnt))) return hipErrorInvalidValue;
    const int ksw = a0.ksw;
    const int nacc = epi == EPI_SILU ? 2 : 1;
    const int tiles = (a0.n_pad + 64 * rw - 1) / (64 * rw);
    int b0 = 0;
    while (b0 < a0.batch) {
        const int rem = a0.batch - b0;
        const bool mf = (fmt == BH_Q4_G32 || fmt == BH_Q4_ROW) && rem >= 16;
        const int B = mf ? (rem >= 32 ? 32 : 16) : (rem >= 8 ? 8 : (rem >= 4 ? 4 : (rem >= 2 ? 2 : 1)));
        const int ks = waves_per_tile(tiles * ksw, rw, (a0.C + ksw - 1) / ksw, nacc, B);
        GemvArgs a = a0;
        a.batch = std::min(B, rem);
        a.x = a0.x + (int64_t)b0 * a0.ldx;
        a.y = a0.y + (int64_t)b0 * a0.ldy;
        if (a0.xw_out) a.xw_out = a0.xw_out + (int64_t)b0 * a0.ldy;
        if (a0.ssq_in) a.ssq_in = a0.ssq_in + (int64_t)b0 * a0.ssq_tiles;
        if (a0.ssq_out) a.ssq_out = a0.ssq_out + (int64_t)b0 * a0.ssq_tiles;
        if (a0.pos) a.pos = a0.pos + b0;
        if (a0.boff) a.boff = a0.boff + b0;
        if (a0.slot) a.slot = a0.slot + b0;
        const int tiles64 = (a0.n_pad + 63) / 64;
        if (a0.part_val) a.part_val = a0.part_val + (int64_t)b0 * tiles64;
        if (a0.part_idx) a.part_idx = a0.part_idx + (int64_t)b0 * tiles64;
        const int cpw = ((a0.C + ksw - 1) / ksw + ks - 1) / ks;  // chunks per wave
        hipError_t e;
        switch (fmt) {
            case BH_F32: e = launch_fmt<BH_F32>(epi, a, B, rw, ks, cpw, st); break;
            case BH_Q8_ROW: e = launch_fmt<BH_Q8_ROW>(epi, a, B, rw, ks, cpw, st); break;
            case BH_Q4_ROW: e = launch_fmt<BH_Q4_ROW>(epi, a, B, rw, ks, cpw, st); break;
            case BH_Q4_G32: e = launch_fmt<BH_Q4_G32>(epi, a, B, rw, ks, cpw, st); break;
            default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
        b0 += B;
    }
    return hipSuccess;
}

}  // namespace bh
