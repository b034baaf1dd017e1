// k_stream.h — the weight-streaming inner loop of the VALU GEMV (k_gemv.hip).
//
// The weight is stored K-major in 16-byte chunks (bh_internal.h, "KM16"): each lane owns one
// output row and a wavefront streams 1 KiB of contiguous weight bytes per chunk step with one
// 128-bit buffer load per lane. The activations of a chunk are identical for all 64 lanes, so
// they arrive through scalar loads and enter the FMAs as SGPR operands. Nibbles are decoded as
// signed int4 (q ^ 8 == q - 8 in two's complement) shifted into the top of a byte and converted
// with the SDWA sign-extending byte convert: one VALU op per element plus three bit ops per 8
// elements; the factor 16 is folded into the scale.
#pragma once

#include <hip/hip_fp16.h>

#include "bh_internal.h"
#include "k_xl.h"

namespace bh {

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

// acc[j][b] += sum over chunks [c0, c1) of weight j's row nl against activation row b of a.x
// (a.W / a.S, and a.W2 / a.S2 for NACC == 2). `mid()` runs once the first stage of loads is in
// flight: whatever it loads overlaps the weight latency. XL (batch 1, Q4_G32): the activations
// are the limb records a.xl (k_xl.h) and each chunk is an integer dot product.
//
// Weight and scale loads are raw buffer loads: an SGPR resource per matrix, the lane's row as
// the VGPR offset and the chunk as the (uniform) SGPR offset, so a stage costs no per-load
// address arithmetic. Every load of a stage is unconditional (chunk index clamped to the wave's
// last chunk, scale kept as raw fp16 bits) so all of a stage's loads are in flight before the
// first of them is waited on. The chunk loop is software-pipelined over two stages of U chunks.
template <int FMT, int B, int NACC, int U, int CP, bool XL, class Mid>
__device__ __forceinline__ void stream_chunks(const GemvArgs& a, int64_t nl, int c0, int c1, float (&acc)[NACC][B],
                                              Mid&& mid) {
    constexpr int E = Fmt<FMT>::E;
    __amdgpu_buffer_rsrc_t rW[NACC], rS[NACC];
    rW[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.C * a.n_pad * 16, 0x00020000);
    rS[0] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S, (short)0, a.C * a.n_pad * 2, 0x00020000);
    if constexpr (NACC == 2) {
        rW[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.W2, (short)0, a.C * a.n_pad * 16, 0x00020000);
        rS[1] = __builtin_amdgcn_make_buffer_rsrc((void*)a.S2, (short)0, a.C * a.n_pad * 2, 0x00020000);
    }
    const int vo_w = (int)nl * 16, vo_s = (int)sc_pos(nl) * 2;
    uint4 q0[NACC][U], q1[NACC][U];
    // scales as raw fp16 bits, each in its own 32-bit register (packing two per register would
    // make the first stage wait on its scale loads before mid() issues anything)
    uint32_t s0[NACC][U], s1[NACC][U];
    auto fetch = [&](int c, uint4 (&q)[NACC][U], uint32_t (&s)[NACC][U]) {
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
    mid();

#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[j][b] = 0.f;

    if constexpr (XL) static_assert(FMT == BH_Q4_G32 && B == 1, "limb activations: batch-1 group-32 passes");

    // Chunks past c1 (clamped re-reads of the last one) are skipped by a uniform branch that
    // holds no vector loads, so the loads' wait counts are unaffected by it.
    auto consume = [&](int c, const uint4 (&q)[NACC][U], const uint32_t (&s)[NACC][U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c + u < c1) {
                const int kb = (c + u) * E;
                if constexpr (XL) {
                    const uint32_t* xr = a.xl + (int64_t)(c + u) * XL_REC;
                    const float f = __uint_as_float(a.xl[(int64_t)a.C * XL_REC + c + u]);
#pragma unroll
                    for (int j = 0; j < NACC; ++j)
                        acc[j][0] = fmaf(xl_dot_chunk(q[j][u], xr, f), __half2float(__ushort_as_half((uint16_t)s[j][u])),
                                         acc[j][0]);
                    continue;
                }
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
                            acc[j][b] = fmaf(p, __half2float(__ushort_as_half((uint16_t)s[j][u])) * 0.0625f, acc[j][b]);
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
}

// Touch of the activations of chunks [wc0, wc1) of B rows: one vector load per 128-byte line
// (clamped, unconditional: one line per thread and row covers 32 blockDim floats, the lines past
// it are left to the scalar loads), so that the scalar loads of the main loop hit L2: the
// activations were just written by the previous kernel, often on another XCD. Each value stays
// in its own register and must only be consumed after the main loop (`touch_sink`); any earlier
// use would wait on the load, and with it on the weight stage issued before it.
// At most TOUCH_ROWS rows are touched: the registers are held through the main loop.
constexpr int TOUCH_ROWS = 2;
template <int B, int E>
__device__ __forceinline__ void touch_activations(const GemvArgs& a, int wc0, int wc1, float (&t)[TOUCH_ROWS]) {
    const int nx = (wc1 - wc0) * E;
    const int i2 = min((int)threadIdx.x * 32, max(nx - 1, 0));
#pragma unroll
    for (int bb = 0; bb < TOUCH_ROWS; ++bb) t[bb] = a.x[(int64_t)min(bb, B - 1) * a.ldx + wc0 * E + i2];
}
// The same touch for limb records: one 128-byte record per thread.
__device__ __forceinline__ void touch_xl(const GemvArgs& a, int wc0, int wc1, float (&t)[TOUCH_ROWS]) {
    const int i = min((int)threadIdx.x, max(wc1 - wc0 - 1, 0));
    t[0] = __uint_as_float(a.xl[(int64_t)(wc0 + i) * XL_REC]);
#pragma unroll
    for (int bb = 1; bb < TOUCH_ROWS; ++bb) t[bb] = 0.f;
}
template <int B>
__device__ __forceinline__ void touch_sink(const float (&t)[TOUCH_ROWS]) {
#pragma unroll
    for (int bb = 0; bb < (B < TOUCH_ROWS ? B : TOUCH_ROWS); ++bb) asm volatile("" ::"v"(t[bb]));
}

}  // namespace bh
