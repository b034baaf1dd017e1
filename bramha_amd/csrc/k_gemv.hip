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
// chunks is in flight while the current one is converted). Waves of a workgroup split
// K and combine in LDS in a fixed order; matrices with few row tiles also split K
// across workgroups, which store partial sums that the next kernel (residual-reduce +
// RMSNorm) adds in a fixed order, so results are deterministic without atomics.
// Epilogues fuse the bias, residual add, SiLU gate, RoPE + KV-cache append, and the
// LM-head repetition penalty + per-tile argmax.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

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

// Per-row factor applied after the sum (row formats); 1 for F32 and Q4_G32.
template <int FMT>
__device__ __forceinline__ float row_scale(const void* S, int64_t n) {
    if constexpr (FMT == BH_Q4_ROW) return ((const float*)S)[n] * 0.0625f;
    else if constexpr (FMT == BH_Q8_ROW) return ((const float*)S)[n];
    else return 1.0f;
}

__device__ __forceinline__ int64_t kv_phys_row(const KvView& kv, int p) {
    if (kv.max_context > 0 && p >= kv.sink) return kv.sink + (p - kv.sink) % (kv.max_context - kv.sink);
    return p;
}

__device__ __forceinline__ void argmax_combine(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

template <int FMT, int B, int EPI, int RW>
__global__ void __launch_bounds__(1024) k_gemv(const GemvArgs a) {
    extern __shared__ float smem[];
    constexpr int E = Fmt<FMT>::E;
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    constexpr int U = NACC == 2 ? 2 : 4;  // chunks per pipeline stage (x2 stages in flight)
    constexpr int TOT = NACC * B * ROWS;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nwaves = blockDim.x >> 6;
    const int ksplit = nwaves / RW;
    const int rw = wave % RW, kw = wave / RW;
    const int r = rw * 64 + lane;
    const int ksw = EPI == EPI_PART ? a.ksw : 1;
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

    const uint4* Wp[NACC];
    const __half* Sp[NACC];
    Wp[0] = (const uint4*)a.W + n;
    Sp[0] = (const __half*)a.S + n;
    if constexpr (NACC == 2) {
        Wp[1] = (const uint4*)a.W2 + n;
        Sp[1] = (const __half*)a.S2 + n;
    }

    uint4 q0[NACC][U], q1[NACC][U];
    float s0[NACC][U], s1[NACC][U];
    auto fetch = [&](int c, uint4 (&q)[NACC][U], float (&s)[NACC][U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (row_ok && c + u < c1) {
#pragma unroll
                for (int j = 0; j < NACC; ++j) {
                    q[j][u] = Wp[j][(int64_t)(c + u) * a.n_pad];
                    if constexpr (FMT == BH_Q4_G32) s[j][u] = __half2float(Sp[j][(int64_t)(c + u) * a.n_pad]);
                }
            }
        }
    };
    fetch(c0, q0, s0);

    float acc[NACC][B];
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int b = 0; b < B; ++b) acc[j][b] = 0.f;

    auto consume = [&](int c, const uint4 (&q)[NACC][U], const float (&s)[NACC][U]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (row_ok && c + u < c1) {
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
                        if constexpr (FMT == BH_Q4_G32) acc[j][b] = fmaf(p, s[j][u] * 0.0625f, acc[j][b]);
                        else acc[j][b] += p;
                    }
                }
            }
        }
    };
    for (int c = c0; c < c1; c += 2 * U) {
        fetch(c + U, q1, s1);
        consume(c, q0, s0);
        if (c + U >= c1) break;
        fetch(c + 2 * U, q0, s0);
        consume(c + U, q1, s1);
    }

    // ---- combine the K-split partial sums in a fixed order ----
#pragma unroll
    for (int j = 0; j < NACC; ++j)
#pragma unroll
        for (int b = 0; b < B; ++b) smem[kw * TOT + (j * B + b) * ROWS + r] = acc[j][b];
    __syncthreads();
    for (int i = threadIdx.x; i < TOT; i += blockDim.x) {
        float sum = smem[i];
        for (int w = 1; w < ksplit; ++w) sum += smem[w * TOT + i];
        smem[i] = sum;
    }
    __syncthreads();
    const int64_t row0 = (int64_t)tile * ROWS;

    const float* fin = smem;

    if constexpr (EPI == EPI_PART) {
        float* part = a.part + (int64_t)kws * a.part_ld;
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            part[(int64_t)b * a.N + nn] = fin[i] * row_scale<FMT>(a.S, nn);
        }
    } else if constexpr (EPI == EPI_STORE || EPI == EPI_RESID) {
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            float v = fin[i] * row_scale<FMT>(a.S, nn);
            if (a.bias) v += a.bias[nn];
            float* yp = a.y + (int64_t)b * a.ldy + nn;
            if constexpr (EPI == EPI_RESID) *yp = *yp + v;
            else *yp = v;
        }
    } else if constexpr (EPI == EPI_SILU) {
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            const float g = fin[i] * row_scale<FMT>(a.S, nn);
            const float u = fin[B * ROWS + i] * row_scale<FMT>(a.S2, nn);
            a.y[(int64_t)b * a.ldy + nn] = g * (1.0f / (1.0f + expf(-g))) * u;
        }
    } else if constexpr (EPI == EPI_QKV) {
        const int half = a.hd >> 1;
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            float val = fin[i] * row_scale<FMT>(a.S, nn);
            if (a.bias) val += a.bias[nn];
            const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
            const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
            const int hh = loc / a.hd, d = loc % a.hd;
            const int p = a.pos[b];
            if (sec < 2) {  // rotate-half RoPE (apply_rope_cpu, cpu_engine.rs:1682-1699)
                const int dp = d < half ? half : -half;
                float pv = fin[i + dp] * row_scale<FMT>(a.S, nn + dp);
                if (a.bias) pv += a.bias[nn + dp];
                const float2 cs = a.rope[(int64_t)p * half + (d < half ? d : d - half)];
                val = d < half ? (val * cs.x - pv * cs.y) : (val * cs.x + pv * cs.y);
            }
            if (sec == 0) {
                a.y[(int64_t)b * a.ldy + nn] = val;
            } else {
                const int64_t row = a.seq_off[a.slot[b]] + kv_phys_row(a.kv, p);
                const int64_t off = ((int64_t)hh * a.kv.kv_rows + row) * a.hd + d;
                void* base = sec == 1 ? a.kv.k : a.kv.v;
                if (a.kv.kv_f16) ((__half*)base)[off] = __float2half(val);
                else ((float*)base)[off] = val;
            }
        }
    } else if constexpr (EPI == EPI_LMHEAD) {
        // raw logits out, then repetition penalty (cpu_engine.rs:2984-2992) in LDS
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            float pv = -INFINITY;
            if (nn < a.N && b < a.batch) {
                float v = fin[i] * row_scale<FMT>(a.S, nn);
                a.y[(int64_t)b * a.ldy + nn] = v;
                const int cnt = a.pen[(int64_t)a.slot[b] * a.vocab + nn];
                for (int t = 0; t < cnt; ++t) v = v > 0.f ? v / 1.15f : v * 1.15f;
                pv = v > -INFINITY ? v : -INFINITY;  // NaN never wins (first-max scan uses `>`)
            }
            smem[TOT + i] = pv;
        }
        __syncthreads();
        for (int b = wave; b < B; b += nwaves) {
            if (b >= a.batch) continue;
            float v = smem[TOT + b * ROWS + lane];
            int idx = v > -INFINITY ? (int)(row0 + lane) : 0x7fffffff;
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const float ov = __shfl_xor(v, off);
                const int oi = __shfl_xor(idx, off);
                argmax_combine(v, idx, ov, oi);
            }
            if (lane == 0) {
                a.part_val[(int64_t)b * tiles + tile] = v;
                a.part_idx[(int64_t)b * tiles + tile] = idx;
            }
        }
    }
}

template <int FMT, int B, int EPI, int RW>
hipError_t launch_one(const GemvArgs& a, int ksplit, int ksw, hipStream_t st) {
    constexpr int NACC = EPI == EPI_SILU ? 2 : 1;
    constexpr int ROWS = 64 * RW;
    const int tiles = (a.n_pad + ROWS - 1) / ROWS;
    size_t shm = (size_t)ksplit * NACC * B * ROWS * sizeof(float);
    if (EPI == EPI_LMHEAD) shm = std::max(shm, (size_t)(NACC * B * ROWS + B * ROWS) * sizeof(float));
    hipLaunchKernelGGL((k_gemv<FMT, B, EPI, RW>), dim3(tiles * ksw), dim3(64 * RW * ksplit), shm, st, a);
    return hipGetLastError();
}

template <int FMT, int EPI, int RW>
hipError_t launch_b(const GemvArgs& a, int B, int ksplit, int ksw, hipStream_t st) {
    switch (B) {
        case 1: return launch_one<FMT, 1, EPI, RW>(a, ksplit, ksw, st);
        case 2: return launch_one<FMT, 2, EPI, RW>(a, ksplit, ksw, st);
        case 4: return launch_one<FMT, 4, EPI, RW>(a, ksplit, ksw, st);
        default: return launch_one<FMT, 8, EPI, RW>(a, ksplit, ksw, st);
    }
}

template <int FMT>
hipError_t launch_fmt(int epi, const GemvArgs& a, int B, int rw, int ksplit, int ksw, hipStream_t st) {
    switch (epi) {
        case EPI_STORE: return launch_b<FMT, EPI_STORE, 1>(a, B, ksplit, ksw, st);
        case EPI_RESID: return launch_b<FMT, EPI_RESID, 1>(a, B, ksplit, ksw, st);
        case EPI_SILU: return launch_b<FMT, EPI_SILU, 1>(a, B, ksplit, ksw, st);
        case EPI_PART: return launch_b<FMT, EPI_PART, 1>(a, B, ksplit, ksw, st);
        case EPI_QKV:
            return rw == 2 ? launch_b<FMT, EPI_QKV, 2>(a, B, ksplit, ksw, st)
                           : launch_b<FMT, EPI_QKV, 1>(a, B, ksplit, ksw, st);
        default:
            if constexpr (FMT == BH_F32 || FMT == BH_Q4_G32) return launch_b<FMT, EPI_LMHEAD, 1>(a, B, ksplit, ksw, st);
            return hipErrorInvalidValue;
    }
}

}  // namespace

// Waves per workgroup along K: aim for ~8 waves per CU and >= 2 chunks per wave.
static int waves_per_tile(int tiles, int rw, int C, int nacc, int B) {
    int ks = (2048 + tiles * rw - 1) / (tiles * rw);
    ks = std::max(1, std::min({ks, 16 / rw, std::max(1, C / 2)}));
    while (ks > 1 && (size_t)ks * nacc * B * 64 * rw * 4 > 60 * 1024) --ks;
    return ks;
}

// Workgroups per row tile for EPI_PART: about one workgroup per CU (256) with at least
// two chunks each, at most 16 splits.
int part_splits(int tiles, int C) {
    const int ksw = 256 / std::max(tiles, 1);
    return std::max(1, std::min({ksw, 16, std::max(1, C / 2)}));
}

// Splits the batch into passes of at most 8 rows; EPI_PART uses a.ksw workgroups per tile.
hipError_t launch_gemv(int fmt, int epi, const GemvArgs& a0, hipStream_t st) {
    const int rw = (epi == EPI_QKV && a0.hd > 64) ? a0.hd / 64 : 1;
    if (rw > 2) return hipErrorInvalidValue;
    if (epi == EPI_PART && (!a0.part || a0.ksw < 1)) return hipErrorInvalidValue;
    const int nacc = epi == EPI_SILU ? 2 : 1;
    const int tiles = (a0.n_pad + 64 * rw - 1) / (64 * rw);
    const int ksw = epi == EPI_PART ? a0.ksw : 1;
    int b0 = 0;
    while (b0 < a0.batch) {
        const int rem = a0.batch - b0;
        const int B = rem >= 8 ? 8 : (rem >= 4 ? 4 : (rem >= 2 ? 2 : 1));
        int ks = waves_per_tile(tiles * ksw, rw, (a0.C + ksw - 1) / ksw, nacc, B);
        GemvArgs a = a0;
        a.batch = B;
        a.x = a0.x + (int64_t)b0 * a0.ldx;
        a.y = a0.y + (int64_t)b0 * a0.ldy;
        if (a0.pos) a.pos = a0.pos + b0;
        if (a0.slot) a.slot = a0.slot + b0;
        if (a0.part_val) a.part_val = a0.part_val + (int64_t)b0 * tiles;
        if (a0.part_idx) a.part_idx = a0.part_idx + (int64_t)b0 * tiles;
        if (a0.part) a.part = a0.part + (int64_t)b0 * a0.N;
        hipError_t e;
        switch (fmt) {
            case BH_F32: e = launch_fmt<BH_F32>(epi, a, B, rw, ks, ksw, st); break;
            case BH_Q8_ROW: e = launch_fmt<BH_Q8_ROW>(epi, a, B, rw, ks, ksw, st); break;
            case BH_Q4_ROW: e = launch_fmt<BH_Q4_ROW>(epi, a, B, rw, ks, ksw, st); break;
            case BH_Q4_G32: e = launch_fmt<BH_Q4_G32>(epi, a, B, rw, ks, ksw, st); break;
            default: return hipErrorInvalidValue;
        }
        if (e != hipSuccess) return e;
        b0 += B;
    }
    return hipSuccess;
}

}  // namespace bh
