// k_epilogue.h — epilogues shared by the GEMV and MFMA GEMM kernels.
//
// Input: fin[(j * B + b) * ROWS + r] holds the finished sums (unscaled for the row formats)
// of weight j (gate/up pair: j = 0, 1), batch row b, weight row row0 + r. rn[b] is the
// token's RMSNorm factor when the activations are a normalized residual stream (else 1).
// `scratch` has room for B * ROWS floats. All threads of the workgroup call it.
#pragma once

#include <hip/hip_fp16.h>

#include "bh_internal.h"
#include "k_xl.h"

namespace bh {

// Workgroup barrier for data exchanged through LDS only: waits for this wave's LDS operations,
// not for its outstanding global loads and stores (__syncthreads() also waits for those).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

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

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

// rnorm of the residual stream for row b: 1/sqrt(sum_t ssq[b][t] / n + eps), the tiles summed in
// order (rms_norm_into, cpu_engine.rs:1292-1302, with the sum of squares computed per tile). The
// tiles are loaded RN_U at a time (index clamped, all in flight) before they are added: a loop of
// dependent loads here delays the first wave of every consumer kernel by one memory round trip
// per tile.
constexpr int RN_U = 16;
__device__ __forceinline__ float rnorm_sum(const float* s, int n, int i0, float t) {
    for (; i0 < n; i0 += RN_U) {
        float v[RN_U];
#pragma unroll
        for (int k = 0; k < RN_U; ++k) v[k] = s[min(i0 + k, n - 1)];
#pragma unroll
        for (int k = 0; k < RN_U; ++k)
            if (i0 + k < n) t += v[k];
    }
    return t;
}
__device__ __forceinline__ float stream_rnorm(const GemvArgs& a, int b) {
    const float t = rnorm_sum(a.ssq_in + (int64_t)b * a.ssq_tiles, a.ssq_tiles, 0, 0.f);
    return 1.0f / sqrtf(t / a.norm_n + a.eps);
}

// The per-token norm factors of a kernel whose activations are a normalized residual stream, in
// two steps: request() issues the loads of the first NV tiles of token threadIdx.x (< B) early,
// finish() adds them (and any further tiles) once the kernel's main loop is done and stores the
// factor (1 without a residual-stream input) to rn[threadIdx.x]. A __syncthreads() must separate
// finish() from the readers of rn.
template <int B, int NV = RN_U>
struct RnormReq {
    float v[NV];
    __device__ __forceinline__ bool mine(const GemvArgs& a) const {
        return a.ssq_in && (int)threadIdx.x < B && (int)threadIdx.x < a.batch;
    }
    __device__ __forceinline__ void request(const GemvArgs& a) {
        if (!mine(a)) return;
        const float* s = a.ssq_in + (int64_t)threadIdx.x * a.ssq_tiles;
#pragma unroll
        for (int k = 0; k < NV; ++k) v[k] = s[min(k, a.ssq_tiles - 1)];
    }
    __device__ __forceinline__ void finish(const GemvArgs& a, float* rn) const {
        if (threadIdx.x >= B) return;
        if (!mine(a)) {
            rn[threadIdx.x] = 1.0f;
            return;
        }
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k)
            if (k < a.ssq_tiles) t += v[k];
        t = rnorm_sum(a.ssq_in + (int64_t)threadIdx.x * a.ssq_tiles, a.ssq_tiles, NV, t);
        rn[threadIdx.x] = 1.0f / sqrtf(t / a.norm_n + a.eps);
    }
};

// The same norm factors for the VALU GEMV (B <= 8, one wave of 64 lanes covers B * NV tiles):
// lane b * NV + k of wave 0 requests tile k of token b, one register per lane, and in finish()
// lane b gathers its NV tiles in order through cross-lane reads. (Per-thread arrays would hold
// NV registers through the main loop, and at B = 1 the compiler turns them into scalar loads
// issued one after another.) All lanes of wave 0 call both; finish() is followed by a
// __syncthreads() before rn is read.
template <int B, int NV>
struct RnormLanes {
    static_assert(B * NV <= 64, "one wave");
    float v = 0.f;
    __device__ __forceinline__ void request(const GemvArgs& a) {
        const int b = (int)threadIdx.x / NV, k = (int)threadIdx.x % NV;
        if (a.ssq_in && (int)threadIdx.x < B * NV && b < a.batch)
            v = a.ssq_in[(int64_t)b * a.ssq_tiles + min(k, a.ssq_tiles - 1)];
    }
    __device__ __forceinline__ void finish(const GemvArgs& a, float* rn) const {
        if (threadIdx.x >= 64) return;  // wave 0
        const int b = (int)threadIdx.x;
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < NV; ++k) {
            const float x = __shfl(v, (b % B) * NV + k);
            if (k < a.ssq_tiles) t += x;
        }
        if (b >= B) return;
        if (!a.ssq_in || b >= a.batch) {
            rn[b] = 1.0f;
            return;
        }
        t = rnorm_sum(a.ssq_in + (int64_t)b * a.ssq_tiles, a.ssq_tiles, NV, t);
        rn[b] = 1.0f / sqrtf(t / a.norm_n + a.eps);
    }
};

// K split over workgroups (a.ksw > 1): publish this split's TOT sums and let the tile's last
// workgroup add all splits in split order; returns false in every other workgroup, which then
// exits. The sums are published with agent-scope atomic exchanges and read back with agent-scope
// atomic loads, both performed at the device-coherent level; the exchanges have returned (the
// barrier's wait) before the arrival is counted, so the last arrival reads every split's sums
// without a cache-wide writeback or invalidate. The counter is reset for the next launch.
template <int TOT>
__device__ __forceinline__ bool split_reduce(const GemvArgs& a, float* comb, int tile, int kws) {
    __shared__ int s_last;
    const int ksw = a.ksw;
    static_assert(TOT % 2 == 0, "partials move as 64-bit pairs");
    __syncthreads();  // a thread publishes a pair of sums written by two threads
    float* mine = a.part + (int64_t)(tile * ksw + kws) * TOT;
    unsigned long long sink = 0;
    for (int i = 2 * threadIdx.x; i < TOT; i += 2 * blockDim.x) {
        const unsigned long long v =
            (unsigned long long)__float_as_uint(comb[i]) | ((unsigned long long)__float_as_uint(comb[i + 1]) << 32);
        sink += __hip_atomic_exchange((unsigned long long*)&mine[i], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("" ::"v"(sink));  // the returned values are consumed: the exchanges have completed
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&a.tile_cnt[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ksw - 1;
    __syncthreads();
    if (!s_last) return false;
    const float* all = a.part + (int64_t)tile * ksw * TOT;
    for (int i = 2 * threadIdx.x; i < TOT; i += 2 * blockDim.x) {
        // all splits' loads in flight at once (index clamped in bounds), added in split order
        unsigned long long v[MAX_KSW];
#pragma unroll
        for (int k = 0; k < MAX_KSW; ++k)
            v[k] = __hip_atomic_load((const unsigned long long*)&all[(int64_t)min(k, ksw - 1) * TOT + i], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        float s0 = 0.f, s1 = 0.f;
#pragma unroll
        for (int k = 0; k < MAX_KSW; ++k) {
            s0 += k < ksw ? __uint_as_float((unsigned)v[k]) : 0.f;
            s1 += k < ksw ? __uint_as_float((unsigned)(v[k] >> 32)) : 0.f;
        }
        comb[i] = s0;
        comb[i + 1] = s1;
    }
    if (threadIdx.x == 0) __hip_atomic_store(&a.tile_cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// split_reduce for one wave holding the tile's 64 sums (batch 1, lane = row): the same pairs
// published, the same arrival count and the same split-order sum, with the pairs gathered by
// cross-lane reads instead of LDS and barriers. Returns false where another workgroup finishes
// the tile; on true, `sum` holds the lane's total.
__device__ __forceinline__ bool split_reduce_wave(const GemvArgs& a, float& sum, int tile, int kws) {
    constexpr int TOT = 64;
    const int lane = threadIdx.x & 63;
    const int ksw = a.ksw;
    const float e0 = __shfl(sum, (2 * lane) & 63), e1 = __shfl(sum, (2 * lane + 1) & 63);
    float* mine = a.part + (int64_t)(tile * ksw + kws) * TOT;
    unsigned long long sink = 0;
    if (lane < TOT / 2) {
        const unsigned long long v = (unsigned long long)__float_as_uint(e0) | ((unsigned long long)__float_as_uint(e1) << 32);
        sink = __hip_atomic_exchange((unsigned long long*)&mine[2 * lane], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("" ::"v"(sink));  // the wave's exchanges have completed before the count
    int last = 0;
    if (lane == 0)
        last = __hip_atomic_fetch_add(&a.tile_cnt[tile], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == ksw - 1;
    if (!__shfl(last, 0)) return false;
    const float* all = a.part + (int64_t)tile * ksw * TOT;
    float s0 = 0.f, s1 = 0.f;
    if (lane < TOT / 2) {
        unsigned long long v[MAX_KSW];
#pragma unroll
        for (int k = 0; k < MAX_KSW; ++k)
            v[k] = __hip_atomic_load((const unsigned long long*)&all[(int64_t)min(k, ksw - 1) * TOT + 2 * lane],
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int k = 0; k < MAX_KSW; ++k) {
            s0 += k < ksw ? __uint_as_float((unsigned)v[k]) : 0.f;
            s1 += k < ksw ? __uint_as_float((unsigned)(v[k] >> 32)) : 0.f;
        }
    }
    // element 2k + j is s_j of lane k
    const float t0 = __shfl(s0, lane >> 1), t1 = __shfl(s1, lane >> 1);
    sum = (lane & 1) ? t1 : t0;
    if (lane == 0) __hip_atomic_store(&a.tile_cnt[tile], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// LM-head element of token b, row nn: the raw logit is stored (when y is set), then the repetition penalty
// (cpu_engine.rs:2984-2992) applied `cnt` times; -inf for rows past the vocabulary, tokens past
// the batch and NaN (the first-max scan uses `>`, so NaN never wins).
template <int FMT>
__device__ __forceinline__ float lm_elem(const GemvArgs& a, float f, int b, int64_t nn, const float* rn, int cnt) {
    if (nn >= a.N || b >= a.batch) return -INFINITY;
    float v = f * row_scale<FMT>(a.S, nn) * rn[b];
    if (a.y) a.y[(int64_t)b * a.ldy + nn] = v;
    for (int t = 0; t < cnt; ++t) v = v > 0.f ? v / 1.15f : v * 1.15f;
    return v > -INFINITY ? v : -INFINITY;
}

// One argmax per token and 64-row sub-tile of scratch [B][ROWS] (partials stay indexed by
// 64-row tiles); ties keep the lower index.
template <int B, int ROWS>
__device__ __forceinline__ void lm_argmax(const GemvArgs& a, const float* scratch, int64_t row0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
    constexpr int SUB = ROWS / 64;
    const int tiles64 = (int)((a.n_pad + 63) / 64);
    for (int q = wave; q < B * SUB; q += nwaves) {
        const int b = q / SUB, sub = q % SUB;
        if (b >= a.batch) continue;
        float v = scratch[b * ROWS + sub * 64 + lane];
        int idx = v > -INFINITY ? (int)(row0 + sub * 64 + lane) : 0x7fffffff;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(v, off);
            const int oi = __shfl_xor(idx, off);
            argmax_combine(v, idx, ov, oi);
        }
        const int64_t t64 = row0 / 64 + sub;
        if (lane == 0 && t64 < tiles64) {
            a.part_val[(int64_t)b * tiles64 + t64] = v;
            a.part_idx[(int64_t)b * tiles64 + t64] = idx;
        }
    }
}

// Penalty counts of the LM-head epilogue of a workgroup of NT threads, requested at kernel start:
// element i = threadIdx.x + k NT of the [B][ROWS] tile at row0. ROWS is a multiple of 64, so a
// wave's elements share their token and its slot arrives through a scalar load; only the count
// loads themselves are vector loads, issued without waiting on the weight stream.
template <int B, int ROWS, int NT>
struct PenPre {
    static constexpr int PER = (B * ROWS + NT - 1) / NT;
    uint32_t c[PER];
    __device__ __forceinline__ void load(const GemvArgs& a, int64_t row0) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = threadIdx.x + k * NT;
            const int b = __builtin_amdgcn_readfirstlane((int)((threadIdx.x + k * NT) / ROWS));
            const int64_t nn = row0 + i % ROWS;
            c[k] = 0;
            if (i < B * ROWS && b < a.batch && nn < a.N) c[k] = a.pen[(int64_t)a.slot[b] * a.vocab + nn];
        }
    }
};

// Batched residual-producer epilogue operands of the elements i = threadIdx.x + k * NT that a
// thread finishes (token i / ROWS, row row0 + i % ROWS): the residual x, the next norm's
// weight and the bias, requested at kernel start so that their latency hides under the weight
// stream. Only the launch's own epilogue writes those x elements.
template <int B, int ROWS, int NT>
struct ResPre {
    static constexpr int PER = (B * ROWS + NT - 1) / NT;
    float x0[PER], w1[PER], bias[PER];
    __device__ __forceinline__ void load(const GemvArgs& a, int64_t row0) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int i = threadIdx.x + k * NT;
            const int b = i / ROWS;
            const int64_t nn = row0 + i % ROWS;
            x0[k] = w1[k] = bias[k] = 0.f;
            if (i < B * ROWS && b < a.batch && nn < a.N) {
                x0[k] = a.y[(int64_t)b * a.ldy + nn];
                w1[k] = a.wnext[nn];
                if (a.bias) bias[k] = a.bias[nn];
            }
        }
    }
};

// Batched EPI_QKV operands of the elements i = threadIdx.x + k * NT that a thread finishes: NT is
// a multiple of ROWS, so the thread keeps one row, row0 + threadIdx.x % ROWS, for the tokens
// threadIdx.x / ROWS + k * NT / ROWS. request() reads each token's position and KV-region offset
// at kernel start, as scalar loads (a wave's elements share their token); rope() reads the row's
// biases and each element's RoPE (cos, sin) once the main loop is done, in flight through the
// split reduction. Without them the epilogue walked position -> RoPE table one token at a time
// after the reduction (Qwen2-7B QKV at 16 tokens: 17.6 -> 16.8 us).
template <int B, int ROWS, int NT>
struct QkvPre {
    static_assert(NT % ROWS == 0, "a thread finishes one row");
    static constexpr int PER = (B * ROWS + NT - 1) / NT;
    int p[PER];
    int64_t off[PER];
    float2 cs[PER];
    float bias = 0.f, pbias = 0.f;
    __device__ __forceinline__ void request(const GemvArgs& a) {
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            const int b = __builtin_amdgcn_readfirstlane((int)(threadIdx.x / ROWS) + k * (NT / ROWS));
            p[k] = -1;
            off[k] = 0;
            if (b < B && b < a.batch) {
                p[k] = a.pos[b];
                if (a.boff) off[k] = a.boff[b];
            }
        }
    }
    __device__ __forceinline__ void rope(const GemvArgs& a, int64_t row0) {
        const int64_t nn = row0 + threadIdx.x % ROWS;
        const int half = a.hd >> 1;
        const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
        const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
        const int d = loc % a.hd;
        if (a.bias && nn < a.N) {
            bias = a.bias[nn];
            if (sec < 2) pbias = a.bias[nn + (d < half ? half : -half)];
        }
#pragma unroll
        for (int k = 0; k < PER; ++k) {
            cs[k] = make_float2(1.f, 0.f);
            if (nn < a.N && sec < 2 && p[k] >= 0) cs[k] = a.rope[(int64_t)p[k] * half + (d < half ? d : d - half)];
        }
    }
};

// run_epilogue's batched EPI_QKV with the operands of QkvPre (same arithmetic and order).
template <int FMT, int B, int ROWS, int NT>
__device__ __forceinline__ void run_qkv_pre(const GemvArgs& a, const float* fin, const float* rn, int64_t row0,
                                            const QkvPre<B, ROWS, NT>& qp) {
    const int half = a.hd >> 1;
    const int64_t nn = row0 + threadIdx.x % ROWS;
    if (nn >= a.N) return;
    const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
    const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
    const int hh = loc / a.hd, d = loc % a.hd;
    const int dp = d < half ? half : -half;
#pragma unroll
    for (int k = 0; k < QkvPre<B, ROWS, NT>::PER; ++k) {
        const int i = threadIdx.x + k * NT;
        const int b = i / ROWS;
        if (i >= B * ROWS || b >= a.batch) continue;
        float val = fin[i] * row_scale<FMT>(a.S, nn) * rn[b];
        if (a.bias) val += qp.bias;
        const int p = qp.p[k];
        if (p < 0) {  // a pad token of a multi-sequence prefill: no RoPE, no KV row
            if (sec == 0) a.y[(int64_t)b * a.ldy + nn] = 0.f;
            continue;
        }
        if (sec < 2) {  // rotate-half RoPE (apply_rope_cpu, cpu_engine.rs:1682-1699)
            float pv = fin[i + dp] * row_scale<FMT>(a.S, nn + dp) * rn[b];
            if (a.bias) pv += qp.pbias;
            const float2 cs = qp.cs[k];
            val = d < half ? (val * cs.x - pv * cs.y) : (val * cs.x + pv * cs.y);
        }
        if (sec == 0) {
            a.y[(int64_t)b * a.ldy + nn] = val;
        } else {
            const int64_t row = qp.off[k] + kv_phys_row(a.kv, p);
            const int64_t head = (int64_t)hh * a.kv.kv_rows * a.hd;
            if (a.kv.kv_f16) {  // MFMA-tile order (kv_k_off / kv_v_off)
                if (sec == 1) ((__half*)a.kv.k)[head + kv_k_off(row, d, a.hd)] = __float2half(val);
                else ((__half*)a.kv.v)[head + kv_v_off(row, d, a.hd)] = __float2half(val);
            } else {
                ((float*)(sec == 1 ? a.kv.k : a.kv.v))[head + row * a.hd + d] = val;
            }
        }
    }
}

// run_epilogue's batched EPI_RESNORM with the operands of ResPre (same arithmetic and order).
template <int FMT, int B, int ROWS, int NT>
__device__ __forceinline__ void run_resnorm_pre(const GemvArgs& a, const float* fin, float* scratch, int64_t row0,
                                                const ResPre<B, ROWS, NT>& rp) {
    static_assert(ROWS % 64 == 0, "one sum of squares per 64-row tile");
#pragma unroll
    for (int k = 0; k < ResPre<B, ROWS, NT>::PER; ++k) {
        const int i = threadIdx.x + k * NT;
        if (i >= B * ROWS) continue;  // uniform over the wavefront
        const int b = i / ROWS;
        const int64_t nn = row0 + i % ROWS;
        float sq = 0.f;
        if (nn < a.N && b < a.batch) {
            float o = fin[i] * row_scale<FMT>(a.S, nn);
            if (a.bias) o += rp.bias[k];
            const float v = rp.x0[k] + o;
            const float xw = v * rp.w1[k];
            a.y[(int64_t)b * a.ldy + nn] = v;
            a.xw_out[(int64_t)b * a.ldy + nn] = xw;
            if (a.xw_hl) {  // element nn of chunk nn / 32 sits at K slot kperm^-1(nn % 8) of its 8
                const int q = (int)(nn & 31), e = q & 7;
                const int slot = (((e & 3) ^ 1) << 1) | (e >> 2);
                const _Float16 h = (_Float16)xw;
                const _Float16 l = (_Float16)(xw - (float)h);
                uint16_t* d = a.xw_hl + ((int64_t)b * (a.N / 32) + (nn >> 5)) * 64 + (q >> 3) * 8 + slot;
                d[0] = __builtin_bit_cast(uint16_t, h);
                d[32] = __builtin_bit_cast(uint16_t, l);
            }
            sq = v * v;
        }
        // the wavefront's 64 elements are rows 64 sub .. + 63 of token b (NT and ROWS are multiples
        // of 64), lane = row: the tile's sum of squares in the order of the other epilogues
        const float t = wave_sum64(sq);
        const int64_t tile = (row0 + i % ROWS) / 64;
        if ((threadIdx.x & 63) == 0 && b < a.batch && tile < a.ssq_tiles) a.ssq_out[(int64_t)b * a.ssq_tiles + tile] = t;
    }
    (void)scratch;
}

// The batched LM-head epilogue with the counts of PenPre (run_epilogue's EPI_LMHEAD otherwise).
template <int FMT, int B, int ROWS, int NT>
__device__ __forceinline__ void run_lmhead_pre(const GemvArgs& a, const float* fin, float* scratch, const float* rn,
                                               int64_t row0, const PenPre<B, ROWS, NT>& pp) {
#pragma unroll
    for (int k = 0; k < PenPre<B, ROWS, NT>::PER; ++k) {
        const int i = threadIdx.x + k * NT;
        if (i < B * ROWS) scratch[i] = lm_elem<FMT>(a, fin[i], i / ROWS, row0 + i % ROWS, rn, (int)pp.c[k]);
    }
    lds_barrier();  // LDS scratch only: the stores above need not complete
    lm_argmax<B, ROWS>(a, scratch, row0);
}

// Epilogue operands of a batch-1 launch for the weight row row0 + threadIdx.x (threadIdx.x <
// ROWS: the thread that finishes that row), loaded at the start of the kernel so that their
// latency — including the position -> RoPE table and slot -> penalty chains — hides under the
// weight stream instead of following it.
template <int EPI>
struct EpiPre {
    float x0 = 0.f, w1 = 0.f, bias = 0.f, pbias = 0.f;  // residual, next norm weight, biases
    float2 cs = {1.f, 0.f};                             // RoPE (cos, sin)
    int64_t kvrow = 0;                                  // KV row of the token
    int cnt = 0;                                        // penalty count
    // All threads call it; thread r < rows takes weight row row0 + r. The token's position, KV
    // offset and slot are read first, outside the per-row branch, so they are scalar loads: a
    // vector load there would make its dependent loads wait for every earlier load (the first
    // weight stage included).
    __device__ __forceinline__ void load(const GemvArgs& a, int64_t row0, int rows) {
        int p = 0, slot0 = 0;
        int64_t boff0 = 0;
        if constexpr (EPI == EPI_QKV) {
            p = a.pos[0];
            boff0 = a.boff[0];
        }
        if constexpr (EPI == EPI_LMHEAD) slot0 = a.slot[0];
        const int64_t nn = row0 + threadIdx.x;
        if ((int)threadIdx.x >= rows || nn >= a.N) return;
        if constexpr (EPI == EPI_STORE) {
            if (a.bias) bias = a.bias[nn];
        } else if constexpr (EPI == EPI_RESNORM) {
            x0 = a.y[nn];
            w1 = a.wnext[nn];
            if (a.bias) bias = a.bias[nn];
        } else if constexpr (EPI == EPI_QKV) {
            const int half = a.hd >> 1;
            const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
            const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
            const int d = loc % a.hd;
            if (a.bias) {
                bias = a.bias[nn];
                if (sec < 2) pbias = a.bias[nn + (d < half ? half : -half)];
            }
            if (sec < 2) cs = a.rope[(int64_t)p * half + (d < half ? d : d - half)];
            if (sec > 0) kvrow = boff0 + kv_phys_row(a.kv, p);
        } else if constexpr (EPI == EPI_LMHEAD) {
            cnt = a.pen[(int64_t)slot0 * a.vocab + nn];
        }
    }
};

// run_epilogue's batch-1 EPI_RESNORM for one 64-row tile finished by one wave whose lane r
// holds row row0 + r's sum (and loaded its operands into `pre`): x += acc + bias, xw = x * w_next,
// the tile's sum of squares, all in registers; with a.xl_out also xw's limb records.
template <int FMT>
__device__ __forceinline__ void resnorm_wave(const GemvArgs& a, float sum, int64_t row0, const EpiPre<EPI_RESNORM>& pre) {
    const int lane = threadIdx.x & 63;
    const int64_t nn = row0 + lane;
    float sq = 0.f, xw = 0.f;
    if (nn < a.N) {
        const float v = pre.x0 + (sum * row_scale<FMT>(a.S, nn) + pre.bias);
        a.y[nn] = v;
        xw = v * pre.w1;
        a.xw_out[nn] = xw;
        sq = v * v;
    }
    const float t = wave_sum64(sq);
    const int64_t tile = row0 / 64;
    if (lane == 0 && tile < a.ssq_tiles) a.ssq_out[tile] = t;
    if (a.xl_out) xl_pack64(xw, a.xl_out, row0 / 32, (a.N + 31) / 32);
}

// Row offset of row nn's rotate-half RoPE partner (+- hd/2 within its head).
__device__ __forceinline__ int qkv_partner(const GemvArgs& a, int64_t nn) {
    const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
    const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
    return loc % a.hd < (a.hd >> 1) ? (a.hd >> 1) : -(a.hd >> 1);
}

// Batch-1 EPI_QKV for row nn < N: its sum and its RoPE partner's (rn0 the token's norm factor,
// operands in `pre`): bias, rotate-half RoPE (apply_rope_cpu, cpu_engine.rs:1682-1699), q to y,
// k and v to the KV cache.
template <int FMT>
__device__ __forceinline__ void qkv_row(const GemvArgs& a, int64_t nn, float sum, float psum, float rn0,
                                        const EpiPre<EPI_QKV>& pre) {
    const int half = a.hd >> 1;
    const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
    const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
    const int hh = loc / a.hd, d = loc % a.hd;
    float val = sum * row_scale<FMT>(a.S, nn) * rn0 + pre.bias;
    if (sec < 2) {
        const int dp = d < half ? half : -half;
        const float pv = psum * row_scale<FMT>(a.S, nn + dp) * rn0 + pre.pbias;
        val = d < half ? (val * pre.cs.x - pv * pre.cs.y) : (val * pre.cs.x + pv * pre.cs.y);
    }
    if (sec == 0) {
        a.y[nn] = val;
    } else {
        const int64_t head = (int64_t)hh * a.kv.kv_rows * a.hd;
        if (a.kv.kv_f16) {
            if (sec == 1) ((__half*)a.kv.k)[head + kv_k_off(pre.kvrow, d, a.hd)] = __float2half(val);
            else ((__half*)a.kv.v)[head + kv_v_off(pre.kvrow, d, a.hd)] = __float2half(val);
        } else {
            ((float*)(sec == 1 ? a.kv.k : a.kv.v))[head + pre.kvrow * a.hd + d] = val;
        }
    }
}

// Batch-1 EPI_QKV for one 64-row tile finished by one wave (lane r = row row0 + r, holding its
// sum and operands): the partner's sum is read from lane r +- hd/2 (heads never straddle a tile).
template <int FMT>
__device__ __forceinline__ void qkv_wave(const GemvArgs& a, float sum, float rn0, int64_t row0, const EpiPre<EPI_QKV>& pre) {
    const int lane = threadIdx.x & 63;
    const int64_t nn = row0 + lane;
    const float psum = __shfl(sum, (lane + qkv_partner(a, nn)) & 63);
    if (nn < a.N) qkv_row<FMT>(a, nn, sum, psum, rn0, pre);
}

template <int FMT, int B, int EPI, int ROWS>
__device__ __forceinline__ void run_epilogue(const GemvArgs& a, const float* fin, float* scratch, const float* rn,
                                             int64_t row0, const EpiPre<EPI>* pre = nullptr) {
    if constexpr (B == 1) {
        if (pre) {  // batch 1 with prefetched operands: thread r finishes row row0 + r
            const int rr = threadIdx.x;
            const int64_t nn = row0 + rr;
            const bool ok = rr < ROWS && nn < a.N;
            if constexpr (EPI == EPI_STORE) {
                if (ok) a.y[nn] = fin[rr] * row_scale<FMT>(a.S, nn) * rn[0] + pre->bias;
            } else if constexpr (EPI == EPI_RESNORM) {
                static_assert(ROWS == 64, "one wave finishes a 64-row tile");
                if (threadIdx.x < 64) resnorm_wave<FMT>(a, fin[threadIdx.x], row0, *pre);
            } else if constexpr (EPI == EPI_SILU) {
                float y = 0.f;
                if (ok) {
                    const float g = fin[rr] * row_scale<FMT>(a.S, nn) * rn[0];
                    const float u = fin[ROWS + rr] * row_scale<FMT>(a.S2, nn) * rn[0];
                    y = g * (1.0f / (1.0f + expf(-g))) * u;
                    a.y[nn] = y;
                }
                // wave 0 holds the tile's 64 rows: their limb records for the down projection
                if (ROWS == 64 && a.xl_out && threadIdx.x < 64) xl_pack64(y, a.xl_out, row0 / 32, (a.N + 31) / 32);
            } else if constexpr (EPI == EPI_QKV) {
                if (ok) qkv_row<FMT>(a, nn, fin[rr], fin[rr + qkv_partner(a, nn)], rn[0], *pre);
            } else if constexpr (EPI == EPI_LMHEAD) {
                if (rr < ROWS) scratch[rr] = lm_elem<FMT>(a, fin[rr], 0, nn, rn, pre->cnt);
                lds_barrier();  // LDS scratch only: the stores above need not complete
                lm_argmax<1, ROWS>(a, scratch, row0);
            }
            return;
        }
    }
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nwaves = blockDim.x >> 6;
    if constexpr (EPI == EPI_STORE) {
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            float v = fin[i] * row_scale<FMT>(a.S, nn) * rn[b];
            if (a.bias) v += a.bias[nn];
            a.y[(int64_t)b * a.ldy + nn] = v;
        }
    } else if constexpr (EPI == EPI_RESNORM) {
        // residual add (cpu_engine.rs:2937-2939, 2966-2968), then the next norm's inputs
        static_assert(ROWS % 64 == 0, "one sum of squares per 64-row tile");
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            float sq = 0.f;
            if (nn < a.N && b < a.batch) {
                float o = fin[i] * row_scale<FMT>(a.S, nn);
                if (a.bias) o += a.bias[nn];
                float* xp = a.y + (int64_t)b * a.ldy + nn;
                const float v = *xp + o;
                *xp = v;
                a.xw_out[(int64_t)b * a.ldy + nn] = v * a.wnext[nn];
                sq = v * v;
            }
            scratch[i] = sq;
        }
        lds_barrier();  // LDS scratch only: the stores above need not complete
        constexpr int SUB = ROWS / 64;
        for (int q = wave; q < B * SUB; q += nwaves) {
            const int b = q / SUB, sub = q % SUB;
            const float t = wave_sum64(scratch[b * ROWS + sub * 64 + lane]);
            const int64_t tile = row0 / 64 + sub;
            if (lane == 0 && b < a.batch && tile < a.ssq_tiles) a.ssq_out[(int64_t)b * a.ssq_tiles + tile] = t;
        }
    } else if constexpr (EPI == EPI_SILU) {
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            const float g = fin[i] * row_scale<FMT>(a.S, nn) * rn[b];
            const float u = fin[B * ROWS + i] * row_scale<FMT>(a.S2, nn) * rn[b];
            a.y[(int64_t)b * a.ldy + nn] = g * (1.0f / (1.0f + expf(-g))) * u;
        }
    } else if constexpr (EPI == EPI_QKV) {
        const int half = a.hd >> 1;
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS, rr = i % ROWS;
            const int64_t nn = row0 + rr;
            if (nn >= a.N || b >= a.batch) continue;
            float val = fin[i] * row_scale<FMT>(a.S, nn) * rn[b];
            if (a.bias) val += a.bias[nn];
            const int sec = nn < a.qd ? 0 : (nn < a.qd + a.kd ? 1 : 2);
            const int loc = (int)nn - (sec == 0 ? 0 : (sec == 1 ? a.qd : a.qd + a.kd));
            const int hh = loc / a.hd, d = loc % a.hd;
            const int p = a.pos[b];
            if (p < 0) {  // a pad token of a multi-sequence prefill: no RoPE, no KV row
                if (sec == 0) a.y[(int64_t)b * a.ldy + nn] = 0.f;
                continue;
            }
            if (sec < 2) {  // rotate-half RoPE (apply_rope_cpu, cpu_engine.rs:1682-1699)
                const int dp = d < half ? half : -half;
                float pv = fin[i + dp] * row_scale<FMT>(a.S, nn + dp) * rn[b];
                if (a.bias) pv += a.bias[nn + dp];
                const float2 cs = a.rope[(int64_t)p * half + (d < half ? d : d - half)];
                val = d < half ? (val * cs.x - pv * cs.y) : (val * cs.x + pv * cs.y);
            }
            if (sec == 0) {
                a.y[(int64_t)b * a.ldy + nn] = val;
            } else {
                const int64_t row = a.boff[b] + kv_phys_row(a.kv, p);
                const int64_t head = (int64_t)hh * a.kv.kv_rows * a.hd;
                if (a.kv.kv_f16) {  // MFMA-tile order (kv_k_off / kv_v_off)
                    if (sec == 1) ((__half*)a.kv.k)[head + kv_k_off(row, d, a.hd)] = __float2half(val);
                    else ((__half*)a.kv.v)[head + kv_v_off(row, d, a.hd)] = __float2half(val);
                } else {
                    ((float*)(sec == 1 ? a.kv.k : a.kv.v))[head + row * a.hd + d] = val;
                }
            }
        }
    } else if constexpr (EPI == EPI_LMHEAD) {
        // raw logits out, then the repetition penalty, in LDS; then the per-tile argmax
        for (int i = threadIdx.x; i < B * ROWS; i += blockDim.x) {
            const int b = i / ROWS;
            const int64_t nn = row0 + i % ROWS;
            const int cnt = (nn < a.N && b < a.batch) ? a.pen[(int64_t)a.slot[b] * a.vocab + nn] : 0;
            scratch[i] = lm_elem<FMT>(a, fin[i], b, nn, rn, cnt);
        }
        lds_barrier();  // LDS scratch only: the stores above need not complete
        lm_argmax<B, ROWS>(a, scratch, row0);
    }
}

}  // namespace bh
