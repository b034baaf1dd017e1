// k_attn.hip — GQA decode attention over the device-resident packed KV cache.
//
// Reference semantics: flash_attention_single_into (src/inference/cpu_engine.rs:1450-1509):
// per query head, online softmax over the cached rows of its KV head
// (kv head = q head / (n_q / n_kv)), scores (q . k) * (1/sqrt(hd)), output o * (1/l).
//
// Design: one workgroup per (query row, KV head, context split); the G = n_q/n_kv query heads
// that share a KV head are processed together, so every K/V byte is read once per
// workgroup instead of once per query head (the reference re-reads each KV head's rows G
// times). Each wavefront takes 64-row tiles of the context.
//
// fp16 cache (k_attn_mf): both products run on MFMA (v_mfma_f32_16x16x32_f16) with the G
// heads in the 16 columns. Scores S^T[t][h] = K[t][:] . Q[h][:] take K rows straight from the
// cache (16-byte loads) and Q as fp16 hi + lo pairs (hi + lo carries ~22 bits of the f32 q);
// the online softmax needs one max across the 4 row groups per tile and defers the sum to the
// end; O^T[d][h] += V^T[d][t] . P^T[t][h] takes V^T from the transposed V cache (16-byte loads
// of 8 consecutive rows of one column) and P as fp16 hi + lo. The K rows each lane loads are
// permuted so that the probabilities a lane holds after the softmax are exactly the 8 rows its
// P operand needs: no cross-lane data movement between the two products.
// f32 cache (k_attn): VALU dot products with q broadcast from LDS and probabilities moved
// between lanes with ds_bpermute.
//
// Splits of long contexts publish (m, l, o) partials; the last workgroup of a (row, KV head)
// to finish merges them with log-sum-exp weights (flash-decoding) — no second kernel.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_attn.h"

namespace bh {
namespace {

constexpr int MAX_SPLITS = 128;

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

template <int KVF16>
__device__ __forceinline__ uint4 load16(const void* base, int64_t elem) {
    if constexpr (KVF16) return *(const uint4*)((const __half*)base + elem);
    else return *(const uint4*)((const float*)base + elem);
}

// 8 consecutive elements starting at `elem`: one 16-byte load for fp16, two for f32.
template <int KVF16>
struct Row8 {
    uint4 a, b;
    __device__ __forceinline__ void load(const void* base, int64_t elem) {
        a = load16<KVF16>(base, elem);
        if constexpr (!KVF16) b = load16<KVF16>(base, elem + 4);
    }
    __device__ __forceinline__ void zero() {
        a = make_uint4(0, 0, 0, 0);
        b = a;
    }
    __device__ __forceinline__ void to_float(float* f) const {
        if constexpr (KVF16) {
            const __half2* h2 = (const __half2*)&a;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 t = __half22float2(h2[i]);
                f[2 * i] = t.x;
                f[2 * i + 1] = t.y;
            }
        } else {
            f[0] = __uint_as_float(a.x); f[1] = __uint_as_float(a.y); f[2] = __uint_as_float(a.z); f[3] = __uint_as_float(a.w);
            f[4] = __uint_as_float(b.x); f[5] = __uint_as_float(b.y); f[6] = __uint_as_float(b.z); f[7] = __uint_as_float(b.w);
        }
    }
};

// The last workgroup of a (row, KV head): log-sum-exp merge of the splits' (m, l, o) partials.
template <int HD, int G>
__device__ __forceinline__ void merge_splits(const AttnArgs& a, int64_t hq0) {
    __shared__ float f_s[G][MAX_SPLITS];
    __shared__ float L_s[G];
    const int S = a.splits;
    for (int i = threadIdx.x; i < G * S; i += blockDim.x) {
        const int g = i / S, s2 = i % S;
        f_s[g][s2] = a.part_ml[((hq0 + g) * S + s2) * 2];
    }
    __syncthreads();
    if (threadIdx.x < G) {
        const int g = threadIdx.x;
        float M = -INFINITY;
        for (int s2 = 0; s2 < S; ++s2) M = fmaxf(M, f_s[g][s2]);
        float L = 0.f;
        for (int s2 = 0; s2 < S; ++s2) {
            const float ms = f_s[g][s2];
            const float f = ms == -INFINITY ? 0.f : expf(ms - M);
            L += a.part_ml[((hq0 + g) * S + s2) * 2 + 1] * f;
            f_s[g][s2] = f;
        }
        L_s[g] = L;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * HD; i += blockDim.x) {
        const int g = i / HD, d = i % HD;
        float O = 0.f;
        for (int s2 = 0; s2 < S; ++s2) O = fmaf(f_s[g][s2], a.part_o[((hq0 + g) * S + s2) * HD + d], O);
        a.out[(hq0 + g) * HD + d] = L_s[g] > 0.f ? O * (1.0f / L_s[g]) : 0.f;
    }
}

template <int HD, int KVF16, int G>
__global__ void __launch_bounds__(256) k_attn(const AttnArgs a) {
    constexpr int DL = HD / 8;   // lanes per row in the value phase
    constexpr int TS = 64 / DL;  // rows per value-phase step
    constexpr int NV = 64 / TS;  // value-phase steps per 64-row tile
    __shared__ float q_s[G][HD];
    __shared__ float w_m[4][G], w_l[4][G];
    __shared__ float w_o[4][G][HD];
    __shared__ int s_last;

    const int b = blockIdx.z, h = blockIdx.y, sp = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;

    // q first: its address depends on nothing loaded
    constexpr int QPT = (G * HD + 255) / 256;
    float qreg[QPT];
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = threadIdx.x + k * 256;
        qreg[k] = i < G * HD ? a.q[((int64_t)b * a.nq + h * G) * HD + i] : 0.f;
    }
    const int64_t off = a.boff[b];
    int len;
    if (a.seq_len) {
        len = a.seq_len[b];
    } else {
        len = a.pos[b] + 1;
        if (a.kv.max_context > 0) len = min(len, a.kv.max_context);
    }
    const int r0 = sp * a.split_rows;
    const int r1 = min(len, r0 + a.split_rows);

    const float scale = 1.0f / sqrtf((float)HD);
    const int64_t kv_base = ((int64_t)h * a.kv.kv_rows + off) * HD;
    float m[G], l[G], o[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
    }
    const int tsub = lane / DL, dl = lane % DL;
    // K rows (lane t owns row t) and V rows (TS rows per step) of a 64-row tile, requested together
    Row8<KVF16> kr[HD / 8], vr[NV];
    auto load_tile = [&](int t0) {
        const int t = t0 + lane;
#pragma unroll
        for (int dc = 0; dc < HD / 8; ++dc) {
            if (t < r1) kr[dc].load(a.kv.k, kv_base + (int64_t)t * HD + dc * 8);
            else kr[dc].zero();
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int t2 = t0 + j * TS + tsub;
            if (t2 < r1) vr[j].load(a.kv.v, kv_base + (int64_t)t2 * HD + dl * 8);
            else vr[j].zero();
        }
    };
    const int tfirst = r0 + wave * 64;
    if (tfirst < r1) load_tile(tfirst);
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = threadIdx.x + k * 256;
        if (i < G * HD) q_s[i / HD][i % HD] = qreg[k];
    }
    __syncthreads();

    for (int t0 = tfirst; t0 < r1; t0 += 4 * 64) {
        if (t0 != tfirst) load_tile(t0);
        const bool valid = t0 + lane < r1;
        float s[G];
#pragma unroll
        for (int g = 0; g < G; ++g) s[g] = 0.f;
#pragma unroll
        for (int dc = 0; dc < HD / 8; ++dc) {
            float kf[8];
            kr[dc].to_float(kf);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float4 qa = *(const float4*)&q_s[g][dc * 8];
                const float4 qb = *(const float4*)&q_s[g][dc * 8 + 4];
                float acc = s[g];
                acc = fmaf(qa.x, kf[0], acc);
                acc = fmaf(qa.y, kf[1], acc);
                acc = fmaf(qa.z, kf[2], acc);
                acc = fmaf(qa.w, kf[3], acc);
                acc = fmaf(qb.x, kf[4], acc);
                acc = fmaf(qb.y, kf[5], acc);
                acc = fmaf(qb.z, kf[6], acc);
                acc = fmaf(qb.w, kf[7], acc);
                s[g] = acc;
            }
            // keep the q reads of later chunks from being hoisted into registers
            __builtin_amdgcn_sched_barrier(0);
        }
    float pg[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float sc = valid ? s[g] * scale : -INFINITY;
            const float mn = fmaxf(m[g], wave_max(sc));
            const float alpha = m[g] == -INFINITY ? 0.f : expf(m[g] - mn);
            const float p = valid ? expf(sc - mn) : 0.f;
            l[g] = l[g] * alpha + wave_sum(p);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[g][e] *= alpha;
            m[g] = mn;
            pg[g] = p;
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            float vf[8];
            vr[j].to_float(vf);
            const int tl = j * TS + tsub;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float pp = __shfl(pg[g], tl);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pp, vf[e], o[g][e]);
            }
        }
    }
    // sum the value accumulators of the lanes that share a column slice
#pragma unroll
    for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            float v = o[g][e];
#pragma unroll
            for (int x = DL; x < 64; x <<= 1) v += __shfl_xor(v, x);
            o[g][e] = v;
        }
    }
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            w_m[wave][g] = m[g];
            w_l[wave][g] = l[g];
        }
    }
    if (tsub == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) w_o[wave][g][dl * 8 + e] = o[g][e];
    }
    __syncthreads();

    const int64_t hq0 = (int64_t)b * a.nq + h * G;
    for (int i = threadIdx.x; i < G * HD; i += blockDim.x) {
        const int g = i / HD, d = i % HD;
        float M = -INFINITY;
        for (int w = 0; w < 4; ++w) M = fmaxf(M, w_m[w][g]);
        float L = 0.f, O = 0.f;
        for (int w = 0; w < 4; ++w) {
            const float f = w_m[w][g] == -INFINITY ? 0.f : expf(w_m[w][g] - M);
            L += w_l[w][g] * f;
            O += w_o[w][g][d] * f;
        }
        if (a.splits == 1) {
            a.out[(hq0 + g) * HD + d] = L > 0.f ? O * (1.0f / L) : 0.f;
        } else {
            a.part_o[((hq0 + g) * a.splits + sp) * HD + d] = O;
            if (d == 0) {
                a.part_ml[((hq0 + g) * a.splits + sp) * 2] = M;
                a.part_ml[((hq0 + g) * a.splits + sp) * 2 + 1] = L;
            }
        }
    }
    if (a.splits == 1) return;

    // ---- the last workgroup of this (row, KV head) merges the splits ----
    __threadfence();
    __syncthreads();
    if (threadIdx.x == 0) s_last = atomicAdd(&a.cnt[b * a.nkv + h], 1) == a.splits - 1;
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    merge_splits<HD, G>(a, hq0);
    if (threadIdx.x == 0) a.cnt[b * a.nkv + h] = 0;  // ready for the next launch
}

__device__ __forceinline__ unsigned long long ld_agent64(const float* p) {
    return __hip_atomic_load((const unsigned long long*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float2 u64_f2(unsigned long long v) {
    return make_float2(__uint_as_float((unsigned)v), __uint_as_float((unsigned)(v >> 32)));
}

// Decode: one workgroup of NW waves per (query row, KV head, context split); the G query heads
// of the KV head are the MFMA columns.
// The second bound is HIP's minimum waves per SIMD (amdgpu_waves_per_eu): 2 for the 4-wave
// form caps the register budget so two workgroups share a CU.
template <int HD, int G, int NW>
__global__ void __launch_bounds__(64 * NW, 8 / NW) k_attn_mf(const AttnArgs a) {
    constexpr int KC = HD / 32;  // 32-wide head-dim chunks of the score product
    constexpr int DB = HD / 16;  // 16-wide head-dim blocks of the value product
    constexpr int NT = 64 * NW;
    constexpr int HP = HD / 2;   // float2 pairs per head
    __shared__ float q_s[16][HD];
    __shared__ float w_m[NW][16], w_l[NW][16];
    __shared__ float w_o[NW][G][HD];
    __shared__ float f_s[MAX_SPLITS][G];  // split maxima, then their merge weights
    __shared__ float m_s[MAX_SPLITS][G];  // split sums
    __shared__ float L_s[G];
    __shared__ int s_last;

    const int b = blockIdx.z, h = blockIdx.y, sp = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;

    // q first: its address depends on nothing loaded
    constexpr int QPT = 16 * HD / NT;
    float qreg[QPT];
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = threadIdx.x + k * NT;
        qreg[k] = i / HD < G ? a.q[((int64_t)b * a.nq + h * G) * HD + i] : 0.f;
    }
    const int64_t off = a.static_off ? a.off_val[b] : a.boff[b];
    const int r0 = sp * a.split_rows;
    const int64_t head = (int64_t)h * a.kv.kv_rows * HD;
    AttnWave<HD, NW, false> aw{(const __half*)a.kv.k + head, (const __half*)a.kv.v + head, off,
                               (off & 63) == 0 && (a.kv.kv_rows & 7) == 0, ((off | a.kv.kv_rows) & 7) == 0,
                               r0, 0, 0, 0};
    aw.wv = wave;
    // first tile requested before the sequence length is known, when it lies in the region and
    // in the split's rows (a tile past the split bound is never used)
    const int tfirst = r0 + wave * AttnWave<HD, NW, false>::TR;
    const bool spec = a.static_off && aw.tiled && tfirst + AttnWave<HD, NW, false>::TR <= a.cap_rows &&
                      tfirst < r0 + a.split_rows;
    if (spec) aw.load_full(aw.A, tfirst);
    int len;
    if (a.seq_len) {
        len = a.seq_len[b];
    } else {
        len = a.pos[b] + 1;
        if (a.kv.max_context > 0) len = min(len, a.kv.max_context);
    }
    const int r1 = min(len, r0 + a.split_rows);
    aw.r1 = aw.lim = aw.lim_all = r1;
    if (!spec) aw.start();  // (a partial first tile's V rows past r1 are zeroed by compute())

    // q rows into LDS, then Q^T as the B operand:
    // lane (lr, lg) holds head lr, head-dim kc*32 + 8lg .. +7
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = threadIdx.x + k * NT;
        q_s[i / HD][i % HD] = qreg[k] * (1.4426950408889634f / sqrtf((float)HD));
    }
    __syncthreads();
    half8 qh[KC], ql[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) split_hl(&q_s[lr][kc * 32 + 8 * lg], qh[kc], ql[kc]);

    float m = -INFINITY, l = 0.f;
    f32x4 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    aw.run(qh, ql, m, l, o);

    // combine the waves: log-sum-exp weights, summed in wave order
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (lg == 0) {
        w_m[wave][lr] = m;
        w_l[wave][lr] = l;
    }
    // O^T D layout: lane holds head lr, head-dim db*16 + 4lg + v
    if (lr < G) {
#pragma unroll
        for (int db = 0; db < DB; ++db)
#pragma unroll
            for (int v = 0; v < 4; ++v) w_o[wave][lr][db * 16 + 4 * lg + v] = o[db][v];
    }
    __syncthreads();

    const int64_t hq0 = (int64_t)b * a.nq + h * G;   // first query head of this KV head
    const int64_t bh = (int64_t)b * a.nkv + h;
    const int S = a.splits;
    float sink = 0.f;
    for (int i = threadIdx.x; i < G * HP; i += NT) {
        const int g = i / HP, d = 2 * (i % HP);
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, w_m[w][g]);
        float L = 0.f, O0 = 0.f, O1 = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float f = w_m[w][g] == -INFINITY ? 0.f : exp2f(w_m[w][g] - M);
            L += w_l[w][g] * f;
            O0 += w_o[w][g][d] * f;
            O1 += w_o[w][g][d + 1] * f;
        }
        if (S == 1) {
            const float r = L > 0.f ? 1.0f / L : 0.f;
            *(float2*)&a.out[(hq0 + g) * HD + d] = make_float2(O0 * r, O1 * r);
        } else {
            // partials [b][kv head][split][G][HD] and (m, l) [b][kv head][split][G]
            const unsigned long long ov =
                (unsigned long long)__float_as_uint(O0) | ((unsigned long long)__float_as_uint(O1) << 32);
            float* po = a.part_o + ((bh * S + sp) * G + g) * HD + d;
            sink += __uint_as_float((unsigned)__hip_atomic_exchange((unsigned long long*)po, ov, __ATOMIC_RELAXED,
                                                                    __HIP_MEMORY_SCOPE_AGENT));
            if (d == 0) {
                const unsigned long long mv =
                    (unsigned long long)__float_as_uint(M) | ((unsigned long long)__float_as_uint(L) << 32);
                float* pm = a.part_ml + ((bh * S + sp) * G + g) * 2;
                sink += __uint_as_float((unsigned)__hip_atomic_exchange((unsigned long long*)pm, mv, __ATOMIC_RELAXED,
                                                                        __HIP_MEMORY_SCOPE_AGENT));
            }
        }
    }
    if (S == 1) return;
    asm volatile("" ::"v"(sink));  // the returned values are consumed: the exchanges have completed
    __syncthreads();
    if (threadIdx.x == 0)
        s_last = __hip_atomic_fetch_add(&a.cnt[bh], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!s_last) return;

    // last workgroup of (b, h): every split's (m, l) into LDS in one round of loads, then per
    // head M = max m_s, weights f_s = 2^(m_s - M), L = sum l_s f_s
    const float* pml = a.part_ml + bh * S * G * 2;
    for (int i = threadIdx.x; i < S * G; i += NT) {
        const float2 ml = u64_f2(ld_agent64(pml + (int64_t)i * 2));
        f_s[i / G][i % G] = ml.x;
        m_s[i / G][i % G] = ml.y;
    }
    __syncthreads();
    for (int g = wave; g < G; g += NW) {
        float mx = -INFINITY;
        for (int s2 = lane; s2 < S; s2 += 64) mx = fmaxf(mx, f_s[s2][g]);
        mx = wave_max(mx);
        float sum = 0.f;
        for (int s2 = lane; s2 < S; s2 += 64) {
            const float ms = f_s[s2][g];
            const float f = ms == -INFINITY ? 0.f : exp2f(ms - mx);
            f_s[s2][g] = f;
            sum += m_s[s2][g] * f;
        }
        sum = wave_sum(sum);
        if (lane == 0) L_s[g] = sum;
    }
    __syncthreads();
    const float* po = a.part_o + bh * S * G * HD;
    constexpr int U = 32;
    for (int i = threadIdx.x; i < G * HP; i += NT) {
        const int g = i / HP, d = 2 * (i % HP);
        float O0 = 0.f, O1 = 0.f;
        for (int s0 = 0; s0 < S; s0 += U) {
            unsigned long long v[U];
#pragma unroll
            for (int k = 0; k < U; ++k) v[k] = ld_agent64(po + ((int64_t)min(s0 + k, S - 1) * G + g) * HD + d);
#pragma unroll
            for (int k = 0; k < U; ++k) {
                if (s0 + k < S) {
                    const float2 x = u64_f2(v[k]);
                    const float f = f_s[s0 + k][g];
                    O0 += x.x * f;
                    O1 += x.y * f;
                }
            }
        }
        const float r = L_s[g] > 0.f ? 1.0f / L_s[g] : 0.f;
        *(float2*)&a.out[(hq0 + g) * HD + d] = make_float2(O0 * r, O1 * r);
    }
    if (threadIdx.x == 0) __hip_atomic_store(&a.cnt[bh], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Prefill: one workgroup of NW waves per (16 consecutive query tokens of one sequence, query
// head); the tokens are the MFMA columns, each masked at its causal limit pos + 1
// (flash_attention_cpu, cpu_engine.rs:1151-1272: kv_len = start_pos + b + 1). K/V rows are
// shared by the 16 tokens, so the cache is read once per 16 queries of a head.
// At least two waves per SIMD (the second bound is amdgpu_waves_per_eu): with the compiler's
// default register budget one wave per SIMD ran, and the tile loads had nothing to hide behind
// (7B-width prefill over 2047 tokens: 223 -> 131 us per layer).
template <int HD, int NW>
__global__ void __launch_bounds__(64 * NW, 2) k_attn_pf(const AttnArgs a) {
    constexpr int KC = HD / 32, DB = HD / 16, NT = 64 * NW;
    __shared__ float q_s[16][HD];
    __shared__ float w_m[NW][16], w_l[NW][16];
    __shared__ float w_o[NW][16][HD + 4];

    const int t0 = blockIdx.x * 16, hq = blockIdx.y;
    const int h = hq / (a.nq / a.nkv);
    const int ntok = min(16, a.batch - t0);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lr = lane & 15, lg = lane >> 4;

    constexpr int QPT = 16 * HD / NT;
    float qreg[QPT];
#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = threadIdx.x + k * NT;
        qreg[k] = i / HD < ntok ? a.q[((int64_t)(t0 + i / HD) * a.nq + hq) * HD + i % HD] : 0.f;
    }
    const int64_t off = a.boff[t0];  // every 16-token group lies in one sequence
    int lim = 0;
    if (lr < ntok) {
        lim = a.pos[t0 + lr] + 1;
        if (a.kv.max_context > 0) lim = min(lim, a.kv.max_context);
    }
    int r1 = lim;
#pragma unroll
    for (int sh = 8; sh > 0; sh >>= 1) r1 = max(r1, __shfl_xor(r1, sh));
    const int64_t head = (int64_t)h * a.kv.kv_rows * HD;
    int lim_all = lr < ntok ? lim : 0x7fffffff;  // columns past the chunk never bind
#pragma unroll
    for (int sh = 8; sh > 0; sh >>= 1) lim_all = min(lim_all, __shfl_xor(lim_all, sh));
    AttnWave<HD, NW, true> aw{(const __half*)a.kv.k + head, (const __half*)a.kv.v + head, off,
                              (off & 63) == 0 && (a.kv.kv_rows & 7) == 0, ((off | a.kv.kv_rows) & 7) == 0,
                              0, r1, lim, __builtin_amdgcn_readfirstlane(lim_all)};
    aw.wv = wave;
    aw.start();

#pragma unroll
    for (int k = 0; k < QPT; ++k) {
        const int i = threadIdx.x + k * NT;
        q_s[i / HD][i % HD] = qreg[k] * (1.4426950408889634f / sqrtf((float)HD));
    }
    __syncthreads();
    half8 qh[KC], ql[KC];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) split_hl(&q_s[lr][kc * 32 + 8 * lg], qh[kc], ql[kc]);
    float m = -INFINITY, l = 0.f;
    f32x4 o[DB];
#pragma unroll
    for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
    aw.run(qh, ql, m, l, o);

    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    if (lg == 0) {
        w_m[wave][lr] = m;
        w_l[wave][lr] = l;
    }
#pragma unroll
    for (int db = 0; db < DB; ++db)
#pragma unroll
        for (int v = 0; v < 4; ++v) w_o[wave][lr][db * 16 + 4 * lg + v] = o[db][v];
    __syncthreads();
    for (int i = threadIdx.x; i < ntok * HD; i += NT) {
        const int c = i / HD, d = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) M = fmaxf(M, w_m[w][c]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) {
            const float f = w_m[w][c] == -INFINITY ? 0.f : exp2f(w_m[w][c] - M);
            L += w_l[w][c] * f;
            O += w_o[w][c][d] * f;
        }
        a.out[((int64_t)(t0 + c) * a.nq + hq) * HD + d] = L > 0.f ? O * (1.0f / L) : 0.f;
    }
}

template <int HD, int KVF16, int G>
hipError_t launch_t(const AttnArgs& a, hipStream_t st) {
    if constexpr (KVF16) {
        // 8 waves once a split holds more than 4 tiles, so that every wave's first tile (requested
        // at kernel start) covers as much of the context as possible
        if (a.split_rows > 4 * 32 * KvTile<HD>::NJ)
            launch_kernel((k_attn_mf<HD, G, 8>), dim3(a.splits, a.nkv, a.batch), dim3(512), 0, st, a);
        else launch_kernel((k_attn_mf<HD, G, 4>), dim3(a.splits, a.nkv, a.batch), dim3(256), 0, st, a);
    } else launch_kernel((k_attn<HD, 0, G>), dim3(a.splits, a.nkv, a.batch), dim3(256), 0, st, a);
    return hipGetLastError();
}

template <int HD, int KVF16>
hipError_t launch_g(const AttnArgs& a, hipStream_t st) {
    switch (a.nq / a.nkv) {
        case 1: return launch_t<HD, KVF16, 1>(a, st);
        case 2: return launch_t<HD, KVF16, 2>(a, st);
        case 4: return launch_t<HD, KVF16, 4>(a, st);
        case 7: return launch_t<HD, KVF16, 7>(a, st);
        case 8: return launch_t<HD, KVF16, 8>(a, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// Context split. Up to 1024 rows a (row, KV head) stays in one workgroup (each wave takes at
// most two 64-row tiles, cheaper than a merge). Longer contexts are cut into splits of at
// least 64 KiB of K and V per head (512 rows at head_dim 64, 256 at 128), as many as it takes
// to give the chip about one workgroup per CU, at most 128: the merge's last workgroup reads
// every split's partials, so fewer, longer splits win (T = 32768: 21.9 -> 14.5 us at batch 1,
// 37.8 -> 31.6 at 8; T = 4096, batch 32: 24.8 -> 19.7 us against 512 workgroups of 256-row
// splits). Splits of more than 4 tiles run 8 waves per workgroup, shorter ones 4.
constexpr int ATTN_TARGET_WG = 256;
constexpr int ATTN_MIN_ROWS_HD64 = 512;
void attn_plan(int max_len, int batch, int nkv, int hd, int* splits, int* split_rows) {
    // the bound is rounded up (64, 128, 256, 512, 1024, then multiples of 1024) so that a decode
    // graph captured for it stays valid while the context grows: rows past a sequence's length
    // cost a skipped tile or an empty split, a new plan costs a graph capture
    max_len = std::max(max_len, 1);
    if (max_len <= 512) {
        int b = 64;
        while (b < max_len) b *= 2;
        max_len = b;
    } else {
        max_len = (max_len + 1023) / 1024 * 1024;
    }
    if (max_len <= 1024) {
        *splits = 1;
        *split_rows = max_len;
        return;
    }
    const int heads = std::max(batch * nkv, 1);
    const int want = std::max(1, (ATTN_TARGET_WG + heads - 1) / heads);
    int rows = (max_len + want - 1) / want;
    rows = std::max(rows, ATTN_MIN_ROWS_HD64 * 64 / std::max(hd, 64));
    rows = std::max(rows, (max_len + MAX_SPLITS - 1) / MAX_SPLITS);
    rows = (rows + 63) / 64 * 64;
    *splits = (max_len + rows - 1) / rows;
    *split_rows = rows;
}

bool attn_supported(int nq, int nkv, int hd) {
    if (nkv <= 0 || nq % nkv) return false;
    const int g = nq / nkv;
    return (hd == 64 || hd == 128) && (g == 1 || g == 2 || g == 4 || g == 7 || g == 8);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    if (!attn_supported(a.nq, a.nkv, a.hd)) return hipErrorInvalidValue;
    if (a.prefill && a.kv.kv_f16) {
        if (a.batch <= 0 || !a.pos || !a.boff) return hipErrorInvalidValue;
        const dim3 grid((a.batch + 15) / 16, a.nq);
        if (a.hd == 64) launch_kernel((k_attn_pf<64, 4>), grid, dim3(256), 0, st, a);
        else launch_kernel((k_attn_pf<128, 4>), grid, dim3(256), 0, st, a);
        return hipGetLastError();
    }
    if (a.splits > MAX_SPLITS || (a.splits > 1 && !a.cnt)) return hipErrorInvalidValue;
    if (a.hd == 64) return a.kv.kv_f16 ? launch_g<64, 1>(a, st) : launch_g<64, 0>(a, st);
    return a.kv.kv_f16 ? launch_g<128, 1>(a, st) : launch_g<128, 0>(a, st);
}

}  // namespace bh
