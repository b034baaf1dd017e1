// k_attn.hip — GQA decode attention over the device-resident packed KV cache.
//
// Reference semantics: flash_attention_single_into (src/inference/cpu_engine.rs:1450-1509):
// per query head, online softmax over the cached rows of its KV head
// (kv head = q head / (n_q / n_kv)), scores (q . k) * (1/sqrt(hd)), output o * (1/l).
//
// Design: one workgroup per (query row, KV head, context split). The G = n_q/n_kv
// query heads that share a KV head are processed together, so every K/V byte is
// read once per workgroup instead of once per query head (the reference re-reads
// each KV head's rows G times). Each wavefront takes 64-row tiles and requests the
// tile's K rows (lane t owns row t, 16-byte loads) and V rows (8 rows per step for
// hd 64, 16-byte loads) together before computing: scores use q broadcast from LDS,
// probabilities move between lanes with ds_bpermute. G is a compile-time constant
// so all per-head state stays in registers. Splits of long contexts publish
// (m, l, o) partials; the last workgroup of a (row, KV head) to finish merges them
// with log-sum-exp weights (flash-decoding) — no second kernel.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

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

    int64_t off;
    int len;
    if (a.seq_len) {
        off = a.seq_off[b];
        len = a.seq_len[b];
    } else {
        off = a.seq_off[a.slot[b]];
        len = a.pos[b] + 1;
        if (a.kv.max_context > 0) len = min(len, a.kv.max_context);
    }
    const int r0 = sp * a.split_rows;
    const int r1 = min(len, r0 + a.split_rows);

    for (int i = threadIdx.x; i < G * HD; i += blockDim.x)
        q_s[i / HD][i % HD] = a.q[((int64_t)b * a.nq + h * G) * HD + i];
    __syncthreads();

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

    for (int t0 = r0 + wave * 64; t0 < r1; t0 += 4 * 64) {
        const int t = t0 + lane;
        const bool valid = t < r1;
        // request the tile's K and V rows together
        Row8<KVF16> kr[HD / 8], vr[NV];
#pragma unroll
        for (int dc = 0; dc < HD / 8; ++dc) {
            if (valid) kr[dc].load(a.kv.k, kv_base + (int64_t)t * HD + dc * 8);
            else kr[dc].zero();
        }
#pragma unroll
        for (int j = 0; j < NV; ++j) {
            const int t2 = t0 + j * TS + tsub;
            if (t2 < r1) vr[j].load(a.kv.v, kv_base + (int64_t)t2 * HD + dl * 8);
            else vr[j].zero();
        }
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
            a.out[(hq0 + g) * HD + d] = O * (1.0f / L);
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
        a.out[(hq0 + g) * HD + d] = O * (1.0f / L_s[g]);
    }
    if (threadIdx.x == 0) a.cnt[b * a.nkv + h] = 0;  // ready for the next launch
}

template <int HD, int KVF16, int G>
hipError_t launch_t(const AttnArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((k_attn<HD, KVF16, G>), dim3(a.splits, a.nkv, a.batch), dim3(256), 0, st, a);
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

// Context split: 256 rows per workgroup (one 64-row tile per wave); 64 when that leaves
// fewer than 256 workgroups; at most 128 splits (longer splits loop over tiles).
void attn_plan(int max_len, int batch, int nkv, int* splits, int* split_rows) {
    max_len = std::max(max_len, 1);
    int rows = 256;
    if ((int64_t)((max_len + 255) / 256) * nkv * batch < 256) rows = 64;
    int s = (max_len + rows - 1) / rows;
    if (s > MAX_SPLITS) {
        rows = ((max_len + MAX_SPLITS - 1) / MAX_SPLITS + 255) / 256 * 256;
        s = (max_len + rows - 1) / rows;
    }
    *splits = s;
    *split_rows = rows;
}

bool attn_supported(int nq, int nkv, int hd) {
    if (nkv <= 0 || nq % nkv) return false;
    const int g = nq / nkv;
    return (hd == 64 || hd == 128) && (g == 1 || g == 2 || g == 4 || g == 7 || g == 8);
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    if (!attn_supported(a.nq, a.nkv, a.hd) || a.splits > MAX_SPLITS || (a.splits > 1 && !a.cnt))
        return hipErrorInvalidValue;
    if (a.hd == 64) return a.kv.kv_f16 ? launch_g<64, 1>(a, st) : launch_g<64, 0>(a, st);
    return a.kv.kv_f16 ? launch_g<128, 1>(a, st) : launch_g<128, 0>(a, st);
}

}  // namespace bh
