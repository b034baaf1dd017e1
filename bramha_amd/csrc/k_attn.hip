// k_attn.hip — GQA decode attention over the device-resident packed KV cache.
//
// Reference semantics: flash_attention_single_into (src/inference/cpu_engine.rs:1450-1509):
// per query head, online softmax over the cached rows of its KV head
// (kv head = q head / (n_q / n_kv)), scores (q . k) * (1/sqrt(hd)), output o * (1/l).
//
// Design: one workgroup per (query row, KV head, context split). The G = n_q/n_kv
// query heads that share a KV head are processed together, so every K/V byte is
// read once per workgroup instead of once per query head (the reference re-reads
// each KV head's rows G times). Each wavefront takes 64-row tiles: in the score
// phase lane t owns row t (16-byte loads of its K row, q broadcast from LDS); in
// the value phase 8 (hd 64) or 4 (hd 128) rows are read per instruction with
// 16-byte loads and the probabilities move between lanes with ds_bpermute. Splits
// over long contexts write (m, l, o) partials that a second kernel merges with
// log-sum-exp weights (flash-decoding).
#include "bh_internal.h"

#include <hip/hip_fp16.h>

namespace bh {
namespace {

constexpr int MAXG = 8;

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
__device__ __forceinline__ void load8(const void* base, int64_t elem, float* f) {
    if constexpr (KVF16) {
        const uint4 u = *(const uint4*)((const __half*)base + elem);
        const __half2* h2 = (const __half2*)&u;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float2 t = __half22float2(h2[i]);
            f[2 * i] = t.x;
            f[2 * i + 1] = t.y;
        }
    } else {
        const float4 a = *(const float4*)((const float*)base + elem);
        const float4 b = *(const float4*)((const float*)base + elem + 4);
        f[0] = a.x; f[1] = a.y; f[2] = a.z; f[3] = a.w;
        f[4] = b.x; f[5] = b.y; f[6] = b.z; f[7] = b.w;
    }
}

template <int HD, int KVF16>
__global__ void __launch_bounds__(256) k_attn(const AttnArgs a) {
    constexpr int DL = HD / 8;   // lanes per row in the value phase
    constexpr int TS = 64 / DL;  // rows per value-phase step
    __shared__ float q_s[MAXG][HD];
    __shared__ float w_m[4][MAXG], w_l[4][MAXG];
    __shared__ float w_o[4][MAXG][HD];

    const int b = blockIdx.z, h = blockIdx.y, sp = blockIdx.x;
    const int G = a.nq / a.nkv;
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
    float m[MAXG], l[MAXG], o[MAXG][8];
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[g][e] = 0.f;
    }
    const int tsub = lane / DL, dl = lane % DL;

    for (int t0 = r0 + wave * 64; t0 < r1; t0 += 4 * 64) {
        const int t = t0 + lane;
        const bool valid = t < r1;
        float s[MAXG];
#pragma unroll
        for (int g = 0; g < MAXG; ++g) s[g] = 0.f;
        if (valid) {
#pragma unroll
            for (int dc = 0; dc < HD / 8; ++dc) {
                float kf[8];
                load8<KVF16>(a.kv.k, kv_base + (int64_t)t * HD + dc * 8, kf);
#pragma unroll
                for (int g = 0; g < MAXG; ++g) {
                    if (g < G) {
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
                }
            }
        }
        float pg[MAXG];
#pragma unroll
        for (int g = 0; g < MAXG; ++g) {
            if (g < G) {
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
        }
#pragma unroll
        for (int j = 0; j < 64 / TS; ++j) {
            const int tl = j * TS + tsub;
            const int t2 = t0 + tl;
            float vf[8];
            if (t2 < r1) {
                load8<KVF16>(a.kv.v, kv_base + (int64_t)t2 * HD + dl * 8, vf);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) vf[e] = 0.f;
            }
#pragma unroll
            for (int g = 0; g < MAXG; ++g) {
                if (g < G) {
                    const float pp = __shfl(pg[g], tl);
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[g][e] = fmaf(pp, vf[e], o[g][e]);
                }
            }
        }
    }
    // sum the value accumulators of the lanes that share a column slice
#pragma unroll
    for (int g = 0; g < MAXG; ++g) {
        if (g < G) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                float v = o[g][e];
#pragma unroll
                for (int x = DL; x < 64; x <<= 1) v += __shfl_xor(v, x);
                o[g][e] = v;
            }
        }
    }
    if (lane == 0)
        for (int g = 0; g < G; ++g) {
            w_m[wave][g] = m[g];
            w_l[wave][g] = l[g];
        }
    if (tsub == 0)
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 8; ++e) w_o[wave][g][dl * 8 + e] = o[g][e];
    __syncthreads();

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
        const int64_t hq = (int64_t)b * a.nq + h * G + g;
        if (a.splits == 1) {
            a.out[hq * HD + d] = O * (1.0f / L);
        } else {
            a.part_o[(hq * a.splits + sp) * HD + d] = O;
            if (d == 0) {
                a.part_ml[(hq * a.splits + sp) * 2] = M;
                a.part_ml[(hq * a.splits + sp) * 2 + 1] = L;
            }
        }
    }
}

// Log-sum-exp merge of the context splits.
__global__ void k_attn_combine(const AttnArgs a) {
    const int hq = blockIdx.x, b = blockIdx.y;
    const int64_t base = ((int64_t)b * a.nq + hq) * a.splits;
    float M = -INFINITY;
    for (int s = 0; s < a.splits; ++s) M = fmaxf(M, a.part_ml[(base + s) * 2]);
    for (int d = threadIdx.x; d < a.hd; d += blockDim.x) {
        float L = 0.f, O = 0.f;
        for (int s = 0; s < a.splits; ++s) {
            const float ms = a.part_ml[(base + s) * 2];
            const float f = ms == -INFINITY ? 0.f : expf(ms - M);
            L += a.part_ml[(base + s) * 2 + 1] * f;
            O += a.part_o[(base + s) * a.hd + d] * f;
        }
        a.out[((int64_t)b * a.nq + hq) * a.hd + d] = O * (1.0f / L);
    }
}

template <int HD, int KVF16>
hipError_t launch_t(const AttnArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((k_attn<HD, KVF16>), dim3(a.splits, a.nkv, a.batch), dim3(256), 0, st, a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || a.splits == 1) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(a.nq, a.batch), dim3(HD), 0, st, a);
    return hipGetLastError();
}

}  // namespace

void attn_plan(int max_len, int batch, int nkv, int* splits, int* split_rows) {
    if (max_len <= 256) {
        *splits = 1;
        *split_rows = std::max(64, (max_len + 63) / 64 * 64);
        return;
    }
    int rows = 256;
    while (rows > 64 && (int64_t)((max_len + rows - 1) / rows) * nkv * batch < 512) rows /= 2;
    int s = (max_len + rows - 1) / rows;
    if (s > 128) {
        rows = ((max_len + 127) / 128 + 63) / 64 * 64;
        s = (max_len + rows - 1) / rows;
    }
    *splits = s;
    *split_rows = rows;
}

hipError_t launch_attention(const AttnArgs& a, hipStream_t st) {
    if (a.nq % a.nkv != 0 || a.nq / a.nkv > MAXG) return hipErrorInvalidValue;
    if (a.hd == 64) return a.kv.kv_f16 ? launch_t<64, 1>(a, st) : launch_t<64, 0>(a, st);
    if (a.hd == 128) return a.kv.kv_f16 ? launch_t<128, 1>(a, st) : launch_t<128, 0>(a, st);
    return hipErrorInvalidValue;
}

}  // namespace bh
