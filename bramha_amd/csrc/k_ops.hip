// k_ops.hip — the small per-token kernels of the decode step.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_xl.h"

namespace bh {
namespace {

__device__ __forceinline__ float block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float s = 0.f;
    for (int w = 0; w < nw; ++w) s += red[w];
    __syncthreads();
    return s;
}

// rms_norm_into (cpu_engine.rs:1292-1302): out = x * (1/sqrt(mean(x^2) + eps)) * w.
__global__ void __launch_bounds__(256) k_rmsnorm(const float* __restrict__ x, const float* __restrict__ w, float eps,
                                                 float* __restrict__ out, int n) {
    __shared__ float red[16];
    const float* xr = x + (int64_t)blockIdx.x * n;
    float* orow = out + (int64_t)blockIdx.x * n;
    float s = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) s += xr[i] * xr[i];
    s = block_sum(s, red);
    const float var = s / (float)n;
    const float scale = 1.0f / sqrtf(var + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) orow[i] = xr[i] * scale * w[i];
}

// apply_rope_cpu (cpu_engine.rs:1682-1699) with a host-computed (cos, sin) table.
__global__ void k_rope(float* __restrict__ v, const int32_t* __restrict__ pos, const float2* __restrict__ tab,
                       int n_heads, int hd) {
    const int row = blockIdx.x, half = hd >> 1;
    const int p = pos[row];
    float* vr = v + (int64_t)row * n_heads * hd;
    for (int i = threadIdx.x; i < n_heads * half; i += blockDim.x) {
        const int h = i / half, d = i % half;
        const float2 cs = tab[(int64_t)p * half + d];
        const float x1 = vr[h * hd + d], x2 = vr[h * hd + d + half];
        vr[h * hd + d] = x1 * cs.x - x2 * cs.y;
        vr[h * hd + d + half] = x2 * cs.x + x1 * cs.y;
    }
}

// cpu_engine.rs:2023-2026
__global__ void k_silu_mul(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ out,
                           int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float gv = g[i];
        out[i] = gv * (1.0f / (1.0f + expf(-gv))) * u[i];
    }
}

// Dequantize KM16 chunks back to the reference row-major f32 layout:
// (q - 8) * scale / q * scale (quantization.rs:86-122). Each product is the single
// rounding the reference performs, so the values are bit-identical.
__global__ void k_dequant(int fmt, const uint4* __restrict__ Q, const void* __restrict__ S, int64_t n, int64_t k,
                          int64_t n_pad, int64_t C, float* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * C) return;
    const int64_t row = t % n, c = t / n;
    const uint4 q = Q[c * n_pad + row];
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    float* o = out + row * k;
    if (fmt == BH_Q4_ROW || fmt == BH_Q4_G32) {
        const float sc = fmt == BH_Q4_G32 ? __half2float(((const __half*)S)[c * n_pad + sc_pos(row)]) : ((const float*)S)[row];
        for (int j = 0; j < 16; ++j) {
            const uint32_t byte = (w[j >> 2] >> (8 * (j & 3))) & 0xFFu;
            o[c * 32 + 2 * j] = ((float)((byte >> 4) & 0x0F) - 8.0f) * sc;
            o[c * 32 + 2 * j + 1] = ((float)(byte & 0x0F) - 8.0f) * sc;
        }
    } else if (fmt == BH_Q8_ROW) {
        const float sc = ((const float*)S)[row];
        for (int j = 0; j < 16; ++j) {
            const int8_t b = (int8_t)((w[j >> 2] >> (8 * (j & 3))) & 0xFFu);
            o[c * 16 + j] = (float)b * sc;
        }
    } else {
        for (int j = 0; j < 4; ++j) o[c * 4 + j] = __uint_as_float(w[j]);
    }
}

// Element i of row `id` of the tied embedding table in KM16 layout (F32 or Q4_G32):
// the embedding row copy of cpu_engine.rs:2820-2825, dequantized bit-exactly like
// dequantize_int4 (quantization.rs:102-122) with the group's fp16 scale.
__device__ __forceinline__ float embed_elem(const DevWeight& t, int64_t id, int i) {
    const int64_t c = t.fmt == BH_F32 ? (i >> 2) : (i >> 5);
    if (t.fmt == BH_F32) return ((const float*)t.q)[(c * t.n_pad + id) * 4 + (i & 3)];
    const uint8_t byte = ((const uint8_t*)t.q)[(c * t.n_pad + id) * 16 + ((i & 31) >> 1)];
    const float nib = (i & 1) ? (float)(byte & 0x0F) : (float)((byte >> 4) & 0x0F);
    return (nib - 8.0f) * __half2float(((const __half*)t.s)[c * t.n_pad + sc_pos(id)]);
}

// Residual stream of token row b from embedding row `id`: x, xw = x * w0, and per-64-element
// sums of squares (one wave per tile, a fixed shuffle order); with xl, xw's limb records too.
__device__ __forceinline__ void embed_stream(const DevWeight& t, int64_t id, const float* w0, float* x, float* xw,
                                             float* ssq, int ssq_tiles, int b, uint32_t* xl) {
    const int hidden = (int)t.k;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    float* xr = x + (int64_t)b * hidden;
    float* xwr = xw + (int64_t)b * hidden;
    for (int tl = wave; tl < ssq_tiles; tl += nw) {
        const int i = tl * 64 + lane;
        float v = 0.f, vw = 0.f;
        if (i < hidden) {
            v = embed_elem(t, id, i);
            xr[i] = v;
            vw = v * w0[i];
            xwr[i] = vw;
        }
        float sq = v * v;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
        if (lane == 0) ssq[(int64_t)b * ssq_tiles + tl] = sq;
        if (xl) xl_pack64(vw, xl, 2 * tl, (hidden + 31) / 32);
    }
}

__global__ void __launch_bounds__(256) k_embed(const DevWeight t, const int32_t* __restrict__ tok,
                                               const float* __restrict__ w0, float* x, float* xw, float* ssq,
                                               int ssq_tiles, int32_t* reset_step, uint32_t* xl) {
    const int b = blockIdx.x;
    const int64_t id = (int64_t)((uint32_t)tok[b] % (uint64_t)t.n);
    if (reset_step && threadIdx.x == 0) reset_step[b] = 0;
    embed_stream(t, id, w0, x, xw, ssq, ssq_tiles, b, b == 0 ? xl : nullptr);
}

// End of a decode step for batch entry b = blockIdx.x: the first-max argmax over the LM head's
// per-tile partials (cpu_engine.rs:3024-3031; ties keep the lowest id), the penalty count of the
// chosen id, the id capture, the next token and position, and the next step's residual stream.
// Sort keys so that the larger value comes first, equal values by ascending index (the order of
// the reference's stable sort by probability). n is a power of two; all threads take part.
__device__ __forceinline__ bool sorts_before(float va, int ia, float vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}
__device__ void bitonic_sort(float* v, int* id, int n) {
    for (int k = 2; k <= n; k <<= 1)
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += blockDim.x) {
                const int l = i ^ j;
                if (l <= i) continue;
                const bool up = (i & k) == 0;
                const bool swap = up ? sorts_before(v[l], id[l], v[i], id[i]) : sorts_before(v[i], id[i], v[l], id[l]);
                if (swap) {
                    const float tv = v[i];
                    v[i] = v[l];
                    v[l] = tv;
                    const int ti = id[i];
                    id[i] = id[l];
                    id[l] = ti;
                }
            }
            __syncthreads();
        }
}

constexpr int SORT_N = 4096;  // tiles of 64 logits for vocabularies up to 262144; 64 x top_k candidates

// Top-k sampling of entry b (temperature > 0): the k largest penalized logits lie in the k tiles
// with the largest tile maxima (each of those k logits is at most its tile's maximum), so the
// tile maxima are sorted first, the k best tiles' 64 k penalized logits second; then
// p_i = exp(l_i/T - l_0/T) / sum over the k, and the first i whose cumulative p reaches the draw
// r is chosen (the first one if rounding leaves every cumulative sum below r). The reference
// normalises over the whole vocabulary first and again over the k (cpu_engine.rs:3003-3014);
// both give the same top-k distribution.
__device__ int sample_topk(const SampleArgs& a, int b, int slot, int pos, float* v, int* id) {
    __shared__ int tsel[SAMPLE_TOPK_MAX];
    __shared__ int s_pick;
    const int K = a.top_k;
    for (int i = threadIdx.x; i < SORT_N; i += blockDim.x) {
        v[i] = i < a.tiles ? a.part_val[(int64_t)b * a.tiles + i] : -INFINITY;
        id[i] = i < a.tiles ? i : 0x7fffffff;
    }
    __syncthreads();
    bitonic_sort(v, id, SORT_N);
    if (threadIdx.x < K) tsel[threadIdx.x] = id[threadIdx.x];
    __syncthreads();
    const uint16_t* pen = a.pen + (int64_t)slot * a.vocab;
    for (int e = threadIdx.x; e < SORT_N; e += blockDim.x) {
        float val = -INFINITY;
        int n = 0x7fffffff;
        if (e < K * 64) {
            const int tile = tsel[e / 64];
            const int nn = tile == 0x7fffffff ? a.vocab : tile * 64 + e % 64;
            if (nn < a.vocab) {
                val = a.logits[(int64_t)b * a.vocab + nn];
                for (int c = pen[nn]; c > 0; --c) val = val > 0.f ? val / 1.15f : val * 1.15f;
                if (!(val > -INFINITY)) val = -INFINITY;  // NaN is never chosen
                n = nn;
            }
        }
        v[e] = val;
        id[e] = n;
    }
    __syncthreads();
    bitonic_sort(v, id, SORT_N);
    if (threadIdx.x == 0) {
        const float inv = 1.0f / a.temperature;
        const float mx = v[0] * inv;
        float ex[SAMPLE_TOPK_MAX];
        float sum = 0.f;
        for (int i = 0; i < K; ++i) {
            ex[i] = v[i] > -INFINITY ? expf(v[i] * inv - mx) : 0.f;
            sum += ex[i];
        }
        const float r = sample_uniform(a.seed, slot, pos);
        int pick = id[0];
        float cum = 0.f;
        for (int i = 0; i < K; ++i) {
            cum += ex[i] / sum;
            if (r <= cum) {
                pick = id[i];
                break;
            }
        }
        s_pick = pick;
    }
    __syncthreads();
    return s_pick;
}

__device__ __forceinline__ void argmax_take(float& v, int& i, float ov, int oi) {
    if (ov > v || (ov == v && oi < i)) {
        v = ov;
        i = oi;
    }
}

constexpr int SAMPLE_THREADS = 1024;

__global__ void __launch_bounds__(SAMPLE_THREADS) k_sample(const SampleArgs a, const DevWeight t) {
    __shared__ float sv[SAMPLE_THREADS / 64];
    __shared__ int si[SAMPLE_THREADS / 64];
    __shared__ int s_id;
    __shared__ float sort_v[SORT_N];
    __shared__ int sort_i[SORT_N];
    const int b = blockIdx.x;
    if (a.temperature > 0.f) {
        const int slot = a.slot[b];
        const int idx = sample_topk(a, b, slot, a.pos[b], sort_v, sort_i);
        if (threadIdx.x == 0) {
            uint16_t* c = a.pen + (int64_t)slot * a.vocab + idx;
            if (*c < 0xFFFF) *c = *c + 1;
            if (a.ids_cap) {
                const int s = a.step[b];
                a.ids_cap[(int64_t)s * a.batch + b] = (uint32_t)idx;
                a.step[b] = s + 1;
            }
            a.tok[b] = idx;
            a.pos[b] = a.pos[b] + 1;
        }
        embed_stream(t, idx, a.w0, a.x, a.xw, a.ssq, a.ssq_tiles, b, b == 0 ? a.xl : nullptr);
        return;
    }
    // Greedy. What does not depend on the chosen id is requested first, in one round of loads:
    // every tile partial (PT per thread), the entry's slot, step and position, and the next norm
    // weight of the residual elements this thread writes (EW tiles per wave); the id then costs
    // one more round (its embedding row, and the penalty count, updated after the barrier).
    constexpr int PT = 4, EW = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const float* pvb = a.part_val + (int64_t)b * a.tiles;
    const int32_t* pib = a.part_idx + (int64_t)b * a.tiles;
    float pv[PT];
    int pi[PT];
#pragma unroll
    for (int k = 0; k < PT; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        pv[k] = i < a.tiles ? pvb[i] : -INFINITY;
        pi[k] = i < a.tiles ? pib[i] : 0x7fffffff;
    }
    int slot = 0, step = 0, pos = 0;
    if (threadIdx.x == 0) {
        slot = a.slot[b];
        pos = a.pos[b];
        if (a.ids_cap) step = a.step[b];
    }
    const int hidden = (int)t.k;
    float w0v[EW];
#pragma unroll
    for (int k = 0; k < EW; ++k) {
        const int i = (wave + k * nw) * 64 + lane;
        w0v[k] = i < hidden ? a.w0[i] : 0.f;
    }
    float v = -INFINITY;
    int idx = 0x7fffffff;
#pragma unroll
    for (int k = 0; k < PT; ++k) argmax_take(v, idx, pv[k], pi[k]);
    for (int i = threadIdx.x + PT * blockDim.x; i < a.tiles; i += blockDim.x) argmax_take(v, idx, pvb[i], pib[i]);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) argmax_take(v, idx, __shfl_xor(v, off), __shfl_xor(idx, off));
    if (lane == 0) {
        sv[wave] = v;
        si[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < nw; ++w) argmax_take(v, idx, sv[w], si[w]);
        if (idx == 0x7fffffff) idx = 0;  // no finite logit: the scan keeps index 0
        if (a.ids_cap) {
            a.ids_cap[(int64_t)step * a.batch + b] = (uint32_t)idx;
            a.step[b] = step + 1;
        }
        a.tok[b] = idx;
        a.pos[b] = pos + 1;
        s_id = idx;
    }
    __syncthreads();
    const int id = s_id;
    if (threadIdx.x == 0) {  // penalty count of the chosen id (cpu_engine.rs:2984-2992 counts it)
        uint16_t* c = a.pen + (int64_t)slot * a.vocab + id;
        if (*c < 0xFFFF) *c = *c + 1;
    }
    // next step's residual stream from the embedding row (embed_stream with the weights loaded)
    float* xr = a.x + (int64_t)b * hidden;
    float* xwr = a.xw + (int64_t)b * hidden;
    uint32_t* xl = b == 0 ? a.xl : nullptr;
    auto put = [&](int tl, float w) {
        const int i = tl * 64 + lane;
        float e = 0.f, ew = 0.f;
        if (i < hidden) {
            e = embed_elem(t, id, i);
            xr[i] = e;
            ew = e * w;
            xwr[i] = ew;
        }
        float sq = e * e;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) sq += __shfl_xor(sq, off);
        if (lane == 0) a.ssq[(int64_t)b * a.ssq_tiles + tl] = sq;
        if (xl) xl_pack64(ew, xl, 2 * tl, (hidden + 31) / 32);
    };
#pragma unroll
    for (int k = 0; k < EW; ++k)
        if (wave + k * nw < a.ssq_tiles) put(wave + k * nw, w0v[k]);
    for (int tl = wave + EW * nw; tl < a.ssq_tiles; tl += nw) {
        const int i = tl * 64 + lane;
        put(tl, i < hidden ? a.w0[i] : 0.f);
    }
}

// Cache rows <-> host-layout f32 rows (one thread per element, grid-stride).
__global__ void __launch_bounds__(256) k_kv_copy(const KvView kv, int nkv, int hd, int64_t row0, int64_t n, float* kh,
                                                 float* vh, int to_host) {
    const int64_t total = n * nkv * hd;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / (nkv * hd);
        const int rem = (int)(i % (nkv * hd));
        const int h = rem / hd, d = rem % hd;
        const int64_t row = row0 + r, head = (int64_t)h * kv.kv_rows * hd;
        if (kv.kv_f16) {
            __half* K = (__half*)kv.k + head + kv_k_off(row, d, hd);
            __half* V = (__half*)kv.v + head + kv_v_off(row, d, hd);
            if (to_host) {
                kh[i] = __half2float(*K);
                vh[i] = __half2float(*V);
            } else {
                *K = __float2half(kh[i]);
                *V = __float2half(vh[i]);
            }
        } else {
            float* K = (float*)kv.k + head + row * hd + d;
            float* V = (float*)kv.v + head + row * hd + d;
            if (to_host) {
                kh[i] = *K;
                vh[i] = *V;
            } else {
                *K = kh[i];
                *V = vh[i];
            }
        }
    }
}

}  // namespace

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* out, int rows, int n, hipStream_t st) {
    launch_kernel(k_rmsnorm, dim3(rows), dim3(256), 0, st, x, w, eps, out, n);
    return hipGetLastError();
}

hipError_t launch_rope(float* v, const int32_t* pos, const float2* tab, int rows, int n_heads, int hd, hipStream_t st) {
    launch_kernel(k_rope, dim3(rows), dim3(256), 0, st, v, pos, tab, n_heads, hd);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t st) {
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    launch_kernel(k_silu_mul, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0, st, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_kv_copy(const KvView& kv, int nkv, int hd, int64_t row0, int64_t n, float* kh, float* vh, int to_host,
                          hipStream_t st) {
    const int64_t total = n * nkv * hd;
    if (total <= 0) return hipSuccess;
    const int64_t blocks = std::min<int64_t>((total + 255) / 256, 16384);
    launch_kernel(k_kv_copy, dim3((unsigned)blocks), dim3(256), 0, st, kv, nkv, hd, row0, n, kh, vh, to_host);
    return hipGetLastError();
}

// Rows [row0, row0 + n) of a group-32 scale matrix from src ([C][n], the reference's row order)
// into dst ([C][n_pad], rows at sc_pos): one thread per scale.
__global__ void k_scatter_scales(uint16_t* __restrict__ dst, const uint16_t* __restrict__ src, int64_t row0, int64_t n,
                                 int64_t n_pad, int64_t C) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= n * C) return;
    const int64_t c = t / n, i = t % n;
    dst[c * n_pad + sc_pos(row0 + i)] = src[t];
}

hipError_t launch_scatter_scales(void* dst, const void* src, int64_t row0, int64_t n, int64_t n_pad, int64_t C,
                                 hipStream_t st) {
    const int64_t total = n * C;
    if (total <= 0) return hipSuccess;
    launch_kernel(k_scatter_scales, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, (uint16_t*)dst,
                  (const uint16_t*)src, row0, n, n_pad, C);
    return hipGetLastError();
}

hipError_t launch_dequant(const DevWeight& w, float* out, hipStream_t st) {
    const int64_t total = w.n * w.chunks;
    launch_kernel(k_dequant, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, w.fmt, (const uint4*)w.q,
                       w.s, w.n, w.k, w.n_pad, w.chunks, out);
    return hipGetLastError();
}

hipError_t launch_embed(const DevWeight& t, const int32_t* tok, const float* w0, float* x, float* xw, float* ssq,
                        int ssq_tiles, int32_t* reset_step, int batch, hipStream_t st, uint32_t* xl) {
    if (batch <= 0) return hipSuccess;
    if (ssq_tiles != (int)((t.k + 63) / 64)) return hipErrorInvalidValue;
    launch_kernel(k_embed, dim3(batch), dim3(256), 0, st, t, tok, w0, x, xw, ssq, ssq_tiles, reset_step, xl);
    return hipGetLastError();
}

hipError_t launch_sample(const SampleArgs& a, hipStream_t st) {
    if (a.batch <= 0) return hipSuccess;
    if (!a.table || a.ssq_tiles != (int)((a.table->k + 63) / 64) || (a.ids_cap && !a.step)) return hipErrorInvalidValue;
    if (a.temperature > 0.f && (!a.logits || a.top_k < 1 || a.top_k > SAMPLE_TOPK_MAX || a.tiles > SORT_N))
        return hipErrorInvalidValue;
    launch_kernel(k_sample, dim3(a.batch), dim3(SAMPLE_THREADS), 0, st, a, *a.table);
    return hipGetLastError();
}

}  // namespace bh
