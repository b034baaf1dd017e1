// k_ops.hip — the small per-token kernels of the decode step.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

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

// The residual add of the O / down projection (cpu_engine.rs:2937-2939, 2966-2968)
// followed by the next RMSNorm (rms_norm_into, :1292-1302), one workgroup per row:
// o = sum of the projection's split-K partial sums in split order (+ bias), x += o,
// h = x * (1/sqrt(mean(x^2) + eps)) * w. Holds up to 16 elements per thread (n <= 4096).
__global__ void __launch_bounds__(256) k_resid_norm(float* __restrict__ x, const float* __restrict__ part,
                                                    int splits, int64_t part_ld, const float* __restrict__ bias,
                                                    const float* __restrict__ w, float eps, float* __restrict__ h,
                                                    int n) {
    __shared__ float red[16];
    constexpr int MAXJ = 16;
    const int b = blockIdx.x;
    float* xr = x + (int64_t)b * n;
    float v[MAXJ];
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int i = threadIdx.x + j * blockDim.x;
        v[j] = 0.f;
        if (i < n) {
            float t = xr[i];
            if (splits > 0) {
                // all (up to 16) partial loads in flight at once: the index is clamped so
                // every load is in bounds, the add is masked past `splits`
                const float* pp = part + (int64_t)b * n + i;
                float pv[16];
#pragma unroll
                for (int s = 0; s < 16; ++s) pv[s] = pp[(int64_t)min(s, splits - 1) * part_ld];
                float o = 0.f;
#pragma unroll
                for (int s = 0; s < 16; ++s) o += s < splits ? pv[s] : 0.f;
                if (bias) o += bias[i];
                t = t + o;
                xr[i] = t;
            }
            v[j] = t;
            ss += t * t;
        }
    }
    ss = block_sum(ss, red);
    const float scale = 1.0f / sqrtf(ss / (float)n + eps);
    float* hr = h + (int64_t)b * n;
#pragma unroll
    for (int j = 0; j < MAXJ; ++j) {
        const int i = threadIdx.x + j * blockDim.x;
        if (i < n) hr[i] = v[j] * scale * w[i];
    }
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
        const float sc = fmt == BH_Q4_G32 ? __half2float(((const __half*)S)[c * n_pad + row]) : ((const float*)S)[row];
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

// Embedding row copy (cpu_engine.rs:2820-2825, id % vocab) from the tied table in KM16
// layout. With the decode prologue, the token comes from the previous step's argmax
// and the position from the sequence's row count, which advances by one.
__global__ void __launch_bounds__(256) k_embed(int fmt, const uint4* __restrict__ Q, const __half* __restrict__ S,
                                               int64_t vocab, int64_t n_pad, int hidden, int32_t* tok, int32_t* pos,
                                               const int32_t* slot, int32_t* seq_len, const uint32_t* next,
                                               int prologue, float* x, int64_t ldx) {
    __shared__ int32_t s_tok;
    const int b = blockIdx.x;
    if (threadIdx.x == 0) {
        int32_t t;
        if (prologue) {
            t = (int32_t)next[b];
            tok[b] = t;
            const int s = slot[b];
            const int32_t p = seq_len[s];
            pos[b] = p;
            seq_len[s] = p + 1;
        } else {
            t = tok[b];
        }
        s_tok = t;
    }
    __syncthreads();
    const int64_t id = (int64_t)((uint32_t)s_tok % (uint64_t)vocab);
    float* xr = x + (int64_t)b * ldx;
    if (fmt == BH_F32) {
        const float* F = (const float*)Q;
        for (int i = threadIdx.x; i < hidden; i += blockDim.x) xr[i] = F[((int64_t)(i >> 2) * n_pad + id) * 4 + (i & 3)];
    } else {
        const uint8_t* B8 = (const uint8_t*)Q;
        for (int i = threadIdx.x; i < hidden; i += blockDim.x) {
            const int64_t c = i >> 5;
            const uint8_t byte = B8[(c * n_pad + id) * 16 + ((i & 31) >> 1)];
            const float nib = (i & 1) ? (float)(byte & 0x0F) : (float)((byte >> 4) & 0x0F);
            xr[i] = (nib - 8.0f) * __half2float(S[c * n_pad + id]);
        }
    }
}

// Final first-max argmax over the LM head's per-tile partials (cpu_engine.rs:3024-3031);
// bumps the sequence's penalty count for the chosen id and records it.
__global__ void __launch_bounds__(256) k_sample_final(const float* __restrict__ pv, const int32_t* __restrict__ pi,
                                                      int tiles, const int32_t* slot, uint16_t* pen, int vocab,
                                                      uint32_t* next, uint32_t* ids_cap, int32_t* step_ctr,
                                                      int batch) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int b = blockIdx.x;
    const int step = step_ctr ? step_ctr[0] : 0;
    float v = -INFINITY;
    int idx = 0x7fffffff;
    for (int t = threadIdx.x; t < tiles; t += blockDim.x) {
        const float ov = pv[(int64_t)b * tiles + t];
        const int oi = pi[(int64_t)b * tiles + t];
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi = __shfl_xor(idx, off);
        if (ov > v || (ov == v && oi < idx)) {
            v = ov;
            idx = oi;
        }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) {
        sv[wave] = v;
        si[wave] = idx;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); ++w)
            if (sv[w] > v || (sv[w] == v && si[w] < idx)) {
                v = sv[w];
                idx = si[w];
            }
        if (idx == 0x7fffffff) idx = 0;  // no finite logit: the scan keeps index 0
        next[b] = (uint32_t)idx;
        uint16_t* c = pen + (int64_t)slot[b] * vocab + idx;
        if (*c < 0xFFFF) *c = *c + 1;
        if (ids_cap) ids_cap[(int64_t)step * batch + b] = (uint32_t)idx;
    }
}

__global__ void k_step_counter(int32_t* ctr, int reset) { ctr[0] = reset ? 0 : ctr[0] + 1; }

}  // namespace

hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* out, int rows, int n, hipStream_t st) {
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), 0, st, x, w, eps, out, n);
    return hipGetLastError();
}

hipError_t launch_resid_norm(float* x, const float* part, int splits, int64_t part_ld, const float* bias,
                             const float* w, float eps, float* h, int rows, int n, hipStream_t st) {
    if (n > 16 * 256 || splits > 16) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_resid_norm, dim3(rows), dim3(256), 0, st, x, part, splits, part_ld, bias, w, eps, h, n);
    return hipGetLastError();
}

hipError_t launch_rope(float* v, const int32_t* pos, const float2* tab, int rows, int n_heads, int hd, hipStream_t st) {
    hipLaunchKernelGGL(k_rope, dim3(rows), dim3(256), 0, st, v, pos, tab, n_heads, hd);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t st) {
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)std::max<int64_t>(blocks, 1)), dim3(256), 0, st, g, u, out, n);
    return hipGetLastError();
}

hipError_t launch_dequant(const DevWeight& w, float* out, hipStream_t st) {
    const int64_t total = w.n * w.chunks;
    hipLaunchKernelGGL(k_dequant, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, w.fmt, (const uint4*)w.q,
                       w.s, w.n, w.k, w.n_pad, w.chunks, out);
    return hipGetLastError();
}

hipError_t launch_embed(const DevWeight& t, int32_t* tok, int32_t* pos, const int32_t* slot, int32_t* seq_len,
                        const uint32_t* next, int prologue, float* x, int64_t ldx, int batch, hipStream_t st) {
    hipLaunchKernelGGL(k_embed, dim3(batch), dim3(256), 0, st, t.fmt, (const uint4*)t.q, (const __half*)t.s, t.n,
                       t.n_pad, (int)t.k, tok, pos, slot, seq_len, next, prologue, x, ldx);
    return hipGetLastError();
}

hipError_t launch_sample_final(const float* part_val, const int32_t* part_idx, int tiles, int batch,
                               const int32_t* slot, uint16_t* pen, int vocab, uint32_t* next, uint32_t* ids_cap,
                               const int32_t* step_ctr, hipStream_t st) {
    hipLaunchKernelGGL(k_sample_final, dim3(batch), dim3(256), 0, st, part_val, part_idx, tiles, slot, pen, vocab, next,
                       ids_cap, (int32_t*)step_ctr, batch);
    return hipGetLastError();
}

hipError_t launch_step_counter(int32_t* ctr, int reset, hipStream_t st) {
    hipLaunchKernelGGL(k_step_counter, dim3(1), dim3(1), 0, st, ctr, reset);
    return hipGetLastError();
}

}  // namespace bh
