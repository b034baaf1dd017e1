// k_attn_o.hip — batch-1 decode attention with the output projection and the residual add in
// one kernel.
//
// Reference semantics: flash_attention_single_into (src/inference/cpu_engine.rs:1450-1509) for
// every query head, then matvec_mul_into (cpu_engine.rs:1307-1444) of the O projection and the
// residual add (cpu_engine.rs:2937-2939) with the next RMSNorm's inputs: the same arithmetic as
// k_attn_mf (k_attn.hip) followed by k_gemv's EPI_RESNORM pass (k_gemv.hip).
//
// Design: at batch 1 a short context's attention is a few microseconds of dependent latency on
// one workgroup per KV head, and the O projection is a second dependent launch that starts by
// reading the attention output back. Here each workgroup owns one 64-row tile of the
// projection and computes the attention of every head itself (the K/V rows of a short context
// are tens of KiB, read from HBM by the first tile of an XCD and from its L2 by the others):
// waves 0 .. n_kv * nwh - 1 run the MFMA attention wave of k_attn.h (nwh waves per KV head,
// the G query heads of the KV head as MFMA columns), their (m, l, o) are merged in LDS into the
// attention output, and every wave then multiplies its share of the projection's K with
// activations broadcast from LDS. The projection's weights are requested at kernel start, so
// their latency hides under the attention. Partial sums are combined in wave order and the
// residual epilogue of k_epilogue.h finishes the tile. Deterministic: no atomics.
//
// Where waves are left over from the attention (PRE), those waves alone take the projection:
// they request and decode their weights to exact fp16 (q - 8) while the attention runs, and
// after the merge spend one mixed-precision FMA per weight instead of the decode's 2.6 VALU
// operations. fma(x, q - 8, p) scaled by s is fma(x, 16 (q - 8), p) scaled by s / 16 bit for bit
// (power-of-two scaling commutes with rounding), so both variants evaluate every chunk exactly
// as k_gemv does (the split of K over waves, and with it the order of the final sum, differs).
//
// Used when the projection needs no K split over workgroups (fewer than 64 chunks of K), for
// Q4_G32 weights, an fp16 cache and contexts of at most 256 KiB of K and V.
#include "bh_internal.h"

#include <hip/hip_fp16.h>

#include "k_attn.h"
#include "k_epilogue.h"
#include "k_stream.h"

namespace bh {
namespace {

constexpr int AO_WAVES = 8;                  // waves per workgroup (256 VGPRs each)
constexpr int64_t AO_KV_BYTES = 256 * 1024;  // K + V bytes of the context, per workgroup

// The slot of dec8's output (k_mfma.h) that holds element e of a dword's 8 nibbles.
__host__ __device__ constexpr int kslot(int e) { return e < 4 ? 2 * (e ^ 1) : 2 * ((e - 4) ^ 1) + 1; }
constexpr bool kslot_inverts_kperm() {
    for (int e = 0; e < 8; ++e)
        if (kperm(kslot(e)) != e) return false;
    return true;
}
static_assert(kslot_inverts_kperm(), "kslot must invert kperm");

// The 32 activations of one chunk from LDS (128-byte aligned) as 16-byte reads.
__device__ __forceinline__ void load_chunk_x(const float* x, float (&xb)[32]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float4 t = ((const float4*)x)[i];
        xb[4 * i] = t.x;
        xb[4 * i + 1] = t.y;
        xb[4 * i + 2] = t.z;
        xb[4 * i + 3] = t.w;
    }
}

// One workgroup of AO_WAVES waves per 64-row tile of the projection. U: chunks per projection
// wave. PRE: the waves past the attention waves take the projection, with pre-decoded weights.
template <int HD, int G, int U, bool PRE>
__global__ void __launch_bounds__(64 * AO_WAVES) k_attn_o(const AttnArgs at, const GemvArgs a, const int nwh) {
    using AW = AttnWave<HD, 1, false>;
    constexpr int KC = HD / 32;  // 32-wide head-dim chunks of the score product
    constexpr int DB = HD / 16;  // 16-wide head-dim blocks of the value product
    constexpr int HP = HD / 2;   // float2 pairs per head
    constexpr int E = Fmt<BH_Q4_G32>::E;
    constexpr int NW = AO_WAVES;
    extern __shared__ float smem[];
    const int na = at.nkv * nwh;          // attention waves
    float* xs = smem;                     // [nq * HD] attention output
    float* comb = xs + at.nq * HD;        // [NW][64] partial sums
    float* w_m = comb + NW * 64;          // [na][16] per-wave running maxima
    float* w_l = w_m + na * 16;           // [na][16] per-wave sums
    float* w_o = w_l + na * 16;           // [na][G][HD] per-wave unnormalised outputs

    const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int tile = blockIdx.x;
    const int64_t n = (int64_t)tile * 64 + lane;
    const int64_t nl = n < a.n_pad ? n : (int64_t)a.n_pad - 1;
    // projection waves: every wave, or (PRE) waves na .. NW - 1
    const int pw = PRE ? wave - na : wave;
    const int npw = PRE ? NW - na : NW;
    const int per = (a.C + npw - 1) / npw;
    const int c0 = pw * per, c1 = min(a.C, c0 + per);

    // the wave's projection weights and scales, one stage of U chunks (clamped, unconditional)
    const __amdgpu_buffer_rsrc_t rW =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.W, (short)0, a.C * a.n_pad * 16, 0x00020000);
    const __amdgpu_buffer_rsrc_t rS =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.S, (short)0, a.C * a.n_pad * 2, 0x00020000);
    uint4 wq[U];
    uint32_t ws[U];
    auto fetch_w = [&] {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int cc = max(min(c0 + u, c1 - 1), 0);
            wq[u] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rW, (int)nl * 16, cc * a.n_pad * 16, 0));
            ws[u] = __builtin_amdgcn_raw_buffer_load_b16(rS, (int)sc_pos(nl) * 2, cc * a.n_pad * 2, 0);
        }
    };
    EpiPre<EPI_RESNORM> pre;

    if (wave < na) {
        // q first (it is waited on first), then the wave's first K/V tile, then the weights
        const int hk = wave / nwh;
        float qv[KC][8];
        const float qscale = 1.4426950408889634f / sqrtf((float)HD);
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) {
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
            if (lr < G) {
                const float4* qp = (const float4*)(at.q + (int64_t)(hk * G + lr) * HD + kc * 32 + 8 * lg);
                x0 = qp[0];
                x1 = qp[1];
            }
            qv[kc][0] = x0.x * qscale; qv[kc][1] = x0.y * qscale; qv[kc][2] = x0.z * qscale; qv[kc][3] = x0.w * qscale;
            qv[kc][4] = x1.x * qscale; qv[kc][5] = x1.y * qscale; qv[kc][6] = x1.z * qscale; qv[kc][7] = x1.w * qscale;
        }
        const int64_t off = at.off_val[0];
        const int64_t head = (int64_t)hk * at.kv.kv_rows * HD;
        AW aw{(const __half*)at.kv.k + head, (const __half*)at.kv.v + head, off,
              (off & 63) == 0 && (at.kv.kv_rows & 7) == 0, ((off | at.kv.kv_rows) & 7) == 0, 0, 0, 0, 0};
        aw.wv = wave - hk * nwh;
        aw.nw = nwh;
        const int tfirst = aw.wv * AW::TR;
        const bool spec = aw.tiled && tfirst + AW::TR <= at.cap_rows;
        if (spec) aw.load_full(aw.A, tfirst);
        if constexpr (!PRE) fetch_w();
        pre.load(a, (int64_t)tile * 64, 64);
        int len = at.pos[0] + 1;
        if (at.kv.max_context > 0) len = min(len, at.kv.max_context);
        const int r1 = min(len, at.split_rows);
        aw.r1 = aw.lim = aw.lim_all = r1;
        if (!spec) aw.start();  // (a partial first tile's V rows past r1 are zeroed by compute())
        half8 qh[KC], ql[KC];
#pragma unroll
        for (int kc = 0; kc < KC; ++kc) split_hl(qv[kc], qh[kc], ql[kc]);
        float m = -INFINITY, l = 0.f;
        f32x4 o[DB];
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] = f32x4{0.f, 0.f, 0.f, 0.f};
        // the wave's tiles in AttnWave::run's order, one tile buffer (the second one of run's
        // pipeline would not fit beside the projection weights; a short context gives each wave
        // one or two tiles)
        for (int t = tfirst; t < r1; t += nwh * AW::TR) {
            if (t != tfirst) aw.load_tile(aw.A, t);
            aw.compute(aw.A, t, qh, ql, m, l, o);
        }
        l += __shfl_xor(l, 16);
        l += __shfl_xor(l, 32);
        if (lg == 0) {
            w_m[wave * 16 + lr] = m;
            w_l[wave * 16 + lr] = l;
        }
        // O^T D layout: lane holds head lr, head-dim db*16 + 4lg + v
        if (lr < G) {
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int v = 0; v < 4; ++v) w_o[(wave * G + lr) * HD + db * 16 + 4 * lg + v] = o[db][v];
        }
    } else {
        fetch_w();
        pre.load(a, (int64_t)tile * 64, 64);
    }
    // PRE: the projection waves' weights as exact fp16 q - 8 (dec8 slot order), decoded while
    // the attention waves run
    half8 wd[PRE ? U : 1][4];
    if constexpr (PRE) {
        if (pw >= 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                wd[u][0] = dec8(wq[u].x);
                wd[u][1] = dec8(wq[u].y);
                wd[u][2] = dec8(wq[u].z);
                wd[u][3] = dec8(wq[u].w);
            }
        }
    }
    __syncthreads();

    // merge the waves of each KV head (log-sum-exp weights, in wave order) into the output
    for (int i = threadIdx.x; i < at.nq * HP; i += blockDim.x) {
        const int hq = i / HP, d = 2 * (i % HP);
        const int g = hq % G, w0 = (hq / G) * nwh;
        float M = -INFINITY;
        for (int w = 0; w < nwh; ++w) M = fmaxf(M, w_m[(w0 + w) * 16 + g]);
        float L = 0.f, O0 = 0.f, O1 = 0.f;
        for (int w = 0; w < nwh; ++w) {
            const float mw = w_m[(w0 + w) * 16 + g];
            const float f = mw == -INFINITY ? 0.f : exp2f(mw - M);
            L += w_l[(w0 + w) * 16 + g] * f;
            O0 += w_o[((w0 + w) * G + g) * HD + d] * f;
            O1 += w_o[((w0 + w) * G + g) * HD + d + 1] * f;
        }
        const float r = L > 0.f ? 1.0f / L : 0.f;
        xs[hq * HD + d] = O0 * r;
        xs[hq * HD + d + 1] = O1 * r;
    }
    __syncthreads();

    // the projection over the wave's chunks, activations broadcast from LDS (the arithmetic and
    // order of k_stream.h's chunk loop)
    float acc = 0.f;
    if constexpr (PRE) {
        if (pw >= 0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (c0 + u < c1) {
                    float xb[E];
                    load_chunk_x(xs + (c0 + u) * E, xb);
                    float p = 0.f;
#pragma unroll
                    for (int e = 0; e < E; ++e) p = fmaf(xb[e], (float)wd[u][e / 8][kslot(e % 8)], p);
                    acc = fmaf(p, __half2float(__ushort_as_half((uint16_t)ws[u])), acc);
                }
            }
        }
    }
#pragma unroll
    for (int u = 0; u < (PRE ? 0 : U); ++u) {
        if (c0 + u < c1) {
            float v[E];
            decode<BH_Q4_G32>(wq[u], v);
            float xb[E];
            load_chunk_x(xs + (c0 + u) * E, xb);
            float p = 0.f;
#pragma unroll
            for (int e = 0; e < E; ++e) p = fmaf(xb[e], v[e], p);
            acc = fmaf(p, __half2float(__ushort_as_half((uint16_t)ws[u])) * 0.0625f, acc);
        }
    }
    comb[wave * 64 + lane] = acc;
    __syncthreads();
    // wave 0 (lane r finishes row tile * 64 + r, whose epilogue operands it loaded): the partial
    // sums in wave order, then the residual epilogue in registers
    if (wave == 0) {
        float sum = comb[lane];
        for (int w = 1; w < NW; ++w) sum += comb[w * 64 + lane];
        resnorm_wave<BH_Q4_G32>(a, sum, (int64_t)tile * 64, pre);
    }
}

struct AoPlan {
    int nwh = 0, u = 0;
    bool pre = false;
    size_t shm = 0;
};

bool ao_plan(int fmt, const AttnArgs& at, const GemvArgs& o, AoPlan* p) {
    if (fmt != BH_Q4_G32 || at.batch != 1 || o.batch != 1 || !at.kv.kv_f16 || !at.static_off || at.splits != 1 ||
        at.prefill || at.seq_len || !at.pos)
        return false;
    if (!attn_supported(at.nq, at.nkv, at.hd)) return false;
    const int G = at.nq / at.nkv;
    if (o.C >= 64 || (int64_t)o.C * Fmt<BH_Q4_G32>::E != (int64_t)at.nq * at.hd || o.ssq_in) return false;
    if (!o.xw_out || !o.wnext || !o.ssq_out || o.ssq_tiles != o.n_pad / 64) return false;
    const int64_t rows = at.kv.max_context > 0 ? std::min(at.split_rows, at.kv.max_context) : at.split_rows;
    if (rows * at.nkv * at.hd * 4 > AO_KV_BYTES) return false;  // fp16 K and V
    if (at.nkv > AO_WAVES) return false;
    // waves per KV head: one tile of the context bound each, as far as the workgroup holds
    // them (every wave's first tile is requested before the length is known, so a wave per tile
    // past the bound would only load rows that are never used: 128 rows at head_dim 64 run 8.0
    // instead of 8.8 us with 2 waves instead of 4)
    const int tr = 32 * KvTile<64>::NJ * 64 / at.hd;  // rows per tile
    p->nwh = std::max(1, std::min((int)((rows + tr - 1) / tr), AO_WAVES / at.nkv));
    const int na = at.nkv * p->nwh;
    // the waves left over from the attention take the projection when they hold at most 8 chunks
    // each as fp16
    p->pre = na < AO_WAVES && (o.C + AO_WAVES - na - 1) / (AO_WAVES - na) <= 8;
    const int per = p->pre ? (o.C + AO_WAVES - na - 1) / (AO_WAVES - na) : (o.C + AO_WAVES - 1) / AO_WAVES;
    p->u = per <= 4 ? 4 : 8;
    p->shm = ((size_t)at.nq * at.hd + AO_WAVES * 64 + (size_t)na * 32 + (size_t)na * G * at.hd) * sizeof(float);
    return p->shm <= 64 * 1024;
}

template <int HD, int G>
hipError_t launch_hg(const AttnArgs& at, const GemvArgs& o, const AoPlan& p, hipStream_t st) {
    const dim3 grid((o.n_pad + 63) / 64), block(64 * AO_WAVES);
    if (p.pre) {
        if (p.u == 4) launch_kernel((k_attn_o<HD, G, 4, true>), grid, block, p.shm, st, at, o, p.nwh);
        else launch_kernel((k_attn_o<HD, G, 8, true>), grid, block, p.shm, st, at, o, p.nwh);
    } else {
        if (p.u == 4) launch_kernel((k_attn_o<HD, G, 4, false>), grid, block, p.shm, st, at, o, p.nwh);
        else launch_kernel((k_attn_o<HD, G, 8, false>), grid, block, p.shm, st, at, o, p.nwh);
    }
    return hipGetLastError();
}

template <int HD>
hipError_t launch_h(const AttnArgs& at, const GemvArgs& o, const AoPlan& p, hipStream_t st) {
    switch (at.nq / at.nkv) {
        case 1: return launch_hg<HD, 1>(at, o, p, st);
        case 2: return launch_hg<HD, 2>(at, o, p, st);
        case 4: return launch_hg<HD, 4>(at, o, p, st);
        case 7: return launch_hg<HD, 7>(at, o, p, st);
        case 8: return launch_hg<HD, 8>(at, o, p, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool attn_o_fusable(int fmt, const AttnArgs& at, const GemvArgs& o) {
    AoPlan p;
    return ao_plan(fmt, at, o, &p);
}

hipError_t launch_attn_o(int fmt, const AttnArgs& at, const GemvArgs& o, hipStream_t st) {
    AoPlan p;
    if (!ao_plan(fmt, at, o, &p)) return hipErrorInvalidValue;
    return at.hd == 64 ? launch_h<64>(at, o, p, st) : launch_h<128>(at, o, p, st);
}

}  // namespace bh
