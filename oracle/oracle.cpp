// oracle.cpp — CPU restatement of the reference's quantized decode path.
//
// TEST INFRASTRUCTURE ONLY. The HIP backend in bramha_amd/ is compared against this
// library; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
// load it. Nothing in the product links or calls it.
//
// The reference (akshaybhlrp/bramha) is Rust and cannot be built in this image,
// so every function below restates one reference function, following its
// arithmetic order exactly: strict IEEE f32, no FMA contraction (build with
// -ffp-contract=off; rustc never fuses a*b+c), glibc expf/sinf/cosf/powf (what
// Rust's f32::exp/sin/cos/powf lower to on Linux), round-half-away-from-zero
// (Rust f32::round == C roundf). Each function cites the reference file:line.
//
// The block-32 / fp16-scale 4-bit format (Q4_G32) does not exist in the
// reference; it is the weight format of the 4-bit throughput workload. Its
// quantizer applies the reference's per-row rule (scale = maxabs/7, clamp to
// +-7, +8 offset, high nibble = even element) per group of 32 with the scale
// rounded to fp16 first, and its GEMV is the reference's Float GEMV over the
// dequantized weights — the equivalence the reference's own
// test_quantization_correctness asserts (cpu_engine.rs:3543-3560).
#include <cmath>
#include <cstdint>
#include <cstring>
#include <cstdio>
#include <vector>
#include <algorithm>
#include <omp.h>

namespace {

enum Fmt : int32_t { F32 = 0, Q8_ROW = 1, Q4_ROW = 2, Q4_G32 = 3 };

// ---------------------------------------------------------------------------
// fp16 <-> f32 (IEEE binary16, round-to-nearest-even). Own implementation.
// ---------------------------------------------------------------------------
inline float half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {  // subnormal: value = man * 2^-24
            float v = (float)man * 5.9604644775390625e-08f;
            uint32_t vb;
            std::memcpy(&vb, &v, 4);
            bits = sign | vb;
        }
    } else if (exp == 31) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 112u) << 23) | (man << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

inline uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {  // inf / nan
        return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);  // rounds to >= 65520 -> inf
    if (ax < 0x38800000u) {  // below 2^-14: subnormal half (or zero)
        // value / 2^-24, rounded to nearest even, as an integer mantissa
        float a;
        std::memcpy(&a, &ax, 4);
        float m = a * 16777216.0f;  // exact scaling by 2^24
        float r = std::nearbyint(m);  // default rounding mode: nearest-even
        return (uint16_t)(sign | (uint16_t)r);
    }
    uint32_t e = (ax >> 23) - 112u;  // rebias 127 -> 15
    uint32_t man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;  // carries into exponent correctly
    return (uint16_t)(sign | h);
}

// Rust `(v).round().clamp(lo, hi) as iN` with NaN -> 0 (saturating cast).
inline float round_clamp(float v, float lo, float hi) {
    float r = std::roundf(v);
    if (std::isnan(r)) return NAN;
    return std::min(std::max(r, lo), hi);
}

// LUT_Q1 / LUT_Q2: cpu_engine.rs:108-126.
struct Luts {
    float q1[256], q2[256];
    Luts() {
        for (int i = 0; i < 256; ++i) {
            q1[i] = (float)((i >> 4) & 0x0F) - 8.0f;
            q2[i] = (float)(i & 0x0F) - 8.0f;
        }
    }
};
const Luts LUT;

// A weight tensor as the reference's WeightTensor (cpu_engine.rs:87-106).
struct WView {
    int32_t fmt;
    const float* f;     // F32
    const int8_t* q8;   // Q8_ROW
    const uint8_t* q4;  // Q4_ROW
    const float* s;     // per-row scales
};

// matvec_mul_into: cpu_engine.rs:1307-1412 (the decode GEMV, 4 partial sums).
// Each output row is computed by one thread, so the result is independent of
// the thread count; rows are split like rayon's with_min_len(256).
void matvec_mul_into(const float* h, int64_t in_f, const WView& w, float* out, int64_t out_f) {
    if (w.fmt == F32 || w.fmt == Q8_ROW) {
        const int64_t chunks = in_f / 4, rem = in_f % 4;
#pragma omp parallel for schedule(static) if (out_f > 256)
        for (int64_t j = 0; j < out_f; ++j) {
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
            if (w.fmt == F32) {
                const float* ws = w.f + j * in_f;
                for (int64_t i = 0; i < chunks; ++i) {
                    const int64_t b = i * 4;
                    s0 += h[b] * ws[b];
                    s1 += h[b + 1] * ws[b + 1];
                    s2 += h[b + 2] * ws[b + 2];
                    s3 += h[b + 3] * ws[b + 3];
                }
                for (int64_t i = chunks * 4; i < chunks * 4 + rem; ++i) s0 += h[i] * ws[i];
                out[j] = s0 + s1 + s2 + s3;
            } else {
                const int8_t* ws = w.q8 + j * in_f;
                for (int64_t i = 0; i < chunks; ++i) {
                    const int64_t b = i * 4;
                    s0 += h[b] * (float)ws[b];
                    s1 += h[b + 1] * (float)ws[b + 1];
                    s2 += h[b + 2] * (float)ws[b + 2];
                    s3 += h[b + 3] * (float)ws[b + 3];
                }
                for (int64_t i = chunks * 4; i < chunks * 4 + rem; ++i) s0 += h[i] * (float)ws[i];
                out[j] = (s0 + s1 + s2 + s3) * w.s[j];
            }
        }
        return;
    }
    // Q4_ROW: cpu_engine.rs:1363-1412
    const int64_t half_in = in_f / 2;
    const int64_t chunks = half_in / 8;
#pragma omp parallel for schedule(static) if (out_f > 256)
    for (int64_t j = 0; j < out_f; ++j) {
        const uint8_t* rb = w.q4 + j * half_in;
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
        for (int64_t c = 0; c < chunks; ++c) {
            const uint8_t* b = rb + c * 8;
            const float* hh = h + c * 16;
            s0 += hh[0] * LUT.q1[b[0]] + hh[1] * LUT.q2[b[0]];
            s1 += hh[2] * LUT.q1[b[1]] + hh[3] * LUT.q2[b[1]];
            s2 += hh[4] * LUT.q1[b[2]] + hh[5] * LUT.q2[b[2]];
            s3 += hh[6] * LUT.q1[b[3]] + hh[7] * LUT.q2[b[3]];
            s0 += hh[8] * LUT.q1[b[4]] + hh[9] * LUT.q2[b[4]];
            s1 += hh[10] * LUT.q1[b[5]] + hh[11] * LUT.q2[b[5]];
            s2 += hh[12] * LUT.q1[b[6]] + hh[13] * LUT.q2[b[6]];
            s3 += hh[14] * LUT.q1[b[7]] + hh[15] * LUT.q2[b[7]];
        }
        float sum = s0 + s1 + s2 + s3;
        for (int64_t i = chunks * 8; i < half_in; ++i) {
            const uint8_t byte = rb[i];
            sum += h[i * 2] * LUT.q1[byte] + h[i * 2 + 1] * LUT.q2[byte];
        }
        out[j] = sum * w.s[j];
    }
}

// One row of matvec_mul's single running sum: cpu_engine.rs:456-495.
inline float matvec_row_single(const float* h, int64_t in_f, const WView& w, int64_t j) {
    float sum = 0.f;
    if (w.fmt == F32) {
        const float* ws = w.f + j * in_f;
        for (int64_t i = 0; i < in_f; ++i) sum += h[i] * ws[i];
        return sum;
    }
    if (w.fmt == Q8_ROW) {
        const int8_t* ws = w.q8 + j * in_f;
        for (int64_t i = 0; i < in_f; ++i) sum += h[i] * (float)ws[i];
        return sum * w.s[j];
    }
    const uint8_t* rb = w.q4 + j * (in_f / 2);
    for (int64_t i = 0; i < in_f / 2; ++i) {
        const uint8_t byte = rb[i];
        const float q1 = (float)((byte >> 4) & 0x0F) - 8.0f;
        const float q2 = (float)(byte & 0x0F) - 8.0f;
        sum += h[i * 2] * q1 + h[i * 2 + 1] * q2;
    }
    return sum * w.s[j];
}

// matvec_mul (single running sum): cpu_engine.rs:355-562 (GPU branch dead: :380).
void matvec_mul(const float* h, int64_t in_f, const WView& w, float* out, int64_t out_f) {
#pragma omp parallel for schedule(static) if (out_f >= 128)
    for (int64_t j = 0; j < out_f; ++j) out[j] = matvec_row_single(h, in_f, w, j);
}

// gemm_cpu: cpu_engine.rs:565-708, the path taken whenever is_cpu (always, :573).
// F32/I8 single sum, U4 the 4-partial-sum order of a5. The reference runs it on one thread;
// this scalar form keeps its loop order, gemm_cpu below computes the same chains in parallel.
void gemm_cpu_scalar(const float* hb, const WView& w, int64_t bs, int64_t in_f, int64_t out_f, float* out) {
    for (int64_t j = 0; j < out_f; ++j) {
        for (int64_t b = 0; b < bs; ++b) {
            const float* hr = hb + b * in_f;
            if (w.fmt == Q4_ROW) {
                const int64_t half_in = in_f / 2, chunks = half_in / 8;
                const uint8_t* rb = w.q4 + j * half_in;
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
                for (int64_t c = 0; c < chunks; ++c) {
                    const uint8_t* bb = rb + c * 8;
                    const float* hh = hr + c * 16;
                    s0 += hh[0] * LUT.q1[bb[0]] + hh[1] * LUT.q2[bb[0]];
                    s1 += hh[2] * LUT.q1[bb[1]] + hh[3] * LUT.q2[bb[1]];
                    s2 += hh[4] * LUT.q1[bb[2]] + hh[5] * LUT.q2[bb[2]];
                    s3 += hh[6] * LUT.q1[bb[3]] + hh[7] * LUT.q2[bb[3]];
                    s0 += hh[8] * LUT.q1[bb[4]] + hh[9] * LUT.q2[bb[4]];
                    s1 += hh[10] * LUT.q1[bb[5]] + hh[11] * LUT.q2[bb[5]];
                    s2 += hh[12] * LUT.q1[bb[6]] + hh[13] * LUT.q2[bb[6]];
                    s3 += hh[14] * LUT.q1[bb[7]] + hh[15] * LUT.q2[bb[7]];
                }
                float sum = s0 + s1 + s2 + s3;
                for (int64_t i = chunks * 8; i < half_in; ++i) {
                    const uint8_t byte = rb[i];
                    sum += hr[i * 2] * LUT.q1[byte] + hr[i * 2 + 1] * LUT.q2[byte];
                }
                out[b * out_f + j] = sum * w.s[j];
            } else {
                out[b * out_f + j] = matvec_row_single(hr, in_f, w, j);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Token-blocked forms for passes over many tokens (prefill). Every (token, row) output is
// ONE sequential chain in exactly the order of the single-token function named beside it:
// the tokens of a block only occupy separate SIMD lanes and the rows are spread over
// threads, so no chain is split or reassociated and the results are bit-identical to the
// scalar loops for any thread count. orc_set_fast(0) selects the scalar forms, against
// which the tests pin these.
// ---------------------------------------------------------------------------
int g_fast = 1;
constexpr int TB = 16;  // tokens per block

// hT[i][t] = hb[b0 + t][i] for t < nb; zero in the padding lanes.
void transpose_tokens(const float* hb, int64_t in_f, int64_t b0, int64_t nb, float* hT) {
    for (int64_t i = 0; i < in_f; ++i)
        for (int t = 0; t < TB; ++t) hT[i * TB + t] = t < nb ? hb[(b0 + t) * in_f + i] : 0.f;
}

// 8 float lanes (one AVX register). With -ffp-contract=off a * b + c stays a multiply and an add.
typedef float v8 __attribute__((vector_size(32)));
inline v8 ld8(const float* p) {
    v8 r;
    std::memcpy(&r, p, sizeof r);
    return r;
}
inline void st8(float* p, v8 v) { std::memcpy(p, &v, sizeof v); }
inline v8 bc8(float x) { return v8{x, x, x, x, x, x, x, x}; }

// One row of matvec_mul's single running sum (matvec_row_single) for a block of tokens.
inline void block_row_single(const float* hT, int64_t in_f, const WView& w, int64_t j, float* res) {
    v8 a0 = bc8(0.f), a1 = bc8(0.f);
    if (w.fmt == F32 || w.fmt == Q8_ROW) {
        const float* wf = w.f + j * in_f;
        const int8_t* w8 = w.q8 + j * in_f;
        const bool f32 = w.fmt == F32;
        for (int64_t i = 0; i < in_f; ++i) {
            const v8 wi = bc8(f32 ? wf[i] : (float)w8[i]);
            a0 += ld8(hT + i * TB) * wi;
            a1 += ld8(hT + i * TB + 8) * wi;
        }
        if (!f32) {
            a0 *= bc8(w.s[j]);
            a1 *= bc8(w.s[j]);
        }
    } else {
        const uint8_t* rb = w.q4 + j * (in_f / 2);
        for (int64_t i = 0; i < in_f / 2; ++i) {
            const v8 q1 = bc8(LUT.q1[rb[i]]), q2 = bc8(LUT.q2[rb[i]]);
            const float* h0 = hT + (2 * i) * TB;
            a0 += ld8(h0) * q1 + ld8(h0 + TB) * q2;
            a1 += ld8(h0 + 8) * q1 + ld8(h0 + TB + 8) * q2;
        }
        a0 *= bc8(w.s[j]);
        a1 *= bc8(w.s[j]);
    }
    st8(res, a0);
    st8(res + 8, a1);
}

// The U4 order of a5 (four partial sums over the bytes of each 8-byte chunk, then the tail
// bytes, then the row scale) for a block of tokens: gemm_cpu's and matvec_mul_into's Q4_ROW rows.
inline void block_row_q4x4(const float* hT, int64_t in_f, const WView& w, int64_t j, float* res) {
    const int64_t half_in = in_f / 2, chunks = half_in / 8;
    const uint8_t* rb = w.q4 + j * half_in;
    v8 s[4][2];
    for (auto& x : s) x[0] = x[1] = bc8(0.f);
    for (int64_t c = 0; c < chunks; ++c) {
        for (int e = 0; e < 8; ++e) {
            const uint8_t b = rb[c * 8 + e];
            const v8 q1 = bc8(LUT.q1[b]), q2 = bc8(LUT.q2[b]);
            const float* h0 = hT + (c * 16 + 2 * e) * TB;
            s[e & 3][0] += ld8(h0) * q1 + ld8(h0 + TB) * q2;
            s[e & 3][1] += ld8(h0 + 8) * q1 + ld8(h0 + TB + 8) * q2;
        }
    }
    v8 sum0 = s[0][0] + s[1][0] + s[2][0] + s[3][0], sum1 = s[0][1] + s[1][1] + s[2][1] + s[3][1];
    for (int64_t i = chunks * 8; i < half_in; ++i) {
        const v8 q1 = bc8(LUT.q1[rb[i]]), q2 = bc8(LUT.q2[rb[i]]);
        const float* h0 = hT + (2 * i) * TB;
        sum0 += ld8(h0) * q1 + ld8(h0 + TB) * q2;
        sum1 += ld8(h0 + 8) * q1 + ld8(h0 + TB + 8) * q2;
    }
    st8(res, sum0 * bc8(w.s[j]));
    st8(res + 8, sum1 * bc8(w.s[j]));
}

// One row of matvec_mul_into (cpu_engine.rs:1311-1412) for a block of tokens: F32/I8 four
// partial sums over stride-4 elements with the tail in s0, then (s0 + s1 + s2 + s3) (x scale).
inline void block_row_into(const float* hT, int64_t in_f, const WView& w, int64_t j, float* res) {
    if (w.fmt == Q4_ROW) {
        block_row_q4x4(hT, in_f, w, j, res);
        return;
    }
    const int64_t chunks = in_f / 4, rem = in_f % 4;
    const float* wf = w.f + j * in_f;
    const int8_t* w8 = w.q8 + j * in_f;
    const bool f32 = w.fmt == F32;
    v8 s[4][2];
    for (auto& x : s) x[0] = x[1] = bc8(0.f);
    for (int64_t c = 0; c < chunks; ++c) {
        const int64_t b = c * 4;
        for (int e = 0; e < 4; ++e) {
            const v8 wi = bc8(f32 ? wf[b + e] : (float)w8[b + e]);
            const float* h = hT + (b + e) * TB;
            s[e][0] += ld8(h) * wi;
            s[e][1] += ld8(h + 8) * wi;
        }
    }
    for (int64_t i = chunks * 4; i < chunks * 4 + rem; ++i) {
        const v8 wi = bc8(f32 ? wf[i] : (float)w8[i]);
        s[0][0] += ld8(hT + i * TB) * wi;
        s[0][1] += ld8(hT + i * TB + 8) * wi;
    }
    v8 r0 = s[0][0] + s[1][0] + s[2][0] + s[3][0], r1 = s[0][1] + s[1][1] + s[2][1] + s[3][1];
    if (!f32) {
        r0 *= bc8(w.s[j]);
        r1 *= bc8(w.s[j]);
    }
    st8(res, r0);
    st8(res + 8, r1);
}

// out[b][j] = row(j) of token b for b < bs, j < out_f: tokens transposed into blocks of TB,
// rows spread over the threads.
template <class Row>
void rows_over_token_blocks(const float* hb, int64_t bs, int64_t in_f, int64_t out_f, float* out, Row row) {
    const int64_t nblk = (bs + TB - 1) / TB;
    std::vector<float> hT((size_t)(nblk * in_f * TB));
#pragma omp parallel for schedule(static)
    for (int64_t blk = 0; blk < nblk; ++blk)
        transpose_tokens(hb, in_f, blk * TB, std::min<int64_t>(TB, bs - blk * TB), &hT[blk * in_f * TB]);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < out_f; ++j) {
        for (int64_t blk = 0; blk < nblk; ++blk) {
            float res[TB];
            row(&hT[blk * in_f * TB], j, res);
            const int64_t nb = std::min<int64_t>(TB, bs - blk * TB);
            for (int64_t t = 0; t < nb; ++t) out[(blk * TB + t) * out_f + j] = res[t];
        }
    }
}

void gemm_cpu(const float* hb, const WView& w, int64_t bs, int64_t in_f, int64_t out_f, float* out) {
    if (!g_fast) {
        gemm_cpu_scalar(hb, w, bs, in_f, out_f, out);
        return;
    }
    if (w.fmt == Q4_ROW)
        rows_over_token_blocks(hb, bs, in_f, out_f, out,
                               [&](const float* hT, int64_t j, float* r) { block_row_q4x4(hT, in_f, w, j, r); });
    else
        rows_over_token_blocks(hb, bs, in_f, out_f, out,
                               [&](const float* hT, int64_t j, float* r) { block_row_single(hT, in_f, w, j, r); });
}

// matvec_mul_into of each of bs tokens (the prefill's per-token MLP GEMVs).
void matvec_into_tokens(const float* hb, int64_t bs, int64_t in_f, const WView& w, float* out, int64_t out_f) {
    if (!g_fast) {
        for (int64_t b = 0; b < bs; ++b) matvec_mul_into(hb + b * in_f, in_f, w, out + b * out_f, out_f);
        return;
    }
    rows_over_token_blocks(hb, bs, in_f, out_f, out,
                           [&](const float* hT, int64_t j, float* r) { block_row_into(hT, in_f, w, j, r); });
}

// rms_norm_into / rms_norm_cpu: cpu_engine.rs:1275-1302.
void rms_norm(const float* x, const float* wt, float eps, float* out, int64_t n) {
    float var = 0.f;
    for (int64_t i = 0; i < n; ++i) var += x[i] * x[i];
    var /= (float)n;
    const float scale = 1.0f / std::sqrt(var + eps);
    for (int64_t i = 0; i < n; ++i) out[i] = x[i] * scale * wt[i];
}

// get_rope_thetas: cpu_engine.rs:1515-1530.
void rope_thetas(int64_t hd, float theta, float* out) {
    for (int64_t i = 0; i < hd / 2; ++i)
        out[i] = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
}

// apply_rope_cpu: cpu_engine.rs:1682-1699 (rotate-half).
void apply_rope(float* v, int64_t pos, int64_t nh, int64_t hd, float theta) {
    const int64_t half = hd / 2;
    std::vector<float> th(half);
    rope_thetas(hd, theta, th.data());
    for (int64_t h = 0; h < nh; ++h) {
        float* p = v + h * hd;
        for (int64_t i = 0; i < half; ++i) {
            const float freq = (float)pos * th[i];
            const float c = cosf(freq), s = sinf(freq);
            const float x1 = p[i], x2 = p[i + half];
            p[i] = x1 * c - x2 * s;
            p[i + half] = x2 * c + x1 * s;
        }
    }
}

// Online-softmax attention for one query row over kv_len cached rows.
// div_out = false: decode form, out = o * (1/l)  (flash_attention_single_into, cpu_engine.rs:1450-1509)
// div_out = true:  prefill form, out = o / l     (flash_attention_cpu, cpu_engine.rs:1166-1214)
void attend_row(const float* q, const float* kc, const float* vc, int64_t kv_len, int64_t nq, int64_t nkv,
                int64_t hd, float* out, bool div_out) {
    const float scale = 1.0f / std::sqrt((float)hd);
    const int64_t per = nq / nkv;
    std::vector<float> o(hd);
    for (int64_t head = 0; head < nq; ++head) {
        const int64_t kvh = head / per;
        const float* qh = q + head * hd;
        std::fill(o.begin(), o.end(), 0.f);
        float m = -INFINITY, l = 0.f;
        for (int64_t t = 0; t < kv_len; ++t) {
            const float* kh = kc + (t * nkv + kvh) * hd;
            const float* vh = vc + (t * nkv + kvh) * hd;
            float dot = 0.f;
            for (int64_t d = 0; d < hd; ++d) dot += qh[d] * kh[d];
            const float score = dot * scale;
            if (score > m) {
                const float e = expf(m - score);
                l = l * e + 1.0f;
                for (int64_t d = 0; d < hd; ++d) o[d] = o[d] * e + vh[d];
                m = score;
            } else {
                const float e = expf(score - m);
                l += e;
                for (int64_t d = 0; d < hd; ++d) o[d] += e * vh[d];
            }
        }
        float* oh = out + head * hd;
        if (div_out) {
            for (int64_t d = 0; d < hd; ++d) oh[d] = o[d] / l;
        } else {
            const float inv = 1.0f / l;
            for (int64_t d = 0; d < hd; ++d) oh[d] = o[d] * inv;
        }
    }
}

// attend_row's chains for the query heads [h0, h0 + nh) that share KV head g (nh <= 8,
// hd <= 128): each head keeps its own online softmax over the rows in order; only the q.k
// dot products of 8 consecutive rows are formed side by side (one lane per head, each dot
// summed over d in order), so every output equals attend_row's.
void attend_group(const float* q, int64_t h0, int64_t nh, int64_t g, const float* kc, const float* vc,
                  int64_t kv_len, int64_t nkv, int64_t hd, float* out, bool div_out) {
    const float scale = 1.0f / std::sqrt((float)hd);
    alignas(32) float qT[128 * 8];
    for (int64_t d = 0; d < hd; ++d)
        for (int hh = 0; hh < 8; ++hh) qT[d * 8 + hh] = hh < nh ? q[(h0 + hh) * hd + d] : 0.f;
    std::vector<float> o((size_t)(nh * hd), 0.f);
    float m[8], l[8];
    for (int hh = 0; hh < 8; ++hh) {
        m[hh] = -INFINITY;
        l[hh] = 0.f;
    }
    for (int64_t t0 = 0; t0 < kv_len; t0 += 8) {
        const int64_t nr = std::min<int64_t>(8, kv_len - t0);
        alignas(32) float dots[8][8] = {};
        const float* kr[8];
        for (int r = 0; r < 8; ++r) kr[r] = kc + (std::min<int64_t>(t0 + r, kv_len - 1) * nkv + g) * hd;  // padding rows unused
        for (int64_t d = 0; d < hd; ++d) {
            const float* qd = qT + d * 8;
            for (int r = 0; r < 8; ++r) {
                const float kv = kr[r][d];
                for (int hh = 0; hh < 8; ++hh) dots[r][hh] += qd[hh] * kv;
            }
        }
        for (int64_t r = 0; r < nr; ++r) {
            const float* vh = vc + ((t0 + r) * nkv + g) * hd;
            for (int64_t hh = 0; hh < nh; ++hh) {
                const float score = dots[r][hh] * scale;
                float* oh = &o[hh * hd];
                if (score > m[hh]) {
                    const float e = expf(m[hh] - score);
                    l[hh] = l[hh] * e + 1.0f;
                    for (int64_t d = 0; d < hd; ++d) oh[d] = oh[d] * e + vh[d];
                    m[hh] = score;
                } else {
                    const float e = expf(score - m[hh]);
                    l[hh] += e;
                    for (int64_t d = 0; d < hd; ++d) oh[d] += e * vh[d];
                }
            }
        }
    }
    for (int64_t hh = 0; hh < nh; ++hh) {
        float* dst = out + (h0 + hh) * hd;
        const float* oh = &o[hh * hd];
        if (div_out) {
            for (int64_t d = 0; d < hd; ++d) dst[d] = oh[d] / l[hh];
        } else {
            const float inv = 1.0f / l[hh];
            for (int64_t d = 0; d < hd; ++d) dst[d] = oh[d] * inv;
        }
    }
}

// Decode attention of one query row: attend_row, or its chains one head per task.
void attend_decode(const float* q, const float* kc, const float* vc, int64_t kv_len, int64_t nq, int64_t nkv,
                   int64_t hd, float* out) {
    if (!g_fast || hd > 128) {
        attend_row(q, kc, vc, kv_len, nq, nkv, hd, out, false);
        return;
    }
    const int64_t per = nq / nkv;
#pragma omp parallel for schedule(static)
    for (int64_t h = 0; h < nq; ++h) attend_group(q, h, 1, h / per, kc, vc, kv_len, nkv, hd, out, false);
}

// Prefill attention of bs query rows at positions start_pos + b, each over cache rows
// [0, start_pos + b] (flash_attention_cpu): attend_row per row, or its chains as tasks of one
// row and one KV head's query heads.
void attend_prefill(const float* qb, const float* kc, const float* vc, int64_t bs, int64_t start_pos, int64_t nq,
                    int64_t nkv, int64_t hd, float* out) {
    const int64_t per = nq / nkv;
    if (!g_fast || hd > 128 || per > 8) {
        for (int64_t b = 0; b < bs; ++b)
            attend_row(qb + b * nq * hd, kc, vc, start_pos + b + 1, nq, nkv, hd, out + b * nq * hd, true);
        return;
    }
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t task = 0; task < bs * nkv; ++task) {
        const int64_t b = task / nkv, g = task % nkv;
        attend_group(qb + b * nq * hd, g * per, per, g, kc, vc, start_pos + b + 1, nkv, hd, out + b * nq * hd, true);
    }
}

// SiLU gate: cpu_engine.rs:2023-2026.
inline float silu_mul(float g, float u) { return g * (1.0f / (1.0f + expf(-g))) * u; }

// Dense SwiGLU MLP, run_mlp_into dense branch with is_cpu: cpu_engine.rs:1990-2033.
void mlp(const float* h2, const WView& wg, const WView& wu, const WView& wd, int64_t H, int64_t I, float* gate,
         float* up, float* mm, float* out) {
    matvec_mul_into(h2, H, wg, gate, I);
    matvec_mul_into(h2, H, wu, up, I);
    for (int64_t d = 0; d < I; ++d) {
        const float sg = gate[d] * (1.0f / (1.0f + expf(-gate[d])));
        mm[d] = sg * up[d];
    }
    matvec_mul_into(mm, I, wd, out, H);
}

}  // namespace

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

// ---- quantization: src/models/quantization.rs ----

// quantize_to_int8: quantization.rs:7-38
void orc_quantize_int8(const float* w, int64_t n, int64_t k, int8_t* q, float* s) {
    for (int64_t j = 0; j < n; ++j) {
        const float* row = w + j * k;
        float mx = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            const float a = std::fabs(row[i]);
            if (a > mx) mx = a;
        }
        const float sc = (mx == 0.f) ? 1.0f : mx / 127.0f;
        s[j] = sc;
        for (int64_t i = 0; i < k; ++i) {
            const float r = round_clamp(row[i] / sc, -127.f, 127.f);
            q[j * k + i] = std::isnan(r) ? (int8_t)0 : (int8_t)r;
        }
    }
}

// quantize_to_int4: quantization.rs:41-83 (K even; high nibble = even element)
int orc_quantize_int4(const float* w, int64_t n, int64_t k, uint8_t* q, float* s) {
    if (k % 2 != 0) return -1;  // the reference asserts (:46-49)
    for (int64_t j = 0; j < n; ++j) {
        const float* row = w + j * k;
        float mx = 0.f;
        for (int64_t i = 0; i < k; ++i) {
            const float a = std::fabs(row[i]);
            if (a > mx) mx = a;
        }
        const float sc = (mx == 0.f) ? 1.0f : mx / 7.0f;
        s[j] = sc;
        for (int64_t i = 0; i < k / 2; ++i) {
            const float r1 = round_clamp(row[2 * i] / sc, -7.f, 7.f) + 8.0f;
            const float r2 = round_clamp(row[2 * i + 1] / sc, -7.f, 7.f) + 8.0f;
            const uint8_t q1 = std::isnan(r1) ? 0 : (uint8_t)r1;
            const uint8_t q2 = std::isnan(r2) ? 0 : (uint8_t)r2;
            q[j * (k / 2) + i] = (uint8_t)((q1 << 4) | (q2 & 0x0F));
        }
    }
    return 0;
}

// dequantize_int8: quantization.rs:86-99
void orc_dequantize_int8(const int8_t* q, const float* s, int64_t n, int64_t k, float* w) {
    for (int64_t j = 0; j < n; ++j)
        for (int64_t i = 0; i < k; ++i) w[j * k + i] = (float)q[j * k + i] * s[j];
}

// dequantize_int4: quantization.rs:102-122
void orc_dequantize_int4(const uint8_t* q, const float* s, int64_t n, int64_t k, float* w) {
    for (int64_t j = 0; j < n; ++j)
        for (int64_t i = 0; i < k / 2; ++i) {
            const uint8_t b = q[j * (k / 2) + i];
            w[j * k + 2 * i] = ((float)((b >> 4) & 0x0F) - 8.0f) * s[j];
            w[j * k + 2 * i + 1] = ((float)(b & 0x0F) - 8.0f) * s[j];
        }
}

// Block-32 extension of quantize_to_int4: per group of 32 along K, scale =
// maxabs/7 rounded to fp16 (1.0 for an all-zero group), q = round(x / f32(scale16))
// clamped to +-7, +8, same packing as quantization.rs:74-78. K % 32 == 0.
int orc_quantize_q4g32(const float* w, int64_t n, int64_t k, uint8_t* q, uint16_t* s16) {
    if (k % 32 != 0) return -1;
    const int64_t G = k / 32;
    for (int64_t j = 0; j < n; ++j) {
        for (int64_t g = 0; g < G; ++g) {
            const float* x = w + j * k + g * 32;
            float mx = 0.f;
            for (int i = 0; i < 32; ++i) {
                const float a = std::fabs(x[i]);
                if (a > mx) mx = a;
            }
            uint16_t h = (mx == 0.f) ? (uint16_t)0x3C00u : float_to_half(mx / 7.0f);
            if ((h & 0x7FFFu) == 0) h = 0x0001u;  // underflowed scale: smallest subnormal
            s16[j * G + g] = h;
            const float sc = half_to_float(h);
            for (int i = 0; i < 16; ++i) {
                const float r1 = round_clamp(x[2 * i] / sc, -7.f, 7.f) + 8.0f;
                const float r2 = round_clamp(x[2 * i + 1] / sc, -7.f, 7.f) + 8.0f;
                const uint8_t q1 = std::isnan(r1) ? 0 : (uint8_t)r1;
                const uint8_t q2 = std::isnan(r2) ? 0 : (uint8_t)r2;
                q[j * (k / 2) + g * 16 + i] = (uint8_t)((q1 << 4) | (q2 & 0x0F));
            }
        }
    }
    return 0;
}

// w = (nib - 8) * f32(scale16): exact in f32 (a 4-bit integer times an 11-bit mantissa).
void orc_dequantize_q4g32(const uint8_t* q, const uint16_t* s16, int64_t n, int64_t k, float* w) {
    const int64_t G = k / 32;
#pragma omp parallel for schedule(static) if (n * k > (1 << 20))
    for (int64_t j = 0; j < n; ++j)
        for (int64_t i = 0; i < k / 2; ++i) {
            const uint8_t b = q[j * (k / 2) + i];
            const float sc = half_to_float(s16[j * G + (2 * i) / 32]);
            w[j * k + 2 * i] = ((float)((b >> 4) & 0x0F) - 8.0f) * sc;
            w[j * k + 2 * i + 1] = ((float)(b & 0x0F) - 8.0f) * sc;
        }
}

float orc_half_to_float(uint16_t h) { return half_to_float(h); }
uint16_t orc_float_to_half(float f) { return float_to_half(f); }

// ---- GEMV / GEMM in the three reference accumulation orders ----
// fmt: 0 = F32 (w), 1 = Q8_ROW (w = int8, s), 2 = Q4_ROW (w = packed bytes, s)
static WView make_view(int32_t fmt, const void* w, const float* s) {
    WView v{fmt, nullptr, nullptr, nullptr, s};
    if (fmt == F32) v.f = (const float*)w;
    if (fmt == Q8_ROW) v.q8 = (const int8_t*)w;
    if (fmt == Q4_ROW) v.q4 = (const uint8_t*)w;
    return v;
}

void orc_matvec_mul_into(int32_t fmt, const float* h, int64_t in_f, const void* w, const float* s, int64_t out_f,
                         float* out) {
    matvec_mul_into(h, in_f, make_view(fmt, w, s), out, out_f);
}
void orc_matvec_mul(int32_t fmt, const float* h, int64_t in_f, const void* w, const float* s, int64_t out_f,
                    float* out) {
    matvec_mul(h, in_f, make_view(fmt, w, s), out, out_f);
}
void orc_gemm_cpu(int32_t fmt, const float* hb, int64_t bs, int64_t in_f, const void* w, const float* s,
                  int64_t out_f, float* out) {
    gemm_cpu(hb, make_view(fmt, w, s), bs, in_f, out_f, out);
}

// ---- elementwise / attention ops ----
void orc_rms_norm(const float* x, const float* w, float eps, int64_t n, float* out) { rms_norm(x, w, eps, out, n); }
void orc_rope_thetas(int64_t hd, float theta, float* out) { rope_thetas(hd, theta, out); }
void orc_apply_rope(float* v, int64_t pos, int64_t nh, int64_t hd, float theta) { apply_rope(v, pos, nh, hd, theta); }
void orc_attn_decode(const float* q, const float* kc, const float* vc, int64_t kv_len, int64_t nq, int64_t nkv,
                     int64_t hd, float* out) {
    attend_decode(q, kc, vc, kv_len, nq, nkv, hd, out);
}
// flash_attention_cpu: block of `bs` query rows at absolute positions start_pos+b,
// each attending to cache rows [0, start_pos+b] (cpu_engine.rs:1151-1214).
void orc_attn_prefill(const float* qb, const float* kc, const float* vc, int64_t bs, int64_t start_pos, int64_t nq,
                      int64_t nkv, int64_t hd, float* out) {
    attend_prefill(qb, kc, vc, bs, start_pos, nq, nkv, hd, out);
}
// 1: token-blocked / parallel forms (default); 0: the scalar loops they are pinned against.
void orc_set_fast(int on) { g_fast = on ? 1 : 0; }
void orc_silu_mul(const float* g, const float* u, int64_t n, float* out) {
    for (int64_t i = 0; i < n; ++i) out[i] = silu_mul(g[i], u[i]);
}

// ---- whole decoder ----
struct orc_config {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    float rope_theta, rms_eps;
    int32_t attn_bias;    // q/k/v biases present
    int32_t o_bias;       // o_proj bias present
    int32_t wfmt;         // projection format: F32, Q8_ROW, Q4_ROW or Q4_G32
    int32_t head_fmt;     // tied embedding / LM head format: F32 or Q4_G32
    int32_t max_context;  // sink-eviction limit (reference: 4096); <= 0 disables
    int32_t sink_tokens;  // sink rows kept on eviction (reference: 4)
};

struct OrcWeight {
    int32_t fmt = F32;
    int64_t n = 0, k = 0;
    std::vector<float> f;
    std::vector<int8_t> q8;
    std::vector<uint8_t> q4;
    std::vector<float> s;
    WView view() const { return WView{fmt, f.data(), q8.data(), q4.data(), s.data()}; }
};

struct OrcLayer {
    OrcWeight q, k, v, o, gate, up, down;
    std::vector<float> ln1, ln2, bq, bk, bv, bo;
};

struct OrcModel {
    orc_config c;
    std::vector<float> embed;  // [V][H] f32 (dequantized when the table is 4-bit)
    std::vector<float> lm;     // untied LM head [V][H] (empty: the embedding)
    std::vector<float> norm;
    std::vector<OrcLayer> layers;
};

struct KvCache {  // LayerKvCache: cpu_engine.rs:1720-1755
    std::vector<float> k, v;
};

// append_and_evict: cpu_engine.rs:1728-1754
static void kv_append(KvCache& c, const float* nk, const float* nv, int64_t rows, int64_t head_size, int64_t max_ctx,
                      int64_t sinks) {
    c.k.insert(c.k.end(), nk, nk + rows * head_size);
    c.v.insert(c.v.end(), nv, nv + rows * head_size);
    if (max_ctx <= 0) return;
    const int64_t cur = (int64_t)c.k.size() / head_size;
    if (cur > max_ctx) {
        const int64_t evict = cur - max_ctx;
        const int64_t ds = sinks * head_size, de = ds + evict * head_size;
        if (de < (int64_t)c.k.size()) {
            c.k.erase(c.k.begin() + ds, c.k.begin() + de);
            c.v.erase(c.v.begin() + ds, c.v.begin() + de);
        }
    }
}

void* orc_model_create(const orc_config* cfg) {
    OrcModel* m = new OrcModel();
    m->c = *cfg;
    m->layers.resize(cfg->n_layers);
    return m;
}
void orc_model_destroy(void* p) { delete (OrcModel*)p; }

static int parse_layer_name(const char* name, int* layer, const char** rest) {
    if (std::strncmp(name, "model.layers.", 13) != 0) return 0;
    const char* p = name + 13;
    int l = 0;
    if (*p < '0' || *p > '9') return 0;
    while (*p >= '0' && *p <= '9') l = l * 10 + (*p++ - '0');
    if (*p != '.') return 0;
    *layer = l;
    *rest = p + 1;
    return 1;
}

// Set a tensor by its Hugging Face name. Projections take the model's wfmt:
// F32: data = f32[n*k]; Q8_ROW: data = int8[n*k], scales = f32[n];
// Q4_ROW: data = u8[n*k/2], scales = f32[n]; Q4_G32: data = u8[n*k/2], scales = fp16 bits [n*k/32]
// (stored dequantized, since the oracle's Q4_G32 GEMV is the Float GEMV of the dequantized weights).
// "model.embed_tokens.weight" takes head_fmt (F32 or Q4_G32). Vectors (norms, biases) are f32.
int orc_model_set(void* p, const char* name, const void* data, const void* scales) {
    OrcModel* m = (OrcModel*)p;
    const orc_config& c = m->c;
    const int64_t H = c.hidden, QD = (int64_t)c.n_heads * c.head_dim, KD = (int64_t)c.n_kv_heads * c.head_dim,
                  I = c.ffn, V = c.vocab;
    auto vec = [](std::vector<float>& dst, const void* src, int64_t n) {
        dst.assign((const float*)src, (const float*)src + n);
    };
    auto proj = [&](OrcWeight& w, int64_t n, int64_t k) {
        w.n = n;
        w.k = k;
        w.fmt = c.wfmt;
        if (c.wfmt == F32) {
            w.f.assign((const float*)data, (const float*)data + n * k);
        } else if (c.wfmt == Q8_ROW) {
            w.q8.assign((const int8_t*)data, (const int8_t*)data + n * k);
            w.s.assign((const float*)scales, (const float*)scales + n);
        } else if (c.wfmt == Q4_ROW) {
            w.q4.assign((const uint8_t*)data, (const uint8_t*)data + n * k / 2);
            w.s.assign((const float*)scales, (const float*)scales + n);
        } else {
            w.fmt = F32;
            w.f.resize(n * k);
            orc_dequantize_q4g32((const uint8_t*)data, (const uint16_t*)scales, n, k, w.f.data());
        }
    };
    if (!std::strcmp(name, "model.embed_tokens.weight")) {
        if (c.head_fmt == F32) {
            vec(m->embed, data, V * H);
        } else {
            m->embed.resize(V * H);
            orc_dequantize_q4g32((const uint8_t*)data, (const uint16_t*)scales, V, H, m->embed.data());
        }
        return 0;
    }
    if (!std::strcmp(name, "lm_head.weight")) {  // cpu_engine.rs:2449-2455: lm_head, else the embedding
        if (c.head_fmt == F32) {
            vec(m->lm, data, V * H);
        } else {
            m->lm.resize(V * H);
            orc_dequantize_q4g32((const uint8_t*)data, (const uint16_t*)scales, V, H, m->lm.data());
        }
        return 0;
    }
    if (!std::strcmp(name, "model.norm.weight")) {
        vec(m->norm, data, H);
        return 0;
    }
    int l;
    const char* r;
    if (!parse_layer_name(name, &l, &r) || l < 0 || l >= c.n_layers) return -1;
    OrcLayer& L = m->layers[l];
    if (!std::strcmp(r, "input_layernorm.weight")) vec(L.ln1, data, H);
    else if (!std::strcmp(r, "post_attention_layernorm.weight")) vec(L.ln2, data, H);
    else if (!std::strcmp(r, "self_attn.q_proj.weight")) proj(L.q, QD, H);
    else if (!std::strcmp(r, "self_attn.k_proj.weight")) proj(L.k, KD, H);
    else if (!std::strcmp(r, "self_attn.v_proj.weight")) proj(L.v, KD, H);
    else if (!std::strcmp(r, "self_attn.o_proj.weight")) proj(L.o, H, QD);
    else if (!std::strcmp(r, "mlp.gate_proj.weight")) proj(L.gate, I, H);
    else if (!std::strcmp(r, "mlp.up_proj.weight")) proj(L.up, I, H);
    else if (!std::strcmp(r, "mlp.down_proj.weight")) proj(L.down, H, I);
    else if (!std::strcmp(r, "self_attn.q_proj.bias")) vec(L.bq, data, QD);
    else if (!std::strcmp(r, "self_attn.k_proj.bias")) vec(L.bk, data, KD);
    else if (!std::strcmp(r, "self_attn.v_proj.bias")) vec(L.bv, data, KD);
    else if (!std::strcmp(r, "self_attn.o_proj.bias")) vec(L.bo, data, H);
    else return -1;
    return 0;
}

// Repetition penalty 1.15 over the generated ids (each occurrence applies once more),
// in place: cpu_engine.rs:2984-2992; then the first-max argmax: :3024-3031.
int64_t orc_penalize_argmax(float* logits, int64_t V, const uint32_t* gen, int64_t n_gen) {
    const float rp = 1.15f;
    for (int64_t g = 0; g < n_gen; ++g) {
        const uint32_t prev = gen[g];
        if ((int64_t)prev < V) {
            const float lg = logits[prev];
            logits[prev] = lg > 0.f ? lg / rp : lg * rp;
        }
    }
    int64_t best = 0;
    float bv = -INFINITY;
    for (int64_t i = 0; i < V; ++i)
        if (logits[i] > bv) {
            bv = logits[i];
            best = i;
        }
    return best;
}

// The temperature > 0 branch of the token choice (cpu_engine.rs:2998-3022) over already
// penalized logits, with the uniform draw r passed in (the reference takes it from thread_rng):
// divide by the temperature, softmax over the whole vocabulary, stable sort by probability
// (descending; incomparable pairs keep their order), keep top_k, renormalise, and return the first
// id whose cumulative probability reaches r (the most likely one if none does).
int64_t orc_sample_topk(const float* penalized, int64_t V, float temperature, int top_k, float r) {
    std::vector<float> v(penalized, penalized + V);
    for (auto& x : v) x /= temperature;
    float mx = -INFINITY;
    for (float x : v) mx = std::isnan(mx) ? x : (std::isnan(x) ? mx : std::max(mx, x));  // f32::max
    std::vector<float> ex(V);
    float sum = 0.f;
    for (int64_t i = 0; i < V; ++i) {
        ex[i] = expf(v[i] - mx);
        sum += ex[i];
    }
    if (sum > 0.f)
        for (auto& e : ex) e /= sum;
    std::vector<int64_t> idx(V);
    for (int64_t i = 0; i < V; ++i) idx[i] = i;
    // the reference's comparator treats NaN as equal to everything; NaN probabilities (from NaN
    // logits) sort here as 0 so that the order stays a strict weak ordering
    std::vector<float> key(ex);
    for (auto& k : key)
        if (std::isnan(k)) k = 0.f;
    std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) { return key[a] > key[b]; });
    if ((int64_t)top_k < V) idx.resize(top_k);
    float top_sum = 0.f;
    for (int64_t i : idx) top_sum += ex[i];
    std::vector<float> p(idx.size());
    for (size_t i = 0; i < idx.size(); ++i) p[i] = top_sum > 0.f ? ex[idx[i]] / top_sum : ex[idx[i]];
    int64_t selected = idx[0];
    float cum = 0.f;
    for (size_t i = 0; i < idx.size(); ++i) {
        cum += p[i];
        if (r <= cum) {
            selected = idx[i];
            break;
        }
    }
    return selected;
}

// generate_cpu_inner_logits with CPU-only mode and temperature 0:
// prefill of tokens [0, n-1) in chunks of 64 (cpu_engine.rs:2586-2757), then the
// single-token decode loop (:2788-3064): embedding row id % V, 24 x [norm, QKV
// (+bias), RoPE, KV append, attention, O (+bias), residual, norm, MLP, residual],
// final norm, LM head, repetition penalty 1.15 over generated ids, first-max
// argmax, stop after emitting 2 / 151645 / 151643.
// raw_logits (optional, max_new * V floats) receives each step's logits BEFORE the
// penalty. Returns the number of generated ids written to out_ids.
//
// With a prefix-cache hit (cpu_engine.rs:2518-2534, 2577-2582) the caches start as the
// entry's rows: k_in / v_in [n_layers][prefix_len][n_kv * head_dim], and the prefill runs
// from position prefix_len (:2590-2606). k_out / v_out (optional) receive the caches after
// the prefill, the rows save_prefix stores (:2746-2756): [n_layers][rows][n_kv * head_dim]
// with rows = the prefill end (at most max_context with eviction), written to *kv_rows_out.
int64_t orc_generate_ex(void* p, const uint32_t* prompt, int64_t n_prompt, int64_t max_new, uint32_t* out_ids,
                        float* raw_logits, int64_t prefix_len, const float* k_in, const float* v_in, float* k_out,
                        float* v_out, int64_t* kv_rows_out) {
    OrcModel* m = (OrcModel*)p;
    const orc_config& c = m->c;
    const int64_t H = c.hidden, NQ = c.n_heads, NKV = c.n_kv_heads, HD = c.head_dim, QD = NQ * HD, KD = NKV * HD,
                  I = c.ffn, V = c.vocab, NL = c.n_layers;
    const float eps = c.rms_eps, theta = c.rope_theta;
    std::vector<uint32_t> tokens(prompt, prompt + n_prompt);
    if (tokens.empty()) tokens.push_back(1);  // :2487-2489
    std::vector<KvCache> kv(NL);
    if (k_in && v_in && prefix_len > 0)
        for (int64_t l = 0; l < NL; ++l) {
            kv[l].k.assign(k_in + l * prefix_len * KD, k_in + (l + 1) * prefix_len * KD);
            kv[l].v.assign(v_in + l * prefix_len * KD, v_in + (l + 1) * prefix_len * KD);
        }
    else
        prefix_len = 0;
    const WView lm{F32, m->lm.empty() ? m->embed.data() : m->lm.data(), nullptr, nullptr, nullptr};

    // ---- prefill ----
    const int64_t pre_end = tokens.size() > 1 ? (int64_t)tokens.size() - 1 : 0;
    // flash_attention_cpu reads rows [0, pos] of the cache by absolute position (:1166-1170):
    // once eviction has dropped rows that is past the cache's end, where the reference's slice
    // indexing panics. The oracle refuses the same inputs.
    if (c.max_context > 0 && pre_end > c.max_context) return -1;
    for (int64_t pos = prefix_len; pos < pre_end; pos += 64) {
        const int64_t end = std::min(pos + 64, pre_end), bs = end - pos;
        std::vector<float> x(bs * H), hb(bs * H), qb(bs * QD), kb(bs * KD), vb(bs * KD), ctx(bs * QD), ob(bs * H),
            h2(bs * H), g(bs * I), u(bs * I), mm(bs * I), dn(bs * H);
        for (int64_t i = 0; i < bs; ++i) {
            const int64_t id = tokens[pos + i] % V;
            std::memcpy(&x[i * H], &m->embed[id * H], H * 4);
        }
        for (int64_t l = 0; l < NL; ++l) {
            const OrcLayer& L = m->layers[l];
            for (int64_t i = 0; i < bs; ++i) rms_norm(&x[i * H], L.ln1.data(), eps, &hb[i * H], H);
            if (bs == 1) {  // :2657-2671 -> matvec_mul (single sum)
                matvec_mul(hb.data(), H, L.q.view(), qb.data(), QD);
                matvec_mul(hb.data(), H, L.k.view(), kb.data(), KD);
                matvec_mul(hb.data(), H, L.v.view(), vb.data(), KD);
            } else {  // fused_qkv_gemm: :3325-3339
                gemm_cpu(hb.data(), L.q.view(), bs, H, QD, qb.data());
                gemm_cpu(hb.data(), L.k.view(), bs, H, KD, kb.data());
                gemm_cpu(hb.data(), L.v.view(), bs, H, KD, vb.data());
            }
            for (int64_t i = 0; i < bs; ++i) {
                if (!L.bq.empty()) for (int64_t j = 0; j < QD; ++j) qb[i * QD + j] += L.bq[j];
            }
            for (int64_t i = 0; i < bs; ++i) {
                if (!L.bk.empty()) for (int64_t j = 0; j < KD; ++j) kb[i * KD + j] += L.bk[j];
            }
            for (int64_t i = 0; i < bs; ++i) {
                if (!L.bv.empty()) for (int64_t j = 0; j < KD; ++j) vb[i * KD + j] += L.bv[j];
            }
#pragma omp parallel for schedule(static) if (g_fast)
            for (int64_t i = 0; i < bs; ++i) {
                apply_rope(&qb[i * QD], pos + i, NQ, HD, theta);
                apply_rope(&kb[i * KD], pos + i, NKV, HD, theta);
            }
            kv_append(kv[l], kb.data(), vb.data(), bs, KD, c.max_context, c.sink_tokens);
            // flash_attention_cpu indexes the cache by absolute position (:2700-2704)
            attend_prefill(qb.data(), kv[l].k.data(), kv[l].v.data(), bs, pos, NQ, NKV, HD, ctx.data());
            if (bs == 1) {
                matvec_mul(ctx.data(), QD, L.o.view(), ob.data(), H);
            } else {
                gemm_cpu(ctx.data(), L.o.view(), bs, QD, H, ob.data());
            }
            if (!L.bo.empty())
                for (int64_t i = 0; i < bs; ++i)
                    for (int64_t j = 0; j < H; ++j) ob[i * H + j] += L.bo[j];
            // per token: residual, norm, run_mlp_into (:2718-2742); the MLP GEMVs of the chunk's
            // tokens run as one token-blocked pass of matvec_mul_into
            for (int64_t i = 0; i < bs; ++i) {
                float* xr = &x[i * H];
                for (int64_t d = 0; d < H; ++d) xr[d] += ob[i * H + d];
                rms_norm(xr, L.ln2.data(), eps, &h2[i * H], H);
            }
            matvec_into_tokens(h2.data(), bs, H, L.gate.view(), g.data(), I);
            matvec_into_tokens(h2.data(), bs, H, L.up.view(), u.data(), I);
            for (int64_t e = 0; e < bs * I; ++e) {
                const float sg = g[e] * (1.0f / (1.0f + expf(-g[e])));
                mm[e] = sg * u[e];
            }
            matvec_into_tokens(mm.data(), bs, I, L.down.view(), dn.data(), H);
            for (int64_t i = 0; i < bs; ++i)
                for (int64_t d = 0; d < H; ++d) x[i * H + d] += dn[i * H + d];
        }
    }
    if (kv_rows_out) *kv_rows_out = (int64_t)kv[0].k.size() / KD;
    if (k_out && v_out)
        for (int64_t l = 0; l < NL; ++l) {
            std::memcpy(k_out + l * (int64_t)kv[l].k.size(), kv[l].k.data(), kv[l].k.size() * 4);
            std::memcpy(v_out + l * (int64_t)kv[l].v.size(), kv[l].v.data(), kv[l].v.size() * 4);
        }

    // ---- decode ----
    std::vector<float> x(H), h(H), q(QD), k(KD), v(KD), att(QD), o(H), h2(H), down(H), fn(H), logits(V);
    std::vector<float> g(I), u(I), mm(I);
    std::vector<uint32_t> gen;
    while ((int64_t)gen.size() < max_new) {
        const int64_t id = tokens.back() % V;
        std::memcpy(x.data(), &m->embed[id * H], H * 4);
        const int64_t pos = (int64_t)tokens.size() - 1;
        for (int64_t l = 0; l < NL; ++l) {
            const OrcLayer& L = m->layers[l];
            rms_norm(x.data(), L.ln1.data(), eps, h.data(), H);
            matvec_mul_into(h.data(), H, L.q.view(), q.data(), QD);
            matvec_mul_into(h.data(), H, L.k.view(), k.data(), KD);
            matvec_mul_into(h.data(), H, L.v.view(), v.data(), KD);
            if (!L.bq.empty()) for (int64_t j = 0; j < QD; ++j) q[j] += L.bq[j];
            if (!L.bk.empty()) for (int64_t j = 0; j < KD; ++j) k[j] += L.bk[j];
            if (!L.bv.empty()) for (int64_t j = 0; j < KD; ++j) v[j] += L.bv[j];
            apply_rope(q.data(), pos, NQ, HD, theta);
            apply_rope(k.data(), pos, NKV, HD, theta);
            kv_append(kv[l], k.data(), v.data(), 1, KD, c.max_context, c.sink_tokens);
            const int64_t kv_len = (int64_t)kv[l].k.size() / KD;
            attend_decode(q.data(), kv[l].k.data(), kv[l].v.data(), kv_len, NQ, NKV, HD, att.data());
            matvec_mul_into(att.data(), QD, L.o.view(), o.data(), H);
            if (!L.bo.empty()) for (int64_t j = 0; j < H; ++j) o[j] += L.bo[j];
            for (int64_t d = 0; d < H; ++d) x[d] += o[d];
            rms_norm(x.data(), L.ln2.data(), eps, h2.data(), H);
            mlp(h2.data(), L.gate.view(), L.up.view(), L.down.view(), H, I, g.data(), u.data(), mm.data(),
                down.data());
            for (int64_t d = 0; d < H; ++d) x[d] += down[d];
        }
        rms_norm(x.data(), m->norm.data(), eps, fn.data(), H);
        matvec_mul_into(fn.data(), H, lm, logits.data(), V);
        if (raw_logits) std::memcpy(raw_logits + gen.size() * V, logits.data(), V * 4);
        const uint32_t tid = (uint32_t)orc_penalize_argmax(logits.data(), V, gen.data(), (int64_t)gen.size());
        gen.push_back(tid);
        tokens.push_back(tid);
        if (tid == 2 || tid == 151645 || tid == 151643) break;  // :3060
    }
    std::memcpy(out_ids, gen.data(), gen.size() * 4);
    return (int64_t)gen.size();
}

int64_t orc_generate(void* p, const uint32_t* prompt, int64_t n_prompt, int64_t max_new, uint32_t* out_ids,
                     float* raw_logits) {
    return orc_generate_ex(p, prompt, n_prompt, max_new, out_ids, raw_logits, 0, nullptr, nullptr, nullptr, nullptr,
                           nullptr);
}

int orc_num_threads(void) { return omp_get_max_threads(); }
// Thread count of the following calls (tests check that results do not depend on it).
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }

}  // extern "C"
