// bh_host.cpp — host-side helpers: synthetic data, quantizers, weight repacking,
// the RoPE table. No device code.
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "bh_internal.h"

namespace bh {

void parallel_for(int64_t n, int64_t min_chunk, const std::function<void(int64_t, int64_t)>& fn) {
    if (n <= 0) return;
    unsigned hw = std::thread::hardware_concurrency();
    if (hw == 0) hw = 1;
    if (hw > 16) hw = 16;
    int64_t nt = std::min<int64_t>(hw, (n + min_chunk - 1) / std::max<int64_t>(min_chunk, 1));
    if (nt <= 1) {
        fn(0, n);
        return;
    }
    std::vector<std::thread> th;
    const int64_t per = (n + nt - 1) / nt;
    for (int64_t t = 0; t < nt; ++t) {
        const int64_t a = t * per, b = std::min(n, a + per);
        if (a >= b) break;
        th.emplace_back([=, &fn] { fn(a, b); });
    }
    for (auto& t : th) t.join();
}

// IEEE binary16 conversions (round to nearest even).
float f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu, m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            const float v = (float)m * 5.9604644775390625e-08f;  // m * 2^-24
            std::memcpy(&bits, &v, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7F800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

uint16_t f32_to_f16_bits(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        float a;
        std::memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint16_t)std::nearbyint(a * 16777216.0f));
    }
    const uint32_t e = (ax >> 23) - 112u, man = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (man >> 13);
    const uint32_t rem = man & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h += 1;
    return (uint16_t)(sign | h);
}

// ---------------------------------------------------------------- synthetic data
namespace {
inline uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
constexpr uint64_t kGamma = 0x9E3779B97F4A7C15ull;
inline uint64_t fnv1a(const char* s) {
    uint64_t h = 0xCBF29CE484222325ull;
    for (; s && *s; ++s) {
        h ^= (uint8_t)*s;
        h *= 0x100000001B3ull;
    }
    return h;
}
// i-th output (i >= 0) of SplitMix64 seeded with key.
inline uint64_t stream_bits(uint64_t key, uint64_t i) { return mix64(key + (i + 1) * kGamma); }
inline double u53(uint64_t bits) { return (double)(bits >> 11) * 0x1.0p-53; }
}  // namespace

// Round-half-away-from-zero with the reference's clamp and saturating cast.
static inline float rclamp(float v, float lo, float hi) {
    const float r = std::roundf(v);
    if (std::isnan(r)) return NAN;
    return std::fmin(std::fmax(r, lo), hi);
}

int quantize_host(int fmt, const float* w, int64_t n, int64_t k, void* q, void* s) {
    if (!w || !q || !s || n < 0 || k < 0) return BH_ERR_INVALID;
    if (fmt == BH_Q8_ROW) {
        parallel_for(n, 16, [&](int64_t a, int64_t b) {
            for (int64_t j = a; j < b; ++j) {
                const float* row = w + j * k;
                float mx = 0.f;
                for (int64_t i = 0; i < k; ++i) mx = std::fabs(row[i]) > mx ? std::fabs(row[i]) : mx;
                const float sc = mx == 0.f ? 1.0f : mx / 127.0f;
                ((float*)s)[j] = sc;
                for (int64_t i = 0; i < k; ++i) {
                    const float r = rclamp(row[i] / sc, -127.f, 127.f);
                    ((int8_t*)q)[j * k + i] = std::isnan(r) ? 0 : (int8_t)r;
                }
            }
        });
        return BH_OK;
    }
    if (fmt == BH_Q4_ROW) {
        if (k % 2) return BH_ERR_INVALID;
        parallel_for(n, 16, [&](int64_t a, int64_t b) {
            for (int64_t j = a; j < b; ++j) {
                const float* row = w + j * k;
                float mx = 0.f;
                for (int64_t i = 0; i < k; ++i) mx = std::fabs(row[i]) > mx ? std::fabs(row[i]) : mx;
                const float sc = mx == 0.f ? 1.0f : mx / 7.0f;
                ((float*)s)[j] = sc;
                for (int64_t i = 0; i < k / 2; ++i) {
                    const float r1 = rclamp(row[2 * i] / sc, -7.f, 7.f) + 8.0f;
                    const float r2 = rclamp(row[2 * i + 1] / sc, -7.f, 7.f) + 8.0f;
                    const uint8_t q1 = std::isnan(r1) ? 0 : (uint8_t)r1, q2 = std::isnan(r2) ? 0 : (uint8_t)r2;
                    ((uint8_t*)q)[j * (k / 2) + i] = (uint8_t)((q1 << 4) | (q2 & 0x0F));
                }
            }
        });
        return BH_OK;
    }
    if (fmt == BH_Q4_G32) {
        if (k % 32) return BH_ERR_INVALID;
        const int64_t G = k / 32;
        parallel_for(n, 16, [&](int64_t a, int64_t b) {
            for (int64_t j = a; j < b; ++j) {
                for (int64_t g = 0; g < G; ++g) {
                    const float* x = w + j * k + g * 32;
                    float mx = 0.f;
                    for (int i = 0; i < 32; ++i) mx = std::fabs(x[i]) > mx ? std::fabs(x[i]) : mx;
                    uint16_t h = mx == 0.f ? (uint16_t)0x3C00u : f32_to_f16_bits(mx / 7.0f);
                    if ((h & 0x7FFFu) == 0) h = 0x0001u;
                    ((uint16_t*)s)[j * G + g] = h;
                    const float sc = f16_bits_to_f32(h);
                    for (int i = 0; i < 16; ++i) {
                        const float r1 = rclamp(x[2 * i] / sc, -7.f, 7.f) + 8.0f;
                        const float r2 = rclamp(x[2 * i + 1] / sc, -7.f, 7.f) + 8.0f;
                        const uint8_t q1 = std::isnan(r1) ? 0 : (uint8_t)r1, q2 = std::isnan(r2) ? 0 : (uint8_t)r2;
                        ((uint8_t*)q)[j * (k / 2) + g * 16 + i] = (uint8_t)((q1 << 4) | (q2 & 0x0F));
                    }
                }
            }
        });
        return BH_OK;
    }
    return BH_ERR_UNSUPPORTED;
}

bool repack_km16(int fmt, int64_t n, int64_t k, const void* q, const void* s, std::string& err, void** out_q,
                 size_t* q_bytes, void** out_s, size_t* s_bytes) {
    const int E = chunk_elems(fmt);
    if (k % E != 0) {
        err = "in_features " + std::to_string(k) + " is not a multiple of " + std::to_string(E) +
              " (16-byte chunk of this format)";
        return false;
    }
    const int64_t C = k / E, np = pad64(n);
    const int64_t row_bytes = fmt == BH_F32 ? k * 4 : (fmt == BH_Q8_ROW ? k : k / 2);
    uint8_t* dq = (uint8_t*)calloc((size_t)(C * np * 16), 1);
    if (!dq) {
        err = "host allocation failed";
        return false;
    }
    parallel_for(n, 64, [&](int64_t a, int64_t b) {
        for (int64_t j = a; j < b; ++j) {
            const uint8_t* src = (const uint8_t*)q + j * row_bytes;
            for (int64_t c = 0; c < C; ++c) std::memcpy(dq + (c * np + j) * 16, src + c * 16, 16);
        }
    });
    *out_q = dq;
    *q_bytes = (size_t)(C * np * 16);
    *out_s = nullptr;
    *s_bytes = 0;
    if (fmt == BH_Q4_G32) {
        uint16_t* ds = (uint16_t*)calloc((size_t)(C * np), 2);
        for (int64_t j = 0; j < n; ++j)
            for (int64_t c = 0; c < C; ++c) ds[c * np + j] = ((const uint16_t*)s)[j * C + c];
        *out_s = ds;
        *s_bytes = (size_t)(C * np * 2);
    } else if (fmt == BH_Q8_ROW || fmt == BH_Q4_ROW) {
        float* ds = (float*)calloc((size_t)np, 4);
        std::memcpy(ds, s, (size_t)n * 4);
        *out_s = ds;
        *s_bytes = (size_t)np * 4;
    }
    return true;
}

// get_rope_thetas (cpu_engine.rs:1515-1530) and the per-position angle of
// apply_rope_cpu (:1688-1690): theta_i = 1 / theta^(2i/hd), freq = (pos as f32) * theta_i.
void rope_table(int hd, float theta, int max_pos, float2* out) {
    const int half = hd / 2;
    std::vector<float> th(half);
    for (int i = 0; i < half; ++i) th[i] = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
    parallel_for(max_pos, 256, [&](int64_t a, int64_t b) {
        for (int64_t p = a; p < b; ++p)
            for (int i = 0; i < half; ++i) {
                const float f = (float)p * th[i];
                out[p * half + i] = make_float2(cosf(f), sinf(f));
            }
    });
}

}  // namespace bh

extern "C" {

int bh_synth_normal(uint64_t seed, const char* name, float sigma, int64_t n, float* out) {
    if (!out || n < 0) return BH_ERR_INVALID;
    const uint64_t key = bh::mix64(seed ^ bh::fnv1a(name));
    const int64_t pairs = (n + 1) / 2;
    bh::parallel_for(pairs, 1 << 16, [&](int64_t a, int64_t b) {
        for (int64_t p = a; p < b; ++p) {
            const double u1 = 1.0 - bh::u53(bh::stream_bits(key, 2 * p));  // (0, 1]
            const double u2 = bh::u53(bh::stream_bits(key, 2 * p + 1));
            const double r = std::sqrt(-2.0 * std::log(u1));
            const double ang = 6.283185307179586 * u2;
            out[2 * p] = (float)(sigma * (r * std::cos(ang)));
            if (2 * p + 1 < n) out[2 * p + 1] = (float)(sigma * (r * std::sin(ang)));
        }
    });
    return BH_OK;
}

int bh_synth_tokens(uint64_t seed, const char* name, int64_t n, uint32_t vocab, uint32_t* out) {
    if (!out || n < 0 || vocab == 0) return BH_ERR_INVALID;
    const uint64_t key = bh::mix64(seed ^ bh::fnv1a(name));
    for (int64_t i = 0; i < n; ++i) {
        uint32_t t = (uint32_t)(bh::u53(bh::stream_bits(key, i)) * (double)vocab);
        out[i] = t < vocab ? t : vocab - 1;
    }
    return BH_OK;
}

int bh_quantize(int fmt, const float* w, int64_t n, int64_t k, void* q, void* scales) {
    return bh::quantize_host(fmt, w, n, k, q, scales);
}

}  // extern "C"
