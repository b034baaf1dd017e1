// k_xl.h — batch-1 activations as signed 4-bit limbs for the integer-dot GEMV.
//
// A 4-bit weight nibble q enters the dot product as q - 8, which is the nibble q ^ 8 read as a
// signed 4-bit value. v_dot8_i32_i4 multiplies 8 such nibbles with 8 signed 4-bit activation
// nibbles and adds the products to a 32-bit integer exactly, so a chunk of 32 weights costs one
// XOR per 8 weights plus one dot per 8 weights and activation limb, instead of one convert and
// one FMA per weight.
//
// The activations of a 32-element chunk share an exponent: with E the biased exponent of the
// chunk's largest |x|, every element becomes the integer m = rint(x * 2^(156 - E)), |m| <= 2^30,
// written in 8 balanced base-16 digits ("limbs", each in [-8, 7]): m = sum_j l_j 16^j. The dot
// product of a chunk is then 2^(E - 156) * (65536 * S_hi + S_lo) with S_hi = sum_k (q_k - 8)
// (sum_{j >= 4} l_kj 16^(j-4)) and S_lo = sum_k (q_k - 8) (sum_{j < 4} l_kj 16^j), each an exact
// integer below 2^24 in magnitude (32 * 8 * (2^14 + 1) and 32 * 8 * 34952), so both convert to float
// exactly and one FMA rounds their combination. Rounding x to m is relative to the chunk's
// largest element: |x - m 2^(E-156)| <= 2^(E-157) <= 2^-30 max|x|; an element more than 2^30
// below its chunk's maximum counts as zero (the f32 product keeps it).
//
// Layout of the records of an activation row of C chunks (XL_REC_BYTES + 4 bytes per chunk):
// record c at word 32 c: word 4 j + d (j < 8, d < 4) holds limb j of elements 8 d .. 8 d + 7 of
// the chunk, element e in nibble e ^ 1 (the weight byte order: byte i holds element 2 i in its
// high nibble and 2 i + 1 in its low one); the factor 2^(E - 156) of chunk c at word 32 C + c
// (0 for a chunk whose largest |x| is below 2^-97, NaN if it holds Inf or NaN).
#pragma once

#include "bh_internal.h"

namespace bh {

constexpr int XL_LIMBS = 8;
constexpr int XL_REC = 32;
constexpr uint32_t XL_BIAS = 0x88888888u;  // 8 in each of the 8 digits
static_assert(XL_REC * 4 == XL_REC_BYTES && XL_LIMBS * 4 == XL_REC, "record size");

// The chunk's factor from the biased exponent of its largest magnitude.
__device__ __forceinline__ float xl_factor(int eb) {
    if (eb == 255) return __uint_as_float(0x7fc00000u);
    return eb >= 30 ? __uint_as_float((uint32_t)(eb - 156 + 127) << 23) : 0.f;
}

// The 8 limbs of v as the nibbles of one word: u = (m + 0x88888888) ^ 0x88888888 holds in hex
// digit j the two's-complement nibble of l_j (digit d of m + 0x88888888 is l_j + 8, and
// d ^ 8 == (d - 8) & 15); m + 0x88888888 stays within [0, 2^32) for |m| <= 2^30.
__device__ __forceinline__ uint32_t xl_digits(float v, int eb) {
    int m = 0;
    if (eb >= 30 && eb < 255) m = (int)rintf(ldexpf(v, 156 - eb));
    return ((uint32_t)m + XL_BIAS) ^ XL_BIAS;
}

// Lane exchanges inside rows of 16 lanes (DPP): XOR 1, XOR 2, the mirror inside 8 lanes (lane i
// reads 7 - i) and inside 16 (15 - i); every lane reads its partner.
template <int CTRL>
__device__ __forceinline__ uint32_t xl_dpp(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xF, 0xF, false);
}
constexpr int DPP_XOR1 = 0xB1, DPP_XOR2 = 0x4E, DPP_MIRROR8 = 0x141, DPP_MIRROR16 = 0x140;

// Records of the 64 elements held by a full wavefront (lane l holds element 32 c0 + l, c0 even)
// of an activation row of C chunks whose records start at `recs`: chunks c0 and c0 + 1 (the
// second only when c0 + 1 < C). Every lane of the wave must call it.
// The chunk maximum is a reduction over lane exchanges (DPP inside 16-lane rows, one swizzle
// across the two rows of a 32-lane half). The limb words are an 8 x 8 transpose of nibbles in
// each group of 8 lanes: lane e holds the 8 limbs of element e as the nibbles of one word and must
// end up with limb e of the 8 elements, element e' in nibble e' ^ 1. Taking the word of lane e ^ 1
// first makes that an exact transpose, done in three stages that each exchange the nibble blocks
// whose lane bit and nibble bit differ with the partner lane (rotate the partner's word by the
// block size, keep the own nibbles whose bit matches the lane's bit: v_alignbit + v_bfi).
__device__ __forceinline__ void xl_pack64(float v, uint32_t* recs, int64_t c0, int64_t C) {
    const int lane = threadIdx.x & 63;
    uint32_t mb = __float_as_uint(v) & 0x7fffffffu;
    mb = max(mb, xl_dpp<DPP_XOR1>(mb));
    mb = max(mb, xl_dpp<DPP_XOR2>(mb));
    mb = max(mb, xl_dpp<DPP_MIRROR8>(mb));
    mb = max(mb, xl_dpp<DPP_MIRROR16>(mb));
    mb = max(mb, (uint32_t)__builtin_amdgcn_ds_swizzle((int)mb, 0x401F));  // lane ^ 16 within 32
    const int eb = (int)(mb >> 23);
    const int e = lane & 7, g = lane >> 3;  // element in its 8-group; group = word d of chunk g / 4
    uint32_t w = xl_dpp<DPP_XOR1>(xl_digits(v, eb));
    {  // lane bit 0 <-> nibble bit 0
        const uint32_t p = xl_dpp<DPP_XOR1>(w), keep = (e & 1) ? 0xF0F0F0F0u : 0x0F0F0F0Fu;
        const uint32_t r = __builtin_amdgcn_alignbit(p, p, (e & 1) ? 4 : 28);
        w = (w & keep) | (r & ~keep);
    }
    {  // lane bit 1 <-> nibble bit 1
        const uint32_t p = xl_dpp<DPP_XOR2>(w), keep = (e & 2) ? 0xFF00FF00u : 0x00FF00FFu;
        const uint32_t r = __builtin_amdgcn_alignbit(p, p, (e & 2) ? 8 : 24);
        w = (w & keep) | (r & ~keep);
    }
    {  // lane bit 2 <-> nibble bit 2
        const uint32_t p = (uint32_t)__builtin_amdgcn_ds_swizzle((int)w, 0x101F), keep = (e & 4) ? 0xFFFF0000u : 0x0000FFFFu;
        const uint32_t r = __builtin_amdgcn_alignbit(p, p, 16);
        w = (w & keep) | (r & ~keep);
    }
    const int64_t c = c0 + (g >> 2);
    if (c < C) {
        recs[c * XL_REC + e * 4 + (g & 3)] = w;
        if (e == 0 && (g & 3) == 0) recs[C * XL_REC + c] = __float_as_uint(xl_factor(eb));
    }
}

// Sum over one chunk of a lane's row: nibbles q (16 bytes: 32 weights), activation record xr,
// factor f. Returns the dot product before the weight's group scale.
__device__ __forceinline__ float xl_dot_chunk(const uint4 q, const uint32_t* xr, float f) {
    const int t[4] = {(int)(q.x ^ 0x88888888u), (int)(q.y ^ 0x88888888u), (int)(q.z ^ 0x88888888u),
                      (int)(q.w ^ 0x88888888u)};
    int hi = 0, lo = 0;
#pragma unroll
    for (int j = XL_LIMBS - 1; j >= XL_LIMBS / 2; --j) {
        hi = (int)((uint32_t)hi << 4);
#pragma unroll
        for (int d = 0; d < 4; ++d) hi = __builtin_amdgcn_sdot8((int)xr[4 * j + d], t[d], hi, false);
    }
#pragma unroll
    for (int j = XL_LIMBS / 2 - 1; j >= 0; --j) {
        lo = (int)((uint32_t)lo << 4);
#pragma unroll
        for (int d = 0; d < 4; ++d) lo = __builtin_amdgcn_sdot8((int)xr[4 * j + d], t[d], lo, false);
    }
    return fmaf((float)hi, 65536.0f * f, (float)lo * f);
}

}  // namespace bh
