// k_mfma.h — operand helpers for v_mfma_f32_16x16x32_f16 over 4-bit weights.
//
// Operand layout of the 16x16x32 MFMA (64 lanes, lane = 16 * lg + lr): A[i][k] is held by lane
// (lr = i, lg = k / 8), 8 consecutive k per lane; B[k][j] by lane (lr = j, lg = k / 8); the result
// D[i][j] by lane (lr = j) in element v of rows i = 4 * lg + v.
#pragma once

#include <hip/hip_fp16.h>

namespace bh {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// One dword of a Q4 chunk (8 weights) -> 8 exact fp16 values q - 8 for the A operand of
// v_mfma_f32_16x16x32_f16. Register pair j holds (nibble j, nibble j + 4): 1024 + q is
// formed in the fp16 mantissa and 1032 subtracted. Nibble t is element t ^ 1 of the 8
// (the high nibble of a byte is the even element), so K slot s of the lane holds element
// kperm(s) = {1, 5, 0, 4, 3, 7, 2, 6}[s]; the activations use the same permutation (the MFMA
// sum over K is order-free). A function, not a table, so that every index folds at compile time.
__host__ __device__ constexpr int kperm(int s) { return ((s >> 1) ^ 1) + 4 * (s & 1); }

__device__ __forceinline__ half8 dec8(uint32_t w) {
    const half2v off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    half8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t p = ((w >> (4 * j)) & 0x000F000Fu) | 0x64006400u;
        const half2v h = __builtin_bit_cast(half2v, p) + off;
        r[2 * j] = h.x;
        r[2 * j + 1] = h.y;
    }
    return r;
}

// dec8 at 11 VALU operations per dword instead of 15: each pair is one v_and_or_b32 after the
// shift. gfx9 VOP3 encodings take no literal, so with both constants literal the compiler emits a
// separate AND and OR; with 0x64006400 held in a VGPR it cannot fold (plus a lane count that is
// always zero), computed once by the caller and kept across its loop, it selects v_and_or_b32
// with the mask in an SGPR.
struct Dec8K {
    uint32_t magic;
};
__device__ __forceinline__ Dec8K dec8_consts() {
    return Dec8K{0x64006400u + __builtin_amdgcn_mbcnt_lo(0u, 0u)};
}
__device__ __forceinline__ half8 dec8(uint32_t w, const Dec8K& k) {
    const half2v off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    half8 r;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t p = ((w >> (4 * j)) & 0x000F000Fu) | k.magic;
        const half2v h = __builtin_bit_cast(half2v, p) + off;
        r[2 * j] = h.x;
        r[2 * j + 1] = h.y;
    }
    return r;
}

// A operands of a 64-row group from one 16-byte load per lane: on entry d[g] is dword g of the
// chunk of row `lane` (lane l loaded row n0 + l); on exit d[rb] is dword lg of row rb * 16 + lr,
// the A operand of row block rb. A 4 x 4 transpose across the four 16-lane groups: lanes swap
// with the lane 32 away, then with the lane 16 away (v_permlane32_swap, v_permlane16_swap).
// One load instead of four per chunk: the four dword loads of every chunk were what the
// memory pipeline of a CU queued most of.
__device__ __forceinline__ void rows_to_a(uint32_t (&d)[4]) {
    const auto p0 = __builtin_amdgcn_permlane32_swap(d[0], d[2], false, false);
    const auto p1 = __builtin_amdgcn_permlane32_swap(d[1], d[3], false, false);
    const auto q0 = __builtin_amdgcn_permlane16_swap(p0[0], p1[0], false, false);
    const auto q1 = __builtin_amdgcn_permlane16_swap(p0[1], p1[1], false, false);
    d[0] = q0[0];
    d[1] = q0[1];
    d[2] = q1[0];
    d[3] = q1[1];
}

// f32 activations -> fp16 hi + lo (hi + lo carries ~22 bits of the f32 mantissa).
__device__ __forceinline__ void split8(const float4& x0, const float4& x1, half8& hi, half8& lo) {
    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const float f = xv[kperm(s)];
        const _Float16 h = (_Float16)f;
        hi[s] = h;
        lo[s] = (_Float16)(f - (float)h);
    }
}

}  // namespace bh
