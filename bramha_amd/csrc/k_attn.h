// k_attn.h — the MFMA attention wave shared by the decode and prefill attention kernels
// (k_attn.hip) and the batch-1 attention + output projection kernel (k_attn_o.hip).
//
// Operand layout of v_mfma_f32_16x16x32_f16 as in k_mfma.h. K rows are loaded from the cache's
// MFMA-tile order (kv_k_off) and V^T from its transposed order (kv_v_off), 16 bytes per load.
#pragma once

#include <hip/hip_fp16.h>

#include "bh_internal.h"
#include "k_mfma.h"

namespace bh {

// f32 x[0..7] -> fp16 hi and lo with hi + lo == x to ~22 bits
__device__ __forceinline__ void split_hl(const float* x, half8& hi, half8& lo) {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const _Float16 h = (_Float16)x[s];
        hi[s] = h;
        lo[s] = (_Float16)(x[s] - (float)h);
    }
}

// Row of the 64-row tile that lane-group row i of 16-row block blk holds: block pairs (2j, 2j+1)
// cover rows 32j .. 32j+31 with row group g = i / 4 owning rows 32j + 8g .. 32j + 8g + 7.
__device__ __forceinline__ int mf_row(int blk, int i) { return 32 * (blk >> 1) + 8 * (i >> 2) + 4 * (blk & 1) + (i & 3); }

// K and V^T operands of one tile of 32 * NJ rows for one wave (NJ = 2 at head_dim 64, 1 at 128:
// 16 KiB of K + V either way, so two tiles in flight fit the register file).
template <int HD>
struct KvTile {
    static constexpr int NJ = HD == 64 ? 2 : 1;
    half8 k[2 * NJ][HD / 32];  // S^T A operand: rows mf_row(blk, lr), head-dim kc*32 + 8lg .. +7
    half8 v[NJ][HD / 16];      // O^T A operand: head-dim db*16 + lr, rows 32j + 8lg .. +7
};

// The wave's share of a context range for the 16 query columns held as fp16 hi + lo (qh, ql):
// tiles of TR rows at r0 + TR*(wave + NW*i) below r1, with the next tile's K/V loads in flight
// while the current one is multiplied. Row t is
// valid for the lane's column while t < lim (the causal limit of the column). Scores are kept in
// the base-2 domain: s2 = (q . k) * log2(e)/sqrt(hd), p = 2^(s2 - m). On return m is the
// column's running max, l this lane's share of its sum and o its unnormalised output
// (O^T layout: head-dim db*16 + 4lg + v). MASKCOL: columns may have no valid row in a tile.
// start() issues the loads of the wave's first tile (before the caller waits on its queries),
// run() multiplies.
template <int HD, int NW, bool MASKCOL>
struct AttnWave {
    static constexpr int KC = HD / 32;  // 32-wide head-dim chunks of the score product
    static constexpr int DB = HD / 16;  // 16-wide head-dim blocks of the value product
    static constexpr int NJ = KvTile<HD>::NJ;
    static constexpr int NB = 2 * NJ;   // 16-row MFMA blocks per tile
    static constexpr int TR = 32 * NJ;  // rows per tile
    const __half* Kh;  // this KV head's K region (MFMA-tile order, kv_k_off)
    const __half* Vh;  // this KV head's V region (kv_v_off)
    int64_t off;       // the sequence's first row in the region
    bool tiled;        // off is a multiple of 64 (tile-aligned) and kv_rows of 8: 1 KiB operand loads
    bool v8;           // off and kv_rows are multiples of 8: 16-byte V loads
    int r0, r1, lim;
    int lim_all;  // the smallest column limit of the wave (wave-uniform): tiles below it need no mask
    KvTile<HD> A, B;
    int wv = 0, nw = NW;  // this wave's index among the waves sharing the range, and their number

    // The tile at t0 for a sequence whose region is not tile-aligned: rows one by one through
    // kv_k_off / kv_v_off, rows at or past r1 zero.
    __device__ __forceinline__ void load_rows(KvTile<HD>& T, int t0) const {
        const int lane = threadIdx.x & 63;
        const int lr = lane & 15, lg = lane >> 4;
        const half8 zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int blk = 0; blk < NB; ++blk) {
            const int t = t0 + mf_row(blk, lr);
#pragma unroll
            for (int kc = 0; kc < KC; ++kc)
                T.k[blk][kc] = t < r1 ? *(const half8*)(Kh + kv_k_off(off + t, kc * 32 + 8 * lg, HD)) : zero;
        }
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int tg = t0 + 32 * j + 8 * lg;
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                half8 v;
                if (v8 && tg + 7 < r1) {
                    v = *(const half8*)(Vh + kv_v_off(off + tg, db * 16 + lr, HD));
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        v[e] = tg + e < r1 ? (_Float16)__half2float(Vh[kv_v_off(off + tg + e, db * 16 + lr, HD)])
                                           : (_Float16)0.f;
                }
                T.v[j][db] = v;
            }
        }
    }

    // The tile at t0. A tile-aligned region reads the whole tile unconditionally: it lies inside
    // the cache (the region starts on a 64-row boundary and kv_rows is a multiple of 64); K rows
    // at or past r1 only give scores that are masked, V rows there are zeroed by compute().
    __device__ __forceinline__ void load_tile(KvTile<HD>& T, int t0) const {
        if (tiled) load_full(T, t0);
        else load_rows(T, t0);
    }

    // The tile at t0 with every row loaded (rows past r1 included: the caller guarantees they
    // are inside the cache).
    __device__ __forceinline__ void load_full(KvTile<HD>& T, int t0) const {
        const int lane = threadIdx.x & 63;
        const __half* kb = Kh + (off + t0) * HD;
        const __half* vb = Vh + (off + t0) * HD;
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) T.k[blk][kc] = *(const half8*)(kb + ((blk * KC + kc) * 64 + lane) * 8);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int db = 0; db < DB; ++db) T.v[j][db] = *(const half8*)(vb + ((j * DB + db) * 64 + lane) * 8);
    }
    // Zero the V rows at or past r1 (their P is 0, but 0 * NaN of a stale row would not be).
    // K rows past r1 need nothing: their scores are replaced, not multiplied.
    __device__ __forceinline__ void zero_tail(KvTile<HD>& T, int t0) const {
        const int lg = (threadIdx.x & 63) >> 4;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int tg = t0 + 32 * j + 8 * lg;
#pragma unroll
            for (int db = 0; db < DB; ++db)
#pragma unroll
                for (int e = 0; e < 8; ++e) T.v[j][db][e] = tg + e < r1 ? T.v[j][db][e] : (_Float16)0.f;
        }
    }

    __device__ __forceinline__ void start() {
        const int t = r0 + wv * TR;
        if (t < r1) load_tile(A, t);
    }

    // MASK: some row of the tile is at or past a column's limit (the tile straddles lim).
    template <bool MASK>
    __device__ __forceinline__ void compute_t(const KvTile<HD>& T, int t0, const half8 (&qh)[KC],
                                              const half8 (&ql)[KC], float& m, float& l, f32x4 (&o)[DB]) const {
        const int lane = threadIdx.x & 63;
        const int lg = lane >> 4;
        // S^T (queries pre-scaled by log2(e)/sqrt(hd)): lane holds rows mf_row(blk, 4lg + v) of column lr
        f32x4 sc[NB];
#pragma unroll
        for (int blk = 0; blk < NB; ++blk) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kc = 0; kc < KC; ++kc) {
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(T.k[blk][kc], qh[kc], acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(T.k[blk][kc], ql[kc], acc, 0, 0, 0);
            }
            sc[blk] = acc;
        }
        float tmax = -INFINITY;
#pragma unroll
        for (int blk = 0; blk < NB; ++blk)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                if constexpr (MASK) sc[blk][v] = t0 + mf_row(blk, 4 * lg + v) < lim ? sc[blk][v] : -INFINITY;
                tmax = fmaxf(tmax, sc[blk][v]);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 16));
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
        const float mn = fmaxf(m, tmax);  // without MASKCOL finite: row t0 of the tile is valid
        float alpha = __builtin_amdgcn_exp2f(m - mn);  // 0 while m is -inf
        if constexpr (MASKCOL) alpha = mn == -INFINITY ? 1.f : alpha;
        m = mn;
        // P as fp16 hi + lo (hi + lo carries ~22 bits of the f32 probability)
        half8 ph[NJ], pl[NJ];
        float ps = 0.f;
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int s = 0; s < 8; ++s) {
                // slots s = 0..3 are block 2j, s = 4..7 block 2j+1: rows 32j + 8lg + s, the rows
                // of the lane's V^T operand
                const float x = sc[2 * j + (s >> 2)][s & 3];
                float p = __builtin_amdgcn_exp2f(x - mn);  // 0 for masked rows
                if constexpr (MASKCOL) p = x == -INFINITY ? 0.f : p;
                const _Float16 h = (_Float16)p;
                ph[j][s] = h;
                pl[j][s] = (_Float16)(p - (float)h);
                ps += p;
            }
        l = l * alpha + ps;
#pragma unroll
        for (int db = 0; db < DB; ++db) o[db] *= alpha;
        // O^T += V^T . P^T over rows 32j .. 32j+31
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
            for (int db = 0; db < DB; ++db) {
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(T.v[j][db], ph[j], o[db], 0, 0, 0);
                o[db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(T.v[j][db], pl[j], o[db], 0, 0, 0);
            }
    }

    __device__ __forceinline__ void compute(KvTile<HD>& T, int t0, const half8 (&qh)[KC], const half8 (&ql)[KC],
                                            float& m, float& l, f32x4 (&o)[DB]) const {
        if (t0 + TR > r1) zero_tail(T, t0);  // wave-uniform: the rows past r1 a whole-tile load brought
        if (t0 + TR <= lim_all) compute_t<false>(T, t0, qh, ql, m, l, o);  // wave-uniform
        else compute_t<true>(T, t0, qh, ql, m, l, o);
    }

    // The wave's tiles t = r0 + TR wv + k step below r1 (A holds the first on entry), the next
    // tile's loads in flight while the current one is multiplied. Loads under a condition leave
    // the compiler unable to count them, and it then waits for every load in flight before each
    // tile, the prefetch included; so a wave with a run of three or more whole tiles requests the
    // next tile unconditionally (past its last tile it re-reads the current one: one tile of
    // extra reads per wave, which costs more than it saves on runs of one or two tiles).
    template <bool PIPE>
    __device__ __forceinline__ void run_t(const half8 (&qh)[KC], const half8 (&ql)[KC], float& m, float& l, f32x4 (&o)[DB]) {
        const int step = nw * TR;
        for (int t = r0 + wv * TR; t < r1;) {
            const int t2 = t + step;
            if constexpr (PIPE) load_full(B, t2 < r1 ? t2 : t);
            else if (t2 < r1) load_tile(B, t2);
            compute(A, t, qh, ql, m, l, o);
            if (t2 >= r1) break;
            const int t3 = t2 + step;
            if constexpr (PIPE) load_full(A, t3 < r1 ? t3 : t2);
            else if (t3 < r1) load_tile(A, t3);
            compute(B, t2, qh, ql, m, l, o);
            t = t3;
        }
    }
    __device__ __forceinline__ void run(const half8 (&qh)[KC], const half8 (&ql)[KC], float& m, float& l, f32x4 (&o)[DB]) {
        if (tiled && r0 + wv * TR + 2 * nw * TR < r1) run_t<true>(qh, ql, m, l, o);
        else run_t<false>(qh, ql, m, l, o);
    }
};

}  // namespace bh
