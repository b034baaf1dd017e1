// bh_internal.h — shared declarations of the backend's host runtime and kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>
#include <functional>
#include <string>

#include "../../include/bramha_hip.h"

namespace bh {

// ---------------------------------------------------------------------------
// Device weight layout ("KM16"): the matrix W[n][k] is cut along k into 16-byte
// chunks of E elements (Q4: 32, Q8: 16, F32: 4) and stored chunk-major:
// chunk (c, n) at byte (c * n_pad + n) * 16, n_pad = n rounded up to 64 (zero
// rows). A wavefront of 64 lanes owns 64 consecutive rows and reads 1 KiB of
// contiguous weights per chunk step while the activations for that chunk are
// the same for every lane (scalar loads). Q4 chunks keep the reference's byte
// order: byte b of the chunk holds elements 2b (high nibble) and 2b+1 (low).
// Scales: BH_Q4_G32 fp16 [C][n_pad] (chunk c == group c), row formats f32 [n_pad].
// ---------------------------------------------------------------------------
inline int chunk_elems(int fmt) { return fmt == BH_Q4_ROW || fmt == BH_Q4_G32 ? 32 : (fmt == BH_Q8_ROW ? 16 : 4); }
inline int64_t pad64(int64_t n) { return (n + 63) / 64 * 64; }

struct DevWeight {
    int fmt = BH_F32;
    int64_t n = 0, k = 0, n_pad = 0, chunks = 0;
    void* q = nullptr;  // uint4 chunks
    void* s = nullptr;  // scales
    size_t bytes = 0;   // device bytes held
};

// Algorithmic bytes of one full read of the weight (reference layout, scales included).
inline double weight_bytes(const DevWeight& w) {
    const double nk = (double)w.n * (double)w.k;
    switch (w.fmt) {
        case BH_Q4_G32: return nk * 0.5 + nk / 32.0 * 2.0;
        case BH_Q4_ROW: return nk * 0.5 + (double)w.n * 4.0;
        case BH_Q8_ROW: return nk + (double)w.n * 4.0;
        default: return nk * 4.0;
    }
}

// ---------------------------------------------------------------------------
// Kernel launch parameters
// ---------------------------------------------------------------------------
enum Epi : int {
    EPI_STORE = 0,   // y = acc (+ bias)
    EPI_RESID = 1,   // y += acc (+ bias)          (O / down projection + residual)
    EPI_SILU = 2,    // y = silu(acc_gate) * acc_up (gate/up pair)
    EPI_QKV = 3,     // bias, RoPE, q -> y, k/v -> KV cache
    EPI_LMHEAD = 4,  // logits -> y, repetition penalty, per-tile argmax -> partial
    EPI_PART = 5,    // K split over workgroups: scaled partial sums -> part[split][b][n]
};

struct KvView {            // packed KV cache of one layer
    void* k = nullptr;     // [n_kv][kv_rows][hd]
    void* v = nullptr;
    int64_t kv_rows = 0;
    int kv_f16 = 1;
    int max_context = 0;   // > 0: ring of (max_context - sink) rows after `sink` fixed rows
    int sink = 0;
};

struct GemvArgs {
    const void* W = nullptr;
    const void* S = nullptr;
    const void* W2 = nullptr;  // EPI_SILU: up projection (W is gate)
    const void* S2 = nullptr;
    const float* x = nullptr;
    int64_t ldx = 0;
    float* y = nullptr;
    int64_t ldy = 0;
    const float* bias = nullptr;
    int N = 0, n_pad = 0, C = 0;
    int batch = 0;
    // EPI_QKV
    int qd = 0, kd = 0, hd = 0;
    const int32_t* pos = nullptr;      // [batch]
    const int32_t* slot = nullptr;     // [batch]
    const int64_t* seq_off = nullptr;  // [slots]
    const float2* rope = nullptr;      // [max_pos][hd/2] (cos, sin)
    KvView kv;
    // EPI_LMHEAD
    const uint16_t* pen = nullptr;     // [slots][vocab] generated-id counts
    int vocab = 0;
    float* part_val = nullptr;         // [batch][tiles]
    int32_t* part_idx = nullptr;
    // EPI_PART: `ksw` workgroups per row tile each write their scaled partial sums to
    // part[split][b][n] (stride part_ld per split, N per row); the consumer adds them.
    float* part = nullptr;
    int ksw = 1;
    int64_t part_ld = 0;
};

// Launchers (k_gemv.hip). Return hipSuccess or the launch error.
hipError_t launch_gemv(int fmt, int epi, const GemvArgs& a, hipStream_t st);

// k_ops.hip
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* out, int rows, int n, hipStream_t st);
// Residual reduce + RMSNorm per row b: x[b] += sum_{s < splits} part[s][b] (+ bias), in a
// fixed order, then h[b] = x[b] * (1/sqrt(mean(x[b]^2) + eps)) * w. splits 0: norm only.
hipError_t launch_resid_norm(float* x, const float* part, int splits, int64_t part_ld, const float* bias,
                             const float* w, float eps, float* h, int rows, int n, hipStream_t st);
// Split count for an EPI_PART GEMV over `tiles` row tiles and C chunks.
int part_splits(int tiles, int C);
hipError_t launch_rope(float* v, const int32_t* pos, const float2* tab, int rows, int n_heads, int hd, hipStream_t st);
hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t st);
hipError_t launch_dequant(const DevWeight& w, float* out, hipStream_t st);
// Embedding rows of the tied table (KM16 layout, F32 or Q4_G32) for tokens tok[b] % vocab.
// decode_prologue != 0: first set tok[b] = next[b], pos[b] = seq_len[slot[b]]++ .
hipError_t launch_embed(const DevWeight& table, int32_t* tok, int32_t* pos, const int32_t* slot, int32_t* seq_len,
                        const uint32_t* next, int decode_prologue, float* x, int64_t ldx, int batch, hipStream_t st);
// Final argmax over the LM head's per-tile partials; writes next ids, bumps penalty counts,
// appends to the id capture buffer (ids_cap + step * batch) when non-null.
hipError_t launch_sample_final(const float* part_val, const int32_t* part_idx, int tiles, int batch,
                               const int32_t* slot, uint16_t* pen, int vocab, uint32_t* next, uint32_t* ids_cap,
                               const int32_t* step_ctr, hipStream_t st);
hipError_t launch_step_counter(int32_t* ctr, int reset, hipStream_t st);

// k_attn.hip — attention for `batch` query rows: row b (slot[b], position pos[b]) attends to the
// rows present for its sequence after its own row was appended.
struct AttnArgs {
    const float* q = nullptr;  // [batch][nq*hd]
    int32_t* cnt = nullptr;    // [batch][nkv] arrival counters of the split merge (zero when idle)
    float* out = nullptr;      // [batch][nq*hd]
    KvView kv;
    const int32_t* pos = nullptr;
    const int32_t* slot = nullptr;
    const int64_t* seq_off = nullptr;
    const int32_t* seq_len = nullptr;  // standalone mode: explicit lengths [batch] (pos/slot unused)
    int batch = 0, nq = 0, nkv = 0, hd = 0;
    int splits = 1, split_rows = 0;    // context split: rows per split (multiple of 64)
    float* part_o = nullptr;           // [batch][nq][splits][hd]
    float* part_ml = nullptr;          // [batch][nq][splits][2]
};
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);
// Head layouts the attention kernel is built for: hd 64/128, n_q/n_kv in {1, 2, 4, 7, 8}.
bool attn_supported(int nq, int nkv, int hd);
// Split plan for contexts up to max_len rows.
void attn_plan(int max_len, int batch, int nkv, int* splits, int* split_rows);

// ---------------------------------------------------------------------------
// Host helpers (bh_host.cpp)
// ---------------------------------------------------------------------------
uint16_t f32_to_f16_bits(float f);
float f16_bits_to_f32(uint16_t h);
// Repack a reference-layout weight into KM16 host buffers (q: C*n_pad*16 bytes,
// s: scales in device layout). Returns false on a size/format error.
bool repack_km16(int fmt, int64_t n, int64_t k, const void* q, const void* s, std::string& err, void** out_q,
                 size_t* q_bytes, void** out_s, size_t* s_bytes);
// RoPE table [max_pos][hd/2] of (cos, sin) with the reference's f32 formulas.
void rope_table(int hd, float theta, int max_pos, float2* out);
int quantize_host(int fmt, const float* w, int64_t n, int64_t k, void* q, void* s);
void parallel_for(int64_t n, int64_t min_chunk, const std::function<void(int64_t, int64_t)>& fn);

}  // namespace bh
