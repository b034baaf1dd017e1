// bh_internal.h — shared declarations of the backend's host runtime and kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
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
// Scales: BH_Q4_G32 fp16 [C][n_pad] (chunk c == group c) with the rows of every 64-row group
// permuted (sc_pos), row formats f32 [n_pad].
// ---------------------------------------------------------------------------
inline int chunk_elems(int fmt) { return fmt == BH_Q4_ROW || fmt == BH_Q4_G32 ? 32 : (fmt == BH_Q8_ROW ? 16 : 4); }
inline int64_t pad64(int64_t n) { return (n + 63) / 64 * 64; }

// Position of row r's fp16 group scale in its chunk's run of n_pad: within a 64-row group, row
// 16 rb + 4 g + v (rb, g, v < 4) sits at 16 g + 4 rb + v. An MFMA wavefront's lanes of group g
// hold D rows 4 g .. 4 g + 3 of each 16-row block rb, so their scales for all four blocks are
// 32 contiguous bytes (two 16-byte loads instead of four 8-byte ones); a lane that owns one row
// (the VALU GEMV) reads its scale at sc_pos(row) as before at row.
__host__ __device__ constexpr inline int64_t sc_pos(int64_t r) {
    return (r & ~(int64_t)63) | (((r >> 2) & 3) << 4) | (((r >> 4) & 3) << 2) | (r & 3);
}

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
    EPI_STORE = 0,    // y = acc (+ bias)
    EPI_RESNORM = 1,  // residual producer (O / down): x += acc (+ bias); xw = x * wnext; ssq per 64 rows
    EPI_SILU = 2,     // y = silu(acc_gate) * acc_up (gate/up pair)
    EPI_QKV = 3,      // bias, RoPE, q -> y, k/v -> KV cache
    EPI_LMHEAD = 4,   // logits -> y, repetition penalty, per-64-row argmax -> partial
};

// Packed KV cache of one layer, one region of kv_rows rows per KV head (K and V alike).
// f32 cache: row-major, element (t, d) of head h at (h * kv_rows + t) * hd + d.
// fp16 cache: "MFMA tiles" — rows grouped in tiles of KV_TILE(hd) rows (64 at hd 64, 32 at
// hd 128: 8 KiB each), and inside a tile the elements stored in the order the attention
// kernel's wavefronts load their v_mfma_f32_16x16x32_f16 operands, so every operand load of a
// wavefront is 1 KiB of contiguous bytes (64 lanes x 16 B). kv_k_off / kv_v_off give the
// offset (in elements, from the head's base h * kv_rows * hd) of element (t, d).
__host__ __device__ constexpr int KV_TILE(int hd) { return hd == 64 ? 64 : 32; }
__host__ __device__ constexpr int KV_TILE_SHIFT(int hd) { return hd == 64 ? 6 : 5; }
static_assert(KV_TILE(64) == 1 << KV_TILE_SHIFT(64) && KV_TILE(128) == 1 << KV_TILE_SHIFT(128), "tile height");
// K operand (16-row block blk, 32-wide chunk kc of the head dim) of lane (lr, lg) holds row
// 32(blk/2) + 8(lr/4) + 4(blk%2) + lr%4 of the tile, dims 32kc + 8lg .. +7.
// (t >= 0, 0 <= d < hd; shifts and masks throughout: a 64-bit division by the run-time tile
// height cost the epilogues that write KV rows more than their stores.)
__host__ __device__ inline int64_t kv_k_off(int64_t t, int d, int hd) {
    const int ts = KV_TILE_SHIFT(hd), kcs = hd >> 5;
    const int r = (int)(t & ((1 << ts) - 1));
    const int blk = 2 * (r >> 5) + ((r & 7) >> 2), lr = 4 * ((r & 31) >> 3) + (r & 3);
    const int kc = d >> 5, lg = (d & 31) >> 3;
    return ((t >> ts) << ts) * hd + ((int64_t)((blk * kcs + kc) * 64 + lr + 16 * lg) * 8 + (d & 7));
}
// V^T operand (32-row group j, 16-wide dim block db) of lane (lr, lg) holds dim 16db + lr of
// rows 32j + 8lg .. +7 of the tile.
__host__ __device__ inline int64_t kv_v_off(int64_t t, int d, int hd) {
    const int ts = KV_TILE_SHIFT(hd), dbs = hd >> 4;
    const int r = (int)(t & ((1 << ts) - 1));
    const int j = r >> 5, lg = (r & 31) >> 3;
    const int db = d >> 4, lr = d & 15;
    return ((t >> ts) << ts) * hd + ((int64_t)((j * dbs + db) * 64 + lr + 16 * lg) * 8 + (r & 7));
}
struct KvView {
    void* k = nullptr;
    void* v = nullptr;
    int64_t kv_rows = 0;
    int kv_f16 = 1;
    int max_context = 0;   // > 0: ring of (max_context - sink) rows after `sink` fixed rows
    int sink = 0;
};

// The residual stream between kernels: x [T][H] (f32), xw = x * (the next RMSNorm's weight),
// and ssq [T][H/64] = sums of x^2 over each 64-element tile. A consumer GEMV reads xw as its
// activations and scales its sums by rnorm = 1/sqrt(sum(ssq)/H + eps): the RMSNorm of
// rms_norm_into (cpu_engine.rs:1292-1302) folded into the projection, since
// sum_k W[n][k] * (x[k] * r * w[k]) = r * sum_k W[n][k] * (x[k] * w[k]).
struct GemvArgs {
    const void* W = nullptr;
    const void* S = nullptr;
    const void* W2 = nullptr;  // EPI_SILU: up projection (W is gate)
    const void* S2 = nullptr;
    const float* x = nullptr;
    int64_t ldx = 0;
    float* y = nullptr;        // EPI_RESNORM: the residual x, updated in place
    int64_t ldy = 0;
    const float* bias = nullptr;
    int N = 0, n_pad = 0, C = 0;
    int batch = 0;
    // consumer side of the residual stream: per-token norm factor from ssq (null: none)
    const float* ssq_in = nullptr;     // [batch][ssq_tiles]
    int ssq_tiles = 0;
    float norm_n = 0.f, eps = 0.f;
    // EPI_RESNORM: xw[b][n] = x[b][n] * wnext[n], ssq_out[b][tile] (stride ssq_tiles)
    float* xw_out = nullptr;
    const float* wnext = nullptr;
    float* ssq_out = nullptr;
    // K split over workgroups: `ksw` workgroups per row tile each store their sums in
    // part[tile * ksw + split][NACC][B][ROWS]; the last to arrive (tile_cnt, reset by it) adds them
    // in split order and runs the epilogue. Needs (tiles * ksw) * NACC * B * ROWS floats of part.
    // ksw = 0 leaves the choice to the launcher (1 without part / tile_cnt).
    int ksw = 0;
    float* part = nullptr;
    int32_t* tile_cnt = nullptr;
    // EPI_QKV
    int qd = 0, kd = 0, hd = 0;
    const int32_t* pos = nullptr;      // [batch] absolute positions
    const int64_t* boff = nullptr;     // [batch] first KV row of each entry's sequence region
    const float2* rope = nullptr;      // [max_pos][hd/2] (cos, sin)
    KvView kv;
    // EPI_LMHEAD
    const int32_t* slot = nullptr;     // [batch]
    const uint16_t* pen = nullptr;     // [n_slots][vocab] generated-id counts
    int n_slots = 0;
    int vocab = 0;
    float* part_val = nullptr;         // [batch][tiles64]
    int32_t* part_idx = nullptr;
    // prefill passes (launch_gemm_pf): scratch of batch * C * 64 fp16 for the activations split
    // once into hi + lo (k_prefill.hip); null: every workgroup splits them itself
    uint16_t* xhl = nullptr;
    // The same hi + lo split, token-major ([batch][N / 32][64] fp16, the order of k_split_act):
    // EPI_RESNORM of the MFMA passes also stores xw_out split there (N % 32 == 0); the batched
    // LM head (k_lmhead.hip) takes its activations from x_hl when set instead of splitting x.
    uint16_t* xw_hl = nullptr;
    const uint16_t* x_hl = nullptr;
    // Batch-1 activations as int4 limb records (k_xl.h: 32 words per 32-element chunk). xl: the
    // records of x, written by its producer; a batch-1 Q4_G32 VALU pass then reads them instead
    // of x. xl_out: a batch-1 EPI_RESNORM / EPI_SILU pass also writes the records of what it
    // stores (xw_out / y). xl_tmp: room for C records where a caller has only x (the single-op
    // entry points): the launcher converts x there first.
    const uint32_t* xl = nullptr;
    uint32_t* xl_out = nullptr;
    uint32_t* xl_tmp = nullptr;
};

// The arguments of tokens b0 .. b0 + n - 1 of `a`: every per-token pointer advanced by b0.
__host__ __device__ inline GemvArgs gemv_tokens(const GemvArgs& a0, int b0, int n) {
    GemvArgs a = a0;
    a.batch = n;
    a.x = a0.x + (int64_t)b0 * a0.ldx;
    a.y = a0.y ? a0.y + (int64_t)b0 * a0.ldy : nullptr;
    if (a0.xw_out) a.xw_out = a0.xw_out + (int64_t)b0 * a0.ldy;
    if (a0.ssq_in) a.ssq_in = a0.ssq_in + (int64_t)b0 * a0.ssq_tiles;
    if (a0.ssq_out) a.ssq_out = a0.ssq_out + (int64_t)b0 * a0.ssq_tiles;
    if (a0.pos) a.pos = a0.pos + b0;
    if (a0.boff) a.boff = a0.boff + b0;
    if (a0.slot) a.slot = a0.slot + b0;
    const int tiles64 = (a0.n_pad + 63) / 64;
    if (a0.xw_hl) a.xw_hl = a0.xw_hl + (int64_t)b0 * (a0.N / 32) * 64;
    if (a0.x_hl) a.x_hl = a0.x_hl + (int64_t)b0 * a0.C * 64;
    if (a0.part_val) a.part_val = a0.part_val + (int64_t)b0 * tiles64;
    if (a0.part_idx) a.part_idx = a0.part_idx + (int64_t)b0 * tiles64;
    return a;
}

// Per-launch timing: while `launch_events` is set (bh_model_time_kernels), every kernel is
// launched with hipExtLaunchKernelGGL, which records the two events at the kernel's own start
// and end on its stream (no separate event commands around the launch).
struct LaunchEvents {
    hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local LaunchEvents* launch_events;
template <typename K, typename... Args>
inline void launch_kernel(K kernel, dim3 grid, dim3 block, size_t shm, hipStream_t st, Args... args) {
    if (launch_events)
        hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)shm, st, launch_events->start, launch_events->stop, 0u,
                              args...);
    else
        hipLaunchKernelGGL(kernel, grid, block, shm, st, args...);
}

// Launchers (k_gemv.hip). Return hipSuccess or the launch error.
hipError_t launch_gemv(int fmt, int epi, const GemvArgs& a, hipStream_t st);
// Limb records (k_xl.h) of the n floats of x (n rounded up to whole 32-element chunks with zeros).
hipError_t launch_xl_pack(const float* x, int n, uint32_t* rec, hipStream_t st);
constexpr int XL_TMP_CHUNKS = 4096;  // chunks of the single-op entry points' record scratch
constexpr int XL_REC_BYTES = 128;    // bytes of one chunk's limb record (plus 4 of its factor)
// MFMA GEMM pass of B = 16 or 32 tokens over 4-bit weights (k_gemm.hip), rw * 64 rows per tile;
// B = 48 .. MF_GROUPED_MAX (multiples of 16): B / 16 groups of 16 tokens in one launch.
constexpr int MF_GROUPED_MAX = 512;
hipError_t launch_gemm_mf(int fmt, int epi, const GemvArgs& a, int B, int rw, hipStream_t st);
// MFMA GEMM over all a.batch tokens at once for prefill chunks (k_prefill.hip): 128-row by
// 128-token tiles (64 tokens for the gate/up pair). Not for EPI_LMHEAD.
hipError_t launch_gemm_pf(int fmt, int epi, const GemvArgs& a, hipStream_t st);
// LM head of 1..32 tokens over a Q4_G32 matrix, about one workgroup per CU with the activations
// in LDS (k_lmhead.hip); lmhead_mf_fits tells whether a pass's shape is within its limits.
bool lmhead_mf_fits(const GemvArgs& a, int n_cu);
hipError_t launch_lmhead_mf(const GemvArgs& a, int n_cu, hipStream_t st);
constexpr int PF_MIN_TOKENS = 64;  // launch_gemv hands passes of at least this many tokens to it
// Workgroups per row tile for a K-split GEMV over `tiles` row tiles and C chunks.
int gemv_splits(int tiles, int C, int min_chunks, int target);
constexpr int MAX_KSW = 16;
// Cache policy of buffer loads for data read once per launch (weights): non-temporal. Used for
// weights of at least STREAM_BYTES packed bytes.
constexpr int CPOL_STREAM = 2;
constexpr size_t STREAM_BYTES = 16u << 20;
constexpr int SPLIT_TOT_MAX = 2 * 32 * 128;  // NACC * B * ROWS floats per workgroup
constexpr int64_t SPLIT_PART_FLOATS = (int64_t)512 * SPLIT_TOT_MAX;  // split sums of one launch
constexpr int SPLIT_TILES_MAX = 4096;  // arrival counters: row tiles (times token groups) of one launch

// k_ops.hip
hipError_t launch_rmsnorm(const float* x, const float* w, float eps, float* out, int rows, int n, hipStream_t st);
hipError_t launch_rope(float* v, const int32_t* pos, const float2* tab, int rows, int n_heads, int hd, hipStream_t st);
hipError_t launch_silu_mul(const float* g, const float* u, float* out, int64_t n, hipStream_t st);
hipError_t launch_dequant(const DevWeight& w, float* out, hipStream_t st);
// Group-32 scales of rows [row0, row0 + n), src [C][n] in device memory, to their sc_pos places.
hipError_t launch_scatter_scales(void* dst, const void* src, int64_t row0, int64_t n, int64_t n_pad, int64_t C,
                                 hipStream_t st);
// Rows [row0, row0 + n) (absolute rows of the packed buffer) of one layer's cache <-> f32
// [n][nkv][hd] (to_host = 1: cache -> kh / vh; 0: kh / vh -> cache).
hipError_t launch_kv_copy(const KvView& kv, int nkv, int hd, int64_t row0, int64_t n, float* kh, float* vh, int to_host,
                          hipStream_t st);
// Start of the residual stream for `batch` tokens tok[b] % vocab: x = embedding row of the tied
// table (KM16, F32 or Q4_G32), xw = x * w0, ssq per 64 elements. reset_step != null: zero it.
hipError_t launch_embed(const DevWeight& table, const int32_t* tok, const float* w0, float* x, float* xw, float* ssq,
                        int ssq_tiles, int32_t* reset_step, int batch, hipStream_t st, uint32_t* xl = nullptr);
// End of a decode step, one workgroup per batch entry: first-max argmax over the LM head's
// per-64-row partials; bumps the penalty count of the chosen id; records it at
// ids_cap[step[b] * batch + b] (ids_cap may be null) and advances step[b]; sets tok[b] to it and
// pos[b] += 1; and starts the next step's residual stream from its embedding row (as launch_embed).
// Uniform [0, 1) draw of a sampling step (24 bits of SplitMix64 over seed, slot and the
// position of the step's input token): reproducible, unlike the reference's thread_rng.
__host__ __device__ inline float sample_uniform(uint64_t seed, int slot, int pos) {
    uint64_t z = seed ^ ((uint64_t)(uint32_t)slot << 32 | (uint32_t)pos);
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return (float)(z >> 40) * (1.0f / 16777216.0f);
}
constexpr int SAMPLE_TOPK_MAX = 64;

struct SampleArgs {
    // temperature > 0: top-k sampling over the penalized logits (cpu_engine.rs:2998-3022)
    float temperature = 0.f;
    int top_k = 40;
    uint64_t seed = 0;
    const float* logits = nullptr;  // raw logits [batch][vocab] (temperature > 0)
    const float* part_val = nullptr;
    const int32_t* part_idx = nullptr;
    int tiles = 0, batch = 0, vocab = 0;
    const int32_t* slot = nullptr;
    uint16_t* pen = nullptr;
    uint32_t* ids_cap = nullptr;
    int32_t* step = nullptr;
    int32_t* tok = nullptr;
    int32_t* pos = nullptr;
    const DevWeight* table = nullptr;
    const float* w0 = nullptr;
    float *x = nullptr, *xw = nullptr, *ssq = nullptr;
    int ssq_tiles = 0;
    uint32_t* xl = nullptr;  // limb records of entry 0's next xw (k_xl.h), for a batch-1 step
};
hipError_t launch_sample(const SampleArgs& a, hipStream_t st);

// k_attn.hip — attention for `batch` query rows: row b attends to the rows of its sequence
// region that start at KV row boff[b]: pos[b] + 1 of them (capped at the sink ring's size) after
// its own row was appended, or seq_len[b] of them in standalone mode.
struct AttnArgs {
    const float* q = nullptr;  // [batch][nq*hd]
    int32_t* cnt = nullptr;    // [batch][nkv] arrival counters of the split merge (zero when idle)
    float* out = nullptr;      // [batch][nq*hd]
    KvView kv;
    const int32_t* pos = nullptr;
    const int64_t* boff = nullptr;     // [batch]
    const int32_t* seq_len = nullptr;  // standalone mode: explicit lengths [batch] (pos unused)
    int batch = 0, nq = 0, nkv = 0, hd = 0;
    int splits = 1, split_rows = 0;    // context split: rows per split (multiple of 64)
    // prefill: the batch rows are prompt tokens at their positions pos[b] in the regions boff[b]
    // (fp16 cache: one workgroup per 16 consecutive rows and query head, the 16 rows of one
    // sequence — a prefill of several sequences pads each to a multiple of 16 rows with pad rows
    // at position -1, which attend to nothing and write no KV row; splits unused)
    int prefill = 0;
    float* part_o = nullptr;           // [batch][nq][splits][hd]
    float* part_ml = nullptr;          // [batch][nq][splits][2]
    // Decode of the device model (fp16 cache, batch <= ATTN_STATIC_B): the entries' first KV
    // rows and the smallest region capacity as launch arguments, fixed while the batch is, so
    // each wave requests its first K/V tile before the positions arrive. 0: read boff.
    int static_off = 0;
    int64_t cap_rows = 0;
    int64_t off_val[32] = {};
};
constexpr int ATTN_STATIC_B = 32;
hipError_t launch_attention(const AttnArgs& a, hipStream_t st);
// Head layouts the attention kernel is built for: hd 64/128, n_q/n_kv in {1, 2, 4, 7, 8}.
bool attn_supported(int nq, int nkv, int hd);
// Split plan for contexts up to max_len rows.
void attn_plan(int max_len, int batch, int nkv, int hd, int* splits, int* split_rows);
// Batch-1 decode: attention, O projection and residual epilogue in one launch (k_attn_o.hip),
// for the configurations attn_o_fusable accepts (Q4_G32, fp16 cache, short contexts).
bool attn_o_fusable(int fmt, const AttnArgs& at, const GemvArgs& o);
hipError_t launch_attn_o(int fmt, const AttnArgs& at, const GemvArgs& o, hipStream_t st);

// k_probe.hip — HBM bandwidth probes: copy = 0 streams `bytes` of src with 16-byte non-temporal
// loads (sink: wgs * 256 words, written only on an impossible value), copy = 1 copies src to dst;
// wgs workgroups of 256 threads, `unroll` (4, 8, 16) loads in flight per thread.
hipError_t launch_probe(int copy, const void* src, void* dst, int64_t bytes, int wgs, int unroll, uint32_t* sink,
                        hipStream_t st);
// Grid-barrier probe: gridbar_phases() barriers over wgs resident workgroups in one launch.
int gridbar_phases();
hipError_t launch_gridbar_probe(int* cnt, float* data, int* err, int wgs, hipStream_t st);

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
