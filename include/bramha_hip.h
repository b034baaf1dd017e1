/*
 * bramha_hip.h — C ABI of the MI355X (gfx950) compute backend for Bramha's
 * quantized decode path.
 *
 * Every entry point returns a bh_status (0 = BH_OK). A non-zero status is the
 * Err(String) of the reference's Result: the text is in bh_last_error(), the
 * call had no effect on its outputs, and the caller falls back to its CPU path
 * exactly as cpu_engine.rs:430-446 does on a wgpu error. No entry point aborts
 * the process.
 *
 * Pointer conventions: functions named bh_matvec_* take and return HOST
 * buffers and block until the result is in `out` (like WgpuComputePlane's
 * methods, which submit and poll(Wait)). Everything else takes DEVICE
 * pointers and is ordered on the given HIP stream (NULL = the context's
 * stream); nothing there synchronises unless its name ends in _sync or it
 * returns host data.
 *
 * Threading: one bh_ctx per device. Calls on one context are serialised by a
 * mutex inside the context (the reference guards its registry with a Mutex,
 * wgpu_backend.rs:111). A bh_model is used by one thread at a time.
 */
#ifndef BRAMHA_HIP_H
#define BRAMHA_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    BH_OK = 0,
    BH_ERR_INVALID = -1,      /* bad argument or size mismatch (wgpu_backend.rs:1096-1104) */
    BH_ERR_NO_DEVICE = -2,    /* no usable gfx950 device: the caller stays on CPU (:1722-1725) */
    BH_ERR_HIP = -3,          /* a HIP runtime call failed */
    BH_ERR_OOM = -4,          /* device allocation failed */
    BH_ERR_NOT_FOUND = -5,    /* unknown tensor name / registry key */
    BH_ERR_INJECTED = -6,     /* failure forced by bh_debug_inject_fault */
    BH_ERR_UNSUPPORTED = -7,  /* shape or format the backend does not run */
    BH_ERR_CAPACITY = -8      /* KV rows, slots or batch size exceeded */
} bh_status;

/* Weight formats. Row formats are the reference's (src/models/quantization.rs):
 *   BH_F32     f32 [n][k]
 *   BH_Q8_ROW  int8 [n][k] + f32 scale per row            (quantize_to_int8, :7-38)
 *   BH_Q4_ROW  u8 [n][k/2] + f32 scale per row, nibble+8,  (quantize_to_int4, :41-83)
 *              high nibble = even element
 *   BH_Q4_G32  u8 [n][k/2] (same nibble order) + fp16 scale per 32 elements
 *              [n][k/32]: the block-32 extension used by the 4-bit workloads. */
typedef enum { BH_F32 = 0, BH_Q8_ROW = 1, BH_Q4_ROW = 2, BH_Q4_G32 = 3 } bh_qfmt;

typedef struct bh_ctx bh_ctx;
typedef struct bh_weight bh_weight;
typedef struct bh_model bh_model;

/* ---------------------------------------------------------------- context */

/* Replaces WgpuComputePlane::new (wgpu_backend.rs:121-477) behind get_wgpu_plane's
 * OnceLock (:1707-1728): opens `device`, creates the context's stream and weight
 * registry. Fails with BH_ERR_NO_DEVICE when the device is not gfx950. */
int bh_init(int device, bh_ctx** out);
void bh_destroy(bh_ctx* ctx);
/* Text of the last error on this context ("" if none). Valid until the next call. */
const char* bh_last_error(const bh_ctx* ctx);
/* Text for a status code (for errors that happen before a context exists). */
const char* bh_status_str(int status);
/* The registry's byte cap, replacing ModelBuffers::max_vram_bytes (wgpu_backend.rs:40-56;
 * 3 GB there). Entries are evicted least-recently-used first when it is exceeded. */
int bh_set_vram_cap(bh_ctx* ctx, size_t bytes);
/* Registry contents: number of keyed weights and their total device bytes. */
int bh_registry_stats(bh_ctx* ctx, size_t* n_entries, size_t* bytes);
/* Make the next `count` calls whose op id matches `op` (BH_OP_*, or BH_OP_ANY) fail
 * with `status` and no side effect. count 0 clears. Host-side only: no kernel runs. */
enum { BH_OP_ANY = 0, BH_OP_MATVEC = 1, BH_OP_UPLOAD = 2, BH_OP_GEMV = 3, BH_OP_DECODE = 4 };
int bh_debug_inject_fault(bh_ctx* ctx, int op, int status, int count);

/* ------------------------------------------------------- device memory */
/* Plain device buffers for callers without their own allocator. Copies are blocking
 * and ordered after all work queued on the context's stream. */
int bh_dev_alloc(bh_ctx* ctx, size_t bytes, void** out);
int bh_dev_free(bh_ctx* ctx, void* p);
int bh_memcpy_h2d(bh_ctx* ctx, void* dst, const void* src, size_t bytes);
int bh_memcpy_d2h(bh_ctx* ctx, void* dst, const void* src, size_t bytes);
/* Wait for all work on the device (every stream of this process). */
int bh_synchronize(bh_ctx* ctx);

/* ------------------------------------------- WgpuComputePlane GEMV mirror */
/* y = W h for one host vector h [in_features] -> host out [out_features].
 * With model_name and layer_name both non-NULL the weight is uploaded once and kept
 * in the registry under "model_name:layer_name" (get_or_create_op, wgpu_backend.rs:603-722):
 * later calls with the same key reuse the device copy and ignore the weight argument's
 * contents. Otherwise a temporary copy is uploaded for this call (:1118-1171).
 * in_features == 0 or out_features == 0 returns BH_OK with out zero-filled (:1093-1095). */

/* Replaces WgpuComputePlane::matvec_mul (wgpu_backend.rs:734-741). weight: f32 [out][in]. */
int bh_matvec_mul(bh_ctx* ctx, const float* h, size_t in_features, const float* weight, size_t weight_len,
                  size_t out_features, const char* model_name, const char* layer_name, float* out);
/* Replaces WgpuComputePlane::matvec_mul_int8 (wgpu_backend.rs:906-914). */
int bh_matvec_mul_int8(bh_ctx* ctx, const float* h, size_t in_features, const int8_t* q_weight, size_t q_len,
                       const float* scales, size_t s_len, size_t out_features, const char* model_name,
                       const char* layer_name, float* out);
/* Replaces WgpuComputePlane::matvec_mul_int4 (wgpu_backend.rs:1083-1091). */
int bh_matvec_mul_int4(bh_ctx* ctx, const float* h, size_t in_features, const uint8_t* q_weight, size_t q_len,
                       const float* scales, size_t s_len, size_t out_features, const char* model_name,
                       const char* layer_name, float* out);
/* Replaces WgpuComputePlane::clear_persistent_buffers (wgpu_backend.rs:724-731). */
int bh_clear_persistent_buffers(bh_ctx* ctx);

/* ------------------------------------------------- device-resident weights */
/* Upload a weight given in its reference (row-major) layout from host memory.
 * scales: NULL for BH_F32; f32 [n] for the row formats; fp16 bits [n][k/32] for BH_Q4_G32.
 * The device copy is repacked K-major in 16-byte chunks for row-per-lane GEMV. */
int bh_weight_upload(bh_ctx* ctx, int fmt, int64_t n_out, int64_t k_in, const void* q, size_t q_bytes,
                     const void* scales, size_t s_bytes, bh_weight** out);
void bh_weight_free(bh_ctx* ctx, bh_weight* w);
/* y[b][n] = sum_k W[n][k] x[b][k] for b < batch (device pointers, f32, row-major).
 * Numerically the reference's matvec_mul_into up to f32 summation order. */
int bh_gemv(bh_ctx* ctx, const bh_weight* w, const float* x, float* y, int batch, void* stream);
/* Dequantize to f32 [n][k] on the device: w = (q - 8) * scale, (q) * scale, bit-exact
 * with dequantize_int4 / dequantize_int8 (quantization.rs:86-122). */
int bh_dequant(bh_ctx* ctx, const bh_weight* w, float* out, void* stream);

/* ------------------------------------------------------ single ops (device) */
/* out[r] = x[r] * (1 / sqrt(mean(x[r]^2) + eps)) * w   (rms_norm_into, cpu_engine.rs:1292-1302) */
int bh_rmsnorm(bh_ctx* ctx, const float* x, const float* w, float eps, float* out, int rows, int n, void* stream);
/* Rotate-half RoPE in place on v[rows][n_heads*head_dim] at positions pos[rows] (device int32)
 * (apply_rope_cpu + get_rope_thetas, cpu_engine.rs:1515-1530, 1682-1699). The cos/sin
 * table is computed on the host with the same f32 formulas; pos must be < max_pos. */
int bh_rope(bh_ctx* ctx, float* v, const int32_t* pos, int rows, int n_heads, int head_dim, float theta,
            int max_pos, void* stream);
/* out = g * (1 / (1 + exp(-g))) * u   (cpu_engine.rs:2023-2026) */
int bh_silu_mul(bh_ctx* ctx, const float* g, const float* u, float* out, int64_t n, void* stream);
/* GQA decode attention for `batch` query rows (flash_attention_single_into,
 * cpu_engine.rs:1450-1509). q: f32 [batch][n_q*head_dim]. The packed cache has one region of
 * kv_rows rows per KV head for K and for V, in the layout the device decoder keeps:
 *  - f32 (kv_f16 = 0): row-major, element (row t, dim d) of head h at (h*kv_rows + t)*head_dim + d;
 *  - fp16 (kv_f16 = 1): "MFMA tiles" of 64 rows (head_dim 64) or 32 rows (head_dim 128), each
 *    stored in the order the attention kernel loads its matrix-core operands; element (t, d) of
 *    head h is at h*kv_rows*head_dim + kv_k_off(t, d) for K and + kv_v_off(t, d) for V, where
 *    with TR the tile rows, r = t % TR, base = (t / TR)*TR*head_dim:
 *      kv_k_off = base + ((blk*(head_dim/32) + d/32)*64 + lr + 16*((d%32)/8))*8 + d%8,
 *        blk = 2*(r/32) + (r%8)/4, lr = 4*((r%32)/8) + r%4;
 *      kv_v_off = base + (((r/32)*(head_dim/16) + d/16)*64 + d%16 + 16*((r%32)/8))*8 + r%8;
 *    kv_rows must be a multiple of 64.
 * Row b attends to cache rows [seq_off[b], seq_off[b] + seq_len[b]) (device int64 / int32
 * arrays; the offsets are prefix sums of the sequences' capacities). fp16 offsets that are
 * multiples of 64 take the 1 KiB operand loads, multiples of 8 16-byte loads; f32 offsets and
 * kv_rows that are multiples of 8 take 16-byte loads. max_len bounds seq_len and sizes the
 * split over the context. out: f32 [batch][n_q*head_dim]. */
int bh_attn_decode(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                   const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv, int head_dim,
                   int max_len, float* out, void* stream);

/* bh_attn_decode without any device allocation (no counterpart in the reference: for callers that
 * cannot allocate, e.g. code under HIP graph capture or a serving loop that forbids hipMalloc).
 * Same arguments, kernels and results as bh_attn_decode; the split partials and merge counters live
 * in a fixed scratch array of 2 MiB + 4096 counters that each device holds for the life of the
 * process, shared by every call on that device. A call whose split plan needs more
 * (batch * n_q * splits * (head_dim + 2) * 4 bytes of partials, batch * n_kv counters) fails with
 * BH_ERR_CAPACITY. Calls that overlap on one device (other streams, other contexts) race on the
 * shared scratch: the caller orders them. */
int bh_attn_decode_noalloc(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                           const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv,
                           int head_dim, int max_len, float* out, void* stream);

/* ------------------------------------------------------------ measurement */
/* Measurement helpers (no counterpart in the reference; used by bench.py for the GEMV and
 * attention sweeps). Each replays a HIP graph of `iters` launches on the context's stream whose
 * operands rotate over device copies of the weight (or K/V cache) totalling at least
 * rotate_bytes, so the data streams from HBM rather than the 256 MB Infinity Cache, and returns
 * the mean time per launch in microseconds. The copies are freed before returning. */
int bh_time_gemv(bh_ctx* ctx, const bh_weight* w, const float* x, float* y, int batch, int iters,
                 size_t rotate_bytes, double* us_per_launch);
int bh_time_attn(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                 const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv, int head_dim,
                 int max_len, float* out, int iters, size_t rotate_bytes, double* us_per_launch);

/* HBM bandwidth probe: a graph of `iters` launches that each stream a `bytes` buffer (larger than
 * the 256 MB Infinity Cache, so every launch reads HBM) with 16-byte non-temporal loads (copy = 0),
 * or copy it into a second buffer (copy = 1); wgs workgroups of 256 threads, `unroll` (4, 8 or 16)
 * loads in flight per thread. Returns the mean microseconds per launch; the achievable read (copy)
 * bandwidth is bytes (2 * bytes) / time. copy = 2 times a chain of dependent launches instead:
 * each of its wgs workgroups reads the bytes / 4 floats the previous launch wrote (workgroup 0
 * writes the next), replayed as a graph like the decode step, so the time per launch is the floor
 * of one dependent decode kernel. copy = 3 times grid barriers instead: one launch of wgs (at most
 * the CU count) resident workgroups that run 64 phases of the chain's work, each ended by a barrier
 * over the grid (an arrival count with release ordering polled with acquire loads, every wait
 * bounded); the result is the time per phase, to compare with a dependent launch (bytes and
 * unroll are checked but unused). The buffers are allocated and freed by the call. */
int bh_time_probe(bh_ctx* ctx, int copy, size_t bytes, int wgs, int unroll, int iters, double* us_per_launch);

/* ------------------------------------------------------------ decoder model */
typedef struct {
    int32_t n_layers, hidden, n_heads, n_kv_heads, head_dim, ffn, vocab;
    float rope_theta, rms_eps;
    int32_t attn_bias;     /* q/k/v projections carry a bias (Qwen2) */
    int32_t o_bias;        /* o_proj carries a bias */
    int32_t wfmt;          /* projection format (bh_qfmt) */
    int32_t head_fmt;      /* tied embedding / LM head: BH_F32 or BH_Q4_G32 */
    int32_t max_context;   /* reference sink eviction (cpu_engine.rs:1728-1754): keep at most this many
                              rows per sequence, the first sink_tokens fixed; <= 0 disables */
    int32_t sink_tokens;
    int32_t kv_f16;        /* KV cache element: 1 fp16, 0 f32 */
    int32_t max_seqs;      /* sequence slots */
    int64_t kv_rows;       /* rows in the packed KV buffer shared by all slots */
    int32_t max_tokens;    /* tokens per forward: prefill chunk or decode batch */
} bh_model_config;

/* Replaces generate_cpu_inner_logits's model setup (cpu_engine.rs:2290-2510) for the dense
 * Qwen2/Llama decoder: allocates activations, the KV buffer and the RoPE table. */
int bh_model_create(bh_ctx* ctx, const bh_model_config* cfg, bh_model** out);
void bh_model_destroy(bh_model* m);
/* Upload one tensor by its Hugging Face name from host memory, reference layout:
 * projections in cfg.wfmt (scales as in bh_weight_upload), "model.embed_tokens.weight"
 * in cfg.head_fmt, norms and biases f32. An optional "lm_head.weight" (cfg.head_fmt) unties the
 * LM head; without it the head is the embedding (cpu_engine.rs:2449-2455). */
int bh_model_set_weight(bh_model* m, const char* name, const void* data, size_t bytes, const void* scales,
                        size_t scale_bytes);
/* Load a model directory in the reference's on-disk format (manifest.json + per-layer shards,
 * written by src/bin/quantize_model.rs:284-306 and read by src/storage/tensor_db.rs:623-724):
 * Int4PerChannel layers as {id}_u4.bin + {id}_scale.bin (cfg.wfmt must be BH_Q4_ROW for
 * them), Int8Linear as {id}_i8.bin + {id}_scale.bin (BH_Q8_ROW), uncompressed layers as
 * {id}.bin f32; '.' in ids becomes '_'. Shards are memory-mapped and uploaded with
 * bh_model_set_weight; a non-empty manifest checksum must equal the shard's SHA-256.
 * Tensors the decoder does not use are skipped; *n_loaded counts the uploaded ones. */
int bh_model_load_dir(bh_model* m, const char* dir, int* n_loaded);
/* KV persistence (the prefix cache of src/inference/paged_kv/prefix_cache.rs:37-120 keeps per
 * layer the flat LayerKvCache vectors, cpu_engine.rs:1720-1755): copy rows [row0, row0 + n) of
 * an open slot between the device cache and host f32 arrays k, v [n_layers][n][n_kv*head_dim].
 * kv_read needs row0 + n <= the slot's length; kv_write needs row0 <= the slot's length, the
 * slot outside the decode batch and the rows inside its capacity, and sets its length to
 * row0 + n (a following prefill continues at that position). With eviction on, rows must stay
 * below max_context. fp16 caches convert exactly to f32 and round back on write. */
int bh_model_kv_read(bh_model* m, int slot, int64_t row0, int64_t n, float* k_out, float* v_out);
int bh_model_kv_write(bh_model* m, int slot, int64_t row0, int64_t n, const float* k_in, const float* v_in);
/* Current length (rows = next position) of a slot; 0 when the slot is not open. */
int bh_model_seq_len(bh_model* m, int slot, int64_t* len);
/* Token selection of the decode step (cpu_engine.rs:2984-3031). temperature 0 (the default):
 * greedy first-max argmax of the penalized logits. temperature > 0: the reference's top-k
 * sampling — logits / temperature, softmax, the top_k (1..64; the reference uses 40) most likely
 * ids renormalised, the first id whose cumulative probability reaches a uniform draw r — on the
 * device, with r = bh_sample_uniform(seed, slot, position of the step's input token) instead of
 * the reference's unseeded thread_rng. The repetition penalty and EOS handling are unchanged. */
int bh_model_set_sampling(bh_model* m, float temperature, int top_k, uint64_t seed);
/* The draw used by a sampling step (no counterpart in the reference; for reproducing a run). */
float bh_sample_uniform(uint64_t seed, int slot, int pos);
/* Number of tensors still missing (0 when the model can run). */
int bh_model_missing(bh_model* m, int* n_missing);
/* (Re)start sequence `slot` with room for `capacity` KV rows (capacity <= max_context when
 * eviction is on). Slots take consecutive regions of the packed buffer; a slot reopened with
 * a capacity no larger than before keeps its region. Clears its repetition-penalty counts.
 * A slot of the decode batch may be reopened for a new sequence; its batch entry must then be
 * replaced (bh_model_decode_replace) before the next decode. */
int bh_model_seq_open(bh_model* m, int slot, int64_t capacity);
/* Run prompt tokens [0, n) of `slot` through the model at its next positions without logits
 * (the reference prefills all prompt tokens but the last, cpu_engine.rs:2586-2757). */
int bh_model_prefill(bh_model* m, int slot, const uint32_t* tokens, int n);
/* Prefill several sequences in one pass (no counterpart in the reference, which prefills one
 * prompt at a time, cpu_engine.rs:2586-2757; for ragged batches that refill several entries at
 * once): sequence s is counts[s] tokens of `tokens` (concatenated in order) into slots[s], at
 * that slot's next positions, as bh_model_prefill would run them one by one. Slots must be
 * distinct and open. */
int bh_model_prefill_batch(bh_model* m, int n_seqs, const int32_t* slots, const uint32_t* tokens,
                           const int32_t* counts);
/* Define the decode batch: batch entry b decodes slot slots[b], whose next input token is
 * first_tokens[b]. */
int bh_model_decode_setup(bh_model* m, int batch, const int32_t* slots, const uint32_t* first_tokens);
/* Replace batch entry b by `slot` with next input token `first_token` (ragged refill). When the
 * new slot has the entry's old KV region (the same slot reopened with no larger capacity) the
 * captured decode step is kept; otherwise it is captured again at the next decode. */
int bh_model_decode_replace(bh_model* m, int b, int slot, uint32_t first_token);
/* Run n_steps greedy decode steps over the batch (one token per entry per step: embedding,
 * layers, final norm, LM head, repetition penalty 1.15 over the entry's generated ids,
 * first-max argmax; cpu_engine.rs:2819-3034). ids_out (host, optional): [n_steps][batch].
 * raw_logits (host, optional): [n_steps][batch][vocab] logits before the penalty. Without it the
 * greedy step keeps the logits on chip (per-tile maxima only).
 * Steps are replayed from a captured HIP graph; the call returns when they are done. */
int bh_model_decode(bh_model* m, int n_steps, uint32_t* ids_out, float* raw_logits);
/* The reference's generate loop at temperature 0 for one sequence: open `slot`, prefill
 * prompt[0, n-1), then decode until max_new ids or an EOS id (2, 151645, 151643), which is
 * emitted (cpu_engine.rs:2175-3064). Returns the count in *n_out. raw_logits as above. */
int bh_model_generate(bh_model* m, int slot, const uint32_t* prompt, int n_prompt, int max_new, uint32_t* ids_out,
                      int* n_out, float* raw_logits);
/* Device stream the model's work is ordered on (hipStream_t). */
void* bh_model_stream(bh_model* m);
/* Per-kernel timing of the next `n_steps` eager (un-graphed) decode steps: every kernel of
 * class `kclass` (BH_K_*) is launched with hipExtLaunchKernelGGL, which records a pair of HIP
 * events at the kernel's own start and end on the model's stream. Returns the mean duration in
 * microseconds and the launch count per class. (BH_K_NORM has no launches: the RMSNorm is folded
 * into the projections. BH_K_ATTN_O is the batch-1 decode launch that computes the attention, the
 * O projection and the residual add together; where it runs, BH_K_ATTN and BH_K_GEMV_O do not.)
 * The steps are those of bh_model_decode without raw_logits: the LM head stores raw logits only
 * under top-k sampling. */
enum { BH_K_GEMV_QKV = 0, BH_K_ATTN = 1, BH_K_GEMV_O = 2, BH_K_GEMV_GATEUP = 3, BH_K_GEMV_DOWN = 4,
       BH_K_LM_HEAD = 5, BH_K_NORM = 6, BH_K_OTHER = 7, BH_K_ATTN_O = 8, BH_K_COUNT = 9 };
int bh_model_time_kernels(bh_model* m, int n_steps, double* mean_us /*[BH_K_COUNT]*/,
                          int64_t* launches /*[BH_K_COUNT]*/);
/* Algorithmic HBM bytes one launch of kernel class `kclass` reads and writes at the
 * current batch (weights, scales, activations; for attention the K/V rows at the current
 * lengths). */
int bh_model_kernel_bytes(bh_model* m, int kclass, double* bytes);

/* ------------------------------------------------ host utilities (no device) */
/* Deterministic synthetic data: element i of the stream named `name` under `seed`
 * (SplitMix64 on seed ^ FNV-1a(name), Box-Muller in f64, rounded to f32). */
int bh_synth_normal(uint64_t seed, const char* name, float sigma, int64_t n, float* out);
/* Token ids uniform in [0, vocab). */
int bh_synth_tokens(uint64_t seed, const char* name, int64_t n, uint32_t vocab, uint32_t* out);
/* Host quantizer into a reference format (bit-identical to the reference quantizers for
 * BH_Q8_ROW / BH_Q4_ROW). q: int8 [n][k] or u8 [n][k/2]; scales f32 [n] or fp16 [n][k/32]. */
int bh_quantize(int fmt, const float* w, int64_t n, int64_t k, void* q, void* scales);

#ifdef __cplusplus
}
#endif

#endif /* BRAMHA_HIP_H */
