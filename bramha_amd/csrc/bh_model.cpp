// bh_model.cpp — the dense Qwen2/Llama decoder on the device: weights, the packed
// KV cache, prefill, and graph-replayed greedy decode steps.
//
// Reference: generate_cpu_inner_logits (src/inference/cpu_engine.rs:2290-3064) with
// CPU-only mode and temperature 0. One forward pass over M tokens is 5 kernels per layer:
//   QKV GEMV (RMSNorm factor, bias, RoPE, KV append) -> attention ->
//   O GEMV (+bias, residual add, next norm's inputs) -> gate/up GEMV (norm factor, SiLU gate) ->
//   down GEMV (residual add, next norm's inputs)
// then, when decoding, the LM head (final norm factor, logits, repetition penalty, per-tile
// argmax) and the sample kernel (argmax, penalty count, next token and position, and the
// next step's embedding row). The residual stream between kernels is x, xw = x * (next norm
// weight) and per-64-element sums of squares, so no kernel runs the RMSNorm on its own.
// Sequences own consecutive regions of one packed KV buffer per layer (offsets are prefix
// sums of the regions' capacities); a decode step reads its token and position from the
// previous step's sample kernel, so the whole step is captured once as a HIP graph and replayed.
#include <algorithm>
#include <cstring>
#include <vector>

#include "bh_ctx.h"

using namespace bh;

namespace {

enum Tensor { T_LN1, T_LN2, T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN, T_BQ, T_BK, T_BV, T_BO, T_COUNT };

struct LayerW {
    DevWeight qkv, o, gate, up, down;
    float* ln1 = nullptr;
    float* ln2 = nullptr;
    float* bqkv = nullptr;
    float* bo = nullptr;
    uint32_t have = 0;
};

struct TimerRec {
    int cls;
    LaunchEvents ev;
};

}  // namespace

struct bh_model {
    bh_ctx* ctx = nullptr;
    bh_model_config c{};
    hipStream_t st = nullptr;
    int64_t QD = 0, KD = 0, NQKV = 0;
    int tiles_lm = 0;
    std::vector<LayerW> L;
    DevWeight embed;
    bool have_embed = false;
    DevWeight lm_head;  // untied LM head ("lm_head.weight"); the embedding when absent
    bool have_lm_head = false;
    float* norm = nullptr;
    bool have_norm = false;

    std::vector<void*> kc, vc;
    int ssq_tiles = 0;             // 64-element tiles of the hidden size
    // residual stream [max_tokens][hidden]: x, xw = x * next norm weight, ssq per tile
    float *x = nullptr, *xw = nullptr, *ssq = nullptr;
    float *q = nullptr, *att = nullptr, *mm = nullptr, *logits = nullptr;
    float* part_val = nullptr;
    int32_t* part_idx = nullptr;
    float* attn_part = nullptr;
    int max_splits = 128;
    int32_t* attn_cnt = nullptr;   // [max_tokens][n_kv] split-merge counters
    size_t attn_rows = 0;          // query rows of attn_part
    float* split_part = nullptr;   // K-split sums of split projections
    uint16_t* xhl = nullptr;       // prefill passes: activations split into fp16 hi + lo
    uint16_t* xw_hl = nullptr;     // decode: final-norm activations split for the batched LM head
    // Batch-1 passes: limb records (k_xl.h) of xw, written by every producer of the residual
    // stream, and of the SwiGLU product mm, written by gate/up; read by the group-32 GEMVs.
    uint32_t *xl_h = nullptr, *xl_f = nullptr;
    int32_t* split_cnt = nullptr;  // their per-tile arrival counters (zero when idle)
    // decode batch state (read by the captured graph) and prefill staging, kept apart so a
    // prefill between decode calls leaves the batch intact
    int32_t *d_tok = nullptr, *d_pos = nullptr, *d_slot = nullptr, *d_step = nullptr;
    int64_t* d_boff = nullptr;
    int32_t *d_ptok = nullptr, *d_ppos = nullptr, *d_pslot = nullptr;
    int64_t* d_pboff = nullptr;
    uint32_t* d_ids = nullptr;
    int64_t ids_steps = 1024;
    uint16_t* d_pen = nullptr;
    const float2* rope = nullptr;
    int max_pos = 0;
    int kv_align = 8;  // rows: every sequence region starts on a multiple
    float temperature = 0.f;  // > 0: top-k sampling instead of greedy argmax
    int top_k = 40;
    uint64_t seed = 0;
    void* h_stage = nullptr;  // pinned staging for small host->device copies

    std::vector<int64_t> off_h, cap_h;
    std::vector<int32_t> len_h;
    std::vector<char> open_h;
    int64_t next_free = 0;

    int B = 0;
    std::vector<int32_t> bslots;
    std::vector<char> stale;       // entry's slot was reopened: it must be replaced before a decode
    hipGraph_t graph = nullptr;
    hipGraphExec_t gexec = nullptr;
    int g_B = 0, g_splits = 0, g_rows = 0;
    bool store_logits = false;  // the next forward stores raw logits
    bool g_logits = false;      // the captured step stores raw logits
    std::vector<int64_t> g_off;    // region offsets the captured step holds as launch arguments
    int64_t g_cap = 0;             // and the smallest region capacity it assumes

    bool timing = false;
    std::vector<TimerRec> recs;
    std::vector<LaunchEvents> ev_pool;
    size_t ev_used = 0;

    std::vector<void*> allocs;  // device buffers owned by the model

    int fail(int s, const std::string& m) { return ctx->fail(s, m); }
};

namespace {

hipError_t dmalloc(bh_model* m, void** p, size_t bytes) {
    *p = nullptr;
    hipError_t e = hipMalloc(p, std::max<size_t>(bytes, 16));
    if (e == hipSuccess) {
        m->allocs.push_back(*p);
        e = hipMemset(*p, 0, std::max<size_t>(bytes, 16));
    }
    return e;
}

LaunchEvents* next_events(bh_model* m) {
    if (m->ev_used == m->ev_pool.size()) {
        LaunchEvents ev;
        hipEventCreate(&ev.start);
        hipEventCreate(&ev.stop);
        m->ev_pool.push_back(ev);
    }
    return &m->ev_pool[m->ev_used++];
}

// Runs one launcher; in timing mode its kernel records a pair of events at its own start and end.
template <class F>
hipError_t timed(bh_model* m, int cls, F&& f) {
    if (!m->timing) return f();
    LaunchEvents* ev = next_events(m);
    launch_events = ev;
    hipError_t e = f();
    launch_events = nullptr;
    m->recs.push_back({cls, *ev});
    return e;
}

KvView kv_view(bh_model* m, int l) {
    KvView v;
    v.k = m->kc[l];
    v.v = m->vc[l];
    v.kv_rows = m->c.kv_rows;
    v.kv_f16 = m->c.kv_f16;
    v.max_context = m->c.max_context > 0 ? m->c.max_context : 0;
    v.sink = m->c.sink_tokens;
    return v;
}

// Consumer side of the residual stream: activations xw, per-token norm factor from ssq.
void stream_input(bh_model* m, GemvArgs& a) {
    a.x = m->xw;
    a.ldx = m->c.hidden;
    a.ssq_in = m->ssq;
    a.ssq_tiles = m->ssq_tiles;
    a.norm_n = (float)m->c.hidden;
    a.eps = m->c.rms_eps;
}

// Producer side: residual add into x, xw with the next norm's weight, ssq.
void stream_output(bh_model* m, GemvArgs& a, const float* wnext) {
    a.y = m->x;
    a.ldy = m->c.hidden;
    a.xw_out = m->xw;
    a.wnext = wnext;
    a.ssq_out = m->ssq;
    a.ssq_tiles = m->ssq_tiles;
}

// Weight operands; the launcher chooses the K split (ksw 0) and may use the model's split scratch.
void weight_args(bh_model* m, GemvArgs& a, const DevWeight& w) {
    a.W = w.q;
    a.S = w.s;
    a.N = (int)w.n;
    a.n_pad = (int)w.n_pad;
    a.C = (int)w.chunks;
    a.ksw = 0;
    a.part = m->split_part;
    a.tile_cnt = m->split_cnt;
    a.xhl = m->xhl;
}

// Whether the last down projection of a decode step over M tokens also stores the final-norm
// activations split into fp16 hi + lo for the LM head: every pass of M (launch_gemv) is then an
// MFMA pass on both sides (4-bit weights, 9..32 tokens; a remainder of at most 8 tokens takes
// the VALU passes on both sides, which neither store nor read the split).
static bool lm_presplit(const bh_model* m, int M) {
    const bh_model_config& c = m->c;
    return m->xw_hl && M > 8 && M < PF_MIN_TOKENS && c.head_fmt == BH_Q4_G32 && c.hidden % 32 == 0 &&
           (c.wfmt == BH_Q4_G32 || c.wfmt == BH_Q4_ROW);
}

// One forward pass over M tokens whose residual stream (x, xw, ssq) holds their embedding rows:
// the decode batch (decode = true: logits, penalty, argmax and the next step's stream) or a
// staged prefill chunk.
// Whether a pass over M tokens carries limb records (k_xl.h) from the producers to the batch-1
// group-32 GEMVs; the stream's start (launch_embed, k_sample) writes them under the same rule.
static bool use_xl(const bh_model* m, int M) {
    return M == 1 && (m->c.wfmt == BH_Q4_G32 || m->c.head_fmt == BH_Q4_G32);
}

hipError_t forward(bh_model* m, int M, bool decode, int splits, int split_rows) {
    const bh_model_config& c = m->c;
    const int H = c.hidden, I = c.ffn;
    hipStream_t st = m->st;
    const bool xl = use_xl(m, M);
    int32_t* pos = decode ? m->d_pos : m->d_ppos;
    int32_t* slot = decode ? m->d_slot : m->d_pslot;
    int64_t* boff = decode ? m->d_boff : m->d_pboff;
    hipError_t e = hipSuccess;
    for (int l = 0; l < c.n_layers && e == hipSuccess; ++l) {
        LayerW& w = m->L[l];
        GemvArgs a;
        weight_args(m, a, w.qkv);
        stream_input(m, a);
        a.y = m->q;
        a.ldy = m->QD;
        a.bias = c.attn_bias ? w.bqkv : nullptr;
        a.batch = M;
        a.qd = (int)m->QD;
        a.kd = (int)m->KD;
        a.hd = c.head_dim;
        a.pos = pos;
        a.boff = boff;
        a.rope = m->rope;
        a.kv = kv_view(m, l);
        if (xl) a.xl = m->xl_h;
        e = timed(m, BH_K_GEMV_QKV, [&] { return launch_gemv(c.wfmt, EPI_QKV, a, st); });
        if (e != hipSuccess) break;
        AttnArgs at;
        at.q = m->q;
        at.out = m->att;
        at.kv = kv_view(m, l);
        at.pos = pos;
        at.boff = boff;
        at.batch = M;
        at.nq = c.n_heads;
        at.nkv = c.n_kv_heads;
        at.hd = c.head_dim;
        at.splits = splits;
        at.split_rows = split_rows;
        at.part_o = m->attn_part;
        at.part_ml = m->attn_part + m->attn_rows * c.n_heads * m->max_splits * c.head_dim;
        at.cnt = m->attn_cnt;
        at.prefill = decode ? 0 : 1;
        if (decode && c.kv_f16 && M <= ATTN_STATIC_B) {
            at.static_off = 1;
            at.cap_rows = INT64_MAX;
            for (int b = 0; b < M; ++b) {
                at.off_val[b] = m->off_h[m->bslots[b]];
                at.cap_rows = std::min<int64_t>(at.cap_rows, m->cap_h[m->bslots[b]]);
            }
        }
        GemvArgs o;
        weight_args(m, o, w.o);
        o.x = m->att;
        o.ldx = m->QD;
        o.bias = c.o_bias ? w.bo : nullptr;
        o.batch = M;
        stream_output(m, o, w.ln2);
        if (xl) o.xl_out = m->xl_h;
        if (decode && M == 1 && attn_o_fusable(c.wfmt, at, o)) {
            // batch 1, short context: attention, O projection and residual add in one launch
            e = timed(m, BH_K_ATTN_O, [&] { return launch_attn_o(c.wfmt, at, o, st); });
            if (e != hipSuccess) break;
        } else {
            e = timed(m, BH_K_ATTN, [&] { return launch_attention(at, st); });
            if (e != hipSuccess) break;
            e = timed(m, BH_K_GEMV_O, [&] { return launch_gemv(c.wfmt, EPI_RESNORM, o, st); });
            if (e != hipSuccess) break;
        }
        GemvArgs gu;
        weight_args(m, gu, w.gate);
        gu.W2 = w.up.q;
        gu.S2 = w.up.s;
        stream_input(m, gu);
        gu.y = m->mm;
        gu.ldy = I;
        gu.batch = M;
        if (xl) {
            gu.xl = m->xl_h;
            gu.xl_out = m->xl_f;
        }
        e = timed(m, BH_K_GEMV_GATEUP, [&] { return launch_gemv(c.wfmt, EPI_SILU, gu, st); });
        if (e != hipSuccess) break;
        GemvArgs d;
        weight_args(m, d, w.down);
        d.x = m->mm;
        d.ldx = I;
        d.batch = M;
        stream_output(m, d, l + 1 < c.n_layers ? m->L[l + 1].ln1 : m->norm);  // final norm after the last layer
        if (xl) {
            d.xl = m->xl_f;
            d.xl_out = m->xl_h;
        }
        if (decode && l + 1 == c.n_layers && lm_presplit(m, M)) d.xw_hl = m->xw_hl;
        e = timed(m, BH_K_GEMV_DOWN, [&] { return launch_gemv(c.wfmt, EPI_RESNORM, d, st); });
    }
    if (e != hipSuccess || !decode) return e;
    GemvArgs lm;
    weight_args(m, lm, m->have_lm_head ? m->lm_head : m->embed);
    stream_input(m, lm);
    // raw logits are stored only for a caller that asked for them and for top-k sampling, which
    // reads them; the greedy step needs only the per-tile partials
    lm.y = (m->store_logits || m->temperature > 0.f) ? m->logits : nullptr;
    lm.ldy = c.vocab;
    lm.batch = M;
    lm.pen = m->d_pen;
    lm.n_slots = c.max_seqs;
    if (lm_presplit(m, M)) lm.x_hl = m->xw_hl;
    if (xl) lm.xl = m->xl_h;
    lm.vocab = c.vocab;
    lm.slot = slot;
    lm.part_val = m->part_val;
    lm.part_idx = m->part_idx;
    e = timed(m, BH_K_LM_HEAD, [&] { return launch_gemv(c.head_fmt, EPI_LMHEAD, lm, st); });
    if (e != hipSuccess) return e;
    SampleArgs sa;
    sa.temperature = m->temperature;
    sa.top_k = m->top_k;
    sa.seed = m->seed;
    sa.logits = m->logits;
    sa.part_val = m->part_val;
    sa.part_idx = m->part_idx;
    sa.tiles = m->tiles_lm;
    sa.batch = M;
    sa.vocab = c.vocab;
    sa.slot = slot;
    sa.pen = m->d_pen;
    sa.ids_cap = m->d_ids;
    sa.step = m->d_step;
    sa.tok = m->d_tok;
    sa.pos = m->d_pos;
    sa.table = &m->embed;
    sa.w0 = m->L[0].ln1;
    sa.x = m->x;
    sa.xw = m->xw;
    sa.ssq = m->ssq;
    sa.ssq_tiles = m->ssq_tiles;
    if (xl) sa.xl = m->xl_h;
    return timed(m, BH_K_OTHER, [&] { return launch_sample(sa, st); });
}

// Start the decode batch's residual stream from its current tokens and zero the id counters.
hipError_t decode_start(bh_model* m) {
    return timed(m, BH_K_OTHER, [&] {
        return launch_embed(m->embed, m->d_tok, m->L[0].ln1, m->x, m->xw, m->ssq, m->ssq_tiles, m->d_step, m->B,
                            m->st, use_xl(m, m->B) ? m->xl_h : nullptr);
    });
}

int64_t layer_tensor_count(const bh_model_config& c) { return 9 + (c.attn_bias ? 3 : 0) + (c.o_bias ? 1 : 0); }

bool parse_layer(const char* name, int* l, const char** rest) {
    if (std::strncmp(name, "model.layers.", 13) != 0) return false;
    const char* p = name + 13;
    if (*p < '0' || *p > '9') return false;
    int v = 0;
    while (*p >= '0' && *p <= '9') v = v * 10 + (*p++ - '0');
    if (*p != '.') return false;
    *l = v;
    *rest = p + 1;
    return true;
}

int set_vec(bh_model* m, float** dst, int64_t n, const void* data, size_t bytes, const char* name) {
    if (bytes != (size_t)n * 4 || !data)
        return m->fail(BH_ERR_INVALID, std::string(name) + ": expected " + std::to_string(n * 4) + " bytes, got " +
                                           std::to_string(bytes));
    if (!*dst) {
        hipError_t e = dmalloc(m, (void**)dst, (size_t)n * 4);
        if (e != hipSuccess) return m->ctx->hip_fail(e, "hipMalloc(vector)");
    }
    hipError_t e = hipMemcpy(*dst, data, (size_t)n * 4, hipMemcpyHostToDevice);
    return e == hipSuccess ? BH_OK : m->ctx->hip_fail(e, "hipMemcpy(vector)");
}

int set_bias_part(bh_model* m, LayerW& w, int64_t off, int64_t n, const void* data, size_t bytes, const char* name) {
    if (bytes != (size_t)n * 4 || !data)
        return m->fail(BH_ERR_INVALID, std::string(name) + ": expected " + std::to_string(n * 4) + " bytes");
    if (!w.bqkv) {
        hipError_t e = dmalloc(m, (void**)&w.bqkv, (size_t)m->NQKV * 4);
        if (e != hipSuccess) return m->ctx->hip_fail(e, "hipMalloc(bias)");
    }
    hipError_t e = hipMemcpy(w.bqkv + off, data, (size_t)n * 4, hipMemcpyHostToDevice);
    return e == hipSuccess ? BH_OK : m->ctx->hip_fail(e, "hipMemcpy(bias)");
}

int ensure_weight(bh_model* m, DevWeight& w, int fmt, int64_t n, int64_t k) {
    if (w.q) return BH_OK;
    return alloc_weight(m->ctx, fmt, n, k, w);
}

void drop_graph(bh_model* m) {
    if (m->gexec) hipGraphExecDestroy(m->gexec);
    if (m->graph) hipGraphDestroy(m->graph);
    m->gexec = nullptr;
    m->graph = nullptr;
    m->g_B = m->g_splits = m->g_rows = 0;
    m->g_off.clear();
    m->g_cap = 0;
}

// Largest attention length the next n_steps decode steps of the batch can reach.
int decode_len_bound(bh_model* m, int n_steps) {
    int64_t mx = 1;
    for (int b = 0; b < m->B; ++b) {
        const int s = m->bslots[b];
        int64_t len = m->len_h[s] + n_steps;
        if (m->c.max_context > 0) len = std::min<int64_t>(len, m->c.max_context);
        mx = std::max(mx, len);
    }
    return (int)mx;
}

int check_decode_room(bh_model* m, int n_steps) {
    for (int b = 0; b < m->B; ++b) {
        const int s = m->bslots[b];
        if (!m->open_h[s]) return m->fail(BH_ERR_INVALID, "decode batch holds a slot that is not open");
        if (m->stale[b])
            return m->fail(BH_ERR_INVALID, "the slot of batch entry " + std::to_string(b) +
                                               " was reopened: replace the entry (bh_model_decode_replace) first");
        const int64_t end = m->len_h[s] + n_steps;
        if (end > m->max_pos) return m->fail(BH_ERR_CAPACITY, "position beyond the RoPE table");
        if (m->c.max_context <= 0 && end > m->cap_h[s])
            return m->fail(BH_ERR_CAPACITY, "slot " + std::to_string(s) + " needs " + std::to_string(end) +
                                                " KV rows, has " + std::to_string(m->cap_h[s]));
    }
    return BH_OK;
}

// Host -> device copy of a few bytes through the pinned staging buffer, completed before return.
hipError_t put(bh_model* m, void* dst, const void* src, size_t bytes) {
    std::memcpy(m->h_stage, src, bytes);
    hipError_t e = hipMemcpyAsync(dst, m->h_stage, bytes, hipMemcpyHostToDevice, m->st);
    return e == hipSuccess ? hipStreamSynchronize(m->st) : e;
}

}  // namespace

extern "C" {

int bh_model_create(bh_ctx* ctx, const bh_model_config* cfg, bh_model** out) {
    if (!ctx || !cfg || !out) return BH_ERR_INVALID;
    *out = nullptr;
    const bh_model_config& c = *cfg;
    if (c.n_layers <= 0 || c.hidden <= 0 || c.n_heads <= 0 || c.n_kv_heads <= 0 || c.ffn <= 0 || c.vocab <= 0 ||
        c.n_heads % c.n_kv_heads || c.max_seqs <= 0 || c.kv_rows <= 0 || c.max_tokens <= 0)
        return ctx->fail(BH_ERR_INVALID, "invalid model config");
    if (!attn_supported(c.n_heads, c.n_kv_heads, c.head_dim))
        return ctx->fail(BH_ERR_UNSUPPORTED, "head_dim must be 64 or 128 with 1, 2, 4, 7 or 8 query heads per KV head");
    if (c.head_fmt != BH_F32 && c.head_fmt != BH_Q4_G32)
        return ctx->fail(BH_ERR_UNSUPPORTED, "tied embedding format must be F32 or Q4_G32");
    if (c.wfmt < BH_F32 || c.wfmt > BH_Q4_G32) return ctx->fail(BH_ERR_INVALID, "unknown weight format");
    const int E = chunk_elems(c.wfmt);
    const int64_t QD = (int64_t)c.n_heads * c.head_dim, KD = (int64_t)c.n_kv_heads * c.head_dim;
    if (c.hidden % E || QD % E || c.ffn % E || c.hidden % chunk_elems(c.head_fmt))
        return ctx->fail(BH_ERR_UNSUPPORTED, "hidden, q_dim and ffn must be multiples of the 16-byte chunk");
    if (c.hidden % 64)
        return ctx->fail(BH_ERR_UNSUPPORTED, "hidden must be a multiple of 64 (residual-stream tiles)");
    if (c.max_context > 0 && (c.sink_tokens < 0 || c.sink_tokens >= c.max_context))
        return ctx->fail(BH_ERR_INVALID, "sink_tokens must be below max_context");
    if (c.max_tokens > 4096) return ctx->fail(BH_ERR_UNSUPPORTED, "max_tokens above 4096");

    std::lock_guard<std::mutex> g(ctx->mu);
    bh_model* m = new bh_model();
    m->ctx = ctx;
    m->c = c;
    // Sequence regions start on KV_ALIGN-row boundaries (fp16: whole MFMA tiles, f32: 16-byte
    // loads); room for every slot's rounding is added so that capacities summing to kv_rows fit.
    m->kv_align = c.kv_f16 ? 64 : 8;
    m->c.kv_rows = (c.kv_rows + m->kv_align - 1) / m->kv_align * m->kv_align + (int64_t)m->kv_align * c.max_seqs;
    m->QD = QD;
    m->KD = KD;
    m->NQKV = QD + 2 * KD;
    m->L.resize(c.n_layers);
    m->max_pos = (int)std::max<int64_t>(65536, c.kv_rows + 1);
    m->tiles_lm = (int)(pad64(c.vocab) / 64);
    m->ssq_tiles = c.hidden / 64;
    auto bail = [&](hipError_t e, const char* what) {
        int rc = ctx->hip_fail(e, what);
        bh_model_destroy(m);
        return rc;
    };
    hipError_t e = hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking);
    if (e != hipSuccess) return bail(e, "hipStreamCreate");
    const size_t kvb = (size_t)m->c.kv_rows * KD * (c.kv_f16 ? 2 : 4);
    m->kc.assign(c.n_layers, nullptr);
    m->vc.assign(c.n_layers, nullptr);
    for (int l = 0; l < c.n_layers; ++l) {
        if ((e = dmalloc(m, &m->kc[l], kvb)) != hipSuccess) return bail(e, "hipMalloc(K cache)");
        if ((e = dmalloc(m, &m->vc[l], kvb)) != hipSuccess) return bail(e, "hipMalloc(V cache)");
    }
    const size_t T = (size_t)c.max_tokens;
    // decode-only buffers hold one row per batch entry (at most one entry per slot); the split
    // partials also serve f32-cache prefill chunks (one query per token)
    const size_t DB = std::min<size_t>(T, (size_t)c.max_seqs);
    m->attn_rows = c.kv_f16 ? DB : T;
    struct {
        void** p;
        size_t bytes;
    } bufs[] = {
        {(void**)&m->x, T * c.hidden * 4},
        {(void**)&m->xw, T * c.hidden * 4},
        {(void**)&m->ssq, T * m->ssq_tiles * 4},
        {(void**)&m->q, T * QD * 4},
        {(void**)&m->att, T * QD * 4},
        {(void**)&m->mm, T * c.ffn * 4},
        {(void**)&m->logits, DB * c.vocab * 4},
        {(void**)&m->part_val, DB * m->tiles_lm * 4},
        {(void**)&m->part_idx, DB * m->tiles_lm * 4},
        {(void**)&m->attn_part, m->attn_rows * c.n_heads * m->max_splits * (c.head_dim + 2) * 4},
        {(void**)&m->attn_cnt, T * c.n_kv_heads * 4},
        {(void**)&m->split_part, (size_t)SPLIT_PART_FLOATS * 4},
        {(void**)&m->split_cnt, (size_t)SPLIT_TILES_MAX * 4},
        {(void**)&m->d_tok, T * 4},
        {(void**)&m->d_pos, T * 4},
        {(void**)&m->d_slot, T * 4},
        {(void**)&m->d_step, T * 4},
        {(void**)&m->d_boff, T * 8},
        {(void**)&m->d_ptok, T * 4},
        {(void**)&m->d_ppos, T * 4},
        {(void**)&m->d_pslot, T * 4},
        {(void**)&m->d_pboff, T * 8},
        {(void**)&m->d_ids, (size_t)m->ids_steps * DB * 4},
        {(void**)&m->d_pen, (size_t)c.max_seqs * c.vocab * 2},
        {(void**)&m->xw_hl, DB * c.hidden * 4},
        {(void**)&m->xl_h, (size_t)(c.hidden + 31) / 32 * (XL_REC_BYTES + 4)},
        {(void**)&m->xl_f, (size_t)(c.ffn + 31) / 32 * (XL_REC_BYTES + 4)},
    };
    for (auto& b : bufs)
        if ((e = dmalloc(m, b.p, b.bytes)) != hipSuccess) return bail(e, "hipMalloc(activations)");
    if (T >= (size_t)PF_MIN_TOKENS) {  // passes that reach the tiled prefill GEMM
        const size_t kmax = std::max<size_t>({(size_t)c.hidden, (size_t)QD, (size_t)c.ffn});
        if ((e = dmalloc(m, (void**)&m->xhl, T * kmax * 4)) != hipSuccess) return bail(e, "hipMalloc(activation split)");
    }
    e = hipHostMalloc(&m->h_stage, (4 * T + 16) * 8, hipHostMallocDefault);
    if (e != hipSuccess) {
        m->h_stage = nullptr;
        return bail(e, "hipHostMalloc");
    }
    m->rope = ctx->rope_tab(c.head_dim, c.rope_theta, m->max_pos);
    if (!m->rope) return bail(hipErrorOutOfMemory, "rope table");
    m->off_h.assign(c.max_seqs, -1);
    m->cap_h.assign(c.max_seqs, 0);
    m->len_h.assign(c.max_seqs, 0);
    m->open_h.assign(c.max_seqs, 0);
    *out = m;
    return BH_OK;
}

void bh_model_destroy(bh_model* m) {
    if (!m) return;
    if (m->st) hipStreamSynchronize(m->st);
    drop_graph(m);
    for (auto& w : m->L) {
        free_weight(w.qkv);
        free_weight(w.o);
        free_weight(w.gate);
        free_weight(w.up);
        free_weight(w.down);
    }
    free_weight(m->embed);
    free_weight(m->lm_head);
    for (void* p : m->allocs) hipFree(p);
    for (auto& ev : m->ev_pool) {
        hipEventDestroy(ev.start);
        hipEventDestroy(ev.stop);
    }
    if (m->h_stage) hipHostFree(m->h_stage);
    if (m->st) hipStreamDestroy(m->st);
    delete m;
}

void* bh_model_stream(bh_model* m) { return m ? (void*)m->st : nullptr; }

int bh_model_set_weight(bh_model* m, const char* name, const void* data, size_t bytes, const void* scales,
                        size_t scale_bytes) {
    if (!m || !name) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    const bh_model_config& c = m->c;
    const int64_t H = c.hidden, I = c.ffn;
    if (!std::strcmp(name, "model.embed_tokens.weight")) {
        int rc = ensure_weight(m, m->embed, c.head_fmt, c.vocab, H);
        if (!rc) rc = upload_rows(m->ctx, m->embed, 0, c.vocab, data, bytes, scales, scale_bytes);
        if (!rc) m->have_embed = true;
        return rc;
    }
    if (!std::strcmp(name, "lm_head.weight")) {  // optional: cpu_engine.rs:2449-2451 falls back to the embedding
        int rc = ensure_weight(m, m->lm_head, c.head_fmt, c.vocab, H);
        if (!rc) rc = upload_rows(m->ctx, m->lm_head, 0, c.vocab, data, bytes, scales, scale_bytes);
        if (!rc) m->have_lm_head = true;
        return rc;
    }
    if (!std::strcmp(name, "model.norm.weight")) {
        int rc = set_vec(m, &m->norm, H, data, bytes, name);
        if (!rc) m->have_norm = true;
        return rc;
    }
    int l;
    const char* r;
    if (!parse_layer(name, &l, &r) || l < 0 || l >= c.n_layers)
        return m->fail(BH_ERR_NOT_FOUND, std::string("unknown tensor ") + name);
    LayerW& w = m->L[l];
    int rc = BH_ERR_NOT_FOUND, t = -1;
    if (!std::strcmp(r, "input_layernorm.weight")) { t = T_LN1; rc = set_vec(m, &w.ln1, H, data, bytes, name); }
    else if (!std::strcmp(r, "post_attention_layernorm.weight")) { t = T_LN2; rc = set_vec(m, &w.ln2, H, data, bytes, name); }
    else if (!std::strcmp(r, "self_attn.q_proj.weight") || !std::strcmp(r, "self_attn.k_proj.weight") ||
             !std::strcmp(r, "self_attn.v_proj.weight")) {
        const int which = r[10] == 'q' ? 0 : (r[10] == 'k' ? 1 : 2);
        t = T_Q + which;
        const int64_t row0 = which == 0 ? 0 : (which == 1 ? m->QD : m->QD + m->KD);
        const int64_t n = which == 0 ? m->QD : m->KD;
        rc = ensure_weight(m, w.qkv, c.wfmt, m->NQKV, H);
        if (!rc) rc = upload_rows(m->ctx, w.qkv, row0, n, data, bytes, scales, scale_bytes);
    } else if (!std::strcmp(r, "self_attn.o_proj.weight")) {
        t = T_O;
        rc = ensure_weight(m, w.o, c.wfmt, H, m->QD);
        if (!rc) rc = upload_rows(m->ctx, w.o, 0, H, data, bytes, scales, scale_bytes);
    } else if (!std::strcmp(r, "mlp.gate_proj.weight")) {
        t = T_GATE;
        rc = ensure_weight(m, w.gate, c.wfmt, I, H);
        if (!rc) rc = upload_rows(m->ctx, w.gate, 0, I, data, bytes, scales, scale_bytes);
    } else if (!std::strcmp(r, "mlp.up_proj.weight")) {
        t = T_UP;
        rc = ensure_weight(m, w.up, c.wfmt, I, H);
        if (!rc) rc = upload_rows(m->ctx, w.up, 0, I, data, bytes, scales, scale_bytes);
    } else if (!std::strcmp(r, "mlp.down_proj.weight")) {
        t = T_DOWN;
        rc = ensure_weight(m, w.down, c.wfmt, H, I);
        if (!rc) rc = upload_rows(m->ctx, w.down, 0, H, data, bytes, scales, scale_bytes);
    } else if (!std::strcmp(r, "self_attn.q_proj.bias")) { t = T_BQ; rc = set_bias_part(m, w, 0, m->QD, data, bytes, name); }
    else if (!std::strcmp(r, "self_attn.k_proj.bias")) { t = T_BK; rc = set_bias_part(m, w, m->QD, m->KD, data, bytes, name); }
    else if (!std::strcmp(r, "self_attn.v_proj.bias")) { t = T_BV; rc = set_bias_part(m, w, m->QD + m->KD, m->KD, data, bytes, name); }
    else if (!std::strcmp(r, "self_attn.o_proj.bias")) { t = T_BO; rc = set_vec(m, &w.bo, H, data, bytes, name); }
    else return m->fail(BH_ERR_NOT_FOUND, std::string("unknown tensor ") + name);
    if (rc == BH_OK) w.have |= 1u << t;
    return rc;
}

const char* model_last_error(bh_model* m) { return m->ctx->err.c_str(); }
int model_load_dir(bh_model* m, const char* dir, int* n_loaded, std::string* err);  // bh_loader.cpp

int bh_model_load_dir(bh_model* m, const char* dir, int* n_loaded) {
    if (!m || !dir || !n_loaded) return BH_ERR_INVALID;
    std::string err;
    const int rc = model_load_dir(m, dir, n_loaded, &err);
    if (rc != BH_OK) {
        std::lock_guard<std::mutex> g(m->ctx->mu);
        return m->fail(rc, err);
    }
    return BH_OK;
}

int bh_model_set_sampling(bh_model* m, float temperature, int top_k, uint64_t seed) {
    if (!m || !(temperature >= 0.f) || (temperature > 0.f && (top_k < 1 || top_k > SAMPLE_TOPK_MAX)))
        return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    if (temperature > 0.f && m->tiles_lm > 4096)
        return m->fail(BH_ERR_UNSUPPORTED, "sampling supports vocabularies up to 262144");
    m->temperature = temperature;
    m->top_k = top_k;
    m->seed = seed;
    drop_graph(m);  // the captured step holds the old sampling arguments
    return BH_OK;
}

int bh_model_missing(bh_model* m, int* n_missing) {
    if (!m || !n_missing) return BH_ERR_INVALID;
    int miss = (m->have_embed ? 0 : 1) + (m->have_norm ? 0 : 1);
    for (auto& w : m->L) {
        uint32_t need = (1u << T_LN1) | (1u << T_LN2) | (1u << T_Q) | (1u << T_K) | (1u << T_V) | (1u << T_O) |
                        (1u << T_GATE) | (1u << T_UP) | (1u << T_DOWN);
        if (m->c.attn_bias) need |= (1u << T_BQ) | (1u << T_BK) | (1u << T_BV);
        if (m->c.o_bias) need |= 1u << T_BO;
        miss += __builtin_popcount(need & ~w.have);
    }
    *n_missing = miss;
    return BH_OK;
}

int bh_model_seq_open(bh_model* m, int slot, int64_t capacity) {
    if (!m) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    if (slot < 0 || slot >= m->c.max_seqs) return m->fail(BH_ERR_INVALID, "slot out of range");
    if (m->c.max_context > 0) capacity = m->c.max_context;
    if (capacity <= 0) return m->fail(BH_ERR_INVALID, "capacity must be positive");
    capacity = (capacity + m->kv_align - 1) / m->kv_align * m->kv_align;  // keeps regions aligned
    // a slot of the decode batch may be reopened for a new sequence (it keeps its region when the
    // capacity fits); its batch entry must then be replaced before the next decode
    int in_batch = -1;
    for (int b = 0; b < m->B; ++b)
        if (m->bslots[b] == slot) in_batch = b;
    if (m->off_h[slot] < 0 || m->cap_h[slot] < capacity) {
        if (m->next_free + capacity > m->c.kv_rows)
            return m->fail(BH_ERR_CAPACITY, "packed KV buffer full: " + std::to_string(m->next_free) + " + " +
                                                std::to_string(capacity) + " > " + std::to_string(m->c.kv_rows));
        m->off_h[slot] = m->next_free;
        m->cap_h[slot] = capacity;
        m->next_free += capacity;
    }
    m->len_h[slot] = 0;
    m->open_h[slot] = 1;
    if (in_batch >= 0) m->stale[in_batch] = 1;
    // repetition-penalty counts of the slot start at zero (an eager copy-engine fill, never captured)
    hipError_t e = hipMemsetAsync(m->d_pen + (size_t)slot * m->c.vocab, 0, (size_t)m->c.vocab * 2, m->st);
    if (e == hipSuccess) e = hipStreamSynchronize(m->st);
    return e == hipSuccess ? BH_OK : m->ctx->hip_fail(e, "seq_open");
}

// KV rows of a slot <-> the reference's per-layer host layout (LayerKvCache, cpu_engine.rs:
// 1720-1755; the flat vectors prefix_cache.rs:11-12 stores): k/v [layer][n][n_kv * head_dim] f32.
static int kv_rows_io(bh_model* m, int slot, int64_t row0, int64_t n, float* k, float* v, int to_host) {
    const bh_model_config& c = m->c;
    if (slot < 0 || slot >= c.max_seqs || !m->open_h[slot]) return m->fail(BH_ERR_INVALID, "slot is not open");
    if (row0 < 0 || n < 0 || row0 + n > m->cap_h[slot]) return m->fail(BH_ERR_CAPACITY, "rows outside the slot's KV region");
    if (c.max_context > 0 && row0 + n > c.max_context)
        return m->fail(BH_ERR_UNSUPPORTED, "KV rows past max_context are ring slots, not positions");
    if (n == 0) return BH_OK;
    const size_t per = (size_t)n * m->KD, bytes = per * 4;
    float* dk = nullptr;
    hipError_t e = hipMalloc(&dk, 2 * bytes);
    float* dv = dk + per;
    for (int l = 0; l < c.n_layers && e == hipSuccess; ++l) {
        if (!to_host) {
            e = hipMemcpyAsync(dk, k + (size_t)l * per, bytes, hipMemcpyHostToDevice, m->st);
            if (e == hipSuccess) e = hipMemcpyAsync(dv, v + (size_t)l * per, bytes, hipMemcpyHostToDevice, m->st);
        }
        if (e == hipSuccess)
            e = launch_kv_copy(kv_view(m, l), c.n_kv_heads, c.head_dim, m->off_h[slot] + row0, n, dk, dv, to_host, m->st);
        if (e == hipSuccess && to_host) {
            e = hipMemcpyAsync(k + (size_t)l * per, dk, bytes, hipMemcpyDeviceToHost, m->st);
            if (e == hipSuccess) e = hipMemcpyAsync(v + (size_t)l * per, dv, bytes, hipMemcpyDeviceToHost, m->st);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(m->st);  // the staging buffer is reused
    }
    if (dk) hipFree(dk);
    return e == hipSuccess ? BH_OK : m->ctx->hip_fail(e, "KV rows copy");
}

int bh_model_kv_read(bh_model* m, int slot, int64_t row0, int64_t n, float* k_out, float* v_out) {
    if (!m || (n > 0 && (!k_out || !v_out))) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    if (slot >= 0 && slot < m->c.max_seqs && row0 + n > m->len_h[slot])
        return m->fail(BH_ERR_INVALID, "rows past the slot's length");
    return kv_rows_io(m, slot, row0, n, k_out, v_out, 1);
}

int bh_model_kv_write(bh_model* m, int slot, int64_t row0, int64_t n, const float* k_in, const float* v_in) {
    if (!m || (n > 0 && (!k_in || !v_in))) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    for (int b = 0; b < m->B; ++b)
        if (m->bslots[b] == slot) return m->fail(BH_ERR_INVALID, "slot is in the decode batch; replace it first");
    if (slot >= 0 && slot < m->c.max_seqs && row0 > m->len_h[slot])
        return m->fail(BH_ERR_INVALID, "rows would leave a gap after the slot's length");
    const int rc = kv_rows_io(m, slot, row0, n, (float*)k_in, (float*)v_in, 0);
    if (rc == BH_OK) m->len_h[slot] = row0 + n;
    return rc;
}

int bh_model_seq_len(bh_model* m, int slot, int64_t* len) {
    if (!m || !len || slot < 0 || slot >= m->c.max_seqs) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    *len = m->open_h[slot] ? m->len_h[slot] : 0;
    return BH_OK;
}

namespace {

// One staged prompt row of a prefill chunk: region offset, token, position (-1: a pad row), slot.
struct PfRow {
    int64_t boff;
    int32_t tok, pos, slot;
};

// Checks of a prefill of n tokens into `slot` (open, positions within the RoPE table, capacity).
int prefill_check(bh_model* m, int slot, int64_t n) {
    if (slot < 0 || slot >= m->c.max_seqs || !m->open_h[slot]) return m->fail(BH_ERR_INVALID, "slot is not open");
    const int64_t end = m->len_h[slot] + n;
    if (end > m->max_pos) return m->fail(BH_ERR_CAPACITY, "position beyond the RoPE table");
    if (m->c.max_context > 0) {
        if (end > m->c.max_context)
            return m->fail(BH_ERR_UNSUPPORTED, "prefill past max_context is not supported with eviction");
    } else if (end > m->cap_h[slot]) {
        return m->fail(BH_ERR_CAPACITY, "prefill exceeds the slot's KV capacity");
    }
    return BH_OK;
}

// Run staged rows through the model in chunks of at most `chunk` rows (the caller's rows keep
// every 16-row group of an fp16-cache chunk inside one sequence when `chunk` is a multiple of 16).
int prefill_rows(bh_model* m, const std::vector<PfRow>& rows, int chunk) {
    size_t done = 0;
    while (done < rows.size()) {
        const int M = (int)std::min<size_t>(rows.size() - done, (size_t)chunk);
        int64_t* bo = (int64_t*)m->h_stage;
        int32_t* tok = (int32_t*)(bo + M);
        int32_t* pos = tok + M;
        int32_t* sl = pos + M;
        int maxpos = 0;
        for (int i = 0; i < M; ++i) {
            const PfRow& r = rows[done + i];
            bo[i] = r.boff;
            tok[i] = r.tok;
            pos[i] = r.pos;
            sl[i] = r.slot;
            maxpos = std::max(maxpos, r.pos);
        }
        hipError_t e = hipMemcpyAsync(m->d_pboff, bo, (size_t)M * 8, hipMemcpyHostToDevice, m->st);
        if (e == hipSuccess) e = hipMemcpyAsync(m->d_ptok, tok, (size_t)M * 4, hipMemcpyHostToDevice, m->st);
        if (e == hipSuccess) e = hipMemcpyAsync(m->d_ppos, pos, (size_t)M * 4, hipMemcpyHostToDevice, m->st);
        if (e == hipSuccess) e = hipMemcpyAsync(m->d_pslot, sl, (size_t)M * 4, hipMemcpyHostToDevice, m->st);
        int splits, srows;
        attn_plan(maxpos + 1, M, m->c.n_kv_heads, m->c.head_dim, &splits, &srows);
        if (e == hipSuccess)
            e = launch_embed(m->embed, m->d_ptok, m->L[0].ln1, m->x, m->xw, m->ssq, m->ssq_tiles, nullptr, M, m->st,
                             use_xl(m, M) ? m->xl_h : nullptr);
        if (e == hipSuccess) e = forward(m, M, false, splits, srows);
        if (e == hipSuccess) e = hipStreamSynchronize(m->st);  // the staging buffer is reused next chunk
        if (e != hipSuccess) return m->ctx->hip_fail(e, "prefill");
        done += M;
    }
    return BH_OK;
}

}  // namespace

int bh_model_prefill(bh_model* m, int slot, const uint32_t* tokens, int n) {
    if (!m || n < 0 || (n > 0 && !tokens)) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    int missing = 0;
    bh_model_missing(m, &missing);
    if (missing) return m->fail(BH_ERR_INVALID, std::to_string(missing) + " tensors not set");
    int rc = prefill_check(m, slot, n);
    if (rc) return rc;
    std::vector<PfRow> rows((size_t)n);
    for (int i = 0; i < n; ++i) rows[i] = PfRow{m->off_h[slot], (int32_t)tokens[i], (int32_t)(m->len_h[slot] + i), slot};
    rc = prefill_rows(m, rows, m->c.max_tokens);
    if (rc) return rc;
    m->len_h[slot] += n;
    return BH_OK;
}

int bh_model_prefill_batch(bh_model* m, int n_seqs, const int32_t* slots, const uint32_t* tokens, const int32_t* counts) {
    if (!m || n_seqs < 0 || (n_seqs > 0 && (!slots || !counts))) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    int missing = 0;
    bh_model_missing(m, &missing);
    if (missing) return m->fail(BH_ERR_INVALID, std::to_string(missing) + " tensors not set");
    int64_t total = 0;
    for (int s = 0; s < n_seqs; ++s) {
        if (counts[s] < 0) return m->fail(BH_ERR_INVALID, "negative token count");
        for (int t = 0; t < s; ++t)
            if (slots[t] == slots[s]) return m->fail(BH_ERR_INVALID, "a slot appears twice in one batch prefill");
        const int rc = prefill_check(m, slots[s], counts[s]);
        if (rc) return rc;
        total += counts[s];
    }
    if (total > 0 && !tokens) return BH_ERR_INVALID;
    // fp16 cache: every sequence padded to whole 16-row groups (the prefill attention's unit),
    // chunks of a multiple of 16 rows
    const int grp = m->c.kv_f16 ? 16 : 1;
    const int chunk = m->c.kv_f16 ? m->c.max_tokens / 16 * 16 : m->c.max_tokens;
    if (chunk <= 0) return m->fail(BH_ERR_UNSUPPORTED, "batch prefill needs max_tokens >= 16 with an fp16 cache");
    std::vector<PfRow> rows;
    int64_t t0 = 0;
    for (int s = 0; s < n_seqs; ++s) {
        const int slot = slots[s], n = counts[s];
        for (int i = 0; i < n; ++i)
            rows.push_back(PfRow{m->off_h[slot], (int32_t)tokens[t0 + i], (int32_t)(m->len_h[slot] + i), slot});
        for (int i = n; i % grp; ++i) rows.push_back(PfRow{m->off_h[slot], 0, -1, slot});
        t0 += n;
    }
    const int rc = prefill_rows(m, rows, chunk);
    if (rc) return rc;
    for (int s = 0; s < n_seqs; ++s) m->len_h[slots[s]] += counts[s];
    return BH_OK;
}

// Device state of batch entry b: its slot, the first KV row of the slot's region, its next input
// token and that token's position.
static hipError_t set_entry(bh_model* m, int b, int slot, uint32_t token) {
    const int32_t s32 = slot, t32 = (int32_t)token, p32 = m->len_h[slot];
    const int64_t bo = m->off_h[slot];
    hipError_t e = put(m, m->d_slot + b, &s32, 4);
    if (e == hipSuccess) e = put(m, m->d_tok + b, &t32, 4);
    if (e == hipSuccess) e = put(m, m->d_pos + b, &p32, 4);
    if (e == hipSuccess) e = put(m, m->d_boff + b, &bo, 8);
    return e;
}

int bh_model_decode_setup(bh_model* m, int batch, const int32_t* slots, const uint32_t* first_tokens) {
    if (!m || batch <= 0 || !slots || !first_tokens) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    if (batch > m->c.max_tokens || batch > m->c.max_seqs)
        return m->fail(BH_ERR_CAPACITY, "decode batch above max_tokens or max_seqs");
    std::vector<int32_t> seen(m->c.max_seqs, 0);
    for (int b = 0; b < batch; ++b) {
        if (slots[b] < 0 || slots[b] >= m->c.max_seqs || !m->open_h[slots[b]])
            return m->fail(BH_ERR_INVALID, "decode slot is not open");
        if (seen[slots[b]]++) return m->fail(BH_ERR_INVALID, "a slot appears twice in the decode batch");
    }
    drop_graph(m);  // the captured step holds the entries' KV offsets as launch arguments
    m->B = batch;
    m->bslots.assign(slots, slots + batch);
    m->stale.assign(batch, 0);
    for (int b = 0; b < batch; ++b) {
        hipError_t e = set_entry(m, b, slots[b], first_tokens[b]);
        if (e != hipSuccess) return m->ctx->hip_fail(e, "decode_setup");
    }
    return BH_OK;
}

int bh_model_decode_replace(bh_model* m, int b, int slot, uint32_t first_token) {
    if (!m) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    if (b < 0 || b >= m->B) return m->fail(BH_ERR_INVALID, "batch entry out of range");
    if (slot < 0 || slot >= m->c.max_seqs || !m->open_h[slot]) return m->fail(BH_ERR_INVALID, "slot is not open");
    for (int i = 0; i < m->B; ++i)
        if (i != b && m->bslots[i] == slot) return m->fail(BH_ERR_INVALID, "slot already in the batch");
    m->bslots[b] = slot;
    m->stale[b] = 0;
    // the captured step holds the entries' region offsets and the smallest capacity as launch
    // arguments: it stays valid when the new sequence has the old region (a reopened slot)
    if (m->gexec && ((int)m->g_off.size() <= b || m->g_off[b] != m->off_h[slot] || m->cap_h[slot] < m->g_cap))
        drop_graph(m);
    hipError_t e = set_entry(m, b, slot, first_token);
    return e == hipSuccess ? BH_OK : m->ctx->hip_fail(e, "decode_replace");
}

static int decode_locked(bh_model* m, int n_steps, uint32_t* ids_out, float* raw_logits) {
    if (m->B <= 0) return m->fail(BH_ERR_INVALID, "no decode batch (bh_model_decode_setup)");
    int missing = 0;
    bh_model_missing(m, &missing);
    if (missing) return m->fail(BH_ERR_INVALID, std::to_string(missing) + " tensors not set");
    int rc = check_decode_room(m, n_steps);
    if (rc) return rc;
    int splits, rows;
    attn_plan(decode_len_bound(m, n_steps), m->B, m->c.n_kv_heads, m->c.head_dim, &splits, &rows);
    hipError_t e = hipSuccess;
    m->store_logits = raw_logits != nullptr;
    if (!m->gexec || m->g_B != m->B || m->g_splits != splits || m->g_rows != rows || m->g_logits != m->store_logits) {
        drop_graph(m);
        e = hipStreamBeginCapture(m->st, hipStreamCaptureModeThreadLocal);
        if (e != hipSuccess) return m->ctx->hip_fail(e, "hipStreamBeginCapture");
        hipError_t fe = forward(m, m->B, true, splits, rows);
        e = hipStreamEndCapture(m->st, &m->graph);
        if (fe != hipSuccess) e = fe;
        if (e == hipSuccess) e = hipGraphInstantiate(&m->gexec, m->graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {
            drop_graph(m);
            return m->ctx->hip_fail(e, "decode graph capture");
        }
        m->g_B = m->B;
        m->g_splits = splits;
        m->g_rows = rows;
        m->g_logits = m->store_logits;
        m->g_off.resize(m->B);
        m->g_cap = INT64_MAX;
        for (int b = 0; b < m->B; ++b) {
            m->g_off[b] = m->off_h[m->bslots[b]];
            m->g_cap = std::min<int64_t>(m->g_cap, m->cap_h[m->bslots[b]]);
        }
    }
    int done = 0;
    while (done < n_steps && e == hipSuccess) {
        const int chunk = (int)std::min<int64_t>(n_steps - done, m->ids_steps);
        e = decode_start(m);
        for (int s = 0; s < chunk && e == hipSuccess; ++s) {
            e = hipGraphLaunch(m->gexec, m->st);
            if (e == hipSuccess && raw_logits)
                e = hipMemcpyAsync(raw_logits + (size_t)(done + s) * m->B * m->c.vocab, m->logits,
                                   (size_t)m->B * m->c.vocab * 4, hipMemcpyDeviceToHost, m->st);
        }
        if (e == hipSuccess && ids_out)
            e = hipMemcpyAsync(ids_out + (size_t)done * m->B, m->d_ids, (size_t)chunk * m->B * 4,
                               hipMemcpyDeviceToHost, m->st);
        if (e == hipSuccess) e = hipStreamSynchronize(m->st);
        done += chunk;
    }
    if (e != hipSuccess) return m->ctx->hip_fail(e, "decode");
    for (int b = 0; b < m->B; ++b) m->len_h[m->bslots[b]] += n_steps;
    return BH_OK;
}

int bh_model_decode(bh_model* m, int n_steps, uint32_t* ids_out, float* raw_logits) {
    if (!m || n_steps < 0) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    int st;
    if (m->ctx->injected(BH_OP_DECODE, &st)) return st;
    if (n_steps == 0) return BH_OK;
    return decode_locked(m, n_steps, ids_out, raw_logits);
}

int bh_model_generate(bh_model* m, int slot, const uint32_t* prompt, int n_prompt, int max_new, uint32_t* ids_out,
                      int* n_out, float* raw_logits) {
    if (!m || n_prompt < 0 || max_new < 0 || (n_prompt > 0 && !prompt) || !n_out || (max_new > 0 && !ids_out))
        return BH_ERR_INVALID;
    *n_out = 0;
    std::vector<uint32_t> toks(prompt, prompt + n_prompt);
    if (toks.empty()) toks.push_back(1);  // cpu_engine.rs:2487-2489
    const int64_t need = (int64_t)toks.size() + max_new;
    for (int b = 0; b < m->B; ++b)
        if (m->bslots[b] == slot) {  // a previous generate on this slot: leave the batch first
            drop_graph(m);
            m->B = 0;
            m->bslots.clear();
            break;
        }
    int rc = bh_model_seq_open(m, slot, need);
    if (rc) return rc;
    rc = bh_model_prefill(m, slot, toks.data(), (int)toks.size() - 1);
    if (rc) return rc;
    const int32_t s = slot;
    const uint32_t last = toks.back();
    rc = bh_model_decode_setup(m, 1, &s, &last);
    if (rc) return rc;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    int got = 0;
    const int chunk = 16;
    std::vector<uint32_t> ids(chunk);
    while (got < max_new) {
        const int n = std::min(chunk, max_new - got);
        rc = decode_locked(m, n, ids.data(), raw_logits ? raw_logits + (size_t)got * m->c.vocab : nullptr);
        if (rc) return rc;
        bool eos = false;
        for (int i = 0; i < n; ++i) {
            ids_out[got++] = ids[i];
            if (ids[i] == 2 || ids[i] == 151645 || ids[i] == 151643) {  // cpu_engine.rs:3060
                eos = true;
                break;
            }
        }
        if (eos) break;
    }
    *n_out = got;
    return BH_OK;
}

int bh_model_time_kernels(bh_model* m, int n_steps, double* mean_us, int64_t* launches) {
    if (!m || n_steps <= 0 || !mean_us || !launches) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(m->ctx->mu);
    if (m->B <= 0) return m->fail(BH_ERR_INVALID, "no decode batch");
    if (n_steps > m->ids_steps) return m->fail(BH_ERR_INVALID, "at most 1024 timed steps per call");
    int rc = check_decode_room(m, n_steps);
    if (rc) return rc;
    int splits, rows;
    attn_plan(decode_len_bound(m, n_steps), m->B, m->c.n_kv_heads, m->c.head_dim, &splits, &rows);
    std::vector<double> tot(BH_K_COUNT, 0.0);
    std::vector<int64_t> cnt(BH_K_COUNT, 0);
    hipError_t e = decode_start(m);
    m->store_logits = false;  // the greedy step as bh_model_decode runs it without raw logits
    for (int s = 0; s < n_steps && e == hipSuccess; ++s) {
        m->timing = true;
        m->recs.clear();
        m->ev_used = 0;
        e = forward(m, m->B, true, splits, rows);
        m->timing = false;
        if (e == hipSuccess) e = hipStreamSynchronize(m->st);
        for (auto& r : m->recs) {
            float ms = 0.f;
            if (hipEventElapsedTime(&ms, r.ev.start, r.ev.stop) == hipSuccess) {
                tot[r.cls] += ms * 1000.0;
                cnt[r.cls] += 1;
            }
        }
    }
    if (e != hipSuccess) return m->ctx->hip_fail(e, "timed decode");
    for (int b = 0; b < m->B; ++b) m->len_h[m->bslots[b]] += n_steps;
    for (int k = 0; k < BH_K_COUNT; ++k) {
        mean_us[k] = cnt[k] ? tot[k] / cnt[k] : 0.0;
        launches[k] = cnt[k];
    }
    return BH_OK;
}

int bh_model_kernel_bytes(bh_model* m, int kclass, double* bytes) {
    if (!m || !bytes) return BH_ERR_INVALID;
    const bh_model_config& c = m->c;
    const double B = m->B > 0 ? m->B : 1, H = c.hidden, I = c.ffn, QD = (double)m->QD, KD = (double)m->KD;
    const double kvb = c.kv_f16 ? 2.0 : 4.0, T = m->ssq_tiles;
    const LayerW& w = m->L[0];
    switch (kclass) {
        case BH_K_GEMV_QKV:  // weights (+bias), xw and ssq in; q out, K/V rows appended
            *bytes = weight_bytes(w.qkv) + (c.attn_bias ? (QD + 2 * KD) * 4 : 0) + B * (H + T) * 4 + B * QD * 4 +
                     B * 2 * KD * kvb;
            return BH_OK;
        case BH_K_GEMV_O:  // weights, attention out in; x read and written, xw and ssq out, norm weight
            *bytes = weight_bytes(w.o) + B * QD * 4 + B * (3 * H + T) * 4 + H * 4;
            return BH_OK;
        case BH_K_GEMV_GATEUP: *bytes = weight_bytes(w.gate) + weight_bytes(w.up) + B * (H + T) * 4 + B * I * 4; return BH_OK;
        case BH_K_GEMV_DOWN: *bytes = weight_bytes(w.down) + B * I * 4 + B * (3 * H + T) * 4 + H * 4; return BH_OK;
        case BH_K_LM_HEAD:  // tied table, xw in, penalty counts read; raw logits out when the greedy
                            // step stores them (top-k sampling)
            *bytes = weight_bytes(m->have_lm_head ? m->lm_head : m->embed) + B * (H + T) * 4 + B * (double)c.vocab * 2 +
                     (m->temperature > 0.f ? B * (double)c.vocab * 4 : 0.0);
            return BH_OK;
        case BH_K_ATTN:
        case BH_K_ATTN_O: {
            double rows = 0;
            for (int b = 0; b < m->B; ++b) {
                int64_t len = m->len_h[m->bslots[b]];
                if (c.max_context > 0) len = std::min<int64_t>(len, c.max_context);
                rows += (double)len;
            }
            if (kclass == BH_K_ATTN) {  // K/V rows and q in, attention out
                *bytes = rows * 2 * KD * kvb + 2 * B * QD * 4;
            } else {  // K/V rows and q in; O weights, x read and written, xw and ssq out, norm weight
                *bytes = rows * 2 * KD * kvb + B * QD * 4 + weight_bytes(w.o) + B * (3 * H + T) * 4 + H * 4;
            }
            return BH_OK;
        }
        default: *bytes = 0; return BH_OK;
    }
}

}  // extern "C"
