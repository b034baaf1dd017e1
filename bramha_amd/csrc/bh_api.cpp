// bh_api.cpp — context, weight registry and single-op entry points of the C ABI.
//
// HipComputePlane below is this backend's counterpart of WgpuComputePlane
// (src/compute/wgpu_backend.rs:100-117): one context per device holding a
// stream and a registry of device-resident weights keyed "model:layer" with
// least-recently-used eviction under a byte cap (ModelBuffers, :25-82;
// get_or_create_op, :603-722). Its matvec_mul* methods keep the reference's
// argument meaning and error behaviour: empty input -> Ok(zeros), size
// mismatch -> Err(text), everything else -> Ok(result).
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "bh_ctx.h"

using namespace bh;

namespace bh {
thread_local LaunchEvents* launch_events = nullptr;
}

// ------------------------------------------------------------------ helpers
int bh_ctx::fail(int status, const std::string& msg) {
    err = msg;
    return status;
}

int bh_ctx::hip_fail(hipError_t e, const char* what) {
    err = std::string(what) + ": " + hipGetErrorString(e);
    return e == hipErrorOutOfMemory ? BH_ERR_OOM : BH_ERR_HIP;
}

bool bh_ctx::injected(int op, int* status) {
    if (inj_count <= 0) return false;
    if (inj_op != BH_OP_ANY && inj_op != op) return false;
    --inj_count;
    *status = inj_status;
    err = "injected fault (op " + std::to_string(op) + ")";
    return true;
}

int bh_ctx::ensure_scratch(size_t xb, size_t yb) {
    if (xb > x_cap) {
        if (d_x) hipFree(d_x);
        d_x = nullptr;
        x_cap = 0;
        hipError_t e = hipMalloc(&d_x, xb);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch x)");
        x_cap = xb;
    }
    if (yb > y_cap) {
        if (d_y) hipFree(d_y);
        d_y = nullptr;
        y_cap = 0;
        hipError_t e = hipMalloc(&d_y, yb);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(scratch y)");
        y_cap = yb;
    }
    return BH_OK;
}

void bh_ctx::split_scratch(bh::GemvArgs& a, hipStream_t st) {
    if (st != stream || !split_part) return;
    a.part = split_part;
    a.tile_cnt = split_cnt;
    if (a.C <= bh::XL_TMP_CHUNKS) a.xl_tmp = xl_tmp;
}

namespace bh {

void free_weight(DevWeight& w) {
    if (w.q) hipFree(w.q);
    if (w.s) hipFree(w.s);
    w = DevWeight();
}

// Allocate a KM16 device weight of n rows (padded) and zero it.
int alloc_weight(bh_ctx* ctx, int fmt, int64_t n, int64_t k, DevWeight& w) {
    const int E = chunk_elems(fmt);
    if (n <= 0 || k <= 0 || k % E != 0)
        return ctx->fail(BH_ERR_UNSUPPORTED, "weight " + std::to_string(n) + "x" + std::to_string(k) +
                                                 ": in_features must be a positive multiple of " + std::to_string(E));
    w.fmt = fmt;
    w.n = n;
    w.k = k;
    w.n_pad = pad64(n);
    w.chunks = k / E;
    // the kernels address a weight with 32-bit buffer offsets
    if (w.chunks * w.n_pad * 16 >= ((int64_t)1 << 31))
        return ctx->fail(BH_ERR_UNSUPPORTED, "weight " + std::to_string(n) + "x" + std::to_string(k) +
                                                 ": 2 GiB or more of packed data (the kernels use 32-bit offsets)");
    const size_t qb = (size_t)(w.chunks * w.n_pad * 16);
    size_t sb = 0;
    if (fmt == BH_Q4_G32) sb = (size_t)(w.chunks * w.n_pad * 2);
    if (fmt == BH_Q8_ROW || fmt == BH_Q4_ROW) sb = (size_t)w.n_pad * 4;
    hipError_t e = hipMalloc(&w.q, qb);
    if (e != hipSuccess) {
        w.q = nullptr;
        return ctx->hip_fail(e, "hipMalloc(weight)");
    }
    e = hipMemset(w.q, 0, qb);
    if (e != hipSuccess) return ctx->hip_fail(e, "hipMemset(weight)");
    if (sb) {
        e = hipMalloc(&w.s, sb);
        if (e != hipSuccess) {
            w.s = nullptr;
            free_weight(w);
            return ctx->hip_fail(e, "hipMalloc(scales)");
        }
        e = hipMemset(w.s, 0, sb);
        if (e != hipSuccess) return ctx->hip_fail(e, "hipMemset(scales)");
    }
    w.bytes = qb + sb;
    return BH_OK;
}

// Expected host byte counts of a reference-layout weight.
bool host_sizes(int fmt, int64_t n, int64_t k, size_t* qb, size_t* sb) {
    switch (fmt) {
        case BH_F32: *qb = (size_t)(n * k * 4); *sb = 0; return true;
        case BH_Q8_ROW: *qb = (size_t)(n * k); *sb = (size_t)n * 4; return true;
        case BH_Q4_ROW: *qb = (size_t)(n * (k / 2)); *sb = (size_t)n * 4; return true;
        case BH_Q4_G32: *qb = (size_t)(n * (k / 2)); *sb = (size_t)(n * (k / 32)) * 2; return true;
        default: return false;
    }
}

// Write rows [row0, row0 + n) of `dst` from a reference-layout host weight.
int upload_rows(bh_ctx* ctx, DevWeight& dst, int64_t row0, int64_t n, const void* q, size_t q_bytes, const void* s,
                size_t s_bytes) {
    size_t eq, es;
    if (!host_sizes(dst.fmt, n, dst.k, &eq, &es)) return ctx->fail(BH_ERR_INVALID, "unknown weight format");
    if (q_bytes != eq || (es && s_bytes != es) || !q || (es && !s))
        return ctx->fail(BH_ERR_INVALID, "weight size mismatch: got " + std::to_string(q_bytes) + "/" +
                                             std::to_string(s_bytes) + " bytes, expected " + std::to_string(eq) +
                                             "/" + std::to_string(es) + " for " + std::to_string(n) + "x" +
                                             std::to_string(dst.k));
    if (row0 < 0 || row0 + n > dst.n) return ctx->fail(BH_ERR_INVALID, "row range outside the weight");
    std::string err;
    void *hq = nullptr, *hs = nullptr;
    size_t hqb = 0, hsb = 0;
    if (!repack_km16(dst.fmt, n, dst.k, q, s, err, &hq, &hqb, &hs, &hsb)) return ctx->fail(BH_ERR_UNSUPPORTED, err);
    const int64_t np_src = pad64(n);
    hipError_t e = hipMemcpy2D((uint8_t*)dst.q + row0 * 16, (size_t)dst.n_pad * 16, hq, (size_t)np_src * 16,
                               (size_t)n * 16, (size_t)dst.chunks, hipMemcpyHostToDevice);
    if (e == hipSuccess && dst.fmt == BH_Q4_G32) {
        // group scales: staged [C][n] on the device, then scattered to their sc_pos places (a row
        // range need not start on a 64-row group, and the other rows of its groups may already hold
        // another upload's scales)
        void* tmp = nullptr;
        e = hipMalloc(&tmp, (size_t)n * 2 * (size_t)dst.chunks);
        if (e == hipSuccess)
            e = hipMemcpy2D(tmp, (size_t)n * 2, hs, (size_t)np_src * 2, (size_t)n * 2, (size_t)dst.chunks,
                            hipMemcpyHostToDevice);
        if (e == hipSuccess) e = launch_scatter_scales(dst.s, tmp, row0, n, dst.n_pad, dst.chunks, nullptr);
        if (e == hipSuccess) e = hipStreamSynchronize(nullptr);
        if (tmp) {
            const hipError_t f = hipFree(tmp);
            if (e == hipSuccess) e = f;
        }
    } else if (e == hipSuccess && (dst.fmt == BH_Q8_ROW || dst.fmt == BH_Q4_ROW))
        e = hipMemcpy((float*)dst.s + row0, hs, (size_t)n * 4, hipMemcpyHostToDevice);
    free(hq);
    free(hs);
    if (e != hipSuccess) return ctx->hip_fail(e, "hipMemcpy(weight)");
    return BH_OK;
}

}  // namespace bh

// --------------------------------------------------------------- registry
void bh_ctx::touch(const std::string& key) {
    auto it = reg.find(key);
    if (it == reg.end()) return;
    lru.erase(it->second.lru_it);
    lru.push_back(key);
    it->second.lru_it = std::prev(lru.end());
}

// ModelBuffers::enforce_limits (wgpu_backend.rs:67-81): evict least recently used
// entries until the new bytes fit under the cap.
void bh_ctx::enforce_limits(size_t new_bytes) {
    while (used + new_bytes > cap && !lru.empty()) {
        const std::string key = lru.front();
        lru.pop_front();
        auto it = reg.find(key);
        if (it != reg.end()) {
            used -= std::min(used, it->second.w.bytes);
            free_weight(it->second.w);
            reg.erase(it);
        }
    }
}

void bh_ctx::clear_registry() {
    for (auto& kv : reg) free_weight(kv.second.w);
    reg.clear();
    lru.clear();
    used = 0;
}

// The shared body of the three matvec mirrors.
static int matvec_common(bh_ctx* ctx, int fmt, const float* h, size_t in_f, const void* q, size_t q_len,
                         size_t q_expect, const float* scales, size_t s_len, size_t out_f, const char* model,
                         const char* layer, float* out) {
    if (!ctx) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    int st;
    if (ctx->injected(BH_OP_MATVEC, &st)) return st;
    if (out_f > 0 && !out) return ctx->fail(BH_ERR_INVALID, "out is NULL");
    if (in_f == 0 || out_f == 0) {  // wgpu_backend.rs:1093-1095
        if (out_f) std::memset(out, 0, out_f * 4);
        return BH_OK;
    }
    if (!h || !q) return ctx->fail(BH_ERR_INVALID, "input is NULL");
    const char* what = fmt == BH_F32 ? "Weight" : (fmt == BH_Q8_ROW ? "Quantized INT8 weight" : "Quantized INT4 weight");
    if (q_len != q_expect)  // wgpu_backend.rs:1096-1104
        return ctx->fail(BH_ERR_INVALID, std::string(what) + " size mismatch: weight length is " +
                                             std::to_string(q_len) + ", expected " + std::to_string(q_expect));
    if (fmt != BH_F32 && (!scales || s_len != out_f))
        return ctx->fail(BH_ERR_INVALID, "scales length is " + std::to_string(s_len) + ", expected " +
                                             std::to_string(out_f));
    const int64_t k = fmt == BH_Q4_ROW ? (int64_t)(in_f / 2) * 2 : (int64_t)in_f;
    if (fmt == BH_Q4_ROW && (in_f % 2))
        return ctx->fail(BH_ERR_UNSUPPORTED, "INT4 GEMV needs an even in_features");

    DevWeight tmp;
    const DevWeight* w = nullptr;
    std::string key;
    const bool keyed = model && layer;
    if (keyed) {
        key = std::string(model) + ":" + layer;
        auto it = ctx->reg.find(key);
        if (it != ctx->reg.end()) {
            const DevWeight& cw = it->second.w;
            if (cw.fmt != fmt || cw.n != (int64_t)out_f || cw.k != k)
                return ctx->fail(BH_ERR_INVALID, "registry entry '" + key + "' holds a " + std::to_string(cw.n) +
                                                     "x" + std::to_string(cw.k) + " weight of another format/shape");
            ctx->touch(key);
            w = &cw;
        }
    }
    if (!w) {
        int rc = alloc_weight(ctx, fmt, (int64_t)out_f, k, tmp);
        if (rc) return rc;
        rc = upload_rows(ctx, tmp, 0, (int64_t)out_f, q, q_len * (fmt == BH_F32 ? 4 : 1), scales,
                         fmt == BH_F32 ? 0 : out_f * 4);
        if (rc) {
            free_weight(tmp);
            return rc;
        }
        if (keyed) {
            ctx->enforce_limits(tmp.bytes);
            auto& ent = ctx->reg[key];
            ent.w = tmp;
            ctx->lru.push_back(key);
            ent.lru_it = std::prev(ctx->lru.end());
            ctx->used += tmp.bytes;
            tmp = DevWeight();
            w = &ent.w;
        } else {
            w = &tmp;
        }
    }
    int rc = ctx->ensure_scratch(in_f * 4, out_f * 4);
    if (rc) {
        free_weight(tmp);
        return rc;
    }
    hipError_t e = hipMemcpyAsync(ctx->d_x, h, in_f * 4, hipMemcpyHostToDevice, ctx->stream);
    GemvArgs a;
    a.W = w->q;
    a.S = w->s;
    a.x = (const float*)ctx->d_x;
    a.ldx = (int64_t)in_f;
    a.y = (float*)ctx->d_y;
    a.ldy = (int64_t)out_f;
    a.N = (int)w->n;
    a.n_pad = (int)w->n_pad;
    a.C = (int)w->chunks;
    a.batch = 1;
    if (e == hipSuccess) e = launch_gemv(fmt, EPI_STORE, a, ctx->stream);
    if (e == hipSuccess) e = hipMemcpyAsync(out, ctx->d_y, out_f * 4, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    free_weight(tmp);
    if (e != hipSuccess) return ctx->hip_fail(e, "matvec");
    return BH_OK;
}

// ------------------------------------------------ no-allocation attention scratch
// Scratch of bh_attn_decode_noalloc: NOALLOC_PART_BYTES of split partials, then NOALLOC_COUNTERS
// int32 split-merge counters. Every launch leaves the counters at zero (the last workgroup of
// each (row, KV head) resets its own); they are cleared once per device at bh_init. Each device
// holds its own copy until the process ends. In host code the name `scratch` stands for the
// array but is not its device address: that is resolved per device with hipGetSymbolAddress and
// only that address is used.
constexpr size_t NOALLOC_PART_BYTES = (size_t)2 << 20;
constexpr int NOALLOC_COUNTERS = 4096;
static __device__ __align__(256) uint8_t scratch[NOALLOC_PART_BYTES + (size_t)NOALLOC_COUNTERS * 4];

static std::mutex g_noalloc_mu;
static uint8_t* g_noalloc_ptr[256] = {};  // per device ordinal

// Resolve this device's copy of `scratch` (the device is current) and clear its counters once.
static int noalloc_setup(bh_ctx* c) {
    if (c->device < 0 || c->device >= 256) return c->fail(BH_ERR_UNSUPPORTED, "device ordinal above 255");
    std::lock_guard<std::mutex> g(g_noalloc_mu);
    if (!g_noalloc_ptr[c->device]) {
        uint8_t* p = nullptr;
        hipError_t e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) return c->hip_fail(e, "hipGetSymbolAddress(no-allocation scratch)");
        e = hipMemsetAsync(p + NOALLOC_PART_BYTES, 0, (size_t)NOALLOC_COUNTERS * 4, c->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
        if (e != hipSuccess) return c->hip_fail(e, "clearing the no-allocation scratch");
        g_noalloc_ptr[c->device] = p;
    }
    c->noalloc_scratch = g_noalloc_ptr[c->device];
    return BH_OK;
}

extern "C" {

const char* bh_status_str(int s) {
    switch (s) {
        case BH_OK: return "ok";
        case BH_ERR_INVALID: return "invalid argument";
        case BH_ERR_NO_DEVICE: return "no usable gfx950 device";
        case BH_ERR_HIP: return "HIP runtime error";
        case BH_ERR_OOM: return "device out of memory";
        case BH_ERR_NOT_FOUND: return "not found";
        case BH_ERR_INJECTED: return "injected fault";
        case BH_ERR_UNSUPPORTED: return "unsupported shape or format";
        case BH_ERR_CAPACITY: return "capacity exceeded";
        default: return "unknown status";
    }
}

int bh_init(int device, bh_ctx** out) {
    if (!out) return BH_ERR_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0 || device < 0 || device >= n) return BH_ERR_NO_DEVICE;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) != hipSuccess) return BH_ERR_NO_DEVICE;
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) return BH_ERR_NO_DEVICE;
    if (hipSetDevice(device) != hipSuccess) return BH_ERR_NO_DEVICE;
    bh_ctx* c = new bh_ctx();
    c->device = device;
    c->n_cu = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return BH_ERR_HIP;
    }
    // split scratch up front, so that no GEMV call (captured or not) allocates
    const size_t pb = (size_t)SPLIT_PART_FLOATS * 4, cb = (size_t)SPLIT_TILES_MAX * 4;
    const size_t xb = (size_t)XL_TMP_CHUNKS * (XL_REC_BYTES + 4);
    if (hipMalloc(&c->split_part, pb) != hipSuccess || hipMalloc(&c->split_cnt, cb) != hipSuccess ||
        hipMalloc(&c->xl_tmp, xb) != hipSuccess || hipMemset(c->split_cnt, 0, cb) != hipSuccess) {
        if (c->split_part) hipFree(c->split_part);
        if (c->split_cnt) hipFree(c->split_cnt);
        if (c->xl_tmp) hipFree(c->xl_tmp);
        hipStreamDestroy(c->stream);
        delete c;
        return BH_ERR_OOM;
    }
    if (noalloc_setup(c) != BH_OK) {
        hipFree(c->split_part);
        hipFree(c->split_cnt);
        hipFree(c->xl_tmp);
        hipStreamDestroy(c->stream);
        delete c;
        return BH_ERR_HIP;
    }
    *out = c;
    return BH_OK;
}

void bh_destroy(bh_ctx* ctx) {
    if (!ctx) return;
    hipSetDevice(ctx->device);
    hipStreamSynchronize(ctx->stream);
    ctx->clear_registry();
    if (ctx->d_x) hipFree(ctx->d_x);
    if (ctx->d_y) hipFree(ctx->d_y);
    for (auto& kv : ctx->rope_tabs) hipFree(kv.second);
    hipDeviceSynchronize();  // calls on the caller's streams used the attention scratch
    for (auto& kv : ctx->attn_scratch) {
        if (kv.second.part) hipFree(kv.second.part);
        if (kv.second.cnt) hipFree(kv.second.cnt);
    }
    for (void* p : ctx->retired) hipFree(p);
    if (ctx->split_part) hipFree(ctx->split_part);
    if (ctx->split_cnt) hipFree(ctx->split_cnt);
    if (ctx->xl_tmp) hipFree(ctx->xl_tmp);
    hipStreamDestroy(ctx->stream);
    delete ctx;
}

const char* bh_last_error(const bh_ctx* ctx) { return ctx ? ctx->err.c_str() : "no context"; }

int bh_set_vram_cap(bh_ctx* ctx, size_t bytes) {
    if (!ctx) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->cap = bytes;
    ctx->enforce_limits(0);
    return BH_OK;
}

int bh_registry_stats(bh_ctx* ctx, size_t* n_entries, size_t* bytes) {
    if (!ctx) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (n_entries) *n_entries = ctx->reg.size();
    if (bytes) *bytes = ctx->used;
    return BH_OK;
}

int bh_debug_inject_fault(bh_ctx* ctx, int op, int status, int count) {
    if (!ctx) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    ctx->inj_op = op;
    ctx->inj_status = status == 0 ? BH_ERR_INJECTED : status;
    ctx->inj_count = count;
    return BH_OK;
}

int bh_dev_alloc(bh_ctx* ctx, size_t bytes, void** out) {
    if (!ctx || !out) return BH_ERR_INVALID;
    *out = nullptr;
    hipError_t e = hipMalloc(out, std::max<size_t>(bytes, 1));
    if (e != hipSuccess) {
        *out = nullptr;
        return ctx->hip_fail(e, "hipMalloc");
    }
    return BH_OK;
}

int bh_dev_free(bh_ctx* ctx, void* p) {
    if (!ctx) return BH_ERR_INVALID;
    if (!p) return BH_OK;
    hipStreamSynchronize(ctx->stream);
    hipError_t e = hipFree(p);
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "hipFree");
}

int bh_memcpy_h2d(bh_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return BH_ERR_INVALID;
    if (!bytes) return BH_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "hipMemcpy H2D");
}

int bh_memcpy_d2h(bh_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx || (bytes && (!dst || !src))) return BH_ERR_INVALID;
    if (!bytes) return BH_OK;
    hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "hipMemcpy D2H");
}

int bh_synchronize(bh_ctx* ctx) {
    if (!ctx) return BH_ERR_INVALID;
    hipError_t e = hipDeviceSynchronize();
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "hipDeviceSynchronize");
}

int bh_matvec_mul(bh_ctx* ctx, const float* h, size_t in_features, const float* weight, size_t weight_len,
                  size_t out_features, const char* model_name, const char* layer_name, float* out) {
    return matvec_common(ctx, BH_F32, h, in_features, weight, weight_len, out_features * in_features, nullptr, 0,
                         out_features, model_name, layer_name, out);
}

int bh_matvec_mul_int8(bh_ctx* ctx, const float* h, size_t in_features, const int8_t* q_weight, size_t q_len,
                       const float* scales, size_t s_len, size_t out_features, const char* model_name,
                       const char* layer_name, float* out) {
    return matvec_common(ctx, BH_Q8_ROW, h, in_features, q_weight, q_len, out_features * in_features, scales, s_len,
                         out_features, model_name, layer_name, out);
}

int bh_matvec_mul_int4(bh_ctx* ctx, const float* h, size_t in_features, const uint8_t* q_weight, size_t q_len,
                       const float* scales, size_t s_len, size_t out_features, const char* model_name,
                       const char* layer_name, float* out) {
    return matvec_common(ctx, BH_Q4_ROW, h, in_features, q_weight, q_len, out_features * (in_features / 2), scales,
                         s_len, out_features, model_name, layer_name, out);
}

int bh_clear_persistent_buffers(bh_ctx* ctx) {
    if (!ctx) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    hipStreamSynchronize(ctx->stream);
    ctx->clear_registry();
    return BH_OK;
}

// ------------------------------------------------------ device-resident weights
int bh_weight_upload(bh_ctx* ctx, int fmt, int64_t n_out, int64_t k_in, const void* q, size_t q_bytes,
                     const void* scales, size_t s_bytes, bh_weight** out) {
    if (!ctx || !out) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    int st;
    if (ctx->injected(BH_OP_UPLOAD, &st)) return st;
    if (fmt < BH_F32 || fmt > BH_Q4_G32) return ctx->fail(BH_ERR_INVALID, "unknown format");
    DevWeight w;
    int rc = alloc_weight(ctx, fmt, n_out, k_in, w);
    if (rc) return rc;
    rc = upload_rows(ctx, w, 0, n_out, q, q_bytes, scales, s_bytes);
    if (rc) {
        free_weight(w);
        return rc;
    }
    *out = (bh_weight*)new DevWeight(w);
    return BH_OK;
}

void bh_weight_free(bh_ctx* ctx, bh_weight* w) {
    if (!w) return;
    if (ctx) hipStreamSynchronize(ctx->stream);
    DevWeight* d = (DevWeight*)w;
    free_weight(*d);
    delete d;
}

static hipStream_t pick(bh_ctx* ctx, void* stream) { return stream ? (hipStream_t)stream : ctx->stream; }

int bh_gemv(bh_ctx* ctx, const bh_weight* wh, const float* x, float* y, int batch, void* stream) {
    if (!ctx || !wh || !x || !y || batch < 0) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    int st;
    if (ctx->injected(BH_OP_GEMV, &st)) return st;
    if (batch == 0) return BH_OK;
    const DevWeight* w = (const DevWeight*)wh;
    GemvArgs a;
    a.W = w->q;
    a.S = w->s;
    a.x = x;
    a.ldx = w->k;
    a.y = y;
    a.ldy = w->n;
    a.N = (int)w->n;
    a.n_pad = (int)w->n_pad;
    a.C = (int)w->chunks;
    a.batch = batch;
    const hipStream_t hs = pick(ctx, stream);
    ctx->split_scratch(a, hs);
    hipError_t e = launch_gemv(w->fmt, EPI_STORE, a, hs);
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "gemv launch");
}

int bh_dequant(bh_ctx* ctx, const bh_weight* wh, float* out, void* stream) {
    if (!ctx || !wh || !out) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    hipError_t e = launch_dequant(*(const DevWeight*)wh, out, pick(ctx, stream));
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "dequant launch");
}

// ------------------------------------------------------------ single ops
int bh_rmsnorm(bh_ctx* ctx, const float* x, const float* w, float eps, float* out, int rows, int n, void* stream) {
    if (!ctx || !x || !w || !out || rows < 0 || n <= 0) return BH_ERR_INVALID;
    if (rows == 0) return BH_OK;
    hipError_t e = launch_rmsnorm(x, w, eps, out, rows, n, pick(ctx, stream));
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "rmsnorm launch");
}

const float2* bh_ctx::rope_tab(int hd, float theta, int max_pos) {
    char key[96];
    std::snprintf(key, sizeof key, "%d:%08x:%d", hd, *(const uint32_t*)&theta, max_pos);
    auto it = rope_tabs.find(key);
    if (it != rope_tabs.end()) return (const float2*)it->second;
    std::vector<float2> h((size_t)max_pos * (hd / 2));
    rope_table(hd, theta, max_pos, h.data());
    void* d = nullptr;
    if (hipMalloc(&d, h.size() * sizeof(float2)) != hipSuccess) return nullptr;
    if (hipMemcpy(d, h.data(), h.size() * sizeof(float2), hipMemcpyHostToDevice) != hipSuccess) {
        hipFree(d);
        return nullptr;
    }
    rope_tabs[key] = d;
    return (const float2*)d;
}

int bh_rope(bh_ctx* ctx, float* v, const int32_t* pos, int rows, int n_heads, int head_dim, float theta, int max_pos,
            void* stream) {
    if (!ctx || !v || !pos || rows < 0 || n_heads <= 0 || head_dim <= 0 || head_dim % 2 || max_pos <= 0)
        return BH_ERR_INVALID;
    if (rows == 0) return BH_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    const float2* tab = ctx->rope_tab(head_dim, theta, max_pos);
    if (!tab) return ctx->fail(BH_ERR_OOM, "rope table");
    hipError_t e = launch_rope(v, pos, tab, rows, n_heads, head_dim, pick(ctx, stream));
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "rope launch");
}

int bh_silu_mul(bh_ctx* ctx, const float* g, const float* u, float* out, int64_t n, void* stream) {
    if (!ctx || !g || !u || !out || n < 0) return BH_ERR_INVALID;
    if (n == 0) return BH_OK;
    hipError_t e = launch_silu_mul(g, u, out, n, pick(ctx, stream));
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "silu launch");
}

// Attention arguments (everything but the split scratch).
static void attn_fill(const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows, const int64_t* seq_off,
                      const int32_t* seq_len, int batch, int n_q, int n_kv, int head_dim, int max_len, float* out,
                      AttnArgs& a) {
    a.q = q;
    a.out = out;
    a.kv.k = (void*)k;
    a.kv.v = (void*)v;
    a.kv.kv_rows = kv_rows;
    a.kv.kv_f16 = kv_f16 ? 1 : 0;
    a.boff = seq_off;
    a.seq_len = seq_len;
    a.batch = batch;
    a.nq = n_q;
    a.nkv = n_kv;
    a.hd = head_dim;
    attn_plan(std::max(max_len, 1), batch, n_kv, head_dim, &a.splits, &a.split_rows);
}

static bool capturing(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

// Attention arguments and the split scratch of `st` for bh_attn_decode (context lock held).
static int attn_args(bh_ctx* ctx, hipStream_t st, const float* q, const void* k, const void* v, int kv_f16,
                     int64_t kv_rows, const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv,
                     int head_dim, int max_len, float* out, AttnArgs& a) {
    attn_fill(q, k, v, kv_f16, kv_rows, seq_off, seq_len, batch, n_q, n_kv, head_dim, max_len, out, a);
    if (a.splits <= 1) return BH_OK;
    const size_t need = (size_t)batch * n_q * a.splits * (head_dim + 2) * 4;
    const int need_cnt = batch * n_kv;
    bh_ctx::AttnScratch& sc = ctx->attn_scratch[st];
    if (need > sc.part_bytes || need_cnt > sc.cnt_len) {
        if (capturing(st))
            return ctx->fail(BH_ERR_CAPACITY, "attention split scratch of this stream is too small for a call made "
                                              "under graph capture: make one uncaptured call of this size first");
        // the old buffers stay allocated (a captured graph may hold them); in-flight work finishes
        hipError_t e = hipStreamSynchronize(st);
        if (e != hipSuccess) return ctx->hip_fail(e, "hipStreamSynchronize");
        bh_ctx::AttnScratch ns;
        ns.part_bytes = std::max(need, sc.part_bytes);
        ns.cnt_len = std::max(need_cnt, sc.cnt_len);
        e = hipMalloc(&ns.part, ns.part_bytes);
        if (e == hipSuccess) e = hipMalloc((void**)&ns.cnt, (size_t)ns.cnt_len * 4);
        if (e == hipSuccess) e = hipMemset(ns.cnt, 0, (size_t)ns.cnt_len * 4);
        if (e != hipSuccess) {
            if (ns.part) hipFree(ns.part);
            if (ns.cnt) hipFree(ns.cnt);
            return ctx->hip_fail(e, "hipMalloc(attention scratch)");
        }
        if (sc.part) ctx->retired.push_back(sc.part);
        if (sc.cnt) ctx->retired.push_back(sc.cnt);
        sc = ns;
    }
    a.part_o = (float*)sc.part;
    a.part_ml = a.part_o + (size_t)batch * n_q * a.splits * head_dim;
    a.cnt = sc.cnt;
    return BH_OK;
}

static int attn_check(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                      const int64_t* seq_off, const int32_t* seq_len, float* out, int batch, int n_q, int n_kv,
                      int head_dim, int max_len) {
    if (!ctx || !q || !k || !v || !seq_off || !seq_len || !out || batch < 0 || n_q <= 0 || n_kv <= 0 ||
        n_q % n_kv || max_len < 0 || kv_rows <= 0)
        return BH_ERR_INVALID;
    if (kv_f16 && kv_rows % 64)
        return ctx->fail(BH_ERR_INVALID, "an fp16 KV cache holds whole 64-row tiles: kv_rows must be a multiple of 64");
    if (!attn_supported(n_q, n_kv, head_dim))
        return ctx->fail(BH_ERR_UNSUPPORTED, "attention supports head_dim 64/128 and 1, 2, 4, 7 or 8 query heads per KV head");
    return BH_OK;
}

int bh_attn_decode(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                   const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv, int head_dim,
                   int max_len, float* out, void* stream) {
    int rc = attn_check(ctx, q, k, v, kv_f16, kv_rows, seq_off, seq_len, out, batch, n_q, n_kv, head_dim, max_len);
    if (rc) return rc;
    if (batch == 0) return BH_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    const hipStream_t st = pick(ctx, stream);
    AttnArgs a;
    rc = attn_args(ctx, st, q, k, v, kv_f16, kv_rows, seq_off, seq_len, batch, n_q, n_kv, head_dim, max_len, out, a);
    if (rc) return rc;
    hipError_t e = launch_attention(a, st);
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "attention launch");
}

int bh_attn_decode_noalloc(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                           const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv,
                           int head_dim, int max_len, float* out, void* stream) {
    int rc = attn_check(ctx, q, k, v, kv_f16, kv_rows, seq_off, seq_len, out, batch, n_q, n_kv, head_dim, max_len);
    if (rc) return rc;
    if (batch == 0) return BH_OK;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (!ctx->noalloc_scratch) return ctx->fail(BH_ERR_HIP, "no-allocation scratch not set up");
    AttnArgs a;
    attn_fill(q, k, v, kv_f16, kv_rows, seq_off, seq_len, batch, n_q, n_kv, head_dim, max_len, out, a);
    if (a.splits > 1) {
        const size_t need = (size_t)batch * n_q * a.splits * (head_dim + 2) * 4;
        if (need > NOALLOC_PART_BYTES || (int64_t)batch * n_kv > NOALLOC_COUNTERS)
            return ctx->fail(BH_ERR_CAPACITY, "attention split scratch of " + std::to_string(need) + " bytes and " +
                                                  std::to_string((int64_t)batch * n_kv) +
                                                  " counters exceeds the no-allocation scratch (" +
                                                  std::to_string(NOALLOC_PART_BYTES) + " bytes, " +
                                                  std::to_string(NOALLOC_COUNTERS) + " counters)");
        a.part_o = (float*)ctx->noalloc_scratch;
        a.part_ml = a.part_o + (size_t)batch * n_q * a.splits * head_dim;
        a.cnt = (int32_t*)(ctx->noalloc_scratch + NOALLOC_PART_BYTES);
    }
    hipError_t e = launch_attention(a, pick(ctx, stream));
    return e == hipSuccess ? BH_OK : ctx->hip_fail(e, "attention launch");
}

// ------------------------------------------------------------ sampling draws
float bh_sample_uniform(uint64_t seed, int slot, int pos) { return sample_uniform(seed, slot, pos); }

// ------------------------------------------------------------ measurement
}  // extern "C"

// Replays a HIP graph of `iters` launches built by `record` (launch i of `copies` rotating
// operands) and returns the mean time per launch in microseconds.
template <class F>
static int time_graph(bh_ctx* ctx, int iters, F&& record, double* us) {
    hipStream_t st = ctx->stream;
    hipGraph_t g = nullptr;
    hipGraphExec_t ge = nullptr;
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return ctx->hip_fail(e, "hipStreamBeginCapture");
    hipError_t le = hipSuccess;
    for (int i = 0; i < iters && le == hipSuccess; ++i) le = record(i, st);
    e = hipStreamEndCapture(st, &g);
    if (le != hipSuccess) e = le;
    if (e == hipSuccess) e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    if (e == hipSuccess) e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = hipGraphLaunch(ge, st);  // warm-up replay
    if (e == hipSuccess) e = hipEventRecord(e0, st);
    const int reps = 3;
    for (int r = 0; r < reps && e == hipSuccess; ++r) e = hipGraphLaunch(ge, st);
    if (e == hipSuccess) e = hipEventRecord(e1, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) hipEventDestroy(e0);
    if (e1) hipEventDestroy(e1);
    if (ge) hipGraphExecDestroy(ge);
    if (g) hipGraphDestroy(g);
    if (e != hipSuccess) return ctx->hip_fail(e, "timed graph");
    *us = ms * 1000.0 / ((double)reps * iters);
    return BH_OK;
}

extern "C" {

int bh_time_gemv(bh_ctx* ctx, const bh_weight* wh, const float* x, float* y, int batch, int iters,
                 size_t rotate_bytes, double* us_per_launch) {
    if (!ctx || !wh || !x || !y || batch <= 0 || iters <= 0 || !us_per_launch) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    const DevWeight& w = *(const DevWeight*)wh;
    const int copies = (int)std::max<size_t>(1, std::min<size_t>(4096, (rotate_bytes + w.bytes - 1) / std::max<size_t>(w.bytes, 1)));
    std::vector<DevWeight> cl(copies);
    int rc = BH_OK;
    cl[0] = w;
    const size_t qb = (size_t)w.chunks * w.n_pad * 16, sb = w.bytes - qb;
    for (int i = 1; i < copies && rc == BH_OK; ++i) {
        cl[i] = w;
        cl[i].q = cl[i].s = nullptr;
        hipError_t e = hipMalloc(&cl[i].q, qb);
        if (e == hipSuccess) e = hipMemcpy(cl[i].q, w.q, qb, hipMemcpyDeviceToDevice);
        if (e == hipSuccess && sb) e = hipMalloc(&cl[i].s, sb);
        if (e == hipSuccess && sb) e = hipMemcpy(cl[i].s, w.s, sb, hipMemcpyDeviceToDevice);
        if (e != hipSuccess) rc = ctx->hip_fail(e, "weight copies");
    }
    // A batch-1 group-32 pass reads its activations as limb records, which in the decode step
    // the producer of x writes: they are converted once here, outside the timed launches.
    const bool xl = batch == 1 && w.fmt == BH_Q4_G32 && w.chunks <= XL_TMP_CHUNKS;
    if (rc == BH_OK && xl) {
        hipError_t e = launch_xl_pack(x, (int)w.chunks * 32, ctx->xl_tmp, ctx->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
        if (e != hipSuccess) rc = ctx->hip_fail(e, "limb records");
    }
    if (rc == BH_OK)
        rc = time_graph(ctx, iters, [&](int i, hipStream_t st) {
            const DevWeight& c = cl[i % copies];
            GemvArgs a;
            a.W = c.q;
            a.S = c.s;
            a.x = x;
            a.ldx = c.k;
            a.y = y;
            a.ldy = c.n;
            a.N = (int)c.n;
            a.n_pad = (int)c.n_pad;
            a.C = (int)c.chunks;
            a.batch = batch;
            ctx->split_scratch(a, st);
            if (xl) a.xl = ctx->xl_tmp;
            return launch_gemv(c.fmt, EPI_STORE, a, st);
        }, us_per_launch);
    for (int i = 1; i < copies; ++i) {
        if (cl[i].q) hipFree(cl[i].q);
        if (cl[i].s) hipFree(cl[i].s);
    }
    return rc;
}

int bh_time_probe(bh_ctx* ctx, int copy, size_t bytes, int wgs, int unroll, int iters, double* us_per_launch) {
    if (!ctx || bytes < 16 || wgs <= 0 || wgs > (1 << 20) || iters <= 0 || !us_per_launch || copy < 0 || copy > 3 ||
        !(unroll == 4 || unroll == 8 || unroll == 16) || (copy == 2 && bytes > (64u << 20)))
        return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    if (copy == 3) {  // grid barriers: time per barrier phase, the grid resident at once
        int dev = 0, cus = 0;
        hipError_t e = hipGetDevice(&dev);
        if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return ctx->hip_fail(e, "device attributes");
        if (wgs > cus) return ctx->fail(BH_ERR_INVALID, "grid-barrier probe: at most one workgroup per CU");
        int* cnt = nullptr;  // [2] counts, then [1] error count, then the data
        e = hipMalloc(&cnt, 16 + (size_t)gridbar_phases() * wgs * 4);
        if (e == hipSuccess) e = hipMemset(cnt, 0, 16);
        int rc = e == hipSuccess ? BH_OK : ctx->hip_fail(e, "hipMalloc(probe buffers)");
        if (rc == BH_OK)
            rc = time_graph(ctx, iters, [&](int, hipStream_t st) {
                return launch_gridbar_probe(cnt, (float*)(cnt + 4), cnt + 2, wgs, st);
            }, us_per_launch);
        int bad = 0;
        if (rc == BH_OK) {
            e = hipMemcpy(&bad, cnt + 2, 4, hipMemcpyDeviceToHost);
            if (e != hipSuccess) rc = ctx->hip_fail(e, "hipMemcpy");
        }
        if (cnt) hipFree(cnt);
        if (rc == BH_OK && bad) rc = ctx->fail(BH_ERR_HIP, "grid-barrier probe: a wait gave up");
        if (rc == BH_OK) *us_per_launch /= gridbar_phases();
        return rc;
    }
    bytes &= ~(size_t)15;
    void *src = nullptr, *dst = nullptr, *sink = nullptr;
    hipError_t e = hipMalloc(&src, bytes);
    if (e == hipSuccess) e = hipMemset(src, 0x5a, bytes);
    if (e == hipSuccess && copy) e = hipMalloc(&dst, bytes);
    if (e == hipSuccess && !copy) e = hipMalloc(&sink, (size_t)wgs * 256 * 4);
    int rc = e == hipSuccess ? BH_OK : ctx->hip_fail(e, "hipMalloc(probe buffers)");
    if (rc == BH_OK)
        rc = time_graph(ctx, iters, [&](int i, hipStream_t st) {
            if (copy == 2)  // the chain ping-pongs between the two buffers
                return launch_probe(2, i & 1 ? dst : src, i & 1 ? src : dst, (int64_t)bytes, wgs, unroll, nullptr, st);
            return launch_probe(copy, src, dst, (int64_t)bytes, wgs, unroll, (uint32_t*)sink, st);
        }, us_per_launch);
    if (src) hipFree(src);
    if (dst) hipFree(dst);
    if (sink) hipFree(sink);
    return rc;
}

int bh_time_attn(bh_ctx* ctx, const float* q, const void* k, const void* v, int kv_f16, int64_t kv_rows,
                 const int64_t* seq_off, const int32_t* seq_len, int batch, int n_q, int n_kv, int head_dim,
                 int max_len, float* out, int iters, size_t rotate_bytes, double* us_per_launch) {
    int rc = attn_check(ctx, q, k, v, kv_f16, kv_rows, seq_off, seq_len, out, batch, n_q, n_kv, head_dim, max_len);
    if (rc) return rc;
    if (batch <= 0 || iters <= 0 || !us_per_launch) return BH_ERR_INVALID;
    std::lock_guard<std::mutex> g(ctx->mu);
    AttnArgs a;
    rc = attn_args(ctx, ctx->stream, q, k, v, kv_f16, kv_rows, seq_off, seq_len, batch, n_q, n_kv, head_dim, max_len,
                   out, a);
    if (rc) return rc;
    const size_t kvb = (size_t)kv_rows * n_kv * head_dim * (kv_f16 ? 2 : 4);
    const int copies = (int)std::max<size_t>(1, std::min<size_t>(256, (rotate_bytes + 2 * kvb - 1) / std::max<size_t>(2 * kvb, 1)));
    std::vector<void*> kc(copies, nullptr), vc(copies, nullptr);
    kc[0] = (void*)k;
    vc[0] = (void*)v;
    for (int i = 1; i < copies && rc == BH_OK; ++i) {
        hipError_t e = hipMalloc(&kc[i], kvb);
        if (e == hipSuccess) e = hipMemcpy(kc[i], k, kvb, hipMemcpyDeviceToDevice);
        if (e == hipSuccess) e = hipMalloc(&vc[i], kvb);
        if (e == hipSuccess) e = hipMemcpy(vc[i], v, kvb, hipMemcpyDeviceToDevice);
        if (e != hipSuccess) rc = ctx->hip_fail(e, "KV copies");
    }
    if (rc == BH_OK)
        rc = time_graph(ctx, iters, [&](int i, hipStream_t st) {
            AttnArgs b = a;
            b.kv.k = kc[i % copies];
            b.kv.v = vc[i % copies];
            return launch_attention(b, st);
        }, us_per_launch);
    for (int i = 1; i < copies; ++i) {
        if (kc[i]) hipFree(kc[i]);
        if (vc[i]) hipFree(vc[i]);
    }
    return rc;
}

}  // extern "C"
