// bh_ctx.h — the context object behind bh_ctx* (one per device).
#pragma once

#include <list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "bh_internal.h"

struct bh_ctx {
    int device = 0;
    int n_cu = 0;
    hipStream_t stream = nullptr;
    std::mutex mu;
    std::string err;

    // Weight registry: "model:layer" -> device weight, least recently used first in `lru`.
    struct Entry {
        bh::DevWeight w;
        std::list<std::string>::iterator lru_it;
    };
    std::unordered_map<std::string, Entry> reg;
    std::list<std::string> lru;
    size_t cap = (size_t)64 << 30;  // 64 GiB of the 288 GB HBM by default
    size_t used = 0;

    // Staging for the host-buffer GEMV mirrors.
    void* d_x = nullptr;
    size_t x_cap = 0;
    void* d_y = nullptr;
    size_t y_cap = 0;
    // Split scratch of bh_attn_decode, one per stream it is called on (calls on one stream run in
    // order, so they may share it): partials and split-merge counters (zero when idle). A buffer
    // that grows is retired, not freed, while the context lives, since a graph captured from an
    // earlier call may still write it.
    struct AttnScratch {
        void* part = nullptr;
        size_t part_bytes = 0;
        int32_t* cnt = nullptr;
        int cnt_len = 0;
    };
    std::unordered_map<hipStream_t, AttnScratch> attn_scratch;
    std::vector<void*> retired;
    // This device's copy of the file-scope scratch of bh_attn_decode_noalloc (bh_api.cpp),
    // resolved at bh_init.
    uint8_t* noalloc_scratch = nullptr;
    std::unordered_map<std::string, void*> rope_tabs;
    // K-split scratch of the GEMVs launched on the context's own stream (split sums and arrival
    // counters, zero when idle); calls on other streams run unsplit so they never share it.
    float* split_part = nullptr;
    int32_t* split_cnt = nullptr;
    // Limb records of a batch-1 activation row (XL_TMP_CHUNKS chunks) for the GEMVs launched on
    // the context's own stream, under the same rule.
    uint32_t* xl_tmp = nullptr;

    // Fault injection (bh_debug_inject_fault).
    int inj_op = 0, inj_status = 0, inj_count = 0;

    int fail(int status, const std::string& msg);
    int hip_fail(hipError_t e, const char* what);
    bool injected(int op, int* status);
    int ensure_scratch(size_t xb, size_t yb);
    // Point a's split scratch at the context's when `st` is the context's stream.
    void split_scratch(bh::GemvArgs& a, hipStream_t st);
    void touch(const std::string& key);
    void enforce_limits(size_t new_bytes);
    void clear_registry();
    const float2* rope_tab(int hd, float theta, int max_pos);
};

namespace bh {
void free_weight(DevWeight& w);
int alloc_weight(bh_ctx* ctx, int fmt, int64_t n, int64_t k, DevWeight& w);
bool host_sizes(int fmt, int64_t n, int64_t k, size_t* qb, size_t* sb);
int upload_rows(bh_ctx* ctx, DevWeight& dst, int64_t row0, int64_t n, const void* q, size_t q_bytes, const void* s,
                size_t s_bytes);
}  // namespace bh
