// k_probe.hip — HBM bandwidth probes (measurement only; no counterpart in the reference).
//
// The read probe streams a buffer larger than the 256 MB Infinity Cache with 16-byte
// non-temporal loads, U independent loads in flight per thread per round, grid-stride over the
// buffer, and folds what it read into one word per lane that is stored only if it equals a value
// the data cannot produce (so the loads stay but nothing is written). The copy probe moves the
// buffer into a second one with 16-byte non-temporal loads and stores. Together they give the
// achievable read and copy bandwidth that the GEMV and attention kernels are compared with.
#include "bh_internal.h"

namespace bh {
namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ void __launch_bounds__(256) k_read_probe(const u32x4* __restrict__ src, int64_t n16, uint32_t* sink) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    uint32_t acc = 0;
    for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < n16; i0 += stride * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u * stride;
            v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x9E3779B9u) sink[(int64_t)blockIdx.x * 256 + threadIdx.x] = acc;
}

template <int U>
__global__ void __launch_bounds__(256) k_copy_probe(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                    int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i0 = (int64_t)blockIdx.x * 256 + threadIdx.x; i0 < n16; i0 += stride * U) {
        u32x4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u * stride;
            v[u] = i < n16 ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t i = i0 + u * stride;
            if (i < n16) __builtin_nontemporal_store(v[u], dst + i);
        }
    }
}

// One link of a dependent launch chain: every workgroup reads the n floats the previous launch
// wrote (from another XCD's L2, as a decode kernel reads its producer's activations) and
// workgroup 0 writes the next n. Nothing else: its graph-replayed time per launch is the floor
// of a dependent kernel in the decode step.
__global__ void __launch_bounds__(256) k_chain_probe(const float* __restrict__ src, float* __restrict__ dst, int n) {
    float v = 0.f;
    for (int i = threadIdx.x; i < n; i += 256) v += src[i];
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < n; i += 256) dst[i] = src[i] + (v == 1.0e30f ? 1.f : 0.f);
}

// Grid-barrier probe: GB_PHASES phases in one launch, each the chain link's work (read what
// another workgroup wrote in the previous phase, write this workgroup's value) followed by a
// barrier over the whole grid (one arrival count incremented with release ordering, polled with
// acquire loads), as a persistent kernel would separate the steps of a decode layer. Its time per
// phase is what such a kernel would pay where the decode step pays a dependent launch. Every wait
// is bounded: a workgroup that polls GB_SPIN times stops and counts itself in *err (the host
// launches at most one workgroup per CU, so the grid is resident at once and no wait should end
// that way).
constexpr int GB_PHASES = 64;
constexpr int GB_SPIN = 1 << 21;
__global__ void __launch_bounds__(256) k_gridbar_probe(int* cnt, float* data, int* err) {
    const int nwg = gridDim.x, wg = blockIdx.x;
    __shared__ int s_bad;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    for (int p = 0; p < GB_PHASES; ++p) {
        if (threadIdx.x == 0) {
            const float v = p ? data[(p - 1) * nwg + (wg + 1) % nwg] : 0.f;
            data[p * nwg + wg] = v + 1.f;
            __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            int spins = 0;
            while (__hip_atomic_load(cnt, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) < (p + 1) * nwg) {
                if (++spins > GB_SPIN) {
                    s_bad = 1;
                    break;
                }
            }
        }
        __syncthreads();
        if (s_bad) {
            if (threadIdx.x == 0) atomicAdd(err, 1);
            return;
        }
    }
    // the last workgroup to finish polling zeroes the counts for the next launch (cnt[1] counts
    // the workgroups done with cnt[0])
    if (threadIdx.x == 0 && __hip_atomic_fetch_add(cnt + 1, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) == nwg - 1) {
        __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(cnt + 1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

}  // namespace

int gridbar_phases() { return GB_PHASES; }

// One grid-barrier probe launch over wgs workgroups (cnt: two counts, zero before the first
// launch and left at zero by every launch; data: GB_PHASES * wgs floats; err: the count of
// workgroups whose wait gave up). The caller keeps wgs at most the device's CU count.
hipError_t launch_gridbar_probe(int* cnt, float* data, int* err, int wgs, hipStream_t st) {
    if (!cnt || !data || !err || wgs <= 0) return hipErrorInvalidValue;
    launch_kernel(k_gridbar_probe, dim3((unsigned)wgs), dim3(256), 0, st, cnt, data, err);
    return hipGetLastError();
}

// One probe launch: copy = 0 reads src (sink holds wgs * 256 words), copy = 1 copies src to dst,
// copy = 2 is one link of the dependent chain (bytes / 4 floats from src to dst).
hipError_t launch_probe(int copy, const void* src, void* dst, int64_t bytes, int wgs, int unroll, uint32_t* sink,
                        hipStream_t st) {
    const int64_t n16 = bytes / 16;
    if (n16 <= 0 || wgs <= 0 || (copy && !dst) || (!copy && !sink)) return hipErrorInvalidValue;
    const dim3 g((unsigned)wgs), b(256);
    const u32x4* s = (const u32x4*)src;
    if (copy == 2) {
        launch_kernel(k_chain_probe, g, b, 0, st, (const float*)src, (float*)dst, (int)(bytes / 4));
    } else if (copy) {
        switch (unroll) {
            case 4: launch_kernel(k_copy_probe<4>, g, b, 0, st, s, (u32x4*)dst, n16); break;
            case 8: launch_kernel(k_copy_probe<8>, g, b, 0, st, s, (u32x4*)dst, n16); break;
            case 16: launch_kernel(k_copy_probe<16>, g, b, 0, st, s, (u32x4*)dst, n16); break;
            default: return hipErrorInvalidValue;
        }
    } else {
        switch (unroll) {
            case 4: launch_kernel(k_read_probe<4>, g, b, 0, st, s, n16, sink); break;
            case 8: launch_kernel(k_read_probe<8>, g, b, 0, st, s, n16, sink); break;
            case 16: launch_kernel(k_read_probe<16>, g, b, 0, st, s, n16, sink); break;
            default: return hipErrorInvalidValue;
        }
    }
    return hipGetLastError();
}

}  // namespace bh
