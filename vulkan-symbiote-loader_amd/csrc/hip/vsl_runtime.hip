// vsl_runtime.hip -- runtime half of the C ABI: errors, HBM arena, pinned packs, streams/events,
// copies, hipGraph helpers, synthetic weight fill, control-block reset.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>

#include "vsl_device.h"
#include "vsl_hip.h"
#include "vsl_internal.h"

static thread_local std::string g_last_error;

void vsl_set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

int vsl_hip_fail(hipError_t e, const char* what, const char* file, int line) {
    vsl_set_error("%s failed: %s (%s:%d)", what, hipGetErrorString(e), file, line);
    return VSL_E_HIP;
}

extern "C" const char* vsl_last_error(void) { return g_last_error.c_str(); }

extern "C" int vsl_device_count(int* n) {
    HIP_TRY(hipGetDeviceCount(n));
    return VSL_OK;
}

extern "C" int vsl_set_device(int device) {
    HIP_TRY(hipSetDevice(device));
    return VSL_OK;
}

extern "C" int vsl_device_sync(void) {
    HIP_TRY(hipDeviceSynchronize());
    return VSL_OK;
}

// ------------------------------------------------------------------------------------------
// Arena: one hipMalloc, first-fit over an offset-ordered free list, coalescing on free.
// ------------------------------------------------------------------------------------------
struct vsl_arena {
    int device = 0;
    char* base = nullptr;
    uint64_t size = 0;
    std::map<uint64_t, uint64_t> free_blocks;  // offset -> size
    std::map<uint64_t, uint64_t> used_blocks;  // offset -> size
    uint64_t used = 0;
    std::mutex mu;
};

extern "C" int vsl_arena_create(int device, uint64_t bytes, vsl_arena** out) {
    if (!out || bytes == 0) return vsl_invalid("vsl_arena_create: bad arguments");
    *out = nullptr;
    HIP_TRY(hipSetDevice(device));
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        vsl_set_error("vsl_arena_create: hipMalloc(%llu) failed: %s", (unsigned long long)bytes,
                      hipGetErrorString(e));
        return VSL_E_OOM;
    }
    vsl_arena* a = new vsl_arena();
    a->device = device;
    a->base = static_cast<char*>(p);
    a->size = bytes;
    a->free_blocks[0] = bytes;
    *out = a;
    return VSL_OK;
}

extern "C" int vsl_arena_destroy(vsl_arena* a) {
    if (!a) return VSL_OK;
    hipError_t e = hipFree(a->base);
    delete a;
    if (e != hipSuccess) return vsl_hip_fail(e, "hipFree", __FILE__, __LINE__);
    return VSL_OK;
}

extern "C" int vsl_arena_alloc(vsl_arena* a, uint64_t bytes, uint64_t align, void** dptr) {
    if (!a || !dptr) return vsl_invalid("vsl_arena_alloc: null argument");
    if (align < 256) align = 256;
    if (align & (align - 1)) return vsl_invalid("vsl_arena_alloc: alignment must be a power of two");
    if (bytes == 0) bytes = 1;
    bytes = (bytes + 255) & ~uint64_t(255);
    std::lock_guard<std::mutex> lk(a->mu);
    for (auto it = a->free_blocks.begin(); it != a->free_blocks.end(); ++it) {
        uint64_t off = it->first, sz = it->second;
        uint64_t aligned = (off + align - 1) & ~(align - 1);
        if (aligned + bytes > off + sz) continue;
        a->free_blocks.erase(it);
        if (aligned > off) a->free_blocks[off] = aligned - off;
        uint64_t end = aligned + bytes;
        if (end < off + sz) a->free_blocks[end] = off + sz - end;
        a->used_blocks[aligned] = bytes;
        a->used += bytes;
        *dptr = a->base + aligned;
        return VSL_OK;
    }
    vsl_set_error("vsl_arena_alloc: %llu bytes do not fit (used %llu of %llu)", (unsigned long long)bytes,
                  (unsigned long long)a->used, (unsigned long long)a->size);
    return VSL_E_OOM;
}

extern "C" int vsl_arena_free(vsl_arena* a, void* dptr) {
    if (!a || !dptr) return vsl_invalid("vsl_arena_free: null argument");
    std::lock_guard<std::mutex> lk(a->mu);
    uint64_t off = static_cast<uint64_t>(static_cast<char*>(dptr) - a->base);
    auto it = a->used_blocks.find(off);
    if (it == a->used_blocks.end()) return vsl_invalid("vsl_arena_free: pointer not allocated here");
    uint64_t sz = it->second;
    a->used_blocks.erase(it);
    a->used -= sz;
    auto nx = a->free_blocks.lower_bound(off);
    if (nx != a->free_blocks.end() && nx->first == off + sz) {
        sz += nx->second;
        nx = a->free_blocks.erase(nx);
    }
    if (nx != a->free_blocks.begin()) {
        auto pv = std::prev(nx);
        if (pv->first + pv->second == off) {
            pv->second += sz;
            return VSL_OK;
        }
    }
    a->free_blocks[off] = sz;
    return VSL_OK;
}

extern "C" int vsl_arena_reset(vsl_arena* a) {
    if (!a) return vsl_invalid("vsl_arena_reset: null arena");
    std::lock_guard<std::mutex> lk(a->mu);
    a->free_blocks.clear();
    a->used_blocks.clear();
    a->free_blocks[0] = a->size;
    a->used = 0;
    return VSL_OK;
}

extern "C" int vsl_arena_stats(const vsl_arena* ac, vsl_pool_stats* out) {
    if (!ac || !out) return vsl_invalid("vsl_arena_stats: null argument");
    vsl_arena* a = const_cast<vsl_arena*>(ac);
    std::lock_guard<std::mutex> lk(a->mu);
    out->total_size = a->size;
    out->used_size = a->used;
    out->free_size = a->size - a->used;
    out->allocation_count = static_cast<uint32_t>(a->used_blocks.size());
    uint64_t largest = 0;
    for (auto& kv : a->free_blocks) largest = kv.second > largest ? kv.second : largest;
    out->fragmentation_ratio =
        out->free_size ? 1.0f - static_cast<float>(static_cast<double>(largest) / out->free_size) : 0.0f;
    return VSL_OK;
}

extern "C" void* vsl_arena_base(const vsl_arena* a) { return a ? a->base : nullptr; }

// ------------------------------------------------------------------------------------------
// Pinned memory, streams, events, copies
// ------------------------------------------------------------------------------------------
extern "C" int vsl_host_pinned_alloc(uint64_t bytes, void** out) {
    if (!out) return vsl_invalid("vsl_host_pinned_alloc: null out");
    HIP_TRY(hipHostMalloc(out, bytes, hipHostMallocDefault));
    return VSL_OK;
}
extern "C" int vsl_host_pinned_free(void* p) {
    if (p) HIP_TRY(hipHostFree(p));
    return VSL_OK;
}
extern "C" int vsl_stream_create(void** stream) {
    hipStream_t s;
    HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return VSL_OK;
}
extern "C" int vsl_stream_destroy(void* stream) {
    if (stream) HIP_TRY(hipStreamDestroy(static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_stream_sync(void* stream) {
    HIP_TRY(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_event_create(void** ev) {
    hipEvent_t e;
    HIP_TRY(hipEventCreate(&e));
    *ev = e;
    return VSL_OK;
}
extern "C" int vsl_event_destroy(void* ev) {
    if (ev) HIP_TRY(hipEventDestroy(static_cast<hipEvent_t>(ev)));
    return VSL_OK;
}
extern "C" int vsl_event_record(void* ev, void* stream) {
    HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(ev), static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_event_sync(void* ev) {
    HIP_TRY(hipEventSynchronize(static_cast<hipEvent_t>(ev)));
    return VSL_OK;
}
extern "C" int vsl_stream_wait_event(void* stream, void* ev) {
    HIP_TRY(hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(ev), 0));
    return VSL_OK;
}
extern "C" int vsl_event_elapsed_ms(void* start, void* stop, float* ms) {
    HIP_TRY(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)));
    return VSL_OK;
}
extern "C" int vsl_pack_upload(void* dst_dev, const void* src_host, uint64_t bytes, void* stream, void* done_event) {
    if (!dst_dev || !src_host) return vsl_invalid("vsl_pack_upload: null pointer");
    HIP_TRY(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)));
    if (done_event) HIP_TRY(hipEventRecord(static_cast<hipEvent_t>(done_event), static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_copy_d2h(void* dst_host, const void* src_dev, uint64_t bytes, void* stream) {
    HIP_TRY(hipMemcpyAsync(dst_host, src_dev, bytes, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_copy_h2d(void* dst_dev, const void* src_host, uint64_t bytes, void* stream) {
    HIP_TRY(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_copy_d2d(void* dst_dev, const void* src_dev, uint64_t bytes, void* stream) {
    HIP_TRY(hipMemcpyAsync(dst_dev, src_dev, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
    return VSL_OK;
}
extern "C" int vsl_memset_d(void* dst_dev, int value, uint64_t bytes, void* stream) {
    HIP_TRY(hipMemsetAsync(dst_dev, value, bytes, static_cast<hipStream_t>(stream)));
    return VSL_OK;
}

// ------------------------------------------------------------------------------------------
// Synthetic weights: Philox4x32-10 + Box-Muller (fp64), same stream as the host generator.
// ------------------------------------------------------------------------------------------
static uint64_t host_hash_string(const char* s) {  // Utils.cpp:9-16, its own offset basis
    uint64_t h = 1469598103934665603ULL;
    for (const unsigned char* p = reinterpret_cast<const unsigned char*>(s); *p; ++p) {
        h ^= *p;
        h *= 1099511628211ULL;
    }
    return h;
}

uint64_t vsl_derive_key(uint64_t seed, const char* name) {
    return host_hash_string(name) ^ (seed * 0x9E3779B97F4A7C15ULL);
}

template <typename T>
__global__ void k_fill_normal(T* out, uint64_t n, uint32_t k0, uint32_t k1, float mean, float stddev) {
    const uint64_t nblk = (n + 3) / 4;
    for (uint64_t b = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; b < nblk;
         b += (uint64_t)gridDim.x * blockDim.x) {
        uint32_t c[4] = {(uint32_t)b, (uint32_t)(b >> 32), 0u, 0u};
        philox4x32_10(c, k0, k1);
        double z[4];
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            double u1 = ((double)c[2 * p] + 1.0) * (1.0 / 4294967296.0);
            double u2 = (double)c[2 * p + 1] * (1.0 / 4294967296.0);
            double r = sqrt(-2.0 * log(u1));
            double t = 6.283185307179586476925286766559 * u2;
            z[2 * p] = r * cos(t);
            z[2 * p + 1] = r * sin(t);
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint64_t e = b * 4 + j;
            if (e < n) {
                float v = (float)((double)mean + (double)stddev * z[j]);
                // The value is defined as double -> float -> output type (two roundings, as the host
                // generator does); the empty asm keeps the compiler from fusing them into one.
                asm volatile("" : "+v"(v));
                store_elem(out + e, v);
            }
        }
    }
}

extern "C" int vsl_fill_normal(void* dst, int dtype, uint64_t n, uint64_t seed, const char* name, float mean,
                               float stddev, void* stream) {
    if (!dst || !name) return vsl_invalid("vsl_fill_normal: null argument");
    if (n == 0) return VSL_OK;
    uint64_t key = vsl_derive_key(seed, name);
    uint64_t nblk = (n + 3) / 4;
    uint32_t grid = (uint32_t)((nblk + 255) / 256 < 65536 ? (nblk + 255) / 256 : 65536);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VSL_DT_F16)
        k_fill_normal<vsl_half><<<grid, 256, 0, s>>>(static_cast<vsl_half*>(dst), n, (uint32_t)key,
                                                    (uint32_t)(key >> 32), mean, stddev);
    else if (dtype == VSL_DT_F32)
        k_fill_normal<float><<<grid, 256, 0, s>>>(static_cast<float*>(dst), n, (uint32_t)key,
                                                 (uint32_t)(key >> 32), mean, stddev);
    else
        return vsl_unsupported("vsl_fill_normal: dtype %d", dtype);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

template <typename T>
__global__ void k_fill_const(T* out, uint64_t n, float v) {
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        store_elem(out + i, v);
}

extern "C" int vsl_fill_const(void* dst, int dtype, uint64_t n, float value, void* stream) {
    if (!dst) return vsl_invalid("vsl_fill_const: null argument");
    if (n == 0) return VSL_OK;
    uint32_t grid = (uint32_t)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == VSL_DT_F16)
        k_fill_const<vsl_half><<<grid, 256, 0, s>>>(static_cast<vsl_half*>(dst), n, value);
    else if (dtype == VSL_DT_F32)
        k_fill_const<float><<<grid, 256, 0, s>>>(static_cast<float*>(dst), n, value);
    else
        return vsl_unsupported("vsl_fill_const: dtype %d", dtype);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// ------------------------------------------------------------------------------------------
// Control block reset: a one-thread kernel (no hipMemsetAsync, so it is safe inside graphs).
// ------------------------------------------------------------------------------------------
__global__ void k_ctrl_reset(vsl_ctrl* c, uint32_t pos, uint32_t max_steps, uint32_t stop, uint32_t cap) {
    c->pos = pos;
    c->step = 0;
    c->done = max_steps == 0 ? 1u : 0u;
    c->stop_on_eos = stop;
    c->max_steps = max_steps;
    c->token = 0;
    c->capacity = cap;
    c->error = 0;
}

extern "C" int vsl_ctrl_reset(vsl_ctrl* ctrl, uint32_t pos, uint32_t max_steps, uint32_t stop_on_eos,
                              uint32_t capacity, void* stream) {
    if (!ctrl) return vsl_invalid("vsl_ctrl_reset: null ctrl");
    k_ctrl_reset<<<1, 1, 0, static_cast<hipStream_t>(stream)>>>(ctrl, pos, max_steps, stop_on_eos, capacity);
    HIP_TRY(hipGetLastError());
    return VSL_OK;
}

// ------------------------------------------------------------------------------------------
// hipGraph helpers
// ------------------------------------------------------------------------------------------
struct vsl_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

extern "C" int vsl_graph_begin(void* stream) {
    HIP_TRY(hipStreamBeginCapture(static_cast<hipStream_t>(stream), hipStreamCaptureModeThreadLocal));
    return VSL_OK;
}

extern "C" int vsl_graph_end(void* stream, vsl_graph** out) {
    if (!out) return vsl_invalid("vsl_graph_end: null out");
    vsl_graph* g = new vsl_graph();
    hipError_t e = hipStreamEndCapture(static_cast<hipStream_t>(stream), &g->graph);
    if (e != hipSuccess) {
        delete g;
        return vsl_hip_fail(e, "hipStreamEndCapture", __FILE__, __LINE__);
    }
    e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(g->graph);
        delete g;
        return vsl_hip_fail(e, "hipGraphInstantiate", __FILE__, __LINE__);
    }
    *out = g;
    return VSL_OK;
}

extern "C" int vsl_graph_launch(vsl_graph* g, void* stream) {
    if (!g) return vsl_invalid("vsl_graph_launch: null graph");
    HIP_TRY(hipGraphLaunch(g->exec, static_cast<hipStream_t>(stream)));
    return VSL_OK;
}

extern "C" int vsl_graph_destroy(vsl_graph* g) {
    if (!g) return VSL_OK;
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    delete g;
    return VSL_OK;
}
