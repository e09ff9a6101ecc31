// Lifecycle, HBM arena, host<->device copies, errors, timing table and launch
// capture of libnnc_hip.so (declared in include/nnc_hip.h).
//
// The reference runtime owns no state: generated tensors.c places tensors in
// a static host pool (codegen/x86_emitters/tensors.py:589-600). Here the pool
// becomes one hipMalloc'd arena and this file owns the device, the stream and
// a grow-only workspace for split-K partials.
#include <stdarg.h>
#include <string.h>

#include <atomic>
#include <string>
#include <vector>

#include "common.h"

namespace nnc {

static Context g_ctx;
static std::atomic<int> g_last_error{0};
static char g_last_msg[512] = "";

Context& ctx() { return g_ctx; }

static bool sync_all(const char* who) {
    for (int k = 0; k < kStreams; ++k)
        if (g_ctx.streams[k] && !hip_ok(hipStreamSynchronize(g_ctx.streams[k]), who, "hipStreamSynchronize"))
            return false;
    return true;
}

void fail(int code, const char* who, const char* fmt, ...) {
    char body[384];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(body, sizeof body, fmt, ap);
    va_end(ap);
    snprintf(g_last_msg, sizeof g_last_msg, "%s: %s", who, body);
    g_last_error.store(code);
    fprintf(stderr, "%s\n", g_last_msg);
    fflush(stderr);
}

bool hip_ok(hipError_t e, const char* who, const char* what) {
    if (e == hipSuccess) return true;
    fail(NNC_HIP_EDEVICE, who, "%s failed: %s", what, hipGetErrorString(e));
    return false;
}

bool ready(const char* who) {
    if (g_ctx.stream) return true;
    fail(NNC_HIP_ESTATE, who, "nnc_hip_init() has not been called");
    return false;
}

// Default workspace: stream-K partials of a full persistent grid (2 slots of
// 128x128 floats for 512 workgroups = 64 MiB) with room; grows outside capture.
static const size_t kDefaultWorkspace = 128u << 20;

// Scratch buffers replaced by larger ones stay allocated until shutdown: a
// hipGraph captured earlier still holds their addresses.
static std::vector<void*> g_retired;
static void retire(void* p) {
    if (p) g_retired.push_back(p);
}

float* workspace(size_t bytes) {
    Context& c = g_ctx;
    const int k = c.cur;
    if (bytes <= c.workspace_bytes[k]) return c.workspace[k];
    if (c.capturing) return nullptr;
    if (!hip_ok(hipStreamSynchronize(c.stream), "workspace", "hipStreamSynchronize")) return nullptr;
    retire(c.workspace[k]);
    c.workspace[k] = nullptr;
    c.workspace_bytes[k] = 0;
    size_t want = bytes < kDefaultWorkspace ? kDefaultWorkspace : bytes;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, want), "workspace", "hipMalloc")) return nullptr;
    c.workspace[k] = static_cast<float*>(p);
    c.workspace_bytes[k] = want;
    return c.workspace[k];
}

size_t workspace_capacity() { return g_ctx.workspace_bytes[g_ctx.cur]; }

float* repack_buffer(size_t bytes) {
    Context& c = g_ctx;
    const int k = c.cur;
    if (bytes <= c.repack_bytes[k]) return c.repack[k];
    if (c.capturing) return nullptr;
    if (!hip_ok(hipStreamSynchronize(c.stream), "repack_buffer", "hipStreamSynchronize")) return nullptr;
    retire(c.repack[k]);
    c.repack[k] = nullptr;
    c.repack_bytes[k] = 0;
    const size_t want = bytes < (16u << 20) ? (16u << 20) : bytes;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, want), "repack_buffer", "hipMalloc")) return nullptr;
    c.repack[k] = static_cast<float*>(p);
    c.repack_bytes[k] = want;
    return c.repack[k];
}

static const size_t kDefaultCounters = 1u << 16;

int* tile_counters(size_t n) {
    Context& c = g_ctx;
    const int k = c.cur;
    if (n <= c.counters_n[k]) return c.counters[k];
    if (c.capturing) return nullptr;
    if (!hip_ok(hipStreamSynchronize(c.stream), "tile_counters", "hipStreamSynchronize")) return nullptr;
    retire(c.counters[k]);
    c.counters[k] = nullptr;
    c.counters_n[k] = 0;
    const size_t want = n < kDefaultCounters ? kDefaultCounters : n;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, want * sizeof(int)), "tile_counters", "hipMalloc")) return nullptr;
    if (!hip_ok(hipMemsetAsync(p, 0, want * sizeof(int), c.stream), "tile_counters", "hipMemsetAsync") ||
        !hip_ok(hipStreamSynchronize(c.stream), "tile_counters", "hipStreamSynchronize")) {
        (void)hipFree(p);
        return nullptr;
    }
    c.counters[k] = static_cast<int*>(p);
    c.counters_n[k] = want;
    return c.counters[k];
}

// ---------------------------------------------------------------------------
// per-kernel timing
// ---------------------------------------------------------------------------
struct Pending {
    std::string name;
    double flops, bytes;
    hipEvent_t start, stop;
};
struct Stat {
    std::string name;
    int64_t launches = 0;
    double ms = 0.0, flops = 0.0, bytes = 0.0;
};
static double g_next_flops = 0.0, g_next_bytes = 0.0;

void set_work(double flops, double bytes) {
    g_next_flops = flops;
    g_next_bytes = bytes;
}
static std::vector<Pending> g_pending;
static std::vector<hipEvent_t> g_event_pool;
static std::vector<Stat> g_stats;

static hipEvent_t take_event() {
    if (!g_event_pool.empty()) {
        hipEvent_t e = g_event_pool.back();
        g_event_pool.pop_back();
        return e;
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

TimedScope::TimedScope(const char* n) : name(n), flops(g_next_flops), bytes(g_next_bytes) {
    g_next_flops = g_next_bytes = 0.0;
    if (!g_ctx.profiling || g_ctx.capturing) return;
    start = take_event();
    stop = take_event();
    (void)hipEventRecord(start, g_ctx.stream);
}

TimedScope::~TimedScope() {
    if (!start) return;
    (void)hipEventRecord(stop, g_ctx.stream);
    g_pending.push_back({name, flops, bytes, start, stop});
}

static void resolve_pending() {
    if (g_pending.empty()) return;
    (void)sync_all("profile");
    for (auto& p : g_pending) {
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, p.start, p.stop);
        Stat* s = nullptr;
        for (auto& st : g_stats)
            if (st.name == p.name) { s = &st; break; }
        if (!s) {
            g_stats.push_back(Stat{p.name, 0, 0.0, 0.0, 0.0});
            s = &g_stats.back();
        }
        s->launches += 1;
        s->ms += ms;
        s->flops += p.flops;
        s->bytes += p.bytes;
        g_event_pool.push_back(p.start);
        g_event_pool.push_back(p.stop);
    }
    g_pending.clear();
}

}  // namespace nnc

using namespace nnc;

extern "C" {

int nnc_hip_init(int device) {
    Context& c = g_ctx;
    if (c.stream && c.device == device) return NNC_HIP_OK;
    if (c.stream) nnc_hip_shutdown();
    int count = 0;
    if (!hip_ok(hipGetDeviceCount(&count), "nnc_hip_init", "hipGetDeviceCount"))
        return NNC_HIP_EDEVICE;
    if (device < 0 || device >= count) {
        fail(NNC_HIP_EINVAL, "nnc_hip_init", "device %d out of range (%d devices)", device, count);
        return NNC_HIP_EINVAL;
    }
    if (!hip_ok(hipSetDevice(device), "nnc_hip_init", "hipSetDevice")) return NNC_HIP_EDEVICE;
    hipDeviceProp_t prop;
    if (hip_ok(hipGetDeviceProperties(&prop, device), "nnc_hip_init", "hipGetDeviceProperties"))
        c.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    // default priority for every stream (streams of different priorities
    // are not used anywhere in this library)
    for (int k = 0; k < kStreams; ++k)
        if (!hip_ok(hipStreamCreateWithFlags(&c.streams[k], hipStreamNonBlocking), "nnc_hip_init",
                    "hipStreamCreate"))
            return NNC_HIP_EDEVICE;
    if (!hip_ok(hipEventCreateWithFlags(&c.fork_ev, hipEventDisableTiming), "nnc_hip_init", "hipEventCreate") ||
        !hip_ok(hipEventCreateWithFlags(&c.join_ev, hipEventDisableTiming), "nnc_hip_init", "hipEventCreate"))
        return NNC_HIP_EDEVICE;
    c.cur = 0;
    c.stream = c.streams[0];
    c.device = device;
    for (int k = 0; k < kStreams; ++k) {
        c.cur = k;
        c.stream = c.streams[k];
        if (!workspace(kDefaultWorkspace)) return NNC_HIP_ENOMEM;
        if (!tile_counters(kDefaultCounters)) return NNC_HIP_ENOMEM;
    }
    c.cur = 0;
    c.stream = c.streams[0];
    return NNC_HIP_OK;
}

void nnc_hip_shutdown(void) {
    Context& c = g_ctx;
    if (!c.stream) return;
    for (int k = 0; k < kStreams; ++k)
        if (c.streams[k]) (void)hipStreamSynchronize(c.streams[k]);
    nnc_hip_graph_destroy();
    for (auto& p : g_pending) {
        (void)hipEventDestroy(p.start);
        (void)hipEventDestroy(p.stop);
    }
    g_pending.clear();
    for (auto e : g_event_pool) (void)hipEventDestroy(e);
    g_event_pool.clear();
    if (c.arena) (void)hipFree(c.arena);
    if (c.spill) (void)hipHostFree(c.spill);
    for (int k = 0; k < kStreams; ++k) {
        if (c.workspace[k]) (void)hipFree(c.workspace[k]);
        if (c.counters[k]) (void)hipFree(c.counters[k]);
        if (c.repack[k]) (void)hipFree(c.repack[k]);
    }
    for (void* p : g_retired) (void)hipFree(p);
    g_retired.clear();
    if (c.fork_ev) (void)hipEventDestroy(c.fork_ev);
    if (c.join_ev) (void)hipEventDestroy(c.join_ev);
    for (int k = 0; k < kStreams; ++k)
        if (c.streams[k]) (void)hipStreamDestroy(c.streams[k]);
    g_ctx = Context{};
}

int nnc_hip_arena_reserve(size_t bytes) {
    if (!ready("nnc_hip_arena_reserve")) return NNC_HIP_ESTATE;
    Context& c = g_ctx;
    if (c.arena && bytes <= c.arena_bytes) return NNC_HIP_OK;
    (void)sync_all("nnc_hip_arena_reserve");
    if (c.arena) (void)hipFree(c.arena);
    c.arena = nullptr;
    c.arena_bytes = 0;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 256), "nnc_hip_arena_reserve", "hipMalloc"))
        return NNC_HIP_ENOMEM;
    c.arena = static_cast<char*>(p);
    c.arena_bytes = bytes;
    return NNC_HIP_OK;
}

void* nnc_hip_arena_base(void) { return g_ctx.arena; }
size_t nnc_hip_arena_size(void) { return g_ctx.arena_bytes; }

int nnc_hip_bind(Tensor* t, size_t offset) {
    if (!t) {
        fail(NNC_HIP_EINVAL, "nnc_hip_bind", "NULL tensor");
        return NNC_HIP_EINVAL;
    }
    if (!g_ctx.arena) {
        fail(NNC_HIP_ESTATE, "nnc_hip_bind", "no arena reserved");
        return NNC_HIP_ESTATE;
    }
    if ((offset & 15u) != 0 || offset + (size_t)t->nbytes > g_ctx.arena_bytes) {
        fail(NNC_HIP_EINVAL, "nnc_hip_bind", "offset %zu + %lld bytes outside arena of %zu (or misaligned)",
             offset, (long long)t->nbytes, g_ctx.arena_bytes);
        return NNC_HIP_EINVAL;
    }
    t->data = g_ctx.arena + offset;
    return NNC_HIP_OK;
}

int nnc_hip_spill_reserve(size_t bytes) {
    const char* who = "nnc_hip_spill_reserve";
    if (!ready(who)) return NNC_HIP_ESTATE;
    Context& c = g_ctx;
    if (c.spill && bytes <= c.spill_bytes) return NNC_HIP_OK;
    if (c.capturing) {
        fail(NNC_HIP_ESTATE, who, "cannot allocate the spill pool during graph capture");
        return NNC_HIP_ESTATE;
    }
    (void)sync_all(who);
    if (c.spill) (void)hipHostFree(c.spill);
    c.spill = nullptr;
    c.spill_bytes = 0;
    void* p = nullptr;
    if (!hip_ok(hipHostMalloc(&p, bytes ? bytes : 256, hipHostMallocDefault), who, "hipHostMalloc"))
        return NNC_HIP_ENOMEM;
    c.spill = static_cast<char*>(p);
    c.spill_bytes = bytes;
    return NNC_HIP_OK;
}

void* nnc_hip_spill_base(void) { return g_ctx.spill; }

int nnc_hip_bind_spill(Tensor* t, size_t offset) {
    const char* who = "nnc_hip_bind_spill";
    if (!t) {
        fail(NNC_HIP_EINVAL, who, "NULL tensor");
        return NNC_HIP_EINVAL;
    }
    if (!g_ctx.spill) {
        fail(NNC_HIP_ESTATE, who, "no spill pool reserved");
        return NNC_HIP_ESTATE;
    }
    if ((offset & 15u) != 0 || offset + (size_t)t->nbytes > g_ctx.spill_bytes) {
        fail(NNC_HIP_EINVAL, who, "offset %zu + %lld bytes outside the spill pool of %zu (or misaligned)", offset,
             (long long)t->nbytes, g_ctx.spill_bytes);
        return NNC_HIP_EINVAL;
    }
    t->data = g_ctx.spill + offset;
    return NNC_HIP_OK;
}

// Spill (HBM -> pinned host) or reload (pinned host -> HBM): one async copy
// on the selected stream, so it orders with the kernels around it and is
// recorded as a memcpy node under graph capture.
void nnc_hip_transfer(Tensor* src, Tensor* dst) {
    const char* who = "nnc_hip_transfer";
    if (!ready(who)) return;
    if (!src || !dst || !src->data || !dst->data) return fail(NNC_HIP_EINVAL, who, "NULL tensor or data pointer");
    if (src->nbytes != dst->nbytes)
        return fail(NNC_HIP_EINVAL, who, "source has %lld bytes, destination %lld", (long long)src->nbytes,
                    (long long)dst->nbytes);
    if (src->nbytes <= 0 || src->data == dst->data) return;
    set_work(0.0, (double)src->nbytes);
    TimedScope scope(who);
    hip_ok(hipMemcpyAsync(dst->data, src->data, (size_t)src->nbytes, hipMemcpyDefault, g_ctx.stream), who,
           "hipMemcpyAsync");
}

void* nnc_hip_malloc(size_t bytes) {
    if (!ready("nnc_hip_malloc")) return nullptr;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 16), "nnc_hip_malloc", "hipMalloc")) return nullptr;
    return p;
}

void nnc_hip_free(void* ptr) {
    if (!ptr || !g_ctx.stream) return;
    (void)sync_all("nnc_hip_free");
    (void)hipFree(ptr);
}

void* nnc_hip_host_malloc(size_t bytes) {
    if (!ready("nnc_hip_host_malloc")) return nullptr;
    void* p = nullptr;
    if (!hip_ok(hipHostMalloc(&p, bytes ? bytes : 16, hipHostMallocDefault), "nnc_hip_host_malloc",
                "hipHostMalloc"))
        return nullptr;
    return p;
}

void nnc_hip_host_free(void* ptr) {
    if (!ptr || !g_ctx.stream) return;
    (void)sync_all("nnc_hip_host_free");
    (void)hipHostFree(ptr);
}

int nnc_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (!ready("nnc_hip_memcpy_h2d")) return NNC_HIP_ESTATE;
    if (!bytes) return NNC_HIP_OK;
    if (!sync_all("nnc_hip_memcpy_h2d") ||
        !hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_ctx.streams[0]),
                "nnc_hip_memcpy_h2d", "hipMemcpyAsync") ||
        !hip_ok(hipStreamSynchronize(g_ctx.streams[0]), "nnc_hip_memcpy_h2d", "hipStreamSynchronize"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (!ready("nnc_hip_memcpy_d2h")) return NNC_HIP_ESTATE;
    if (!bytes) return NNC_HIP_OK;
    if (!sync_all("nnc_hip_memcpy_d2h") ||
        !hip_ok(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_ctx.streams[0]),
                "nnc_hip_memcpy_d2h", "hipMemcpyAsync") ||
        !hip_ok(hipStreamSynchronize(g_ctx.streams[0]), "nnc_hip_memcpy_d2h", "hipStreamSynchronize"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_upload(Tensor* t, const void* host_src) {
    if (!t || !t->data || !host_src) {
        fail(NNC_HIP_EINVAL, "nnc_hip_upload", "NULL tensor, data or source");
        return NNC_HIP_EINVAL;
    }
    return nnc_hip_memcpy_h2d(t->data, host_src, (size_t)t->nbytes);
}

int nnc_hip_download(const Tensor* t, void* host_dst) {
    if (!t || !t->data || !host_dst) {
        fail(NNC_HIP_EINVAL, "nnc_hip_download", "NULL tensor, data or destination");
        return NNC_HIP_EINVAL;
    }
    return nnc_hip_memcpy_d2h(host_dst, t->data, (size_t)t->nbytes);
}

int nnc_hip_sync(void) {
    if (!ready("nnc_hip_sync")) return NNC_HIP_ESTATE;
    for (int k = 0; k < kStreams; ++k)
        if (!hip_ok(hipStreamSynchronize(g_ctx.streams[k]), "nnc_hip_sync", "hipStreamSynchronize"))
            return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

void* nnc_hip_stream(void) { return g_ctx.streams[0]; }

int nnc_hip_stream_fork(void) {
    if (!ready("nnc_hip_stream_fork")) return NNC_HIP_ESTATE;
    Context& c = g_ctx;
    if (!hip_ok(hipEventRecord(c.fork_ev, c.streams[0]), "nnc_hip_stream_fork", "hipEventRecord") ||
        !hip_ok(hipStreamWaitEvent(c.streams[1], c.fork_ev, 0), "nnc_hip_stream_fork", "hipStreamWaitEvent"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_stream_select(int slot) {
    if (!ready("nnc_hip_stream_select")) return NNC_HIP_ESTATE;
    if (slot < 0 || slot >= kStreams) {
        fail(NNC_HIP_EINVAL, "nnc_hip_stream_select", "stream %d out of range (0..%d)", slot, kStreams - 1);
        return NNC_HIP_EINVAL;
    }
    g_ctx.cur = slot;
    g_ctx.stream = g_ctx.streams[slot];
    return NNC_HIP_OK;
}

int nnc_hip_stream_join(void) {
    if (!ready("nnc_hip_stream_join")) return NNC_HIP_ESTATE;
    Context& c = g_ctx;
    if (!hip_ok(hipEventRecord(c.join_ev, c.streams[1]), "nnc_hip_stream_join", "hipEventRecord") ||
        !hip_ok(hipStreamWaitEvent(c.streams[0], c.join_ev, 0), "nnc_hip_stream_join", "hipStreamWaitEvent"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_last_error(void) { return g_last_error.load(); }
const char* nnc_hip_last_error_message(void) { return g_last_msg; }
void nnc_hip_clear_error(void) {
    g_last_error.store(0);
    g_last_msg[0] = '\0';
}

void nnc_hip_profile_enable(int on) {
    if (!on) resolve_pending();
    g_ctx.profiling = on != 0;
}

void nnc_hip_profile_reset(void) {
    resolve_pending();
    g_stats.clear();
}

int nnc_hip_profile_count(void) {
    resolve_pending();
    return (int)g_stats.size();
}

int nnc_hip_profile_entry(int i, char* name, int cap, int64_t* launches, double* total_ms) {
    resolve_pending();
    if (i < 0 || i >= (int)g_stats.size()) return NNC_HIP_EINVAL;
    if (name && cap > 0) {
        strncpy(name, g_stats[i].name.c_str(), (size_t)cap - 1);
        name[cap - 1] = '\0';
    }
    if (launches) *launches = g_stats[i].launches;
    if (total_ms) *total_ms = g_stats[i].ms;
    return NNC_HIP_OK;
}

int nnc_hip_profile_work(int i, double* flops, double* bytes) {
    resolve_pending();
    if (i < 0 || i >= (int)g_stats.size()) return NNC_HIP_EINVAL;
    if (flops) *flops = g_stats[i].flops;
    if (bytes) *bytes = g_stats[i].bytes;
    return NNC_HIP_OK;
}

int nnc_hip_debug_dump(const Tensor* t, const char* name, int node_idx, void* file) {
    const char* fn = "nnc_hip_debug_dump";
    if (!ready(fn)) return NNC_HIP_ESTATE;
    if (g_ctx.capturing) {
        fail(NNC_HIP_ESTATE, fn, "cannot dump while a graph is being captured");
        return NNC_HIP_ESTATE;
    }
    if (!t || !t->data || !name || (t->ndim > 0 && !t->shape) || t->nbytes < 0) {
        fail(NNC_HIP_EINVAL, fn, "NULL tensor, data, shape or name");
        return NNC_HIP_EINVAL;
    }
    int64_t n = 1;
    for (int d = 0; d < t->ndim; ++d) n *= t->shape[d];
    size_t esize = 4;
    switch (t->dtype) {
        case NNC_DTYPE_BOOL: case NNC_DTYPE_INT8: case NNC_DTYPE_UINT8: esize = 1; break;
        case NNC_DTYPE_FLOAT16: esize = 2; break;
        case NNC_DTYPE_INT64: esize = 8; break;
        default: esize = 4; break;
    }
    if (n < 0 || (size_t)n * esize > (size_t)t->nbytes) n = (int64_t)((size_t)t->nbytes / esize);
    std::vector<unsigned char> host((size_t)t->nbytes);
    if (!host.empty() && nnc_hip_memcpy_d2h(host.data(), t->data, host.size()) != NNC_HIP_OK) return NNC_HIP_EDEVICE;
    FILE* f = file ? static_cast<FILE*>(file) : stdout;
    fprintf(f, "DEBUG_TENSOR_START %s %d\n", name, node_idx);
    fprintf(f, "SHAPE %d\n", t->ndim);
    for (int d = 0; d < t->ndim; ++d) fprintf(f, "DIM %d %d\n", d, (int)t->shape[d]);
    fprintf(f, "DATA_START\n");
    const unsigned char* b = host.data();
    for (int64_t i = 0; i < n; ++i) {
        float v;
        switch (t->dtype) {
            case NNC_DTYPE_BOOL: case NNC_DTYPE_UINT8: v = (float)b[i]; break;
            case NNC_DTYPE_INT8: v = (float)reinterpret_cast<const int8_t*>(b)[i]; break;
            case NNC_DTYPE_INT32: v = (float)reinterpret_cast<const int32_t*>(b)[i]; break;
            case NNC_DTYPE_INT64: v = (float)reinterpret_cast<const int64_t*>(b)[i]; break;
            case NNC_DTYPE_FLOAT16: v = (float)reinterpret_cast<const _Float16*>(b)[i]; break;
            default: v = reinterpret_cast<const float*>(b)[i]; break;
        }
        fprintf(f, "%f\n", (double)v);
    }
    fprintf(f, "DATA_END\n");
    fprintf(f, "DEBUG_TENSOR_END %s\n\n", name);
    return ferror(f) ? NNC_HIP_EINVAL : NNC_HIP_OK;
}

int nnc_hip_graph_begin(void) {
    if (!ready("nnc_hip_graph_begin")) return NNC_HIP_ESTATE;
    nnc_hip_graph_destroy();
    resolve_pending();
    if (g_ctx.cur != 0) {
        fail(NNC_HIP_ESTATE, "nnc_hip_graph_begin", "capture starts on stream 0 (stream %d selected)", g_ctx.cur);
        return NNC_HIP_ESTATE;
    }
    if (!hip_ok(hipStreamBeginCapture(g_ctx.streams[0], hipStreamCaptureModeRelaxed),
                "nnc_hip_graph_begin", "hipStreamBeginCapture"))
        return NNC_HIP_EDEVICE;
    g_ctx.capturing = true;
    return NNC_HIP_OK;
}

int nnc_hip_graph_end(void) {
    if (!ready("nnc_hip_graph_end")) return NNC_HIP_ESTATE;
    if (!g_ctx.capturing) {
        fail(NNC_HIP_ESTATE, "nnc_hip_graph_end", "no capture in progress");
        return NNC_HIP_ESTATE;
    }
    g_ctx.capturing = false;
    hipGraph_t g = nullptr;
    g_ctx.cur = 0;
    g_ctx.stream = g_ctx.streams[0];
    if (!hip_ok(hipStreamEndCapture(g_ctx.streams[0], &g), "nnc_hip_graph_end", "hipStreamEndCapture"))
        return NNC_HIP_EDEVICE;
    g_ctx.graph = g;
    if (!hip_ok(hipGraphInstantiate(&g_ctx.graph_exec, g, nullptr, nullptr, 0), "nnc_hip_graph_end",
                "hipGraphInstantiate"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_graph_launch(void) {
    if (!ready("nnc_hip_graph_launch")) return NNC_HIP_ESTATE;
    if (!g_ctx.graph_exec) {
        fail(NNC_HIP_ESTATE, "nnc_hip_graph_launch", "no captured graph");
        return NNC_HIP_ESTATE;
    }
    TimedScope scope("graph");
    return hip_ok(hipGraphLaunch(g_ctx.graph_exec, g_ctx.streams[0]), "nnc_hip_graph_launch",
                  "hipGraphLaunch")
               ? NNC_HIP_OK
               : NNC_HIP_EDEVICE;
}

void nnc_hip_graph_destroy(void) {
    if (g_ctx.graph_exec) (void)hipGraphExecDestroy(g_ctx.graph_exec);
    if (g_ctx.graph) (void)hipGraphDestroy(g_ctx.graph);
    g_ctx.graph_exec = nullptr;
    g_ctx.graph = nullptr;
}

}  // extern "C"
