// Lifecycle, HBM arena, host<->device copies, errors, timing table and launch
// capture of libnnc_hip.so (declared in include/nnc_hip.h).
//
// The reference runtime owns no state: generated tensors.c places tensors in
// a static host pool (codegen/x86_emitters/tensors.py:589-600). Here the pool
// becomes one hipMalloc'd arena and this file owns the device and, per
// calling host thread, a pair of streams with grow-only scratch for split-K
// partials (the reference's O3 runtime calls the ops from four pthreads,
// codegen/x86_emitters/model_source.py:609-674).
#include <stdarg.h>
#include <string.h>

#include <atomic>
#include <string>
#include <vector>

#include "common.h"

namespace nnc {

static Device g_dev;
static std::atomic<int> g_last_error{0};
static std::mutex g_err_mutex;
static char g_last_msg[512] = "";

// Calling-thread states: created on a thread's first call, released for
// reuse when the thread exits, freed by nnc_hip_shutdown. A state found
// through t_state is current only while t_gen equals g_gen (shutdown and a
// new init start a new generation).
static std::mutex g_state_mutex;
static std::vector<ThreadState*> g_states;
static std::atomic<int> g_gen{0};
static thread_local ThreadState* t_state = nullptr;
static thread_local int t_gen = -1;

Device& dev() { return g_dev; }
static int last_code() { return g_last_error.load(); }
// conv.hip: looks up the device address of its static scratch on the
// current device (once per device)
int conv_static_scratch_setup(int device);
ThreadState& ts() { return *t_state; }

static bool sync_thread(const char* who) {
    ThreadState& t = ts();
    for (int k = 0; k < kStreams; ++k)
        if (t.streams[k] && !hip_ok(hipStreamSynchronize(t.streams[k]), who, "hipStreamSynchronize")) return false;
    return true;
}

void fail(int code, const char* who, const char* fmt, ...) {
    char body[384];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(body, sizeof body, fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lock(g_err_mutex);
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

// Default workspace: stream-K partials of a full persistent grid (2 slots of
// 128x128 floats for 512 workgroups = 64 MiB) with room; grows outside capture.
static const size_t kDefaultWorkspace = 128u << 20;
static const size_t kDefaultCounters = 1u << 16;

// Scratch buffers replaced by larger ones stay allocated until shutdown: a
// hipGraph captured earlier still holds their addresses.
static std::mutex g_retired_mutex;
static std::vector<void*> g_retired;
static void retire(void* p) {
    if (!p) return;
    std::lock_guard<std::mutex> lock(g_retired_mutex);
    g_retired.push_back(p);
}

static void free_state(ThreadState* t) {
    for (int k = 0; k < kStreams; ++k)
        if (t->streams[k]) (void)hipStreamSynchronize(t->streams[k]);
    if (t->graph_exec) (void)hipGraphExecDestroy(t->graph_exec);
    if (t->graph) (void)hipGraphDestroy(t->graph);
    for (int k = 0; k < kStreams; ++k) {
        if (t->workspace[k]) (void)hipFree(t->workspace[k]);
        if (t->counters[k]) (void)hipFree(t->counters[k]);
        if (t->repack[k]) (void)hipFree(t->repack[k]);
    }
    if (t->fork_ev) (void)hipEventDestroy(t->fork_ev);
    if (t->join_ev) (void)hipEventDestroy(t->join_ev);
    for (int k = 0; k < kStreams; ++k)
        if (t->streams[k]) (void)hipStreamDestroy(t->streams[k]);
    delete t;
}

// Hands the calling thread's state back for reuse when the thread exits
// (work it queued stays ordered on the state's streams).
struct ThreadRelease {
    ~ThreadRelease() {
        if (!t_state || t_gen != g_gen.load()) return;
        std::lock_guard<std::mutex> lock(g_state_mutex);
        if (t_gen == g_gen.load()) t_state->in_use = false;
        t_state = nullptr;
    }
};
static ThreadRelease& thread_release() {
    static thread_local ThreadRelease r;
    return r;
}

// Streams (default priority: streams of different priorities are not used
// anywhere in this library), fork/join events and the default scratch of a
// new thread state.
static ThreadState* new_state(const char* who) {
    ThreadState* t = new ThreadState();
    bool ok = true;
    for (int k = 0; ok && k < kStreams; ++k)
        ok = hip_ok(hipStreamCreateWithFlags(&t->streams[k], hipStreamNonBlocking), who, "hipStreamCreate");
    ok = ok && hip_ok(hipEventCreateWithFlags(&t->fork_ev, hipEventDisableTiming), who, "hipEventCreate") &&
         hip_ok(hipEventCreateWithFlags(&t->join_ev, hipEventDisableTiming), who, "hipEventCreate");
    if (!ok) {
        free_state(t);
        return nullptr;
    }
    ThreadState* saved = t_state;
    const int saved_gen = t_gen;
    t_state = t;  // workspace()/tile_counters() act on the current thread's state
    t_gen = g_gen.load();
    for (int k = 0; ok && k < kStreams; ++k) {
        t->cur = k;
        ok = workspace(kDefaultWorkspace) && tile_counters(kDefaultCounters);
    }
    t->cur = 0;
    t_state = saved;
    t_gen = saved_gen;
    if (!ok) {
        free_state(t);
        return nullptr;
    }
    return t;
}

// Gives the calling thread a state: a released one if any, else a new one.
static bool attach_thread(const char* who) {
    // HIP's current device is per host thread
    if (!hip_ok(hipSetDevice(g_dev.device), who, "hipSetDevice")) return false;
    ThreadState* t = nullptr;
    {
        std::lock_guard<std::mutex> lock(g_state_mutex);
        for (ThreadState* s : g_states)
            if (!s->in_use) {
                t = s;
                break;
            }
        if (t) t->in_use = true;
    }
    if (!t) {
        t = new_state(who);
        if (!t) return false;
        t->in_use = true;
        std::lock_guard<std::mutex> lock(g_state_mutex);
        g_states.push_back(t);
    }
    t->cur = 0;
    t->fixed = nullptr;
    t_state = t;
    t_gen = g_gen.load();
    (void)thread_release();
    return true;
}

bool thread_ready() { return t_state && t_gen == g_gen.load(); }

bool ready(const char* who) {
    if (t_state && t_gen == g_gen.load()) return true;
    if (g_dev.device < 0) {
        fail(NNC_HIP_ESTATE, who, "nnc_hip_init() has not been called");
        return false;
    }
    return attach_thread(who);
}

void partials_fail(const char* who, size_t bytes) {
    const FixedScratch* f = ts().fixed;
    if (f)
        return fail(NNC_HIP_EUNSUPP, who, "needs %zu bytes of stream-K scratch, more than the %zu-byte static buffer",
                    bytes, f->ws_bytes);
    fail(NNC_HIP_ENOMEM, who, "no workspace for %zu bytes of stream-K partials", bytes);
}

float* workspace(size_t bytes) {
    ThreadState& t = ts();
    if (t.fixed) return bytes <= t.fixed->ws_bytes ? t.fixed->ws : nullptr;
    const int k = t.cur;
    if (bytes <= t.workspace_bytes[k]) return t.workspace[k];
    if (t.capturing) return nullptr;
    if (!hip_ok(hipStreamSynchronize(t.stream()), "workspace", "hipStreamSynchronize")) return nullptr;
    retire(t.workspace[k]);
    t.workspace[k] = nullptr;
    t.workspace_bytes[k] = 0;
    size_t want = bytes < kDefaultWorkspace ? kDefaultWorkspace : bytes;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, want), "workspace", "hipMalloc")) return nullptr;
    t.workspace[k] = static_cast<float*>(p);
    t.workspace_bytes[k] = want;
    return t.workspace[k];
}

size_t workspace_capacity() {
    ThreadState& t = ts();
    return t.fixed ? t.fixed->ws_bytes : t.workspace_bytes[t.cur];
}

float* repack_buffer(size_t bytes) {
    ThreadState& t = ts();
    if (t.fixed) return nullptr;
    const int k = t.cur;
    if (bytes <= t.repack_bytes[k]) return t.repack[k];
    if (t.capturing) return nullptr;
    if (!hip_ok(hipStreamSynchronize(t.stream()), "repack_buffer", "hipStreamSynchronize")) return nullptr;
    retire(t.repack[k]);
    t.repack[k] = nullptr;
    t.repack_bytes[k] = 0;
    const size_t want = bytes < (16u << 20) ? (16u << 20) : bytes;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, want), "repack_buffer", "hipMalloc")) return nullptr;
    t.repack[k] = static_cast<float*>(p);
    t.repack_bytes[k] = want;
    return t.repack[k];
}

int* tile_counters(size_t n) {
    ThreadState& t = ts();
    if (t.fixed) return n <= t.fixed->cnt_n ? t.fixed->cnt : nullptr;
    const int k = t.cur;
    if (n <= t.counters_n[k]) return t.counters[k];
    if (t.capturing) return nullptr;
    if (!hip_ok(hipStreamSynchronize(t.stream()), "tile_counters", "hipStreamSynchronize")) return nullptr;
    retire(t.counters[k]);
    t.counters[k] = nullptr;
    t.counters_n[k] = 0;
    const size_t want = n < kDefaultCounters ? kDefaultCounters : n;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, want * sizeof(int)), "tile_counters", "hipMalloc")) return nullptr;
    if (!hip_ok(hipMemsetAsync(p, 0, want * sizeof(int), t.stream()), "tile_counters", "hipMemsetAsync") ||
        !hip_ok(hipStreamSynchronize(t.stream()), "tile_counters", "hipStreamSynchronize")) {
        (void)hipFree(p);
        return nullptr;
    }
    t.counters[k] = static_cast<int*>(p);
    t.counters_n[k] = want;
    return t.counters[k];
}

// ---------------------------------------------------------------------------
// per-kernel timing (one table for the process, behind a mutex)
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
static std::atomic<bool> g_profiling{false};
static std::mutex g_prof_mutex;
static std::vector<Pending> g_pending;
static std::vector<hipEvent_t> g_event_pool;
static std::vector<Stat> g_stats;

void set_work(double flops, double bytes) {
    ThreadState& t = ts();
    t.next_flops = flops;
    t.next_bytes = bytes;
}

static hipEvent_t take_event() {
    {
        std::lock_guard<std::mutex> lock(g_prof_mutex);
        if (!g_event_pool.empty()) {
            hipEvent_t e = g_event_pool.back();
            g_event_pool.pop_back();
            return e;
        }
    }
    hipEvent_t e = nullptr;
    (void)hipEventCreate(&e);
    return e;
}

TimedScope::TimedScope(const char* n) : name(n) {
    ThreadState& t = ts();
    flops = t.next_flops;
    bytes = t.next_bytes;
    t.next_flops = t.next_bytes = 0.0;
    // no events under capture, nor in an allocation-free call (creating one allocates)
    if (!g_profiling.load() || t.capturing || t.fixed) return;
    start = take_event();
    stop = take_event();
    (void)hipEventRecord(start, t.stream());
}

TimedScope::~TimedScope() {
    if (!start) return;
    (void)hipEventRecord(stop, cur_stream());
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    g_pending.push_back({name, flops, bytes, start, stop});
}

static void resolve_pending() {
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    for (auto& p : g_pending) {
        float ms = 0.f;
        (void)hipEventSynchronize(p.stop);
        (void)hipEventElapsedTime(&ms, p.start, p.stop);
        Stat* s = nullptr;
        for (auto& st : g_stats)
            if (st.name == p.name) {
                s = &st;
                break;
            }
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
    if (g_dev.device == device && t_state && t_gen == g_gen.load()) return NNC_HIP_OK;
    if (g_dev.device == device) return ready("nnc_hip_init") ? NNC_HIP_OK : last_code();
    if (g_dev.device >= 0) nnc_hip_shutdown();
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
        g_dev.cu_count = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
    if (conv_static_scratch_setup(device) != NNC_HIP_OK) return last_code();
    g_dev.device = device;
    if (!ready("nnc_hip_init")) {
        const int code = last_code();
        g_dev.device = -1;
        return code;
    }
    return NNC_HIP_OK;
}

void nnc_hip_shutdown(void) {
    if (g_dev.device < 0) return;
    (void)hipDeviceSynchronize();
    {
        std::lock_guard<std::mutex> lock(g_state_mutex);
        for (ThreadState* t : g_states) free_state(t);
        g_states.clear();
        g_gen.fetch_add(1);
        t_state = nullptr;
        t_gen = -1;
    }
    {
        std::lock_guard<std::mutex> lock(g_prof_mutex);
        for (auto& p : g_pending) {
            (void)hipEventDestroy(p.start);
            (void)hipEventDestroy(p.stop);
        }
        g_pending.clear();
        for (auto e : g_event_pool) (void)hipEventDestroy(e);
        g_event_pool.clear();
    }
    if (g_dev.arena) (void)hipFree(g_dev.arena);
    if (g_dev.spill) (void)hipHostFree(g_dev.spill);
    {
        std::lock_guard<std::mutex> lock(g_retired_mutex);
        for (void* p : g_retired) (void)hipFree(p);
        g_retired.clear();
    }
    g_dev = Device{};
}

int nnc_hip_arena_reserve(size_t bytes) {
    if (!ready("nnc_hip_arena_reserve")) return NNC_HIP_ESTATE;
    if (g_dev.arena && bytes <= g_dev.arena_bytes) return NNC_HIP_OK;
    (void)hipDeviceSynchronize();
    if (g_dev.arena) (void)hipFree(g_dev.arena);
    g_dev.arena = nullptr;
    g_dev.arena_bytes = 0;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 256), "nnc_hip_arena_reserve", "hipMalloc"))
        return NNC_HIP_ENOMEM;
    g_dev.arena = static_cast<char*>(p);
    g_dev.arena_bytes = bytes;
    return NNC_HIP_OK;
}

void* nnc_hip_arena_base(void) { return g_dev.arena; }
size_t nnc_hip_arena_size(void) { return g_dev.arena_bytes; }

int nnc_hip_bind(Tensor* t, size_t offset) {
    if (!t) {
        fail(NNC_HIP_EINVAL, "nnc_hip_bind", "NULL tensor");
        return NNC_HIP_EINVAL;
    }
    if (!g_dev.arena) {
        fail(NNC_HIP_ESTATE, "nnc_hip_bind", "no arena reserved");
        return NNC_HIP_ESTATE;
    }
    if ((offset & 15u) != 0 || offset + (size_t)t->nbytes > g_dev.arena_bytes) {
        fail(NNC_HIP_EINVAL, "nnc_hip_bind", "offset %zu + %lld bytes outside arena of %zu (or misaligned)",
             offset, (long long)t->nbytes, g_dev.arena_bytes);
        return NNC_HIP_EINVAL;
    }
    t->data = g_dev.arena + offset;
    return NNC_HIP_OK;
}

int nnc_hip_spill_reserve(size_t bytes) {
    const char* who = "nnc_hip_spill_reserve";
    if (!ready(who)) return NNC_HIP_ESTATE;
    if (g_dev.spill && bytes <= g_dev.spill_bytes) return NNC_HIP_OK;
    if (ts().capturing) {
        fail(NNC_HIP_ESTATE, who, "cannot allocate the spill pool during graph capture");
        return NNC_HIP_ESTATE;
    }
    (void)hipDeviceSynchronize();
    if (g_dev.spill) (void)hipHostFree(g_dev.spill);
    g_dev.spill = nullptr;
    g_dev.spill_bytes = 0;
    void* p = nullptr;
    if (!hip_ok(hipHostMalloc(&p, bytes ? bytes : 256, hipHostMallocDefault), who, "hipHostMalloc"))
        return NNC_HIP_ENOMEM;
    g_dev.spill = static_cast<char*>(p);
    g_dev.spill_bytes = bytes;
    return NNC_HIP_OK;
}

void* nnc_hip_spill_base(void) { return g_dev.spill; }

int nnc_hip_bind_spill(Tensor* t, size_t offset) {
    const char* who = "nnc_hip_bind_spill";
    if (!t) {
        fail(NNC_HIP_EINVAL, who, "NULL tensor");
        return NNC_HIP_EINVAL;
    }
    if (!g_dev.spill) {
        fail(NNC_HIP_ESTATE, who, "no spill pool reserved");
        return NNC_HIP_ESTATE;
    }
    if ((offset & 15u) != 0 || offset + (size_t)t->nbytes > g_dev.spill_bytes) {
        fail(NNC_HIP_EINVAL, who, "offset %zu + %lld bytes outside the spill pool of %zu (or misaligned)", offset,
             (long long)t->nbytes, g_dev.spill_bytes);
        return NNC_HIP_EINVAL;
    }
    t->data = g_dev.spill + offset;
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
    hip_ok(hipMemcpyAsync(dst->data, src->data, (size_t)src->nbytes, hipMemcpyDefault, cur_stream()), who,
           "hipMemcpyAsync");
}

void* nnc_hip_malloc(size_t bytes) {
    if (!ready("nnc_hip_malloc")) return nullptr;
    void* p = nullptr;
    if (!hip_ok(hipMalloc(&p, bytes ? bytes : 16), "nnc_hip_malloc", "hipMalloc")) return nullptr;
    return p;
}

// Freeing waits for the whole device: any thread's queued work may still
// read the buffer.
void nnc_hip_free(void* ptr) {
    if (!ptr || g_dev.device < 0) return;
    (void)hipDeviceSynchronize();
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
    if (!ptr || g_dev.device < 0) return;
    (void)hipDeviceSynchronize();
    (void)hipHostFree(ptr);
}

// Host copies wait for the calling thread's queued work, copy on its stream
// 0 and wait for the copy.
static int host_copy(void* dst, const void* src, size_t bytes, hipMemcpyKind kind, const char* who) {
    if (!ready(who)) return NNC_HIP_ESTATE;
    if (!bytes) return NNC_HIP_OK;
    ThreadState& t = ts();
    if (!sync_thread(who) || !hip_ok(hipMemcpyAsync(dst, src, bytes, kind, t.streams[0]), who, "hipMemcpyAsync") ||
        !hip_ok(hipStreamSynchronize(t.streams[0]), who, "hipStreamSynchronize"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    return host_copy(dst, src, bytes, hipMemcpyHostToDevice, "nnc_hip_memcpy_h2d");
}

int nnc_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    return host_copy(dst, src, bytes, hipMemcpyDeviceToHost, "nnc_hip_memcpy_d2h");
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
    return sync_thread("nnc_hip_sync") ? NNC_HIP_OK : NNC_HIP_EDEVICE;
}

void* nnc_hip_stream(void) { return ready("nnc_hip_stream") ? ts().streams[0] : nullptr; }

int nnc_hip_stream_fork(void) {
    if (!ready("nnc_hip_stream_fork")) return NNC_HIP_ESTATE;
    ThreadState& t = ts();
    if (!hip_ok(hipEventRecord(t.fork_ev, t.streams[0]), "nnc_hip_stream_fork", "hipEventRecord") ||
        !hip_ok(hipStreamWaitEvent(t.streams[1], t.fork_ev, 0), "nnc_hip_stream_fork", "hipStreamWaitEvent"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_stream_select(int slot) {
    if (!ready("nnc_hip_stream_select")) return NNC_HIP_ESTATE;
    if (slot < 0 || slot >= kStreams) {
        fail(NNC_HIP_EINVAL, "nnc_hip_stream_select", "stream %d out of range (0..%d)", slot, kStreams - 1);
        return NNC_HIP_EINVAL;
    }
    ts().cur = slot;
    return NNC_HIP_OK;
}

int nnc_hip_stream_join(void) {
    if (!ready("nnc_hip_stream_join")) return NNC_HIP_ESTATE;
    ThreadState& t = ts();
    if (!hip_ok(hipEventRecord(t.join_ev, t.streams[1]), "nnc_hip_stream_join", "hipEventRecord") ||
        !hip_ok(hipStreamWaitEvent(t.streams[0], t.join_ev, 0), "nnc_hip_stream_join", "hipStreamWaitEvent"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_last_error(void) { return g_last_error.load(); }

// A copy per calling thread, so another thread's failure cannot rewrite the
// text while the caller reads it.
const char* nnc_hip_last_error_message(void) {
    static thread_local char copy[512];
    std::lock_guard<std::mutex> lock(g_err_mutex);
    memcpy(copy, g_last_msg, sizeof copy);
    return copy;
}

void nnc_hip_clear_error(void) {
    std::lock_guard<std::mutex> lock(g_err_mutex);
    g_last_error.store(0);
    g_last_msg[0] = '\0';
}

void nnc_hip_profile_enable(int on) {
    if (!on) resolve_pending();
    g_profiling.store(on != 0);
}

void nnc_hip_profile_reset(void) {
    resolve_pending();
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    g_stats.clear();
}

int nnc_hip_profile_count(void) {
    resolve_pending();
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    return (int)g_stats.size();
}

int nnc_hip_profile_entry(int i, char* name, int cap, int64_t* launches, double* total_ms) {
    resolve_pending();
    std::lock_guard<std::mutex> lock(g_prof_mutex);
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
    std::lock_guard<std::mutex> lock(g_prof_mutex);
    if (i < 0 || i >= (int)g_stats.size()) return NNC_HIP_EINVAL;
    if (flops) *flops = g_stats[i].flops;
    if (bytes) *bytes = g_stats[i].bytes;
    return NNC_HIP_OK;
}

int nnc_hip_debug_dump(const Tensor* t, const char* name, int node_idx, void* file) {
    const char* fn = "nnc_hip_debug_dump";
    if (!ready(fn)) return NNC_HIP_ESTATE;
    if (ts().capturing) {
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

// Capture records the calling thread's stream 0 (and its side stream once
// forked); other threads keep running eagerly on their own streams.
int nnc_hip_graph_begin(void) {
    if (!ready("nnc_hip_graph_begin")) return NNC_HIP_ESTATE;
    nnc_hip_graph_destroy();
    resolve_pending();
    ThreadState& t = ts();
    if (t.cur != 0) {
        fail(NNC_HIP_ESTATE, "nnc_hip_graph_begin", "capture starts on stream 0 (stream %d selected)", t.cur);
        return NNC_HIP_ESTATE;
    }
    if (!hip_ok(hipStreamBeginCapture(t.streams[0], hipStreamCaptureModeRelaxed), "nnc_hip_graph_begin",
                "hipStreamBeginCapture"))
        return NNC_HIP_EDEVICE;
    t.capturing = true;
    return NNC_HIP_OK;
}

int nnc_hip_graph_end(void) {
    if (!ready("nnc_hip_graph_end")) return NNC_HIP_ESTATE;
    ThreadState& t = ts();
    if (!t.capturing) {
        fail(NNC_HIP_ESTATE, "nnc_hip_graph_end", "no capture in progress");
        return NNC_HIP_ESTATE;
    }
    t.capturing = false;
    hipGraph_t g = nullptr;
    t.cur = 0;
    if (!hip_ok(hipStreamEndCapture(t.streams[0], &g), "nnc_hip_graph_end", "hipStreamEndCapture"))
        return NNC_HIP_EDEVICE;
    t.graph = g;
    if (!hip_ok(hipGraphInstantiate(&t.graph_exec, g, nullptr, nullptr, 0), "nnc_hip_graph_end",
                "hipGraphInstantiate"))
        return NNC_HIP_EDEVICE;
    return NNC_HIP_OK;
}

int nnc_hip_graph_launch(void) {
    if (!ready("nnc_hip_graph_launch")) return NNC_HIP_ESTATE;
    ThreadState& t = ts();
    if (!t.graph_exec) {
        fail(NNC_HIP_ESTATE, "nnc_hip_graph_launch", "no captured graph");
        return NNC_HIP_ESTATE;
    }
    TimedScope scope("graph");
    return hip_ok(hipGraphLaunch(t.graph_exec, t.streams[0]), "nnc_hip_graph_launch", "hipGraphLaunch")
               ? NNC_HIP_OK
               : NNC_HIP_EDEVICE;
}

void nnc_hip_graph_destroy(void) {
    if (!t_state || t_gen != g_gen.load()) return;
    ThreadState& t = ts();
    if (t.graph_exec) (void)hipGraphExecDestroy(t.graph_exec);
    if (t.graph) (void)hipGraphDestroy(t.graph);
    t.graph_exec = nullptr;
    t.graph = nullptr;
}

}  // extern "C"
