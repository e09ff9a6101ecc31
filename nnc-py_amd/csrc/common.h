// Internal header of libnnc_hip.so: device context, error reporting, launch
// wrapper with optional per-kernel timing, small tensor helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include <mutex>

#include "nnc_hip.h"
#include "nnc_ops.h"

namespace nnc {

// ---------------------------------------------------------------------------
// device and calling-thread state
// ---------------------------------------------------------------------------
// The process drives one device (nnc_hip_init); its arena and spill pool are
// process-wide. Everything a call mutates is per calling host thread: each
// thread gets its own pair of library streams with their own scratch on its
// first call, so threads calling nnc_* concurrently (the reference's O3
// runtime runs its steps on four pthreads) never share partial tiles,
// counters, repacked weights, a stream selection or a capture.
// Stream 0 carries a thread's calls unless it selects 1, the side stream of
// a forked branch (nnc_hip_stream_fork/select/join).
static constexpr int kStreams = 2;

struct Device {
    int device = -1;
    int cu_count = 256;
    char* arena = nullptr;
    size_t arena_bytes = 0;
    // pinned host memory: the slow pool that spilled tensors wait in
    char* spill = nullptr;
    size_t spill_bytes = 0;
};

// Caller-provided scratch that replaces the grow-only buffers for the
// duration of one call (the allocation-free entry point): stream-K partials
// and tile counters; nothing is allocated while it is set.
struct FixedScratch {
    float* ws = nullptr;
    size_t ws_bytes = 0;
    int* cnt = nullptr;
    size_t cnt_n = 0;
};

struct ThreadState {
    hipStream_t streams[kStreams] = {};
    int cur = 0;
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;
    // per stream: split-K partials and other per-call scratch; grown outside capture only
    float* workspace[kStreams] = {};
    size_t workspace_bytes[kStreams] = {};
    // per stream: per-tile arrival counters of the stream-K kernels; zero
    // between kernels (each kernel returns the counters it used to zero)
    int* counters[kStreams] = {};
    size_t counters_n[kStreams] = {};
    // per stream: tap-major copies of reference-layout conv weights (grown outside capture)
    float* repack[kStreams] = {};
    size_t repack_bytes[kStreams] = {};
    bool capturing = false;
    hipGraph_t graph = nullptr;
    hipGraphExec_t graph_exec = nullptr;
    const FixedScratch* fixed = nullptr;
    // algorithmic work of this thread's next launch (set_work)
    double next_flops = 0.0, next_bytes = 0.0;
    bool in_use = false;  // held by a live thread (released at thread exit, reused)
    hipStream_t stream() const { return streams[cur]; }
};

Device& dev();
inline int cu_count() { return dev().cu_count; }

// The calling thread's state; valid once ready() has returned true on this
// thread.
ThreadState& ts();
inline hipStream_t cur_stream() { return ts().stream(); }

// Returns false (and records NNC_HIP_ESTATE) if nnc_hip_init has not run;
// otherwise makes sure the calling thread has its streams and scratch
// (created on its first call, NNC_HIP_EDEVICE / ENOMEM if that fails).
bool ready(const char* who);
// Whether the calling thread already has its state (never creates it).
bool thread_ready();

// Record an error code + message (printed once to stderr, kept for
// nnc_hip_last_error()).
void fail(int code, const char* who, const char* fmt, ...);

// Check a HIP runtime call; on failure record NNC_HIP_EDEVICE.
bool hip_ok(hipError_t e, const char* who, const char* what);

// Ensure the selected stream's workspace holds at least `bytes`; returns
// nullptr if it cannot (inside graph capture the workspace cannot grow; with
// fixed scratch: more than it holds).
float* workspace(size_t bytes);
size_t workspace_capacity();

// At least `n` zeroed tile counters, or nullptr if they cannot be provided
// (inside graph capture the buffer cannot grow; fixed scratch too small).
// Kernels leave them zero; counters in fixed scratch are cleared by the
// caller before the launch that uses them.
int* tile_counters(size_t n);

// At least `bytes` of scratch for a repacked weight tensor, or nullptr if it
// cannot be provided (inside graph capture the buffer cannot grow; never
// with fixed scratch).
float* repack_buffer(size_t bytes);

// Record the failure of a call whose stream-K partials did not fit: ENOMEM
// for the grow-only workspace, EUNSUPP with the sizes for fixed scratch.
void partials_fail(const char* who, size_t bytes);

// ---------------------------------------------------------------------------
// kernel launch with optional hipEvent timing (keyed by kernel name)
// ---------------------------------------------------------------------------
// Algorithmic work of the next launch: flops for matrix kernels, bytes that
// must cross HBM at least once for bandwidth kernels. Recorded with the
// launch's time in the timing table (roofline figures). Cleared by launch().
void set_work(double flops, double bytes);

struct TimedScope {
    const char* name;
    double flops = 0.0, bytes = 0.0;
    hipEvent_t start = nullptr, stop = nullptr;
    explicit TimedScope(const char* n);
    ~TimedScope();
};

template <typename Kernel, typename... Args>
inline void launch(const char* name, Kernel kernel, dim3 grid, dim3 block, size_t lds,
                   Args... args) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return;
    TimedScope scope(name);
    hipLaunchKernelGGL(kernel, grid, block, lds, cur_stream(), args...);
    hip_ok(hipGetLastError(), name, "launch");
}

// Streaming stores. The streaming kernels (copies, concat/split,
// element-wise, the softmax and layernorm rows) write an output of at least
// kNtStoreBytes - twice one XCD's 4 MB L2 - with non-temporal stores, which
// go to HBM without displacing the inputs being streamed. Measured as
// hipGraph replays of ten calls: a 205 MB device copy 5.2 -> 7.2 TB/s; a
// 16 MB copy 5.26 -> 4.32 us, softmax [4096,1024] (16.8 MB out) 6.25 ->
// 4.90 us, layernorm [8192,768] (25 MB out) 9.34 -> 7.03 us; outputs of 1
// MB, read by the next GEMM, the same either way, and so was a threshold of
// 0 against this one.
static constexpr int64_t kNtStoreBytes = (int64_t)8 << 20;
typedef float nt_f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int nt_u32x4 __attribute__((ext_vector_type(4)));

template <bool NT>
__device__ __forceinline__ void store_f4(float* p, float4 v) {
    if (NT) {
        nt_f32x4 w = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<nt_f32x4*>(p));
    } else {
        *reinterpret_cast<float4*>(p) = v;
    }
}

template <bool NT>
__device__ __forceinline__ void store_u4(uint4* p, uint4 v) {
    if (NT) {
        nt_u32x4 w = {v.x, v.y, v.z, v.w};
        __builtin_nontemporal_store(w, reinterpret_cast<nt_u32x4*>(p));
    } else {
        *p = v;
    }
}

// Copy `bytes` bytes device-to-device on the library stream with a kernel
// (16-byte vector path when aligned; no memset/memcpy nodes under capture).
// src == dst is a no-op. Defined in movement.hip.
void device_copy(const char* name, const void* src, void* dst, size_t bytes);

// ---------------------------------------------------------------------------
// tensor helpers (host side)
// ---------------------------------------------------------------------------
inline int64_t numel(const Tensor* t) {
    int64_t n = 1;
    for (int d = 0; d < t->ndim; ++d) n *= t->shape[d];
    return n;
}

inline int64_t prod(const int64_t* s, int lo, int hi) {
    int64_t p = 1;
    for (int d = lo; d < hi; ++d) p *= s[d];
    return p;
}

inline bool has_data(const Tensor* t) { return t && t->data && (t->shape || t->ndim == 0); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Grid size for a grid-stride element-wise kernel over n items with `per`
// items per thread.
inline unsigned grid_for(int64_t n, int per, int block = 256) {
    int64_t g = ceil_div(ceil_div(n, per), block);
    const int64_t cap = (int64_t)cu_count() * 16;
    if (g > cap) g = cap;
    return (unsigned)(g < 1 ? 1 : g);
}

}  // namespace nnc
