/*
 * TEST INFRASTRUCTURE ONLY: a host-memory stand-in for the lifecycle half of
 * include/nnc_hip.h, so that code generated for the mi355x target can be
 * linked with the CPU oracle (oracle/liboracle.so) and its nnc_run() checked
 * on a machine without a GPU. The arena is a host allocation; copies are
 * memcpy; graph capture reports "unsupported" so generated code takes its
 * node-by-node path. Never linked into the product.
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nnc_hip.h"

static char* arena = NULL;
static size_t arena_size = 0;

int nnc_hip_init(int device) { (void)device; return 0; }
void nnc_hip_shutdown(void) { free(arena); arena = NULL; arena_size = 0; }
int nnc_hip_arena_reserve(size_t bytes) {
    if (arena && bytes <= arena_size) return 0;
    free(arena);
    arena = aligned_alloc(256, (bytes + 255) / 256 * 256);
    arena_size = arena ? bytes : 0;
    return arena ? 0 : NNC_HIP_ENOMEM;
}
void* nnc_hip_arena_base(void) { return arena; }
size_t nnc_hip_arena_size(void) { return arena_size; }
int nnc_hip_bind(Tensor* t, size_t offset) {
    if (!arena || offset + (size_t)t->nbytes > arena_size) return NNC_HIP_EINVAL;
    t->data = arena + offset;
    return 0;
}
static char* spill = NULL;
static size_t spill_size = 0;
int nnc_hip_spill_reserve(size_t bytes) {
    if (spill && bytes <= spill_size) return 0;
    free(spill);
    spill = aligned_alloc(256, (bytes + 255) / 256 * 256 + 256);
    spill_size = spill ? bytes : 0;
    return spill ? 0 : NNC_HIP_ENOMEM;
}
void* nnc_hip_spill_base(void) { return spill; }
int nnc_hip_bind_spill(Tensor* t, size_t offset) {
    if (!spill || offset + (size_t)t->nbytes > spill_size) return NNC_HIP_EINVAL;
    t->data = spill + offset;
    return 0;
}
void* nnc_hip_malloc(size_t bytes) { return malloc(bytes); }
void* nnc_hip_host_malloc(size_t bytes) { return malloc(bytes); }
void nnc_hip_host_free(void* p) { free(p); }
void nnc_hip_free(void* p) { free(p); }
int nnc_hip_upload(Tensor* t, const void* src) { memcpy(t->data, src, (size_t)t->nbytes); return 0; }
int nnc_hip_download(const Tensor* t, void* dst) { memcpy(dst, t->data, (size_t)t->nbytes); return 0; }
int nnc_hip_memcpy_h2d(void* d, const void* s, size_t n) { memcpy(d, s, n); return 0; }
int nnc_hip_memcpy_d2h(void* d, const void* s, size_t n) { memcpy(d, s, n); return 0; }
int nnc_hip_sync(void) { return 0; }
void* nnc_hip_stream(void) { return NULL; }
int nnc_hip_last_error(void) { return 0; }
const char* nnc_hip_last_error_message(void) { return "host shim"; }
void nnc_hip_clear_error(void) {}
void nnc_hip_profile_enable(int on) { (void)on; }
void nnc_hip_profile_reset(void) {}
int nnc_hip_profile_count(void) { return 0; }
int nnc_hip_profile_entry(int i, char* n, int c, int64_t* l, double* m) {
    (void)i; (void)n; (void)c; (void)l; (void)m;
    return NNC_HIP_EINVAL;
}
int nnc_hip_profile_work(int i, double* f, double* b) { (void)i; (void)f; (void)b; return NNC_HIP_EINVAL; }
int nnc_hip_stream_fork(void) { return 0; }
int nnc_hip_stream_select(int slot) { (void)slot; return 0; }
int nnc_hip_stream_join(void) { return 0; }
int nnc_hip_graph_begin(void) { return NNC_HIP_EUNSUPP; }
int nnc_hip_graph_end(void) { return NNC_HIP_EUNSUPP; }
int nnc_hip_graph_launch(void) { return NNC_HIP_EUNSUPP; }
void nnc_hip_graph_destroy(void) {}
/* the dump format of nnc_hip_debug_dump, for float32 / uint8 / int64 tensors in host memory */
int nnc_hip_debug_dump(const Tensor* t, const char* name, int node_idx, void* file) {
    FILE* f = file ? (FILE*)file : stdout;
    int64_t n = 1;
    for (int d = 0; d < t->ndim; ++d) n *= t->shape[d];
    fprintf(f, "DEBUG_TENSOR_START %s %d\n", name, node_idx);
    fprintf(f, "SHAPE %d\n", t->ndim);
    for (int d = 0; d < t->ndim; ++d) fprintf(f, "DIM %d %d\n", d, (int)t->shape[d]);
    fprintf(f, "DATA_START\n");
    for (int64_t i = 0; i < n; ++i) {
        float v;
        if (t->dtype == NNC_DTYPE_BOOL || t->dtype == NNC_DTYPE_UINT8) v = (float)((const uint8_t*)t->data)[i];
        else if (t->dtype == NNC_DTYPE_INT64) v = (float)((const int64_t*)t->data)[i];
        else v = ((const float*)t->data)[i];
        fprintf(f, "%f\n", (double)v);
    }
    fprintf(f, "DATA_END\n");
    fprintf(f, "DEBUG_TENSOR_END %s\n\n", name);
    return 0;
}
