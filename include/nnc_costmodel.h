/*
 * nnc_costmodel.h - queries of libnnc_costmodel.so, the cost-model runtime of
 * the mi355x target.
 *
 * Replaces runtime/x86/costmodel.c of the reference (selected with
 * NNC_RUNTIME_IMPL=costmodel, codegen/x86_emitters/build_files.py:50-81):
 * the same nnc_* ABI (nnc_ops.h) and lifecycle (nnc_hip.h), but instead of
 * computing, every call adds the kernels libnnc_hip.so would launch for it -
 * the same tile choice and stream-K plan - to a simulated MI355X timeline,
 * each priced by an analytic roofline (fp32 MFMA and HBM peaks, per-kernel
 * efficiencies measured on the GPU). Generated programs link it unchanged
 * (`make NNC_RUNTIME_IMPL=costmodel`), so planners can be tuned without the
 * hardware. Tensor data is never read or written by the nnc_* calls.
 *
 * Each call prints a trace line `[costmodel] #n op=... kernel=... stream=s
 * start=... end=... us=...` unless NNC_COSTMODEL_QUIET is set; a summary
 * is printed at exit (also unless NNC_COSTMODEL_QUIET is set).
 */
#ifndef NNC_COSTMODEL_H
#define NNC_COSTMODEL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Clear the timeline and the per-kernel table. */
void nnc_costmodel_reset(void);
/* Simulated time from the last reset to the end of the last kernel, in
 * microseconds (the two streams joined). */
double nnc_costmodel_elapsed_us(void);
/* Number of distinct kernel names in the table. */
int nnc_costmodel_kernel_count(void);
/* Entry i: kernel name (NUL-terminated, truncated to cap), launches, summed
 * microseconds, flops and algorithmic HBM bytes. Returns 0 on success. */
int nnc_costmodel_kernel(int i, char* name, int cap, int64_t* launches, double* us, double* flops,
                         double* bytes);

#ifdef __cplusplus
}
#endif

#endif /* NNC_COSTMODEL_H */
