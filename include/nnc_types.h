/*
 * nnc_types.h - tensor descriptor shared by generated model code and every
 * implementation of the nnc operator ABI (the x86 reference runtime, the CPU
 * oracle under oracle/, and the gfx950 HIP library libnnc_hip.so).
 *
 * Layout and enum values must stay identical to the reference
 * (runtime/include/nnc_types.h:16-33) so that generated model.c/tensors.c and
 * ctypes mirrors (tests/test_x86_runtime.py:265-272) bind unchanged.
 *
 * For the HIP library, Tensor.data is a DEVICE pointer (normally an offset into
 * the one hipMalloc'd HBM arena, see nnc_hip.h); Tensor.shape stays a host
 * array that the host side reads before launching a kernel.
 */
#ifndef NNC_TYPES_H
#define NNC_TYPES_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    NNC_DTYPE_FLOAT32 = 0,
    NNC_DTYPE_FLOAT16 = 1,
    NNC_DTYPE_INT32 = 2,
    NNC_DTYPE_INT8 = 3,
    NNC_DTYPE_UINT8 = 4,
    NNC_DTYPE_BOOL = 5,
    NNC_DTYPE_INT64 = 6,
} nnc_dtype_t;

typedef struct {
    void* data;        /* element storage (device pointer for libnnc_hip) */
    nnc_dtype_t dtype; /* element type */
    int64_t* shape;    /* host array of ndim extents */
    int ndim;          /* rank */
    int64_t nbytes;    /* storage size in bytes */
} Tensor;

#ifdef __cplusplus
}
#endif

#endif /* NNC_TYPES_H */
