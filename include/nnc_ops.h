/*
 * nnc_ops.h - the nnc operator ABI.
 *
 * Every entry point here has the signature of the reference declaration it
 * replaces (runtime/include/nnc_ops.h, line cited per group) so that model.c
 * emitted by the nnc code generator links against libnnc_hip.so exactly as it
 * links against runtime/x86/ops.c (build_files.py:57 selects the runtime at
 * link time). Semantics are those of runtime/x86/ops.c (lines cited per
 * group); documented divergences are marked DIVERGES.
 *
 * In libnnc_hip.so:
 *   - every Tensor.data is a device pointer; shapes are host arrays;
 *   - every call enqueues work on the library stream and returns without
 *     waiting (nnc_hip_sync() in nnc_hip.h waits);
 *   - ops return void like the reference; a bad argument prints one line to
 *     stderr, leaves the output untouched and sets nnc_hip_last_error().
 *   - element-wise ops are safe with out == in (the cost_aware planner aliases
 *     outputs onto dying inputs, cost_aware_allocator.py:39-48).
 */
#ifndef NNC_OPS_H
#define NNC_OPS_H

#include <stdint.h>
#include "nnc_types.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- binary element-wise (ref nnc_ops.h:21-24, ops.c:82-224) ------------
 * out[i] = a[i % a_n] OP b[i % b_n] for i < n when a_n == n or b_n == n
 * (flat-modulo broadcast); when both operands are smaller than out only the
 * first min(a_n, b_n, n) elements are written. */
void nnc_add(Tensor* a, Tensor* b, Tensor* out);
void nnc_mul(Tensor* a, Tensor* b, Tensor* out);
void nnc_sub(Tensor* a, Tensor* b, Tensor* out);
void nnc_div(Tensor* a, Tensor* b, Tensor* out);

/* ---- comparison / logical (ref nnc_ops.h:36,44,304,316,323;
 *      ops.c:2342-2428, 2655-2699) ---------------------------------------- */
void nnc_equal(Tensor* a, Tensor* b, Tensor* out);   /* float 1/0 out */
void nnc_and(Tensor* a, Tensor* b, Tensor* out);     /* float 1/0 out */
void nnc_greater(Tensor* a, Tensor* b, Tensor* out); /* uint8 out     */
void nnc_or(Tensor* a, Tensor* b, Tensor* out);      /* uint8 in/out  */
void nnc_not(Tensor* input, Tensor* output);         /* uint8 in/out  */

/* ---- convolution (ref nnc_ops.h:63-90, 385-412; ops.c:720-1504,
 *      3122-3227) -------------------------------------------------------
 * NCHW fp32. pad_h/pad_w are the top/left pads; bottom/right follow from the
 * output shape. Groups and dilations are not supported (as in the reference).
 * The reference accumulates in fp64; libnnc_hip uses fp32 MFMA with
 * compensated tile accumulation (tolerance parity, not bit-exact). */
void nnc_conv(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output,
              int kernel_h, int kernel_w, int stride_h, int stride_w,
              int pad_h, int pad_w);
void nnc_conv1x1(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output,
                 int stride_h, int stride_w, int pad_h, int pad_w);
/* 3x3 stride 1 pad 1; rejects outputs whose H/W differ from the input
 * (ops.c:1089-1093). */
void nnc_conv3x3_s1(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output);
/* 7x7 stride 2 with the pad fixed at 3 (ops.c:1310-1311, 1403). */
void nnc_conv7x7_s2(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output);
void nnc_conv_relu(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output,
                   int kernel_h, int kernel_w, int stride_h, int stride_w,
                   int pad_h, int pad_w);
void nnc_conv_relu1x1(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output,
                      int stride_h, int stride_w, int pad_h, int pad_w);
void nnc_conv_relu3x3_s1(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output);
void nnc_conv_relu7x7_s2(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output);
void nnc_conv_sigmoid(Tensor* input, Tensor* weight, Tensor* bias, Tensor* output,
                      int kernel_h, int kernel_w, int stride_h, int stride_w,
                      int pad_h, int pad_w);

/* ---- activations (ref nnc_ops.h:93-96, 250; ops.c:230-310, 2253-2262) --- */
void nnc_relu(Tensor* input, Tensor* output);
void nnc_sigmoid(Tensor* input, Tensor* output);
void nnc_tanh(Tensor* input, Tensor* output);
/* softmax along one axis: max with strict '>', exp(x-max)/sum */
void nnc_softmax(Tensor* input, Tensor* output, int axis);
void nnc_clip(Tensor* input, Tensor* output, float min_val, float max_val);

/* ---- unary math (ref nnc_ops.h:107-142; ops.c:2434-2515) --------------- */
void nnc_sqrt(Tensor* input, Tensor* output); /* NaN for x < 0          */
void nnc_pow(Tensor* input, Tensor* output);  /* always x*x (ops.c:2449) */
void nnc_exp(Tensor* input, Tensor* output);
void nnc_log(Tensor* input, Tensor* output);  /* NaN for x <= 0         */
void nnc_abs(Tensor* input, Tensor* output);
void nnc_neg(Tensor* input, Tensor* output);

/* ---- pooling (ref nnc_ops.h:159-172; ops.c:316-461) ---------------------
 * Windows are clamped to the input. MaxPool starts from -3.402823e38f and an
 * empty window yields that value; AvgPool divides by the in-bounds count. */
void nnc_maxpool2d(Tensor* input, Tensor* output, int kernel_h, int kernel_w,
                   int stride_h, int stride_w, int pad_h, int pad_w);
void nnc_avgpool2d(Tensor* input, Tensor* output, int kernel_h, int kernel_w,
                   int stride_h, int stride_w, int pad_h, int pad_w);

/* ---- shape manipulation (ref nnc_ops.h:178-191; ops.c:1510-1601,
 *      2264-2336) ------------------------------------------------------- */
void nnc_reshape(Tensor* input, Tensor* output, int64_t* shape, int ndim);
void nnc_flatten(Tensor* input, Tensor* output, int axis);
/* perm == NULL reverses the axes; at most 8 dims */
void nnc_transpose(Tensor* input, Tensor* output, int64_t* perm, int ndim);
void nnc_squeeze(Tensor* input, Tensor* output, int axis);
void nnc_unsqueeze(Tensor* input, Tensor* output, int axis);
void nnc_tile(Tensor* input, Tensor* output, int64_t* repeats, int ndim);

/* ---- matrix products (ref nnc_ops.h:197-205; ops.c:1607-1886) ----------
 * nnc_matmul: 2-D, vec x mat, mat x vec and batched with a 2-D B broadcast.
 * DIVERGES for batched inputs with more than one batch: the reference steps
 * A and B by the batch COUNT instead of the matrix size (ops.c:1687-1704);
 * libnnc_hip steps by M*K and K*N (numpy/ONNX MatMul semantics). */
void nnc_matmul(Tensor* a, Tensor* b, Tensor* output);
/* output = alpha * op(A) op(B) + beta * C; C is [N] when 1-D else [M,N] */
void nnc_gemm(Tensor* a, Tensor* b, Tensor* c, Tensor* output,
              float alpha, float beta, int trans_a, int trans_b);
/* as nnc_gemm with B stored [N,K] (emitted when Gemm B is a constant with
 * transB=1, prepack_lowering.py:89-118) */
void nnc_gemm_nt(Tensor* a, Tensor* b, Tensor* c, Tensor* output,
                 float alpha, float beta);

/* ---- reductions (ref nnc_ops.h:211-212; ops.c:1892-1989) ---------------
 * One axis (negative counts from the end). keepdims only changes the output
 * rank, not the element order. */
void nnc_reducemean(Tensor* input, Tensor* output, int axis, int keepdims);
void nnc_reducesum(Tensor* input, Tensor* output, int axis, int keepdims);

/* ---- other (ref nnc_ops.h:218-250; ops.c:1995-2251) --------------------
 * nnc_concat/nnc_split: float32 or int64 (by dtype). DIVERGES: no 64 MiB
 * staging cap (the reference refuses larger outputs, ops.c:2019-2024).
 * nnc_split cuts equal parts of size dim/num_outputs like the reference. */
void nnc_concat(Tensor** inputs, Tensor* output, int num_inputs, int axis);
/* a no-op, as in the reference (ops.c:2088-2093) */
void nnc_batchnorm(Tensor* input, Tensor* scale, Tensor* bias, Tensor* mean,
                   Tensor* var, Tensor* output, float epsilon, int momentum);
/* normalizes over dims [axis:], scale/bias indexed by the axis dim only */
void nnc_layernorm(Tensor* input, Tensor* scale, Tensor* bias, Tensor* output,
                   int axis, float epsilon);
void nnc_identity(Tensor* input, Tensor* output);
void nnc_split(Tensor* input, Tensor** outputs, int num_outputs, int axis);

/* ---- type / shape utilities (ref nnc_ops.h:262-292; ops.c:2517-2653) --- */
void nnc_cast(Tensor* input, Tensor* output, int to_dtype);
void nnc_shape(Tensor* input, Tensor* output, int64_t* shape_data, int ndim);
void nnc_constantofshape(Tensor* output, float value, int ndim);
void nnc_expand(Tensor* input, Tensor* output, int64_t* shape, int ndim);

/* ---- indexing / recurrent (ref nnc_ops.h:339, 360; ops.c:2705-3116) ---- */
void nnc_gather(Tensor* data, Tensor* indices, Tensor* output, int axis,
                int data_dtype);
void nnc_lstm(Tensor* X, Tensor* W, Tensor* R, Tensor* B, Tensor* Y,
              Tensor* Y_h, Tensor* Y_c, int direction, int hidden_size);

/* ---- fused element-wise (ref nnc_ops.h:422, 432; ops.c:3233-3346) ------ */
void nnc_add_relu(Tensor* a, Tensor* b, Tensor* out);    /* s > 0 ? s : 0 */
void nnc_add_sigmoid(Tensor* a, Tensor* b, Tensor* out);

/* ---- MatMul + Relu -------------------------------------------------------
 * The reference code generator emits this call, with the argument list
 * (a, b, bias or NULL, output), for the matmul_relu fusion pattern
 * (c_emitter.py:1143-1171, fusion_patterns.py:145-153), but no reference
 * runtime defines it, so such models fail to link there. Defined here as
 * relu(nnc_matmul(a, b) + bias), bias being [N] (per column) or [M, N]. */
void nnc_matmul_relu(Tensor* a, Tensor* b, Tensor* bias, Tensor* output);

#ifdef __cplusplus
}
#endif

#endif /* NNC_OPS_H */
