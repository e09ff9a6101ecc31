/*
 * nnc_hip.h - lifecycle, memory and measurement entry points of
 * libnnc_hip.so, the gfx950 (MI355X) implementation of the nnc operator ABI
 * declared in nnc_ops.h.
 *
 * The reference has no device: generated tensors.c points every Tensor into a
 * static host pool (codegen/x86_emitters/tensors.py:589-600, 826-868) and
 * constants_loader.c fread()s weights into static arrays
 * (x86_emitters/constants_loader.py:196-291). The HIP target keeps the memory
 * plan (cost_aware offsets) but places it in ONE hipMalloc'd HBM arena:
 *
 *     nnc_hip_init(0);
 *     nnc_hip_arena_reserve(NNC_MEMORY_SIZE);   // one allocation
 *     nnc_hip_bind(&tensor_x, OFFSET_x);        // per tensor, at load time
 *     nnc_hip_upload(&tensor_w, host_bytes);    // constants, inputs
 *     nnc_run();                                // enqueues nnc_* kernels
 *     nnc_hip_download(&tensor_output, host);   // waits, copies back
 *
 * Threads: the O0-O2 generated code is serial (c_emitter.py:832-847); the
 * reference's O3 runtime calls ops from four pthreads
 * (codegen/x86_emitters/model_source.py:609-674). Every nnc_* entry point is
 * reentrant: each calling host thread gets its own pair of library streams
 * with its own stream-K scratch on its first call (released for reuse when
 * the thread exits), and its calls run in order on its own streams. Work is
 * not ordered across threads: a thread that hands a tensor to another calls
 * nnc_hip_sync() first. The arena, the spill pool, nnc_hip_init and
 * nnc_hip_shutdown are process-wide: reserve and shut down while no other
 * thread is calling. Return codes: 0 = success, otherwise an NNC_HIP_E*
 * value, also kept (process-wide) for nnc_hip_last_error().
 */
#ifndef NNC_HIP_H
#define NNC_HIP_H

#include <stddef.h>
#include <stdint.h>
#include "nnc_types.h"

#ifdef __cplusplus
extern "C" {
#endif

enum {
    NNC_HIP_OK = 0,
    NNC_HIP_EINVAL = 1,   /* bad argument (NULL tensor, bad rank, shape) */
    NNC_HIP_ENOMEM = 2,   /* device allocation failed / arena too small  */
    NNC_HIP_EDEVICE = 3,  /* a HIP runtime call failed                   */
    NNC_HIP_EUNSUPP = 4,  /* argument combination not implemented        */
    NNC_HIP_ESTATE = 5    /* called before nnc_hip_init                  */
};

/* Select the device and create the calling thread's library streams
 * (default priority) and workspace. Idempotent for the same device; another
 * thread's first call (this or any nnc_* call) sets up that thread. */
int nnc_hip_init(int device);
/* Wait for the device, free the arena, every thread's streams and scratch. */
void nnc_hip_shutdown(void);

/* ---- the HBM arena ----------------------------------------------------- */
/* Reserve the arena with one hipMalloc (256-byte aligned base). Calling it
 * again with a larger size replaces the arena (previous bindings dangle). */
int nnc_hip_arena_reserve(size_t bytes);
void* nnc_hip_arena_base(void);
size_t nnc_hip_arena_size(void);
/* t->data = arena + offset; fails if [offset, offset + t->nbytes) is outside
 * the arena or offset is not 16-byte aligned. */
int nnc_hip_bind(Tensor* t, size_t offset);

/* ---- the spill pool (a fast-memory budget below the plan's peak) ------- */
/* Replaces the reference's `_nnc_slow_pool` and the memcpy calls of its
 * spill/reload code (codegen/x86_emitters/model_source.py:259-290,
 * 1535-1659): the HBM arena is the fast pool, pinned host memory the slow
 * one. nnc_hip_spill_reserve allocates it with one hipHostMalloc (again with
 * a larger size: replaced, previous bindings dangle; refused during graph
 * capture); nnc_hip_bind_spill sets t->data = pool + offset like
 * nnc_hip_bind. */
int nnc_hip_spill_reserve(size_t bytes);
void* nnc_hip_spill_base(void);
int nnc_hip_bind_spill(Tensor* t, size_t offset);
/* Copy src's t->nbytes bytes to dst (same nbytes) asynchronously on the
 * selected library stream: a spill (arena -> pool) or a reload (pool ->
 * arena); under graph capture a memcpy node. Errors as for nnc_* calls. */
void nnc_hip_transfer(Tensor* src, Tensor* dst);

/* ---- explicit allocations (tests and callers without an arena) --------- */
void* nnc_hip_malloc(size_t bytes);
void nnc_hip_free(void* ptr);
/* pinned host memory (hipHostMalloc): a spill pool of one's own */
void* nnc_hip_host_malloc(size_t bytes);
void nnc_hip_host_free(void* ptr);

/* ---- host <-> device (synchronous with respect to the calling thread's
 * library streams) ---------------------------------------------------------- */
int nnc_hip_upload(Tensor* t, const void* host_src);    /* t->nbytes bytes */
int nnc_hip_download(const Tensor* t, void* host_dst);  /* t->nbytes bytes */
int nnc_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int nnc_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);

/* ---- synchronisation and errors ---------------------------------------- */
int nnc_hip_sync(void);             /* waits for the calling thread's streams */
void* nnc_hip_stream(void);         /* the calling thread's stream 0, for callers
                                       that order their own work after ours */
int nnc_hip_last_error(void);       /* last non-zero code since reset */
const char* nnc_hip_last_error_message(void);
void nnc_hip_clear_error(void);

/* ---- a second stream for independent branches ---------------------------
 * Per calling thread: its calls go to its stream 0 unless it selects its
 * stream 1. The compiler's O3
 * schedule (mi355x target) runs a branch that only depends on the fork
 * point - a residual block's 1x1 downsample convolution - on stream 1 while
 * the main branch continues on stream 0:
 *   nnc_hip_stream_fork();       stream 1 waits for stream 0's work so far
 *   nnc_hip_stream_select(1); ...branch calls...; nnc_hip_stream_select(0);
 *   ...main calls...
 *   nnc_hip_stream_join();       stream 0 waits for stream 1's work so far
 * Both streams have default priority and their own scratch (stream-K
 * partials, counters), so concurrent calls never share it; nnc_hip_sync and
 * the host copies wait for both. A graph capture starts and ends on stream
 * 0 and records forked branches as parallel graph branches. No counterpart
 * in the reference, whose O3 executor runs its resource queues on host
 * threads (codegen/x86_emitters/model_source.py:502-735). */
int nnc_hip_stream_fork(void);
int nnc_hip_stream_select(int slot);
int nnc_hip_stream_join(void);

/* ---- per-kernel timing --------------------------------------------------
 * While enabled, every kernel launch is bracketed by hipEvents recorded on
 * the stream it runs on; durations accumulate per kernel name in one
 * process-wide table. Reading the table waits for the recorded events. Used
 * by bench.py for the roofline figures. */
void nnc_hip_profile_enable(int on);
void nnc_hip_profile_reset(void);
int nnc_hip_profile_count(void);
/* Entry i: copies the kernel name (NUL-terminated, truncated to cap), the
 * number of launches and the summed milliseconds. Returns 0 on success. */
int nnc_hip_profile_entry(int i, char* name, int cap, int64_t* launches,
                          double* total_ms);
/* Entry i: algorithmic work summed over its launches - flops for the matrix
 * kernels, bytes every launch must move through HBM at least once for the
 * bandwidth-bound kernels (0 where not applicable). */
int nnc_hip_profile_work(int i, double* flops, double* bytes);

/* ---- launch capture ------------------------------------------------------
 * Record every kernel the calling thread's following nnc_* calls enqueue
 * into a hipGraph (one per thread) and replay it with one launch on that
 * thread's stream 0. Between begin and end nothing of it executes. The graph
 * keeps the device pointers of the captured calls. */
int nnc_hip_graph_begin(void);
int nnc_hip_graph_end(void);
int nnc_hip_graph_launch(void);
void nnc_hip_graph_destroy(void);

/* ---- per-tensor debug dump ------------------------------------------------
 * Replaces the dump code the reference emits into nnc_run() in debug mode
 * (src/nnc_py/codegen/x86_emitters/model_source.py:136-184, 297-428): waits
 * for the library stream, copies the tensor to the host and writes it in the
 * reference's text format,
 *   DEBUG_TENSOR_START <name> <node_idx>
 *   SHAPE <ndim>
 *   DIM <i> <extent>                      (one line per dimension)
 *   DATA_START
 *   <value printed with %f>               (one line per element)
 *   DATA_END
 *   DEBUG_TENSOR_END <name>               (then an empty line)
 * to `file` (a FILE*; NULL: stdout), so the reference's parser
 * (src/nnc_py/tools/debug_compare.py:17-106) reads it unchanged. Float32
 * elements print as themselves, bool/uint8/int8 and int32/int64 as their
 * value converted to float. Not while a graph is being captured
 * (NNC_HIP_ESTATE). */
int nnc_hip_debug_dump(const Tensor* t, const char* name, int node_idx, void* file);

/* ---- fused operators of the mi355x target --------------------------------
 * No counterpart in the reference ABI (runtime/include/nnc_ops.h); emitted by
 * the mi355x compiler target at O3.
 *
 * nnc_hip_conv_add_relu: a residual block's Conv -> Add -> Relu in one
 * kernel: out = relu(conv(in, w) + bias + res), equal to nnc_conv followed by
 * nnc_add_relu(conv_out, res, out) (same rounding sequence). `res` has the
 * output's shape and may be the same buffer as `out`; `b` may be NULL. */
void nnc_hip_conv_add_relu(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw,
                           int sh, int sw, int ph, int pw);

/* nnc_hip_conv_packed: convolution with the weights packed tap-major,
 * [Co][kh][kw][Ci] (the compiler transposes the constant), which lets the
 * kernel stream weights and input straight into LDS. out = act(conv(in, w) +
 * bias (+ res)); act 0 none, 1 relu, 2 sigmoid. `b` and `res` may be NULL;
 * `res` has the output's shape and may be the same buffer as `out`. Needs
 * Ci % 32 == 0, a 1x1 or 3x3 kernel and 16-byte aligned weights
 * (NNC_HIP_EUNSUPP otherwise). */
void nnc_hip_conv_packed(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh,
                         int sw, int ph, int pw, int act);

/* nnc_hip_conv_proj: a residual block's last convolution with its 1x1
 * projection shortcut folded into the same contraction:
 *   out = act(conv(in, W3) + conv1x1(x, Wp, stride psh x psw) + b)
 * with w packed [Co][kh*kw*Ci + Cx]: each row is W3 tap-major
 * ([kh][kw][Ci]) followed by the Cx projection weights, and b the sum of the
 * two biases. Equal to nnc_conv + nnc_conv1x1 + nnc_add_relu (act 1) up to
 * fp32 accumulation order. Needs a 3x3 kernel, Ci and Cx multiples of 32,
 * every (oh * psh, ow * psw) inside x, 16-byte aligned weights
 * (NNC_HIP_EUNSUPP / NNC_HIP_EINVAL otherwise). */
void nnc_hip_conv_proj(Tensor* in, Tensor* w, Tensor* b, Tensor* x, Tensor* out, int kh, int kw, int sh, int sw,
                       int ph, int pw, int psh, int psw, int act);

/* nnc_hip_conv_maxpool: ResNet's stem - convolution on packed [Co][Kp]
 * rows (3 channels, 7x7), bias, relu - streamed into the 3x3 / stride 2 /
 * pad 1 max pool that follows it:
 *   out = maxpool(relu(conv(in, w) + b)), out [N][Co][Ho/2][Wo/2]
 * with Ho, Wo the convolution's output size from in, the kernel, stride and
 * pads. The convolution output never reaches HBM: each workgroup pools the
 * rows it computes. Same convolution (within the conv bar of the reference's
 * double sums) and the same max (bit for bit on that convolution) as
 * nnc_hip_conv_packed + nnc_maxpool2d. Needs Co <= 64, Ho and Wo even,
 * Wo <= 128 (NNC_HIP_EUNSUPP otherwise). Emitted by the mi355x target's O3
 * tile-streaming pass. No counterpart in the reference ABI. */
void nnc_hip_conv_maxpool(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph,
                          int pw);

/* nnc_hip_gap_gemm_nt: GlobalAveragePool -> Flatten -> Gemm(transB = 1) in
 * one kernel, the pooled [N, C] tensor never leaving the workgroup:
 *   out[n][o] = alpha * sum_c mean_hw(in[n][c]) * w[o][c] + beta * c
 * with in [N][C][H][W], w [O][C], c [O] or [N][O] or NULL, out [N][O]. The
 * means are nnc_avgpool2d's over the whole plane, bit for bit; the dot
 * products are nnc_gemm_nt's exact float products summed in double in
 * another fixed order (per-lane sums and a shuffle tree instead of one
 * chain: the float result differs only where the double sums straddle a
 * float rounding boundary). Needs C % 4 == 0, C <= 1024, C * (H*W + 2)
 * floats <= 128 KB, at most 65535 images and 16-byte aligned in and w
 * (NNC_HIP_EUNSUPP otherwise). Emitted by the mi355x target's O3 tile-streaming pass. No
 * counterpart in the reference ABI. */
void nnc_hip_gap_gemm_nt(Tensor* in, Tensor* w, Tensor* c, Tensor* out, float alpha, float beta);

/* nnc_hip_fused_eltwise: a chain of element-wise ops evaluated in registers
 * in one pass over HBM, no intermediate tensor written. ins: n_in (1..4)
 * tensors of numel(out) elements each (no broadcast). prog: n_steps (1..8)
 * steps of three ints {op, x, y} computing acc = op(x, y), an operand being
 * -1 (acc, the previous step's value; not in step 0) or an input index; y is
 * ignored by the unary ops. consts: two floats per step, Clip's lo and hi
 * (may be NULL without Clip steps). out = acc after the last step; out may be
 * one of the inputs. Ops (NNC_EW_*): ADD 0, SUB 1, MUL 2, DIV 3, ADD_RELU 4
 * (s > 0 ? s : 0, as nnc_add_relu), ADD_SIGMOID 5, RELU 6 (as nnc_relu),
 * SIGMOID 7, TANH 8, CLIP 9. Every step is the corresponding nnc_* op's
 * arithmetic, so the result equals the ops run one call after another
 * through temporaries (bit for bit on this library). NNC_HIP_EINVAL for a
 * malformed program or a short input. Emitted by the mi355x target's O3
 * pass for element-wise nodes each feeding only the next. No counterpart in
 * the reference ABI (which runs each op as its own call, runtime/x86/
 * ops.c:82-258, 2253-2262, 3233-3346). */
enum { NNC_EW_ADD = 0, NNC_EW_SUB, NNC_EW_MUL, NNC_EW_DIV, NNC_EW_ADD_RELU, NNC_EW_ADD_SIGMOID, NNC_EW_RELU,
       NNC_EW_SIGMOID, NNC_EW_TANH, NNC_EW_CLIP, NNC_EW_OPS };
void nnc_hip_fused_eltwise(Tensor** ins, int n_in, const int* prog, int n_steps, const float* consts, Tensor* out);

/* nnc_hip_ew_chain_specialized: 1 if nnc_hip_fused_eltwise runs this chain
 * (n_in inputs, prog of n_steps steps as that call takes them) on a kernel
 * compiled for it - its steps as compile-time code, for the chains the
 * mi355x O3 compiler emits and a few common short ones - and 0 if it runs on
 * the general kernel that reads the steps at run time (same results). A
 * table lookup on the host: no GPU, no device call. No counterpart in the
 * reference ABI. */
int nnc_hip_ew_chain_specialized(int n_in, const int* prog, int n_steps);

/* nnc_hip_add_layernorm: out = layernorm(a + b) over dims [axis:] with
 * scale and bias indexed by the axis dimension - a transformer's residual
 * add and the normalisation after it in one pass, the sum never written.
 * a and b have the same element count (no broadcast). The same bits as
 * nnc_add(a, b, t) then nnc_layernorm(t, scale, bias, out, axis, eps) on this
 * library (the sum is that of nnc_add, the normalisation that of
 * nnc_layernorm). Emitted by the mi355x target's O3 pass for an Add whose
 * only reader is a LayerNormalization. No counterpart in the reference ABI
 * (runtime/x86/ops.c:82-119 then 2095-2171). */
void nnc_hip_add_layernorm(Tensor* a, Tensor* b, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps);

/* nnc_hip_scaled_softmax: out = softmax(in / div[0]) over axis - attention's
 * score scaling and the softmax after it in one pass, the quotient never
 * written. div has one element; out is the size of in. The same bits as
 * nnc_div(in, div, t) then nnc_softmax(t, out, axis) on this library.
 * Emitted by the mi355x target's O3 pass for a Div by a one-element tensor
 * whose only reader is a Softmax. No counterpart in the reference ABI
 * (runtime/x86/ops.c:82-224 then 260-310). */
void nnc_hip_scaled_softmax(Tensor* in, Tensor* div, Tensor* out, int axis);

/* nnc_hip_transpose_slice: out = transpose(view, perm), where view is the
 * block of columns [col0, col0 + width) of in (in read as rows of its last
 * extent W), taken row-major and shaped as out and perm imply (view.shape
 * [perm[d]] = out.shape[d]) - a Split piece along the last axis, reshaped
 * and transposed, read straight from the unsplit tensor. 4-byte elements.
 * The same bits as nnc_split, then nnc_transpose of the reshaped piece.
 * Emitted by the mi355x target's O3 pass for attention's head split. No
 * counterpart in the reference ABI (runtime/x86/ops.c:2183-2251 nnc_split,
 * then 1531-1581 nnc_transpose). */
void nnc_hip_transpose_slice(Tensor* in, Tensor* out, int64_t* perm, int ndim, int col0, int width);

/* nnc_hip_attention: a transformer layer's attention block in one kernel.
 * qkv holds batch * seq rows of ld = qkv.shape[-1] floats (the fused QKV
 * projection's output); head h of Q is columns q_col + h * head_dim ..
 * + head_dim of a batch's seq rows, K and V likewise from k_col and v_col.
 * For every batch b and head h: out[b * seq + i][h * head_dim + d] =
 * sum_j P[i][j] V[j][d], P = softmax over j of (Q K^T)[i][j] / div[0] - the
 * context in the merged-head layout the output projection reads, out of
 * batch * seq rows of heads * head_dim floats. Float32; div one element;
 * head_dim 32 or 64; seq a multiple of 32 up to 128; qkv rows, ld and the
 * three column offsets 16-byte aligned (NNC_HIP_EUNSUPP otherwise). fp32
 * MFMA products and the hardware exponential: within 1e-4 abs / 1e-3 rel of
 * the calls it replaces. Emitted by the mi355x target's O3 pass for the
 * head split (nnc_hip_transpose_slice of the QKV projection), Q K^T, the
 * scaled softmax, the product with V and the head merge. No counterpart in
 * the reference ABI (runtime/x86/ops.c:2183-2251 nnc_split, 1531-1581
 * nnc_transpose, 1607-1730 nnc_matmul, 82-224 nnc_div, 260-310 nnc_softmax;
 * tests/__snapshots__/test_snapshots_simple_transformer.ambr:114-216). */
void nnc_hip_attention(Tensor* qkv, Tensor* div, Tensor* out, int batch, int seq, int heads, int head_dim, int q_col,
                       int k_col, int v_col);

/* nnc_hip_conv_packed_noalloc: nnc_hip_conv_packed for callers that cannot
 * allocate device memory (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference ABI.
 * Same arguments, kernels and results (to the bit) as nnc_hip_conv_packed,
 * but it allocates nothing: its stream-K partial tiles and tile counters
 * live in a static device array of 64 MiB + 16384 counters that each GPU
 * holds until the process ends; a shape needing more fails with
 * NNC_HIP_EUNSUPP before any launch. Calls on one GPU share that array, so
 * they are ordered on the device: each call's stream first waits for the
 * previous call's work (an event recorded after every call, whatever thread
 * or stream made it); inside a graph capture the captured calls are ordered
 * by the graph, and a replay is not ordered against calls made outside it.
 * The calling thread must have its library state already (nnc_hip_init on that thread, or any
 * earlier nnc_* call there): NNC_HIP_ESTATE otherwise. */
void nnc_hip_conv_packed_noalloc(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw,
                                 int sh, int sw, int ph, int pw, int act);

#ifdef __cplusplus
}
#endif

#endif /* NNC_HIP_H */
