/*
 * nnc_oracle.c - CPU restatement of the reference operator arithmetic
 * (runtime/x86/ops.c) behind the same nnc_* ABI (include/nnc_ops.h), on HOST
 * pointers.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the oracle: tests/, the smoke()
 * hook and bench.py's cpu_baseline leg load it to produce expected values or
 * to time the CPU baseline. The product (libnnc_hip.so) never links, loads or
 * falls back to it.
 *
 * Every function reproduces the reference's accumulation order and quirks so
 * that, compiled with -O2 -ffp-contract=off, its results are bit-identical to
 * runtime/x86/ops.c on the same inputs. That claim is pinned three ways:
 *   - tests/test_oracle.py compares every entry point bit-for-bit against the
 *     committed golden vectors in tests/golden/ (produced from the reference
 *     runtime compiled by oracle/Makefile into oracle/_ref/);
 *   - the same file replays the reference's literal known-answer tests
 *     (tests/test_x86_runtime.py, tests/test_numerical_accuracy.py);
 *   - closed forms: float64 numpy for conv/gemm (exact products, one
 *     rounding), numpy for the copies, pools and element-wise ops.
 * Functions whose check is weaker say so in their comment.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "nnc_hip.h"
#include "nnc_ops.h"

#define MAXPOOL_INIT (-3.402823e38f) /* ops.c:347, 366 */
#define CONCAT_STAGING_CAP (64 * 1024 * 1024) /* ops.c:36 */

static int64_t numel(const Tensor* t) {
    int64_t n = 1;
    for (int d = 0; d < t->ndim; ++d) n *= t->shape[d];
    return n;
}

static int64_t prod_range(const int64_t* s, int lo, int hi) {
    int64_t p = 1;
    for (int d = lo; d < hi; ++d) p *= s[d];
    return p;
}

/* ------------------------------------------------------------------------
 * Flat-modulo binary broadcast (ops.c:82-224, 2342-2428, 3233-3346).
 * The reference first writes min(n, a_n, b_n) elements element-wise, then
 * fills the tail only when one operand has exactly n elements and the other
 * fewer; that is out[i] = a[i % a_n] op b[i % b_n] over the returned count.
 * ---------------------------------------------------------------------- */
static int64_t flat_mod_count(int64_t n, int64_t an, int64_t bn) {
    if (an <= 0 || bn <= 0) return 0;
    if (an >= n && bn >= n) return n;
    if ((an == n && bn < n) || (bn == n && an < n)) return n;
    int64_t m = n;
    if (an < m) m = an;
    if (bn < m) m = bn;
    return m;
}

enum { OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_ADD_RELU, OP_ADD_SIGMOID, OP_EQ, OP_AND };

static float apply_binary(int op, float x, float y) {
    switch (op) {
        case OP_ADD: return x + y;
        case OP_SUB: return x - y;
        case OP_MUL: return x * y;
        case OP_DIV: return x / y;
        case OP_ADD_RELU: { float s = x + y; return s > 0.0f ? s : 0.0f; }
        case OP_ADD_SIGMOID: { float s = x + y; return 1.0f / (1.0f + expf(-s)); }
        case OP_EQ: return (x == y) ? 1.0f : 0.0f;
        default: return (x != 0.0f && y != 0.0f) ? 1.0f : 0.0f; /* OP_AND */
    }
}

static void binary(int op, Tensor* a, Tensor* b, Tensor* out) {
    int64_t n = numel(out), an = numel(a), bn = numel(b);
    int64_t cnt = flat_mod_count(n, an, bn);
    const float* x = (const float*)a->data;
    const float* y = (const float*)b->data;
    float* z = (float*)out->data;
    for (int64_t i = 0; i < cnt; ++i) z[i] = apply_binary(op, x[i % an], y[i % bn]);
}

void nnc_add(Tensor* a, Tensor* b, Tensor* o) { binary(OP_ADD, a, b, o); }
void nnc_sub(Tensor* a, Tensor* b, Tensor* o) { binary(OP_SUB, a, b, o); }
void nnc_mul(Tensor* a, Tensor* b, Tensor* o) { binary(OP_MUL, a, b, o); }
void nnc_div(Tensor* a, Tensor* b, Tensor* o) { binary(OP_DIV, a, b, o); }
void nnc_add_relu(Tensor* a, Tensor* b, Tensor* o) { binary(OP_ADD_RELU, a, b, o); }
void nnc_add_sigmoid(Tensor* a, Tensor* b, Tensor* o) { binary(OP_ADD_SIGMOID, a, b, o); }
void nnc_equal(Tensor* a, Tensor* b, Tensor* o) { binary(OP_EQ, a, b, o); }
void nnc_and(Tensor* a, Tensor* b, Tensor* o) { binary(OP_AND, a, b, o); }

/* ops.c:2655-2672: every output element, modulo both operands, uint8 out */
void nnc_greater(Tensor* a, Tensor* b, Tensor* out) {
    int64_t n = numel(out), an = numel(a), bn = numel(b);
    const float* x = (const float*)a->data;
    const float* y = (const float*)b->data;
    uint8_t* z = (uint8_t*)out->data;
    for (int64_t i = 0; i < n; ++i) z[i] = x[i % an] > y[i % bn] ? 1 : 0;
}

/* ops.c:2674-2699: uint8 logic over numel(out), no broadcast */
void nnc_or(Tensor* a, Tensor* b, Tensor* out) {
    int64_t n = numel(out);
    const uint8_t* x = (const uint8_t*)a->data;
    const uint8_t* y = (const uint8_t*)b->data;
    uint8_t* z = (uint8_t*)out->data;
    for (int64_t i = 0; i < n; ++i) z[i] = (x[i] || y[i]) ? 1 : 0;
}

void nnc_not(Tensor* in, Tensor* out) {
    int64_t n = numel(out);
    const uint8_t* x = (const uint8_t*)in->data;
    uint8_t* z = (uint8_t*)out->data;
    for (int64_t i = 0; i < n; ++i) z[i] = x[i] ? 0 : 1;
}

/* ------------------------------------------------------------------------
 * Unary element-wise over numel(output) (ops.c:230-258, 2253-2262,
 * 2434-2515).
 * ---------------------------------------------------------------------- */
enum { U_RELU, U_SIGMOID, U_TANH, U_SQRT, U_POW, U_EXP, U_LOG, U_ABS, U_NEG };

static float apply_unary(int op, float v) {
    switch (op) {
        case U_RELU: return fmaxf(0.0f, v);
        case U_SIGMOID: return 1.0f / (1.0f + expf(-v));
        case U_TANH: return tanhf(v);
        case U_SQRT: return v >= 0.0f ? sqrtf(v) : NAN;
        case U_POW: return v * v;
        case U_EXP: return expf(v);
        case U_LOG: return v > 0.0f ? logf(v) : NAN;
        case U_ABS: return fabsf(v);
        default: return -v;
    }
}

static void unary(int op, Tensor* in, Tensor* out) {
    int64_t n = numel(out);
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    for (int64_t i = 0; i < n; ++i) z[i] = apply_unary(op, x[i]);
}

void nnc_relu(Tensor* i, Tensor* o) { unary(U_RELU, i, o); }
void nnc_sigmoid(Tensor* i, Tensor* o) { unary(U_SIGMOID, i, o); }
void nnc_tanh(Tensor* i, Tensor* o) { unary(U_TANH, i, o); }
void nnc_sqrt(Tensor* i, Tensor* o) { unary(U_SQRT, i, o); }
void nnc_pow(Tensor* i, Tensor* o) { unary(U_POW, i, o); }
void nnc_exp(Tensor* i, Tensor* o) { unary(U_EXP, i, o); }
void nnc_log(Tensor* i, Tensor* o) { unary(U_LOG, i, o); }
void nnc_abs(Tensor* i, Tensor* o) { unary(U_ABS, i, o); }
void nnc_neg(Tensor* i, Tensor* o) { unary(U_NEG, i, o); }

void nnc_clip(Tensor* in, Tensor* out, float lo, float hi) {
    int64_t n = numel(out);
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    for (int64_t i = 0; i < n; ++i) z[i] = fminf(fmaxf(x[i], lo), hi);
}

/* ------------------------------------------------------------------------
 * nnc_hip_fused_eltwise (include/nnc_hip.h): a chain of element-wise ops,
 * target-only, no reference counterpart. Restated as the op-by-op calls it
 * replaces: each step is this file's apply_binary / apply_unary / clip
 * arithmetic (ops.c:82-258, 2253-2262, 3233-3346), applied element by
 * element - with every tensor of numel(out) elements that equals running
 * the steps one call after another through temporaries (every input of an
 * element is read before its output is written, so out may alias an
 * input). Pinned against that composition by tests/test_oracle.py.
 * ---------------------------------------------------------------------- */
/* ------------------------------------------------------------------------
 * nnc_hip_add_layernorm (include/nnc_hip.h): target-only, no reference
 * counterpart. Restated as the two calls it replaces: nnc_add into a
 * temporary (ops.c:82-119), then nnc_layernorm of it (ops.c:2095-2171).
 * ---------------------------------------------------------------------- */
void nnc_hip_add_layernorm(Tensor* a, Tensor* b, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps) {
    int64_t n = numel(a);
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    Tensor t = *a;
    t.data = tmp;
    nnc_add(a, b, &t);
    nnc_layernorm(&t, scale, bias, out, axis, eps);
    free(tmp);
}

/* ------------------------------------------------------------------------
 * nnc_hip_scaled_softmax (include/nnc_hip.h): target-only, no reference
 * counterpart. Restated as the two calls it replaces: nnc_div by the
 * one-element div into a temporary (ops.c:82-224), then nnc_softmax of it
 * (ops.c:260-310).
 * ---------------------------------------------------------------------- */
void nnc_hip_scaled_softmax(Tensor* in, Tensor* div, Tensor* out, int axis) {
    int64_t n = numel(in);
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    Tensor t = *in;
    t.data = tmp;
    nnc_div(in, div, &t);
    nnc_softmax(&t, out, axis);
    free(tmp);
}

void nnc_hip_fused_eltwise(Tensor** ins, int n_in, const int* prog, int n_steps, const float* consts, Tensor* out) {
    static const int bin[] = {OP_ADD, OP_SUB, OP_MUL, OP_DIV, OP_ADD_RELU, OP_ADD_SIGMOID};
    static const int un[] = {U_RELU, U_SIGMOID, U_TANH};
    int64_t n = numel(out);
    float* z = (float*)out->data;
    for (int64_t i = 0; i < n; ++i) {
        float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < n_in && k < 4; ++k) v[k] = ((const float*)ins[k]->data)[i];
        float acc = 0.0f;
        for (int s = 0; s < n_steps; ++s) {
            int op = prog[3 * s], xi = prog[3 * s + 1], yi = prog[3 * s + 2];
            float x = xi < 0 ? acc : v[xi];
            if (op <= NNC_EW_ADD_SIGMOID) {
                float y = yi < 0 ? acc : v[yi];
                acc = apply_binary(bin[op], x, y);
            } else if (op <= NNC_EW_TANH) {
                acc = apply_unary(un[op - NNC_EW_RELU], x);
            } else {
                acc = fminf(fmaxf(x, consts[2 * s]), consts[2 * s + 1]);
            }
        }
        z[i] = acc;
    }
}

/* ------------------------------------------------------------------------
 * Softmax (ops.c:260-310): per (outer, inner) column, max with strict '>'
 * from -inf, sequential float sum of expf(x - max), then a second expf.
 * ---------------------------------------------------------------------- */
void nnc_softmax(Tensor* in, Tensor* out, int axis) {
    int nd = in->ndim;
    if (axis < 0) axis += nd;
    int64_t outer = prod_range(in->shape, 0, axis);
    int64_t dim = in->shape[axis];
    int64_t inner = prod_range(in->shape, axis + 1, nd);
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t q = 0; q < inner; ++q) {
            const int64_t base = o * dim * inner + q;
            float mx = -INFINITY;
            for (int64_t s = 0; s < dim; ++s)
                if (x[base + s * inner] > mx) mx = x[base + s * inner];
            float den = 0.0f;
            for (int64_t s = 0; s < dim; ++s) den += expf(x[base + s * inner] - mx);
            for (int64_t s = 0; s < dim; ++s)
                z[base + s * inner] = expf(x[base + s * inner] - mx) / den;
        }
    }
}

/* ------------------------------------------------------------------------
 * Pooling (ops.c:316-461). N and C come from the input, H_out/W_out from the
 * output; windows are clamped, padding never contributes.
 * ---------------------------------------------------------------------- */
static int pool_args_ok(Tensor* in, Tensor* out) {
    if (!in || !out || !in->data || !out->data) return 0;
    return in->ndim == 4 && out->ndim == 4;
}

void nnc_maxpool2d(Tensor* in, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    if (!pool_args_ok(in, out)) return;
    const int N = (int)in->shape[0], C = (int)in->shape[1];
    const int H = (int)in->shape[2], W = (int)in->shape[3];
    const int Ho = (int)out->shape[2], Wo = (int)out->shape[3];
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    const int64_t total = numel(out);
    for (int64_t i = 0; i < total; ++i) z[i] = MAXPOOL_INIT; /* ops.c:345-348 */
    for (int nc = 0; nc < N * C; ++nc) {
        const float* plane = x + (int64_t)nc * H * W;
        for (int oh = 0; oh < Ho; ++oh) {
            int h0 = oh * sh - ph, h1 = h0 + kh;
            if (h0 < 0) h0 = 0;
            if (h1 > H) h1 = H;
            for (int ow = 0; ow < Wo; ++ow) {
                int w0 = ow * sw - pw, w1 = w0 + kw;
                if (w0 < 0) w0 = 0;
                if (w1 > W) w1 = W;
                float best = MAXPOOL_INIT;
                int seen = 0;
                for (int h = h0; h < h1; ++h)
                    for (int w = w0; w < w1; ++w) {
                        float v = plane[(int64_t)h * W + w];
                        if (!seen || v > best) { best = v; seen = 1; }
                    }
                z[((int64_t)nc * Ho + oh) * Wo + ow] = best;
            }
        }
    }
}

void nnc_avgpool2d(Tensor* in, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    if (!pool_args_ok(in, out)) return;
    const int N = (int)in->shape[0], C = (int)in->shape[1];
    const int H = (int)in->shape[2], W = (int)in->shape[3];
    const int Ho = (int)out->shape[2], Wo = (int)out->shape[3];
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    for (int nc = 0; nc < N * C; ++nc) {
        const float* plane = x + (int64_t)nc * H * W;
        for (int oh = 0; oh < Ho; ++oh) {
            int h0 = oh * sh - ph, h1 = h0 + kh;
            if (h0 < 0) h0 = 0;
            if (h1 > H) h1 = H;
            for (int ow = 0; ow < Wo; ++ow) {
                int w0 = ow * sw - pw, w1 = w0 + kw;
                if (w0 < 0) w0 = 0;
                if (w1 > W) w1 = W;
                float acc = 0.0f;
                int cnt = 0;
                for (int h = h0; h < h1; ++h)
                    for (int w = w0; w < w1; ++w) { acc += plane[(int64_t)h * W + w]; ++cnt; }
                z[((int64_t)nc * Ho + oh) * Wo + ow] = cnt > 0 ? acc / cnt : 0.0f;
            }
        }
    }
}

/* ------------------------------------------------------------------------
 * Convolution (ops.c:720-1504, 3122-3227). Every specialised reference path
 * (1x1, no-pad, 3x3 s1/s2 interiors incl. the SSE2 lanes, 7x7 s2 interior)
 * accumulates in double in the order bias, c_in, kh, kw and skips
 * out-of-bounds taps, so one generic loop reproduces all of them bit-exactly.
 * The fp32 result is rounded once, then the activation is applied
 * (ops.c:473-481).
 * ---------------------------------------------------------------------- */
enum { ACT_NONE, ACT_RELU, ACT_SIGMOID };

static float activate(float v, int act) {
    if (act == ACT_RELU) return v > 0.0f ? v : 0.0f;
    if (act == ACT_SIGMOID) return 1.0f / (1.0f + expf(-v));
    return v;
}

static int conv_args_ok(Tensor* in, Tensor* w, Tensor* out, const char* name, int need_4d) {
    if (!in || !w || !out) {
        fprintf(stderr, "%s: NULL tensor pointer\n", name);
        return 0;
    }
    if (!in->data || !w->data || !out->data) {
        fprintf(stderr, "%s: NULL data pointer\n", name);
        return 0;
    }
    if (!in->shape || !w->shape || !out->shape) {
        fprintf(stderr, "%s: NULL shape pointer\n", name);
        return 0;
    }
    if (need_4d && (in->ndim != 4 || w->ndim != 4 || out->ndim != 4)) {
        fprintf(stderr, "%s: expected 4D tensors\n", name);
        return 0;
    }
    return 1;
}

static void conv_generic(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw,
                         int sh, int sw, int ph, int pw, int act) {
    const int N = (int)in->shape[0], Ci = (int)in->shape[1];
    const int H = (int)in->shape[2], W = (int)in->shape[3];
    const int Co = (int)w->shape[0];
    const int Ho = (int)out->shape[2], Wo = (int)out->shape[3];
    const float* x = (const float*)in->data;
    const float* wt = (const float*)w->data;
    const float* bias = b ? (const float*)b->data : NULL;
    float* z = (float*)out->data;
    const int64_t taps = (int64_t)Ci * kh * kw;
    /* output planes are independent and each element's sum is the same
     * sequential loop whichever thread runs it: threads change the time, not
     * a bit of the result */
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
    for (int n = 0; n < N; ++n) {
        for (int co = 0; co < Co; ++co) {
            const float* img = x + (int64_t)n * Ci * H * W;
            const float* filt = wt + (int64_t)co * taps;
            float* plane = z + ((int64_t)n * Co + co) * Ho * Wo;
            for (int oh = 0; oh < Ho; ++oh) {
                for (int ow = 0; ow < Wo; ++ow) {
                    double acc = bias ? (double)bias[co] : 0.0;
                    const int hb = oh * sh - ph, wb = ow * sw - pw;
                    for (int ci = 0; ci < Ci; ++ci) {
                        const float* chan = img + (int64_t)ci * H * W;
                        const float* f = filt + (int64_t)ci * kh * kw;
                        for (int r = 0; r < kh; ++r) {
                            const int h = hb + r;
                            if (h < 0 || h >= H) continue;
                            for (int c = 0; c < kw; ++c) {
                                const int ww = wb + c;
                                if (ww < 0 || ww >= W) continue;
                                acc += (double)chan[(int64_t)h * W + ww] * (double)f[r * kw + c];
                            }
                        }
                    }
                    plane[(int64_t)oh * Wo + ow] = activate((float)acc, act);
                }
            }
        }
    }
}

#define CONV_ENTRY(fname, act)                                                        \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, \
               int sw, int ph, int pw) {                                              \
        if (!conv_args_ok(in, w, out, #fname, 0)) return;                             \
        conv_generic(in, w, b, out, kh, kw, sh, sw, ph, pw, act);                     \
    }
CONV_ENTRY(nnc_conv, ACT_NONE)
CONV_ENTRY(nnc_conv_relu, ACT_RELU)
CONV_ENTRY(nnc_conv_sigmoid, ACT_SIGMOID)

#define CONV1X1_ENTRY(fname, act)                                                      \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int sh, int sw, int ph,  \
               int pw) {                                                               \
        if (!conv_args_ok(in, w, out, #fname, 1)) return;                              \
        conv_generic(in, w, b, out, 1, 1, sh, sw, ph, pw, act);                        \
    }
CONV1X1_ENTRY(nnc_conv1x1, ACT_NONE)
CONV1X1_ENTRY(nnc_conv_relu1x1, ACT_RELU)

#define CONV3X3_ENTRY(fname, act)                                                  \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {                    \
        if (!conv_args_ok(in, w, out, #fname, 1)) return;                          \
        if (out->shape[2] != in->shape[2] || out->shape[3] != in->shape[3]) {      \
            fprintf(stderr, "%s: expected same-padding output shape\n", #fname);   \
            return;                                                                \
        }                                                                          \
        conv_generic(in, w, b, out, 3, 3, 1, 1, 1, 1, act);                        \
    }
CONV3X3_ENTRY(nnc_conv3x3_s1, ACT_NONE)
CONV3X3_ENTRY(nnc_conv_relu3x3_s1, ACT_RELU)

#define CONV7X7_ENTRY(fname, act)                               \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out) { \
        if (!conv_args_ok(in, w, out, #fname, 1)) return;       \
        conv_generic(in, w, b, out, 7, 7, 2, 2, 3, 3, act);     \
    }
CONV7X7_ENTRY(nnc_conv7x7_s2, ACT_NONE)
CONV7X7_ENTRY(nnc_conv_relu7x7_s2, ACT_RELU)

/* ------------------------------------------------------------------------
 * Shape manipulation (ops.c:1510-1601, 2264-2336): element copies of
 * numel(output) floats.
 * ---------------------------------------------------------------------- */
static void copy_out_count(Tensor* in, Tensor* out) {
    int64_t n = numel(out);
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    if (x == z) return;
    for (int64_t i = 0; i < n; ++i) z[i] = x[i];
}

void nnc_reshape(Tensor* in, Tensor* out, int64_t* shape, int ndim) {
    (void)shape; (void)ndim;
    copy_out_count(in, out);
}
void nnc_flatten(Tensor* in, Tensor* out, int axis) { (void)axis; copy_out_count(in, out); }
void nnc_squeeze(Tensor* in, Tensor* out, int axis) { (void)axis; copy_out_count(in, out); }
void nnc_unsqueeze(Tensor* in, Tensor* out, int axis) { (void)axis; copy_out_count(in, out); }

/* ops.c:1531-1581: out index decomposed with output strides, each output
 * axis d reads input axis perm[d]; perm NULL = reversed axes. */
void nnc_transpose(Tensor* in, Tensor* out, int64_t* perm, int ndim) {
    int64_t rev[8], is[8], os[8];
    if (!perm) {
        for (int d = 0; d < ndim; ++d) rev[d] = ndim - 1 - d;
        perm = rev;
    }
    is[ndim - 1] = 1;
    os[ndim - 1] = 1;
    for (int d = ndim - 2; d >= 0; --d) {
        is[d] = is[d + 1] * in->shape[d + 1];
        os[d] = os[d + 1] * out->shape[d + 1];
    }
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    const int64_t total = numel(out);
    for (int64_t o = 0; o < total; ++o) {
        int64_t rem = o, src = 0;
        for (int d = 0; d < ndim; ++d) {
            src += (rem / os[d]) * is[perm[d]];
            rem %= os[d];
        }
        z[o] = x[src];
    }
}

/* ops.c:2264-2336: output coordinate modulo input extent per axis; repeats
 * only decide the NULL shortcut (the output shape already encodes them). */
void nnc_tile(Tensor* in, Tensor* out, int64_t* repeats, int ndim) {
    (void)ndim;
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    if (!repeats) { copy_out_count(in, out); return; }
    int64_t is[8];
    is[in->ndim - 1] = 1;
    for (int d = in->ndim - 2; d >= 0; --d) is[d] = is[d + 1] * in->shape[d + 1];
    const int64_t total = numel(out);
    for (int64_t o = 0; o < total; ++o) {
        int64_t coord[8], rem = o, src = 0;
        for (int d = out->ndim - 1; d >= 0; --d) { coord[d] = rem % out->shape[d]; rem /= out->shape[d]; }
        for (int d = 0; d < in->ndim; ++d) src += (coord[d] % in->shape[d]) * is[d];
        z[o] = x[src];
    }
}

/* ------------------------------------------------------------------------
 * MatMul (ops.c:1607-1730): every dot product is a Kahan-compensated float
 * sum of float products, k ascending. Batched case reproduces the
 * reference's batch stepping (A and B advance by their batch COUNT per
 * batch, ops.c:1687-1704); it equals true batched MatMul only for one batch.
 * ---------------------------------------------------------------------- */
static float kahan_dot(const float* a, int64_t sa, const float* b, int64_t sb, int K) {
    float s = 0.0f, c = 0.0f;
    for (int k = 0; k < K; ++k) {
        float y = a[(int64_t)k * sa] * b[(int64_t)k * sb] - c;
        float t = s + y;
        c = (t - s) - y;
        s = t;
    }
    return s;
}

void nnc_matmul(Tensor* a, Tensor* b, Tensor* out) {
    const float* A = (const float*)a->data;
    const float* B = (const float*)b->data;
    float* Z = (float*)out->data;
    const int an = a->ndim, bnd = b->ndim, on = out->ndim;
    if (an == 2 && bnd == 2) {
        const int M = (int)a->shape[0], K = (int)a->shape[1], N = (int)b->shape[1];
        for (int i = 0; i < M; ++i)
            for (int j = 0; j < N; ++j) Z[i * N + j] = kahan_dot(A + i * K, 1, B + j, N, K);
    } else if (an == 1 && bnd == 2) {
        const int K = (int)a->shape[0], N = (int)b->shape[1];
        for (int j = 0; j < N; ++j) Z[j] = kahan_dot(A, 1, B + j, N, K);
    } else if (an == 2 && bnd == 1) {
        const int M = (int)a->shape[0], K = (int)a->shape[1];
        for (int i = 0; i < M; ++i) Z[i] = kahan_dot(A + i * K, 1, B, 1, K);
    } else if (an >= 2 && bnd >= 2) {
        const int64_t batches = prod_range(out->shape, 0, on - 2);
        const int M = (int)out->shape[on - 2], N = (int)out->shape[on - 1];
        const int K = (int)a->shape[an - 1];
        const int64_t a_step = numel(a) / (a->shape[an - 2] * a->shape[an - 1]);
        const int64_t b_step = bnd < on ? 0 : numel(b) / (b->shape[bnd - 2] * b->shape[bnd - 1]);
        for (int64_t q = 0; q < batches; ++q) {
            const float* Aq = A + q * a_step;
            const float* Bq = B + q * b_step;
            float* Zq = Z + q * (int64_t)M * N;
            for (int i = 0; i < M; ++i)
                for (int j = 0; j < N; ++j) Zq[i * N + j] = kahan_dot(Aq + i * K, 1, Bq + j, N, K);
        }
    }
}

/* relu(matmul + bias) for the emitted-but-undefined reference call
 * (c_emitter.py:1143-1171 passes a, b, bias-or-NULL, out); the bias is added
 * per column ([N]) or element-wise ([M, N]) before the Relu. */
void nnc_matmul_relu(Tensor* a, Tensor* b, Tensor* bias, Tensor* out) {
    nnc_matmul(a, b, out);
    if (bias && bias->data) {
        const int64_t n = numel(out), bn = numel(bias);
        float* z = (float*)out->data;
        const float* bb = (const float*)bias->data;
        for (int64_t i = 0; i < n; ++i) z[i] += bb[i % bn];
    }
    nnc_relu(out, out);
}

/* ------------------------------------------------------------------------
 * Gemm (ops.c:1732-1841) and Gemm_nt (ops.c:1843-1886): double dot product
 * in k order, times alpha, plus beta*C in double, rounded once.
 * ---------------------------------------------------------------------- */
static float gemm_finish(double acc, float alpha, float beta, const Tensor* c, const float* cd,
                         int i, int j, int N) {
    acc *= (double)alpha;
    if (cd) {
        float cv = c->ndim == 1 ? cd[j] : cd[(int64_t)i * N + j];
        acc += (double)beta * (double)cv;
    }
    return (float)acc;
}

void nnc_gemm(Tensor* a, Tensor* b, Tensor* c, Tensor* out, float alpha, float beta, int ta,
              int tb) {
    const float* A = (const float*)a->data;
    const float* B = (const float*)b->data;
    const float* Cd = c ? (const float*)c->data : NULL;
    float* Z = (float*)out->data;
    int M, K, N;
    if (a->ndim == 2 && b->ndim == 2) {
        M = (int)(ta ? a->shape[1] : a->shape[0]);
        K = (int)(ta ? a->shape[0] : a->shape[1]);
        N = (int)(tb ? b->shape[0] : b->shape[1]);
    } else if (a->ndim == 1 && b->ndim == 2) {
        M = 1; K = (int)a->shape[0]; N = (int)b->shape[1]; ta = 0;
    } else if (a->ndim == 2 && b->ndim == 1) {
        M = (int)a->shape[0]; K = (int)a->shape[1]; N = 1; tb = 0;
    } else {
        M = 1; K = (int)numel(a); N = (int)numel(b);
    }
    for (int i = 0; i < M; ++i) {
        for (int j = 0; j < N; ++j) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) {
                const float av = ta ? A[(int64_t)k * M + i] : A[(int64_t)i * K + k];
                const float bv = tb ? B[(int64_t)j * K + k] : B[(int64_t)k * N + j];
                acc += (double)av * (double)bv;
            }
            Z[(int64_t)i * N + j] = gemm_finish(acc, alpha, beta, c, Cd, i, j, N);
        }
    }
}

void nnc_gemm_nt(Tensor* a, Tensor* b, Tensor* c, Tensor* out, float alpha, float beta) {
    const float* A = (const float*)a->data;
    const float* B = (const float*)b->data;
    const float* Cd = c ? (const float*)c->data : NULL;
    float* Z = (float*)out->data;
    int M, K, N;
    if (a->ndim == 2 && b->ndim == 2) {
        M = (int)a->shape[0]; K = (int)a->shape[1]; N = (int)b->shape[0];
    } else if (a->ndim == 1 && b->ndim == 2) {
        M = 1; K = (int)a->shape[0]; N = (int)b->shape[0];
    } else {
        M = 1; K = (int)numel(a); N = b->ndim == 2 ? (int)b->shape[0] : (int)numel(b);
    }
    for (int i = 0; i < M; ++i) {
        const float* arow = a->ndim == 1 ? A : A + (int64_t)i * K;
        for (int j = 0; j < N; ++j) {
            const float* brow = B + (int64_t)j * K;
            double acc = 0.0;
            for (int k = 0; k < K; ++k) acc += (double)arow[k] * (double)brow[k];
            Z[(int64_t)i * N + j] = gemm_finish(acc, alpha, beta, c, Cd, i, j, N);
        }
    }
}

/* ------------------------------------------------------------------------
 * ReduceMean / ReduceSum over one axis (ops.c:1892-1989): Kahan float sum
 * in axis order; mean = sum / (float)len. keepdims does not move elements.
 * ---------------------------------------------------------------------- */
static void reduce_axis(Tensor* in, Tensor* out, int axis, int mean) {
    const int nd = in->ndim;
    if (axis < 0) axis += nd;
    const int64_t outer = prod_range(in->shape, 0, axis);
    const int64_t len = in->shape[axis];
    const int64_t inner = prod_range(in->shape, axis + 1, nd);
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    for (int64_t o = 0; o < outer; ++o)
        for (int64_t q = 0; q < inner; ++q) {
            float s = 0.0f, c = 0.0f;
            for (int64_t r = 0; r < len; ++r) {
                float y = x[(o * len + r) * inner + q] - c;
                float t = s + y;
                c = (t - s) - y;
                s = t;
            }
            z[o * inner + q] = mean ? s / (float)len : s;
        }
}

void nnc_reducemean(Tensor* in, Tensor* out, int axis, int keepdims) {
    (void)keepdims;
    reduce_axis(in, out, axis, 1);
}
void nnc_reducesum(Tensor* in, Tensor* out, int axis, int keepdims) {
    (void)keepdims;
    reduce_axis(in, out, axis, 0);
}

/* ------------------------------------------------------------------------
 * Concat (ops.c:1995-2086): element size 8 for INT64 outputs else 4; the
 * reference stages through a 64 MiB buffer and refuses larger outputs with
 * a message, leaving the output untouched. Restated with the same cap.
 * ---------------------------------------------------------------------- */
void nnc_concat(Tensor** ins, Tensor* out, int n_in, int axis) {
    if (axis < 0) axis += out->ndim;
    const size_t esz = out->dtype == NNC_DTYPE_INT64 ? 8 : 4;
    const int64_t total = numel(out);
    if ((size_t)total * esz > (size_t)CONCAT_STAGING_CAP) {
        fprintf(stderr, "nnc_concat: output size %zu exceeds slow memory buffer %d\n",
                (size_t)total * esz, CONCAT_STAGING_CAP);
        return;
    }
    const int64_t outer = prod_range(out->shape, 0, axis);
    const int64_t inner = prod_range(out->shape, axis + 1, out->ndim);
    const int64_t out_row = out->shape[axis] * inner;
    char* staging = (char*)malloc((size_t)total * esz + 1);
    int64_t col = 0;
    for (int t = 0; t < n_in; ++t) {
        const int64_t slab = ins[t]->shape[axis] * inner;
        const char* src = (const char*)ins[t]->data;
        for (int64_t o = 0; o < outer; ++o)
            memcpy(staging + (size_t)(o * out_row + col) * esz, src + (size_t)(o * slab) * esz,
                   (size_t)slab * esz);
        col += slab;
    }
    memcpy(out->data, staging, (size_t)total * esz);
    free(staging);
}

/* ops.c:2183-2251: equal parts of dim / num_outputs; int64 when the INPUT
 * dtype is INT64. */
void nnc_split(Tensor* in, Tensor** outs, int n_out, int axis) {
    if (axis < 0) axis += in->ndim;
    const size_t esz = in->dtype == NNC_DTYPE_INT64 ? 8 : 4;
    const int64_t outer = prod_range(in->shape, 0, axis);
    const int64_t dim = in->shape[axis];
    const int64_t part = dim / n_out;
    const int64_t inner = prod_range(in->shape, axis + 1, in->ndim);
    const char* src = (const char*)in->data;
    for (int t = 0; t < n_out; ++t) {
        char* dst = (char*)outs[t]->data;
        for (int64_t o = 0; o < outer; ++o)
            memcpy(dst + (size_t)(o * part * inner) * esz,
                   src + (size_t)(o * dim * inner + t * part * inner) * esz,
                   (size_t)(part * inner) * esz);
    }
}

/* ops.c:2088-2093 */
void nnc_batchnorm(Tensor* in, Tensor* s, Tensor* b, Tensor* m, Tensor* v, Tensor* out, float eps,
                   int momentum) {
    (void)in; (void)s; (void)b; (void)m; (void)v; (void)out; (void)eps; (void)momentum;
}

/* ------------------------------------------------------------------------
 * LayerNorm (ops.c:2095-2171): per outer slice of norm_size*inner floats,
 * sequential float mean, then sequential float variance of (x - mean),
 * std = sqrtf(var + eps), y = scale[i] * ((x - mean) / std) + bias[i] where i
 * indexes the axis dimension only.
 * ---------------------------------------------------------------------- */
void nnc_layernorm(Tensor* in, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps) {
    const int nd = in->ndim;
    if (axis < 0) axis += nd;
    const int64_t D = in->shape[axis];
    const int64_t outer = prod_range(in->shape, 0, axis);
    const int64_t inner = prod_range(in->shape, axis + 1, nd);
    const int64_t span = D * inner;
    const float* x = (const float*)in->data;
    const float* g = scale ? (const float*)scale->data : NULL;
    const float* bb = bias ? (const float*)bias->data : NULL;
    float* z = (float*)out->data;
    for (int64_t o = 0; o < outer; ++o) {
        const float* row = x + o * span;
        float* dst = z + o * span;
        float mu = 0.0f;
        for (int64_t e = 0; e < span; ++e) mu += row[e];
        mu /= (float)span;
        float var = 0.0f;
        for (int64_t e = 0; e < span; ++e) { float d = row[e] - mu; var += d * d; }
        var /= (float)span;
        const float sd = sqrtf(var + eps);
        for (int64_t i = 0; i < D; ++i) {
            const float gi = g ? g[i] : 1.0f, bi = bb ? bb[i] : 0.0f;
            for (int64_t q = 0; q < inner; ++q) {
                const float nv = (row[i * inner + q] - mu) / sd;
                dst[i * inner + q] = gi * nv + bi;
            }
        }
    }
}

/* ops.c:2173-2181: min(numel(out), numel(in)) floats */
void nnc_identity(Tensor* in, Tensor* out) {
    int64_t n = numel(out), m = numel(in);
    if (m < n) n = m;
    memmove(out->data, in->data, (size_t)n * sizeof(float));
}

/* ------------------------------------------------------------------------
 * Cast / Shape / ConstantOfShape / Expand (ops.c:2517-2653).
 * ---------------------------------------------------------------------- */
void nnc_cast(Tensor* in, Tensor* out, int to) {
    const int64_t n = numel(in);
    const int from_bool = in->dtype == NNC_DTYPE_BOOL;
    const uint8_t* xb = (const uint8_t*)in->data;
    const float* xf = (const float*)in->data;
    switch (to) {
        case NNC_DTYPE_FLOAT32:
            if (from_bool) {
                float* z = (float*)out->data;
                for (int64_t i = 0; i < n; ++i) z[i] = (float)xb[i];
            } else {
                memmove(out->data, in->data, (size_t)n * 4);
            }
            break;
        case NNC_DTYPE_INT32: {
            int32_t* z = (int32_t*)out->data;
            for (int64_t i = 0; i < n; ++i) z[i] = from_bool ? (int32_t)xb[i] : (int32_t)xf[i];
            break;
        }
        case NNC_DTYPE_INT64: {
            int64_t* z = (int64_t*)out->data;
            for (int64_t i = 0; i < n; ++i) z[i] = from_bool ? (int64_t)xb[i] : (int64_t)xf[i];
            break;
        }
        case NNC_DTYPE_BOOL: {
            uint8_t* z = (uint8_t*)out->data;
            if (from_bool) memmove(z, xb, (size_t)n);
            else for (int64_t i = 0; i < n; ++i) z[i] = xf[i] != 0.0f ? 1 : 0;
            break;
        }
        default: /* FLOAT16 and unknown targets: 4-byte copy (ops.c:2539-2542, 2593-2596) */
            memmove(out->data, in->data, (size_t)n * 4);
            break;
    }
}

void nnc_shape(Tensor* in, Tensor* out, int64_t* shape_data, int ndim) {
    int64_t* z = (int64_t*)out->data;
    for (int d = 0; d < ndim; ++d) z[d] = shape_data ? shape_data[d] : in->shape[d];
}

void nnc_constantofshape(Tensor* out, float value, int ndim) {
    (void)ndim;
    const int64_t n = numel(out);
    float* z = (float*)out->data;
    for (int64_t i = 0; i < n; ++i) z[i] = value;
}

void nnc_expand(Tensor* in, Tensor* out, int64_t* shape, int ndim) {
    (void)shape; (void)ndim;
    const int64_t m = numel(in), n = numel(out);
    const float* x = (const float*)in->data;
    float* z = (float*)out->data;
    if (m == n) { memmove(z, x, (size_t)n * 4); return; }
    for (int64_t i = 0; i < n; ++i) z[i] = x[i % m];
}

/* ------------------------------------------------------------------------
 * Gather (ops.c:2705-2913). The reference handles a scalar / single index
 * for rank 1-3 data, a 1-D index list for rank-1 int64 and rank-2 float data,
 * and otherwise copies data[i % numel(data)]. Indices are int64, negative
 * ones wrap once, then clamp to [0, dim-1].
 * ---------------------------------------------------------------------- */
static int64_t clamp_index(int64_t v, int64_t dim) {
    if (v < 0) v += dim;
    if (v < 0) v = 0;
    if (v >= dim) v = dim - 1;
    return v;
}

void nnc_gather(Tensor* data, Tensor* indices, Tensor* out, int axis, int data_dtype) {
    const int64_t* idx = (const int64_t*)indices->data;
    const int rank = data->ndim, irank = indices->ndim, orank = out->ndim;
    if (axis < 0) axis += rank;
    if (axis < 0) axis = 0;
    if (axis >= rank) axis = rank - 1;
    const int64_t on = numel(out);
    if (irank == 0 || (irank == 1 && indices->shape[0] == 1)) {
        const int64_t g = clamp_index(idx[0], data->shape[axis]);
        if (data_dtype == 1) {
            const int64_t* d = (const int64_t*)data->data;
            int64_t* z = (int64_t*)out->data;
            if (rank == 1) { z[0] = d[g]; return; }
            const int64_t row = prod_range(data->shape, axis + 1, rank);
            for (int64_t i = 0; i < row; ++i) z[i] = d[g * row + i];
            return;
        }
        const float* d = (const float*)data->data;
        float* z = (float*)out->data;
        if (rank == 1) { for (int64_t i = 0; i < on; ++i) z[i] = d[g]; return; }
        if (rank == 2 && orank == 2) {
            const int64_t d1 = data->shape[1], o0 = out->shape[0], o1 = out->shape[1];
            for (int64_t i = 0; i < o0; ++i)
                for (int64_t j = 0; j < o1; ++j)
                    z[i * o1 + j] = axis == 0 ? d[g * d1 + j] : d[i * d1 + g];
            return;
        }
        if (rank == 3) {
            const int64_t d0 = data->shape[0], d1 = data->shape[1], d2 = data->shape[2];
            if (axis == 0 && orank == 2) {
                for (int64_t i = 0; i < d1 * d2; ++i) z[i] = d[g * d1 * d2 + i];
                return;
            }
            if (axis == 0 && orank == 3) {
                const int64_t o0 = out->shape[0], o1 = out->shape[1], o2 = out->shape[2];
                for (int64_t i = 0; i < o0; ++i)
                    for (int64_t j = 0; j < o1; ++j)
                        for (int64_t k = 0; k < o2; ++k)
                            z[(i * o1 + j) * o2 + k] = d[g * d1 * d2 + j * d2 + k];
                return;
            }
            if (axis == 1) {
                for (int64_t i = 0; i < d0; ++i)
                    for (int64_t k = 0; k < d2; ++k) z[i * d2 + k] = d[(i * d1 + g) * d2 + k];
                return;
            }
            if (axis == 2) {
                for (int64_t i = 0; i < d0; ++i)
                    for (int64_t j = 0; j < d1; ++j) z[i * d1 + j] = d[(i * d1 + j) * d2 + g];
                return;
            }
        }
    }
    if (irank == 1) {
        const int64_t cnt = indices->shape[0];
        if (data_dtype == 1 && rank == 1) {
            const int64_t* d = (const int64_t*)data->data;
            int64_t* z = (int64_t*)out->data;
            for (int64_t i = 0; i < cnt; ++i) z[i] = d[clamp_index(idx[i], data->shape[0])];
            return;
        }
        if (rank == 2) {
            const float* d = (const float*)data->data;
            float* z = (float*)out->data;
            const int64_t d1 = data->shape[1];
            for (int64_t t = 0; t < cnt; ++t) {
                const int64_t g = clamp_index(idx[t], data->shape[axis]);
                if (axis == 0) {
                    for (int64_t j = 0; j < d1; ++j) z[t * d1 + j] = d[g * d1 + j];
                } else {
                    for (int64_t i = 0; i < data->shape[0]; ++i) z[i * cnt + t] = d[i * d1 + g];
                }
            }
            return;
        }
    }
    const int64_t dn = numel(data);
    if (data_dtype == 1) {
        const int64_t* d = (const int64_t*)data->data;
        int64_t* z = (int64_t*)out->data;
        for (int64_t i = 0; i < on; ++i) z[i] = d[i % dn];
    } else {
        const float* d = (const float*)data->data;
        float* z = (float*)out->data;
        for (int64_t i = 0; i < on; ++i) z[i] = d[i % dn];
    }
}

/* ------------------------------------------------------------------------
 * LSTM (ops.c:2918-3116). Gate order I, O, F, C; each gate is a float sum
 * W.x then R.h then (Wb + Rb). As in the reference, one (h, c) state runs
 * through the batch elements of a time step in order, and the Y layout is
 * [seq][dirs][batch][hidden].
 * ---------------------------------------------------------------------- */
static float lstm_gate(const float* Wg, const float* Rg, const float* x, const float* h, int in_sz,
                       int hid) {
    float g = 0.0f;
    for (int j = 0; j < in_sz; ++j) g += Wg[j] * x[j];
    for (int j = 0; j < hid; ++j) g += Rg[j] * h[j];
    return g;
}

void nnc_lstm(Tensor* X, Tensor* W, Tensor* R, Tensor* B, Tensor* Y, Tensor* Yh, Tensor* Yc,
              int direction, int hid) {
    const int64_t T = X->shape[0], Bt = X->shape[1];
    const int in_sz = (int)X->shape[2];
    const int dirs = direction == 2 ? 2 : 1;
    const float* xd = (const float*)X->data;
    const float* wd = (const float*)W->data;
    const float* rd = (const float*)R->data;
    const float* bd = B ? (const float*)B->data : NULL;
    float* yd = (float*)Y->data;
    float* yh = (float*)Yh->data;
    float* yc = (float*)Yc->data;
    float* h = (float*)calloc((size_t)hid, sizeof(float));
    float* c = (float*)calloc((size_t)hid, sizeof(float));
    float* hn = (float*)malloc((size_t)hid * sizeof(float));
    float* cn = (float*)malloc((size_t)hid * sizeof(float));
    for (int dir = 0; dir < dirs; ++dir) {
        memset(h, 0, (size_t)hid * sizeof(float));
        memset(c, 0, (size_t)hid * sizeof(float));
        const float* Wd = wd + (int64_t)dir * 4 * hid * in_sz;
        const float* Rd = rd + (int64_t)dir * 4 * hid * hid;
        const float* Bd = bd ? bd + (int64_t)dir * 8 * hid : NULL;
        for (int64_t t = 0; t < T; ++t) {
            const int64_t ts = dir == 1 ? T - 1 - t : t;
            for (int64_t b = 0; b < Bt; ++b) {
                const float* xt = xd + (ts * Bt + b) * in_sz;
                for (int i = 0; i < hid; ++i) {
                    float gate[4];
                    for (int q = 0; q < 4; ++q) {
                        gate[q] = lstm_gate(Wd + ((int64_t)q * hid + i) * in_sz,
                                            Rd + ((int64_t)q * hid + i) * hid, xt, h, in_sz, hid);
                        if (Bd) gate[q] += Bd[q * hid + i] + Bd[(4 + q) * hid + i];
                    }
                    const float ig = 1.0f / (1.0f + expf(-gate[0]));
                    const float og = 1.0f / (1.0f + expf(-gate[1]));
                    const float fg = 1.0f / (1.0f + expf(-gate[2]));
                    const float gg = tanhf(gate[3]);
                    cn[i] = fg * c[i] + ig * gg;
                    hn[i] = og * tanhf(cn[i]);
                }
                memcpy(h, hn, (size_t)hid * sizeof(float));
                memcpy(c, cn, (size_t)hid * sizeof(float));
                float* yt = yd + ((t * dirs + dir) * Bt + b) * hid;
                memcpy(yt, h, (size_t)hid * sizeof(float));
            }
        }
        for (int64_t b = 0; b < Bt; ++b) {
            memcpy(yh + (dir * Bt + b) * hid, h, (size_t)hid * sizeof(float));
            memcpy(yc + (dir * Bt + b) * hid, c, (size_t)hid * sizeof(float));
        }
    }
    free(h); free(c); free(hn); free(cn);
}

/* ------------------------------------------------------------------------
 * Fused operator of the mi355x target (include/nnc_hip.h), no reference
 * counterpart: restated as the composition it replaces, nnc_conv into a
 * temporary and nnc_add_relu(conv_out, res, out) (ops.c:1449-1463,
 * 3233-3288). `res` may alias `out`. Pinned by composition of two pinned
 * entry points.
 * ---------------------------------------------------------------------- */
void nnc_hip_conv_add_relu(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw,
                           int sh, int sw, int ph, int pw) {
    const int64_t n = numel(out);
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!tmp) return;
    Tensor t = *out;
    t.data = tmp;
    nnc_conv(in, w, b, &t, kh, kw, sh, sw, ph, pw);
    nnc_add_relu(&t, res, out);
    free(tmp);
}

/* ------------------------------------------------------------------------
 * Spill / reload of the mi355x target (include/nnc_hip.h): a byte copy of
 * src into dst, as the reference's spill and reload code copies between its
 * fast and slow pools (codegen/x86_emitters/model_source.py:276-287). Pinned
 * by the spill tests: a program under a memory budget computes the same
 * bytes as without one.
 * ---------------------------------------------------------------------- */
void nnc_hip_transfer(Tensor* src, Tensor* dst) {
    if (!src || !dst || !src->data || !dst->data || src->nbytes != dst->nbytes) return;
    memmove(dst->data, src->data, (size_t)src->nbytes);
}

/* ------------------------------------------------------------------------
 * Packed-weight convolution of the mi355x target (include/nnc_hip.h), no
 * reference counterpart: the weights, [Co][kh][kw][Ci] or [Co][Kp] (rows of
 * K = kh*kw*Ci tap-major values padded to Kp), are unpacked to the
 * reference layout [Co][Ci][kh][kw], then nnc_conv into a temporary
 * (ops.c:720-1050) followed by the element-wise op that applies residual and
 * activation: nnc_add / nnc_add_relu / nnc_add_sigmoid with `res`
 * (ops.c:82-110, 3233-3346), or nnc_relu / nnc_sigmoid without it
 * (ops.c:230-246). Pinned by composition of pinned entry points.
 * ---------------------------------------------------------------------- */
void nnc_hip_conv_packed(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh,
                         int sw, int ph, int pw, int act) {
    if (!in || !w || !out || (w->ndim != 4 && w->ndim != 2) || in->ndim != 4) return;
    const int64_t co = w->shape[0], ci = in->shape[1], taps = (int64_t)kh * kw;
    const int64_t row = w->ndim == 2 ? w->shape[1] : taps * ci;
    const int64_t n = numel(out);
    float* wt = (float*)malloc((size_t)(co * ci * taps > 0 ? co * ci * taps : 1) * sizeof(float));
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!wt || !tmp) {
        free(wt);
        free(tmp);
        return;
    }
    const float* wp = (const float*)w->data;
    for (int64_t o = 0; o < co; ++o)
        for (int64_t t = 0; t < taps; ++t)
            for (int64_t c = 0; c < ci; ++c) wt[(o * ci + c) * taps + t] = wp[o * row + t * ci + c];
    int64_t wshape[4] = {co, ci, kh, kw};
    Tensor wu = *w;
    wu.data = wt;
    wu.shape = wshape;
    wu.nbytes = (size_t)(co * ci * taps) * sizeof(float);
    Tensor t = *out;
    t.data = tmp;
    nnc_conv(in, &wu, b, &t, kh, kw, sh, sw, ph, pw);
    if (res) {
        if (act == 1)
            nnc_add_relu(&t, res, out);
        else if (act == 2)
            nnc_add_sigmoid(&t, res, out);
        else
            nnc_add(&t, res, out);
    } else if (act == 1) {
        nnc_relu(&t, out);
    } else if (act == 2) {
        nnc_sigmoid(&t, out);
    } else {
        memcpy(out->data, tmp, (size_t)n * sizeof(float));
    }
    free(wt);
    free(tmp);
}

/* ------------------------------------------------------------------------
 * Convolution with a folded 1x1 projection of the mi355x target
 * (include/nnc_hip.h), no reference counterpart: the rows of w, [Co][kh*kw*Ci
 * + Cx], are split into the tap-major kernel and the projection weights;
 * nnc_conv of x with the projection (1x1, stride psh x psw, no bias,
 * ops.c:720-1050) gives the residual that nnc_hip_conv_packed (above) adds
 * before the activation, as the reference's Conv -> Conv -> Add -> Relu
 * sequence would. Pinned by composition of pinned entry points.
 * ---------------------------------------------------------------------- */
void nnc_hip_conv_proj(Tensor* in, Tensor* w, Tensor* b, Tensor* x, Tensor* out, int kh, int kw, int sh, int sw,
                       int ph, int pw, int psh, int psw, int act) {
    if (!in || !w || !x || !out || w->ndim != 2 || in->ndim != 4 || x->ndim != 4 || out->ndim != 4) return;
    const int64_t co = w->shape[0], ci = in->shape[1], cx = x->shape[1], taps = (int64_t)kh * kw;
    const int64_t row = w->shape[1], k3 = taps * ci;
    if (row != k3 + cx) return;
    const int64_t n = numel(out);
    float* w3 = (float*)malloc((size_t)(co * k3 > 0 ? co * k3 : 1) * sizeof(float));
    float* wp = (float*)malloc((size_t)(co * cx > 0 ? co * cx : 1) * sizeof(float));
    float* proj = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!w3 || !wp || !proj) {
        free(w3);
        free(wp);
        free(proj);
        return;
    }
    const float* src = (const float*)w->data;
    for (int64_t o = 0; o < co; ++o) {
        memcpy(w3 + o * k3, src + o * row, (size_t)k3 * sizeof(float));
        memcpy(wp + o * cx, src + o * row + k3, (size_t)cx * sizeof(float));
    }
    int64_t w3shape[4] = {co, kh, kw, ci}, wpshape[4] = {co, cx, 1, 1};
    Tensor tw3 = *w, twp = *w, tproj = *out;
    tw3.data = w3;
    tw3.ndim = 4;
    tw3.shape = w3shape;
    tw3.nbytes = (size_t)(co * k3) * sizeof(float);
    twp.data = wp;
    twp.ndim = 4;
    twp.shape = wpshape;
    twp.nbytes = (size_t)(co * cx) * sizeof(float);
    tproj.data = proj;
    nnc_conv(x, &twp, NULL, &tproj, 1, 1, psh, psw, 0, 0);
    nnc_hip_conv_packed(in, &tw3, b, &tproj, out, kh, kw, sh, sw, ph, pw, act);
    free(w3);
    free(wp);
    free(proj);
}

/* ------------------------------------------------------------------------
 * Global average pool streamed into the classifier (include/nnc_hip.h), no
 * reference counterpart: restated as the composition it replaces,
 * nnc_avgpool2d over the whole plane into a temporary [N][C][1][1]
 * (ops.c:393-461), then nnc_gemm_nt of that temporary viewed as [N, C] with
 * w [O][C] (ops.c:1843-1886). Pinned by composition of two pinned entry
 * points (tests/test_oracle.py checks it against float64 numpy too).
 * ---------------------------------------------------------------------- */
void nnc_hip_gap_gemm_nt(Tensor* in, Tensor* w, Tensor* c, Tensor* out, float alpha, float beta) {
    if (!in || !w || !out || !in->data || !w->data || !out->data || in->ndim != 4 || w->ndim != 2) return;
    const int64_t N = in->shape[0], C = in->shape[1];
    float* pooled = (float*)malloc((size_t)(N * C > 0 ? N * C : 1) * sizeof(float));
    if (!pooled) return;
    int64_t shape4[4] = {N, C, 1, 1}, shape2[2] = {N, C};
    Tensor t4 = {pooled, NNC_DTYPE_FLOAT32, shape4, 4, (int64_t)(N * C * 4)};
    Tensor t2 = {pooled, NNC_DTYPE_FLOAT32, shape2, 2, (int64_t)(N * C * 4)};
    const int H = (int)in->shape[2], W = (int)in->shape[3];
    nnc_avgpool2d(in, &t4, H, W, H, W, 0, 0);
    nnc_gemm_nt(&t2, w, c, out, alpha, beta);
    free(pooled);
}

/* ------------------------------------------------------------------------
 * ResNet's stem streamed into its max pool (include/nnc_hip.h), no
 * reference counterpart: restated as the composition it replaces, the
 * packed-weight convolution with relu (nnc_hip_conv_packed above, act 1:
 * nnc_conv_relu, ops.c:720-1050) into a temporary [N][Co][Ho][Wo] with Ho,
 * Wo from the input, kernel, stride and pad, then nnc_maxpool2d 3x3 /
 * stride 2 / pad 1 (ops.c:316-391). Pinned by composition of pinned entry
 * points.
 * ---------------------------------------------------------------------- */
void nnc_hip_conv_maxpool(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph,
                          int pw) {
    if (!in || !w || !out || !in->data || !w->data || !out->data || in->ndim != 4 || sh <= 0 || sw <= 0) return;
    const int64_t N = in->shape[0], Co = w->shape[0];
    const int64_t Ho = (in->shape[2] + 2 * ph - kh) / sh + 1, Wo = (in->shape[3] + 2 * pw - kw) / sw + 1;
    const int64_t n = N * Co * Ho * Wo;
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    if (!tmp) return;
    int64_t shape[4] = {N, Co, Ho, Wo};
    Tensor t = {tmp, NNC_DTYPE_FLOAT32, shape, 4, (int64_t)(n * 4)};
    nnc_hip_conv_packed(in, w, b, NULL, &t, kh, kw, sh, sw, ph, pw, 1);
    nnc_maxpool2d(&t, out, 3, 3, 2, 2, 1, 1);
    free(tmp);
}

/* ------------------------------------------------------------------------
 * nnc_hip_transpose_slice (include/nnc_hip.h): target-only, no reference
 * counterpart. Restated as the calls it replaces: the Split piece (columns
 * [col0, col0 + width) of every row of in) copied out row-major into a
 * temporary shaped as the transpose's input, then nnc_transpose of it.
 * ---------------------------------------------------------------------- */
void nnc_hip_transpose_slice(Tensor* in, Tensor* out, int64_t* perm, int ndim, int col0, int width) {
    int64_t w_full = in->shape[in->ndim - 1];
    int64_t rows = numel(in) / w_full, n = rows * width;
    int64_t vs[8], pm[8];
    for (int d = 0; d < ndim; ++d) {
        pm[d] = perm ? perm[d] : ndim - 1 - d;
        vs[pm[d]] = out->shape[d];
    }
    float* tmp = (float*)malloc((size_t)(n > 0 ? n : 1) * sizeof(float));
    const float* x = (const float*)in->data;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < width; ++c) tmp[r * width + c] = x[r * w_full + col0 + c];
    Tensor t = *in;
    t.data = tmp;
    t.shape = vs;
    t.ndim = ndim;
    t.nbytes = n * (int64_t)sizeof(float);
    nnc_transpose(&t, out, perm, ndim);
    free(tmp);
}

/* ------------------------------------------------------------------------
 * nnc_hip_attention (include/nnc_hip.h): target-only, no reference
 * counterpart. Restated, per batch b and head h, as the calls of the
 * attention block it replaces on two-dimensional operands (the reference's
 * batched MatMul stepping, ops.c:1687-1704, is not the model's arithmetic
 * for more than one batch): the head's Q, K^T and V copied out of the qkv
 * rows (the Split / Reshape / Transpose copies, ops.c:2183-2251,
 * 1531-1581), S = nnc_matmul(Q, K^T) (ops.c:1607-1730), nnc_div(S, div)
 * (ops.c:82-224), nnc_softmax over the keys (ops.c:260-310), C =
 * nnc_matmul(P, V), and C copied into columns h * dh .. of the batch's rows
 * of out (the head merge). Pinned against float64 numpy in
 * tests/test_oracle.py.
 * ---------------------------------------------------------------------- */
void nnc_hip_attention(Tensor* qkv, Tensor* div, Tensor* out, int batch, int seq, int heads, int head_dim, int q_col,
                       int k_col, int v_col) {
    const int64_t ld = qkv->shape[qkv->ndim - 1], width = (int64_t)heads * head_dim;
    const int64_t sd = (int64_t)seq * head_dim, ss = (int64_t)seq * seq;
    float* q = (float*)malloc((size_t)(sd > 0 ? sd : 1) * sizeof(float));
    float* kt = (float*)malloc((size_t)(sd > 0 ? sd : 1) * sizeof(float));
    float* v = (float*)malloc((size_t)(sd > 0 ? sd : 1) * sizeof(float));
    float* s = (float*)malloc((size_t)(ss > 0 ? ss : 1) * sizeof(float));
    float* s2 = (float*)malloc((size_t)(ss > 0 ? ss : 1) * sizeof(float));
    float* p = (float*)malloc((size_t)(ss > 0 ? ss : 1) * sizeof(float));
    float* c = (float*)malloc((size_t)(sd > 0 ? sd : 1) * sizeof(float));
    int64_t sh_q[2] = {seq, head_dim}, sh_kt[2] = {head_dim, seq}, sh_s[2] = {seq, seq};
    Tensor tq = {q, NNC_DTYPE_FLOAT32, sh_q, 2, sd * 4}, tkt = {kt, NNC_DTYPE_FLOAT32, sh_kt, 2, sd * 4};
    Tensor tv = {v, NNC_DTYPE_FLOAT32, sh_q, 2, sd * 4}, tc = {c, NNC_DTYPE_FLOAT32, sh_q, 2, sd * 4};
    Tensor ts = {s, NNC_DTYPE_FLOAT32, sh_s, 2, ss * 4}, ts2 = {s2, NNC_DTYPE_FLOAT32, sh_s, 2, ss * 4};
    Tensor tp = {p, NNC_DTYPE_FLOAT32, sh_s, 2, ss * 4};
    const float* x = (const float*)qkv->data;
    float* y = (float*)out->data;
    for (int b = 0; b < batch; ++b)
        for (int h = 0; h < heads; ++h) {
            for (int i = 0; i < seq; ++i)
                for (int d = 0; d < head_dim; ++d) {
                    const float* row = x + ((int64_t)b * seq + i) * ld + (int64_t)h * head_dim + d;
                    q[(int64_t)i * head_dim + d] = row[q_col];
                    kt[(int64_t)d * seq + i] = row[k_col];
                    v[(int64_t)i * head_dim + d] = row[v_col];
                }
            nnc_matmul(&tq, &tkt, &ts);
            nnc_div(&ts, div, &ts2);
            nnc_softmax(&ts2, &tp, -1);
            nnc_matmul(&tp, &tv, &tc);
            for (int i = 0; i < seq; ++i)
                for (int d = 0; d < head_dim; ++d)
                    y[((int64_t)b * seq + i) * width + (int64_t)h * head_dim + d] = c[(int64_t)i * head_dim + d];
        }
    free(q), free(kt), free(v), free(s), free(s2), free(p), free(c);
}
