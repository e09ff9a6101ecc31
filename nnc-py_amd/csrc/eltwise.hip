// Element-wise operators of the nnc ABI on gfx950: binary ops with the
// reference's flat-modulo broadcast (runtime/x86/ops.c:82-224, 3233-3346),
// unary math and activations (ops.c:230-258, 2253-2262, 2434-2515), logic and
// comparison ops (ops.c:2342-2428, 2655-2699), Cast / ConstantOfShape /
// Expand (ops.c:2517-2653).
//
// All of them are HBM-bound: one read per input element and one write per
// output element. Kernels are grid-stride loops over float4 (16-byte global
// loads and stores) with a scalar kernel for the tail and for unaligned
// tensors. Every thread reads its elements before writing them, so out may
// alias an input of the same size (the cost_aware planner does this).
#include <math.h>

#include <utility>

#include "common.h"
#include "ew_chains.h"

namespace nnc {

// glibc's x86-64 fmaxf/fminf (maxss/minss) return the second operand when the
// operands compare equal (so fmaxf(0.0f, -0.0f) == -0.0f) and the non-NaN
// operand when one is NaN. The reference's Relu and Clip go through them.
__device__ __forceinline__ float ref_fmaxf(float x, float y) {
    if (y != y) return x;
    if (x != x) return y;
    return x > y ? x : y;
}
__device__ __forceinline__ float ref_fminf(float x, float y) {
    if (y != y) return x;
    if (x != x) return y;
    return x < y ? x : y;
}

enum BinOp { kAdd, kSub, kMul, kDiv, kAddRelu, kAddSigmoid, kEqual, kAnd };

template <int OP>
__device__ __forceinline__ float binop(float x, float y) {
    if (OP == kAdd) return x + y;
    if (OP == kSub) return x - y;
    if (OP == kMul) return x * y;
    if (OP == kDiv) return x / y;
    if (OP == kAddRelu) {
        float s = x + y;
        return s > 0.0f ? s : 0.0f;
    }
    if (OP == kAddSigmoid) {
        float s = x + y;
        return 1.0f / (1.0f + expf(-s));
    }
    if (OP == kEqual) return x == y ? 1.0f : 0.0f;
    return (x != 0.0f && y != 0.0f) ? 1.0f : 0.0f;  // kAnd
}

// operand addressing: 0 = element i, 1 = element 0 (scalar), 2 = i % period
enum Mode { kDirect = 0, kScalar = 1, kModulo = 2 };

template <int M>
__device__ __forceinline__ uint32_t src_index(uint32_t i, uint32_t period) {
    if (M == kDirect) return i;
    if (M == kScalar) return 0;
    return i % period;
}

template <int OP, int AM, int BM>
__global__ void __launch_bounds__(256) binary_scalar_k(const float* __restrict__ a,
                                                       const float* __restrict__ b, float* out,
                                                       uint32_t begin, uint32_t n, uint32_t an,
                                                       uint32_t bn) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = begin + blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = binop<OP>(a[src_index<AM>(i, an)], b[src_index<BM>(i, bn)]);
}

// n4 float4 groups starting at element 0; a modulo period must be a multiple
// of 4 so a group never wraps.
template <int OP, int AM, int BM, bool NT>
__global__ void __launch_bounds__(256) binary_vec4_k(const float* __restrict__ a,
                                                     const float* __restrict__ b, float* out,
                                                     uint32_t n4, uint32_t an, uint32_t bn) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < n4; g += stride) {
        const uint32_t i = g * 4;
        float4 x, y;
        if (AM == kScalar) {
            float s = a[0];
            x = make_float4(s, s, s, s);
        } else {
            x = *reinterpret_cast<const float4*>(a + src_index<AM>(i, an));
        }
        if (BM == kScalar) {
            float s = b[0];
            y = make_float4(s, s, s, s);
        } else {
            y = *reinterpret_cast<const float4*>(b + src_index<BM>(i, bn));
        }
        float4 z;
        z.x = binop<OP>(x.x, y.x);
        z.y = binop<OP>(x.y, y.y);
        z.z = binop<OP>(x.z, y.z);
        z.w = binop<OP>(x.w, y.w);
        store_f4<NT>(out + i, z);
    }
}

template <int OP, int AM, int BM>
static void launch_binary(const char* name, const float* a, const float* b, float* out, int64_t cnt,
                          int64_t an, int64_t bn) {
    const bool vec = aligned16(a) && aligned16(b) && aligned16(out) &&
                     (AM != kModulo || an % 4 == 0) && (BM != kModulo || bn % 4 == 0);
    uint32_t done = 0;
    if (vec && cnt >= 4) {
        const uint32_t n4 = (uint32_t)(cnt / 4);
        if (4 * cnt >= kNtStoreBytes)
            launch(name, binary_vec4_k<OP, AM, BM, true>, dim3(grid_for(n4, 4)), dim3(256), 0, a, b, out, n4,
                   (uint32_t)an, (uint32_t)bn);
        else
            launch(name, binary_vec4_k<OP, AM, BM, false>, dim3(grid_for(n4, 4)), dim3(256), 0, a, b, out, n4,
                   (uint32_t)an, (uint32_t)bn);
        done = n4 * 4;
    }
    if (done < cnt)
        launch(name, binary_scalar_k<OP, AM, BM>, dim3(grid_for(cnt - done, 4)), dim3(256), 0, a, b,
               out, done, (uint32_t)cnt, (uint32_t)an, (uint32_t)bn);
}

// Number of outputs the reference writes (ops.c:82-119): all n when one
// operand has exactly n elements and the other at most n (or both >= n),
// otherwise min(n, a_n, b_n).
static int64_t flat_mod_count(int64_t n, int64_t an, int64_t bn) {
    if (an <= 0 || bn <= 0) return 0;
    if (an >= n && bn >= n) return n;
    if ((an == n && bn < n) || (bn == n && an < n)) return n;
    int64_t m = n < an ? n : an;
    return m < bn ? m : bn;
}

template <int OP>
static void binary_entry(const char* name, Tensor* a, Tensor* b, Tensor* out) {
    if (!ready(name)) return;
    if (!has_data(a) || !has_data(b) || !has_data(out)) {
        fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
        return;
    }
    const int64_t n = numel(out), an = numel(a), bn = numel(b);
    const int64_t cnt = flat_mod_count(n, an, bn);
    if (cnt == 0) return;
    if (cnt >= (int64_t)1 << 31) {
        fail(NNC_HIP_EUNSUPP, name, "more than 2^31 elements");
        return;
    }
    const float* x = static_cast<const float*>(a->data);
    const float* y = static_cast<const float*>(b->data);
    float* z = static_cast<float*>(out->data);
    const bool a_direct = an >= cnt, b_direct = bn >= cnt;
    set_work(0.0, 4.0 * ((double)(an < cnt ? an : cnt) + (double)(bn < cnt ? bn : cnt) + (double)cnt));
    if (a_direct && b_direct)
        launch_binary<OP, kDirect, kDirect>(name, x, y, z, cnt, an, bn);
    else if (a_direct && bn == 1)
        launch_binary<OP, kDirect, kScalar>(name, x, y, z, cnt, an, bn);
    else if (b_direct && an == 1)
        launch_binary<OP, kScalar, kDirect>(name, x, y, z, cnt, an, bn);
    else if (a_direct)
        launch_binary<OP, kDirect, kModulo>(name, x, y, z, cnt, an, bn);
    else
        launch_binary<OP, kModulo, kDirect>(name, x, y, z, cnt, an, bn);
}

// ---------------------------------------------------------------------------
// unary
// ---------------------------------------------------------------------------
enum UnOp { kRelu, kSigmoid, kTanh, kSqrt, kPow, kExp, kLog, kAbs, kNeg, kClip };

template <int OP>
__device__ __forceinline__ float unop(float v, float lo, float hi) {
    if (OP == kRelu) return ref_fmaxf(0.0f, v);
    if (OP == kSigmoid) return 1.0f / (1.0f + expf(-v));
    if (OP == kTanh) return tanhf(v);
    if (OP == kSqrt) return v >= 0.0f ? sqrtf(v) : __builtin_nanf("");
    if (OP == kPow) return v * v;
    if (OP == kExp) return expf(v);
    if (OP == kLog) return v > 0.0f ? logf(v) : __builtin_nanf("");
    if (OP == kAbs) return fabsf(v);
    if (OP == kNeg) return -v;
    return ref_fminf(ref_fmaxf(v, lo), hi);  // kClip
}

template <int OP, bool NT>
__global__ void __launch_bounds__(256) unary_vec4_k(const float* x, float* out, uint32_t n4,
                                                    float lo, float hi) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < n4; g += stride) {
        float4 v = reinterpret_cast<const float4*>(x)[g];
        v.x = unop<OP>(v.x, lo, hi);
        v.y = unop<OP>(v.y, lo, hi);
        v.z = unop<OP>(v.z, lo, hi);
        v.w = unop<OP>(v.w, lo, hi);
        store_f4<NT>(out + 4 * (size_t)g, v);
    }
}

template <int OP>
__global__ void __launch_bounds__(256) unary_scalar_k(const float* x, float* out, uint32_t begin,
                                                      uint32_t n, float lo, float hi) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = begin + blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = unop<OP>(x[i], lo, hi);
}

template <int OP>
static void unary_entry(const char* name, Tensor* in, Tensor* out, float lo = 0.f, float hi = 0.f) {
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out)) {
        fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
        return;
    }
    const int64_t n = numel(out);
    if (n <= 0) return;
    if (numel(in) < n) return fail(NNC_HIP_EINVAL, name, "input smaller than output");
    if (n >= (int64_t)1 << 31) {
        fail(NNC_HIP_EUNSUPP, name, "more than 2^31 elements");
        return;
    }
    const float* x = static_cast<const float*>(in->data);
    float* z = static_cast<float*>(out->data);
    set_work(0.0, 8.0 * (double)n);
    uint32_t done = 0;
    if (aligned16(x) && aligned16(z) && n >= 4) {
        const uint32_t n4 = (uint32_t)(n / 4);
        if (4 * n >= kNtStoreBytes)
            launch(name, unary_vec4_k<OP, true>, dim3(grid_for(n4, 4)), dim3(256), 0, x, z, n4, lo, hi);
        else
            launch(name, unary_vec4_k<OP, false>, dim3(grid_for(n4, 4)), dim3(256), 0, x, z, n4, lo, hi);
        done = n4 * 4;
    }
    if (done < n)
        launch(name, unary_scalar_k<OP>, dim3(grid_for(n - done, 4)), dim3(256), 0, x, z, done,
               (uint32_t)n, lo, hi);
}

// ---------------------------------------------------------------------------
// fused element-wise chains (nnc_hip_fused_eltwise): every step in registers,
// the inputs read and the result written once. Each step calls the binop /
// unop of the op's own kernel, so the values equal those of the op-by-op
// calls. Operands are picked by selects over the loaded inputs (no indexing
// of registers by a runtime value); the op of a step is uniform over the
// grid, so its switch is a scalar branch.
// ---------------------------------------------------------------------------
static constexpr int kEwMaxIn = 4, kEwMaxSteps = 8;
static_assert(kEwChainMaxSteps == kEwMaxSteps, "ew_chains.h and the interpreter take the same step count");
struct EwProg {
    const float* in[kEwMaxIn];
    float* out;
    int n_in, n_steps;
    int op[kEwMaxSteps], x[kEwMaxSteps], y[kEwMaxSteps];
    float lo[kEwMaxSteps], hi[kEwMaxSteps];
};

__device__ __forceinline__ float ew_apply(int op, float x, float y, float lo, float hi) {
    switch (op) {
        case NNC_EW_ADD: return binop<kAdd>(x, y);
        case NNC_EW_SUB: return binop<kSub>(x, y);
        case NNC_EW_MUL: return binop<kMul>(x, y);
        case NNC_EW_DIV: return binop<kDiv>(x, y);
        case NNC_EW_ADD_RELU: return binop<kAddRelu>(x, y);
        case NNC_EW_ADD_SIGMOID: return binop<kAddSigmoid>(x, y);
        case NNC_EW_RELU: return unop<kRelu>(x, lo, hi);
        case NNC_EW_SIGMOID: return unop<kSigmoid>(x, lo, hi);
        case NNC_EW_TANH: return unop<kTanh>(x, lo, hi);
        default: return unop<kClip>(x, lo, hi);
    }
}

// operand slot s: an input 0..3, or kEwMaxIn the running value (selects
// over scalars)
__device__ __forceinline__ float ew_pick(int s, float acc, float a0, float a1, float a2, float a3) {
    float r = a3;
    r = s == 2 ? a2 : r;
    r = s == 1 ? a1 : r;
    r = s == 0 ? a0 : r;
    return s >= kEwMaxIn ? acc : r;
}

// the chain on one element whose inputs are a0..a3
__device__ __forceinline__ float ew_eval(const EwProg& p, float a0, float a1, float a2, float a3) {
    float acc = 0.f;
#pragma unroll
    for (int s = 0; s < kEwMaxSteps; ++s)
        if (s < p.n_steps)
            acc = ew_apply(p.op[s], ew_pick(p.x[s], acc, a0, a1, a2, a3), ew_pick(p.y[s], acc, a0, a1, a2, a3),
                           p.lo[s], p.hi[s]);
    return acc;
}

__device__ __forceinline__ float4 ew_load4(const EwProg& p, int i, uint32_t g) {
    return i < p.n_in ? reinterpret_cast<const float4*>(p.in[i])[g] : make_float4(0.f, 0.f, 0.f, 0.f);
}

template <int BOP>
__device__ __forceinline__ float4 ew_bin4(float4 a, float4 b) {
    return make_float4(binop<BOP>(a.x, b.x), binop<BOP>(a.y, b.y), binop<BOP>(a.z, b.z), binop<BOP>(a.w, b.w));
}
template <int UOP>
__device__ __forceinline__ float4 ew_un4(float4 a, float lo, float hi) {
    return make_float4(unop<UOP>(a.x, lo, hi), unop<UOP>(a.y, lo, hi), unop<UOP>(a.z, lo, hi), unop<UOP>(a.w, lo, hi));
}

// The program on one float4: inputs in slots 0..3 and the running value in
// slot 4 of one register array, an operand read by its slot - a uniform
// index, so one indexed register read per component (the slot of operand
// -1 is 4, set on the host).
__device__ __forceinline__ float4 ew_eval4(const EwProg& p, float4 v0, float4 v1, float4 v2, float4 v3) {
    float r[20] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w, v2.x, v2.y, v2.z, v2.w,
                   v3.x, v3.y, v3.z, v3.w, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < kEwMaxSteps; ++s) {
        if (s >= p.n_steps) continue;
        const int xs = 4 * p.x[s], ys = 4 * p.y[s];
        const float4 a = make_float4(r[xs], r[xs + 1], r[xs + 2], r[xs + 3]);
        const float4 b = make_float4(r[ys], r[ys + 1], r[ys + 2], r[ys + 3]);
        float4 acc;
        switch (p.op[s]) {  // one scalar branch per step, the op applied to all four
            case NNC_EW_ADD: acc = ew_bin4<kAdd>(a, b); break;
            case NNC_EW_SUB: acc = ew_bin4<kSub>(a, b); break;
            case NNC_EW_MUL: acc = ew_bin4<kMul>(a, b); break;
            case NNC_EW_DIV: acc = ew_bin4<kDiv>(a, b); break;
            case NNC_EW_ADD_RELU: acc = ew_bin4<kAddRelu>(a, b); break;
            case NNC_EW_ADD_SIGMOID: acc = ew_bin4<kAddSigmoid>(a, b); break;
            case NNC_EW_RELU: acc = ew_un4<kRelu>(a, 0.f, 0.f); break;
            case NNC_EW_SIGMOID: acc = ew_un4<kSigmoid>(a, 0.f, 0.f); break;
            case NNC_EW_TANH: acc = ew_un4<kTanh>(a, 0.f, 0.f); break;
            default: acc = ew_un4<kClip>(a, p.lo[s], p.hi[s]); break;
        }
        r[16] = acc.x, r[17] = acc.y, r[18] = acc.z, r[19] = acc.w;
    }
    return make_float4(r[16], r[17], r[18], r[19]);
}

template <bool NT>
__global__ void __launch_bounds__(256) fused_eltwise_vec4_k(EwProg p, uint32_t n4) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < n4; g += stride) {
        const float4 v0 = ew_load4(p, 0, g), v1 = ew_load4(p, 1, g), v2 = ew_load4(p, 2, g), v3 = ew_load4(p, 3, g);
        store_f4<NT>(p.out + 4 * (size_t)g, ew_eval4(p, v0, v1, v2, v3));
    }
}

// ---------------------------------------------------------------------------
// Chains known when the library is built, one kernel each: the steps are
// template arguments, so operands are registers named at compile time and
// each op is its own straight-line code (the interpreter above spends about
// 4.6 VALU instructions per element on a five-step chain, enough to make an
// HBM-bound pass VALU-bound). The chains are ew_chains.h's kEwChains (those
// the mi355x O3 compiler emits for its model set and a few common short
// ones); any other chain runs on the interpreter. An empty asm statement after each step keeps the step's
// result a rounded float that the next step reads, as the op-by-op calls
// do through memory (no multiply-add contraction across steps).
// ---------------------------------------------------------------------------
template <int OP, int X, int Y = X>
struct EwStep {
    static constexpr int op = OP, x = X, y = Y;
};

template <int OP>
__device__ __forceinline__ float ew_op(float x, float y, float lo, float hi) {
    if constexpr (OP == NNC_EW_ADD) return binop<kAdd>(x, y);
    else if constexpr (OP == NNC_EW_SUB) return binop<kSub>(x, y);
    else if constexpr (OP == NNC_EW_MUL) return binop<kMul>(x, y);
    else if constexpr (OP == NNC_EW_DIV) return binop<kDiv>(x, y);
    else if constexpr (OP == NNC_EW_ADD_RELU) return binop<kAddRelu>(x, y);
    else if constexpr (OP == NNC_EW_ADD_SIGMOID) return binop<kAddSigmoid>(x, y);
    else if constexpr (OP == NNC_EW_RELU) return unop<kRelu>(x, lo, hi);
    else if constexpr (OP == NNC_EW_SIGMOID) return unop<kSigmoid>(x, lo, hi);
    else if constexpr (OP == NNC_EW_TANH) return unop<kTanh>(x, lo, hi);
    else return unop<kClip>(x, lo, hi);
}

template <int S>
__device__ __forceinline__ float4 ew_operand(const float4 (&v)[kEwMaxIn], float4 acc) {
    if constexpr (S < 0) return acc;
    else return v[S];
}

template <class St>
__device__ __forceinline__ float4 ew_step4(const float4 (&v)[kEwMaxIn], float4 acc, float lo, float hi) {
    const float4 a = ew_operand<St::x>(v, acc), b = ew_operand<St::y>(v, acc);
    float4 r = make_float4(ew_op<St::op>(a.x, b.x, lo, hi), ew_op<St::op>(a.y, b.y, lo, hi),
                           ew_op<St::op>(a.z, b.z, lo, hi), ew_op<St::op>(a.w, b.w, lo, hi));
    asm volatile("" : "+v"(r.x), "+v"(r.y), "+v"(r.z), "+v"(r.w));
    return r;
}

template <bool NT, int NIN, class... Steps>
__global__ void __launch_bounds__(256) ew_chain_k(EwProg p, uint32_t n4) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t g = blockIdx.x * blockDim.x + threadIdx.x; g < n4; g += stride) {
        float4 v[kEwMaxIn];
#pragma unroll
        for (int i = 0; i < kEwMaxIn; ++i)
            v[i] = i < NIN ? reinterpret_cast<const float4*>(p.in[i])[g] : make_float4(0.f, 0.f, 0.f, 0.f);
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        int s = 0;
        ((acc = ew_step4<Steps>(v, acc, p.lo[s], p.hi[s]), ++s), ...);
        store_f4<NT>(p.out + 4 * (size_t)g, acc);
    }
}

template <int NIN, class... Steps>
static void launch_ew_chain(const char* name, const EwProg& p, uint32_t n4, bool nt) {
    if (nt) launch(name, ew_chain_k<true, NIN, Steps...>, dim3(grid_for(n4, 4)), dim3(256), 0, p, n4);
    else launch(name, ew_chain_k<false, NIN, Steps...>, dim3(grid_for(n4, 4)), dim3(256), 0, p, n4);
}

// the kernel of kEwChains[C] (ew_chains.h): its steps as template arguments
template <int C, size_t... S>
static void launch_ew_chain_c(const char* name, const EwProg& p, uint32_t n4, bool nt, std::index_sequence<S...>) {
    constexpr EwChainDef d = kEwChains[C];
    launch_ew_chain<d.n_in, EwStep<d.prog[3 * S], d.prog[3 * S + 1], d.prog[3 * S + 2]>...>(name, p, n4, nt);
}

template <int C>
static void launch_ew_chain_at(const char* name, const EwProg& p, uint32_t n4, bool nt) {
    static_assert(kEwChains[C].n_steps >= 1 && kEwChains[C].n_steps <= kEwMaxSteps, "1 to kEwMaxSteps steps");
    static_assert(kEwChains[C].n_in >= 1 && kEwChains[C].n_in <= kEwMaxIn, "1 to kEwMaxIn inputs");
    launch_ew_chain_c<C>(name, p, n4, nt, std::make_index_sequence<kEwChains[C].n_steps>{});
}

typedef void (*EwChainLaunch)(const char*, const EwProg&, uint32_t, bool);

template <size_t... C>
static const EwChainLaunch* ew_chain_launchers(std::index_sequence<C...>) {
    static const EwChainLaunch table[] = {&launch_ew_chain_at<(int)C>...};
    return table;
}

__global__ void __launch_bounds__(256) fused_eltwise_scalar_k(EwProg p, uint32_t begin, uint32_t n) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = begin + blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const float a0 = p.in[0][i], a1 = p.n_in > 1 ? p.in[1][i] : 0.f;
        const float a2 = p.n_in > 2 ? p.in[2][i] : 0.f, a3 = p.n_in > 3 ? p.in[3][i] : 0.f;
        p.out[i] = ew_eval(p, a0, a1, a2, a3);
    }
}

// ---------------------------------------------------------------------------
// uint8 logic, comparisons, casts, fills
// ---------------------------------------------------------------------------
__global__ void greater_k(const float* a, const float* b, uint8_t* out, uint32_t n, uint32_t an,
                          uint32_t bn) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = a[i % an] > b[i % bn] ? 1 : 0;
}

__global__ void or_k(const uint8_t* a, const uint8_t* b, uint8_t* out, uint32_t n) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = (a[i] || b[i]) ? 1 : 0;
}

__global__ void not_k(const uint8_t* a, uint8_t* out, uint32_t n) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = a[i] ? 0 : 1;
}

// float -> integer as x86 cvttss2si: truncation, and the "integer
// indefinite" value (most negative integer) for NaN and out-of-range inputs.
__device__ __forceinline__ int32_t cvt_i32(float x) {
    return (x > -2147483904.0f && x < 2147483648.0f) ? (int32_t)x : INT32_MIN;
}
__device__ __forceinline__ int64_t cvt_i64(float x) {
    return (x > -9223373136366403584.0f && x < 9223372036854775808.0f) ? (int64_t)x : INT64_MIN;
}

enum CastKind { kBoolToF32, kF32ToI32, kBoolToI32, kF32ToI64, kBoolToI64, kF32ToBool };

template <int K>
__global__ void cast_k(const void* in, void* out, uint32_t n) {
    const uint32_t stride = gridDim.x * blockDim.x;
    const float* xf = static_cast<const float*>(in);
    const uint8_t* xb = static_cast<const uint8_t*>(in);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        if (K == kBoolToF32) static_cast<float*>(out)[i] = (float)xb[i];
        if (K == kF32ToI32) static_cast<int32_t*>(out)[i] = cvt_i32(xf[i]);
        if (K == kBoolToI32) static_cast<int32_t*>(out)[i] = (int32_t)xb[i];
        if (K == kF32ToI64) static_cast<int64_t*>(out)[i] = cvt_i64(xf[i]);
        if (K == kBoolToI64) static_cast<int64_t*>(out)[i] = (int64_t)xb[i];
        if (K == kF32ToBool) static_cast<uint8_t*>(out)[i] = xf[i] != 0.0f ? 1 : 0;
    }
}

__global__ void fill_k(float* out, uint32_t n, float v) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = v;
}

__global__ void copy_bytes_k(const uint8_t* in, uint8_t* out, uint64_t n) {
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        out[i] = in[i];
}

__global__ void modulo_copy_k(const float* in, float* out, uint32_t n, uint32_t m) {
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = in[i % m];
}

}  // namespace nnc

using namespace nnc;

extern "C" {

void nnc_add(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kAdd>("nnc_add", a, b, o); }
void nnc_sub(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kSub>("nnc_sub", a, b, o); }
void nnc_mul(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kMul>("nnc_mul", a, b, o); }
void nnc_div(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kDiv>("nnc_div", a, b, o); }
void nnc_add_relu(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kAddRelu>("nnc_add_relu", a, b, o); }
void nnc_add_sigmoid(Tensor* a, Tensor* b, Tensor* o) {
    binary_entry<kAddSigmoid>("nnc_add_sigmoid", a, b, o);
}
void nnc_equal(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kEqual>("nnc_equal", a, b, o); }
void nnc_and(Tensor* a, Tensor* b, Tensor* o) { binary_entry<kAnd>("nnc_and", a, b, o); }

void nnc_relu(Tensor* i, Tensor* o) { unary_entry<kRelu>("nnc_relu", i, o); }
void nnc_sigmoid(Tensor* i, Tensor* o) { unary_entry<kSigmoid>("nnc_sigmoid", i, o); }
void nnc_tanh(Tensor* i, Tensor* o) { unary_entry<kTanh>("nnc_tanh", i, o); }
void nnc_sqrt(Tensor* i, Tensor* o) { unary_entry<kSqrt>("nnc_sqrt", i, o); }
void nnc_pow(Tensor* i, Tensor* o) { unary_entry<kPow>("nnc_pow", i, o); }
void nnc_exp(Tensor* i, Tensor* o) { unary_entry<kExp>("nnc_exp", i, o); }
void nnc_log(Tensor* i, Tensor* o) { unary_entry<kLog>("nnc_log", i, o); }
void nnc_abs(Tensor* i, Tensor* o) { unary_entry<kAbs>("nnc_abs", i, o); }
void nnc_neg(Tensor* i, Tensor* o) { unary_entry<kNeg>("nnc_neg", i, o); }
void nnc_clip(Tensor* i, Tensor* o, float lo, float hi) { unary_entry<kClip>("nnc_clip", i, o, lo, hi); }

// No reference counterpart: a chain of element-wise ops in one pass (the
// mi355x target's O3 fusion of element-wise nodes each feeding only the next).
void nnc_hip_fused_eltwise(Tensor** ins, int n_in, const int* prog, int n_steps, const float* consts, Tensor* out) {
    const char* name = "nnc_hip_fused_eltwise";
    if (!ready(name)) return;
    if (!ins || !prog || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL argument");
    if (out->dtype != NNC_DTYPE_FLOAT32) return fail(NNC_HIP_EUNSUPP, name, "float32 output only");
    if (n_in < 1 || n_in > kEwMaxIn) return fail(NNC_HIP_EINVAL, name, "1 to %d inputs, got %d", kEwMaxIn, n_in);
    if (n_steps < 1 || n_steps > kEwMaxSteps)
        return fail(NNC_HIP_EINVAL, name, "1 to %d steps, got %d", kEwMaxSteps, n_steps);
    const int64_t n = numel(out);
    if (n <= 0) return;
    if (n >= (int64_t)1 << 31) return fail(NNC_HIP_EUNSUPP, name, "more than 2^31 elements");
    EwProg p{};
    p.out = static_cast<float*>(out->data);
    p.n_in = n_in;
    p.n_steps = n_steps;
    bool vec = aligned16(p.out);
    for (int i = 0; i < n_in; ++i) {
        if (!has_data(ins[i]) || numel(ins[i]) != n)
            return fail(NNC_HIP_EINVAL, name, "input %d must have numel(out) = %lld elements", i, (long long)n);
        if (ins[i]->dtype != NNC_DTYPE_FLOAT32) return fail(NNC_HIP_EUNSUPP, name, "input %d: float32 only", i);
        p.in[i] = static_cast<const float*>(ins[i]->data);
        vec = vec && aligned16(p.in[i]);
    }
    for (int s = 0; s < n_steps; ++s) {
        const int op = prog[3 * s], x = prog[3 * s + 1], y = prog[3 * s + 2];
        const bool binary = op <= NNC_EW_ADD_SIGMOID;
        if (op < 0 || op >= NNC_EW_OPS) return fail(NNC_HIP_EINVAL, name, "step %d: unknown op %d", s, op);
        if (x < -1 || x >= n_in || (binary && (y < -1 || y >= n_in)))
            return fail(NNC_HIP_EINVAL, name, "step %d: operand out of range", s);
        if (s == 0 && (x < 0 || (binary && y < 0)))
            return fail(NNC_HIP_EINVAL, name, "step 0 reads the running value");
        if (op == NNC_EW_CLIP && !consts) return fail(NNC_HIP_EINVAL, name, "step %d: Clip without bounds", s);
        p.op[s] = op;
        p.x[s] = x < 0 ? kEwMaxIn : x;  // (the running value's slot)
        p.y[s] = binary ? (y < 0 ? kEwMaxIn : y) : p.x[s];
        p.lo[s] = consts ? consts[2 * s] : 0.f;
        p.hi[s] = consts ? consts[2 * s + 1] : 0.f;
    }
    set_work(0.0, 4.0 * (double)n * (n_in + 1));
    uint32_t done = 0;
    if (vec && n >= 4) {
        const uint32_t n4 = (uint32_t)(n / 4);
        const int chain = ew_chain_index(n_in, prog, n_steps);
        if (chain >= 0)
            ew_chain_launchers(std::make_index_sequence<kEwChainCount>{})[chain](name, p, n4, 4 * n >= kNtStoreBytes);
        else if (4 * n >= kNtStoreBytes)
            launch(name, fused_eltwise_vec4_k<true>, dim3(grid_for(n4, 4)), dim3(256), 0, p, n4);
        else
            launch(name, fused_eltwise_vec4_k<false>, dim3(grid_for(n4, 4)), dim3(256), 0, p, n4);
        done = n4 * 4;
    }
    if (done < n)
        launch(name, fused_eltwise_scalar_k, dim3(grid_for(n - done, 4)), dim3(256), 0, p, done, (uint32_t)n);
}

int nnc_hip_ew_chain_specialized(int n_in, const int* prog, int n_steps) {
    if (!prog || n_in < 1 || n_in > kEwMaxIn || n_steps < 1 || n_steps > kEwMaxSteps) return 0;
    return ew_chain_index(n_in, prog, n_steps) >= 0 ? 1 : 0;
}

void nnc_greater(Tensor* a, Tensor* b, Tensor* out) {
    const char* name = "nnc_greater";
    if (!ready(name)) return;
    if (!has_data(a) || !has_data(b) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    const int64_t n = numel(out), an = numel(a), bn = numel(b);
    if (n <= 0) return;
    if (an <= 0 || bn <= 0) return fail(NNC_HIP_EINVAL, name, "empty operand");
    launch(name, greater_k, dim3(grid_for(n, 1)), dim3(256), 0, (const float*)a->data,
           (const float*)b->data, (uint8_t*)out->data, (uint32_t)n, (uint32_t)an, (uint32_t)bn);
}

void nnc_or(Tensor* a, Tensor* b, Tensor* out) {
    const char* name = "nnc_or";
    if (!ready(name)) return;
    if (!has_data(a) || !has_data(b) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    const int64_t n = numel(out);
    if (numel(a) < n || numel(b) < n) return fail(NNC_HIP_EINVAL, name, "operand smaller than output");
    launch(name, or_k, dim3(grid_for(n, 1)), dim3(256), 0, (const uint8_t*)a->data,
           (const uint8_t*)b->data, (uint8_t*)out->data, (uint32_t)n);
}

void nnc_not(Tensor* in, Tensor* out) {
    const char* name = "nnc_not";
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    const int64_t n = numel(out);
    if (numel(in) < n) return fail(NNC_HIP_EINVAL, name, "input smaller than output");
    launch(name, not_k, dim3(grid_for(n, 1)), dim3(256), 0, (const uint8_t*)in->data,
           (uint8_t*)out->data, (uint32_t)n);
}

void nnc_cast(Tensor* in, Tensor* out, int to) {
    const char* name = "nnc_cast";
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    const int64_t n = numel(in);
    if (n <= 0) return;
    if (numel(out) < n) return fail(NNC_HIP_EINVAL, name, "output smaller than input");
    const bool from_bool = in->dtype == NNC_DTYPE_BOOL;
    const dim3 g(grid_for(n, 1)), blk(256);
    switch (to) {
        case NNC_DTYPE_FLOAT32:
            if (from_bool) launch(name, cast_k<kBoolToF32>, g, blk, 0, in->data, out->data, (uint32_t)n);
            else device_copy(name, in->data, out->data, (size_t)n * 4);
            break;
        case NNC_DTYPE_INT32:
            if (from_bool) launch(name, cast_k<kBoolToI32>, g, blk, 0, in->data, out->data, (uint32_t)n);
            else launch(name, cast_k<kF32ToI32>, g, blk, 0, in->data, out->data, (uint32_t)n);
            break;
        case NNC_DTYPE_INT64:
            if (from_bool) launch(name, cast_k<kBoolToI64>, g, blk, 0, in->data, out->data, (uint32_t)n);
            else launch(name, cast_k<kF32ToI64>, g, blk, 0, in->data, out->data, (uint32_t)n);
            break;
        case NNC_DTYPE_BOOL:
            if (from_bool) device_copy(name, in->data, out->data, (size_t)n);
            else launch(name, cast_k<kF32ToBool>, g, blk, 0, in->data, out->data, (uint32_t)n);
            break;
        default:  // FLOAT16 and unknown targets copy 4-byte elements (ops.c:2539-2542, 2593-2596)
            device_copy(name, in->data, out->data, (size_t)n * 4);
            break;
    }
}

void nnc_constantofshape(Tensor* out, float value, int ndim) {
    (void)ndim;
    const char* name = "nnc_constantofshape";
    if (!ready(name)) return;
    if (!has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    const int64_t n = numel(out);
    launch(name, fill_k, dim3(grid_for(n, 1)), dim3(256), 0, (float*)out->data, (uint32_t)n, value);
}

void nnc_expand(Tensor* in, Tensor* out, int64_t* shape, int ndim) {
    (void)shape;
    (void)ndim;
    const char* name = "nnc_expand";
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    const int64_t m = numel(in), n = numel(out);
    if (n <= 0) return;
    if (m <= 0) return fail(NNC_HIP_EINVAL, name, "empty input");
    if (m == n) return device_copy(name, in->data, out->data, (size_t)n * 4);
    launch(name, modulo_copy_k, dim3(grid_for(n, 1)), dim3(256), 0, (const float*)in->data,
           (float*)out->data, (uint32_t)n, (uint32_t)m);
}

}  // extern "C"
