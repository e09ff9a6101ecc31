// Scaled dot-product attention in one kernel (nnc_hip_attention): the
// mi355x target's O3 fusion of a transformer layer's attention block -
// head split of the QKV projection, Q K^T, division by the scale, softmax
// over the keys, the product with V and the head merge - which the
// reference runs as separate calls (runtime/x86/ops.c:2183-2251 nnc_split,
// 1531-1581 nnc_transpose, 1607-1730 nnc_matmul, 82-224 nnc_div, 260-310
// nnc_softmax; call sequence test_snapshots_simple_transformer.ambr:114-216).
//
// Layout: qkv is [batch * seq][ld] row-major (the projection's output); head
// h of Q is columns q_col + h * dh .. + dh of the batch's seq rows, K and V
// likewise from k_col and v_col. out is [batch * seq][heads * dh]: head h's
// context in columns h * dh .. + dh (the merged-head layout the output
// projection reads).
//
// head_dim 64: attention16_k (below), 16 query rows per workgroup, operands
// straight into registers. head_dim 32: attention_k, one workgroup of four
// waves per (batch, head, block of 32 query rows).
// The block's Q rows and the head's K and V rows go into LDS with 16-byte
// loads (rows padded to dh + 4 floats). Scores: wave w computes the 32 x 32
// block of keys 32w .. 32w + 31 with v_mfma_f32_32x32x2_f32 (lane half h
// takes d = 16h .. 16h + 15 of each 32-wide slice of the head dimension, as
// in the conv and GEMM tile engine) and stores the scores divided by the
// scale (nnc_div's x / y) to LDS; eight threads per query row then take the
// row's maximum and sum over 16 keys each and three xor shuffles, and write
// the probabilities exp(s - max) / sum back. Context: each wave computes a
// 32-column block of the head over a quarter or half of the keys, and the
// key groups' sums are added in group order (deterministic). Keys past seq
// (seq < 128) get probability 0 and their V rows are zero.
#include <math.h>

#include "mfma_tile.h"

namespace nnc {

struct AttnArgs {
    const float* qkv;
    const float* div;
    float* out;
    int seq, heads, ld, q_col, k_col, v_col;
};

static constexpr int kAttnMaxSeq = 128;

template <int DH>
struct AttnLds {
    static constexpr int LDQ = DH + 4;  // row stride of Q, K, V (floats, 16-byte aligned rows)
    static constexpr int LDP = kAttnMaxSeq + 4;
    static constexpr int Q = 0, K = 32 * LDQ, V = K + kAttnMaxSeq * LDQ, P = V + kAttnMaxSeq * LDQ;
    static constexpr int FLOATS = P + 32 * LDP;
};

// Staging of R rows (a compile-time bound) of a head's dh columns at `col`
// of the qkv rows from `row0`: every thread's 16-byte loads are issued
// before any LDS store (one memory round trip, not one per row group); rows
// at or past `rows` read as zeros (out-of-range buffer offsets).
template <int DH, int R>
struct AttnStage {
    static constexpr int C4 = DH / 4, PER = R * C4 / 256;
    static_assert(R * C4 % 256 == 0, "whole passes");
    f32x4 v[PER];
    __device__ void load(const AttnArgs& a, __amdgpu_buffer_rsrc_t rq, int64_t row0, int col, int rows) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int i = threadIdx.x + 256 * p, r = i / C4, c = (i - r * C4) * 4;
            const uint32_t off = (uint32_t)(((row0 + r) * a.ld + col + c) * 4);
            v[p] = load_f32x4(rq, r < rows ? off : kOutOfRange);
        }
    }
    __device__ void store(float* dst) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int i = threadIdx.x + 256 * p, r = i / C4, c = (i - r * C4) * 4;
            *reinterpret_cast<f32x4*>(dst + r * AttnLds<DH>::LDQ + c) = v[p];
        }
    }
};

template <int DH>
__global__ void __launch_bounds__(256) attention_k(AttnArgs a) {
    typedef AttnLds<DH> L;
    constexpr int LDQ = L::LDQ, LDP = L::LDP;
    extern __shared__ __align__(16) float lds[];
    float* qs = lds + L::Q;
    float* ks = lds + L::K;
    float* vs = lds + L::V;
    float* ps = lds + L::P;
    const int lane = threadIdx.x & 63, l32 = lane & 31, half = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qblocks = a.seq / 32;
    const int qb = blockIdx.x % qblocks, bh = blockIdx.x / qblocks;
    const int h = bh % a.heads, b = bh / a.heads;
    const int64_t row0 = (int64_t)b * a.seq;
    {
        const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qkv);
        AttnStage<DH, 32> sq;
        AttnStage<DH, kAttnMaxSeq> sk, sv;
        sq.load(a, rq, row0 + qb * 32, a.q_col + h * DH, 32);
        sk.load(a, rq, row0, a.k_col + h * DH, a.seq);
        sv.load(a, rq, row0, a.v_col + h * DH, a.seq);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the first store
        sq.store(qs);
        sk.store(ks);
        sv.store(vs);
    }
    const float dv = a.div[0];
    __syncthreads();

    // scores of keys 32 * wave .. + 31 for the block's 32 query rows:
    // s[r] is row 8 (r / 4) + 4 half + r % 4, key 32 * wave + l32
    const bool keys_in = 32 * wave < a.seq;  // wave-uniform
    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.f;
    if (keys_in) {
        const float* qrow = qs + l32 * LDQ + 16 * half;
        const float* krow = ks + (32 * wave + l32) * LDQ + 16 * half;
#pragma unroll
        for (int t = 0; t < DH / 32; ++t) {
            f32x4 qa[4], kb[4];
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                qa[u] = *reinterpret_cast<const f32x4*>(qrow + 32 * t + 4 * u);
                kb[u] = *reinterpret_cast<const f32x4*>(krow + 32 * t + 4 * u);
            }
#pragma unroll
            for (int c = 0; c < 16; ++c) s = __builtin_amdgcn_mfma_f32_32x32x2f32(qa[c >> 2][c & 3], kb[c >> 2][c & 3], s, 0, 0, 0);
        }
    }
    // scaled scores to LDS (keys past seq: -inf, probability 0)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float x = s[r];  // (element copied first: this compiler's ext-vector element reads)
        ps[(8 * (r >> 2) + 4 * half + (r & 3)) * LDP + 32 * wave + l32] = keys_in ? x / dv : -INFINITY;
    }
    __syncthreads();
    // softmax over the keys: eight threads per query row, 16 keys each; the
    // row maximum and sum are combined over the eight lanes by three xor
    // shuffles
    {
        float* prow_s = ps + (threadIdx.x >> 3) * LDP + (threadIdx.x & 7) * 16;
        f32x4 x[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const f32x4*>(prow_s + 4 * u);
        float m = x[0][0];
#pragma unroll
        for (int c = 1; c < 16; ++c) m = fmaxf(m, x[c >> 2][c & 3]);
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        float t = 0.f;
#pragma unroll
        for (int c = 0; c < 16; ++c) {
            const float e = __expf(x[c >> 2][c & 3] - m);
            x[c >> 2][c & 3] = e;
            t += e;
        }
#pragma unroll
        for (int o = 1; o < 8; o <<= 1) t += __shfl_xor(t, o);
        const float inv = 1.0f / t;
#pragma unroll
        for (int u = 0; u < 4; ++u) *reinterpret_cast<f32x4*>(prow_s + 4 * u) = x[u] * inv;
    }
    __syncthreads();

    // context: column block cb of the head over key group kg
    constexpr int CB = DH / 32, KG = 4 / CB, KEYS = kAttnMaxSeq / KG;
    const int cb = wave % CB, kg = wave / CB;
    floatx16 o;
#pragma unroll
    for (int r = 0; r < 16; ++r) o[r] = 0.f;
    const float* prow = ps + l32 * LDP + kg * KEYS + 16 * half;
    const float* vcol = vs + (kg * KEYS + 16 * half) * LDQ + cb * 32 + l32;
#pragma unroll
    for (int t = 0; t < KEYS / 32; ++t) {
        f32x4 pa[4];
        float vb[16];
#pragma unroll
        for (int u = 0; u < 4; ++u) pa[u] = *reinterpret_cast<const f32x4*>(prow + 32 * t + 4 * u);
#pragma unroll
        for (int c = 0; c < 16; ++c) vb[c] = vcol[(32 * t + c) * LDQ];
#pragma unroll
        for (int c = 0; c < 16; ++c) o = __builtin_amdgcn_mfma_f32_32x32x2f32(pa[c >> 2][c & 3], vb[c], o, 0, 0, 0);
    }
    // key groups 1.. hand their sums to group 0 through LDS (K's rows are
    // no longer read), which adds them in group order and stores
    if (kg > 0) {
        float* part = ks + ((kg - 1) * CB + cb) * 1024;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float x = o[r];
            part[(8 * (r >> 2) + 4 * half + (r & 3)) * 32 + l32] = x;
        }
    }
    __syncthreads();
    if (kg > 0) return;
    float* orow = a.out + (row0 + qb * 32) * (int64_t)(a.heads * DH) + h * DH + cb * 32 + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = 8 * (r >> 2) + 4 * half + (r & 3);
        float v = o[r];
        for (int g = 1; g < KG; ++g) v += ks[((g - 1) * CB + cb) * 1024 + row * 32 + l32];
        orow[(int64_t)row * (a.heads * DH)] = v;
    }
}

// head_dim 64: one workgroup per (batch, head, block of 16 query rows) with
// v_mfma_f32_16x16x4f32 (lane (li = lane % 16, g = lane / 16): A[li][g],
// B[g][li]; accumulator r is row 4g + r, column li). The dot products'
// terms are taken in any order both operands agree on: lane group g takes
// d = 16g + t (Q K^T) and keys 64c + 16g + t (P V) at step t, so Q, K and P
// rows are 16-byte loads. Q, K and V go straight from global memory into
// the operand registers (no LDS staging): wave w computes the scores of keys
// 32w .. 32w + 31 (two 16 x 16 blocks over the 16 d steps) and, after the
// softmax, output columns 16w .. 16w + 15 over all keys (two chunks of 64).
// The scaled scores go to LDS, 16 threads per row take its maximum and sum
// (eight keys each, four xor shuffles) and write exp(s - max) / sum back.
__global__ void __launch_bounds__(256) attention16_k(AttnArgs a) {
    constexpr int DH = 64, LDP = kAttnMaxSeq + 4;
    __shared__ __align__(16) float ps[16 * LDP];
    const int lane = threadIdx.x & 63, li = lane & 15, g4 = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int qblocks = a.seq / 16;
    const int qb = blockIdx.x % qblocks, bh = blockIdx.x / qblocks;
    const int h = bh % a.heads, b = bh / a.heads;
    const int64_t row0 = (int64_t)b * a.seq;
    const __amdgpu_buffer_rsrc_t rq = make_rsrc(a.qkv);
    // operands: every load issued before the first MFMA
    f32x4 qa[4], kk[2][4];
    float vv[2][16];
    {
        const uint32_t qoff = (uint32_t)(((row0 + qb * 16 + li) * a.ld + a.q_col + h * DH + 16 * g4) * 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) qa[u] = load_f32x4(rq, qoff + 16u * u);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int key = 32 * wave + 16 * kb + li;
            const uint32_t koff = (uint32_t)(((row0 + key) * a.ld + a.k_col + h * DH + 16 * g4) * 4);
#pragma unroll
            for (int u = 0; u < 4; ++u) kk[kb][u] = load_f32x4(rq, key < a.seq ? koff + 16u * u : kOutOfRange);
        }
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int t = 0; t < 16; ++t) {
                const int key = 64 * c + 16 * g4 + t;
                const uint32_t voff = (uint32_t)(((row0 + key) * a.ld + a.v_col + h * DH + 16 * wave + li) * 4);
                vv[c][t] = load_f32(rq, key < a.seq ? voff : kOutOfRange);
            }
    }
    const float dv = a.div[0];
    __builtin_amdgcn_sched_barrier(0);
    // scores of keys 32 wave + 16 kb + li for rows 4 g4 + r
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            // (element copies first: this compiler's ext-vector element reads)
            const float x = qa[t >> 2][t & 3], y = kk[kb][t >> 2][t & 3];
            s = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, s, 0, 0, 0);
        }
        const int key = 32 * wave + 16 * kb + li;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float x = s[r];
            ps[(4 * g4 + r) * LDP + key] = key < a.seq ? x / dv : -INFINITY;
        }
    }
    __syncthreads();
    {
        // softmax: 16 threads per row (a 16-lane group), 8 keys each
        float* prow = ps + (threadIdx.x >> 4) * LDP + (threadIdx.x & 15) * 8;
        f32x4 x0 = *reinterpret_cast<const f32x4*>(prow), x1 = *reinterpret_cast<const f32x4*>(prow + 4);
        float m = fmaxf(fmaxf(fmaxf(x0[0], x0[1]), fmaxf(x0[2], x0[3])), fmaxf(fmaxf(x1[0], x1[1]), fmaxf(x1[2], x1[3])));
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) m = fmaxf(m, __shfl_xor(m, o));
        float t = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            x0[c] = __expf(x0[c] - m);
            x1[c] = __expf(x1[c] - m);
            t += x0[c] + x1[c];
        }
#pragma unroll
        for (int o = 1; o < 16; o <<= 1) t += __shfl_xor(t, o);
        const float inv = 1.0f / t;
        *reinterpret_cast<f32x4*>(prow) = x0 * inv;
        *reinterpret_cast<f32x4*>(prow + 4) = x1 * inv;
    }
    __syncthreads();
    // context: columns 16 wave + li for rows 4 g4 + r, keys 64 c + 16 g4 + t
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        f32x4 pa[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) pa[u] = *reinterpret_cast<const f32x4*>(&ps[li * LDP + 64 * c + 16 * g4 + 4 * u]);
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float x = pa[t >> 2][t & 3];
            o = __builtin_amdgcn_mfma_f32_16x16x4f32(x, vv[c][t], o, 0, 0, 0);
        }
    }
    float* orow = a.out + (row0 + qb * 16 + 4 * g4) * (int64_t)(a.heads * DH) + h * DH + 16 * wave + li;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float x = o[r];
        orow[(int64_t)r * (a.heads * DH)] = x;
    }
}

template <int DH>
static void launch_attention(const AttnArgs& a, int blocks, const char* name) {
    auto kernel = attention_k<DH>;
    const size_t lds = (size_t)AttnLds<DH>::FLOATS * sizeof(float);
    static const bool ok =
        hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) == hipSuccess;
    if (!ok) return fail(NNC_HIP_EDEVICE, name, "hipFuncSetAttribute failed");
    launch(name, kernel, dim3((unsigned)blocks), dim3(256), lds, a);
}

}  // namespace nnc

using namespace nnc;

extern "C" {

// No reference counterpart: a transformer layer's attention block in one
// kernel (the mi355x target's O3 fusion); see the file's head comment.
void nnc_hip_attention(Tensor* qkv, Tensor* div, Tensor* out, int batch, int seq, int heads, int head_dim, int q_col,
                       int k_col, int v_col) {
    const char* name = "nnc_hip_attention";
    if (!ready(name)) return;
    if (!has_data(qkv) || !has_data(div) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    if (qkv->dtype != NNC_DTYPE_FLOAT32 || div->dtype != NNC_DTYPE_FLOAT32 || out->dtype != NNC_DTYPE_FLOAT32)
        return fail(NNC_HIP_EUNSUPP, name, "float32 tensors only");
    if (batch < 0 || heads < 1 || qkv->ndim < 1) return fail(NNC_HIP_EINVAL, name, "bad batch / heads / rank");
    if (numel(div) != 1) return fail(NNC_HIP_EINVAL, name, "the divisor must have one element");
    if (head_dim != 32 && head_dim != 64) return fail(NNC_HIP_EUNSUPP, name, "head_dim %d (32 or 64)", head_dim);
    if (seq < 32 || seq > kAttnMaxSeq || seq % 32 != 0)
        return fail(NNC_HIP_EUNSUPP, name, "seq %d (a multiple of 32 up to %d)", seq, kAttnMaxSeq);
    const int64_t ld = qkv->shape[qkv->ndim - 1], rows = (int64_t)batch * seq, width = (int64_t)heads * head_dim;
    if (numel(qkv) != rows * ld) return fail(NNC_HIP_EINVAL, name, "qkv is not [batch * seq][ld]");
    for (int col : {q_col, k_col, v_col})
        if (col < 0 || col + width > ld) return fail(NNC_HIP_EINVAL, name, "columns [%d, %lld) outside rows of %lld",
                                                     col, (long long)(col + width), (long long)ld);
    if (numel(out) != rows * width) return fail(NNC_HIP_EINVAL, name, "out is not [batch * seq][heads * head_dim]");
    if (!aligned16(qkv->data) || ld % 4 != 0 || q_col % 4 != 0 || k_col % 4 != 0 || v_col % 4 != 0)
        return fail(NNC_HIP_EUNSUPP, name, "qkv rows and columns must be 16-byte aligned");
    if (rows == 0) return;
    if (numel(qkv) * 4 >= ((int64_t)1 << 31)) return fail(NNC_HIP_EUNSUPP, name, "qkv of 2 GiB or more");
    AttnArgs a{(const float*)qkv->data, (const float*)div->data, (float*)out->data, seq, heads, (int)ld,
               q_col, k_col, v_col};
    set_work(4.0 * batch * heads * (double)seq * seq * head_dim, 0.0);
    if (head_dim == 64)
        launch("attention16_d64", attention16_k, dim3((unsigned)(batch * heads * (seq / 16))), dim3(256), 0, a);
    else
        launch_attention<32>(a, (int)(batch * heads * (seq / 32)), "attention32_d32");
}

}  // extern "C"
