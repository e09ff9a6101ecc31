// Softmax, LayerNorm and single-axis ReduceMean/ReduceSum of the nnc ABI
// (runtime/x86/ops.c:260-310, 2095-2171, 1892-1989).
//
// All three view the input as [outer][len][inner] around one axis.
//
// inner == 1 (the reduced / normalised elements are contiguous): one wave64
// per row. Rows of up to 4096 floats are read once with 16-byte loads into
// registers; max / sums are combined across the wave with DPP lane moves, and
// the row is written once: one HBM read + one HBM write per element
// (non-temporal stores for outputs of kNtStoreBytes or more). Longer rows
// loop over global memory (re-reads come from L2).
//
// inner > 1 (strided axis): one thread per (outer, inner) column, lanes along
// inner so every load coalesces; the column is walked in the reference's
// order. For ReduceMean/Sum that walk is the reference's own Kahan sum, so the
// strided reduction is bit-exact with it.
//
// Arithmetic follows the reference's formulas: softmax = exp(x - max) / sum
// with max by strict '>' from -inf; layernorm y = g[i] * ((x - mean) / std) +
// b[i], std = sqrtf(var + eps), var the mean of squared deviations. Parallel
// sums change the summation order, so these are tolerance parity
// (1e-4 abs / 1e-3 rel), except the strided reduction. The row kernels take
// exp from the hardware exp2 (__expf, a few ulp for the arguments x - max
// <= 0) and divide by the row's sum / std through one reciprocal per row:
// both within the bar, and per-element divisions with full-range expf made
// the row kernels VALU-bound (softmax [4096,1024] 8.9 -> 7.2 us).
#include <math.h>

#include "common.h"

namespace nnc {

// Wave-wide sum / max through DPP lane moves (no LDS round trips): xor 1
// and xor 2 within quads, the half-row and row mirrors (every lane then
// holds its 16-lane row's result), then the four rows read out with
// v_readlane and combined in a fixed order. The same tree for every wave:
// deterministic, and the result is wave-uniform.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppRowHalfMirror = 0x141, kDppRowMirror = 0x140;

__device__ __forceinline__ float row_lane(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_move<kDppXor1>(v);
    v += dpp_move<kDppXor2>(v);
    v += dpp_move<kDppRowHalfMirror>(v);
    v += dpp_move<kDppRowMirror>(v);
    return (row_lane(v, 0) + row_lane(v, 16)) + (row_lane(v, 32) + row_lane(v, 48));
}

// max by '>' (callers never pass NaN: their per-lane maxima start at -inf
// and take only values that compare greater)
__device__ __forceinline__ float max_gt(float a, float b) { return b > a ? b : a; }
__device__ __forceinline__ float wave_max(float v) {
    v = max_gt(v, dpp_move<kDppXor1>(v));
    v = max_gt(v, dpp_move<kDppXor2>(v));
    v = max_gt(v, dpp_move<kDppRowHalfMirror>(v));
    v = max_gt(v, dpp_move<kDppRowMirror>(v));
    return max_gt(max_gt(row_lane(v, 0), row_lane(v, 16)), max_gt(row_lane(v, 32), row_lane(v, 48)));
}

// ---------------------------------------------------------------------------
// softmax
// ---------------------------------------------------------------------------
// PER float4 per lane: rows up to 256*PER floats, dim % 4 == 0, aligned.
// Each wave walks its rows with the next row's loads issued before the
// current row's reductions, so reads of one row overlap the arithmetic and
// the stores of the previous one.
// the next row is prefetched while its registers fit (rows up to 2048 floats)
template <int PER>
constexpr bool kPrefetch = PER <= 8;

// FULL: the row is exactly 64 * PER float4 (every lane's PER float4 inside
// it), so no lane is masked off and the kernels carry no per-lane bounds
// tests - the exec-mask branches they cost made the row kernels' arithmetic
// phase, which runs between all rows' loads and stores, the longer
template <int PER, bool FULL = false>
__device__ __forceinline__ void load_row4(float4 (&v)[PER], const float* base, int n4, int lane, float fill) {
    const float4* x = reinterpret_cast<const float4*>(base);
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int idx = lane + 64 * q;
        v[q] = FULL || idx < n4 ? x[idx] : make_float4(fill, fill, fill, fill);
    }
}

// DIV: the row's elements divided by the scalar *dv first (nnc_div's x / y)
// - the attention score scaling of nnc_hip_scaled_softmax; the -inf fill of
// lanes past the row stays as it is
template <int PER, bool DIV, bool FULL>
__device__ __forceinline__ void load_sm_row(float4 (&v)[PER], const float* base, int d4, int lane, float dv) {
    load_row4<PER, FULL>(v, base, d4, lane, -INFINITY);
    if (DIV) {
#pragma unroll
        for (int q = 0; q < PER; ++q)
            if (FULL || lane + 64 * q < d4) v[q] = make_float4(v[q].x / dv, v[q].y / dv, v[q].z / dv, v[q].w / dv);
    }
}

template <int PER, bool DIV, bool FULL, bool NT>
__global__ void __launch_bounds__(256) softmax_rows_v4_k(const float* in, const float* div, float* out,
                                                         int64_t rows, int dim) {
    const int lane = threadIdx.x & 63;
    const int64_t wstride = (int64_t)gridDim.x * 4;
    const int d4 = dim / 4;
    int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float dv = DIV ? div[0] : 1.0f;
    float4 v[PER];
    load_sm_row<PER, DIV, FULL>(v, in + row * dim, d4, lane, dv);
    while (true) {
        const int64_t nrow = row + wstride;
        const bool more = nrow < rows;
        float4 nx[PER];
        if (kPrefetch<PER> && more) load_sm_row<PER, DIV, FULL>(nx, in + nrow * dim, d4, lane, dv);
        float m = -INFINITY;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (FULL || lane + 64 * q < d4) {
                if (v[q].x > m) m = v[q].x;
                if (v[q].y > m) m = v[q].y;
                if (v[q].z > m) m = v[q].z;
                if (v[q].w > m) m = v[q].w;
            }
        }
        m = wave_max(m);
        float s = 0.f;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (FULL || lane + 64 * q < d4) {
                v[q].x = __expf(v[q].x - m);
                v[q].y = __expf(v[q].y - m);
                v[q].z = __expf(v[q].z - m);
                v[q].w = __expf(v[q].w - m);
                s += (v[q].x + v[q].y) + (v[q].z + v[q].w);
            }
        }
        s = wave_sum(s);
        float4* y = reinterpret_cast<float4*>(out + row * dim);
        const float rs = 1.0f / s;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int idx = lane + 64 * q;
            if (FULL || idx < d4)
                store_f4<NT>(reinterpret_cast<float*>(y + idx), make_float4(v[q].x * rs, v[q].y * rs, v[q].z * rs, v[q].w * rs));
        }
        if (!more) break;
        if (!kPrefetch<PER>) load_sm_row<PER, DIV, FULL>(nx, in + nrow * dim, d4, lane, dv);
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = nx[q];
        row = nrow;
    }
}

// any contiguous row: three passes over global memory
__global__ void __launch_bounds__(256) softmax_rows_k(const float* in, float* out, int64_t rows,
                                                      int dim) {
    const int lane = threadIdx.x & 63;
    const int64_t wstride = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += wstride) {
        const float* x = in + row * dim;
        float m = -INFINITY;
        for (int i = lane; i < dim; i += 64)
            if (x[i] > m) m = x[i];
        m = wave_max(m);
        float s = 0.f;
        for (int i = lane; i < dim; i += 64) s += expf(x[i] - m);
        s = wave_sum(s);
        float* y = out + row * dim;
        for (int i = lane; i < dim; i += 64) y[i] = expf(x[i] - m) / s;
    }
}

// strided axis: thread per (outer, inner)
__global__ void __launch_bounds__(256) softmax_cols_k(const float* in, float* out, int64_t outer,
                                                      int dim, int64_t inner) {
    const int64_t total = outer * inner;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int64_t o = e / inner, q = e - o * inner;
        const float* x = in + o * dim * inner + q;
        float* y = out + o * dim * inner + q;
        float m = -INFINITY;
        for (int s = 0; s < dim; ++s)
            if (x[s * inner] > m) m = x[s * inner];
        float den = 0.f;
        for (int s = 0; s < dim; ++s) den += expf(x[s * inner] - m);
        for (int s = 0; s < dim; ++s) y[s * inner] = expf(x[s * inner] - m) / den;
    }
}

// ---------------------------------------------------------------------------
// layernorm over a contiguous span of D*inner floats per outer row
// ---------------------------------------------------------------------------
// ADD: the row is in + in2 (same size, nnc_add's element-wise sum) - the
// residual add of nnc_hip_add_layernorm, summed in registers
template <int PER, bool ADD, bool FULL>
__device__ __forceinline__ void load_ln_row(float4 (&v)[PER], const float* in, const float* in2, int64_t off, int s4,
                                            int lane) {
    load_row4<PER, FULL>(v, in + off, s4, lane, 0.f);
    if (ADD) {
        float4 w[PER];
        load_row4<PER, FULL>(w, in2 + off, s4, lane, 0.f);
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = make_float4(v[q].x + w[q].x, v[q].y + w[q].y, v[q].z + w[q].z, v[q].w + w[q].w);
    }
}

template <int PER, bool INNER1, bool ADD, bool FULL, bool NT>
__global__ void __launch_bounds__(256) layernorm_rows_v4_k(const float* in, const float* in2, const float* g,
                                                           const float* b, float* out, int64_t rows,
                                                           int span, int inner, float eps) {
    const int lane = threadIdx.x & 63;
    const int64_t wstride = (int64_t)gridDim.x * 4;
    const int s4 = span / 4;
    int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float4 v[PER];
    load_ln_row<PER, ADD, FULL>(v, in, in2, row * span, s4, lane);
    while (true) {
        const int64_t nrow = row + wstride;
        const bool more = nrow < rows;
        float4 nx[PER];
        if (kPrefetch<PER> && more) load_ln_row<PER, ADD, FULL>(nx, in, in2, nrow * span, s4, lane);
        float acc = 0.f;
#pragma unroll
        for (int q = 0; q < PER; ++q) acc += (v[q].x + v[q].y) + (v[q].z + v[q].w);
        const float mean = wave_sum(acc) / (float)span;
        float sq = 0.f;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            if (FULL || lane + 64 * q < s4) {
                const float dx = v[q].x - mean, dy = v[q].y - mean;
                const float dz = v[q].z - mean, dw = v[q].w - mean;
                sq += (dx * dx + dy * dy) + (dz * dz + dw * dw);
            }
        }
        const float var = wave_sum(sq) / (float)span;
        const float sd = sqrtf(var + eps);
        const float rsd = 1.0f / sd;
        float4* y = reinterpret_cast<float4*>(out + row * span);
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int idx = lane + 64 * q;
            if (FULL || idx < s4) {
                const int e = idx * 4;
                float r[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
                float gv[4] = {1.0f, 1.0f, 1.0f, 1.0f}, bv[4] = {0.0f, 0.0f, 0.0f, 0.0f};
                if (INNER1) {
                    // scale/bias indexed by the element itself: 16-byte loads
                    if (g) {
                        const float4 t = reinterpret_cast<const float4*>(g)[idx];
                        gv[0] = t.x, gv[1] = t.y, gv[2] = t.z, gv[3] = t.w;
                    }
                    if (b) {
                        const float4 t = reinterpret_cast<const float4*>(b)[idx];
                        bv[0] = t.x, bv[1] = t.y, bv[2] = t.z, bv[3] = t.w;
                    }
                } else {
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int i = (e + c) / inner;
                        if (g) gv[c] = g[i];
                        if (b) bv[c] = b[i];
                    }
                }
#pragma unroll
                for (int c = 0; c < 4; ++c) r[c] = gv[c] * ((r[c] - mean) * rsd) + bv[c];
                store_f4<NT>(reinterpret_cast<float*>(y + idx), make_float4(r[0], r[1], r[2], r[3]));
            }
        }
        if (!more) break;
        if (!kPrefetch<PER>) load_ln_row<PER, ADD, FULL>(nx, in, in2, nrow * span, s4, lane);
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = nx[q];
        row = nrow;
    }
}

// any span: one workgroup per row, three passes
__global__ void __launch_bounds__(256) layernorm_rows_k(const float* in, const float* g,
                                                        const float* b, float* out, int64_t rows,
                                                        int64_t span, int64_t inner, float eps) {
    __shared__ float part[4];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const float* x = in + row * span;
        float acc = 0.f;
        for (int64_t e = threadIdx.x; e < span; e += 256) acc += x[e];
        acc = wave_sum(acc);
        if (lane == 0) part[wave] = acc;
        __syncthreads();
        const float mean = ((part[0] + part[1]) + (part[2] + part[3])) / (float)span;
        __syncthreads();
        float sq = 0.f;
        for (int64_t e = threadIdx.x; e < span; e += 256) {
            const float d = x[e] - mean;
            sq += d * d;
        }
        sq = wave_sum(sq);
        if (lane == 0) part[wave] = sq;
        __syncthreads();
        const float var = ((part[0] + part[1]) + (part[2] + part[3])) / (float)span;
        __syncthreads();
        const float sd = sqrtf(var + eps);
        float* y = out + row * span;
        for (int64_t e = threadIdx.x; e < span; e += 256) {
            const int64_t i = e / inner;
            const float gi = g ? g[i] : 1.0f, bi = b ? b[i] : 0.0f;
            y[e] = gi * ((x[e] - mean) / sd) + bi;
        }
    }
}

// ---------------------------------------------------------------------------
// single-axis reductions
// ---------------------------------------------------------------------------
// contiguous rows: wave per row, Kahan per lane, shuffle tree across lanes
template <bool MEAN>
__global__ void __launch_bounds__(256) reduce_rows_k(const float* in, float* out, int64_t rows,
                                                     int64_t len) {
    const int lane = threadIdx.x & 63;
    const int64_t wstride = (int64_t)gridDim.x * 4;
    for (int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6); row < rows; row += wstride) {
        const float* x = in + row * len;
        float s = 0.f, c = 0.f;
        for (int64_t i = lane; i < len; i += 64) {
            const float y = x[i] - c;
            const float t = s + y;
            c = (t - s) - y;
            s = t;
        }
        s = wave_sum(s);
        if (lane == 0) out[row] = MEAN ? s / (float)len : s;
    }
}

// contiguous rows of len % 4 == 0 (16-byte aligned), up to 256*PER floats:
// the row is loaded into registers with 16-byte loads first (all loads in
// flight at once), then Kahan-summed per lane and combined by shuffles
template <bool MEAN, int PER>
__global__ void __launch_bounds__(256) reduce_rows_v4_k(const float* in, float* out, int64_t rows, int len) {
    const int lane = threadIdx.x & 63;
    const int64_t wstride = (int64_t)gridDim.x * 4;
    const int l4 = len / 4;
    int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;
    float4 v[PER];
    load_row4<PER>(v, in + row * len, l4, lane, 0.f);
    while (true) {
        const int64_t nrow = row + wstride;
        const bool more = nrow < rows;
        float4 nx[PER];
        if (kPrefetch<PER> && more) load_row4<PER>(nx, in + nrow * len, l4, lane, 0.f);
        float s = 0.f, c = 0.f;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const float e[4] = {v[q].x, v[q].y, v[q].z, v[q].w};
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const float y = e[u] - c;
                const float t = s + y;
                c = (t - s) - y;
                s = t;
            }
        }
        s = wave_sum(s);
        if (lane == 0) out[row] = MEAN ? s / (float)len : s;
        if (!more) break;
        if (!kPrefetch<PER>) load_row4<PER>(nx, in + nrow * len, l4, lane, 0.f);
#pragma unroll
        for (int q = 0; q < PER; ++q) v[q] = nx[q];
        row = nrow;
    }
}

// strided axis: thread per (outer, inner), the reference's sequential Kahan sum
template <bool MEAN>
__global__ void __launch_bounds__(256) reduce_cols_k(const float* in, float* out, int64_t outer,
                                                     int64_t len, int64_t inner) {
    const int64_t total = outer * inner;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int64_t o = e / inner, q = e - o * inner;
        const float* x = in + o * len * inner + q;
        float s = 0.f, c = 0.f;
        for (int64_t r = 0; r < len; ++r) {
            const float y = x[r * inner] - c;
            const float t = s + y;
            c = (t - s) - y;
            s = t;
        }
        out[e] = MEAN ? s / (float)len : s;
    }
}

static bool split_axis(const char* name, Tensor* in, int& axis, int64_t& outer, int64_t& len,
                       int64_t& inner) {
    const int nd = in->ndim;
    if (axis < 0) axis += nd;
    if (axis < 0 || axis >= nd) {
        fail(NNC_HIP_EINVAL, name, "axis out of range");
        return false;
    }
    outer = prod(in->shape, 0, axis);
    len = in->shape[axis];
    inner = prod(in->shape, axis + 1, nd);
    return true;
}

// one row per wave (measured fastest: every row's loads in flight at once);
// past the grid cap a wave walks several rows, prefetching the next
static unsigned row_grid(int64_t rows) { return grid_for(rows, 4, 1); }

template <int PER, bool FULL, bool NT>
static void softmax_v4_at(const float* x, const float* dv, float* y, int64_t rows, int dim, const char* name) {
    if (dv) launch(name, softmax_rows_v4_k<PER, true, FULL, NT>, dim3(row_grid(rows)), dim3(256), 0, x, dv, y, rows, dim);
    else launch(name, softmax_rows_v4_k<PER, false, FULL, NT>, dim3(row_grid(rows)), dim3(256), 0, x, dv, y, rows, dim);
}
template <int PER>
static void softmax_v4(const float* x, const float* dv, float* y, int64_t rows, int dim, const char* name) {
    const bool full = dim == 256 * PER, nt = 4 * rows * dim >= kNtStoreBytes;
    if (full && nt) softmax_v4_at<PER, true, true>(x, dv, y, rows, dim, name);
    else if (full) softmax_v4_at<PER, true, false>(x, dv, y, rows, dim, name);
    else if (nt) softmax_v4_at<PER, false, true>(x, dv, y, rows, dim, name);
    else softmax_v4_at<PER, false, false>(x, dv, y, rows, dim, name);
}

template <int PER, bool FULL, bool NT>
static void layernorm_v4_at(const float* x, const float* x2, const float* g, const float* b, float* y, int64_t rows,
                            int span, int inner, float eps, const char* name) {
    // inner == 1 with 16-byte aligned scale/bias: vector loads of those too
    const bool in1 = inner == 1 && (!g || aligned16(g)) && (!b || aligned16(b));
    const dim3 grid(row_grid(rows)), block(256);
    if (x2 && in1) launch(name, layernorm_rows_v4_k<PER, true, true, FULL, NT>, grid, block, 0, x, x2, g, b, y, rows, span, inner, eps);
    else if (x2) launch(name, layernorm_rows_v4_k<PER, false, true, FULL, NT>, grid, block, 0, x, x2, g, b, y, rows, span, inner, eps);
    else if (in1) launch(name, layernorm_rows_v4_k<PER, true, false, FULL, NT>, grid, block, 0, x, x2, g, b, y, rows, span, inner, eps);
    else launch(name, layernorm_rows_v4_k<PER, false, false, FULL, NT>, grid, block, 0, x, x2, g, b, y, rows, span, inner, eps);
}
template <int PER>
static void layernorm_v4(const float* x, const float* x2, const float* g, const float* b, float* y, int64_t rows,
                         int span, int inner, float eps, const char* name) {
    const bool full = span == 256 * PER, nt = 4 * rows * span >= kNtStoreBytes;
    if (full && nt) layernorm_v4_at<PER, true, true>(x, x2, g, b, y, rows, span, inner, eps, name);
    else if (full) layernorm_v4_at<PER, true, false>(x, x2, g, b, y, rows, span, inner, eps, name);
    else if (nt) layernorm_v4_at<PER, false, true>(x, x2, g, b, y, rows, span, inner, eps, name);
    else layernorm_v4_at<PER, false, false>(x, x2, g, b, y, rows, span, inner, eps, name);
}

}  // namespace nnc

using namespace nnc;

extern "C" {

// softmax over axis of in (divided first by the one-element div: the
// attention scaling of nnc_hip_scaled_softmax, out the size of in)
static void softmax_run(Tensor* in, Tensor* div, Tensor* out, int axis, const char* name) {
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out) || (div && !has_data(div))) return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    int64_t outer, len, inner;
    if (!split_axis(name, in, axis, outer, len, inner)) return;
    if (numel(out) < numel(in)) return fail(NNC_HIP_EINVAL, name, "output smaller than input");
    if (div && numel(div) != 1) return fail(NNC_HIP_EINVAL, name, "the divisor is not one element");
    if (div && numel(out) != numel(in)) return fail(NNC_HIP_EINVAL, name, "output and input differ in size");
    if (outer * len * inner == 0) return;
    const float* x = (const float*)in->data;
    const float* dv = div ? (const float*)div->data : nullptr;
    float* y = (float*)out->data;
    if (len >= (1 << 30)) return fail(NNC_HIP_EUNSUPP, name, "axis too long");
    set_work(0.0, 8.0 * (double)(outer * len * inner) + (div ? 4.0 : 0.0));
    if (inner == 1) {
        const int dim = (int)len;
        const bool v4 = dim % 4 == 0 && aligned16(x) && aligned16(y);
        if (v4 && dim <= 256) return softmax_v4<1>(x, dv, y, outer, dim, name);
        if (v4 && dim <= 512) return softmax_v4<2>(x, dv, y, outer, dim, name);
        if (v4 && dim <= 1024) return softmax_v4<4>(x, dv, y, outer, dim, name);
        if (v4 && dim <= 2048) return softmax_v4<8>(x, dv, y, outer, dim, name);
        if (v4 && dim <= 4096) return softmax_v4<16>(x, dv, y, outer, dim, name);
    }
    if (div) {
        // other rows: the quotient into out, then the softmax over it in
        // place (each lane reads an element before it writes it)
        nnc_div(in, div, out);
        x = y;
    }
    if (inner == 1) {
        launch(name, softmax_rows_k, dim3(grid_for(outer, 4, 1)), dim3(256), 0, x, y, outer, (int)len);
        return;
    }
    launch(name, softmax_cols_k, dim3(grid_for(outer * inner, 1)), dim3(256), 0, x, y, outer, (int)len,
           inner);
}

void nnc_softmax(Tensor* in, Tensor* out, int axis) { softmax_run(in, nullptr, out, axis, "nnc_softmax"); }

// No reference counterpart: the attention scaling (a Div by a one-element
// tensor) and the softmax after it in one pass (the mi355x target's O3
// fusion of Div -> Softmax).
void nnc_hip_scaled_softmax(Tensor* in, Tensor* div, Tensor* out, int axis) {
    if (!div) return fail(NNC_HIP_EINVAL, "nnc_hip_scaled_softmax", "NULL divisor");
    softmax_run(in, div, out, axis, "nnc_hip_scaled_softmax");
}

// layernorm of in (+ in2, same size: the residual add of
// nnc_hip_add_layernorm) over [axis:]
static void layernorm_run(Tensor* in, Tensor* in2, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps,
                          const char* name) {
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out) || (in2 && !has_data(in2))) return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    int64_t outer, len, inner;
    if (!split_axis(name, in, axis, outer, len, inner)) return;
    const int64_t span = len * inner;
    if (numel(out) < numel(in)) return fail(NNC_HIP_EINVAL, name, "output smaller than input");
    if (in2 && numel(in2) != numel(in)) return fail(NNC_HIP_EINVAL, name, "the two addends differ in size");
    if (outer * span == 0) return;
    const float* x = (const float*)in->data;
    const float* x2 = in2 ? (const float*)in2->data : nullptr;
    const float* g = (scale && scale->data) ? (const float*)scale->data : nullptr;
    const float* b = (bias && bias->data) ? (const float*)bias->data : nullptr;
    if ((g && numel(scale) < len) || (b && numel(bias) < len))
        return fail(NNC_HIP_EINVAL, name, "scale/bias shorter than the axis");
    float* y = (float*)out->data;
    set_work(0.0, (x2 ? 12.0 : 8.0) * (double)(outer * span) + (g ? 4.0 * len : 0.0) + (b ? 4.0 * len : 0.0));
    const bool v4 = span % 4 == 0 && span < (1 << 30) && aligned16(x) && aligned16(y) && (!x2 || aligned16(x2));
    const int sp = (int)span, inn = (int)inner;
    if (v4 && span <= 256) return layernorm_v4<1>(x, x2, g, b, y, outer, sp, inn, eps, name);
    if (v4 && span <= 512) return layernorm_v4<2>(x, x2, g, b, y, outer, sp, inn, eps, name);
    if (v4 && span == 768) return layernorm_v4<3>(x, x2, g, b, y, outer, sp, inn, eps, name);
    if (v4 && span <= 1024) return layernorm_v4<4>(x, x2, g, b, y, outer, sp, inn, eps, name);
    if (v4 && span <= 2048) return layernorm_v4<8>(x, x2, g, b, y, outer, sp, inn, eps, name);
    if (v4 && span <= 4096) return layernorm_v4<16>(x, x2, g, b, y, outer, sp, inn, eps, name);
    if (x2) {
        // other spans: the sum into out, then the layernorm over it in place
        // (each pass reads an element before writing it)
        nnc_add(in, in2, out);
        x = y;
    }
    unsigned grid = (unsigned)(outer < 65536 ? outer : 65536);
    launch(name, layernorm_rows_k, dim3(grid), dim3(256), 0, x, g, b, y, outer, span, inner, eps);
}

void nnc_layernorm(Tensor* in, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps) {
    layernorm_run(in, nullptr, scale, bias, out, axis, eps, "nnc_layernorm");
}

// No reference counterpart: the residual add and the layernorm after it in
// one pass (the mi355x target's O3 fusion of Add -> LayerNormalization).
void nnc_hip_add_layernorm(Tensor* a, Tensor* b, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps) {
    if (!b) return fail(NNC_HIP_EINVAL, "nnc_hip_add_layernorm", "NULL addend");
    layernorm_run(a, b, scale, bias, out, axis, eps, "nnc_hip_add_layernorm");
}

static void reduce_entry(const char* name, Tensor* in, Tensor* out, int axis, bool mean) {
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    int64_t outer, len, inner;
    if (!split_axis(name, in, axis, outer, len, inner)) return;
    if (numel(out) < outer * inner) return fail(NNC_HIP_EINVAL, name, "output smaller than the reduction");
    if (outer * inner == 0) return;
    const float* x = (const float*)in->data;
    float* y = (float*)out->data;
    set_work(0.0, 4.0 * (double)(outer * len * inner + outer * inner));
    if (inner == 1) {
        const dim3 grid(grid_for(outer, 4, 1));
        const dim3 grid_v4(row_grid(outer));
        if (len % 4 == 0 && len <= 4096 && aligned16(x)) {
#define NNC_REDUCE_V4(PER)                                                                             \
    if (len <= 256 * PER) {                                                                            \
        if (mean) launch(name, reduce_rows_v4_k<true, PER>, grid_v4, dim3(256), 0, x, y, outer, (int)len); \
        else launch(name, reduce_rows_v4_k<false, PER>, grid_v4, dim3(256), 0, x, y, outer, (int)len); \
        return;                                                                                        \
    }
            NNC_REDUCE_V4(1)
            NNC_REDUCE_V4(2)
            NNC_REDUCE_V4(4)
            NNC_REDUCE_V4(8)
            NNC_REDUCE_V4(16)
#undef NNC_REDUCE_V4
        }
        if (mean) launch(name, reduce_rows_k<true>, grid, dim3(256), 0, x, y, outer, len);
        else launch(name, reduce_rows_k<false>, grid, dim3(256), 0, x, y, outer, len);
        return;
    }
    const dim3 g(grid_for(outer * inner, 1));
    if (mean) launch(name, reduce_cols_k<true>, g, dim3(256), 0, x, y, outer, len, inner);
    else launch(name, reduce_cols_k<false>, g, dim3(256), 0, x, y, outer, len, inner);
}

void nnc_reducemean(Tensor* in, Tensor* out, int axis, int keepdims) {
    (void)keepdims;
    reduce_entry("nnc_reducemean", in, out, axis, true);
}

void nnc_reducesum(Tensor* in, Tensor* out, int axis, int keepdims) {
    (void)keepdims;
    reduce_entry("nnc_reducesum", in, out, axis, false);
}

}  // extern "C"
