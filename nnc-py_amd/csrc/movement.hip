// Data-movement operators of the nnc ABI: Reshape / Flatten / Squeeze /
// Unsqueeze / Identity (ops.c:1510-1601, 2173-2181), Transpose (ops.c:1531),
// Concat / Split (ops.c:1995-2086, 2183-2251), Tile / Shape / Gather
// (ops.c:2264-2336, 2601-2619, 2705-2913) and the no-op BatchNorm
// (ops.c:2088-2093). All of them copy bits, so they are bit-exact.
//
// Copies are kernels (not hipMemcpy) so they time like every other op and
// record as kernel nodes under graph capture. HBM-bound: 16-byte loads and
// stores where source, destination and size allow.
#include <type_traits>

#include "common.h"

namespace nnc {

template <bool NT>
__global__ void __launch_bounds__(256) copy16_k(const uint4* src, uint4* dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
        store_u4<NT>(dst + i, src[i]);
}

__global__ void __launch_bounds__(256) copy1_k(const uint8_t* src, uint8_t* dst, int64_t n) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
        dst[i] = src[i];
}

void device_copy(const char* name, const void* src, void* dst, size_t bytes) {
    if (src == dst || bytes == 0) return;
    set_work(0.0, 2.0 * (double)bytes);
    const uint8_t* s = static_cast<const uint8_t*>(src);
    uint8_t* d = static_cast<uint8_t*>(dst);
    size_t done = 0;
    if (aligned16(s) && aligned16(d) && bytes >= 16) {
        const int64_t n16 = (int64_t)(bytes / 16);
        if ((int64_t)bytes >= kNtStoreBytes)
            launch(name, copy16_k<true>, dim3(grid_for(n16, 2)), dim3(256), 0, (const uint4*)s, (uint4*)d, n16);
        else
            launch(name, copy16_k<false>, dim3(grid_for(n16, 2)), dim3(256), 0, (const uint4*)s, (uint4*)d, n16);
        done = (size_t)n16 * 16;
    }
    if (done < bytes)
        launch(name, copy1_k, dim3(grid_for((int64_t)(bytes - done), 1)), dim3(256), 0, s + done,
               d + done, (int64_t)(bytes - done));
}

// ---------------------------------------------------------------------------
// transpose: output index decomposed over the output extents, each output
// axis d advancing the input by the stride of input axis perm[d]
// ---------------------------------------------------------------------------
struct PermArgs {
    int ndim;
    int64_t out_ext[8];
    int64_t in_stride_of_out_axis[8];
};

template <typename E>
__global__ void __launch_bounds__(256) permute_k(const E* in, E* out, int64_t total, PermArgs p) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
        int64_t rem = o, src = 0;
        for (int d = p.ndim - 1; d >= 0; --d) {
            const int64_t ext = p.out_ext[d];
            const int64_t idx = rem % ext;
            rem /= ext;
            src += idx * p.in_stride_of_out_axis[d];
        }
        out[o] = in[src];
    }
}

// permute_k over a column slice: the permuted tensor is the [rows][width]
// block at column col0 of a [rows][W] buffer, read row-major (a Split's
// piece, reshaped); p's strides are the slice's own, each source index f
// lands at row f / width, column col0 + f % width of the buffer
__global__ void __launch_bounds__(256) permute_slice_k(const float* in, float* out, int64_t total, PermArgs p,
                                                       int64_t width, int64_t W, int64_t col0) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
        int64_t rem = o, src = 0;
        for (int d = p.ndim - 1; d >= 0; --d) {
            const int64_t ext = p.out_ext[d];
            const int64_t idx = rem % ext;
            rem /= ext;
            src += idx * p.in_stride_of_out_axis[d];
        }
        const int64_t r = src / width;
        out[o] = in[r * W + col0 + (src - r * width)];
    }
}

// 2-D tile transpose through LDS for batched [B][R][C] -> [B][C][R]
// (the innermost axis moves): coalesced reads along C and writes along R.
__global__ void __launch_bounds__(256) transpose2d_k(const float* in, float* out, int64_t R, int64_t C) {
    __shared__ float tile[32][33];
    const int64_t b = blockIdx.z;
    const float* src = in + b * R * C;
    float* dst = out + b * R * C;
    const int64_t r0 = (int64_t)blockIdx.y * 32, c0 = (int64_t)blockIdx.x * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int k = ty; k < 32; k += 8) {
        const int64_t r = r0 + k, c = c0 + tx;
        if (r < R && c < C) tile[k][tx] = src[r * C + c];
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int64_t c = c0 + k, r = r0 + tx;
        if (r < R && c < C) dst[c * R + r] = tile[tx][k];
    }
}

// ---------------------------------------------------------------------------
// concat / split: strided 2-D copies [outer][slab] <-> [outer][row] at column
// ---------------------------------------------------------------------------
// grid (ceil(slab / 256), rows): one element per thread, 32-bit index
// within a row, rows strided by grid.y; no per-element division
template <typename E, bool NT>
__global__ void __launch_bounds__(256) slab_copy_k(const E* src, int64_t src_row, E* dst,
                                                   int64_t dst_row, int64_t outer, uint32_t slab) {
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    if (i >= slab) return;
    for (int64_t o = blockIdx.y; o < outer; o += gridDim.y) {
        if constexpr (NT && std::is_same<E, uint4>::value)
            store_u4<true>(dst + o * dst_row + i, src[o * src_row + i]);
        else
            dst[o * dst_row + i] = src[o * src_row + i];
    }
}

// `nt`: non-temporal stores (a large total output, kNtStoreBytes)
template <typename E>
static void slab_launch(const char* name, const E* src, int64_t src_row, E* dst, int64_t dst_row, int64_t outer,
                        int64_t slab, bool nt) {
    if (slab >= ((int64_t)1 << 32) - 256) {
        // rows longer than 2^32 elements: one launch per 2^31-element chunk
        const int64_t chunk = (int64_t)1 << 31;
        for (int64_t c = 0; c < slab; c += chunk)
            slab_launch(name, src + c, src_row, dst + c, dst_row, outer, slab - c < chunk ? slab - c : chunk, nt);
        return;
    }
    const int64_t gy = outer < 65535 ? outer : 65535;
    const dim3 grid((unsigned)ceil_div(slab, 256), (unsigned)gy);
    if (nt)
        launch(name, slab_copy_k<E, true>, grid, dim3(256), 0, src, src_row, dst, dst_row, outer, (uint32_t)slab);
    else
        launch(name, slab_copy_k<E, false>, grid, dim3(256), 0, src, src_row, dst, dst_row, outer, (uint32_t)slab);
}

// `total_out_bytes`: the whole output the caller's copies fill (a concat's
// or a split's), which decides the store kind
template <typename E>
static void slab_copy(const char* name, const void* src, int64_t src_row, void* dst, int64_t dst_row,
                      int64_t outer, int64_t slab, int64_t total_out_bytes) {
    if (outer * slab == 0) return;
    set_work(0.0, 2.0 * (double)(outer * slab) * sizeof(E));
    const bool nt = total_out_bytes >= kNtStoreBytes;
    // 16-byte granules when every row start stays aligned
    const int64_t per16 = 16 / (int64_t)sizeof(E);
    if (aligned16(src) && aligned16(dst) && slab % per16 == 0 && src_row % per16 == 0 &&
        dst_row % per16 == 0) {
        slab_launch(name, (const uint4*)src, src_row / per16, (uint4*)dst, dst_row / per16, outer, slab / per16, nt);
        return;
    }
    slab_launch(name, (const E*)src, src_row, (E*)dst, dst_row, outer, slab, false);
}

// ---------------------------------------------------------------------------
// tile: output coordinate modulo input extent on every axis
// ---------------------------------------------------------------------------
struct TileArgs {
    int in_ndim, out_ndim;
    int64_t out_ext[8];
    int64_t in_ext[8];
    int64_t in_stride[8];
};

__global__ void __launch_bounds__(256) tile_k(const float* in, float* out, int64_t total, TileArgs t) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; o < total; o += stride) {
        int64_t coord[8];
        int64_t rem = o;
        for (int d = t.out_ndim - 1; d >= 0; --d) {
            coord[d] = rem % t.out_ext[d];
            rem /= t.out_ext[d];
        }
        int64_t src = 0;
        for (int d = 0; d < t.in_ndim; ++d) src += (coord[d] % t.in_ext[d]) * t.in_stride[d];
        out[o] = in[src];
    }
}

struct I64x8 {
    int64_t v[8];
};

__global__ void write_i64_k(int64_t* out, I64x8 vals, int n) {
    const int i = threadIdx.x;
    if (i < n) out[i] = vals.v[i];
}

// ---------------------------------------------------------------------------
// gather: the reference's cases (ops.c:2705-2913); the index is read on the
// device, wrapped once if negative and clamped to [0, dim-1].
// ---------------------------------------------------------------------------
enum GatherMode {
    kGScalarI64Flat,  // int64 data, out[i] = d[g*row + i]
    kGScalarF32Fill,  // rank-1 float data, out[i] = d[g]
    kGScalar2D,       // rank-2 data, out[i][j] = axis0 ? d[g*d1+j] : d[i*d1+g]
    kGScalar3D0,      // out[(i*o1+j)*o2+k] = d[g*d1*d2 + j*d2 + k]
    kGScalar3D1,      // out[i*d2+k] = d[(i*d1+g)*d2+k]
    kGScalar3D2,      // out[i*d1+j] = d[(i*d1+j)*d2+g]
    kGListI64,        // rank-1 int64 data, out[t] = d[idx[t]]
    kGList2D0,        // out[t*d1+j] = d[idx[t]*d1+j]
    kGList2D1,        // out[i*cnt+t] = d[i*d1+idx[t]]
    kGModulo          // out[i] = d[i % numel(data)]
};

struct GatherArgs {
    const void* data;
    const int64_t* idx;
    void* out;
    int mode, esz;  // element size 4 or 8
    int64_t dim;    // extent of the gathered axis
    int64_t d0, d1, d2, o0, o1, o2, row, cnt, dn, on;
    int axis;
};

__device__ __forceinline__ int64_t clamp_index(int64_t v, int64_t dim) {
    if (v < 0) v += dim;
    if (v < 0) v = 0;
    if (v >= dim) v = dim - 1;
    return v;
}

__device__ __forceinline__ void copy_elem(const GatherArgs& a, int64_t dst, int64_t src) {
    if (src < 0 || src >= a.dn) return;  // never read outside the data tensor
    if (a.esz == 8)
        static_cast<int64_t*>(a.out)[dst] = static_cast<const int64_t*>(a.data)[src];
    else
        static_cast<float*>(a.out)[dst] = static_cast<const float*>(a.data)[src];
}

__global__ void __launch_bounds__(256) gather_k(GatherArgs a, int64_t total) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        switch (a.mode) {
            case kGScalarI64Flat: {
                const int64_t g = clamp_index(a.idx[0], a.dim);
                copy_elem(a, e, g * a.row + e);
                break;
            }
            case kGScalarF32Fill: copy_elem(a, e, clamp_index(a.idx[0], a.dim)); break;
            case kGScalar2D: {
                const int64_t g = clamp_index(a.idx[0], a.dim);
                const int64_t i = e / a.o1, j = e - i * a.o1;
                copy_elem(a, e, a.axis == 0 ? g * a.d1 + j : i * a.d1 + g);
                break;
            }
            case kGScalar3D0: {
                const int64_t g = clamp_index(a.idx[0], a.dim);
                const int64_t k = e % a.o2, j = (e / a.o2) % a.o1;
                copy_elem(a, e, g * a.d1 * a.d2 + j * a.d2 + k);
                break;
            }
            case kGScalar3D1: {
                const int64_t g = clamp_index(a.idx[0], a.dim);
                const int64_t i = e / a.d2, k = e - i * a.d2;
                copy_elem(a, e, (i * a.d1 + g) * a.d2 + k);
                break;
            }
            case kGScalar3D2: {
                const int64_t g = clamp_index(a.idx[0], a.dim);
                copy_elem(a, e, e * a.d2 + g);  // (i*d1 + j)*d2 + g with e = i*d1 + j
                break;
            }
            case kGListI64: copy_elem(a, e, clamp_index(a.idx[e], a.dim)); break;
            case kGList2D0: {
                const int64_t t = e / a.d1, j = e - t * a.d1;
                copy_elem(a, e, clamp_index(a.idx[t], a.dim) * a.d1 + j);
                break;
            }
            case kGList2D1: {
                const int64_t i = e / a.cnt, t = e - i * a.cnt;
                copy_elem(a, e, i * a.d1 + clamp_index(a.idx[t], a.dim));
                break;
            }
            default: copy_elem(a, e, e % a.dn); break;
        }
    }
}

static bool two(const char* name, Tensor* a, Tensor* b) {
    if (!ready(name)) return false;
    if (!has_data(a) || !has_data(b)) {
        fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
        return false;
    }
    return true;
}

// copy numel(out) floats (reshape-like ops read numel(output) elements)
static void copy_out_count(const char* name, Tensor* in, Tensor* out) {
    if (!two(name, in, out)) return;
    const int64_t n = numel(out);
    if (numel(in) < n) return fail(NNC_HIP_EINVAL, name, "input smaller than output");
    device_copy(name, in->data, out->data, (size_t)n * 4);
}

}  // namespace nnc

using namespace nnc;

extern "C" {

void nnc_reshape(Tensor* in, Tensor* out, int64_t* shape, int ndim) {
    (void)shape;
    (void)ndim;
    copy_out_count("nnc_reshape", in, out);
}
void nnc_flatten(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    copy_out_count("nnc_flatten", in, out);
}
void nnc_squeeze(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    copy_out_count("nnc_squeeze", in, out);
}
void nnc_unsqueeze(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    copy_out_count("nnc_unsqueeze", in, out);
}

void nnc_identity(Tensor* in, Tensor* out) {
    const char* name = "nnc_identity";
    if (!two(name, in, out)) return;
    int64_t n = numel(out), m = numel(in);
    device_copy(name, in->data, out->data, (size_t)(m < n ? m : n) * 4);
}

void nnc_transpose(Tensor* in, Tensor* out, int64_t* perm, int ndim) {
    const char* name = "nnc_transpose";
    if (!two(name, in, out)) return;
    if (ndim < 1 || ndim > 8 || in->ndim != ndim || out->ndim != ndim)
        return fail(NNC_HIP_EINVAL, name, "rank %d (tensors %d/%d, at most 8)", ndim, in->ndim, out->ndim);
    int64_t pm[8];
    for (int d = 0; d < ndim; ++d) pm[d] = perm ? perm[d] : ndim - 1 - d;
    int64_t is[8];
    is[ndim - 1] = 1;
    for (int d = ndim - 2; d >= 0; --d) is[d] = is[d + 1] * in->shape[d + 1];
    for (int d = 0; d < ndim; ++d)
        if (pm[d] < 0 || pm[d] >= ndim || out->shape[d] != in->shape[pm[d]])
            return fail(NNC_HIP_EINVAL, name, "permutation does not match the shapes");
    const int64_t total = numel(out);
    if (total == 0) return;
    set_work(0.0, 8.0 * (double)total);
    // [B..][R][C] -> [B..][C][R]: leading axes kept, last two swapped
    bool swap_last = ndim >= 2 && pm[ndim - 1] == ndim - 2 && pm[ndim - 2] == ndim - 1;
    for (int d = 0; d < ndim - 2 && swap_last; ++d) swap_last = pm[d] == d;
    if (swap_last && in->dtype != NNC_DTYPE_INT64) {
        const int64_t R = in->shape[ndim - 2], C = in->shape[ndim - 1];
        const int64_t B = total / (R * C);
        if (B < 65536) {
            launch(name, transpose2d_k, dim3((unsigned)ceil_div(C, 32), (unsigned)ceil_div(R, 32), (unsigned)B),
                   dim3(256), 0, (const float*)in->data, (float*)out->data, R, C);
            return;
        }
    }
    PermArgs p{};
    p.ndim = ndim;
    for (int d = 0; d < ndim; ++d) {
        p.out_ext[d] = out->shape[d];
        p.in_stride_of_out_axis[d] = is[pm[d]];
    }
    launch(name, permute_k<float>, dim3(grid_for(total, 1)), dim3(256), 0, (const float*)in->data,
           (float*)out->data, total, p);
}

// No reference counterpart: a Split piece's reshape and transpose read
// straight from the unsplit tensor (the mi355x target's O3 fusion of Split
// -> Reshape -> Transpose).
void nnc_hip_transpose_slice(Tensor* in, Tensor* out, int64_t* perm, int ndim, int col0, int width) {
    const char* name = "nnc_hip_transpose_slice";
    if (!two(name, in, out)) return;
    if (ndim < 1 || ndim > 8 || out->ndim != ndim || in->ndim < 1)
        return fail(NNC_HIP_EINVAL, name, "rank %d (output %d, at most 8)", ndim, out->ndim);
    // the gather moves 4-byte words: float32 or int32 on both sides
    const bool four_in = in->dtype == NNC_DTYPE_FLOAT32 || in->dtype == NNC_DTYPE_INT32;
    const bool four_out = out->dtype == NNC_DTYPE_FLOAT32 || out->dtype == NNC_DTYPE_INT32;
    if (!four_in || !four_out || in->dtype != out->dtype)
        return fail(NNC_HIP_EUNSUPP, name, "float32 or int32 elements of one type only (dtypes %d, %d)",
                    (int)in->dtype, (int)out->dtype);
    const int64_t W = in->shape[in->ndim - 1];
    if (col0 < 0 || width < 1 || col0 + width > W)
        return fail(NNC_HIP_EINVAL, name, "columns [%lld, %lld) outside rows of %lld", (long long)col0,
                    (long long)(col0 + width), (long long)W);
    const int64_t rows = numel(in) / W, total = numel(out);
    if (total != rows * width)
        return fail(NNC_HIP_EINVAL, name, "output of %lld elements, the slice holds %lld", (long long)total,
                    (long long)(rows * width));
    int64_t pm[8], vs[8], vst[8];
    unsigned seen = 0;
    for (int d = 0; d < ndim; ++d) {
        pm[d] = perm ? perm[d] : ndim - 1 - d;
        if (pm[d] < 0 || pm[d] >= ndim || (seen >> pm[d] & 1u)) return fail(NNC_HIP_EINVAL, name, "not a permutation");
        seen |= 1u << pm[d];
        vs[pm[d]] = out->shape[d];
    }
    vst[ndim - 1] = 1;
    for (int d = ndim - 2; d >= 0; --d) vst[d] = vst[d + 1] * vs[d + 1];
    if (total == 0) return;
    PermArgs p{};
    p.ndim = ndim;
    for (int d = 0; d < ndim; ++d) {
        p.out_ext[d] = out->shape[d];
        p.in_stride_of_out_axis[d] = vst[pm[d]];
    }
    set_work(0.0, 8.0 * (double)total);
    launch(name, permute_slice_k, dim3(grid_for(total, 1)), dim3(256), 0, (const float*)in->data,
           (float*)out->data, total, p, width, W, col0);
}

void nnc_tile(Tensor* in, Tensor* out, int64_t* repeats, int ndim) {
    (void)ndim;
    const char* name = "nnc_tile";
    if (!two(name, in, out)) return;
    if (!repeats) return copy_out_count(name, in, out);
    if (in->ndim < 1 || in->ndim > 8 || out->ndim > 8 || out->ndim < in->ndim)
        return fail(NNC_HIP_EINVAL, name, "unsupported ranks");
    TileArgs t{};
    t.in_ndim = in->ndim;
    t.out_ndim = out->ndim;
    for (int d = 0; d < out->ndim; ++d) t.out_ext[d] = out->shape[d];
    for (int d = 0; d < in->ndim; ++d) {
        t.in_ext[d] = in->shape[d];
        if (t.in_ext[d] <= 0) return;
    }
    t.in_stride[in->ndim - 1] = 1;
    for (int d = in->ndim - 2; d >= 0; --d) t.in_stride[d] = t.in_stride[d + 1] * in->shape[d + 1];
    const int64_t total = numel(out);
    launch(name, tile_k, dim3(grid_for(total, 1)), dim3(256), 0, (const float*)in->data, (float*)out->data,
           total, t);
}

void nnc_concat(Tensor** ins, Tensor* out, int n_in, int axis) {
    const char* name = "nnc_concat";
    if (!ready(name)) return;
    if (!has_data(out) || (n_in > 0 && !ins)) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    if (axis < 0) axis += out->ndim;
    if (axis < 0 || axis >= out->ndim) return fail(NNC_HIP_EINVAL, name, "axis out of range");
    const bool i64 = out->dtype == NNC_DTYPE_INT64;
    const int64_t outer = prod(out->shape, 0, axis);
    const int64_t inner = prod(out->shape, axis + 1, out->ndim);
    const int64_t out_row = out->shape[axis] * inner;
    int64_t col = 0;
    for (int t = 0; t < n_in; ++t) {
        if (!has_data(ins[t]) || ins[t]->ndim <= axis) return fail(NNC_HIP_EINVAL, name, "bad input %d", t);
        const int64_t slab = ins[t]->shape[axis] * inner;
        if (col + slab > out_row) return fail(NNC_HIP_EINVAL, name, "inputs exceed the output axis");
        char* dst = (char*)out->data + col * (i64 ? 8 : 4);
        const int64_t total = outer * out_row * (i64 ? 8 : 4);
        if (i64) slab_copy<int64_t>(name, ins[t]->data, slab, dst, out_row, outer, slab, total);
        else slab_copy<float>(name, ins[t]->data, slab, dst, out_row, outer, slab, total);
        col += slab;
    }
}

void nnc_split(Tensor* in, Tensor** outs, int n_out, int axis) {
    const char* name = "nnc_split";
    if (!ready(name)) return;
    if (!has_data(in) || n_out <= 0 || !outs) return fail(NNC_HIP_EINVAL, name, "NULL tensor");
    if (axis < 0) axis += in->ndim;
    if (axis < 0 || axis >= in->ndim) return fail(NNC_HIP_EINVAL, name, "axis out of range");
    const bool i64 = in->dtype == NNC_DTYPE_INT64;
    const int64_t outer = prod(in->shape, 0, axis);
    const int64_t dim = in->shape[axis];
    const int64_t part = dim / n_out;
    const int64_t inner = prod(in->shape, axis + 1, in->ndim);
    for (int t = 0; t < n_out; ++t) {
        if (!has_data(outs[t])) return fail(NNC_HIP_EINVAL, name, "bad output %d", t);
        if (numel(outs[t]) < outer * part * inner) return fail(NNC_HIP_EINVAL, name, "output %d too small", t);
        const char* src = (const char*)in->data + t * part * inner * (i64 ? 8 : 4);
        const int64_t total = outer * dim * inner * (i64 ? 8 : 4);
        if (i64) slab_copy<int64_t>(name, src, dim * inner, outs[t]->data, part * inner, outer, part * inner, total);
        else slab_copy<float>(name, src, dim * inner, outs[t]->data, part * inner, outer, part * inner, total);
    }
}

void nnc_shape(Tensor* in, Tensor* out, int64_t* shape_data, int ndim) {
    const char* name = "nnc_shape";
    if (!ready(name)) return;
    if (!has_data(out) || ndim < 0 || ndim > 8) return fail(NNC_HIP_EINVAL, name, "bad arguments");
    if (!shape_data && (!in || in->ndim < ndim)) return fail(NNC_HIP_EINVAL, name, "no shape source");
    I64x8 v{};
    for (int d = 0; d < ndim; ++d) v.v[d] = shape_data ? shape_data[d] : in->shape[d];
    launch(name, write_i64_k, dim3(1), dim3(64), 0, (int64_t*)out->data, v, ndim);
}

void nnc_gather(Tensor* data, Tensor* indices, Tensor* out, int axis, int data_dtype) {
    const char* name = "nnc_gather";
    if (!ready(name)) return;
    if (!has_data(data) || !has_data(indices) || !has_data(out))
        return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    const int rank = data->ndim, irank = indices->ndim, orank = out->ndim;
    if (rank < 1) return fail(NNC_HIP_EINVAL, name, "rank-0 data");
    if (axis < 0) axis += rank;
    if (axis < 0) axis = 0;
    if (axis >= rank) axis = rank - 1;
    GatherArgs a{};
    a.data = data->data;
    a.idx = (const int64_t*)indices->data;
    a.out = out->data;
    a.esz = 4;
    a.axis = axis;
    a.dim = data->shape[axis];
    a.dn = numel(data);
    a.on = numel(out);
    int64_t total = a.on;
    int mode = -1;
    const bool single = irank == 0 || (irank == 1 && indices->shape[0] == 1);
    if (single) {
        if (data_dtype == 1) {
            a.esz = 8;
            if (rank == 1) {
                mode = kGListI64;  // out[0] = d[clamp(idx[0])]
                total = 1;
            } else {
                mode = kGScalarI64Flat;
                a.row = prod(data->shape, axis + 1, rank);
                total = a.row;
            }
        } else if (rank == 1) {
            mode = kGScalarF32Fill;
        } else if (rank == 2 && orank == 2) {
            mode = kGScalar2D;
            a.d1 = data->shape[1];
            a.o1 = out->shape[1];
            total = out->shape[0] * out->shape[1];
        } else if (rank == 3) {
            a.d0 = data->shape[0];
            a.d1 = data->shape[1];
            a.d2 = data->shape[2];
            if (axis == 0 && orank == 2) {
                mode = kGScalarI64Flat;  // out[i] = d[g*d1*d2 + i], i < d1*d2
                a.row = a.d1 * a.d2;
                total = a.row;
            } else if (axis == 0 && orank == 3) {
                mode = kGScalar3D0;
                a.o1 = out->shape[1];
                a.o2 = out->shape[2];
                total = out->shape[0] * a.o1 * a.o2;
            } else if (axis == 1) {
                mode = kGScalar3D1;
                total = a.d0 * a.d2;
            } else if (axis == 2) {
                mode = kGScalar3D2;
                total = a.d0 * a.d1;
            }
        }
    }
    if (mode < 0 && irank == 1) {
        const int64_t cnt = indices->shape[0];
        if (data_dtype == 1 && rank == 1) {
            mode = kGListI64;
            a.esz = 8;
            total = cnt;
        } else if (rank == 2) {
            a.d1 = data->shape[1];
            a.cnt = cnt;
            a.esz = 4;
            if (axis == 0) {
                mode = kGList2D0;
                total = cnt * a.d1;
            } else {
                mode = kGList2D1;
                total = data->shape[0] * cnt;
            }
        }
    }
    if (mode < 0) {
        mode = kGModulo;
        a.esz = data_dtype == 1 ? 8 : 4;
        total = a.on;
    }
    a.mode = mode;
    if (total > a.on && mode != kGModulo) return fail(NNC_HIP_EINVAL, name, "output too small");
    if (total <= 0 || a.dn <= 0) return;
    launch(name, gather_k, dim3(grid_for(total, 1)), dim3(256), 0, a, total);
}

void nnc_batchnorm(Tensor* in, Tensor* s, Tensor* b, Tensor* m, Tensor* v, Tensor* out, float eps,
                   int momentum) {
    (void)in; (void)s; (void)b; (void)m; (void)v; (void)out; (void)eps; (void)momentum;
}

}  // extern "C"
