// MaxPool / AvgPool of the nnc ABI (runtime/x86/ops.c:316-461).
//
// One thread per output element, lanes along the output row so stores
// coalesce; each window is read straight from HBM/L2 (a 3x3 s2 window
// re-reads ~2.25x the input, served by L2). The 3x3 / stride 2 / pad 1 max
// pool (ResNet's stem pool) has its own kernels that read each input row of a
// band of output rows once (maxpool3s2_v4_k: 16-byte loads, two outputs per
// lane; maxpool3s2_k: 8-byte loads, for widths not a multiple of 4). Global
// average pooling has its own kernel that stages whole planes through LDS
// with coalesced loads. The window is clamped to the
// input like the reference, scanned in the same h-major order with the same
// comparisons / float additions, so both kernels are bit-exact with it:
//   MaxPool: start at -3.402823e38f, take v when no element was seen yet or
//            v > max (ops.c:372-383); an empty window yields -3.402823e38f.
//   AvgPool: sequential float sum of the in-bounds elements divided by their
//            count (padding excluded, ops.c:442-456); empty window -> 0.
// N and C come from the input and Ho/Wo from the output, as in the reference.
#include "common.h"
#include "mfma_tile.h"

namespace nnc {

struct PoolArgs {
    const float* in;
    float* out;
    int NC, H, W, Ho, Wo, kh, kw, sh, sw, ph, pw;
};

// grid (ceil(Ho*Wo / 256), min(NC, 65535)): blockIdx.y strides over the
// N*C planes, x over the output positions of a plane (32-bit index math).
template <bool MAX>
__global__ void __launch_bounds__(256) pool2d_k(PoolArgs a) {
    const int hw_out = a.Ho * a.Wo;
    const int pos = blockIdx.x * 256 + threadIdx.x;
    if (pos >= hw_out) return;
    const int oh = pos / a.Wo, ow = pos - oh * a.Wo;
    int h0 = oh * a.sh - a.ph, h1 = h0 + a.kh;
    int w0 = ow * a.sw - a.pw, w1 = w0 + a.kw;
    if (h0 < 0) h0 = 0;
    if (w0 < 0) w0 = 0;
    if (h1 > a.H) h1 = a.H;
    if (w1 > a.W) w1 = a.W;
    for (int nc = blockIdx.y; nc < a.NC; nc += gridDim.y) {
        const float* plane = a.in + (int64_t)nc * a.H * a.W;
        float* o = a.out + (int64_t)nc * hw_out + pos;
        if (MAX) {
            float best = -3.402823e38f;
            bool seen = false;
            for (int h = h0; h < h1; ++h)
                for (int w = w0; w < w1; ++w) {
                    const float v = plane[h * a.W + w];
                    if (!seen || v > best) {
                        best = v;
                        seen = true;
                    }
                }
            *o = best;
        } else {
            float acc = 0.0f;
            int cnt = 0;
            for (int h = h0; h < h1; ++h)
                for (int w = w0; w < w1; ++w) {
                    acc += plane[h * a.W + w];
                    ++cnt;
                }
            *o = cnt > 0 ? acc / (float)cnt : 0.0f;
        }
    }
}

// Global average pool (window = whole plane, one output per plane): the
// workgroup's `planes` consecutive planes (at most 64) are one contiguous
// block, read with coalesced loads (16-byte when aligned) into LDS rows
// padded by one float; then thread t sums plane t sequentially in the
// reference's h-major order (bit-exact).
__global__ void __launch_bounds__(256) global_avgpool_k(const float* __restrict__ in, float* __restrict__ out,
                                                        int NC, int HW, int planes_per_wg) {
    extern __shared__ float tile[];
    const int p0 = blockIdx.x * planes_per_wg;
    const int planes = min(planes_per_wg, NC - p0);
    const int n = planes * HW;
    const float* src = in + (int64_t)p0 * HW;
    const int ld = HW + 1;
    int done = 0;
    if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
        const int n4 = n / 4;
        for (int i = threadIdx.x; i < n4; i += 256) {
            const float4 v = reinterpret_cast<const float4*>(src)[i];
            const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int e = 4 * i + q;
                const int pl = e / HW;
                tile[pl * ld + (e - pl * HW)] = vals[q];
            }
        }
        done = n4 * 4;
    }
    for (int e = done + threadIdx.x; e < n; e += 256) {
        const int pl = e / HW;
        tile[pl * ld + (e - pl * HW)] = src[e];
    }
    __syncthreads();
    if (threadIdx.x < planes) {
        const float* row = tile + threadIdx.x * ld;
        float acc = 0.0f;
        for (int i = 0; i < HW; ++i) acc += row[i];
        out[p0 + threadIdx.x] = acc / (float)HW;
    }
}

// One workgroup per plane (grid.x strides over planes) when the plane fits
// in LDS: the plane is read once from HBM with coalesced loads (16-byte when
// aligned), then every window is evaluated from LDS in the same order and
// with the same comparisons / additions as pool2d_k (bit-exact). Removes the
// 2.25x window re-reads of the direct kernel.
template <bool MAX>
__global__ void __launch_bounds__(256) pool2d_lds_k(PoolArgs a) {
    extern __shared__ float plane_s[];
    const int hw = a.H * a.W, hw_out = a.Ho * a.Wo;
    for (int nc = blockIdx.x; nc < a.NC; nc += gridDim.x) {
        const float* src = a.in + (int64_t)nc * hw;
        int done = 0;
        if ((reinterpret_cast<uintptr_t>(src) & 15) == 0) {
            const int n4 = hw / 4;
            for (int i = threadIdx.x; i < n4; i += 256)
                reinterpret_cast<float4*>(plane_s)[i] = reinterpret_cast<const float4*>(src)[i];
            done = n4 * 4;
        }
        for (int i = done + threadIdx.x; i < hw; i += 256) plane_s[i] = src[i];
        __syncthreads();
        float* dst = a.out + (int64_t)nc * hw_out;
        for (int pos = threadIdx.x; pos < hw_out; pos += 256) {
            const int oh = pos / a.Wo, ow = pos - oh * a.Wo;
            int h0 = oh * a.sh - a.ph, h1 = h0 + a.kh;
            int w0 = ow * a.sw - a.pw, w1 = w0 + a.kw;
            if (h0 < 0) h0 = 0;
            if (w0 < 0) w0 = 0;
            if (h1 > a.H) h1 = a.H;
            if (w1 > a.W) w1 = a.W;
            if (MAX) {
                float best = -3.402823e38f;
                bool seen = false;
                for (int h = h0; h < h1; ++h)
                    for (int w = w0; w < w1; ++w) {
                        const float v = plane_s[h * a.W + w];
                        if (!seen || v > best) {
                            best = v;
                            seen = true;
                        }
                    }
                dst[pos] = best;
            } else {
                float acc = 0.0f;
                int cnt = 0;
                for (int h = h0; h < h1; ++h)
                    for (int w = w0; w < w1; ++w) {
                        acc += plane_s[h * a.W + w];
                        ++cnt;
                    }
                dst[pos] = cnt > 0 ? acc / (float)cnt : 0.0f;
            }
        }
        __syncthreads();
    }
}

// 3x3 stride-2 max pooling with one row and one column of padding (the
// ResNet stem's pool), straight from HBM: one wave per (plane, band of R
// output rows, 64 output columns). Lane l owns output column ow = ow0 + l
// and loads input columns 2ow and 2ow+1 of every input row of the band as
// one 8-byte load; column 2ow-1 is its left neighbour's second element (a
// lane shuffle; lane 0 of a later chunk loads it itself). All 2R+1 rows of
// the band are loaded up front (the row two vertically adjacent windows
// share stays in registers), so the input is read once plus one halo row
// per band. Each window is scanned in the reference's order - rows top to
// bottom, columns left to right, the first in-bounds element taken, then
// strict > - so the result is bit-exact with pool2d_k. Needs an even W and
// an input below 2 GiB (buffer offsets), checked by the caller.
template <int R>
__global__ void __launch_bounds__(256) maxpool3s2_k(PoolArgs a, int nbands, int nchunks) {
    const int lane = threadIdx.x & 63;
    const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int chunk = wid % nchunks;
    const int rest = wid / nchunks;
    const int band = rest % nbands;
    const int nc = rest / nbands;
    if (nc >= a.NC) return;  // wave-uniform
    const int ow = chunk * 64 + lane;
    const int oh0 = band * R;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.in);
    // in-bounds columns of this lane's window: 2ow-1, 2ow, 2ow+1 (W even:
    // 2ow < W implies 2ow+1 < W)
    const bool c0 = ow >= 1 && 2 * ow - 1 < a.W;
    const bool c1 = 2 * ow < a.W;
    const int hbase = 2 * oh0 - 1;
    float x0[2 * R + 1], x1[2 * R + 1], x2[2 * R + 1];
#pragma unroll
    for (int i = 0; i < 2 * R + 1; ++i) {
        const int h = hbase + i;
        const bool row_in = h >= 0 && h < a.H;
        const uint32_t rowoff = row_in ? (uint32_t)((nc * a.H + h) * a.W) * 4u : 0u;
        const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, (int)(row_in && c1 ? rowoff + (uint32_t)ow * 8u : kOutOfRange),
                                                            0, 0);
        // element copies first: bit_cast of an ext-vector element is miscompiled
        const uint32_t lo = v[0], hi = v[1];
        x1[i] = __uint_as_float(lo);
        x2[i] = __uint_as_float(hi);
        float left = __shfl_up(x2[i], 1);
        if (lane == 0 && c0)
            left = load_f32(rs, row_in ? rowoff + (uint32_t)(2 * ow - 1) * 4u : kOutOfRange);
        x0[i] = left;
    }
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int oh = oh0 + j;
        if (oh >= a.Ho) break;
        float best = -3.402823e38f;
        bool seen = false;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int h = hbase + 2 * j + r;
            if (h < 0 || h >= a.H) continue;
            const float v3[3] = {x0[2 * j + r], x1[2 * j + r], x2[2 * j + r]};
            const bool ok3[3] = {c0, c1, c1};
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                if (ok3[c] && (!seen || v3[c] > best)) {
                    best = v3[c];
                    seen = true;
                }
            }
        }
        if (ow < a.Wo) a.out[((int64_t)nc * a.Ho + oh) * a.Wo + ow] = best;
    }
}

// The same pool with 16-byte loads (W % 4 == 0, 16-byte aligned rows): lane
// l of a segment owns the output column pair 2p, 2p + 1 (p = chunk * LPS +
// l) and loads input columns 4p .. 4p + 3 of each row of its band as one
// 16-byte load; column 4p - 1 is its left neighbour's last element (lane 0
// of a segment loads it itself). A wave holds 64 / LPS segments of LPS
// lanes (LPS = 16, 32 or 64, the smallest that covers a row's pairs), each
// its own (plane, band, chunk): narrow rows do not leave lanes idle. Same
// scan order and comparisons as maxpool3s2_k - bit-exact. Outputs leave as
// 8-byte stores.
template <int R>
__global__ void __launch_bounds__(256) maxpool3s2_v4_k(PoolArgs a, int nbands, int nchunks, int lps_log2,
                                                     int64_t items) {
    const int lane = threadIdx.x & 63;
    const int lps = 1 << lps_log2;
    const int seg = lane >> lps_log2, l = lane & (lps - 1);
    const int64_t item = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * (64 >> lps_log2) + seg;
    if (item >= items) return;  // uniform over a segment; the shuffles stay inside it
    const int chunk = (int)(item % nchunks);
    const int64_t rest = item / nchunks;
    const int band = (int)(rest % nbands);
    const int nc = (int)(rest / nbands);
    const int pr = chunk * lps + l;    // this lane's column pair
    const int pairs = a.Wo >> 1;       // Wo == W / 2, W % 4 == 0
    const bool active = pr < pairs;
    const int oh0 = band * R;
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(a.in);
    const bool cleft = active && pr >= 1;  // column 4p - 1 inside the image
    const int hbase = 2 * oh0 - 1;
    float xl[2 * R + 1], x[2 * R + 1][4];
#pragma unroll
    for (int i = 0; i < 2 * R + 1; ++i) {
        const int h = hbase + i;
        const bool row_in = h >= 0 && h < a.H;
        const uint32_t rowoff = row_in ? (uint32_t)((nc * a.H + h) * a.W) * 4u : 0u;
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(
            rs, (int)(row_in && active ? rowoff + (uint32_t)pr * 16u : kOutOfRange), 0, 0);
        // element copies first: bit_cast of an ext-vector element is miscompiled
        const uint32_t e0 = v[0], e1 = v[1], e2 = v[2], e3 = v[3];
        x[i][0] = __uint_as_float(e0);
        x[i][1] = __uint_as_float(e1);
        x[i][2] = __uint_as_float(e2);
        x[i][3] = __uint_as_float(e3);
        float left = __shfl_up(x[i][3], 1, lps);
        if (l == 0 && cleft) left = load_f32(rs, row_in ? rowoff + (uint32_t)(4 * pr - 1) * 4u : kOutOfRange);
        xl[i] = left;
    }
    if (!active) return;
#pragma unroll
    for (int j = 0; j < R; ++j) {
        const int oh = oh0 + j;
        if (oh >= a.Ho) break;
        float best0 = -3.402823e38f, best1 = -3.402823e38f;
        bool seen0 = false, seen1 = false;
#pragma unroll
        for (int r = 0; r < 3; ++r) {
            const int h = hbase + 2 * j + r;
            if (h < 0 || h >= a.H) continue;
            const float* xr = x[2 * j + r];
            // output 2p: columns 4p - 1, 4p, 4p + 1
            const float w0[3] = {xl[2 * j + r], xr[0], xr[1]};
            const bool ok0[3] = {cleft, true, true};
#pragma unroll
            for (int c = 0; c < 3; ++c)
                if (ok0[c] && (!seen0 || w0[c] > best0)) {
                    best0 = w0[c];
                    seen0 = true;
                }
            // output 2p + 1: columns 4p + 1, 4p + 2, 4p + 3
#pragma unroll
            for (int c = 1; c < 4; ++c)
                if (!seen1 || xr[c] > best1) {
                    best1 = xr[c];
                    seen1 = true;
                }
        }
        float2* o = reinterpret_cast<float2*>(a.out + ((int64_t)nc * a.Ho + oh) * a.Wo) + pr;
        *o = make_float2(best0, best1);
    }
}

template <int R>
static void maxpool3s2_launch(const char* name, const PoolArgs& a, int64_t nc, int nchunks) {
    const int nbands = (int)ceil_div(a.Ho, R);
    const int64_t waves = nc * nbands * nchunks;
    launch(name, maxpool3s2_k<R>, dim3((unsigned)ceil_div(waves, 4)), dim3(256), 0, a, nbands, nchunks);
}

__global__ void fill_value_k(float* out, int64_t n, float v) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) out[i] = v;
}

template <bool MAX>
static void pool_entry(const char* name, Tensor* in, Tensor* out, int kh, int kw, int sh, int sw,
                       int ph, int pw) {
    if (!ready(name)) return;
    // the reference returns silently on these (ops.c:329-334)
    if (!in || !out || !in->data || !out->data || in->ndim != 4 || out->ndim != 4) return;
    PoolArgs a{};
    a.in = (const float*)in->data;
    a.out = (float*)out->data;
    const int64_t nc = in->shape[0] * in->shape[1];
    a.H = (int)in->shape[2];
    a.W = (int)in->shape[3];
    a.Ho = (int)out->shape[2];
    a.Wo = (int)out->shape[3];
    a.kh = kh;
    a.kw = kw;
    a.sh = sh;
    a.sw = sw;
    a.ph = ph;
    a.pw = pw;
    if (nc * a.Ho * a.Wo > numel(out)) return fail(NNC_HIP_EINVAL, name, "output smaller than N*C*Ho*Wo");
    if (nc >= (1 << 30)) return fail(NNC_HIP_EUNSUPP, name, "too many planes");
    a.NC = (int)nc;
    if (MAX && numel(out) > nc * a.Ho * a.Wo) {
        // the reference pre-fills the whole output (ops.c:345-348)
        launch(name, fill_value_k, dim3(grid_for(numel(out), 1)), dim3(256), 0, a.out, numel(out),
               -3.402823e38f);
    }
    set_work(0.0, 4.0 * ((double)numel(in) + (double)nc * a.Ho * a.Wo));
    const int64_t hw = (int64_t)a.H * a.W;
    if (!MAX && a.Ho == 1 && a.Wo == 1 && kh >= a.H && kw >= a.W && ph == 0 && pw == 0 && hw > 0 &&
        hw <= 4096) {
        // global pool: every output is the mean of one whole plane; as many
        // planes per workgroup as fit 64 KB of LDS (at most 64)
        int planes = (int)(16384 / (hw + 1));
        planes = planes < 1 ? 1 : (planes > 64 ? 64 : planes);
        const size_t lds = (size_t)planes * (hw + 1) * sizeof(float);
        launch("nnc_avgpool2d_global", global_avgpool_k, dim3((unsigned)ceil_div(nc, planes)), dim3(256), lds,
               a.in, a.out, a.NC, (int)hw, planes);
        return;
    }
    if ((int64_t)a.Ho * a.Wo >= (1 << 30)) return fail(NNC_HIP_EUNSUPP, name, "output plane too large");
    if (MAX && kh == 3 && kw == 3 && sh == 2 && sw == 2 && ph == 1 && pw == 1 && a.W % 2 == 0 && a.H > 0 &&
        a.Ho > 0 && a.Wo > 0 && nc > 0 && numel(in) * 4 < ((int64_t)1 << 31)) {
        // 8 output rows per wave, fewer where that leaves the GPU short of
        // waves (ResNet-18 stem pool: batch 1 448 waves -> 2 rows, 11.9 ->
        // 6.2 us; batch 8 3584 waves -> 4 rows, 13.4 -> 10.3 us)
        if (a.W % 4 == 0 && a.Wo * 2 == a.W && aligned16(a.in) && aligned16(a.out)) {
            // 16-byte loads; bands of 2 output rows, 1 where 2 leave fewer
            // than 2048 waves (ResNet-18 stem pool on MI355X: batch 32 27.0 ->
            // 23.8 us, batch 8 8.1 -> 6.2 us, batch 1 3.5 -> 3.0 us against
            // maxpool3s2_k; bands of 3, 4 and 8 rows measured slower)
            const int pairs = a.Wo / 2;
            const int lps_log2 = pairs <= 16 ? 4 : (pairs <= 32 ? 5 : 6);
            const int nchunks = (int)ceil_div(pairs, 1 << lps_log2);
            const int64_t items2 = nc * ceil_div(a.Ho, 2) * nchunks;
            const bool one = ceil_div(items2, 64 >> lps_log2) < 2048;
            const int nbands = (int)ceil_div(a.Ho, one ? 1 : 2);
            const int64_t items = nc * nbands * nchunks;
            const int64_t waves = ceil_div(items, 64 >> lps_log2);
            if (waves < ((int64_t)1 << 30)) {
                const dim3 grid((unsigned)ceil_div(waves, 4));
                if (one) return launch(name, maxpool3s2_v4_k<1>, grid, dim3(256), 0, a, nbands, nchunks, lps_log2, items);
                return launch(name, maxpool3s2_v4_k<2>, grid, dim3(256), 0, a, nbands, nchunks, lps_log2, items);
            }
        }
        const int nchunks = (int)ceil_div(a.Wo, 64);
        const int64_t waves8 = nc * ceil_div(a.Ho, 8) * nchunks;
        if (waves8 < ((int64_t)1 << 28)) {
            if (waves8 < 1024) return maxpool3s2_launch<2>(name, a, nc, nchunks);
            if (waves8 < 4096) return maxpool3s2_launch<4>(name, a, nc, nchunks);
            return maxpool3s2_launch<8>(name, a, nc, nchunks);
        }
    }
    if (hw <= 16384 && hw > 0 && a.Ho > 0 && a.Wo > 0 && nc > 0) {
        // whole plane in LDS (at most 64 KB): the input is read once
        const int64_t cap = (int64_t)cu_count() * 8;
        const unsigned grid = (unsigned)(nc < cap ? nc : cap);
        launch(name, pool2d_lds_k<MAX>, dim3(grid), dim3(256), (size_t)hw * sizeof(float), a);
        return;
    }
    const unsigned gy = (unsigned)(nc < 65535 ? nc : 65535);
    if (nc > 0 && a.Ho > 0 && a.Wo > 0)
        launch(name, pool2d_k<MAX>, dim3((unsigned)ceil_div((int64_t)a.Ho * a.Wo, 256), gy), dim3(256), 0, a);
}

// ---------------------------------------------------------------------------
// Global average pool streamed into the classifier GEMM (nnc_hip_gap_gemm_nt)
// ---------------------------------------------------------------------------
// out[n][o] = alpha * sum_c mean[n][c] * w[o][c] + beta * c_o, with mean the
// global average pool of in[n] - the reference's nnc_avgpool2d over the whole
// plane followed by nnc_gemm_nt on the flattened [N, C] result (ops.c:393-461,
// 1843-1886) - without the pooled tensor ever leaving the workgroup.
//
// Built for small batches, where the two reference ops are two launches of
// little work each and the time goes to memory round trips: every load of a
// workgroup is issued before it waits for any. Grid (ceil(O / 16), N), 256
// threads: a workgroup takes one image and 16 classes. Wave q first loads
// its 4 rows of w into registers (lane l: channels l, l + 64, ...; coalesced
// along c), then the whole workgroup copies the image's planes into LDS
// (coalesced, rows padded by one float) - both in flight together. Thread t
// sums planes t, t + 256, ... sequentially in the reference's h-major order
// and divides by H*W: the reference's float means, bit for bit. Each row's
// dot product: exact float products summed in double per lane, the 64 lane
// sums by a shuffle tree, times alpha, plus beta * c, rounded once to float.
// The reference adds the same exact products in one sequential double chain:
// another order of double additions, below float rounding almost always.
static constexpr int GG_OT = 16, GG_ROWS = GG_OT / 4;
static constexpr int GG_F4 = 4;   // float4 of a row per lane: C <= 1024
static constexpr int GG_U = 28;   // float4 of the image per thread in flight at once

__device__ __forceinline__ double wave_sum_f64(double v) {
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d);
    return v;
}

// Needs C % 4 == 0 and 16-byte aligned x and w (checked on the host).
__global__ void __launch_bounds__(256) gap_gemm_nt_k(const float* __restrict__ x, const float* __restrict__ w,
                                                     const float* __restrict__ cv, float* __restrict__ out, int C,
                                                     int HW, int O, int c_mode, float alpha, float beta) {
    extern __shared__ float sm[];
    float* mean = sm;        // C floats
    float* stage = sm + C;   // C planes of HW + 1 floats
    const int n = blockIdx.y;
    const int tid = threadIdx.x, q = tid >> 6, lane = tid & 63;
    const int o0 = blockIdx.x * GG_OT + q * GG_ROWS;
    // this wave's rows of w: lane l holds channels 4l .. 4l + 3 (+ 256 m)
    float4 wr[GG_ROWS][GG_F4];
#pragma unroll
    for (int r = 0; r < GG_ROWS; ++r)
#pragma unroll
        for (int m = 0; m < GG_F4; ++m) {
            const int c = 4 * lane + 256 * m;
            wr[r][m] = (o0 + r < O && c < C) ? *reinterpret_cast<const float4*>(w + (int64_t)(o0 + r) * C + c)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    // the image's planes into LDS, GG_U float4 per thread in flight
    const int ld = HW + 1;
    const float4* img = reinterpret_cast<const float4*>(x + (int64_t)n * C * HW);
    const int run4 = C * HW / 4;
    for (int base = tid; base < run4; base += 256 * GG_U) {
        float4 v[GG_U];
#pragma unroll
        for (int u = 0; u < GG_U; ++u) {
            const int i = base + 256 * u;
            v[u] = i < run4 ? img[i] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < GG_U; ++u) {
            const int i = base + 256 * u;
            if (i >= run4) break;
            const float e4[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int e = 4 * i + j, pl = e / HW;
                stage[pl * ld + (e - pl * HW)] = e4[j];
            }
        }
    }
    __syncthreads();
    for (int pl = tid; pl < C; pl += 256) {
        const float* plane = stage + pl * ld;
        float acc = 0.0f;
        for (int k = 0; k < HW; ++k) acc += plane[k];
        mean[pl] = acc / (float)HW;
    }
    __syncthreads();
    double mv[GG_F4][4];
#pragma unroll
    for (int m = 0; m < GG_F4; ++m)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int c = 4 * lane + 256 * m + j;
            mv[m][j] = c < C ? (double)mean[c] : 0.0;
        }
#pragma unroll
    for (int r = 0; r < GG_ROWS; ++r) {
        double acc = 0.0;
#pragma unroll
        for (int m = 0; m < GG_F4; ++m)
            acc += mv[m][0] * (double)wr[r][m].x + mv[m][1] * (double)wr[r][m].y + mv[m][2] * (double)wr[r][m].z +
                   mv[m][3] * (double)wr[r][m].w;
        acc = wave_sum_f64(acc);
        const int o = o0 + r;
        if (lane == 0 && o < O) {
            acc *= (double)alpha;
            if (c_mode == 1) acc += (double)beta * (double)cv[o];
            else if (c_mode == 2) acc += (double)beta * (double)cv[(int64_t)n * O + o];
            out[(int64_t)n * O + o] = (float)acc;
        }
    }
}

}  // namespace nnc

using namespace nnc;

extern "C" {

void nnc_maxpool2d(Tensor* in, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    pool_entry<true>("nnc_maxpool2d", in, out, kh, kw, sh, sw, ph, pw);
}

void nnc_avgpool2d(Tensor* in, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    pool_entry<false>("nnc_avgpool2d", in, out, kh, kw, sh, sw, ph, pw);
}

// No reference counterpart: GlobalAveragePool -> Flatten -> Gemm (transB) as
// one kernel, emitted by the mi355x target at O3 when the pooled tensor only
// feeds the classifier. in [N][C][H][W], w [O][C], c [O] or [N][O] or NULL,
// out [N][O]; nnc_avgpool2d over the whole plane followed by
// nnc_gemm_nt(pooled as [N, C], w, c, out, alpha, beta), the double sums of
// the second in another fixed order (gap_gemm_nt_k).
void nnc_hip_gap_gemm_nt(Tensor* in, Tensor* w, Tensor* c, Tensor* out, float alpha, float beta) {
    const char* name = "nnc_hip_gap_gemm_nt";
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(w) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    if (in->ndim != 4 || w->ndim != 2) return fail(NNC_HIP_EINVAL, name, "expected in [N][C][H][W] and w [O][C]");
    const int64_t N = in->shape[0], C = in->shape[1], HW = in->shape[2] * in->shape[3], O = w->shape[0];
    if (w->shape[1] != C) return fail(NNC_HIP_EINVAL, name, "w has %lld columns for %lld channels",
                                      (long long)w->shape[1], (long long)C);
    if (numel(out) < N * O) return fail(NNC_HIP_EINVAL, name, "output smaller than N x O");
    int c_mode = 0;
    if (c && c->data) {
        if (numel(c) == O && c->ndim == 1) c_mode = 1;
        else if (numel(c) >= N * O) c_mode = 2;
        else return fail(NNC_HIP_EINVAL, name, "c is neither [O] nor [N][O]");
    }
    if (N == 0 || O == 0) return;
    // the means and every plane of one image in LDS (at most 128 KB); the rows
    // of w in registers, GG_F4 float4 per lane (C <= 1024)
    const int64_t lds_floats = C + C * (HW + 1);
    if (HW <= 0 || C <= 0 || C % 4 || C > 256 * GG_F4 || lds_floats > 32768 || N > 65535 ||
        !aligned16(in->data) || !aligned16(w->data))
        return fail(NNC_HIP_EUNSUPP, name, "needs C %% 4 == 0, C <= %d, C * (H*W + 2) floats <= 128 KB, aligned data",
                    256 * GG_F4);
    const size_t lds = (size_t)lds_floats * sizeof(float);
    // more than 64 KB of dynamic LDS needs the attribute (once, thread-safe)
    static const bool big_lds = hipFuncSetAttribute((const void*)gap_gemm_nt_k,
                                                    hipFuncAttributeMaxDynamicSharedMemorySize, 32768 * 4) ==
                                hipSuccess;
    if (!big_lds && lds > 65536) return fail(NNC_HIP_EDEVICE, name, "hipFuncSetAttribute failed");
    set_work(2.0 * N * O * C, 4.0 * (double)(N * C * HW + O * C + N * O + (c_mode ? O : 0)));
    launch(name, gap_gemm_nt_k, dim3((unsigned)ceil_div(O, GG_OT), (unsigned)N), dim3(256), lds,
           (const float*)in->data, (const float*)w->data, c_mode ? (const float*)c->data : nullptr, (float*)out->data,
           (int)C, (int)HW, (int)O, c_mode, alpha, beta);
}

}  // extern "C"
