// MaxPool / AvgPool of the nnc ABI (runtime/x86/ops.c:316-461).
//
// One thread per output element, lanes along the output row so stores
// coalesce; each window is read straight from HBM/L2 (a 3x3 s2 window
// re-reads ~2.25x the input, served by L2). The window is clamped to the
// input like the reference, scanned in the same h-major order with the same
// comparisons / float additions, so both kernels are bit-exact with it:
//   MaxPool: start at -3.402823e38f, take v when no element was seen yet or
//            v > max (ops.c:372-383); an empty window yields -3.402823e38f.
//   AvgPool: sequential float sum of the in-bounds elements divided by their
//            count (padding excluded, ops.c:442-456); empty window -> 0.
// N and C come from the input and Ho/Wo from the output, as in the reference.
#include "common.h"

namespace nnc {

struct PoolArgs {
    const float* in;
    float* out;
    int NC, H, W, Ho, Wo, kh, kw, sh, sw, ph, pw;
};

template <bool MAX>
__global__ void __launch_bounds__(256) pool2d_k(PoolArgs a) {
    const int64_t total = (int64_t)a.NC * a.Ho * a.Wo;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int ow = (int)(e % a.Wo);
        const int64_t t = e / a.Wo;
        const int oh = (int)(t % a.Ho);
        const int64_t nc = t / a.Ho;
        int h0 = oh * a.sh - a.ph, h1 = h0 + a.kh;
        int w0 = ow * a.sw - a.pw, w1 = w0 + a.kw;
        if (h0 < 0) h0 = 0;
        if (w0 < 0) w0 = 0;
        if (h1 > a.H) h1 = a.H;
        if (w1 > a.W) w1 = a.W;
        const float* plane = a.in + nc * a.H * a.W;
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
            a.out[e] = best;
        } else {
            float acc = 0.0f;
            int cnt = 0;
            for (int h = h0; h < h1; ++h)
                for (int w = w0; w < w1; ++w) {
                    acc += plane[h * a.W + w];
                    ++cnt;
                }
            a.out[e] = cnt > 0 ? acc / (float)cnt : 0.0f;
        }
    }
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
    launch(name, pool2d_k<MAX>, dim3(grid_for(nc * a.Ho * a.Wo, 1)), dim3(256), 0, a);
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

}  // extern "C"
