// Convolution entry points of the nnc ABI as implicit GEMM on fp32 MFMA
// (reference: runtime/x86/ops.c:720-1504 and 3122-3227).
//
// GEMM view of one convolution (NCHW, weights [Co][Ci][kh][kw]):
//   i = output channel co            (M = Co)
//   j = output pixel (n, oh, ow)     (N = batch * Ho * Wo)
//   k = (ci, r, c) weight tap        (K = Ci * kh * kw)
//   A[i][k] = weight[co][k]          row-major, k contiguous
//   B[k][j] = input[n][ci][oh*sh - ph + r][ow*sw - pw + c], 0 outside
// The B tile is gathered straight from the NCHW input (no im2col buffer);
// consecutive lanes take consecutive pixels, so the gathers coalesce along
// the input rows. D's 32x32 MFMA layout puts consecutive pixels in
// consecutive lanes, so the NCHW stores coalesce too. Bias and the fused
// activation are applied in the epilogue.
//
// Padding follows the reference: only the top/left pads are arguments, the
// bottom/right extent comes from the output shape (c_emitter.py:1051-1058).
//
// When Co x pixels gives too few workgroups to fill the 256 CUs (the 14x14
// and 7x7 stages), K is split over workgroups; each writes an fp32 partial
// tile to the workspace and a second kernel sums the partials in a fixed
// order and applies bias + activation (deterministic, no atomics).
#include <math.h>

#include "mfma_tile.h"

namespace nnc {

enum { kActNone = 0, kActRelu = 1, kActSigmoid = 2 };

__device__ __forceinline__ float activate(float v, int act) {
    if (act == kActRelu) return v > 0.0f ? v : 0.0f;
    if (act == kActSigmoid) return 1.0f / (1.0f + expf(-v));
    return v;
}

struct ConvArgs {
    const float* in;
    const float* w;
    const float* bias;
    float* out;
    float* ws;  // split-K partials [split][Co][Npix] or null
    int N, Ci, H, W, Co, Ho, Wo, kh, kw, sh, sw, ph, pw;
    int K, Npix;
    int tiles_m, tiles_n, splits, k_per_split, act;
};

// B operand: gathers input taps for X consecutive output pixels.
// KH/KW > 0 fix the kernel size at compile time (cheap k -> (ci, r, c)).
template <int X, int BK, int LD, int KH, int KW>
struct ConvGather {
    static constexpr int KROWS = 256 / X;
    static constexpr int PER = X * BK / 256;
    static_assert(256 % X == 0 && BK % KROWS == 0, "gather shape");
    const float* img;
    int h0, w0, H, W, K, kw_rt, khw_rt;
    int64_t HW;
    bool valid;
    int xx, kk;
    float v[PER];

    __device__ void init(const ConvArgs& a, int j0) {
        xx = threadIdx.x % X;
        kk = threadIdx.x / X;
        const int pix = j0 + xx;
        valid = pix < a.Npix;
        const int p = valid ? pix : 0;
        const int hw = a.Ho * a.Wo;
        const int n = p / hw;
        const int rem = p - n * hw;
        const int oh = rem / a.Wo;
        const int ow = rem - oh * a.Wo;
        h0 = oh * a.sh - a.ph;
        w0 = ow * a.sw - a.pw;
        H = a.H;
        W = a.W;
        HW = (int64_t)a.H * a.W;
        K = a.K;
        kw_rt = a.kw;
        khw_rt = a.kh * a.kw;
        img = a.in + (int64_t)n * a.Ci * HW;
    }
    __device__ void load(int k0) {
        const int khw = KH > 0 ? KH * KW : khw_rt;
        const int kwid = KW > 0 ? KW : kw_rt;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int k = k0 + kk + p * KROWS;
            const int ci = k / khw;
            const int t = k - ci * khw;
            const int r = t / kwid;
            const int c = t - r * kwid;
            const int h = h0 + r, w = w0 + c;
            float val = 0.f;
            if (valid && k < K && (unsigned)h < (unsigned)H && (unsigned)w < (unsigned)W)
                val = img[ci * HW + (int64_t)h * W + w];
            v[p] = val;
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) S[(kk + p * KROWS) * LD + xx] = v[p];
    }
};

template <class T, int KH, int KW, bool AVEC>
__global__ void __launch_bounds__(256, 2) conv_igemm_k(ConvArgs a) {
    __shared__ float lds[T::LDS_FLOATS];
    float* As = lds;
    float* Bs = lds + T::BK * T::LDA;
    const int total = a.tiles_m * a.tiles_n * a.splits;
    const int lin = xcd_remap(blockIdx.x, total);
    const int mt = lin % a.tiles_m;
    const int rest = lin / a.tiles_m;
    const int nt = rest % a.tiles_n;
    const int s = rest / a.tiles_n;
    const int i0 = mt * T::BM, j0 = nt * T::BN;
    const int kb = s * a.k_per_split;
    const int ke = min(a.K, kb + a.k_per_split);

    typedef typename std::conditional<AVEC, KContigLoader4<T::BM, T::BK, T::LDA>,
                                      KContigLoader<T::BM, T::BK, T::LDA>>::type LA;
    LA la;
    la.init(a.w + (int64_t)i0 * a.K, a.K, a.Co - i0, a.K);
    ConvGather<T::BN, T::BK, T::LDB, KH, KW> lb;
    lb.init(a, j0);

    floatx16 sum[T::TM][T::TN];
    mfma_mainloop<T>(la, lb, kb, ke, As, Bs, sum);

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wi = (wave / T::WN) * T::WAVE_M;
    const int wj = (wave % T::WN) * T::WAVE_N;
    const int hw = a.Ho * a.Wo;
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn) {
        const int pix = j0 + wj + tn * 32 + (lane & 31);
        if (pix >= a.Npix) continue;
        const int n = pix / hw;
        const int p = pix - n * hw;
        float* obase = a.ws ? a.ws + (int64_t)s * a.Co * a.Npix + pix
                            : a.out + (int64_t)n * a.Co * hw + p;
        const int64_t cstride = a.ws ? (int64_t)a.Npix : (int64_t)hw;
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = i0 + wi + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (co >= a.Co) continue;
                float v = sum[tm][tn][r];
                if (!a.ws) v = activate(v + (a.bias ? a.bias[co] : 0.f), a.act);
                obase[co * cstride] = v;
            }
    }
}

// out[n][co][p] = act(bias[co] + sum over splits of ws[s][co][n*hw + p])
__global__ void __launch_bounds__(256) conv_splitk_reduce_k(const float* ws, const float* bias,
                                                            float* out, int splits, int Co, int Npix,
                                                            int hw, int act) {
    const int64_t total = (int64_t)Co * Npix;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const int co = (int)(e / Npix);
        const int pix = (int)(e - (int64_t)co * Npix);
        float v = 0.f;
        for (int s = 0; s < splits; ++s) v += ws[((int64_t)s * Co + co) * Npix + pix];
        v = activate(v + (bias ? bias[co] : 0.f), act);
        const int n = pix / hw;
        const int p = pix - n * hw;
        out[((int64_t)n * Co + co) * hw + p] = v;
    }
}

typedef Tile<128, 128, 32, 2, 2> ConvT128;  // Co >= 128: 2x2 blocks per wave
typedef Tile<64, 128, 32, 1, 4> ConvT64;    // Co == 64: 2x1 blocks per wave
typedef Tile<64, 64, 32, 2, 2> ConvTSmall;  // small problems: 1 block per wave

// Timing-table key of one kernel instance: conv_igemm_<BM>x<BN>_k<kh>x<kw>_<v4|s1>
template <class T, int KH, int KW>
static void launch_conv_t(const ConvArgs& a, bool avec, const char*) {
    const dim3 grid(a.tiles_m * a.tiles_n * a.splits), block(256);
    char name[64];
    if (KH > 0)
        snprintf(name, sizeof name, "conv_igemm_%dx%d_k%dx%d_%s", T::BM, T::BN, KH, KW, avec ? "v4" : "s1");
    else
        snprintf(name, sizeof name, "conv_igemm_%dx%d_kany_%s", T::BM, T::BN, avec ? "v4" : "s1");
    set_work(2.0 * a.Co * (double)a.Npix * a.K, 0.0);
    if (avec)
        launch(name, conv_igemm_k<T, KH, KW, true>, grid, block, 0, a);
    else
        launch(name, conv_igemm_k<T, KH, KW, false>, grid, block, 0, a);
}

template <class T>
static void launch_conv_k(ConvArgs& a, bool avec, const char* name) {
    a.tiles_m = (int)ceil_div(a.Co, T::BM);
    a.tiles_n = (int)ceil_div(a.Npix, T::BN);
    // split K when the tiles alone leave CUs idle
    const int tiles = a.tiles_m * a.tiles_n;
    const int target = 2 * ctx().cu_count;
    int splits = 1;
    if (tiles < target) {
        const int max_by_k = (int)(a.K / (4 * T::BK));
        splits = (int)ceil_div(target, tiles);
        if (splits > max_by_k) splits = max_by_k;
        if (splits > 32) splits = 32;
        if (splits < 1) splits = 1;
    }
    a.ws = nullptr;
    if (splits > 1) {
        size_t need = (size_t)splits * a.Co * a.Npix * sizeof(float);
        float* ws = workspace(need);
        while (!ws && splits > 1) {  // capture in progress: fit what exists
            --splits;
            need = (size_t)splits * a.Co * a.Npix * sizeof(float);
            ws = need <= workspace_capacity() ? workspace(need) : nullptr;
        }
        a.ws = splits > 1 ? ws : nullptr;
    }
    a.splits = splits;
    a.k_per_split = (int)(ceil_div(ceil_div(a.K, splits), T::BK) * T::BK);
    a.splits = (int)ceil_div(a.K, a.k_per_split);
    if (a.splits <= 1) a.ws = nullptr;
    if (a.kh == 1 && a.kw == 1)
        launch_conv_t<T, 1, 1>(a, avec, name);
    else if (a.kh == 3 && a.kw == 3)
        launch_conv_t<T, 3, 3>(a, avec, name);
    else if (a.kh == 7 && a.kw == 7)
        launch_conv_t<T, 7, 7>(a, avec, name);
    else
        launch_conv_t<T, 0, 0>(a, avec, name);
    if (a.ws) {
        const int64_t total = (int64_t)a.Co * a.Npix;
        set_work(0.0, 4.0 * (double)total * (a.splits + 1));
        launch("conv_splitk_reduce", conv_splitk_reduce_k, dim3(grid_for(total, 1)), dim3(256), 0,
               (const float*)a.ws, a.bias, a.out, a.splits, a.Co, a.Npix, a.Ho * a.Wo, a.act);
    }
}

static bool conv_check(Tensor* in, Tensor* w, Tensor* out, const char* name) {
    if (!ready(name)) return false;
    if (!in || !w || !out) {
        fail(NNC_HIP_EINVAL, name, "NULL tensor pointer");
        return false;
    }
    if (!in->data || !w->data || !out->data) {
        fail(NNC_HIP_EINVAL, name, "NULL data pointer");
        return false;
    }
    if (!in->shape || !w->shape || !out->shape) {
        fail(NNC_HIP_EINVAL, name, "NULL shape pointer");
        return false;
    }
    if (in->ndim != 4 || w->ndim != 4 || out->ndim != 4) {
        fail(NNC_HIP_EINVAL, name, "expected 4D tensors");
        return false;
    }
    return true;
}

static void conv_run(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw,
                     int ph, int pw, int act, const char* name) {
    ConvArgs a{};
    a.in = (const float*)in->data;
    a.w = (const float*)w->data;
    a.bias = (b && b->data) ? (const float*)b->data : nullptr;
    a.out = (float*)out->data;
    a.N = (int)in->shape[0];
    a.Ci = (int)in->shape[1];
    a.H = (int)in->shape[2];
    a.W = (int)in->shape[3];
    a.Co = (int)w->shape[0];
    a.Ho = (int)out->shape[2];
    a.Wo = (int)out->shape[3];
    a.kh = kh;
    a.kw = kw;
    a.sh = sh;
    a.sw = sw;
    a.ph = ph;
    a.pw = pw;
    a.act = act;
    if (kh <= 0 || kw <= 0 || sh <= 0 || sw <= 0 || ph < 0 || pw < 0)
        return fail(NNC_HIP_EINVAL, name, "bad kernel/stride/pad");
    // The reference indexes weights with the kernel-size arguments and the
    // output with the input batch and weight channel count; reject shapes for
    // which that would step outside a buffer.
    if (numel(w) < (int64_t)a.Co * a.Ci * kh * kw)
        return fail(NNC_HIP_EINVAL, name, "weight smaller than Co*Ci*kh*kw");
    if (out->shape[0] < a.N || out->shape[1] < a.Co)
        return fail(NNC_HIP_EINVAL, name, "output smaller than N x Co");
    if (a.bias && numel(b) < a.Co) return fail(NNC_HIP_EINVAL, name, "bias smaller than Co");
    const int64_t K = (int64_t)a.Ci * kh * kw;
    const int64_t npix = (int64_t)a.N * a.Ho * a.Wo;
    if (K >= (1 << 30) || npix >= (1 << 30) || numel(in) >= ((int64_t)1 << 31))
        return fail(NNC_HIP_EUNSUPP, name, "tensor too large for 32-bit indexing");
    a.K = (int)K;
    a.Npix = (int)npix;
    if (a.N == 0 || a.Co == 0 || a.Ho <= 0 || a.Wo <= 0) return;
    const bool avec = (a.K % 4 == 0) && aligned16(a.w);
    const int64_t work = (int64_t)a.Co * a.Npix;
    if (a.Co <= 64 && work < 64 * 64 * 512) {
        launch_conv_k<ConvTSmall>(a, avec, name);
    } else if (a.Co <= 64) {
        launch_conv_k<ConvT64>(a, avec, name);
    } else {
        launch_conv_k<ConvT128>(a, avec, name);
    }
}

}  // namespace nnc

using namespace nnc;

extern "C" {

#define NNC_CONV_ENTRY(fname, act)                                                                \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw,      \
               int ph, int pw) {                                                                  \
        if (!conv_check(in, w, out, #fname)) return;                                       \
        conv_run(in, w, b, out, kh, kw, sh, sw, ph, pw, act, #fname);                              \
    }
NNC_CONV_ENTRY(nnc_conv, kActNone)
NNC_CONV_ENTRY(nnc_conv_relu, kActRelu)
NNC_CONV_ENTRY(nnc_conv_sigmoid, kActSigmoid)

#define NNC_CONV1X1_ENTRY(fname, act)                                                              \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int sh, int sw, int ph, int pw) {     \
        if (!conv_check(in, w, out, #fname)) return;                                         \
        conv_run(in, w, b, out, 1, 1, sh, sw, ph, pw, act, #fname);                                 \
    }
NNC_CONV1X1_ENTRY(nnc_conv1x1, kActNone)
NNC_CONV1X1_ENTRY(nnc_conv_relu1x1, kActRelu)

// ops.c:1089-1093: the 3x3 s1 entry requires a same-size output and
// otherwise leaves the output untouched.
#define NNC_CONV3X3_ENTRY(fname, act)                                                  \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {                        \
        if (!conv_check(in, w, out, #fname)) return;                             \
        if (out->shape[2] != in->shape[2] || out->shape[3] != in->shape[3])            \
            return fail(NNC_HIP_EINVAL, #fname, "expected same-padding output shape"); \
        conv_run(in, w, b, out, 3, 3, 1, 1, 1, 1, act, #fname);                         \
    }
NNC_CONV3X3_ENTRY(nnc_conv3x3_s1, kActNone)
NNC_CONV3X3_ENTRY(nnc_conv_relu3x3_s1, kActRelu)

// ops.c:1310-1311, 1403: stride 2 with the pad fixed at 3.
#define NNC_CONV7X7_ENTRY(fname, act)                                   \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {         \
        if (!conv_check(in, w, out, #fname)) return;              \
        conv_run(in, w, b, out, 7, 7, 2, 2, 3, 3, act, #fname);          \
    }
NNC_CONV7X7_ENTRY(nnc_conv7x7_s2, kActNone)
NNC_CONV7X7_ENTRY(nnc_conv_relu7x7_s2, kActRelu)

}  // extern "C"
