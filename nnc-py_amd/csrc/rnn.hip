// LSTM of the nnc ABI (runtime/x86/ops.c:2918-3116).
//
// The reference runs one (h, c) state through every batch element of a time
// step in order (the state is not per batch element) and writes
// Y[t][dir][b][:] = h after each element. That recurrence is sequential, so
// one workgroup walks it: per step each thread computes whole gate rows (the
// four gate dot products over x_t and h, summed in the reference's order:
// W.x, then R.h, then Wb + Rb), the new (h, c) are staged in LDS and
// published after a barrier. Gate order I, O, F, C; sigmoid / tanh as in the
// reference. Not on the ResNet/Transformer hot path; latency-bound.
#include <math.h>

#include "common.h"

namespace nnc {

struct LstmArgs {
    const float* X;
    const float* W;
    const float* R;
    const float* B;
    float* Y;
    float* Yh;
    float* Yc;
    int T, Bt, in_sz, hid, dirs;
};

__device__ __forceinline__ float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

__global__ void __launch_bounds__(256) lstm_k(LstmArgs a) {
    extern __shared__ float st[];
    float* h = st;
    float* c = st + a.hid;
    float* hn = st + 2 * a.hid;
    float* cn = st + 3 * a.hid;
    for (int dir = 0; dir < a.dirs; ++dir) {
        for (int i = threadIdx.x; i < a.hid; i += blockDim.x) h[i] = c[i] = 0.f;
        __syncthreads();
        const float* Wd = a.W + (int64_t)dir * 4 * a.hid * a.in_sz;
        const float* Rd = a.R + (int64_t)dir * 4 * a.hid * a.hid;
        const float* Bd = a.B ? a.B + (int64_t)dir * 8 * a.hid : nullptr;
        for (int t = 0; t < a.T; ++t) {
            const int ts = dir == 1 ? a.T - 1 - t : t;
            for (int b = 0; b < a.Bt; ++b) {
                const float* xt = a.X + ((int64_t)ts * a.Bt + b) * a.in_sz;
                for (int i = threadIdx.x; i < a.hid; i += blockDim.x) {
                    float gate[4];
                    for (int q = 0; q < 4; ++q) {
                        const float* wr = Wd + ((int64_t)q * a.hid + i) * a.in_sz;
                        const float* rr = Rd + ((int64_t)q * a.hid + i) * a.hid;
                        float g = 0.f;
                        for (int j = 0; j < a.in_sz; ++j) g += wr[j] * xt[j];
                        for (int j = 0; j < a.hid; ++j) g += rr[j] * h[j];
                        if (Bd) g += Bd[q * a.hid + i] + Bd[(4 + q) * a.hid + i];
                        gate[q] = g;
                    }
                    const float ig = sigm(gate[0]), og = sigm(gate[1]), fg = sigm(gate[2]);
                    const float gg = tanhf(gate[3]);
                    const float cv = fg * c[i] + ig * gg;
                    cn[i] = cv;
                    hn[i] = og * tanhf(cv);
                }
                __syncthreads();
                float* yt = a.Y + (((int64_t)t * a.dirs + dir) * a.Bt + b) * a.hid;
                for (int i = threadIdx.x; i < a.hid; i += blockDim.x) {
                    h[i] = hn[i];
                    c[i] = cn[i];
                    yt[i] = hn[i];
                }
                __syncthreads();
            }
        }
        for (int b = 0; b < a.Bt; ++b)
            for (int i = threadIdx.x; i < a.hid; i += blockDim.x) {
                a.Yh[((int64_t)dir * a.Bt + b) * a.hid + i] = h[i];
                a.Yc[((int64_t)dir * a.Bt + b) * a.hid + i] = c[i];
            }
        __syncthreads();
    }
}

}  // namespace nnc

using namespace nnc;

extern "C" void nnc_lstm(Tensor* X, Tensor* W, Tensor* R, Tensor* B, Tensor* Y, Tensor* Yh, Tensor* Yc,
                         int direction, int hidden) {
    const char* name = "nnc_lstm";
    if (!ready(name)) return;
    if (!has_data(X) || !has_data(W) || !has_data(R) || !has_data(Y) || !has_data(Yh) || !has_data(Yc))
        return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    if (X->ndim != 3 || hidden <= 0 || hidden > 4096) return fail(NNC_HIP_EINVAL, name, "bad shape");
    LstmArgs a{};
    a.X = (const float*)X->data;
    a.W = (const float*)W->data;
    a.R = (const float*)R->data;
    a.B = (B && B->data) ? (const float*)B->data : nullptr;
    a.Y = (float*)Y->data;
    a.Yh = (float*)Yh->data;
    a.Yc = (float*)Yc->data;
    a.T = (int)X->shape[0];
    a.Bt = (int)X->shape[1];
    a.in_sz = (int)X->shape[2];
    a.hid = hidden;
    a.dirs = direction == 2 ? 2 : 1;
    const int64_t need_w = (int64_t)a.dirs * 4 * hidden * a.in_sz, need_r = (int64_t)a.dirs * 4 * hidden * hidden;
    if (numel(W) < need_w || numel(R) < need_r || (a.B && numel(B) < (int64_t)a.dirs * 8 * hidden) ||
        numel(Y) < (int64_t)a.T * a.dirs * a.Bt * hidden || numel(Yh) < (int64_t)a.dirs * a.Bt * hidden ||
        numel(Yc) < (int64_t)a.dirs * a.Bt * hidden)
        return fail(NNC_HIP_EINVAL, name, "tensor smaller than the LSTM shapes");
    launch(name, lstm_k, dim3(1), dim3(256), (size_t)4 * hidden * sizeof(float), a);
}
