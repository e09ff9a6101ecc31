// fp32 MFMA tile engine for gfx950 shared by implicit-GEMM convolution and
// GEMM/MatMul.
//
// One workgroup = 256 threads = 4 wave64s computes a BM x BN tile of
// D[i][j] = sum_k A[i][k] * B[k][j]. The waves form a WM x WN grid; each wave
// owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 blocks, each block one
// v_mfma_f32_32x32x2_f32 accumulator (16 VGPRs per lane).
//
// Operand staging: every BK-deep slice of A and B is read from HBM/L2 into
// registers by a loader, stored into LDS as S[k][x] (x = i for A, j for B,
// rows padded so that both the transposed stores and the MFMA operand reads
// stay bank-conflict-free), and consumed by the MFMAs. The next slice's
// global loads are issued before the current slice's MFMAs so their latency
// overlaps the matrix work.
//
// Accumulation is two-level: the MFMAs of one BK slice accumulate into a
// fresh accumulator which is then added to a running fp32 sum. This keeps the
// longest fp32 rounding chain at BK/2 MFMA steps plus K/BK slice additions
// instead of K/2, which holds the error of K = 4608 contractions well inside
// 1e-4 absolute / 1e-3 relative of the fp64-accumulated reference.
//
// MFMA 32x32x2 f32 operand/result layout (lane l of 64):
//   A operand: A[i = l % 32][k = l / 32]
//   B operand: B[k = l / 32][j = l % 32]
//   D register r: D[i = 8*(r/4) + 4*(l/32) + r%4][j = l % 32]
#pragma once

#include "common.h"

namespace nnc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

template <int BM_, int BN_, int BK_, int WM_, int WN_>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int THREADS = 256;
    static_assert(WM * WN == 4, "four waves per workgroup");
    static constexpr int WAVE_M = BM / WM, WAVE_N = BN / WN;
    static constexpr int TM = WAVE_M / 32, TN = WAVE_N / 32;
    static_assert(TM >= 1 && TN >= 1 && WAVE_M % 32 == 0 && WAVE_N % 32 == 0, "32x32 blocks");
    static_assert(BK % 2 == 0, "k step of 2");
    // LDS row lengths (floats). +1 keeps transposed scalar stores conflict-free.
    static constexpr int LDA = BM + 1, LDB = BN + 1;
    static constexpr int LDS_FLOATS = BK * (LDA + LDB);
};

// ---------------------------------------------------------------------------
// operand loaders: fill S[k][x] for x in [0, X), k in [k0, k0 + BK)
// ---------------------------------------------------------------------------

// element (x, k) at base[x * ld + k]  (row-major A, or B stored [N][K])
template <int X, int BK, int LD>
struct KContigLoader {
    static constexpr int ROWS_PER_PASS = 256 / BK;
    static constexpr int PER = X * BK / 256;
    static_assert(256 % BK == 0 && X % ROWS_PER_PASS == 0, "loader shape");
    const float* base;
    int64_t ld;
    int xlim, K, kk, xx;
    float v[PER];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        base = b;
        ld = ld_;
        xlim = xlim_;
        K = K_;
        kk = threadIdx.x % BK;
        xx = threadIdx.x / BK;
    }
    __device__ void load(int k0) {
        const int k = k0 + kk;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int x = xx + p * ROWS_PER_PASS;
            float t = 0.f;
            if (x < xlim && k < K) t = base[(int64_t)x * ld + k];
            v[p] = t;
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) S[kk * LD + xx + p * ROWS_PER_PASS] = v[p];
    }
};

// As KContigLoader with 16-byte loads; requires ld % 4 == 0, K % 4 == 0 and a
// 16-byte aligned base.
template <int X, int BK, int LD>
struct KContigLoader4 {
    static constexpr int KQ = BK / 4;
    static constexpr int ROWS_PER_PASS = 256 / KQ;
    static constexpr int PER = X * BK / (256 * 4);
    static_assert(BK % 4 == 0 && 256 % KQ == 0 && X % ROWS_PER_PASS == 0 && PER >= 1, "loader4");
    const float* base;
    int64_t ld;
    int xlim, K, kk, xx;
    float4 v[PER];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        base = b;
        ld = ld_;
        xlim = xlim_;
        K = K_;
        kk = (threadIdx.x % KQ) * 4;
        xx = threadIdx.x / KQ;
    }
    __device__ void load(int k0) {
        const int k = k0 + kk;
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int x = xx + p * ROWS_PER_PASS;
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            if (x < xlim && k < K) t = *reinterpret_cast<const float4*>(base + (int64_t)x * ld + k);
            v[p] = t;
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int x = xx + p * ROWS_PER_PASS;
            S[(kk + 0) * LD + x] = v[p].x;
            S[(kk + 1) * LD + x] = v[p].y;
            S[(kk + 2) * LD + x] = v[p].z;
            S[(kk + 3) * LD + x] = v[p].w;
        }
    }
};

// element (x, k) at base[k * ld + x]  (A stored [K][M], or row-major B)
template <int X, int BK, int LD>
struct XContigLoader {
    static constexpr int KROWS_PER_PASS = 256 / X;
    static constexpr int PER = X * BK / 256;
    static_assert(256 % X == 0 && BK % KROWS_PER_PASS == 0, "loader shape");
    const float* base;
    int64_t ld;
    int xlim, K, xx, kk;
    float v[PER];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        base = b;
        ld = ld_;
        xlim = xlim_;
        K = K_;
        xx = threadIdx.x % X;
        kk = threadIdx.x / X;
    }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int k = k0 + kk + p * KROWS_PER_PASS;
            float t = 0.f;
            if (xx < xlim && k < K) t = base[(int64_t)k * ld + xx];
            v[p] = t;
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) S[(kk + p * KROWS_PER_PASS) * LD + xx] = v[p];
    }
};

// 16-byte variant: requires ld % 4 == 0 and a 16-byte aligned base; x bounds
// are checked per element so any xlim works.
template <int X, int BK, int LD>
struct XContigLoader4 {
    static constexpr int XQ = X / 4;
    static constexpr int KROWS_PER_PASS = 256 / XQ;
    static constexpr int PER = X * BK / (256 * 4);
    static_assert(X % 4 == 0 && 256 % XQ == 0 && BK % KROWS_PER_PASS == 0 && PER >= 1, "loader4");
    const float* base;
    int64_t ld;
    int xlim, K, xx, kk;
    float4 v[PER];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        base = b;
        ld = ld_;
        xlim = xlim_;
        K = K_;
        xx = (threadIdx.x % XQ) * 4;
        kk = threadIdx.x / XQ;
    }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            const int k = k0 + kk + p * KROWS_PER_PASS;
            float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k < K) {
                const float* src = base + (int64_t)k * ld + xx;
                if (xx + 3 < xlim) {
                    t = *reinterpret_cast<const float4*>(src);
                } else {
                    if (xx + 0 < xlim) t.x = src[0];
                    if (xx + 1 < xlim) t.y = src[1];
                    if (xx + 2 < xlim) t.z = src[2];
                }
            }
            v[p] = t;
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) {
            float* dst = S + (kk + p * KROWS_PER_PASS) * LD + xx;
            dst[0] = v[p].x;
            dst[1] = v[p].y;
            dst[2] = v[p].z;
            dst[3] = v[p].w;
        }
    }
};

// ---------------------------------------------------------------------------
// main loop over k in [k_begin, k_end): loaders must zero-fill k >= K.
// ---------------------------------------------------------------------------
template <class T, class LA, class LB>
__device__ __forceinline__ void mfma_mainloop(LA& la, LB& lb, int k_begin, int k_end, float* As,
                                              float* Bs, floatx16 (&sum)[T::TM][T::TN]) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wi = (wave / T::WN) * T::WAVE_M;
    const int wj = (wave % T::WN) * T::WAVE_N;
    const int lrow = lane >> 5, lcol = lane & 31;
    const float* Ap = As + lrow * T::LDA + wi + lcol;
    const float* Bp = Bs + lrow * T::LDB + wj + lcol;

#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int r = 0; r < 16; ++r) sum[tm][tn][r] = 0.f;

    if (k_begin >= k_end) return;
    la.load(k_begin);
    lb.load(k_begin);
    la.store(As);
    lb.store(Bs);
    __syncthreads();

    for (int k0 = k_begin; k0 < k_end; k0 += T::BK) {
        const bool more = k0 + T::BK < k_end;
        if (more) {
            la.load(k0 + T::BK);
            lb.load(k0 + T::BK);
        }
        floatx16 acc[T::TM][T::TN];
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[tm][tn][r] = 0.f;
#pragma unroll
        for (int kk = 0; kk < T::BK; kk += 2) {
            float a[T::TM], b[T::TN];
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm) a[tm] = Ap[kk * T::LDA + tm * 32];
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn) b[tn] = Bp[kk * T::LDB + tn * 32];
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < T::TN; ++tn)
                    acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[tm], b[tn], acc[tm][tn], 0, 0, 0);
        }
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn) sum[tm][tn] += acc[tm][tn];
        __syncthreads();
        if (more) {
            la.store(As);
            lb.store(Bs);
        }
        __syncthreads();
    }
}

// Visit every (i, j, value) of the wave's accumulators in tile coordinates.
template <class T, class F>
__device__ __forceinline__ void for_each_acc(const floatx16 (&sum)[T::TM][T::TN], F&& f) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wi = (wave / T::WN) * T::WAVE_M;
    const int wj = (wave % T::WN) * T::WAVE_N;
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = wi + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int j = wj + tn * 32 + (lane & 31);
                f(i, j, sum[tm][tn][r]);
            }
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Remap the launch index so that consecutive logical tiles - which share
// an operand slice - run on the same XCD. Bijective on [0, total).
__device__ __forceinline__ int xcd_remap(int lin, int total) {
    const int per = total / 8;
    if (lin >= per * 8) return lin;
    return (lin % 8) * per + lin / 8;
}

}  // namespace nnc
