// fp32 MFMA tile engine for gfx950 shared by implicit-GEMM convolution and
// GEMM/MatMul.
//
// One workgroup = 256 threads = 4 wave64s computes BM x BN tiles of
// D[i][j] = sum_k A[i][k] * B[k][j]. The waves form a WM x WN grid; each wave
// owns a (BM/WM) x (BN/WN) sub-tile made of 32x32 blocks, each block one
// v_mfma_f32_32x32x2_f32 accumulator (16 VGPRs per lane).
//
// Operand staging: every BK = 32 deep slice of A and B is read from HBM/L2
// into registers by a loader and stored into LDS as S[x][k] (x = i for A, j
// for B), k contiguous, rows padded to 36 floats so 16-byte reads and writes
// of eight consecutive rows hit distinct banks. An MFMA step consumes one k
// per lane half; lane half h takes k = 16h + s at step s, so over the slice
// each lane reads 16 consecutive k of its row: one ds_read_b128 per operand
// block feeds four MFMA steps. Loaders write runs of 4 consecutive k as
// ds_write_b128 where their thread mapping allows. LDS is double-buffered:
// while the MFMAs consume slice t from one buffer, slice t+1's global loads
// are in flight and are then stored to the other buffer, so each slice costs
// one barrier. Loads are raw buffer loads (buffer resource in SGPRs, 32-bit
// byte offsets): an out-of-range element gets an offset past the resource's
// size and the hardware returns 0, so loads need no branch and no select
// afterwards, the loaded registers go straight to LDS and the wait for the
// loads falls after the slice's MFMAs. Byte offsets must stay below 2^31
// (checked on the host).
//
// Scheduling is hybrid stream-K: a persistent grid of G workgroups (at
// most the number resident on the GPU at once). Tiles [0, sk_tiles) form
// the stream-K region: their tiles x (K/BK) slice iterations are split into
// G equal contiguous ranges, one per workgroup. Tiles [sk_tiles, tiles) are
// whole tiles dealt round-robin (tile sk_tiles + g + m*G to workgroup g).
// A workgroup writes tiles it covers completely straight to the output; for
// a tile shared by several workgroups each writes its partial tile to the
// workspace and a fixup kernel adds the partials in workgroup order
// (deterministic) and applies the epilogue. The region sizes keep every CU
// busy to the end whatever the tile count (a tiles-times-splits grid cannot:
// 588 workgroups on 512 slots leave the second round 15% full) while
// splitting no more tiles than needed.
//
// MFMA 32x32x2 f32 operand/result layout (lane l of 64): the instruction
// sums over its two k, one per lane half:
//   A operand: A[i = l % 32][k-half l / 32]
//   B operand: B[k-half l / 32][j = l % 32]
//   D register r: D[i = 8*(r/4) + 4*(l/32) + r%4][j = l % 32]
#pragma once

#include "common.h"
#include "plan.h"

namespace nnc {

typedef float floatx16 __attribute__((ext_vector_type(16)));

// ---------------------------------------------------------------------------
// raw buffer loads. gfx9 buffer resource: base, stride 0, num_records bytes,
// dword3 0x00020000 (32-bit data format). An offset >= num_records reads 0.
// ---------------------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
static constexpr uint32_t kOutOfRange = 0x80000000u;  // any offset >= kRecords
static constexpr int kRecords = 0x7FFFFFFF;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const float* base) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, kRecords, 0x00020000);
}
__device__ __forceinline__ float load_f32(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, (int)byte_off, 0, 0));
}
__device__ __forceinline__ f32x4 load_f32x4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte_off, 0, 0));
}

template <int BM_, int BN_, int BK_, int WM_, int WN_, int NW_ = 4>
struct Tile {
    static constexpr int BM = BM_, BN = BN_, BK = BK_, WM = WM_, WN = WN_;
    static constexpr int NW = NW_;  // waves per workgroup (the staging loaders take 4)
    static constexpr int THREADS = 64 * NW;
    static_assert(WM * WN == NW, "one wave per (WM, WN) cell");
    static constexpr int WAVE_M = BM / WM, WAVE_N = BN / WN;
    static constexpr int TM = WAVE_M / 32, TN = WAVE_N / 32;
    static_assert(TM >= 1 && TN >= 1 && WAVE_M % 32 == 0 && WAVE_N % 32 == 0, "32x32 blocks");
    static_assert(BK == 32, "lane halves take 16 consecutive k each");
    static constexpr int LDK = BK + 4;  // row stride of S[x][k] in floats
    static constexpr int A_FLOATS = BM * LDK, B_FLOATS = BN * LDK;
    static constexpr int STAGE = A_FLOATS + B_FLOATS;  // floats per LDS buffer
    static constexpr int LDS_FLOATS = 2 * STAGE;
    static_assert((BM * BN) % 1024 == 0, "fixup chunks of 256 float4");
};

// four consecutive floats of one LDS row (16-byte aligned)
__device__ __forceinline__ void lds_store4(float* dst, float a, float b, float c, float d) {
    *reinterpret_cast<f32x4*>(dst) = f32x4{a, b, c, d};
}

// ---------------------------------------------------------------------------
// operand loaders: fill S[x][k] (row stride LD) for x in [0, X), k in
// [k0, k0 + BK); elements outside [0, xlim) x [0, K) are zero. `base` is the
// tile origin; every in-range element's byte offset from it is below 2^31.
// ---------------------------------------------------------------------------

// element (x, k) at base[x * ld + k]  (row-major A, or B stored [N][K]);
// lanes along k
template <int X, int BK, int LD>
struct KContigLoader {
    static constexpr int ROWS_PER_PASS = 256 / BK;
    static constexpr int PER = X * BK / 256;
    static_assert(256 % BK == 0 && X % ROWS_PER_PASS == 0, "loader shape");
    __amdgpu_buffer_rsrc_t rsrc;
    int ld, xlim, K, kk, xx;
    float v[PER];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        rsrc = make_rsrc(b);
        ld = (int)ld_;
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
            const bool ok = x < xlim && k < K;
            v[p] = load_f32(rsrc, ok ? (uint32_t)(x * ld + k) * 4u : kOutOfRange);
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) S[(xx + p * ROWS_PER_PASS) * LD + kk] = v[p];
    }
};

// 16-byte loads along k; requires ld % 4 == 0, K % 4 == 0, 16-byte aligned
// base. Each thread's float4 is one 16-byte LDS write.
template <int X, int BK, int LD>
struct KContigLoader4 {
    static constexpr int KQ = BK / 4;
    static constexpr int ROWS_PER_PASS = 256 / KQ;
    static constexpr int PER = X * BK / (256 * 4);
    static_assert(BK % 4 == 0 && 256 % KQ == 0 && X % ROWS_PER_PASS == 0 && PER >= 1, "loader4");
    __amdgpu_buffer_rsrc_t rsrc;
    int ld, xlim, K, kk, xx;
    f32x4 v[PER];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        rsrc = make_rsrc(b);
        ld = (int)ld_;
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
            const bool ok = x < xlim && k < K;
            v[p] = load_f32x4(rsrc, ok ? (uint32_t)(x * ld + k) * 4u : kOutOfRange);
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < PER; ++p) *reinterpret_cast<f32x4*>(S + (xx + p * ROWS_PER_PASS) * LD + kk) = v[p];
    }
};

// element (x, k) at base[k * ld + x]  (A stored [K][M], or row-major B);
// lanes along x, each thread a run of KRUN consecutive k of one x
template <int X, int BK, int LD>
struct XContigLoader {
    static constexpr int KRUN = X * BK / 256;
    static_assert(256 % X == 0 && KRUN % 4 == 0, "loader shape");
    __amdgpu_buffer_rsrc_t rsrc;
    int ld, xlim, K, xx, kbase;
    float v[KRUN];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        rsrc = make_rsrc(b);
        ld = (int)ld_;
        xlim = xlim_;
        K = K_;
        xx = threadIdx.x % X;
        kbase = (threadIdx.x / X) * KRUN;
    }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < KRUN; ++p) {
            const int k = k0 + kbase + p;
            const bool ok = xx < xlim && k < K;
            v[p] = load_f32(rsrc, ok ? (uint32_t)(k * ld + xx) * 4u : kOutOfRange);
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < KRUN; p += 4) lds_store4(S + xx * LD + kbase + p, v[p], v[p + 1], v[p + 2], v[p + 3]);
    }
};

// 16-byte loads along x: requires ld % 4 == 0, xlim % 4 == 0 (so a group of
// four is wholly inside or outside) and a 16-byte aligned base. A thread
// loads a 4 (x) by KRUN (k) block and writes it transposed, one run of KRUN
// floats per x.
template <int X, int BK, int LD>
struct XContigLoader4 {
    static constexpr int XQ = X / 4;
    static constexpr int KG = 256 / XQ;
    static constexpr int KRUN = BK / KG;
    static_assert(X % 4 == 0 && 256 % XQ == 0 && BK % KG == 0 && (KRUN == 2 || KRUN == 4), "loader4");
    __amdgpu_buffer_rsrc_t rsrc;
    int ld, xlim, K, xx, kbase;
    f32x4 v[KRUN];

    __device__ void init(const float* b, int64_t ld_, int xlim_, int K_) {
        rsrc = make_rsrc(b);
        ld = (int)ld_;
        xlim = xlim_;
        K = K_;
        xx = (threadIdx.x % XQ) * 4;
        kbase = (threadIdx.x / XQ) * KRUN;
    }
    __device__ void load(int k0) {
#pragma unroll
        for (int p = 0; p < KRUN; ++p) {
            const int k = k0 + kbase + p;
            const bool ok = xx < xlim && k < K;
            v[p] = load_f32x4(rsrc, ok ? (uint32_t)(k * ld + xx) * 4u : kOutOfRange);
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float* dst = S + (xx + i) * LD + kbase;
            if constexpr (KRUN == 4) {
                lds_store4(dst, v[0][i], v[1][i], v[2][i], v[3][i]);
            } else {
                typedef float f32x2 __attribute__((ext_vector_type(2)));
                *reinterpret_cast<f32x2*>(dst) = f32x2{v[0][i], v[1][i]};
            }
        }
    }
};

// ---------------------------------------------------------------------------
// main loop over k in [k_begin, k_end) (k_begin a multiple of BK); LDS holds
// two stages of T::STAGE floats (A rows, then B rows). TWO_LEVEL adds each
// slice's products into the running sum through a fresh accumulator
// (shorter fp32 rounding chains for very long K); otherwise the MFMAs
// accumulate into `sum` directly.
//
// Per slice (four quads of four k per lane half): the next slice's global
// loads are issued first; quad q+1's LDS operands are read while quad q's
// MFMAs run; after quad 2 the loaded registers are stored to the other
// stage and the workgroup barrier is taken, then the next slice's quad 0 is
// read from the other stage while quad 3's MFMAs (operands already in
// registers) run. So no LDS read latency sits in front of a slice's first
// MFMA. Hazards: stage s is written in slice t+1 only after slice t's
// barrier, and every wave's reads of stage s were waited for before it
// passed that barrier (the barrier's LDS fence); stage s^1 is read only
// after the barrier that follows its writes.
// ---------------------------------------------------------------------------
template <class T>
__device__ __forceinline__ void read_quad(const float* Ap, const float* Bp, int q, f32x4 (&a)[T::TM],
                                          f32x4 (&b)[T::TN]) {
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm) a[tm] = *reinterpret_cast<const f32x4*>(Ap + tm * 32 * T::LDK + 4 * q);
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn) b[tn] = *reinterpret_cast<const f32x4*>(Bp + tn * 32 * T::LDK + 4 * q);
}

template <class T>
__device__ __forceinline__ void mfma_quad(const f32x4 (&a)[T::TM], const f32x4 (&b)[T::TN],
                                          floatx16 (&acc)[T::TM][T::TN]) {
#pragma unroll
    for (int st = 0; st < 4; ++st)
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
                acc[tm][tn] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[tm][st], b[tn][st], acc[tm][tn], 0, 0, 0);
}

template <class T, bool TWO_LEVEL, class LA, class LB>
__device__ __forceinline__ void mfma_mainloop(LA& la, LB& lb, int k_begin, int k_end, float* lds,
                                              floatx16 (&sum)[T::TM][T::TN]) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wi = (wave / T::WN) * T::WAVE_M;
    const int wj = (wave % T::WN) * T::WAVE_N;
    // this lane's row of A (i) and of B (j), and its half of the slice's k
    const int a_off = (wi + (lane & 31)) * T::LDK + 16 * (lane >> 5);
    const int b_off = T::A_FLOATS + (wj + (lane & 31)) * T::LDK + 16 * (lane >> 5);

#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int r = 0; r < 16; ++r) sum[tm][tn][r] = 0.f;
    if (k_begin >= k_end) return;

    la.load(k_begin);
    lb.load(k_begin);
    la.store(lds);
    lb.store(lds + T::A_FLOATS);
    __syncthreads();

    f32x4 a[T::TM], b[T::TN];
    read_quad<T>(lds + a_off, lds + b_off, 0, a, b);
    int stage = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += T::BK) {
        const bool more = k0 + T::BK < k_end;
        if (more) {
            la.load(k0 + T::BK);
            lb.load(k0 + T::BK);
        }
        const float* Ap = lds + stage * T::STAGE + a_off;
        const float* Bp = lds + stage * T::STAGE + b_off;
        floatx16 acc[T::TM][T::TN];
        if (TWO_LEVEL) {
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                    for (int r = 0; r < 16; ++r) acc[tm][tn][r] = 0.f;
        }
#pragma unroll
        for (int q = 0; q < 3; ++q) {
            f32x4 an[T::TM], bn[T::TN];
            read_quad<T>(Ap, Bp, q + 1, an, bn);
            if (TWO_LEVEL)
                mfma_quad<T>(a, b, acc);
            else
                mfma_quad<T>(a, b, sum);
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm) a[tm] = an[tm];
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn) b[tn] = bn[tn];
        }
        float* next = lds + (stage ^ 1) * T::STAGE;
        if (more) {
            la.store(next);
            lb.store(next + T::A_FLOATS);
        }
        __syncthreads();
        f32x4 an[T::TM], bn[T::TN];
        if (more) read_quad<T>(next + a_off, next + b_off, 0, an, bn);
        if (TWO_LEVEL) {
            mfma_quad<T>(a, b, acc);
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int tn = 0; tn < T::TN; ++tn) sum[tm][tn] += acc[tm][tn];
        } else {
            mfma_quad<T>(a, b, sum);
        }
        if (more) {
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm) a[tm] = an[tm];
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn) b[tn] = bn[tn];
        }
        stage ^= 1;
    }
}

// Tile-local coordinates of accumulator element (tm, tn, r) for this lane.
template <class T>
__device__ __forceinline__ int acc_row(int tm, int r) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return (wave / T::WN) * T::WAVE_M + tm * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
}
template <class T>
__device__ __forceinline__ int acc_col(int tn) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return (wave % T::WN) * T::WAVE_N + tn * 32 + (lane & 31);
}

// Workgroups are dispatched round-robin over the 8 XCDs (each with its own
// L2). Remap the launch index so that consecutive logical workgroups - whose
// stream-K ranges hold neighbouring tiles sharing operand slices - run on the
// same XCD. Bijective on [0, total).
__device__ __forceinline__ int xcd_remap(int lin, int total) {
    const int per = total / 8;
    if (lin >= per * 8) return lin;
    return (lin % 8) * per + lin / 8;
}

// One unit of a workgroup's work: slices [kb, ke) of `tile`. `slot` is the
// partial slot (0: first segment of the range, 1: last) or -1 for a whole
// tile written straight to the output.
struct Segment {
    int tile, kb, ke, slot;
};

// Walks workgroup g's work: its stream-K range, then its whole tiles.
struct SegmentWalker {
    int64_t it, lo, hi;
    int dp;
    __host__ __device__ SegmentWalker(const StreamK& sk, int g) {
        lo = sk.sk_tiles ? sk.lo(g) : 0;
        hi = sk.sk_tiles ? sk.hi(g) : 0;
        it = lo;
        dp = sk.sk_tiles + g;
    }
    __host__ __device__ bool next(const StreamK& sk, Segment& s) {
        if (it < hi) {
            s.tile = (int)(it / sk.iters);
            s.kb = (int)(it - (int64_t)s.tile * sk.iters);
            const int64_t left = hi - it;
            s.ke = left < sk.iters - s.kb ? s.kb + (int)left : sk.iters;
            s.slot = (s.kb == 0 && s.ke == sk.iters) ? -1 : (it == lo ? 0 : 1);
            it += s.ke - s.kb;
            return true;
        }
        if (dp < sk.tiles) {
            s.tile = dp;
            s.kb = 0;
            s.ke = sk.iters;
            s.slot = -1;
            dp += sk.G;
            return true;
        }
        return false;
    }
};

// Partials of shared stream-K tile t: workgroups g0..g1 in order; g0's
// segment sits in slot `first_slot`, the others in slot 0 (their ranges
// start inside the tile). Returns false if one workgroup covers the tile.
__host__ __device__ inline bool tile_partials(const StreamK& sk, int t, int& g0, int& g1, int& first_slot) {
    const int64_t start = (int64_t)t * sk.iters, end = start + sk.iters;
    g0 = sk.first_owner(t);
    const int64_t lo0 = sk.lo(g0);
    if (lo0 <= start && sk.hi(g0) >= end) return false;
    first_slot = lo0 < start ? 1 : 0;
    g1 = g0;
    while (g1 + 1 < sk.G && sk.lo(g1 + 1) < end) ++g1;
    return true;
}

// Fixup cost in slice times, measured on ResNet-18 and transformer layers:
// about one slice for 128x128 tiles, scaled by tile area for smaller tiles
// (shorter slices). Round-robin wins only when stream-K saves less.
template <class T>
constexpr int fixup_slices() {
    return fixup_slices_for(T::BM, T::BN);
}

// Persistent-grid size: workgroups of `kernel` resident on the device at once.
template <typename K>
static int resident_groups(K kernel, size_t lds_bytes, int threads = 256) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, threads, lds_bytes) != hipSuccess ||
        per_cu < 1)
        per_cu = 1;
    return per_cu * cu_count();
}

// Partial-tile slots in the workspace: two per workgroup (the segment where
// its range starts, and the one where it ends), each BM*BN floats, row-major
// in tile coordinates.
template <class T>
__device__ __forceinline__ float* partial_slot(float* ws, int g, int which) {
    return ws + ((int64_t)g * 2 + which) * (T::BM * T::BN);
}

// In-kernel stream-K finish. Every workgroup that computes part of a split
// tile stores its partial into its slot and arrives at the tile's counter;
// the last to arrive sums the tile's partials and writes the tile. The
// partials cross XCDs (each XCD has its own L2), and the hand-off is the
// agent-scope release/acquire pair of the AMDGPU memory model (LLVM's
// AMDGPUUsage, GFX942 memory-model table) with its two whole-L2 cache
// operations left out, because they have nothing to do here:
//   release  The model emits `buffer_wbl2 sc1; s_waitcnt vmcnt(0)` before
//            the atomic. The write-back flushes ordinary stores held in the
//            XCD's L2; every byte published here is stored with the sc1
//            (device-scope) bit instead, which writes it through the L2, so
//            the wait for the stores' completion is the whole release.
//   acquire  The model emits `s_waitcnt vmcnt(0); buffer_inv sc1` after the
//            atomic. The invalidate drops stale L2 lines for ordinary loads;
//            the partials are read back with the sc1 bit, which does not
//            return a stale L2 line, so the wait for the atomic's return (its
//            value decides who finishes) is the whole acquire.
// Written as __ATOMIC_ACQ_REL the compiler emits both cache operations; the
// write-back of the tile's ordinary output stores and the invalidate of the
// next tile's operands in L2 then cost the split kernels 9-24% (ResNet-18
// batch 32 stem 119 -> 147 us, 3x3 64-channel layer 84 -> 106 us, GEMM
// 2048^3 174 -> 191 us, measured on MI355X). tests/native/finish_order.hip
// checks the emitted instruction order of this protocol.
static constexpr int kDeviceScope = 16;  // sc1: device-scope coherent buffer access

template <class T>
__device__ __forceinline__ uint32_t slot_byte_offset(int g, int which) {
    return (uint32_t)((g * 2 + which) * (T::BM * T::BN)) * 4u;
}

// One float of a partial, stored with device-scope coherence.
__device__ __forceinline__ void store_partial(__amdgpu_buffer_rsrc_t ws, uint32_t byte_off, float x) {
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), ws, (int)byte_off, 0, kDeviceScope);
}

// One float of a partial, loaded with device-scope coherence.
__device__ __forceinline__ float load_partial(__amdgpu_buffer_rsrc_t ws, uint32_t byte_off) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(ws, (int)byte_off, 0, kDeviceScope));
}

// Four floats of a partial, loaded with device-scope coherence.
__device__ __forceinline__ f32x4 load_partial4(__amdgpu_buffer_rsrc_t ws, uint32_t byte_off) {
    return __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(ws, (int)byte_off, 0, kDeviceScope));
}

// Called by every thread of the workgroup after its store_partial calls.
// `arrivals_before_last` = the number of workgroups that share the tile,
// minus one. Returns, in every thread, whether this workgroup arrived last;
// the last one also resets the counter to 0 for the next launch (kernel
// boundaries order it before that launch's arrivals).
__device__ __forceinline__ bool finish_arrive(int* counter, int arrivals_before_last) {
    __shared__ int last;
    // Release: this thread's sc1 stores have completed (vmcnt(0)), then the
    // barrier orders every thread's completion before thread 0's atomic.
    // The signal fences keep the compiler from moving memory operations
    // across the wait.
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        // Acquire: `old` is used here, so the atomic has returned before the
        // barrier below and before any thread issues its partial loads.
        last = old == arrivals_before_last;
        if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    return last;
}

// finish_arrive for a workgroup that shares two pieces of work, each with
// one other workgroup (counter c0 when on0, c1 when on1; the flags uniform
// over the workgroup): the same release and acquire, both atomics between
// one pair of barriers. last0 / last1: this workgroup arrived second.
__device__ __forceinline__ void finish_arrive_pair(int* c0, bool on0, int* c1, bool on1, bool& last0, bool& last1) {
    __shared__ int last[2];
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __syncthreads();
    if (threadIdx.x == 0) {
        int l0 = 0, l1 = 0;
        if (on0) {
            l0 = __hip_atomic_fetch_add(c0, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
            if (l0) __hip_atomic_store(c0, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (on1) {
            l1 = __hip_atomic_fetch_add(c1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 1;
            if (l1) __hip_atomic_store(c1, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        last[0] = l0;
        last[1] = l1;
    }
    __syncthreads();
    last0 = last[0];
    last1 = last[1];
}

// Direct-to-LDS buffer loads: lane l's `size` bytes land at LDS[lds_dst +
// size * l] (lds_dst wave-uniform), no VGPR staging and no LDS store.
typedef __attribute__((address_space(3))) void* lds_ptr;
__device__ __forceinline__ void dma_load4(__amdgpu_buffer_rsrc_t r, float* lds_dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds_dst, 4, voff, soff, 0, 0);
}
__device__ __forceinline__ void dma_load16(__amdgpu_buffer_rsrc_t r, float* lds_dst, uint32_t voff, uint32_t soff) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds_dst, 16, voff, soff, 0, 0);
}

// s_waitcnt vmcnt(0): the direct-to-LDS loads of this wave have landed
__device__ __forceinline__ void wait_dma() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Workgroup barrier for a multi-stage direct-to-LDS pipeline: each wave
// waits until at most N of its vector memory operations are outstanding
// (its direct-to-LDS loads complete in issue order, so all but the newest N
// have written LDS) and its LDS reads and writes are done (lgkmcnt(0)), then
// s_barrier. __syncthreads cannot be used: its fence makes the compiler wait
// for every outstanding vector memory operation (vmcnt(0)) - the loads of
// the slices meant to stay in flight. The signal fences keep the compiler
// from moving memory accesses across the barrier; gfx950's barrier needs no
// other wait (the compiler inserts none before it).
template <int N>
__device__ __forceinline__ void dma_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4));  // vmcnt(N) expcnt(7) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// `addr` if `keep`, else exactly kOutOfRange (adding an SGPR offset below
// 2^31 cannot wrap it back into range); without branches
__device__ __forceinline__ uint32_t keep_or_oob(uint32_t addr, bool keep) {
    const uint32_t m = 0u - (uint32_t)keep;
    return (addr & m) | (kOutOfRange & ~m);
}

}  // namespace nnc
