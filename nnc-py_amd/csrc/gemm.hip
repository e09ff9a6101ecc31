// Gemm, Gemm_nt and MatMul of the nnc ABI (runtime/x86/ops.c:1607-1886).
//
// Dense products run on the fp32 MFMA tile engine (mfma_tile.h), stream-K
// scheduled over batches x tiles x K slices. Operands whose rows are 16-byte
// aligned on both sides (k-contiguous or x-contiguous) go straight from
// global memory into LDS (gemm_dma_k: 64x64 tiles with four LDS stages,
// 128x128 tiles with two); shared tiles are finished inside the kernel by
// the last workgroup to arrive, or by a fixup kernel when split further.
// Other layouts (unaligned rows, K or M/N not a multiple of 4) stage through
// registers (gemm_streamk_k, scalar loads where needed). Both sum a shared
// tile's partials in fixed workgroup order. Products with one
// output row or column are HBM-bound and use dedicated kernels:
//   gemv_xc_k  out[j] = sum_k a[k] * B[k][j]   (B row-major; float4 columns,
//              K split across workgroups, deterministic partial reduction)
//   dot_k      out[i][j] = sum_k A[i][k] * B[j][k]  (both k-contiguous; one
//              wave per output, shuffle reduction)
// and products with at most 32 output rows, both operands k-contiguous, one
// MFMA launch without partials (gemm_skinny_nt_k: 16 columns per workgroup,
// K split over its waves, summed in LDS).
//
// The reference accumulates Gemm in fp64 and MatMul with a Kahan fp32 sum;
// here every product accumulates in fp32 (two-level in the register-staged
// kernel), within the 1e-4 absolute / 1e-3 relative bar.
//
// DIVERGES: batched MatMul steps A by M*K and B by K*N per batch (numpy /
// ONNX semantics). The reference steps by the batch count (ops.c:1687-1704),
// which is only correct for a single batch.
#include "mfma_tile.h"

#include <stdlib.h>

#include <algorithm>
#include <type_traits>

namespace nnc {

struct GemmArgs {
    const float* A;
    const float* B;
    const float* C;
    float* out;
    float* ws;
    int M, N, K;
    int64_t lda, ldb, sa, sb, so;
    float alpha, beta;
    int c_mode;  // 0 none, 1 C[j], 2 C[i*N + j]
    int relu;
    int tiles_m, tiles_n, splits;  // splits: K-split count of the GEMV path
    int* cnt;  // stream-K tile counters of the in-kernel finish, or null
    int out32;  // one batch of out (and C) below 2 GiB: whole tiles use 32-bit buffer offsets
};

__device__ __forceinline__ float gemm_finish(const GemmArgs& g, int i, int j, float v) {
    float o = g.alpha * v;
    if (g.c_mode == 1) o += g.beta * g.C[j];
    else if (g.c_mode == 2) o += g.beta * g.C[(int64_t)i * g.N + j];
    if (g.relu) o = o > 0.0f ? o : 0.0f;
    return o;
}

// A whole output tile: alpha*v (+ beta*C) (+ relu) per element as
// gemm_finish, one 32-row block (tm) at a time with the block's C loads
// issued before its first store - one memory round trip per block (C may
// alias out as far as the compiler knows, so per-element loads after stores
// were serialised, each waiting for the earlier stores). Out-of-range rows
// and columns get an out-of-range buffer offset: loads read 0, stores are
// dropped.
template <class T>
__device__ __forceinline__ void gemm_store_tile(const GemmArgs& g, int batch, int i0, int j0,
                                                const floatx16 (&sum)[T::TM][T::TN]) {
    const __amdgpu_buffer_rsrc_t ro = make_rsrc(g.out + batch * g.so), rc = make_rsrc(g.C);
    int jj[T::TN];
    float cj[T::TN];  // C[j] (c_mode 1)
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn) {
        jj[tn] = j0 + acc_col<T>(tn);
        cj[tn] = g.c_mode == 1 ? load_f32(rc, jj[tn] < g.N ? (uint32_t)jj[tn] * 4u : kOutOfRange) : 0.f;
    }
    const int ib = i0 + acc_row<T>(0, 0);  // this lane's first row; row (tm, r) adds a wave-uniform step
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm) {
        float cv[T::TN][16];
        if (g.c_mode == 2) {
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = ib + tm * 32 + 8 * (r >> 2) + (r & 3);
                    const bool ok = i < g.M && jj[tn] < g.N;
                    cv[tn][r] = load_f32(rc, ok ? (uint32_t)(i * g.N + jj[tn]) * 4u : kOutOfRange);
                }
        }
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int i = ib + tm * 32 + 8 * (r >> 2) + (r & 3);
                const bool ok = i < g.M && jj[tn] < g.N;
                float o = g.alpha * sum[tm][tn][r];
                if (g.c_mode == 1) o += g.beta * cj[tn];
                else if (g.c_mode == 2) o += g.beta * cv[tn][r];
                if (g.relu) o = o > 0.0f ? o : 0.0f;
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(o), ro,
                                                      (int)(ok ? (uint32_t)(i * g.N + jj[tn]) * 4u : kOutOfRange), 0, 0);
            }
    }
}

// Loader kinds: element (x, k) at base[x*ld + k] (K*) or base[k*ld + x] (X*)
enum LoadKind { kKC4 = 0, kKC = 1, kXC4 = 2, kXC = 3 };

template <int KIND, int X, int BK, int LD>
struct PickLoader;
template <int X, int BK, int LD>
struct PickLoader<kKC4, X, BK, LD> {
    typedef KContigLoader4<X, BK, LD> type;
    static __device__ int64_t offset(int x0, int64_t ld) { return (int64_t)x0 * ld; }
};
template <int X, int BK, int LD>
struct PickLoader<kKC, X, BK, LD> {
    typedef KContigLoader<X, BK, LD> type;
    static __device__ int64_t offset(int x0, int64_t ld) { return (int64_t)x0 * ld; }
};
template <int X, int BK, int LD>
struct PickLoader<kXC4, X, BK, LD> {
    typedef XContigLoader4<X, BK, LD> type;
    static __device__ int64_t offset(int x0, int64_t) { return x0; }
};
template <int X, int BK, int LD>
struct PickLoader<kXC, X, BK, LD> {
    typedef XContigLoader<X, BK, LD> type;
    static __device__ int64_t offset(int x0, int64_t) { return x0; }
};

template <class T, int AK, int BKIND>
__global__ void __launch_bounds__(256, 2) gemm_streamk_k(GemmArgs g, StreamK sk) {
    extern __shared__ __align__(16) float lds[];
    const int wg = xcd_remap(blockIdx.x, sk.G);
    const int per_batch = g.tiles_m * g.tiles_n;
    typedef PickLoader<AK, T::BM, T::BK, T::LDK> PA;
    typedef PickLoader<BKIND, T::BN, T::BK, T::LDK> PB;
    SegmentWalker walk(sk, wg);
    Segment seg;
    while (walk.next(sk, seg)) {
        const int batch = seg.tile / per_batch, rem = seg.tile - batch * per_batch;
        const int mt = rem % g.tiles_m, nt = rem / g.tiles_m;
        const int i0 = mt * T::BM, j0 = nt * T::BN;
        typename PA::type la;
        typename PB::type lb;
        la.init(g.A + batch * g.sa + PA::offset(i0, g.lda), g.lda, g.M - i0, g.K);
        lb.init(g.B + batch * g.sb + PB::offset(j0, g.ldb), g.ldb, g.N - j0, g.K);
        floatx16 sum[T::TM][T::TN];
        mfma_mainloop<T, true>(la, lb, seg.kb * T::BK, min(g.K, seg.ke * T::BK), lds, sum);
        // (128x128 tiles keep the per-element path: their kernels are at the register limit)
        if (T::BM * T::BN < 128 * 128 && seg.slot < 0 && g.out32) {
            gemm_store_tile<T>(g, batch, i0, j0, sum);
        } else if (seg.slot < 0) {
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn) {
                const int j = j0 + acc_col<T>(tn);
                if (j >= g.N) continue;
#pragma unroll
                for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int i = i0 + acc_row<T>(tm, r);
                        if (i < g.M) g.out[batch * g.so + (int64_t)i * g.N + j] = gemm_finish(g, i, j, sum[tm][tn][r]);
                    }
            }
        } else {
            float* slot = partial_slot<T>(g.ws, wg, seg.slot);
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                    for (int r = 0; r < 16; ++r) slot[acc_row<T>(tm, r) * T::BN + acc_col<T>(tn)] = sum[tm][tn][r];
        }
    }
}

// Grid (chunks, stream-K tiles): workgroup (c, t) finishes chunk c of tile t
// (256 float4 of the BM x BN tile): shared tiles sum their partials in
// workgroup order and apply alpha / beta * C / relu. Each thread handles 4
// consecutive columns of a tile row.
template <class T>
__global__ void __launch_bounds__(256) gemm_fixup_k(GemmArgs g, StreamK sk) {
    const int t = blockIdx.y;
    int g0, g1, first_slot;
    if (!tile_partials(sk, t, g0, g1, first_slot)) return;
    const int e4 = blockIdx.x * 256 + threadIdx.x;
    if (e4 >= T::BM * T::BN / 4) return;
    const int per_batch = g.tiles_m * g.tiles_n;
    const int batch = t / per_batch, rem = t - batch * per_batch;
    const int i = (rem % g.tiles_m) * T::BM + (e4 * 4) / T::BN;
    const int j = (rem / g.tiles_m) * T::BN + (e4 * 4) % T::BN;
    if (i >= g.M || j >= g.N) return;
    float4 v = reinterpret_cast<const float4*>(partial_slot<T>(g.ws, g0, first_slot))[e4];
    for (int w = g0 + 1; w <= g1; ++w) {
        const float4 p = reinterpret_cast<const float4*>(partial_slot<T>(g.ws, w, 0))[e4];
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    float* o = g.out + batch * g.so + (int64_t)i * g.N;
    const float vals[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int q = 0; q < 4; ++q)
        if (j + q < g.N) o[j + q] = gemm_finish(g, i, j + q, vals[q]);
}

// ---------------------------------------------------------------------------
// Direct-to-LDS GEMM: operands go from global memory straight into LDS
// (`buffer_load ... lds`), 16 bytes per lane: no VGPR staging and no LDS
// store instructions. A stage holds the A operand (BM x 32 k) then the B
// operand (BN x 32 k), each in one of two layouts:
//   KC  (element (x, k) at base[x*ld + k]: A row-major, B stored [N][K])
//       [X rows][32 k], 16-byte chunks XOR-swizzled: chunk kc of row x sits
//       at position kc ^ (x & 7). One load instruction covers 8 rows (lane
//       l: row l / 8, global chunk (l % 8) ^ (row % 8)); an MFMA lane reads
//       its four k of a quad as one ds_read_b128, eight consecutive rows on
//       eight different bank groups.
//   XC  (element (x, k) at base[k*ld + x]: B row-major [K][N], A stored
//       [K][M]) [32 k][X]: one load instruction covers 256 / X rows of k
//       (lane l: row l / (X/4), four consecutive x); an MFMA lane reads its k
//       one ds_read_b32 at a time, 32 lanes on 32 consecutive floats.
// Both need 16-byte aligned rows (ld % 4 == 0, aligned base and batch
// stride); KC needs K % 4 == 0 and XC needs the tile's x extent (M or N) %
// 4 == 0, so a 16-byte chunk is wholly inside or wholly outside the matrix
// and out-of-range chunks get an out-of-range offset (the hardware writes 0
// to LDS). Checked by the host.
// ---------------------------------------------------------------------------
template <class T, int NS>
struct GemmDma {
    static constexpr int A_FLOATS = T::BM * 32, B_FLOATS = T::BN * 32;
    static constexpr int STAGE = A_FLOATS + B_FLOATS;
    static constexpr int LDS_FLOATS = NS * STAGE;  // NS stages: NS - 1 slices in flight
    // waves per SIMD that the LDS stages allow (160 KB per CU), at most 4:
    // the register budget the kernel is compiled for
    static constexpr int LDS_WAVES = (160 * 1024 / (LDS_FLOATS * 4)) * T::NW / 4;
    static constexpr int MIN_WAVES = LDS_WAVES < 2 ? 2 : (LDS_WAVES > 4 ? 4 : LDS_WAVES);
    static_assert(T::BK == 32 && T::NW == 4 && NS >= 2, "direct-to-LDS gemm tile");
};

template <class T, int X, int OFF>
struct KcOperand {
    static constexpr int LOADS = X / (8 * T::NW);  // load instructions per wave per slice
    static_assert(X % (8 * T::NW) == 0, "rows split evenly over the waves");
    static __device__ int64_t origin(int x0, int64_t ld) { return (int64_t)x0 * ld; }
    __amdgpu_buffer_rsrc_t r;
    uint32_t vo[LOADS];  // this lane's byte offset from the tile origin, or kOutOfRange
    int kc4;             // k of this lane's chunk within a slice
    int rb, sw;          // read side: LDS offset of this lane's row, swizzle of its k-half
    __device__ void init_read(int xw, int lane) {
        rb = OFF + (xw + (lane & 31)) * 32;
        sw = (4 * (lane >> 5)) ^ (lane & 7);
    }
    __device__ void tile(const float* base, int64_t ld, int xlim, int wave, int lane) {
        r = make_rsrc(base);
        const int kc = (lane & 7) ^ ((lane >> 3) & 7);
        kc4 = 4 * kc;
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int x = (wave + T::NW * i) * 8 + (lane >> 3);
            vo[i] = keep_or_oob((uint32_t)(x * ld) * 4u + (uint32_t)kc * 16u, x < xlim);
        }
    }
    __device__ void issue(float* S, int wave, int k0, int K, bool on) const {
        const bool in = on && k0 + kc4 < K;
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            dma_load16(r, S + OFF + (wave + T::NW * i) * 8 * 32, in ? vo[i] : kOutOfRange, (uint32_t)k0 * 4u);
    }
    template <int N>
    __device__ void read(const float* S, int q, f32x4 (&v)[N]) const {
#pragma unroll
        for (int t = 0; t < N; ++t) v[t] = *reinterpret_cast<const f32x4*>(S + rb + t * 32 * 32 + ((sw ^ q) << 2));
    }
};

template <class T, int X, int OFF>
struct XcOperand {
    static constexpr int RP = 256 / X;                // k rows per load instruction
    static constexpr int LOADS = 32 / (RP * T::NW);  // load instructions per wave per slice
    static_assert(32 % (RP * T::NW) == 0, "k rows split evenly over the waves");
    static __device__ int64_t origin(int x0, int64_t) { return x0; }
    __amdgpu_buffer_rsrc_t r;
    uint32_t vo[LOADS];
    uint32_t ld4;  // row pitch in bytes
    int kr0;       // this lane's k row (within a slice) in its first load
    int rb;        // read side: LDS offset of this lane's column in its k-half
    __device__ void init_read(int xw, int lane) { rb = OFF + 16 * (lane >> 5) * X + xw + (lane & 31); }
    __device__ void tile(const float* base, int64_t ld, int xlim, int wave, int lane) {
        r = make_rsrc(base);
        ld4 = (uint32_t)ld * 4u;
        const int xx = 4 * (lane % (X / 4));
        kr0 = wave * LOADS * RP + lane / (X / 4);
#pragma unroll
        for (int i = 0; i < LOADS; ++i)
            vo[i] = keep_or_oob((uint32_t)(kr0 + i * RP) * ld4 + (uint32_t)xx * 4u, xx < xlim);
    }
    __device__ void issue(float* S, int wave, int k0, int K, bool on) const {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const bool in = on && k0 + kr0 + i * RP < K;
            dma_load16(r, S + OFF + (wave * LOADS + i) * RP * X, in ? vo[i] : kOutOfRange, (uint32_t)k0 * ld4);
        }
    }
    template <int N>
    __device__ void read(const float* S, int q, f32x4 (&v)[N]) const {
#pragma unroll
        for (int t = 0; t < N; ++t)
#pragma unroll
            for (int s = 0; s < 4; ++s) v[t][s] = S[rb + (4 * q + s) * X + t * 32];
    }
};

// Shared stream-K tile t finished by the workgroup whose partial arrived
// last: partials summed in workgroup order g0..g1 (the order of
// gemm_fixup_k, so the result is the same to the bit), then alpha / beta * C
// / relu. Each thread handles 4 consecutive columns of a tile row.
template <class T>
__device__ void gemm_finish_tile(const GemmArgs& g, int t, int g0, int g1, int first_slot) {
    constexpr int E = T::BM * T::BN / 1024;  // float4 per thread
    constexpr int CH = E < 4 ? E : 4;         // float4 in flight per partial (register budget)
    const __amdgpu_buffer_rsrc_t rws = make_rsrc(g.ws);
    const int per_batch = g.tiles_m * g.tiles_n;
    const int batch = t / per_batch, rem = t - batch * per_batch;
    const int i0 = (rem % g.tiles_m) * T::BM, j0 = (rem / g.tiles_m) * T::BN;
    const uint32_t first = slot_byte_offset<T>(g0, first_slot);
    for (int e0 = 0; e0 < E; e0 += CH) {
        f32x4 v[CH];
#pragma unroll
        for (int e = 0; e < CH; ++e)
            v[e] = load_partial4(rws, first + (uint32_t)((e0 + e) * 256 + threadIdx.x) * 16u);
        for (int w = g0 + 1; w <= g1; ++w) {
            const uint32_t base = slot_byte_offset<T>(w, 0);
            f32x4 p[CH];
#pragma unroll
            for (int e = 0; e < CH; ++e)
                p[e] = load_partial4(rws, base + (uint32_t)((e0 + e) * 256 + threadIdx.x) * 16u);
#pragma unroll
            for (int e = 0; e < CH; ++e) v[e] += p[e];
        }
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int e4 = (e0 + e) * 256 + threadIdx.x;
            const int i = i0 + (e4 * 4) / T::BN;
            const int j = j0 + (e4 * 4) % T::BN;
            if (i >= g.M || j >= g.N) continue;
            float* o = g.out + batch * g.so + (int64_t)i * g.N;
            const f32x4 x = v[e];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                if (j + q < g.N) o[j + q] = gemm_finish(g, i, j + q, x[q]);
        }
    }
}

// A finished segment: a whole tile to the output, or a partial tile to the
// workgroup's slot. With tile counters (g.cnt) each writer of a partial then
// counts itself in, and the last to arrive finishes the tile (no workgroup
// waits for another) and returns the counter to zero.
template <class T, bool FIN>
__device__ __forceinline__ void gemm_segment_out(const GemmArgs& g, const StreamK& sk, const Segment& seg, int wg,
                                                 int batch, int i0, int j0, const floatx16 (&sum)[T::TM][T::TN]) {
    if (T::BM * T::BN < 128 * 128 && seg.slot < 0 && g.out32) {
        gemm_store_tile<T>(g, batch, i0, j0, sum);
        return;
    }
    if (seg.slot < 0) {
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn) {
            const int j = j0 + acc_col<T>(tn);
            if (j >= g.N) continue;
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int i = i0 + acc_row<T>(tm, r);
                    if (i < g.M) g.out[batch * g.so + (int64_t)i * g.N + j] = gemm_finish(g, i, j, sum[tm][tn][r]);
                }
        }
        return;
    }
    if (!FIN || !g.cnt) {  // the fixup kernel reads the partials after this kernel
        float* slot = partial_slot<T>(g.ws, wg, seg.slot);
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int r = 0; r < 16; ++r) slot[acc_row<T>(tm, r) * T::BN + acc_col<T>(tn)] = sum[tm][tn][r];
        return;
    }
    if constexpr (FIN) {
        const __amdgpu_buffer_rsrc_t rws = make_rsrc(g.ws);
        const uint32_t base = slot_byte_offset<T>(wg, seg.slot);
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const float x = sum[tm][tn][r];
                    store_partial(rws, base + (uint32_t)(acc_row<T>(tm, r) * T::BN + acc_col<T>(tn)) * 4u, x);
                }
        int g0, g1, first_slot;
        tile_partials(sk, seg.tile, g0, g1, first_slot);
        if (finish_arrive(g.cnt + seg.tile, g1 - g0)) gemm_finish_tile<T>(g, seg.tile, g0, g1, first_slot);
    }
}

// A workgroup's slices in order, across its segments (stream-K range, then
// whole tiles).
struct SliceCursor {
    SegmentWalker walk;
    Segment seg;
    int it;
    bool valid;
    __device__ SliceCursor(const StreamK& sk, int wg) : walk(sk, wg) {
        valid = walk.next(sk, seg);
        it = seg.kb;
    }
    // to the next slice; true if it starts a new segment
    __device__ bool advance(const StreamK& sk) {
        if (++it < seg.ke) return false;
        valid = walk.next(sk, seg);
        it = seg.kb;
        return valid;
    }
};

// Stream-K over batches x tiles x K slices, NS LDS stages: the loads run
// NS - 1 slices ahead of the MFMAs, across segment boundaries (a load cursor
// walks the workgroup's slices ahead of the compute cursor, so a new tile
// starts with its first slices already in LDS). Each slice is one wait and
// one barrier: the wait leaves at most (NS - 2) x L vector memory operations
// outstanding. Loads complete in issue order, so at least the oldest slice's
// L loads have landed even with an epilogue's stores among the outstanding
// operations (the count can reach the bound only after L + (stores) of them
// completed, and at most (stores) of those were stores). Products accumulate
// in fp32 straight into the tile's accumulators.
template <class T, int NS, class OA, class OB, bool FIN>
__global__ void __launch_bounds__(T::THREADS, (GemmDma<T, NS>::MIN_WAVES)) gemm_dma_k(GemmArgs g, StreamK sk) {
    typedef GemmDma<T, NS> D;
    constexpr int L = OA::LOADS + OB::LOADS;  // load instructions per wave per slice
    extern __shared__ __align__(16) float lds[];
    const int wg = xcd_remap(blockIdx.x, sk.G);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int per_batch = g.tiles_m * g.tiles_n;
    OA oa;
    OB ob;
    oa.init_read((wave / T::WN) * T::WAVE_M, lane);
    ob.init_read((wave % T::WN) * T::WAVE_N, lane);
    auto set_tile = [&](int tile) {
        const int batch = tile / per_batch, rem = tile - batch * per_batch;
        const int i0 = (rem % g.tiles_m) * T::BM, j0 = (rem / g.tiles_m) * T::BN;
        oa.tile(g.A + batch * g.sa + OA::origin(i0, g.lda), g.lda, g.M - i0, wave, lane);
        ob.tile(g.B + batch * g.sb + OB::origin(j0, g.ldb), g.ldb, g.N - j0, wave, lane);
    };
    SliceCursor lc(sk, wg);  // load cursor
    if (!lc.valid) return;
    SegmentWalker walk(sk, wg);  // compute cursor
    Segment seg;
    walk.next(sk, seg);
    set_tile(lc.seg.tile);
    // slices 0 .. NS-2 into stages 0 .. NS-2 (past the end: out-of-range
    // loads, which keep the wait counts uniform)
#pragma unroll
    for (int s = 0; s < NS - 1; ++s) {
        oa.issue(lds + s * D::STAGE, wave, lc.it * T::BK, g.K, lc.valid);
        ob.issue(lds + s * D::STAGE, wave, lc.it * T::BK, g.K, lc.valid);
        if (lc.valid && lc.advance(sk)) set_tile(lc.seg.tile);
    }
    dma_barrier<(NS - 2) * L>();
    // operands of quads 0 and 2 in set 0, quads 1 and 3 in set 1
    f32x4 a0[T::TM], b0[T::TN], a1[T::TM], b1[T::TN];
    oa.read(lds, 0, a0);
    ob.read(lds, 0, b0);
    int cs = 0, ls = NS - 1;  // stages being computed and loaded
    while (true) {
        const int batch = seg.tile / per_batch, rem = seg.tile - batch * per_batch;
        const int i0 = (rem % g.tiles_m) * T::BM, j0 = (rem / g.tiles_m) * T::BN;
        floatx16 sum[T::TM][T::TN];
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int r = 0; r < 16; ++r) sum[tm][tn][r] = 0.f;
        for (int it = seg.kb; it < seg.ke; ++it) {
            float* ld_stage = lds + ls * D::STAGE;
            const float* S = lds + cs * D::STAGE;
            const int cn = cs + 1 == NS ? 0 : cs + 1;
            oa.issue(ld_stage, wave, lc.it * T::BK, g.K, lc.valid);
            oa.read(S, 1, a1);
            ob.read(S, 1, b1);
            mfma_quad<T>(a0, b0, sum);
            ob.issue(ld_stage, wave, lc.it * T::BK, g.K, lc.valid);
            if (lc.valid && lc.advance(sk)) set_tile(lc.seg.tile);
            oa.read(S, 2, a0);
            ob.read(S, 2, b0);
            mfma_quad<T>(a1, b1, sum);
            oa.read(S, 3, a1);
            ob.read(S, 3, b1);
            mfma_quad<T>(a0, b0, sum);
            dma_barrier<(NS - 2) * L>();
            oa.read(lds + cn * D::STAGE, 0, a0);
            ob.read(lds + cn * D::STAGE, 0, b0);
            mfma_quad<T>(a1, b1, sum);
            cs = cn;
            ls = ls + 1 == NS ? 0 : ls + 1;
        }
        gemm_segment_out<T, FIN>(g, sk, seg, wg, batch, i0, j0, sum);
        if (!walk.next(sk, seg)) break;
    }
    // the loads issued past the last slice (out of range: they write zeros to
    // LDS) land before the workgroup ends and its LDS is handed on
    wait_dma();
}

// out[j] partials: thread owns 4 consecutive columns (VEC) or 1.
template <bool VEC>
__global__ void __launch_bounds__(256) gemv_xc_k(const float* a, int64_t a_stride, const float* B,
                                                 int64_t ldb, float* ws, int N, int K, int k_per) {
    const int s = blockIdx.y;
    const int kb = s * k_per, ke = min(K, kb + k_per);
    if (VEC) {
        const int j = (blockIdx.x * 256 + threadIdx.x) * 4;
        if (j >= N) return;
        float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
        if (j + 3 < N) {
            for (int k = kb; k < ke; ++k) {
                const float av = a[k * a_stride];
                const float4 bv = *reinterpret_cast<const float4*>(B + (int64_t)k * ldb + j);
                acc.x += av * bv.x;
                acc.y += av * bv.y;
                acc.z += av * bv.z;
                acc.w += av * bv.w;
            }
            *reinterpret_cast<float4*>(ws + (int64_t)s * N + j) = acc;
        } else {
            for (int k = kb; k < ke; ++k) {
                const float av = a[k * a_stride];
                const float* row = B + (int64_t)k * ldb + j;
                acc.x += av * row[0];
                if (j + 1 < N) acc.y += av * row[1];
                if (j + 2 < N) acc.z += av * row[2];
            }
            float* dst = ws + (int64_t)s * N + j;
            dst[0] = acc.x;
            if (j + 1 < N) dst[1] = acc.y;
            if (j + 2 < N) dst[2] = acc.z;
        }
    } else {
        const int j = blockIdx.x * 256 + threadIdx.x;
        if (j >= N) return;
        float acc = 0.f;
        for (int k = kb; k < ke; ++k) acc += a[k * a_stride] * B[(int64_t)k * ldb + j];
        ws[(int64_t)s * N + j] = acc;
    }
}

// Sums the K-split partials of 64 columns per workgroup: each wave adds a
// contiguous quarter of the splits in order (lanes on consecutive columns,
// loads issued eight at a time), then the four quarter sums are added in
// wave order: a fixed summation order, whatever the timing.
__global__ void __launch_bounds__(256) gemv_reduce_k(GemmArgs g) {
    __shared__ float part[4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = blockIdx.x * 64 + lane;
    const int q = (g.splits + 3) / 4;
    const int s0 = wave * q, s1 = min(g.splits, s0 + q);
    float v = 0.f;
    if (j < g.N) {
        const float* col = g.ws + j;
        int s = s0;
        for (; s + 8 <= s1; s += 8) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = col[(int64_t)(s + u) * g.N];
#pragma unroll
            for (int u = 0; u < 8; ++u) v += t[u];
        }
        for (; s < s1; ++s) v += col[(int64_t)s * g.N];
    }
    part[wave][lane] = v;
    __syncthreads();
    if (wave == 0 && j < g.N)
        g.out[j] = gemm_finish(g, 0, j, ((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]);
}

// One output row, B row-major (MatMul [1, K] x [K, N]), in one launch:
// grid (ceil(N / 64), S), workgroup (c, s) takes columns 64c .. 64c + 63
// over rows k_per s ..: thread t owns the four columns 64c + 4 (t % 16) on
// row lane t / 16, i.e. rows kb + t / 16 + 16 i (a wave reads four 256-byte
// row segments per load), with UN rows' 16-byte loads in flight; the 16 row
// lanes' sums are added in row-lane order through LDS. S == 1: that sum is
// the output. Otherwise the workgroup stores its 256-byte partial (device
// scope) and the last of the column block's S workgroups to arrive
// (finish_arrive, the stream-K protocol of mfma_tile.h) adds the S partials
// in split order, so the sum is the same whichever workgroup finishes.
// At most kGemvMaxSplits workgroups arrive at one counter (64 on one
// counter measured 6 us slower than the two-launch form). Needs N % 4 == 0
// and 16-byte aligned B rows.
constexpr int kGemvMaxSplits = 16;
typedef unsigned int gemv_u32x4 __attribute__((ext_vector_type(4)));

template <int UN>
__global__ void __launch_bounds__(256) gemv_fin_k(GemmArgs g, int64_t a_stride, int S, int k_per) {
    __shared__ f32x4 red[16][16];
    const int t = threadIdx.x, c4 = t & 15, rr = t >> 4;
    const int c = blockIdx.x, s = blockIdx.y;
    const int j = c * 64 + 4 * c4;
    const int kb = s * k_per, ke = min(g.K, kb + k_per);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    if (j < g.N) {
        const float* col = g.B + j;
        int k = kb + rr;
        for (; k + 16 * (UN - 1) < ke; k += 16 * UN) {
            f32x4 b[UN];
            float av[UN];
#pragma unroll
            for (int u = 0; u < UN; ++u) {
                b[u] = *reinterpret_cast<const f32x4*>(col + (int64_t)(k + 16 * u) * g.ldb);
                av[u] = g.A[(int64_t)(k + 16 * u) * a_stride];
            }
#pragma unroll
            for (int u = 0; u < UN; ++u) {
                acc.x += av[u] * b[u].x;
                acc.y += av[u] * b[u].y;
                acc.z += av[u] * b[u].z;
                acc.w += av[u] * b[u].w;
            }
        }
        for (; k < ke; k += 16) {
            const f32x4 b = *reinterpret_cast<const f32x4*>(col + (int64_t)k * g.ldb);
            const float av = g.A[(int64_t)k * a_stride];
            acc.x += av * b.x;
            acc.y += av * b.y;
            acc.z += av * b.z;
            acc.w += av * b.w;
        }
    }
    red[rr][c4] = acc;
    __syncthreads();
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (t < 16) {
        v = red[0][t];
#pragma unroll
        for (int q = 1; q < 16; ++q) v += red[q][t];
    }
    if (S > 1) {
        const __amdgpu_buffer_rsrc_t rws = make_rsrc(g.ws);
        const uint32_t base = (uint32_t)c * (uint32_t)S * 256u;
        if (t < 16)
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(gemv_u32x4, v), rws,
                                                   (int)(base + (uint32_t)s * 256u + (uint32_t)t * 16u), 0, kDeviceScope);
        if (!finish_arrive(g.cnt + c, S - 1)) return;  // uniform
        // thread t: partial t / 16, float4 t % 16 (red was read before
        // finish_arrive's barriers)
        if (t < 16 * S) red[rr][c4] = load_partial4(rws, base + (uint32_t)t * 16u);
        __syncthreads();
        if (t < 16) {
            v = red[0][t];
            for (int q = 1; q < S; ++q) v += red[q][t];
        }
    }
    if (t >= 16 || j >= g.N) return;
#pragma unroll
    for (int q = 0; q < 4; ++q) g.out[j + q] = gemm_finish(g, 0, j + q, v[q]);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

// one wave per output (i, j): sum_k A[i*lda + k] * B[j*ldb + k]
template <bool VEC>
__global__ void __launch_bounds__(256) dot_k(GemmArgs g) {
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (w >= (int64_t)g.M * g.N) return;
    const int i = (int)(w / g.N), j = (int)(w - (int64_t)(w / g.N) * g.N);
    const float* a = g.A + (int64_t)i * g.lda;
    const float* b = g.B + (int64_t)j * g.ldb;
    float acc = 0.f;
    if (VEC) {
        const int K4 = g.K / 4;
        for (int q = lane; q < K4; q += 64) {
            const float4 x = reinterpret_cast<const float4*>(a)[q];
            const float4 y = reinterpret_cast<const float4*>(b)[q];
            acc += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
        }
        for (int k = K4 * 4 + lane; k < g.K; k += 64) acc += a[k] * b[k];
    } else {
        for (int k = lane; k < g.K; k += 64) acc += a[k] * b[k];
    }
    acc = wave_sum(acc);
    if (lane == 0) g.out[(int64_t)i * g.N + j] = gemm_finish(g, i, j, acc);
}

// Few output rows, both operands k-contiguous (a classifier at small batch:
// [M <= 32, K] x [N, K]^T). The tile kernels would give each 64x64 tile to
// many workgroups and finish it in a second launch; here a workgroup owns 16
// output columns for all rows and its 8 waves split K, so the whole product
// is one launch with no partials in memory. Wave w takes K chunks of 16
// [w*C/8, (w+1)*C/8); lane (i = lane % 16, q = lane / 16) loads A row i and B
// row j0 + i at k = 16c + 4q .. +3 as one 16-byte load each, and the four
// 16x16x4 MFMAs of a chunk take element e of those loads (k = 16c + 4q + e for
// lane group q: every k exactly once). MB 16-row blocks (M <= 16 MB). The
// waves' 16 x 16 sums meet in LDS and are added in wave order. Needs K <= 1024
// (at most 8 chunks per wave, all loads issued before the first MFMA), K % 4
// == 0, 16-byte aligned rows, and both operands under 2 GiB of byte offsets;
// rows beyond M or N and k beyond K read 0.
static constexpr int kSkinnyWaves = 8, kSkinnyMaxK = 1024, kSkinnyRows = 32;
template <int MB>
__global__ void __launch_bounds__(64 * kSkinnyWaves) gemm_skinny_nt_k(GemmArgs g) {
    constexpr int CH = kSkinnyMaxK / 16 / kSkinnyWaves;  // chunks per wave at most
    __shared__ float part[kSkinnyWaves][MB][4][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int li = lane & 15, q = lane >> 4;
    const int j0 = blockIdx.x * 16;
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.A), rb = make_rsrc(g.B);
    const int chunks = (g.K + 15) >> 4;
    const int c0 = wave * chunks / kSkinnyWaves, c1 = (wave + 1) * chunks / kSkinnyWaves;
    uint32_t arow[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) arow[m] = 16 * m + li < g.M ? (uint32_t)((16 * m + li) * g.lda) * 4u : kOutOfRange;
    const uint32_t brow = j0 + li < g.N ? (uint32_t)((j0 + li) * g.ldb) * 4u : kOutOfRange;
    f32x4 xa[CH][MB], xb[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) {
        const int k = 16 * (c0 + u) + 4 * q;
        const bool in = c0 + u < c1 && k < g.K;
#pragma unroll
        for (int m = 0; m < MB; ++m)
            xa[u][m] = load_f32x4(ra, in && arow[m] != kOutOfRange ? arow[m] + 4u * k : kOutOfRange);
        xb[u] = load_f32x4(rb, in && brow != kOutOfRange ? brow + 4u * k : kOutOfRange);
    }
    f32x4 acc[MB];
#pragma unroll
    for (int m = 0; m < MB; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < CH; ++u) {
        if (c0 + u >= c1) break;  // wave-uniform
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            // element copies first: bit_cast of an ext-vector element is miscompiled
            const float b = xb[u][e];
#pragma unroll
            for (int m = 0; m < MB; ++m) {
                const float a = xa[u][m][e];
                acc[m] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc[m], 0, 0, 0);
            }
        }
    }
    // lane's acc[m][r] is row 16 m + 4 q + r, column j0 + li
#pragma unroll
    for (int m = 0; m < MB; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float v = acc[m][r];
            part[wave][m][r][lane] = v;
        }
    __syncthreads();
    const int t = threadIdx.x, row = t >> 4, jj = t & 15;
    if (row >= 16 * MB) return;
    const int m = row >> 4, rr = row & 15, src = 16 * (rr >> 2) + jj;
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kSkinnyWaves; ++w) s += part[w][m][rr & 3][src];
    if (row < g.M && j0 + jj < g.N) g.out[(int64_t)row * g.N + j0 + jj] = gemm_finish(g, row, j0 + jj, s);
}

typedef Tile<128, 128, 32, 2, 2> GemmT128;
typedef Tile<64, 64, 32, 2, 2> GemmT64;

// Stream-K launch over batches x tiles x (K / BK) slice iterations.
template <class T, int AK, int BKIND>
static void launch_mfma(GemmArgs& g, int batches, const char* name) {
    auto kernel = gemm_streamk_k<T, AK, BKIND>;
    const size_t lds = (size_t)T::LDS_FLOATS * sizeof(float);
    // once per kernel, thread-safe (C++ static initialisation): the LDS limit
    // and the persistent grid size; -1 if the attribute could not be set
    static const int slots = [&] {
        if (hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
            return -1;
        return resident_groups(kernel, lds);
    }();
    if (slots < 0) return fail(NNC_HIP_EDEVICE, name, "hipFuncSetAttribute failed");
    g.tiles_m = (int)ceil_div(g.M, T::BM);
    g.tiles_n = (int)ceil_div(g.N, T::BN);
    if ((int64_t)g.tiles_m * g.tiles_n * batches >= (1 << 30))
        return fail(NNC_HIP_EUNSUPP, name, "too many output tiles");
    const StreamK sk = plan_streamk(g.tiles_m * g.tiles_n * batches, (int)ceil_div(g.K, T::BK), slots,
                                    fixup_slices<T>());
    if (sk.G < 1) return;
    const size_t ws_bytes = (size_t)sk.G * 2 * T::BM * T::BN * sizeof(float);
    g.ws = workspace(ws_bytes);
    if (!g.ws) return partials_fail(name, ws_bytes);
    static const char* kinds[4] = {"k4", "k1", "x4", "x1"};
    char kname[64];
    snprintf(kname, sizeof kname, "gemm_mfma_%dx%d_%s%s", T::BM, T::BN, kinds[AK], kinds[BKIND]);
    set_work(2.0 * g.M * (double)g.N * g.K * batches, 0.0);
    launch(kname, kernel, dim3(sk.G), dim3(256), lds, g, sk);
    if (sk.needs_fixup()) {
        set_work(0.0, 0.0);
        launch("gemm_streamk_fixup", gemm_fixup_k<T>, dim3(T::BM * T::BN / 1024, sk.sk_tiles), dim3(256), 0, g, sk);
    }
}

// Shared tiles with at most this many partials are finished inside the
// direct-to-LDS kernel by the last workgroup to arrive; tiles split further
// by gemm_fixup_k, which spreads the sum over many workgroups.
static constexpr int kMaxInKernelParts = 4;

// Clears tile counters held in fixed scratch, which keeps whatever the last
// call on the device left there.
__global__ void __launch_bounds__(256) gemm_zero_counters_k(int* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

// LDS stages of the direct-to-LDS kernel: 64x64 tiles have short slices
// (16 MFMAs per wave) and keep three slices in flight; 128x128 tiles one
template <class T>
constexpr int dma_stages() {
    return T::BM * T::BN < 128 * 128 ? 4 : 2;
}

// Direct-to-LDS stream-K launch; OA / OB: KcOperand or XcOperand.
// 64x64 tiles over 16 or more K slices run one workgroup per CU: whole
// tiles then need no partials (Gemm 1024^3 on MI355X: 29.5 us against
// 33.6 us with two workgroups per CU, each tile split in two and finished
// in-kernel, and 33.5 us with the separate fixup kernel); over fewer slices
// the second workgroup per CU hides the tile's load latency (1024x768x256:
// 10.3 against 11.3 us).
template <class T, class OA, class OB>
static void launch_gemm_dma(GemmArgs& g, int batches, const char* name, const char* kname) {
    constexpr int NS = dma_stages<T>();
    auto kernel = gemm_dma_k<T, NS, OA, OB, true>;
    const size_t lds = (size_t)GemmDma<T, NS>::LDS_FLOATS * sizeof(float);
    // once per kernel, thread-safe (C++ static initialisation): the LDS limit
    // and the persistent grid size; -1 if the attribute could not be set
    static const int slots = [&] {
        if (hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
            return -1;
        return resident_groups(kernel, lds, T::THREADS);
    }();
    if (slots < 0) return fail(NNC_HIP_EDEVICE, name, "hipFuncSetAttribute failed");
    g.tiles_m = (int)ceil_div(g.M, T::BM);
    g.tiles_n = (int)ceil_div(g.N, T::BN);
    if ((int64_t)g.tiles_m * g.tiles_n * batches >= (1 << 30))
        return fail(NNC_HIP_EUNSUPP, name, "too many output tiles");
    const int iters = (int)ceil_div(g.K, T::BK);
    const int use_slots = (T::BM * T::BN < 128 * 128 && iters >= 16) ? std::min(slots, cu_count()) : slots;
    const StreamK sk = plan_streamk(g.tiles_m * g.tiles_n * batches, iters, use_slots, fixup_slices<T>());
    if (sk.G < 1) return;
    const size_t ws_bytes = (size_t)sk.G * 2 * T::BM * T::BN * sizeof(float);
    g.ws = workspace(ws_bytes);
    if (!g.ws) return partials_fail(name, ws_bytes);
    const int64_t per = sk.total() / sk.G;  // slices per workgroup range (>= 1)
    const bool in_kernel = sk.needs_fixup() && (sk.iters + per - 1) / per + 1 <= kMaxInKernelParts;
    g.cnt = in_kernel ? tile_counters((size_t)sk.sk_tiles) : nullptr;
    if (g.cnt && ts().fixed)
        launch("zero_tile_counters", gemm_zero_counters_k, dim3((unsigned)ceil_div(sk.sk_tiles, 256)), dim3(256), 0,
               g.cnt, (int)sk.sk_tiles);
    set_work(2.0 * g.M * (double)g.N * g.K * batches, 0.0);
    launch(kname, kernel, dim3(sk.G), dim3(T::THREADS), lds, g, sk);
    if (sk.needs_fixup() && !g.cnt) {
        set_work(0.0, 0.0);
        launch("gemm_streamk_fixup", gemm_fixup_k<T>, dim3(T::BM * T::BN / 1024, sk.sk_tiles), dim3(256), 0, g, sk);
    }
}

template <class T, bool A_KC, bool B_KC>
static void launch_gemm_dma_kinds(GemmArgs& g, int batches, const char* name) {
    typedef typename std::conditional<A_KC, KcOperand<T, T::BM, 0>, XcOperand<T, T::BM, 0>>::type OA;
    typedef typename std::conditional<B_KC, KcOperand<T, T::BN, T::BM * 32>, XcOperand<T, T::BN, T::BM * 32>>::type
        OB;
    char kname[64];
    snprintf(kname, sizeof kname, "gemm_dma_%dx%d_%s%s", T::BM, T::BN, A_KC ? "k4" : "x4", B_KC ? "k4" : "x4");
    launch_gemm_dma<T, OA, OB>(g, batches, name, kname);
}

template <class T>
static void dispatch_dma(GemmArgs& g, bool a_kc, bool b_kc, int batches, const char* name) {
    if (a_kc && b_kc) return launch_gemm_dma_kinds<T, true, true>(g, batches, name);
    if (a_kc) return launch_gemm_dma_kinds<T, true, false>(g, batches, name);
    if (b_kc) return launch_gemm_dma_kinds<T, false, true>(g, batches, name);
    return launch_gemm_dma_kinds<T, false, false>(g, batches, name);
}

template <int AK, int BKIND>
static void launch_mfma_small(GemmArgs& g, int batches, const char* name) {
    launch_mfma<GemmT64, AK, BKIND>(g, batches, name);
}

template <int AK>
static void dispatch_b_small(GemmArgs& g, int bkind, int batches, const char* name) {
    switch (bkind) {
        case kKC4: return launch_mfma_small<AK, kKC4>(g, batches, name);
        case kKC: return launch_mfma_small<AK, kKC>(g, batches, name);
        case kXC4: return launch_mfma_small<AK, kXC4>(g, batches, name);
        default: return launch_mfma_small<AK, kXC>(g, batches, name);
    }
}

// ---------------------------------------------------------------------------
// Short GEMMs: gemm_ws_k, the GEMM form of conv.hip's conv_ws_k. A
// workgroup owns one 32 x 32 output tile of one batch over a contiguous
// range of K slices; its four waves split the range (wave w takes slices w,
// w + 4, ...), each computing the whole tile with v_mfma_f32_32x32x2_f32, and
// the four sums are added through LDS in wave order. Operands go straight
// into the MFMA operand registers: lane half h takes k = 16h .. 16h + 15 of
// each 32-wide slice, so a k-contiguous operand row is four 16-byte loads
// per slice and an x-contiguous one sixteen 4-byte loads coalesced across
// the lanes' rows. All of a wave's slices (NS) are loaded before its first
// MFMA. A tile split over S workgroups is finished in the kernel by the last
// to arrive (store_partial4 / finish_arrive / load_partial4, the stream-K
// protocol of mfma_tile.h), the partials added in range order. Epilogue as
// gemm_finish.
// ---------------------------------------------------------------------------
typedef unsigned int gws_u32x4 __attribute__((ext_vector_type(4)));

template <int NS, bool A_KC, bool B_KC>
__global__ void __launch_bounds__(256, 2) gemm_ws_k(GemmArgs g, int S, int iters, int tiles) {
    __shared__ __align__(16) float red[4][32 * 32];
    const int lane = threadIdx.x & 63, h = lane >> 5, l32 = lane & 31;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int part = blockIdx.x % S, rest = blockIdx.x / S;
    const int t = rest % tiles, batch = rest / tiles;
    const int i0 = (t % g.tiles_m) * 32, j0 = (t / g.tiles_m) * 32;
    const int kb = (int)((int64_t)part * iters / S), ke = (int)((int64_t)(part + 1) * iters / S);
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(g.A + batch * g.sa), rb = make_rsrc(g.B + batch * g.sb);
    const int i = i0 + l32, j = j0 + l32;
    const bool iok = i < g.M, jok = j < g.N;
    const int lda = (int)g.lda, ldb = (int)g.ldb;

    // The C values of this thread's four outputs after the reduction below
    // (tile row t / 8, columns 4 (t % 8) ..), loaded ahead of the operands,
    // so the epilogue waits for no load (a split tile's finish for its
    // partials only): straight-line buffer loads from C's one base, the row
    // chosen once (C[j] or C[oi*N + j]; per element through gemm_finish,
    // hipcc 7.2 addressed elements 1..3 of a bias row at C + oi*N, past the
    // end of C), out-of-range offsets reading 0. A branch around per-element
    // loads, or loads between the operands', rescheduled the operand loads.
    // The epilogue loads C itself where its offsets would not fit 32 bits
    // (never within this kernel's 1 GFLOP limit).
    const int row = threadIdx.x >> 3, c4 = (threadIdx.x & 7) * 4;
    const int oi = i0 + row;
    const bool has_c = g.c_mode != 0;
    const bool pre_c = has_c && (int64_t)g.M * g.N < ((int64_t)1 << 29);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(g.C);
    const uint32_t crow = g.c_mode == 2 ? (uint32_t)oi * (uint32_t)g.N : 0u;
    float cv[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int oj = j0 + c4 + e;
        cv[e] = load_f32(rc, pre_c && oi < g.M && oj < g.N ? (crow + (uint32_t)oj) * 4u : kOutOfRange);
    }

    float av[NS][16], bv[NS][16];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const int sl = kb + wave + 4 * q;  // wave-uniform
        const bool on = sl < ke;
        const int k0 = sl * 32 + 16 * h;
        if constexpr (A_KC) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool ok = on && iok && k0 + 4 * u < g.K;
                const f32x4 v = load_f32x4(ra, ok ? (uint32_t)(i * lda + k0 + 4 * u) * 4u : kOutOfRange);
                av[q][4 * u] = v[0], av[q][4 * u + 1] = v[1], av[q][4 * u + 2] = v[2], av[q][4 * u + 3] = v[3];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const bool ok = on && iok && k0 + c < g.K;
                av[q][c] = load_f32(ra, ok ? (uint32_t)((k0 + c) * lda + i) * 4u : kOutOfRange);
            }
        }
        if constexpr (B_KC) {
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bool ok = on && jok && k0 + 4 * u < g.K;
                const f32x4 v = load_f32x4(rb, ok ? (uint32_t)(j * ldb + k0 + 4 * u) * 4u : kOutOfRange);
                bv[q][4 * u] = v[0], bv[q][4 * u + 1] = v[1], bv[q][4 * u + 2] = v[2], bv[q][4 * u + 3] = v[3];
            }
        } else {
#pragma unroll
            for (int c = 0; c < 16; ++c) {
                const bool ok = on && jok && k0 + c < g.K;
                bv[q][c] = load_f32(rb, ok ? (uint32_t)((k0 + c) * ldb + j) * 4u : kOutOfRange);
            }
        }
    }
    // every load above is issued before the first MFMA (a wave with fewer
    // slices multiplies zeros in its last one: straight-line code)
    __builtin_amdgcn_sched_barrier(0);
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int c = 0; c < 16; ++c) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][c], bv[q][c], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float x = acc[r];  // (element copied first: see store_tile)
        red[wave][(8 * (r >> 2) + 4 * h + (r & 3)) * 32 + l32] = x;
    }
    __syncthreads();
    f32x4 v = *reinterpret_cast<const f32x4*>(&red[0][row * 32 + c4]);
#pragma unroll
    for (int w = 1; w < 4; ++w) v += *reinterpret_cast<const f32x4*>(&red[w][row * 32 + c4]);
    if (S > 1) {
        const __amdgpu_buffer_rsrc_t rws = make_rsrc(g.ws);
        const uint32_t slot = (uint32_t)rest * (uint32_t)S * 4096u + threadIdx.x * 16u;
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(gws_u32x4, v), rws,
                                               (int)(slot + (uint32_t)part * 4096u), 0, kDeviceScope);
        if (!finish_arrive(g.cnt + rest, S - 1)) return;  // uniform
        f32x4 p[kWsMaxSplit];
#pragma unroll
        for (int q = 0; q < kWsMaxSplit; ++q)
            p[q] = load_partial4(rws, q < S && q != part ? slot + (uint32_t)q * 4096u : kOutOfRange);
        f32x4 sum = part == 0 ? v : p[0];
#pragma unroll
        for (int q = 1; q < kWsMaxSplit; ++q)
            if (q < S) sum += q == part ? v : p[q];
        v = sum;
    }
    if (oi >= g.M) return;
    float* o = g.out + batch * g.so + (int64_t)oi * g.N;
    if (has_c && !pre_c) {
        const float* cr = g.C + (g.c_mode == 2 ? (int64_t)oi * g.N : (int64_t)0);
#pragma unroll
        for (int e = 0; e < 4; ++e) cv[e] = j0 + c4 + e < g.N ? cr[j0 + c4 + e] : 0.f;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int oj = j0 + c4 + e;
        if (oj < g.N) {
            float x = g.alpha * v[e];
            if (has_c) x += g.beta * cv[e];
            if (g.relu) x = x > 0.0f ? x : 0.0f;
            o[oj] = x;
        }
    }
}

template <int NS, bool A_KC, bool B_KC>
static void launch_gws_ns(const GemmArgs& g, int S, int iters, int tiles, unsigned grid, const char* kname) {
    launch(kname, gemm_ws_k<NS, A_KC, B_KC>, dim3(grid), dim3(256), 0, g, S, iters, tiles);
}

template <bool A_KC, bool B_KC>
static void launch_gws(const GemmArgs& g, int NS, int S, int iters, int tiles, unsigned grid, const char* kname) {
    switch (NS) {
        case 1: return launch_gws_ns<1, A_KC, B_KC>(g, S, iters, tiles, grid, kname);
        case 2: return launch_gws_ns<2, A_KC, B_KC>(g, S, iters, tiles, grid, kname);
        case 3: return launch_gws_ns<3, A_KC, B_KC>(g, S, iters, tiles, grid, kname);
        default: return launch_gws_ns<4, A_KC, B_KC>(g, S, iters, tiles, grid, kname);  // NS <= kGwsMaxSlices
    }
}

// Describe operands as: A element (i, k) = A[i*lda + k] if a_kc else A[k*lda + i];
// B element (k, j) = B[j*ldb + k] if b_kc else B[k*ldb + j].
struct GemmProblem {
    const float* A;
    const float* B;
    const float* C;
    float* out;
    int M, N, K, batches;
    int64_t lda, ldb, sa, sb, so;
    bool a_kc, b_kc;
    float alpha, beta;
    int c_mode, relu;
};

static void gemm_run(const GemmProblem& p, const char* name) {
    if (p.M <= 0 || p.N <= 0 || p.batches <= 0) return;
    GemmArgs g{};
    g.A = p.A;
    g.B = p.B;
    g.C = p.C;
    g.out = p.out;
    g.M = p.M;
    g.N = p.N;
    g.K = p.K;
    g.lda = p.lda;
    g.ldb = p.ldb;
    g.sa = p.sa;
    g.sb = p.sb;
    g.so = p.so;
    g.alpha = p.alpha;
    g.beta = p.beta;
    g.c_mode = p.c_mode;
    g.relu = p.relu;
    g.splits = 1;
    g.out32 = (int64_t)p.M * p.N * 4 < ((int64_t)1 << 31);
    if (p.K <= 0) {
        // empty contraction: out = beta*C (alpha*0)
        GemmArgs z = g;
        z.K = 0;
        z.ws = nullptr;
        // reuse the dot kernel with K = 0
        launch(name, dot_k<false>, dim3((unsigned)ceil_div((int64_t)p.M * p.N, 4)), dim3(256), 0, z);
        return;
    }
    if (p.batches == 1 && p.M == 1 && !p.b_kc) {
        // one output row, B row-major: stream B once
        const int64_t a_stride = p.a_kc ? 1 : p.lda;
        const bool vec = aligned16(p.B) && p.ldb % 4 == 0 && p.N % 4 == 0;
        if (vec) {
            // one launch, the K splits finished in the kernel (gemv_fin_k):
            // about four workgroups per CU, at most kGemvMaxSplits splits
            const int col_blocks = (int)ceil_div(p.N, 64);
            int S = (int)ceil_div(4 * cu_count(), col_blocks);
            if (S > kGemvMaxSplits) S = kGemvMaxSplits;
            if (S > p.K) S = p.K;
            if (S < 1) S = 1;
            const int k_per = (int)ceil_div(p.K, S);
            S = (int)ceil_div(p.K, k_per);
            bool ok = true;
            if (S > 1) {
                g.ws = workspace((size_t)col_blocks * S * 256);
                g.cnt = g.ws ? tile_counters((size_t)col_blocks) : nullptr;
                ok = g.cnt != nullptr;
                if (ok && ts().fixed)
                    launch("zero_tile_counters", gemm_zero_counters_k, dim3((unsigned)ceil_div(col_blocks, 256)),
                           dim3(256), 0, g.cnt, col_blocks);
            }
            if (ok) {
                set_work(2.0 * p.K * (double)p.N, 4.0 * ((double)p.K * p.N + p.K + p.N));
                launch("gemv_v4", gemv_fin_k<8>, dim3(col_blocks, S), dim3(256), 0, g, a_stride, S, k_per);
                return;
            }
            g.ws = nullptr;
            g.cnt = nullptr;
        }
        const int cols_per_block = vec ? 1024 : 256;
        const int col_blocks = (int)ceil_div(p.N, cols_per_block);
        int splits = (int)ceil_div(4 * cu_count(), col_blocks);
        const int max_by_k = (int)ceil_div(p.K, 16);
        if (splits > max_by_k) splits = max_by_k;
        if (splits < 1) splits = 1;
        float* ws = workspace((size_t)splits * p.N * sizeof(float));
        if (!ws) return fail(NNC_HIP_ENOMEM, name, "workspace");
        const int k_per = (int)ceil_div(p.K, splits);
        splits = (int)ceil_div(p.K, k_per);
        g.ws = ws;
        g.splits = splits;
        set_work(2.0 * p.K * (double)p.N, 4.0 * ((double)p.K * p.N + p.K + (double)p.N * splits));
        if (vec)
            launch("gemv_xc_v4", gemv_xc_k<true>, dim3(col_blocks, splits), dim3(256), 0, p.A, a_stride, p.B,
                   p.ldb, ws, p.N, p.K, k_per);
        else
            launch("gemv_xc_s1", gemv_xc_k<false>, dim3(col_blocks, splits), dim3(256), 0, p.A, a_stride,
                   p.B, p.ldb, ws, p.N, p.K, k_per);
        set_work(0.0, 4.0 * (double)p.N * (splits + 1));
        launch("gemv_reduce", gemv_reduce_k, dim3((unsigned)ceil_div(p.N, 64)), dim3(256), 0, g);
        return;
    }
    if (p.batches == 1 && p.a_kc && p.b_kc && (p.M == 1 || p.N == 1 || (int64_t)p.M * p.N <= 64)) {
        const bool vec = aligned16(p.A) && aligned16(p.B) && p.lda % 4 == 0 && p.ldb % 4 == 0;
        const dim3 grid((unsigned)ceil_div((int64_t)p.M * p.N, 4));
        set_work(2.0 * p.M * (double)p.N * p.K, 4.0 * ((double)p.M * p.K + (double)p.N * p.K + (double)p.M * p.N));
        if (vec) launch("dot_rows_v4", dot_k<true>, grid, dim3(256), 0, g);
        else launch("dot_rows_s1", dot_k<false>, grid, dim3(256), 0, g);
        return;
    }
    if (p.batches == 1 && p.a_kc && p.b_kc && p.M <= kSkinnyRows && p.K <= kSkinnyMaxK && p.K % 4 == 0 &&
        aligned16(p.A) && aligned16(p.B) && p.lda % 4 == 0 && p.ldb % 4 == 0 &&
        (int64_t)p.M * p.lda * 4 < ((int64_t)1 << 31) && (int64_t)p.N * p.ldb * 4 < ((int64_t)1 << 31)) {
        const dim3 grid((unsigned)ceil_div(p.N, 16)), block(64 * kSkinnyWaves);
        set_work(2.0 * p.M * (double)p.N * p.K, 0.0);
        if (p.M <= 16) launch("gemm_skinny_nt_16", gemm_skinny_nt_k<1>, grid, block, 0, g);
        else launch("gemm_skinny_nt_32", gemm_skinny_nt_k<2>, grid, block, 0, g);
        return;
    }
    // short products: gemm_ws_k, where plan_gemm_ws takes them and each
    // operand is either k-contiguous with 16-byte rows (and K % 4 == 0) or
    // x-contiguous, one batch of each below 2 GiB (32-bit buffer offsets)
    {
        WsPlan wp;
        const bool a_kc4 = p.a_kc && aligned16(p.A) && p.lda % 4 == 0 && p.sa % 4 == 0 && p.K % 4 == 0;
        const bool b_kc4 = p.b_kc && aligned16(p.B) && p.ldb % 4 == 0 && p.sb % 4 == 0 && p.K % 4 == 0;
        const int64_t a_elems = p.a_kc ? (int64_t)p.M * p.lda : (int64_t)p.K * p.lda;
        const int64_t b_elems = p.b_kc ? (int64_t)p.N * p.ldb : (int64_t)p.K * p.ldb;
        if ((a_kc4 || !p.a_kc) && (b_kc4 || !p.b_kc) && a_elems * 4 < ((int64_t)1 << 31) &&
            b_elems * 4 < ((int64_t)1 << 31) && plan_gemm_ws(p.M, p.N, p.K, p.batches, wp)) {
            g.tiles_m = (int)ceil_div(p.M, 32);
            g.tiles_n = (int)ceil_div(p.N, 32);
            const int tiles = g.tiles_m * g.tiles_n;
            bool ok = true;
            if (wp.S > 1) {
                g.ws = workspace((size_t)wp.tiles * wp.S * 4096);
                g.cnt = g.ws ? tile_counters((size_t)wp.tiles) : nullptr;
                ok = g.cnt != nullptr;
                if (ok && ts().fixed)
                    launch("zero_tile_counters", gemm_zero_counters_k, dim3((unsigned)ceil_div(wp.tiles, 256)),
                           dim3(256), 0, g.cnt, (int)wp.tiles);
            }
            if (ok) {
                char kname[48];
                snprintf(kname, sizeof kname, "gemm_ws_32x32_%s%s", p.a_kc ? "k4" : "x1", p.b_kc ? "k4" : "x1");
                set_work(2.0 * p.M * (double)p.N * p.K * p.batches, 0.0);
                const unsigned grid = (unsigned)(wp.tiles * wp.S);
                if (p.a_kc && p.b_kc) launch_gws<true, true>(g, wp.NS, wp.S, wp.iters, tiles, grid, kname);
                else if (p.a_kc) launch_gws<true, false>(g, wp.NS, wp.S, wp.iters, tiles, grid, kname);
                else if (p.b_kc) launch_gws<false, true>(g, wp.NS, wp.S, wp.iters, tiles, grid, kname);
                else launch_gws<false, false>(g, wp.NS, wp.S, wp.iters, tiles, grid, kname);
                return;
            }
            g.ws = nullptr;
            g.cnt = nullptr;
        }
    }
    // MFMA tiles address each operand tile with 32-bit byte offsets from the
    // tile origin: at most 128 rows of lda (k-contiguous) or K rows of lda
    // (x-contiguous).
    const int64_t a_span = p.a_kc ? 128 * p.lda + p.K : (int64_t)p.K * p.lda + 128;
    const int64_t b_span = p.b_kc ? 128 * p.ldb + p.K : (int64_t)p.K * p.ldb + 128;
    if (a_span * 4 >= ((int64_t)1 << 31) || b_span * 4 >= ((int64_t)1 << 31))
        return fail(NNC_HIP_EUNSUPP, name, "operand tile spans 2 GiB or more");
    // 16-byte loads need 4-float alignment of every row/batch start.
    const bool a_al = aligned16(p.A) && p.lda % 4 == 0 && p.sa % 4 == 0;
    const bool b_al = aligned16(p.B) && p.ldb % 4 == 0 && p.sb % 4 == 0;
    // (the x-contiguous 16-byte loader also needs the row length M or N to be
    // a multiple of 4)
    const int akind = p.a_kc ? ((a_al && p.K % 4 == 0) ? kKC4 : kKC) : ((a_al && p.M % 4 == 0) ? kXC4 : kXC);
    const int bkind = p.b_kc ? ((b_al && p.K % 4 == 0) ? kKC4 : kKC) : ((b_al && p.N % 4 == 0) ? kXC4 : kXC);
    const bool big = (int64_t)p.M * p.N * p.batches >= (int64_t)128 * 128 * 2 * cu_count() / 4 &&
                     p.M >= 128 && p.N >= 128;
    // 16-byte rows on both sides: direct-to-LDS staging
    if ((akind == kKC4 || akind == kXC4) && (bkind == kKC4 || bkind == kXC4)) {
        if (big) return dispatch_dma<GemmT128>(g, akind == kKC4, bkind == kKC4, p.batches, name);
        return dispatch_dma<GemmT64>(g, akind == kKC4, bkind == kKC4, p.batches, name);
    }
    switch (akind) {
        case kKC4: return dispatch_b_small<kKC4>(g, bkind, p.batches, name);
        case kKC: return dispatch_b_small<kKC>(g, bkind, p.batches, name);
        case kXC4: return dispatch_b_small<kXC4>(g, bkind, p.batches, name);
        default: return dispatch_b_small<kXC>(g, bkind, p.batches, name);
    }
}

static bool args_ok(const char* name, Tensor* a, Tensor* b, Tensor* out) {
    if (!ready(name)) return false;
    if (!has_data(a) || !has_data(b) || !has_data(out)) {
        fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
        return false;
    }
    return true;
}

static void matmul_impl(Tensor* a, Tensor* b, Tensor* bias, Tensor* out, int relu, const char* name) {
    if (!args_ok(name, a, b, out)) return;
    GemmProblem p{};
    p.A = (const float*)a->data;
    p.B = (const float*)b->data;
    p.out = (float*)out->data;
    p.alpha = 1.f;
    p.beta = 1.f;
    p.relu = relu;
    p.batches = 1;
    const int an = a->ndim, bn = b->ndim, on = out->ndim;
    if (an == 2 && bn == 2) {
        p.M = (int)a->shape[0];
        p.K = (int)a->shape[1];
        p.N = (int)b->shape[1];
        if (b->shape[0] != p.K) return fail(NNC_HIP_EINVAL, name, "inner dimensions differ");
        p.lda = p.K;
        p.ldb = p.N;
        p.a_kc = true;
        p.b_kc = false;
    } else if (an == 1 && bn == 2) {
        p.M = 1;
        p.K = (int)a->shape[0];
        p.N = (int)b->shape[1];
        if (b->shape[0] != p.K) return fail(NNC_HIP_EINVAL, name, "inner dimensions differ");
        p.lda = p.K;
        p.ldb = p.N;
        p.a_kc = true;
        p.b_kc = false;
    } else if (an == 2 && bn == 1) {
        p.M = (int)a->shape[0];
        p.K = (int)a->shape[1];
        p.N = 1;
        if (b->shape[0] != p.K) return fail(NNC_HIP_EINVAL, name, "inner dimensions differ");
        p.lda = p.K;
        p.ldb = p.K;  // the vector as one k-contiguous column
        p.a_kc = true;
        p.b_kc = true;
    } else if (an >= 2 && bn >= 2) {
        p.M = (int)out->shape[on - 2];
        p.N = (int)out->shape[on - 1];
        p.K = (int)a->shape[an - 1];
        if (a->shape[an - 2] != p.M || b->shape[bn - 2] != p.K || b->shape[bn - 1] != p.N)
            return fail(NNC_HIP_EINVAL, name, "matrix dimensions do not match the output");
        const int64_t batches = prod(out->shape, 0, on - 2);
        const int64_t abat = prod(a->shape, 0, an - 2), bbat = prod(b->shape, 0, bn - 2);
        if ((abat != batches && abat != 1) || (bbat != batches && bbat != 1))
            return fail(NNC_HIP_EUNSUPP, name, "batch broadcast other than full or none");
        if (batches >= 65536) return fail(NNC_HIP_EUNSUPP, name, "more than 65535 batches");
        p.batches = (int)batches;
        p.lda = p.K;
        p.ldb = p.N;
        p.sa = abat == 1 ? 0 : (int64_t)p.M * p.K;
        p.sb = bbat == 1 ? 0 : (int64_t)p.K * p.N;
        p.so = (int64_t)p.M * p.N;
        p.a_kc = true;
        p.b_kc = false;
    } else {
        return;  // the reference computes nothing for other ranks
    }
    if (bias && bias->data) {
        const int64_t bn = numel(bias);
        p.C = (const float*)bias->data;
        if (bn == p.N) p.c_mode = 1;
        else if (bn == (int64_t)p.M * p.N) p.c_mode = 2;
        else return fail(NNC_HIP_EINVAL, name, "bias must have N or M*N elements");
    }
    gemm_run(p, name);
}

}  // namespace nnc

using namespace nnc;

extern "C" {

void nnc_matmul(Tensor* a, Tensor* b, Tensor* out) { matmul_impl(a, b, nullptr, out, 0, "nnc_matmul"); }

// Emitted by the reference code generator as (a, b, bias or NULL, out)
// (c_emitter.py:1143-1171); relu(a @ b + bias).
void nnc_matmul_relu(Tensor* a, Tensor* b, Tensor* bias, Tensor* out) {
    matmul_impl(a, b, bias, out, 1, "nnc_matmul_relu");
}

// ops.c:1732-1841: dimension logic of the reference, including its 1-D cases.
void nnc_gemm(Tensor* a, Tensor* b, Tensor* c, Tensor* out, float alpha, float beta, int ta, int tb) {
    const char* name = "nnc_gemm";
    if (!args_ok(name, a, b, out)) return;
    GemmProblem p{};
    p.A = (const float*)a->data;
    p.B = (const float*)b->data;
    p.out = (float*)out->data;
    p.alpha = alpha;
    p.beta = beta;
    p.batches = 1;
    if (a->ndim == 2 && b->ndim == 2) {
        p.M = (int)(ta ? a->shape[1] : a->shape[0]);
        p.K = (int)(ta ? a->shape[0] : a->shape[1]);
        p.N = (int)(tb ? b->shape[0] : b->shape[1]);
    } else if (a->ndim == 1 && b->ndim == 2) {
        p.M = 1;
        p.K = (int)a->shape[0];
        p.N = (int)b->shape[1];
        ta = 0;
    } else if (a->ndim == 2 && b->ndim == 1) {
        p.M = (int)a->shape[0];
        p.K = (int)a->shape[1];
        p.N = 1;
        tb = 0;
    } else {
        // the reference's flatten fallback reads B outside its buffer
        return fail(NNC_HIP_EUNSUPP, name, "operand ranks %d x %d", a->ndim, b->ndim);
    }
    if (numel(a) < (int64_t)p.M * p.K || numel(b) < (int64_t)p.K * p.N)
        return fail(NNC_HIP_EINVAL, name, "operand smaller than M*K or K*N");
    p.a_kc = !ta;
    p.lda = ta ? p.M : p.K;
    p.b_kc = tb != 0;
    p.ldb = tb ? p.K : p.N;
    if (c && c->data) {
        p.C = (const float*)c->data;
        p.c_mode = c->ndim == 1 ? 1 : 2;
        if (numel(c) < (p.c_mode == 1 ? p.N : (int64_t)p.M * p.N))
            return fail(NNC_HIP_EINVAL, name, "C smaller than the output");
    }
    if (numel(out) < (int64_t)p.M * p.N) return fail(NNC_HIP_EINVAL, name, "output too small");
    gemm_run(p, name);
}

// ops.c:1843-1886: B stored [N, K].
void nnc_gemm_nt(Tensor* a, Tensor* b, Tensor* c, Tensor* out, float alpha, float beta) {
    const char* name = "nnc_gemm_nt";
    if (!args_ok(name, a, b, out)) return;
    GemmProblem p{};
    p.A = (const float*)a->data;
    p.B = (const float*)b->data;
    p.out = (float*)out->data;
    p.alpha = alpha;
    p.beta = beta;
    p.batches = 1;
    if (a->ndim == 2 && b->ndim == 2) {
        p.M = (int)a->shape[0];
        p.K = (int)a->shape[1];
        p.N = (int)b->shape[0];
    } else if (a->ndim == 1 && b->ndim == 2) {
        p.M = 1;
        p.K = (int)a->shape[0];
        p.N = (int)b->shape[0];
    } else {
        p.M = 1;
        p.K = (int)numel(a);
        p.N = b->ndim == 2 ? (int)b->shape[0] : (int)numel(b);
    }
    if (numel(b) < (int64_t)p.N * p.K) return fail(NNC_HIP_EINVAL, name, "B smaller than N*K");
    p.a_kc = true;
    p.lda = p.K;
    p.b_kc = true;
    p.ldb = p.K;
    if (c && c->data) {
        p.C = (const float*)c->data;
        p.c_mode = c->ndim == 1 ? 1 : 2;
        if (numel(c) < (p.c_mode == 1 ? p.N : (int64_t)p.M * p.N))
            return fail(NNC_HIP_EINVAL, name, "C smaller than the output");
    }
    if (numel(out) < (int64_t)p.M * p.N) return fail(NNC_HIP_EINVAL, name, "output too small");
    gemm_run(p, name);
}

}  // extern "C"
