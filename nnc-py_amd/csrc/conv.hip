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
// input rows. D's 32x32 MFMA layout puts consecutive pixels in consecutive
// lanes, so the NCHW stores coalesce too. Bias and the fused activation are
// applied in the epilogue (or in the stream-K fixup for shared tiles).
//
// Padding follows the reference: only the top/left pads are arguments, the
// bottom/right extent comes from the output shape (c_emitter.py:1051-1058).
//
// Accumulation: one fp32 MFMA chain per workgroup segment (K <= 4608 at
// ResNet-18 scale stays inside 1e-4 abs / 1e-3 rel of the reference's fp64
// sum); shared tiles add their segments in fixed workgroup order.
#include <math.h>
#include <stdlib.h>

#include <algorithm>

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
    const float* res;  // residual added before the activation (nullable)
    float* out;
    float* ws;  // stream-K partial tiles
    int* cnt;   // stream-K tile arrival counters (nullptr: conv_fixup_k finishes shared tiles)
    int N, Ci, H, W, Co, Ho, Wo, kh, kw, sh, sw, ph, pw;
    int K, Npix, act;
    int ldw;  // weight row stride in floats (packed weights may pad K)
    int tiles_m, tiles_n;
    int vec_out;  // out (and res) 16-byte aligned: the fixup may store float4
    int out32;    // output (and residual) below 2 GiB: whole tiles use 32-bit buffer offsets
    // 1x1 projection folded into the contraction (nnc_hip_conv_proj): input
    // [N][pci][pH][pW] read at (oh * psh, ow * psw); its weights are the last
    // pci of each packed weight row
    const float* pin;
    int pci, pH, pW, psh, psw;
};

// B operand: gathers input taps for X consecutive output pixels; each thread
// takes one pixel and a run of KRUN consecutive k, so loads coalesce across
// lanes (consecutive pixels) and the run is written to LDS as 16-byte
// stores. k -> (ci, tap) is decomposed once per slice and then stepped. KH/KW
// > 0 fix the kernel size at compile time; then the taps inside the image
// are a per-tile bit mask. Buffer loads over the whole input tensor (byte
// offsets < 2^31, checked on the host); out-of-image taps get an
// out-of-range offset and read 0.
template <int X, int BK, int LD, int KH, int KW>
struct ConvGather {
    static constexpr int KRUN = X * BK / 256;
    static constexpr bool MASK = KH > 0 && KH * KW <= 64;
    static_assert(256 % X == 0 && KRUN % 4 == 0, "gather shape");
    __amdgpu_buffer_rsrc_t rsrc;
    int pix_off, h0, w0, H, W, K, kw_rt, khw_rt, HW;
    uint64_t taps;  // bit t: tap t of this pixel is inside the image (MASK)
    bool valid;
    int xx, kbase;
    float v[KRUN];

    __device__ void init(const ConvArgs& a, int j0) {
        xx = threadIdx.x % X;
        kbase = (threadIdx.x / X) * KRUN;
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
        HW = a.H * a.W;
        K = a.K;
        kw_rt = a.kw;
        khw_rt = a.kh * a.kw;
        pix_off = n * a.Ci * HW + h0 * W + w0;  // element offset of tap (0, 0), channel 0
        rsrc = make_rsrc(a.in);
        taps = 0;
        if constexpr (MASK) {
#pragma unroll
            for (int r = 0; r < KH; ++r)
#pragma unroll
                for (int c = 0; c < KW; ++c) {
                    const bool in = valid && (unsigned)(h0 + r) < (unsigned)H && (unsigned)(w0 + c) < (unsigned)W;
                    taps |= (uint64_t)in << (r * KW + c);
                }
        }
    }
    __device__ void load(int k0) {
        const int khw = KH > 0 ? KH * KW : khw_rt;
        const int kwid = KW > 0 ? KW : kw_rt;
        const int kstart = k0 + kbase;
        int ci = kstart / khw;
        int t = kstart - ci * khw;
#pragma unroll
        for (int p = 0; p < KRUN; ++p) {
            const int r = t / kwid;
            const int c = t - r * kwid;
            bool ok;
            if constexpr (MASK)
                ok = ((taps >> t) & 1) != 0;
            else
                ok = valid && (unsigned)(h0 + r) < (unsigned)H && (unsigned)(w0 + c) < (unsigned)W;
            ok = ok && kstart + p < K;
            v[p] = load_f32(rsrc, ok ? (uint32_t)(pix_off + ci * HW + r * W + c) * 4u : kOutOfRange);
            // step to k + 1
            ++t;
            const bool wrap = t == khw;
            t = wrap ? 0 : t;
            ci += wrap ? 1 : 0;
        }
    }
    __device__ void store(float* S) const {
#pragma unroll
        for (int p = 0; p < KRUN; p += 4) lds_store4(S + xx * LD + kbase + p, v[p], v[p + 1], v[p + 2], v[p + 3]);
    }
};

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Bias (+ residual) + act for 4 consecutive output pixels p0..p0+3 of
// channel co (one row of a tile), float4 when they are in one image and the
// output (and residual) are 16-byte aligned. Split into the loads
// (fixup_load) and the arithmetic and stores (fixup_apply), so a thread
// finishing several rows issues all its loads before its first store: the
// compiler cannot move a load above a store that may alias it.
struct FixupIn {
    float b;
    float4 r;
};

__device__ __forceinline__ bool fixup_vec(const ConvArgs& a, int p0) {
    return a.vec_out && ((a.Ho * a.Wo) & 3) == 0 && p0 + 3 < a.Npix;
}

__device__ __forceinline__ FixupIn fixup_load(const ConvArgs& a, int co, int p0) {
    const int hw = a.Ho * a.Wo;
    FixupIn f;
    f.b = a.bias ? a.bias[co] : 0.f;
    f.r = make_float4(0.f, 0.f, 0.f, 0.f);
    if (!a.res) return f;
    if (fixup_vec(a, p0)) {
        const int n = p0 / hw;
        f.r = *reinterpret_cast<const float4*>(a.res + ((int64_t)n * a.Co + co) * hw + (p0 - n * hw));
        return f;
    }
    float r[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int pix = p0 + q;
        if (pix >= a.Npix) break;
        const int nq = pix / hw;
        r[q] = a.res[((int64_t)nq * a.Co + co) * hw + (pix - nq * hw)];
    }
    f.r = make_float4(r[0], r[1], r[2], r[3]);
    return f;
}

__device__ __forceinline__ void fixup_apply(const ConvArgs& a, int co, int p0, float4 v, const FixupIn& f) {
    const int hw = a.Ho * a.Wo;
    const float b = f.b;
    if (fixup_vec(a, p0)) {
        const int n = p0 / hw;
        const int64_t o = ((int64_t)n * a.Co + co) * hw + (p0 - n * hw);
        float4 x = make_float4(v.x + b, v.y + b, v.z + b, v.w + b);
        if (a.res) {
            x.x += f.r.x;
            x.y += f.r.y;
            x.z += f.r.z;
            x.w += f.r.w;
        }
        *reinterpret_cast<float4*>(a.out + o) =
            make_float4(activate(x.x, a.act), activate(x.y, a.act), activate(x.z, a.act), activate(x.w, a.act));
        return;
    }
    const float vals[4] = {v.x, v.y, v.z, v.w};
    const float rs[4] = {f.r.x, f.r.y, f.r.z, f.r.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int pix = p0 + q;
        if (pix >= a.Npix) break;
        const int nq = pix / hw;
        const int64_t oq = ((int64_t)nq * a.Co + co) * hw + (pix - nq * hw);
        float x = vals[q] + b;
        if (a.res) x += rs[q];
        a.out[oq] = activate(x, a.act);
    }
}

__device__ __forceinline__ void fixup_store(const ConvArgs& a, int co, int p0, float4 v) {
    fixup_apply(a, co, p0, v, fixup_load(a, co, p0));
}

// Shared stream-K tile t finished inside the kernel by the workgroup whose
// partial arrived last: partials summed in workgroup order g0..g1 (the
// order of conv_fixup_k, so the result is the same to the bit), then bias
// (+ residual) + act.
template <class T>
__device__ void conv_finish_tile(const ConvArgs& a, int t, int g0, int g1, int first_slot) {
    constexpr int E = T::BM * T::BN / 1024;  // float4 per thread
    constexpr int CH = E < 4 ? E : 4;         // float4 in flight per partial (register budget)
    const __amdgpu_buffer_rsrc_t rws = make_rsrc(a.ws);
    const int mt = t % a.tiles_m, nt = t / a.tiles_m;
    const uint32_t first = slot_byte_offset<T>(g0, first_slot);
    const int hw = a.Ho * a.Wo;
    if (a.out32 && a.vec_out && (hw & 3) == 0) {
        // Every float4 of a chunk inside the output (Npix is a multiple of
        // 4 here): its bias and residual loads go out first and its partials'
        // after them, so one wait covers the chunk's loads (they complete in
        // order) - one memory round trip per chunk where loading the bias and
        // residual after the sum took two. Out-of-range offsets read 0 and
        // drop the stores. Same operations in the same order as fixup_apply.
        const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias), rr = make_rsrc(a.res), ro = make_rsrc(a.out);
        for (int e0 = 0; e0 < E; e0 += CH) {
            uint32_t off[CH];
            float b[CH];
            f32x4 r[CH], v[CH];
#pragma unroll
            for (int e = 0; e < CH; ++e) {
                const int e4 = (e0 + e) * 256 + threadIdx.x;
                const int co = mt * T::BM + (e4 * 4) / T::BN;
                const int p0 = nt * T::BN + (e4 * 4) % T::BN;
                const bool ok = co < a.Co && p0 < a.Npix;
                const int n = p0 / hw;
                off[e] = ok ? (uint32_t)((n * a.Co + co) * hw + (p0 - n * hw)) * 4u : kOutOfRange;
                b[e] = load_f32(rb, a.bias && ok ? (uint32_t)co * 4u : kOutOfRange);
                r[e] = load_f32x4(rr, a.res ? off[e] : kOutOfRange);
            }
#pragma unroll
            for (int e = 0; e < CH; ++e)
                v[e] = load_partial4(rws, first + (uint32_t)((e0 + e) * 256 + threadIdx.x) * 16u);
            for (int g = g0 + 1; g <= g1; ++g) {
                const uint32_t base = slot_byte_offset<T>(g, 0);
                f32x4 p[CH];
#pragma unroll
                for (int e = 0; e < CH; ++e)
                    p[e] = load_partial4(rws, base + (uint32_t)((e0 + e) * 256 + threadIdx.x) * 16u);
#pragma unroll
                for (int e = 0; e < CH; ++e) v[e] += p[e];
            }
#pragma unroll
            for (int e = 0; e < CH; ++e) {
                f32x4 x = v[e] + b[e];
                if (a.res) x += r[e];
                const f32x4 y = {activate(x[0], a.act), activate(x[1], a.act), activate(x[2], a.act),
                                 activate(x[3], a.act)};
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, y), ro, (int)off[e], 0, 0);
            }
        }
        return;
    }
    for (int e0 = 0; e0 < E; e0 += CH) {
        // a chunk of one partial's loads in flight at once, partial after partial
        f32x4 v[CH];
#pragma unroll
        for (int e = 0; e < CH; ++e)
            v[e] = load_partial4(rws, first + (uint32_t)((e0 + e) * 256 + threadIdx.x) * 16u);
        for (int g = g0 + 1; g <= g1; ++g) {
            const uint32_t base = slot_byte_offset<T>(g, 0);
            f32x4 p[CH];
#pragma unroll
            for (int e = 0; e < CH; ++e)
                p[e] = load_partial4(rws, base + (uint32_t)((e0 + e) * 256 + threadIdx.x) * 16u);
#pragma unroll
            for (int e = 0; e < CH; ++e) v[e] += p[e];
        }
        // the chunk's bias / residual loads, then its stores
        FixupIn fin[CH];
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int e4 = (e0 + e) * 256 + threadIdx.x;
            const int co = mt * T::BM + (e4 * 4) / T::BN;
            const int p0 = nt * T::BN + (e4 * 4) % T::BN;
            if (co < a.Co && p0 < a.Npix) fin[e] = fixup_load(a, co, p0);
        }
#pragma unroll
        for (int e = 0; e < CH; ++e) {
            const int e4 = (e0 + e) * 256 + threadIdx.x;
            const int co = mt * T::BM + (e4 * 4) / T::BN;
            const int p0 = nt * T::BN + (e4 * 4) % T::BN;
            if (co < a.Co && p0 < a.Npix) fixup_apply(a, co, p0, make_float4(v[e].x, v[e].y, v[e].z, v[e].w), fin[e]);
        }
    }
}

// Writes a finished segment: a whole tile straight to the output with bias
// (+ residual) + act, or a partial tile to the workgroup's stream-K slot.
// With tile counters (a.cnt) each writer of a partial then counts itself in
// on the tile, and the last to arrive finishes the tile (no spinning: no
// workgroup ever waits for another); the last arriver also returns the
// counter to zero for the next kernel.
// A whole tile straight to the output: bias (+ residual) + act per element
// in the order of the per-element path below (same bits). The tile goes out
// one 32-row block (tm) at a time, every bias and residual load of a block
// issued before its first store: one memory round trip per block (loads
// interleaved with stores made the compiler wait for each element's load -
// and, counting in order, for every earlier store). Out-of-range rows and
// pixels get an out-of-range buffer offset: loads read 0, stores are
// dropped. Needs output (and residual) below 2 GiB.
template <class T, bool RES>
__device__ __forceinline__ void store_tile(const ConvArgs& a, int i0, int j0, const floatx16 (&sum)[T::TM][T::TN]) {
    const int hw = a.Ho * a.Wo;
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(a.bias), rr = make_rsrc(a.res), ro = make_rsrc(a.out);
    uint32_t pbase[T::TN];  // element offset of (pixel, channel 0), or kOutOfRange
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn) {
        const int pix = j0 + acc_col<T>(tn);
        const int n = pix / hw;
        pbase[tn] = pix < a.Npix ? (uint32_t)(n * a.Co * hw + (pix - n * hw)) : kOutOfRange;
    }
    const int co0 = i0 + acc_row<T>(0, 0);  // this lane's first row; row (tm, r) adds a wave-uniform step
    const int act = a.act;
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm) {
        float bv[16];
        float rv[T::TN][16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = co0 + tm * 32 + 8 * (r >> 2) + (r & 3);
            bv[r] = a.bias ? load_f32(rb, co < a.Co ? (uint32_t)co * 4u : kOutOfRange) : 0.f;
        }
        if (RES) {
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int co = co0 + tm * 32 + 8 * (r >> 2) + (r & 3);
                    const bool ok = pbase[tn] != kOutOfRange && co < a.Co;
                    rv[tn][r] = load_f32(rr, ok ? (pbase[tn] + (uint32_t)(co * hw)) * 4u : kOutOfRange);
                }
        }
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = co0 + tm * 32 + 8 * (r >> 2) + (r & 3);
                const bool ok = pbase[tn] != kOutOfRange && co < a.Co;
                float v = sum[tm][tn][r] + bv[r];
                if (RES) v += rv[tn][r];
                v = activate(v, act);
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), ro,
                                                      (int)(ok ? (pbase[tn] + (uint32_t)(co * hw)) * 4u : kOutOfRange),
                                                      0, 0);
            }
    }
}

// BATCHED: whole tiles through store_tile. 128x128 tiles keep the
// per-element path: their kernels are at the register limit, and the
// block's loads held live made the 3x3 kernel's main loop 3x slower.
template <class T, bool FIN, bool BATCHED = (T::BM * T::BN < 128 * 128)>
__device__ __forceinline__ void conv_segment_out(const ConvArgs& a, const StreamK& sk, const Segment& seg, int g,
                                                 int i0, int j0, const floatx16 (&sum)[T::TM][T::TN]) {
    const int hw = a.Ho * a.Wo;
    if (BATCHED && seg.slot < 0 && a.out32) {
        if (a.res)
            store_tile<T, true>(a, i0, j0, sum);
        else
            store_tile<T, false>(a, i0, j0, sum);
        return;
    }
    if (seg.slot < 0) {
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn) {
            const int pix = j0 + acc_col<T>(tn);
            if (pix >= a.Npix) continue;
            const int n = pix / hw;
            float* obase = a.out + (int64_t)n * a.Co * hw + (pix - n * hw);
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int co = i0 + acc_row<T>(tm, r);
                    if (co < a.Co) {
                        float v = sum[tm][tn][r] + (a.bias ? a.bias[co] : 0.f);
                        if (a.res) v += a.res[(obase - a.out) + (int64_t)co * hw];
                        obase[(int64_t)co * hw] = activate(v, a.act);
                    }
                }
        }
        return;
    }
    if (!FIN || !a.cnt) {  // the fixup kernel reads the partials after this kernel
        if constexpr (!FIN) {
            // device-scope stores write the partials through the L2 instead
            // of leaving them dirty there, so the 40 MB or so of partial
            // tiles a batch-32 launch writes do not evict its operands: the
            // 128x128 kernels 1-1.5 us faster per launch, their fixups
            // unchanged (ResNet-18 batch 32 +0.8%, batch 8 +4%). The
            // in-kernel-finish instance keeps ordinary stores here: the same
            // change in it made its main loop slower (77 -> 91 us).
            const __amdgpu_buffer_rsrc_t rws = make_rsrc(a.ws);
            const uint32_t base = slot_byte_offset<T>(g, seg.slot);
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const float x = sum[tm][tn][r];  // (element copied first: see the FIN path)
                        store_partial(rws, base + (uint32_t)(acc_row<T>(tm, r) * T::BN + acc_col<T>(tn)) * 4u, x);
                    }
            return;
        }
        float* slot = partial_slot<T>(a.ws, g, seg.slot);
#pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
                for (int r = 0; r < 16; ++r) slot[acc_row<T>(tm, r) * T::BN + acc_col<T>(tn)] = sum[tm][tn][r];
        return;
    }
    if constexpr (FIN) {
        const __amdgpu_buffer_rsrc_t rws = make_rsrc(a.ws);
        const uint32_t base = slot_byte_offset<T>(g, seg.slot);
    #pragma unroll
        for (int tn = 0; tn < T::TN; ++tn)
    #pragma unroll
            for (int tm = 0; tm < T::TM; ++tm)
    #pragma unroll
                for (int r = 0; r < 16; ++r) {
                    // copy the element first: this compiler's __builtin_bit_cast of
                    // an ext-vector element reads the wrong element
                    const float x = sum[tm][tn][r];
                    store_partial(rws, base + (uint32_t)(acc_row<T>(tm, r) * T::BN + acc_col<T>(tn)) * 4u, x);
                }
        int g0, g1, first_slot;
        tile_partials(sk, seg.tile, g0, g1, first_slot);
        if (finish_arrive(a.cnt + seg.tile, g1 - g0)) conv_finish_tile<T>(a, seg.tile, g0, g1, first_slot);
    }
}

template <class T, int KH, int KW, bool AVEC>
__global__ void __launch_bounds__(256, 2) conv_streamk_k(ConvArgs a, StreamK sk) {
    extern __shared__ __align__(16) float lds[];
    const int g = xcd_remap(blockIdx.x, sk.G);
    SegmentWalker walk(sk, g);
    Segment seg;
    while (walk.next(sk, seg)) {
        const int mt = seg.tile % a.tiles_m, nt = seg.tile / a.tiles_m;
        const int i0 = mt * T::BM, j0 = nt * T::BN;

        typedef typename std::conditional<AVEC, KContigLoader4<T::BM, T::BK, T::LDK>,
                                          KContigLoader<T::BM, T::BK, T::LDK>>::type LA;
        LA la;
        la.init(a.w + (int64_t)i0 * a.K, a.K, a.Co - i0, a.K);
        ConvGather<T::BN, T::BK, T::LDK, KH, KW> lb;
        lb.init(a, j0);
        floatx16 sum[T::TM][T::TN];
        mfma_mainloop<T, false>(la, lb, seg.kb * T::BK, min(a.K, seg.ke * T::BK), lds, sum);

        conv_segment_out<T, false>(a, sk, seg, g, i0, j0, sum);
    }
}

// ---------------------------------------------------------------------------
// Direct-to-LDS convolution. Operands go from global memory straight into
// LDS (`buffer_load ... lds`, which writes lane l's data to LDS[M0 + size *
// l]): no VGPR staging and no LDS store instructions. Stage layout:
//   A: [BM rows][32 k], 16-byte chunks XOR-swizzled: chunk kc of row x sits
//     at position kc ^ (x & 7). An MFMA lane reads its four k of a quad as
//     one ds_read_b128, and eight consecutive rows hit eight different
//     positions, so the reads are free of bank conflicts.
//   B: [32 k][BN pixels]. One dword load covers 64 consecutive pixels of one
//     k (one channel and tap), so the gather coalesces along image rows; an
//     MFMA lane reads its k one ds_read_b32 at a time.
// Out-of-range lanes (co >= Co, pixel >= Npix, tap outside the image, k >=
// K) get an out-of-range offset, and the hardware writes 0 to LDS. The
// loader (DmaPacked) needs Ci % 32 == 0 and weights packed tap-major
// [Co][kh][kw][Ci] (for 1x1 kernels the reference layout). K is walked
// tap-major: slice s is one tap t and 32 consecutive channels, so the tap -
// and each pixel's in-image test and offset - is uniform over the slice and
// channels differ by an SGPR offset. A: one dwordx4 load per 8 rows (lane l:
// row l / 8, 16 bytes of the packed row).
// ---------------------------------------------------------------------------
template <class T>
struct DmaStage {
    static constexpr int A_FLOATS = T::BM * 32, B_FLOATS = T::BN * 32;
    static constexpr int STAGE = A_FLOATS + B_FLOATS;
    static constexpr int LDS_FLOATS = 2 * STAGE;
    // waves per SIMD that the LDS stages allow (160 KB per CU): the register
    // budget the kernel is compiled for, so registers never lower occupancy
    static constexpr int LDS_WAVES = (160 * 1024 / (LDS_FLOATS * 4)) * T::NW / 4;
    static constexpr int MIN_WAVES = LDS_WAVES < 2 ? 2 : (LDS_WAVES > 4 ? 4 : LDS_WAVES);
    static constexpr int PX_GROUPS = T::BN / 64;             // 64-pixel groups of a B row
    static constexpr int B_LOADS = 32 * PX_GROUPS / T::NW;  // dword loads per wave per slice
    static_assert(T::NW % PX_GROUPS == 0 && B_LOADS % 2 == 0, "B rows split evenly over the waves");
    static_assert(T::BM % 32 == 0 && (T::BN == 64 || T::BN == 128) && T::BK == 32, "dma tile");
};

// Per-tile pixel data of the B loaders: this lane's pixel (one per wave's
// 64-pixel group), element offset of its tap (0, 0) at channel 0, and the
// taps inside the image as a bit mask.
template <int KH, int KW>
struct PixelTaps {
    typedef typename std::conditional<(KH * KW > 32), uint64_t, uint32_t>::type Mask;
    int bpo;
    Mask mask;
    __device__ void init(const ConvArgs& a, int px) {
        const bool valid = px < a.Npix;
        const int hw = a.Ho * a.Wo;
        const int p = valid ? px : 0;
        const int n = p / hw;
        const int rem = p - n * hw;
        const int oh = rem / a.Wo;
        const int ow = rem - oh * a.Wo;
        const int h0 = oh * a.sh - a.ph, w0 = ow * a.sw - a.pw;
        bpo = n * a.Ci * (a.H * a.W) + h0 * a.W + w0;
        mask = 0;
#pragma unroll
        for (int r = 0; r < KH; ++r)
#pragma unroll
            for (int c = 0; c < KW; ++c) {
                const bool in = valid && (unsigned)(h0 + r) < (unsigned)a.H && (unsigned)(w0 + c) < (unsigned)a.W;
                mask |= (Mask)in << (r * KW + c);
            }
    }
    __device__ bool inside(int tap) const { return ((mask >> tap) & 1u) != 0; }
    __device__ uint32_t bit(int tap) const { return (uint32_t)(mask >> tap) & 1u; }
};

template <class T, int KH, int KW>
struct DmaPacked {
    typedef DmaStage<T> D;
    static constexpr bool kFinishInKernel = true;
    static constexpr int EXTRA_LDS_FLOATS = 0;
    __device__ void prepare(float*, const ConvArgs&) {}
    static constexpr int A_LOADS = T::BM / (8 * T::NW);  // dwordx4 loads per wave per slice, 8 rows each
    static_assert(T::BM % (8 * T::NW) == 0, "A rows split evenly over the waves");
    __amdgpu_buffer_rsrc_t rin, rw;
    int wave, b_grp, b_kr0, CB, HW, W, Ci;
    uint32_t avo[A_LOADS];
    PixelTaps<KH, KW> px;
    int t, cb;       // slice cursor: tap, 32-channel block
    uint32_t bv;     // B offset of the slice being issued

    __device__ void init(const ConvArgs& a, int wave_, int lane) {
        rin = make_rsrc(a.in);
        rw = make_rsrc(a.w);
        wave = wave_;
        b_grp = wave % D::PX_GROUPS;
        b_kr0 = (wave / D::PX_GROUPS) * D::B_LOADS;
        CB = a.Ci >> 5;
        HW = a.H * a.W;
        W = a.W;
        Ci = a.Ci;
    }
    __device__ void tile(const ConvArgs& a, int i0, int j0, int lane) {
        const int a_kc = (lane & 7) ^ ((lane >> 3) & 7);
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int co = i0 + (wave + T::NW * i) * 8 + (lane >> 3);
            avo[i] = keep_or_oob((uint32_t)(co * a.ldw) * 4u + (uint32_t)a_kc * 16u, co < a.Co);
        }
        px.init(a, j0 + b_grp * 64 + lane);
    }
    __device__ void begin(int kb) {
        t = kb / CB;
        cb = kb - t * CB;
    }
    __device__ void step(bool more) {
        const int cb1 = cb + 1 == CB ? 0 : cb + 1;
        const int t1 = cb + 1 == CB ? t + 1 : t;
        t = more ? t1 : t;
        cb = more ? cb1 : cb;
    }
    // part 0: A and the first half of B; part 1: the rest of B
    __device__ void issue(float* S, bool on, int part) {
        if (part == 0) {
            const uint32_t sa = (uint32_t)(t * Ci + cb * 32) * 4u;
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i)
                dma_load16(rw, S + (wave + T::NW * i) * 8 * 32, on ? avo[i] : kOutOfRange, sa);
            const int r = t / KW, c = t - r * KW;
            bv = keep_or_oob((uint32_t)(px.bpo + r * W + c) * 4u, on && px.inside(t));
        }
        const uint32_t s0 = (uint32_t)((cb * 32 + b_kr0) * HW) * 4u;
        float* d0 = S + D::A_FLOATS + b_kr0 * T::BN + b_grp * 64;
        constexpr int H = D::B_LOADS / 2;
#pragma unroll
        for (int i = part * H; i < (part + 1) * H; ++i) dma_load4(rin, d0 + i * T::BN, bv, s0 + (uint32_t)(i * HW) * 4u);
    }
};

// A KH x KW convolution of `in` and a 1x1 projection of a second input (a
// residual block's strided downsample) as one contraction, so the
// projection needs no launch and no tensor of its own: k < KH*KW*Ci walks
// `in` as DmaPacked does, the last pci k walk `pin` at the output pixel's
// position times the projection stride (always inside that image). Weights
// [Co][KH*KW*Ci + pci]: slice s starts at k = 32 s in both parts. Needs Ci
// and pci multiples of 32.
template <class T, int KH, int KW>
struct DmaProj {
    typedef DmaStage<T> D;
    static constexpr bool kFinishInKernel = true;
    static constexpr int EXTRA_LDS_FLOATS = 0;
    __device__ void prepare(float*, const ConvArgs&) {}
    static constexpr int A_LOADS = T::BM / (8 * T::NW);
    static constexpr int TAPS = KH * KW;  // cursor tap TAPS: the projection
    static_assert(T::BM % (8 * T::NW) == 0, "A rows split evenly over the waves");
    __amdgpu_buffer_rsrc_t rin, rx, rw;
    int wave, b_grp, b_kr0, CB, CBX, HW, HWX, W, Ci;
    uint32_t avo[A_LOADS];
    PixelTaps<KH, KW> px;
    uint32_t xvo;  // this lane's pixel in the projection input at channel 0 (bytes; out of range past Npix)
    int t, cb;     // slice cursor: tap (TAPS: projection), 32-channel block
    uint32_t bv;

    __device__ void init(const ConvArgs& a, int wave_, int lane) {
        rin = make_rsrc(a.in);
        rx = make_rsrc(a.pin);
        rw = make_rsrc(a.w);
        wave = wave_;
        b_grp = wave % D::PX_GROUPS;
        b_kr0 = (wave / D::PX_GROUPS) * D::B_LOADS;
        CB = a.Ci >> 5;
        CBX = a.pci >> 5;
        HW = a.H * a.W;
        HWX = a.pH * a.pW;
        W = a.W;
        Ci = a.Ci;
    }
    __device__ void tile(const ConvArgs& a, int i0, int j0, int lane) {
        const int a_kc = (lane & 7) ^ ((lane >> 3) & 7);
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int co = i0 + (wave + T::NW * i) * 8 + (lane >> 3);
            avo[i] = keep_or_oob((uint32_t)(co * a.ldw) * 4u + (uint32_t)a_kc * 16u, co < a.Co);
        }
        const int p = j0 + b_grp * 64 + lane;
        px.init(a, p);
        const bool valid = p < a.Npix;
        const int q = valid ? p : 0;
        const int hw = a.Ho * a.Wo;
        const int n = q / hw, rem = q - n * hw;
        const int oh = rem / a.Wo, ow = rem - oh * a.Wo;
        xvo = keep_or_oob((uint32_t)(n * a.pci * HWX + oh * a.psh * a.pW + ow * a.psw) * 4u, valid);
    }
    __device__ void begin(int kb) {
        const bool proj = kb >= TAPS * CB;
        t = proj ? TAPS : kb / CB;
        cb = proj ? kb - TAPS * CB : kb - t * CB;
    }
    __device__ void step(bool more) {
        const bool wrap = t < TAPS && cb + 1 == CB;
        const int cb1 = wrap ? 0 : cb + 1;
        const int t1 = wrap ? t + 1 : t;
        t = more ? t1 : t;
        cb = more ? cb1 : cb;
    }
    // part 0: A and the first half of B; part 1: the rest of B
    __device__ void issue(float* S, bool on, int part) {
        const bool proj = t == TAPS;
        if (part == 0) {
            const uint32_t sa = (uint32_t)(t * Ci + cb * 32) * 4u;
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i)
                dma_load16(rw, S + (wave + T::NW * i) * 8 * 32, on ? avo[i] : kOutOfRange, sa);
            const int r = t / KW, c = t - r * KW;
            const uint32_t tap = keep_or_oob((uint32_t)(px.bpo + r * W + c) * 4u, on && !proj && px.inside(t));
            bv = proj ? (on ? xvo : kOutOfRange) : tap;
        }
        const int hw = proj ? HWX : HW;
        const uint32_t s0 = (uint32_t)((cb * 32 + b_kr0) * hw) * 4u;
        float* d0 = S + D::A_FLOATS + b_kr0 * T::BN + b_grp * 64;
        constexpr int H = D::B_LOADS / 2;
        if (proj) {
#pragma unroll
            for (int i = part * H; i < (part + 1) * H; ++i) dma_load4(rx, d0 + i * T::BN, bv, s0 + (uint32_t)(i * hw) * 4u);
        } else {
#pragma unroll
            for (int i = part * H; i < (part + 1) * H; ++i) dma_load4(rin, d0 + i * T::BN, bv, s0 + (uint32_t)(i * hw) * 4u);
        }
    }
};

// Few input channels (the RGB stem): weights packed [Co][Kp], k = tap * CI +
// ci tap-major, zero past K = kh*kw*CI up to Kp, a multiple of 32. A as in
// DmaPacked; each B load is one k, whose tap and channel are uniform (the
// divisions by compile-time constants run on the scalar unit), and each lane
// applies its pixel's in-image test for that tap.
template <class T, int KH, int KW, int CI>
struct DmaSmallC {
    typedef DmaStage<T> D;
    // shared tiles finished in the kernel: the stem at batch 32 grows from
    // 100 to 111 us but its 15 us fixup launch goes (batch 32 even, batch 8
    // +1%)
    static constexpr bool kFinishInKernel = true;
    static constexpr int A_LOADS = T::BM / (8 * T::NW);
    static constexpr int KMAX = 256;  // table entries (Kp <= KMAX, checked on the host)
    static_assert(KH * KW < 64, "tap 63 marks k >= K");
    // per k of the packed rows, filled once per workgroup: the byte offset of
    // (channel, tap) from the pixel's (0, 0) tap at channel 0, and the tap
    // index for the in-image bit (63 past K: never inside)
    static constexpr int EXTRA_LDS_FLOATS = 2 * KMAX;
    __amdgpu_buffer_rsrc_t rin, rw;
    int wave, b_grp, b_kr0;
    uint32_t avo[A_LOADS];
    PixelTaps<KH, KW> px;
    const int* tab;
    int k0;  // slice cursor

    __device__ void init(const ConvArgs& a, int wave_, int lane) {
        rin = make_rsrc(a.in);
        rw = make_rsrc(a.w);
        wave = wave_;
        b_grp = wave % D::PX_GROUPS;
        b_kr0 = (wave / D::PX_GROUPS) * D::B_LOADS;
    }
    // fills the table (the caller's barrier publishes it)
    __device__ void prepare(float* extra, const ConvArgs& a) {
        int* t = reinterpret_cast<int*>(extra);
        for (int k = threadIdx.x; k < KMAX; k += T::THREADS) {
            const int tap = k / CI, ci = k - tap * CI;
            const int r = tap / KW, c = tap - r * KW;
            const bool in = k < a.K;
            t[2 * k] = in ? (ci * (a.H * a.W) + r * a.W + c) * 4 : 0;
            t[2 * k + 1] = in ? tap : 63;
        }
        tab = t;
    }
    __device__ void tile(const ConvArgs& a, int i0, int j0, int lane) {
        const int a_kc = (lane & 7) ^ ((lane >> 3) & 7);
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) {
            const int co = i0 + (wave + T::NW * i) * 8 + (lane >> 3);
            avo[i] = keep_or_oob((uint32_t)(co * a.ldw) * 4u + (uint32_t)a_kc * 16u, co < a.Co);
        }
        px.init(a, j0 + b_grp * 64 + lane);
    }
    __device__ void begin(int kb) { k0 = kb * 32; }
    __device__ void step(bool more) { k0 += more ? 32 : 0; }
    __device__ void issue(float* S, bool on, int part) {
        if (part == 0) {
#pragma unroll
            for (int i = 0; i < A_LOADS; ++i)
                dma_load16(rw, S + (wave + T::NW * i) * 8 * 32, on ? avo[i] : kOutOfRange, (uint32_t)k0 * 4u);
        }
        constexpr int H = D::B_LOADS / 2;
        float* d0 = S + D::A_FLOATS + b_kr0 * T::BN + b_grp * 64;
        // this half's H table entries (broadcast LDS reads), then per load
        // one add and a bit select: no per-load division or branch
        const int kstart = k0 + b_kr0 + part * H;
        int e[2 * H];
#pragma unroll
        for (int q = 0; q < 2 * H; q += 4) {
            const int4 v = *reinterpret_cast<const int4*>(tab + 2 * kstart + q);
            e[q] = v.x, e[q + 1] = v.y, e[q + 2] = v.z, e[q + 3] = v.w;
        }
        const uint32_t base = (uint32_t)px.bpo * 4u;
        const uint32_t onm = 0u - (uint32_t)on;
#pragma unroll
        for (int i = 0; i < H; ++i) {
            const uint32_t m = (0u - px.bit(e[2 * i + 1])) & onm;
            dma_load4(rin, d0 + (part * H + i) * T::BN, ((base + (uint32_t)e[2 * i]) & m) | (kOutOfRange & ~m), 0u);
        }
    }
};

// MFMA operands of quad q from a direct-to-LDS stage: A as one 16-byte read
// per 32-row block, B as four single floats per 32-column block.
template <class T>
__device__ __forceinline__ void read_quad_dma(const float* Sa, int a_row, int a_sw, const float* Sb, int q,
                                              f32x4 (&a)[T::TM], f32x4 (&b)[T::TN]) {
#pragma unroll
    for (int tm = 0; tm < T::TM; ++tm)
        a[tm] = *reinterpret_cast<const f32x4*>(Sa + (a_row + tm * 32) * 32 + ((a_sw ^ q) << 2));
#pragma unroll
    for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
        for (int s = 0; s < 4; ++s) b[tn][s] = Sb[(4 * q + s) * T::BN + tn * 32];
}

template <class T, class L, bool FIN>
__global__ void __launch_bounds__(T::THREADS, DmaStage<T>::MIN_WAVES) conv_dma_k(ConvArgs a, StreamK sk) {
    typedef DmaStage<T> D;
    extern __shared__ __align__(16) float lds[];
    const int g = xcd_remap(blockIdx.x, sk.G);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // MFMA read side: A row and swizzled chunk of quad 0 (kc = 4h), B column
    const int wi = (wave / T::WN) * T::WAVE_M, wj = (wave % T::WN) * T::WAVE_N;
    const int a_row = wi + (lane & 31);
    const int a_sw = (4 * (lane >> 5)) ^ (lane & 7);
    const int b_off = D::A_FLOATS + 16 * (lane >> 5) * T::BN + wj + (lane & 31);
    L ld;
    ld.init(a, wave, lane);
    if (L::EXTRA_LDS_FLOATS) {
        ld.prepare(lds + 2 * D::STAGE, a);
        __syncthreads();
    }

    SegmentWalker walk(sk, g);
    Segment seg;
    // The slice loop runs on across segment boundaries: during a segment's
    // last slice the loads of the next segment's first slice are issued, so
    // a new tile starts with its operands already in LDS (short-K
    // convolutions - the stem, 1x1 - have only a few slices per tile).
    if (!walk.next(sk, seg)) return;
    {
        const int mt = seg.tile % a.tiles_m, nt = seg.tile / a.tiles_m;
        ld.tile(a, mt * T::BM, nt * T::BN, lane);
        ld.begin(seg.kb);
        ld.issue(lds, true, 0);
        ld.issue(lds, true, 1);
        wait_dma();
        __syncthreads();
    }
    // operands of quads 0 and 2 in set 0, quads 1 and 3 in set 1: the
    // registers carried from one slice to the next (quad 0) stay put
    f32x4 a0[T::TM], b0[T::TN], a1[T::TM], b1[T::TN];
    read_quad_dma<T>(lds, a_row, a_sw, lds + b_off, 0, a0, b0);
    int stage = 0;
    while (true) {
        const int mt = seg.tile % a.tiles_m, nt = seg.tile / a.tiles_m;
        const int i0 = mt * T::BM, j0 = nt * T::BN;
        floatx16 sum[T::TM][T::TN];
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int tn = 0; tn < T::TN; ++tn)
#pragma unroll
                for (int r = 0; r < 16; ++r) sum[tm][tn][r] = 0.f;
        Segment nxt;
        bool have_next = false;
        for (int it = seg.kb; it < seg.ke; ++it) {
            // next slice: this segment's, or the first of the next segment
            // (the loader switches tiles once this tile's loads are all issued);
            // past the walk's end its loads are no-ops
            const bool last = it + 1 == seg.ke;
            if (last) {
                have_next = walk.next(sk, nxt);
                if (have_next) {
                    const int nmt = nxt.tile % a.tiles_m, nnt = nxt.tile / a.tiles_m;
                    ld.tile(a, nmt * T::BM, nnt * T::BN, lane);
                    ld.begin(nxt.kb);
                }
            } else {
                ld.step(true);
            }
            const bool more = !last || have_next;
            float* next = lds + (stage ^ 1) * D::STAGE;
            const float* S = lds + stage * D::STAGE;
            // the loads issue in two halves ahead of quads 0 and 1; quad 2
            // leaves them time to land before the barrier
            ld.issue(next, more, 0);
            read_quad_dma<T>(S, a_row, a_sw, S + b_off, 1, a1, b1);
            mfma_quad<T>(a0, b0, sum);
            ld.issue(next, more, 1);
            read_quad_dma<T>(S, a_row, a_sw, S + b_off, 2, a0, b0);
            mfma_quad<T>(a1, b1, sum);
            read_quad_dma<T>(S, a_row, a_sw, S + b_off, 3, a1, b1);
            mfma_quad<T>(a0, b0, sum);
            wait_dma();
            __syncthreads();
            read_quad_dma<T>(next, a_row, a_sw, next + b_off, 0, a0, b0);
            mfma_quad<T>(a1, b1, sum);
            stage ^= 1;
        }
        conv_segment_out<T, FIN>(a, sk, seg, g, i0, j0, sum);
        if (!have_next) break;
        seg = nxt;
    }
}

// ---------------------------------------------------------------------------
// Short convolutions (ResNet-18 at batch 1 and 2: few output tiles, K up to
// 4608): `conv_ws_k`. A workgroup owns one 32 x 32 output tile (32 channels
// x 32 pixels) over a contiguous range of K slices, and its four waves split
// that range among themselves - wave w takes the range's slices w, w + 4,
// ... - each computing the whole tile into its own v_mfma_f32_32x32x2_f32
// accumulator; the four sums are added through LDS in wave order. Operands
// go straight from global memory into the MFMA operand registers, with no
// LDS staging and no barrier in the main loop: per slice (one tap and 32
// channels of the tap-major weights, or 32 channels of the folded 1x1
// projection) lane half h of a wave takes the slice's k = 16h .. 16h + 15,
// so lane (row i, half h) loads A[i][16h ..] as four 16-byte loads and lane
// (pixel j, half h) gathers B[16h + c][j] for c < 16 (one input channel
// each, 0 outside the image), and MFMA step c multiplies those pairs. All
// of a wave's slices (at most NS) are loaded before its first MFMA.
//
// A tile with more K than one workgroup should take is split over S <= 16
// workgroups (contiguous slice ranges): each stores its 4 KB partial with
// device-scope stores and the last to arrive adds the S partials in range
// order and writes the tile (the stream-K finish protocol of mfma_tile.h:
// store_partial4, finish_arrive, load_partial4). The sums are the same
// whichever workgroup finishes: deterministic. Every shared tile is finished
// in the launch: no fixup kernel.
// ---------------------------------------------------------------------------

// One 16-byte partial, stored with device-scope coherence.
__device__ __forceinline__ void store_partial4(__amdgpu_buffer_rsrc_t ws, uint32_t byte_off, f32x4 v) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), ws, (int)byte_off, 0, kDeviceScope);
}

template <int NS, bool PROJ>
__global__ void __launch_bounds__(256, 2) conv_ws_k(ConvArgs a, int S, int iters) {
    __shared__ __align__(16) float red[4][32 * 32];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int t = blockIdx.x / S, part = blockIdx.x - t * S;
    const int mt = t % a.tiles_m, nt = t / a.tiles_m;
    const int i0 = mt * 32, j0 = nt * 32;
    const int kb = (int)((int64_t)part * iters / S), ke = (int)((int64_t)(part + 1) * iters / S);
    const int h = lane >> 5, l32 = lane & 31;

    // A: this lane's weight row, from k = 16h of a slice
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w), rin = make_rsrc(a.in);
    const int co = i0 + l32;
    const uint32_t arow = keep_or_oob((uint32_t)(co * a.ldw + 16 * h) * 4u, co < a.Co);
    // B: this lane's pixel; taps inside the image as a bit mask
    const int px = j0 + l32;
    const bool valid = px < a.Npix;
    const int hw = a.Ho * a.Wo, HW = a.H * a.W;
    const int pq = valid ? px : 0;
    const int n = pq / hw, rem = pq - n * hw;
    const int oh = rem / a.Wo, ow = rem - oh * a.Wo;
    const int h0 = oh * a.sh - a.ph, w0 = ow * a.sw - a.pw;
    uint32_t mask = 0;
    for (int r = 0; r < a.kh; ++r)
        for (int c = 0; c < a.kw; ++c) {
            const bool in = valid && (unsigned)(h0 + r) < (unsigned)a.H && (unsigned)(w0 + c) < (unsigned)a.W;
            mask |= (uint32_t)in << (r * a.kw + c);
        }
    const int bpo = n * a.Ci * HW + h0 * a.W + w0 + 16 * h * HW;  // tap (0, 0), channel 16h
    const int CB = a.Ci >> 5, taps = a.kh * a.kw;
    __amdgpu_buffer_rsrc_t rx = rin;
    int xvo = 0, pHW = 0;
    if constexpr (PROJ) {
        rx = make_rsrc(a.pin);
        pHW = a.pH * a.pW;
        xvo = n * a.pci * pHW + oh * a.psh * a.pW + ow * a.psw + 16 * h * pHW;
    }

    f32x4 av[NS][4];
    float bv[NS][16];
#pragma unroll
    for (int q = 0; q < NS; ++q) {
        const int sl = kb + wave + 4 * q;  // wave-uniform
        const bool on = sl < ke;
#pragma unroll
        for (int u = 0; u < 4; ++u)
            av[q][u] = load_f32x4(rw, on ? arow + (uint32_t)sl * 128u + 16u * u : kOutOfRange);
        const int tap = sl / CB, cb = sl - tap * CB;
        const int r = tap / a.kw, cc = tap - r * a.kw;
        bool in = on && ((mask >> (tap & 31)) & 1u);
        uint32_t base = (uint32_t)(bpo + r * a.W + cc + cb * 32 * HW) * 4u;
        uint32_t step = (uint32_t)HW * 4u;
        __amdgpu_buffer_rsrc_t rb = rin;
        if constexpr (PROJ) {
            // the folded projection's slices: selects, not a branch (the
            // loads stay one straight run)
            const bool proj = tap >= taps;
            const int pcb = sl - taps * CB;
            in = proj ? on && valid : in;
            base = proj ? (uint32_t)(xvo + pcb * 32 * pHW) * 4u : base;
            step = proj ? (uint32_t)pHW * 4u : step;
            rb = proj ? rx : rin;
        }
#pragma unroll
        for (int c = 0; c < 16; ++c) bv[q][c] = load_f32(rb, in ? base + step * (uint32_t)c : kOutOfRange);
    }
    // every load above is issued before the first MFMA below
    __builtin_amdgcn_sched_barrier(0);
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    // a wave with fewer slices multiplies zeros in its last one (straight-line
    // code: a branch around it made the compiler sink that slice's loads
    // into it, one round trip per load); its workgroup waits for the waves
    // with NS slices anyway
#pragma unroll
    for (int q = 0; q < NS; ++q)
#pragma unroll
        for (int c = 0; c < 16; ++c) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[q][c >> 2][c & 3], bv[q][c], acc, 0, 0, 0);
    // the four waves' sums in wave order; thread t then holds 4 consecutive
    // pixels (columns 4 (t % 8) ..) of tile row t / 8
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float x = acc[r];  // (element copied first: see store_tile)
        red[wave][(8 * (r >> 2) + 4 * h + (r & 3)) * 32 + l32] = x;
    }
    __syncthreads();
    const int row = threadIdx.x >> 3, c4 = (threadIdx.x & 7) * 4;
    f32x4 v = *reinterpret_cast<const f32x4*>(&red[0][row * 32 + c4]);
#pragma unroll
    for (int w = 1; w < 4; ++w) v += *reinterpret_cast<const f32x4*>(&red[w][row * 32 + c4]);
    const int oco = i0 + row, op0 = j0 + c4;
    if (S > 1) {
        const __amdgpu_buffer_rsrc_t rws = make_rsrc(a.ws);
        const uint32_t slot = (uint32_t)t * (uint32_t)S * 4096u + threadIdx.x * 16u;
        store_partial4(rws, slot + (uint32_t)part * 4096u, v);
        if (!finish_arrive(a.cnt + t, S - 1)) return;  // uniform
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
    if (oco < a.Co && op0 < a.Npix) fixup_store(a, oco, op0, make_float4(v.x, v.y, v.z, v.w));
}

// ---------------------------------------------------------------------------
// Convolution + relu streamed into a 3x3 / stride 2 / pad 1 max pool
// (nnc_hip_conv_maxpool): ResNet's stem without its 103 MB (batch 32)
// activation in HBM.
// ---------------------------------------------------------------------------
// The convolution output is viewed with rows of 128 pixels (a.Wo = 128, the
// real width pb.Wr <= 128 pixels used), so one 64 x 128 tile is one output
// row of 64 channels. The conv rows of all images, in order, are split into
// G contiguous ranges of whole pool-row pairs (rows 2p, 2p + 1), one per
// workgroup of a persistent grid (G = resident workgroups): workgroup g
// computes its rows one after the other, the next row's first slice loaded
// during the current row's last (as in conv_dma_k). For each row: bias +
// relu (the conv epilogue's rounding), then the max over conv columns 2j-1,
// 2j, 2j+1 by lane shuffles (consecutive pixels are consecutive lanes of a
// wave; a wave's first pixel takes its left neighbour from the previous wave
// through LDS), held by the lane of pixel 2j; then down the rows in
// registers: row 2p starts pool row p (with row 2p-1's maxima unless p = 0),
// row 2p + 1 completes it and it is stored. A range's first pool row p > 0
// is missing row 2p - 1, which the previous range ends with: that range
// writes its last row's maxima to pb.side, and conv_pool_fixup_k takes the
// max of the two. Relu values are never NaN or -0, so the max is exact and
// order-free: the same bits as nnc_maxpool2d's scan of the same convolution.
struct PoolBand {
    float* out;   // [N][Co][Hp][Wp]
    float* side;  // [G][Co][Wp]: a range's last-row maxima for the next range's first pool row
    int* cnt;     // conv_stem_pool_k: [G] range-boundary arrival counters, zero between launches
    int Wr, Hp, Wp;
    int pairs;    // N * Hp: pool rows of all images, two conv rows each
};

__device__ __forceinline__ int pool_range_begin(int g, int G, int pairs) { return (int)((int64_t)g * pairs / G); }

// Two waves per SIMD: the running maxima of a row stay in registers beside
// the accumulators, more than the three-wave budget of conv_dma_k holds.
template <class T, class L>
__global__ void __launch_bounds__(T::THREADS, 2) conv_pool_k(ConvArgs a, PoolBand pb) {
    static_assert(T::BM == 64 && T::BN == 128 && T::WM == 1 && T::WN == 4 && T::TM == 2 && T::TN == 1,
                  "one 64-channel row of 128 pixels per tile, 32 pixels per wave");
    typedef DmaStage<T> D;
    extern __shared__ __align__(16) float lds[];
    __shared__ float xch[T::NW][2][32];  // each wave's last pixel (per lane half) for the next wave
    __shared__ float bias_s[T::BM];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wi = (wave / T::WN) * T::WAVE_M, wj = (wave % T::WN) * T::WAVE_N;
    const int a_row = wi + (lane & 31);
    const int a_sw = (4 * (lane >> 5)) ^ (lane & 7);
    const int b_off = D::A_FLOATS + 16 * (lane >> 5) * T::BN + wj + (lane & 31);
    L ld;
    ld.init(a, wave, lane);
    if (L::EXTRA_LDS_FLOATS) {
        ld.prepare(lds + 2 * D::STAGE, a);
        __syncthreads();
    }
    const int G = gridDim.x;
    const int g = xcd_remap(blockIdx.x, G);
    const int t0 = 2 * pool_range_begin(g, G, pb.pairs), t1 = 2 * pool_range_begin(g + 1, G, pb.pairs);
    if (t0 >= t1) return;  // uniform over the workgroup; never with G <= pairs
    const int iters = (a.K + T::BK - 1) / T::BK;
    const int q = lane & 31, half = lane >> 5;
    const int px = wj + q;  // pixel of the row (virtual width 128)
    if (threadIdx.x < T::BM) bias_s[threadIdx.x] = (a.bias && (int)threadIdx.x < a.Co) ? a.bias[threadIdx.x] : 0.f;
    ld.tile(a, 0, t0 * T::BN, lane);
    ld.begin(0);
    ld.issue(lds, true, 0);
    ld.issue(lds, true, 1);
    wait_dma();
    __syncthreads();
    f32x4 a0[T::TM], b0[T::TN], a1[T::TM], b1[T::TN];
    read_quad_dma<T>(lds, a_row, a_sw, lds + b_off, 0, a0, b0);
    int stage = 0;
    float run[T::TM][16];
    for (int t = t0; t < t1; ++t) {
        const int n = t / a.Ho, y = t - n * a.Ho;
        floatx16 sum[T::TM][T::TN];
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) sum[tm][0][r] = 0.f;
        const bool have_next = t + 1 < t1;
        for (int it = 0; it < iters; ++it) {
            const bool last = it + 1 == iters;
            if (last) {
                if (have_next) {
                    ld.tile(a, 0, (t + 1) * T::BN, lane);
                    ld.begin(0);
                }
            } else {
                ld.step(true);
            }
            const bool more = !last || have_next;
            float* next = lds + (stage ^ 1) * D::STAGE;
            const float* S = lds + stage * D::STAGE;
            ld.issue(next, more, 0);
            read_quad_dma<T>(S, a_row, a_sw, S + b_off, 1, a1, b1);
            mfma_quad<T>(a0, b0, sum);
            ld.issue(next, more, 1);
            read_quad_dma<T>(S, a_row, a_sw, S + b_off, 2, a0, b0);
            mfma_quad<T>(a1, b1, sum);
            read_quad_dma<T>(S, a_row, a_sw, S + b_off, 3, a1, b1);
            mfma_quad<T>(a0, b0, sum);
            wait_dma();
            __syncthreads();
            read_quad_dma<T>(next, a_row, a_sw, next + b_off, 0, a0, b0);
            mfma_quad<T>(a1, b1, sum);
            stage ^= 1;
        }
        // bias + relu (in the accumulators), then the max over columns
        // 2j-1 .. 2j+1 at the lane of 2j
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float x = sum[tm][0][r];  // copied out of the vector first
                const float v = activate(x + bias_s[acc_row<T>(tm, r)], kActRelu);
                sum[tm][0][r] = v;
                if (q == 31) xch[wave][half][tm * 16 + r] = v;
            }
        __syncthreads();
        const bool has_left = px >= 1, has_right = px + 1 < pb.Wr;
        const bool store = (q & 1) == 0 && px < pb.Wr;
        const bool fresh = (y & 1) == 0 && (t == t0 || y == 0);  // pool row without its row 2p - 1 here
        const int j = px >> 1, p = y >> 1;
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float v = sum[tm][0][r];
                const float right = __shfl(v, (lane + 1) & 63);
                float left = __shfl(v, (lane - 1) & 63);
                if (q == 0) left = wave > 0 ? xch[wave - 1][half][tm * 16 + r] : 0.f;
                float m = v;
                if (has_right) m = fmaxf(m, right);
                if (has_left) m = fmaxf(m, left);
                // down the rows: y = 2p starts pool row p, y = 2p + 1 completes it
                if ((y & 1) == 0) {
                    run[tm][r] = fresh ? m : fmaxf(run[tm][r], m);
                } else {
                    const int co = acc_row<T>(tm, r);
                    if (store && co < a.Co)
                        pb.out[(((int64_t)n * a.Co + co) * pb.Hp + p) * pb.Wp + j] = fmaxf(run[tm][r], m);
                    run[tm][r] = m;
                }
            }
    }
    // the last row's maxima: the top row of the next range's first pool row
    const int y_last = (t1 - 1) % a.Ho;
    if (y_last + 1 < a.Ho) {
#pragma unroll
        for (int tm = 0; tm < T::TM; ++tm)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = acc_row<T>(tm, r);
                if ((q & 1) == 0 && px < pb.Wr && co < a.Co)
                    pb.side[((int64_t)g * a.Co + co) * pb.Wp + (px >> 1)] = run[tm][r];
            }
    }
}

// Completes each range's first pool row (when it is not an image's first)
// with the previous range's last-row maxima. Grid (ceil(Co * Wp / 256),
// ranges - 1): one thread per (channel, column) of range g = blockIdx.y + 1.
__global__ void __launch_bounds__(256) conv_pool_fixup_k(PoolBand pb, int Co, int Ho, int G) {
    const int g = blockIdx.y + 1;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= Co * pb.Wp) return;
    const int t0 = 2 * pool_range_begin(g, G, pb.pairs);
    const int n = t0 / Ho, y0 = t0 - n * Ho;
    if (y0 == 0) return;  // an image's first pool row is complete
    const int co = i / pb.Wp, j = i - co * pb.Wp;
    float* o = pb.out + (((int64_t)n * Co + co) * pb.Hp + y0 / 2) * pb.Wp + j;
    *o = fmaxf(*o, pb.side[((int64_t)(g - 1) * Co + co) * pb.Wp + j]);
}

// Grid (chunks, stream-K tiles): workgroup (c, t) finishes chunk c of tile t
// (256 float4 of the BM x BN tile). Tiles covered by a single workgroup were
// written by it; shared tiles sum their partials in workgroup order, then
// bias (+ residual) + act. Each thread handles 4 consecutive pixels of a
// tile row; partial loads are issued four at a time, and when the 4 pixels
// are in one image (Ho*Wo % 4 == 0) residual and output move as float4.
template <class T>
__global__ void __launch_bounds__(256) conv_fixup_k(ConvArgs a, StreamK sk) {
    const int t = blockIdx.y;
    int g0, g1, first_slot;
    if (!tile_partials(sk, t, g0, g1, first_slot)) return;
    const int e4 = blockIdx.x * 256 + threadIdx.x;
    if (e4 >= T::BM * T::BN / 4) return;
    const int mt = t % a.tiles_m, nt = t / a.tiles_m;
    const int co = mt * T::BM + (e4 * 4) / T::BN;
    const int p0 = nt * T::BN + (e4 * 4) % T::BN;
    if (co >= a.Co || p0 >= a.Npix) return;
    float4 v = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g0, first_slot))[e4];
    int g = g0 + 1;
    // many partials per tile (short problems): 16 loads in flight per thread
    for (; g + 15 <= g1; g += 16) {
        float4 p[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) p[q] = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g + q, 0))[e4];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            v.x += p[q].x;
            v.y += p[q].y;
            v.z += p[q].z;
            v.w += p[q].w;
        }
    }
    for (; g + 3 <= g1; g += 4) {
        float4 p[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) p[q] = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g + q, 0))[e4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v.x += p[q].x;
            v.y += p[q].y;
            v.z += p[q].z;
            v.w += p[q].w;
        }
    }
    for (; g <= g1; ++g) {
        const float4 p = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g, 0))[e4];
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    fixup_store(a, co, p0, v);
}

// Shared tiles with many partials (short problems: few tiles, long K): the
// partial list is split over four groups of 64 threads (group q sums
// partials q, q + 4, ... in workgroup order), and group 0 adds the four
// sums in group order through LDS - deterministic, and each thread waits
// on a quarter of the loads. Grid (BM*BN/256, stream-K tiles): a workgroup
// finishes 64 float4 of a tile.
template <class T>
__global__ void __launch_bounds__(256) conv_fixup_split_k(ConvArgs a, StreamK sk) {
    __shared__ float4 part[3][64];
    const int t = blockIdx.y;
    int g0, g1, first_slot;
    if (!tile_partials(sk, t, g0, g1, first_slot)) return;  // uniform over the workgroup
    const int grp = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int e4 = blockIdx.x * 64 + lane;
    const int mt = t % a.tiles_m, nt = t / a.tiles_m;
    const int co = mt * T::BM + (e4 * 4) / T::BN;
    const int p0 = nt * T::BN + (e4 * 4) % T::BN;
    const bool valid = e4 < T::BM * T::BN / 4 && co < a.Co && p0 < a.Npix;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (valid) {
        int g = g0 + grp;
        if (grp == 0) {
            v = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g0, first_slot))[e4];
            g += 4;
        }
        for (; g + 12 <= g1; g += 16) {
            float4 p[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) p[q] = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g + 4 * q, 0))[e4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v.x += p[q].x;
                v.y += p[q].y;
                v.z += p[q].z;
                v.w += p[q].w;
            }
        }
        for (; g <= g1; g += 4) {
            const float4 p = reinterpret_cast<const float4*>(partial_slot<T>(a.ws, g, 0))[e4];
            v.x += p.x;
            v.y += p.y;
            v.z += p.z;
            v.w += p.w;
        }
    }
    if (grp > 0) part[grp - 1][lane] = v;
    __syncthreads();
    if (grp > 0 || !valid) return;
#pragma unroll
    for (int q = 0; q < 3; ++q) {
        const float4 p = part[q][lane];
        v.x += p.x;
        v.y += p.y;
        v.z += p.z;
        v.w += p.w;
    }
    fixup_store(a, co, p0, v);
}

// The fixup launch of a stream-K conv. The split kernel only where the
// plain one leaves the GPU nearly empty (at most kSplitFixupGroups
// workgroups) and each shared tile has at least kSplitFixupParts partials:
// ResNet-18's layers 3 and 4 at batch 1 (+1.3%); with larger grids its 4x
// workgroups measured slower (batch 8 -3 to -12%).
static constexpr int kSplitFixupParts = 16, kSplitFixupGroups = 64;
template <class T>
static void launch_conv_fixup(ConvArgs& a, const StreamK& sk) {
    set_work(0.0, 0.0);
    const int64_t per = sk.total() / sk.G;  // slices per workgroup range (>= 1)
    const int64_t parts = (sk.iters + per - 1) / per + 1;
    if (parts >= kSplitFixupParts && (int64_t)(T::BM * T::BN / 1024) * sk.sk_tiles <= kSplitFixupGroups)
        launch("conv_streamk_fixup", conv_fixup_split_k<T>, dim3(T::BM * T::BN / 256, sk.sk_tiles), dim3(256), 0, a,
               sk);
    else
        launch("conv_streamk_fixup", conv_fixup_k<T>, dim3(T::BM * T::BN / 1024, sk.sk_tiles), dim3(256), 0, a, sk);
}

// Reference-layout weights [Co][Ci][T] to tap-major [Co][T][Ci] (T = kh*kw),
// so that reference-layout 3x3 calls reach the direct-to-LDS kernel. One
// thread per output element: writes coalesce, reads stride T (cached).
__global__ void __launch_bounds__(256) repack_taps_k(const float* w, float* wp, int Ci, int T, int64_t n) {
    const int64_t o = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (o >= n) return;
    const int ci = (int)(o % Ci);
    const int64_t rest = o / Ci;  // co * T + t
    const int t = (int)(rest % T);
    const int64_t co = rest / T;
    wp[o] = w[(co * Ci + ci) * T + t];
}

// direct-to-LDS kernels finish shared stream-K tiles themselves when a tile
// has at most kMaxInKernelParts partials
static constexpr bool kInKernelFixup = true;
// reference-layout 3x3 convolutions from this much work on are repacked
static constexpr double kRepackMinFlops = 1e9;
static constexpr int kMaxInKernelParts = 4;

typedef Tile<128, 128, 32, 2, 2> ConvT128;  // Co >= 128: 2x2 blocks per wave
typedef Tile<64, 128, 32, 1, 4> ConvT64;    // Co == 64, many pixels: 2x1 blocks per wave
typedef Tile<64, 64, 32, 2, 2> ConvTSmall;  // short K or few pixels: 1 block per wave

template <class T, int KH, int KW, bool AVEC>
static void launch_conv_t(ConvArgs& a, const char* entry) {
    auto kernel = conv_streamk_k<T, KH, KW, AVEC>;
    const size_t lds = (size_t)T::LDS_FLOATS * sizeof(float);
    // once per kernel, thread-safe (C++ static initialisation): the LDS limit
    // and the persistent grid size; -1 if the attribute could not be set
    static const int slots = [&] {
        if (hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
            return -1;
        return resident_groups(kernel, lds);
    }();
    if (slots < 0) return fail(NNC_HIP_EDEVICE, entry, "hipFuncSetAttribute failed");
    // K == 0 (no input channels) still runs one empty slice so the epilogue
    // writes act(bias)
    const int iters = a.K > 0 ? (int)ceil_div(a.K, T::BK) : 1;
    const StreamK sk = plan_streamk(a.tiles_m * a.tiles_n, iters, slots, fixup_slices<T>());
    if (sk.G < 1) return;
    const size_t ws_bytes = (size_t)sk.G * 2 * T::BM * T::BN * sizeof(float);
    float* ws = workspace(ws_bytes);
    if (!ws) return partials_fail(entry, ws_bytes);
    a.ws = ws;
    char name[64];
    if (KH > 0)
        snprintf(name, sizeof name, "conv_igemm_%dx%d_k%dx%d_%s", T::BM, T::BN, KH, KW, AVEC ? "v4" : "s1");
    else
        snprintf(name, sizeof name, "conv_igemm_%dx%d_kany_%s", T::BM, T::BN, AVEC ? "v4" : "s1");
    set_work(2.0 * a.Co * (double)a.Npix * a.K, 0.0);
    launch(name, kernel, dim3(sk.G), dim3(256), lds, a, sk);
    if (sk.needs_fixup()) launch_conv_fixup<T>(a, sk);
}

// Clears tile counters held in fixed scratch, which keeps whatever the last
// call on the device left there.
__global__ void __launch_bounds__(256) zero_counters_k(int* p, int n) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = 0;
}

template <class T, class L>
static void launch_conv_dma_t(ConvArgs& a, const char* entry, const char* name) {
    // the in-kernel finish only where it measured faster than the fixup
    // kernel (64x128 tiles: ResNet's 64-channel layers and the stem);
    // elsewhere its code costs the main loop registers (128x128 tiles on
    // ResNet-18's batch-32 layers: 62.0 -> 69.0 us per launch, the
    // finishing workgroups' partial reads on the kernel's critical path)
    constexpr bool FIN = kInKernelFixup && L::kFinishInKernel && T::NW == 4 && T::BM == 64 && T::BN == 128;
    auto kernel = conv_dma_k<T, L, FIN>;
    const size_t lds = (size_t)(DmaStage<T>::LDS_FLOATS + L::EXTRA_LDS_FLOATS) * sizeof(float);
    // once per kernel, thread-safe (C++ static initialisation): the LDS limit
    // and the persistent grid size; -1 if the attribute could not be set
    static const int slots = [&] {
        if (hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
            return -1;
        return resident_groups(kernel, lds, T::THREADS);
    }();
    if (slots < 0) return fail(NNC_HIP_EDEVICE, entry, "hipFuncSetAttribute failed");
    // K == 0 (no input channels) still runs one empty slice so the epilogue
    // writes act(bias)
    const int iters = a.K > 0 ? (int)ceil_div(a.K, T::BK) : 1;
    const StreamK sk = plan_streamk(a.tiles_m * a.tiles_n, iters, slots, fixup_slices<T>());
    if (sk.G < 1) return;
    const size_t ws_bytes = (size_t)sk.G * 2 * T::BM * T::BN * sizeof(float);
    float* ws = workspace(ws_bytes);
    if (!ws) return partials_fail(entry, ws_bytes);
    a.ws = ws;
    // shared tiles with at most kMaxInKernelParts contributors are finished
    // inside the kernel by the last to arrive; tiles split further (short
    // problems) by the fixup kernel, which spreads the sum over many
    // workgroups; so also when no counters can be had (capture before growth)
    const int64_t per = sk.total() / sk.G;  // slices per workgroup range (>= 1)
    const bool in_kernel = FIN && sk.needs_fixup() && (sk.iters + per - 1) / per + 1 <= kMaxInKernelParts;
    a.cnt = in_kernel ? tile_counters((size_t)sk.sk_tiles) : nullptr;
    if (a.cnt && ts().fixed)
        launch("zero_tile_counters", zero_counters_k, dim3((unsigned)ceil_div(sk.sk_tiles, 256)), dim3(256), 0, a.cnt,
               (int)sk.sk_tiles);
    set_work(2.0 * a.Co * (double)a.Npix * a.K, 0.0);
    launch(name, kernel, dim3(sk.G), dim3(T::THREADS), lds, a, sk);
    if (sk.needs_fixup() && !a.cnt) launch_conv_fixup<T>(a, sk);
}

template <class T, int KH, int KW>
static void launch_conv_dma(ConvArgs& a, const char* entry) {
    char name[64];
    snprintf(name, sizeof name, "conv_igemm_%dx%d_k%dx%d_dma", T::BM, T::BN, KH, KW);
    launch_conv_dma_t<T, DmaPacked<T, KH, KW>>(a, entry, name);
}

template <int NS, bool PROJ>
static void launch_ws_ns(const ConvArgs& a, int S, int iters, unsigned grid, const char* name) {
    launch(name, conv_ws_k<NS, PROJ>, dim3(grid), dim3(256), 0, a, S, iters);
}

// conv_ws_k where plan_ws (plan.h) takes the convolution. Needs tap-major
// packed weights (k = tap * Ci + ci, then the projection's channels), Ci
// (and the projection's channels) multiples of 32, 16-byte aligned weights,
// at most 32 taps: checked by the callers. Returns false (nothing launched)
// where plan_ws declines or the split's scratch cannot be had (capture
// before growth); the caller then takes its usual path.
template <bool PROJ>
static bool launch_conv_ws(ConvArgs& a, const char* entry) {
    WsPlan wp;
    if (!plan_ws(a.Co, a.Npix, a.K, wp)) return false;
    const int64_t tiles = wp.tiles;
    const int iters = wp.iters, S = wp.S, NS = wp.NS;
    a.tiles_m = (int)ceil_div(a.Co, 32);
    a.tiles_n = (int)ceil_div(a.Npix, 32);
    a.ws = nullptr;
    a.cnt = nullptr;
    if (S > 1) {
        a.ws = workspace((size_t)tiles * S * 4096);
        a.cnt = a.ws ? tile_counters((size_t)tiles) : nullptr;
        if (!a.cnt) return false;
        if (ts().fixed)
            launch("zero_tile_counters", zero_counters_k, dim3((unsigned)ceil_div(tiles, 256)), dim3(256), 0, a.cnt,
                   (int)tiles);
    }
    char name[64];
    snprintf(name, sizeof name, "conv_ws_32x32_k%dx%d%s", a.kh, a.kw, PROJ ? "p" : "");
    set_work(2.0 * a.Co * (double)a.Npix * a.K, 0.0);
    const unsigned grid = (unsigned)(tiles * S);
    switch (NS) {
        case 1: launch_ws_ns<1, PROJ>(a, S, iters, grid, name); break;
        case 2: launch_ws_ns<2, PROJ>(a, S, iters, grid, name); break;
        case 3: launch_ws_ns<3, PROJ>(a, S, iters, grid, name); break;
        case 4: launch_ws_ns<4, PROJ>(a, S, iters, grid, name); break;
        case 5: launch_ws_ns<5, PROJ>(a, S, iters, grid, name); break;
        default: launch_ws_ns<6, PROJ>(a, S, iters, grid, name); break;
    }
    (void)entry;
    return true;
}

// ---------------------------------------------------------------------------
// The RGB stem (3 channels, 7x7, stride 2, pad 3, H == 2 Ho, W == 2 Wo,
// Wo = 16 * BPR, Co <= 64) as a persistent kernel over output rows. A tile
// is one output row of one image: 64 channels x Wo pixels. Its input
// window, the 7 input rows x 3 channels it reads, goes into LDS with
// 16-byte direct-to-LDS loads (a row of W floats at offset 4 of an LDS row
// of W + 8, whose 4 + 4 pad columns stay zero: the left and right image
// padding), double-buffered: the next tile's window loads while this one
// computes. The contraction then reads its B operand straight out of the
// window (im2col on the read side: k = tap * 3 + ci of the packed weight
// rows -> LDS row (ci, ky), column 2 ox + kx + 1), so the input crosses the
// memory system once per tile as wide loads instead of one 4-byte gather
// per k and pixel. MFMA 16x16x4 computing out^T (pixels x channels): wave w
// owns output channels 16w..16w+15 and all Wo / 16 pixel blocks of the row;
// its weights (K = 147 in 37 steps of 4) stay in registers for the whole
// kernel, and each lane ends with 4 consecutive pixels of one channel: one
// 16-byte store per block.
//   v_mfma_f32_16x16x4_f32, lane l: A[i = l % 16][k = l / 16] (window: pixel
//   i), B[k = l / 16][j = l % 16] (weights: channel j), D register r:
//   D[i = 4 (l / 16) + r][j = l % 16]
// ---------------------------------------------------------------------------
struct StemArgs {
    const float* in;
    const float* w;  // [Co][ldw], k = tap * 3 + ci, zero past 147
    const float* bias;
    float* out;
    int N, H, W, Co, Ho, Wo, ldw, act, tiles;
};

static constexpr int kStemK = 147, kStemSteps = 37;  // 3 * 7 * 7, rounded up to steps of 4

// LDS requested per workgroup: at most two workgroups per CU, so that a
// grid of 2 per CU puts exactly two on every CU (tiles spread evenly)
static constexpr int kStemLdsBytes = 56 * 1024;

template <int BPR>
struct StemShape {
    static constexpr int WO = 16 * BPR, W = 2 * WO, LW = W + 8;  // LDS row: 4 pad, W data, 4 pad
    static constexpr int CP = 7 * LW, BUF = 3 * CP;              // channel pitch, one window
    static constexpr int CHUNKS = W / 4;                         // 16-byte pieces per input row
    static_assert(CHUNKS <= 64, "one load instruction per input row");
    static_assert(2 * BUF * 4 <= kStemLdsBytes, "two windows in the requested LDS");
};

// one tile's window: rows (ci, ky) of input row 2 oy - 3 + ky, wave w
// loading rows w, w + 4, ...; rows outside the image read as zeros
template <int BPR>
__device__ __forceinline__ void stem_window(const StemArgs& a, __amdgpu_buffer_rsrc_t rin, float* buf, int t,
                                            int wave, int lane) {
    typedef StemShape<BPR> S;
    const int n = t / a.Ho, oy = t - n * a.Ho;
    for (int r = wave; r < 21; r += 4) {
        const int ci = r / 7, ky = r - ci * 7;
        const int iy = 2 * oy - 3 + ky;
        const bool in_img = iy >= 0 && iy < a.H;
        const uint32_t voff =
            in_img ? (uint32_t)(((n * 3 + ci) * a.H + iy) * a.W) * 4u + (uint32_t)lane * 16u : kOutOfRange;
        if (lane < S::CHUNKS) dma_load16(rin, buf + ci * S::CP + ky * S::LW + 4, voff, 0);
    }
}

template <int BPR>
__global__ void __launch_bounds__(256, 2) __attribute__((amdgpu_waves_per_eu(2, 2))) conv_stem_k(StemArgs a) {
    typedef StemShape<BPR> S;
    extern __shared__ __align__(16) float lds[];  // [2][3 ci][7 ky][LW]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kq = lane >> 4;
    const int G = gridDim.x;
    int t = xcd_remap(blockIdx.x, G);
    if (t >= a.tiles) return;  // the host launches at most `tiles` workgroups
    const __amdgpu_buffer_rsrc_t rin = make_rsrc(a.in);
    // zero pad columns of both windows, once (the loads never write them)
    for (int r = threadIdx.x; r < 2 * 3 * 7; r += 256) {
        float* lrow = lds + r * S::LW;
        *reinterpret_cast<float4*>(lrow) = make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(lrow + 4 + S::W) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    stem_window<BPR>(a, rin, lds, t, wave, lane);
    if (t + G < a.tiles) stem_window<BPR>(a, rin, lds + S::BUF, t + G, wave, lane);
    // weights of this wave's 16 channels (rows past Co read as zeros) and
    // the per-step window offsets of this lane's k
    const int co_a = 16 * wave + j;  // also this lane's output channel
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.w), (short)0, a.Co * a.ldw * 4, 0x00020000);
    float A[kStemSteps];
    int koff[kStemSteps];
#pragma unroll
    for (int s = 0; s < kStemSteps; ++s) {
        const int k = 4 * s + kq;
        A[s] = load_f32(rw, (uint32_t)(co_a * a.ldw + k) * 4u);
        const int tap = k / 3, ci = k - tap * 3, ky = tap / 7, kx = tap - ky * 7;
        koff[s] = k < kStemK ? ci * S::CP + ky * S::LW + kx + 1 + 2 * j : 0;
    }
    const float bias = a.bias && co_a < a.Co ? a.bias[co_a] : 0.f;
    dma_barrier<0>();  // both windows landed, pad columns written
    for (int i = 0; t < a.tiles; ++i, t += G) {
        const float* B = lds + (i & 1) * S::BUF;
        f32x4 acc[BPR];
#pragma unroll
        for (int b = 0; b < BPR; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        // B values one step ahead of the MFMAs that use them
        float x[BPR];
#pragma unroll
        for (int b = 0; b < BPR; ++b) x[b] = B[koff[0] + 32 * b];
#pragma unroll
        for (int s = 0; s < kStemSteps; ++s) {
            float xn[BPR];
            if (s + 1 < kStemSteps) {
#pragma unroll
                for (int b = 0; b < BPR; ++b) xn[b] = B[koff[s + 1] + 32 * b];
            }
            if (s == kStemSteps - 1 && 4 * s + kq >= kStemK) {
#pragma unroll
                for (int b = 0; b < BPR; ++b) x[b] = 0.f;  // k past K: no input term, not even 0 * inf
            }
#pragma unroll
            for (int b = 0; b < BPR; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[b], A[s], acc[b], 0, 0, 0);
            if (s + 1 < kStemSteps) {
#pragma unroll
                for (int b = 0; b < BPR; ++b) x[b] = xn[b];
                // schedule the next step's LDS reads ahead of this step's
                // MFMAs (left alone, the scheduler waits on each read right
                // before its MFMA)
                __builtin_amdgcn_sched_group_barrier(0x100, (BPR + 1) / 2, 0);  // DS reads (paired)
                __builtin_amdgcn_sched_group_barrier(0x008, BPR, 0);            // MFMAs
            }
        }
        // the next window landed (loaded a whole tile ago) and every wave is
        // done with this one: refill it with the tile after next
        dma_barrier<0>();
        if (t + 2 * G < a.tiles) stem_window<BPR>(a, rin, lds + (i & 1) * S::BUF, t + 2 * G, wave, lane);
        const int n = t / a.Ho, oy = t - n * a.Ho;
        if (co_a < a.Co) {
            float* orow = a.out + (((int64_t)n * a.Co + co_a) * a.Ho + oy) * a.Wo + 4 * kq;
#pragma unroll
            for (int b = 0; b < BPR; ++b) {
                // element copies first: bit_cast of an ext-vector element is miscompiled
                const float v0 = acc[b][0], v1 = acc[b][1], v2 = acc[b][2], v3 = acc[b][3];
                *reinterpret_cast<float4*>(orow + 16 * b) =
                    make_float4(activate(v0 + bias, a.act), activate(v1 + bias, a.act), activate(v2 + bias, a.act),
                                activate(v3 + bias, a.act));
            }
        }
    }
}

template <int BPR>
static void launch_conv_stem_rows(const ConvArgs& c, const char* entry) {
    auto kernel = conv_stem_k<BPR>;
    static const int ok = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              kStemLdsBytes) == hipSuccess;
    if (!ok) return fail(NNC_HIP_EDEVICE, entry, "hipFuncSetAttribute failed");
    StemArgs a{c.in, c.w, c.bias, c.out, c.N, c.H, c.W, c.Co, c.Ho, c.Wo, c.ldw, c.act, c.N * c.Ho};
    // two workgroups on every CU, each taking every G-th row
    const int G = std::min(a.tiles, 2 * cu_count());
    set_work(2.0 * c.Co * (double)c.Npix * kStemK, 0.0);
    char name[64];
    snprintf(name, sizeof name, "conv_stem_rows_w%d", 16 * BPR);
    launch(name, kernel, dim3(G), dim3(256), kStemLdsBytes, a);
}

// The row kernel's shapes: ResNet's 224x224 stem (Wo 112) and 64x64 inputs,
// once there are at least two rows per CU (ResNet-18 stem on MI355X: batch
// 32 118.6 -> 90.8 us, batch 8 43.5 -> 32.3 us against the 64x128 tile
// kernel; batch 1, 112 rows, 9.9 -> 13.5 us, so the tile kernel keeps it).
// Tiles of two rows (8-wave workgroups, one per CU, one 9-row window for
// both rows) measured slower: 94.7 / 35.7 / 21.0 us.
static bool conv_stem_rows(const ConvArgs& a, const char* entry) {
    if (!(a.sh == 2 && a.sw == 2 && a.ph == 3 && a.pw == 3 && a.H == 2 * a.Ho && a.W == 2 * a.Wo && a.Co <= 64 &&
          !a.res && a.ldw >= 4 * kStemSteps && aligned16(a.in) && aligned16(a.out) && a.N * a.Ho < (1 << 30) &&
          a.N * a.Ho >= 2 * cu_count()))
        return false;
    if (a.Wo == 112) return launch_conv_stem_rows<7>(a, entry), true;
    if (a.Wo == 32) return launch_conv_stem_rows<2>(a, entry), true;
    return false;
}

// ---------------------------------------------------------------------------
// The stem's row kernel with the 3x3 / stride 2 / pad 1 max pool of its relu
// output folded in (nnc_hip_conv_maxpool where the unfused stem runs
// conv_stem_k): the conv rows of all images, in order, split into G
// contiguous ranges of two or more rows, one per workgroup, each row
// computed as in conv_stem_k (the next row's window loading during the
// current row). Per row: bias + relu, then the max over conv columns 2j-1,
// 2j, 2j+1 - a lane's four pixels 4q .. 4q+3 give pool columns 2q and 2q+1,
// pixel 4q-1 comes from the lane 16 below (for the first lane group, the
// previous block's last), the image's padding column counts as 0 - then down
// the rows in registers: row 2p starts pool row p (with row 2p-1's maxima
// when the range holds it), row 2p+1 completes it and it is stored. A
// range's first pool row lacks the rows before the range unless the range
// starts an image: the previous range writes its last maxima to pb.side
// (with ranges of two or more rows, at most one range boundary falls inside
// a pool row's three conv rows). Both ranges of a boundary write their part
// with device-scope stores and count themselves in on the boundary's
// counter (pb.cnt) at the end, and the second to arrive takes the max and
// writes the pool row (the stream-K finish's protocol, finish_arrive_pair).
// Relu values are never
// NaN or -0 and all are >= 0, so the max is exact: the same bits as
// nnc_maxpool2d over conv_stem_k's output.
template <int BPR>
__global__ void __launch_bounds__(256, 2) __attribute__((amdgpu_waves_per_eu(2, 2)))
conv_stem_pool_k(StemArgs a, PoolBand pb) {
    typedef StemShape<BPR> S;
    extern __shared__ __align__(16) float lds[];  // [2][3 ci][7 ky][LW]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int j = lane & 15, kq = lane >> 4;
    const int G = gridDim.x;
    const int g = xcd_remap(blockIdx.x, G);
    const int t0 = (int)((int64_t)g * a.tiles / G), t1 = (int)((int64_t)(g + 1) * a.tiles / G);
    if (t0 >= t1) return;  // (the host gives every range two or more rows)
    const __amdgpu_buffer_rsrc_t rin = make_rsrc(a.in);
    for (int r = threadIdx.x; r < 2 * 3 * 7; r += 256) {
        float* row = lds + r * S::LW;
        *reinterpret_cast<float4*>(row) = make_float4(0.f, 0.f, 0.f, 0.f);
        *reinterpret_cast<float4*>(row + 4 + S::W) = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    stem_window<BPR>(a, rin, lds, t0, wave, lane);
    if (t0 + 1 < t1) stem_window<BPR>(a, rin, lds + S::BUF, t0 + 1, wave, lane);
    const int co_a = 16 * wave + j;  // also this lane's output channel
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.w), (short)0, a.Co * a.ldw * 4, 0x00020000);
    float A[kStemSteps];
    int koff[kStemSteps];
#pragma unroll
    for (int s = 0; s < kStemSteps; ++s) {
        const int k = 4 * s + kq;
        A[s] = load_f32(rw, (uint32_t)(co_a * a.ldw + k) * 4u);
        const int tap = k / 3, ci = k - tap * 3, ky = tap / 7, kx = tap - ky * 7;
        koff[s] = k < kStemK ? ci * S::CP + ky * S::LW + kx + 1 + 2 * j : 0;
    }
    const float bias = a.bias && co_a < a.Co ? a.bias[co_a] : 0.f;
    dma_barrier<0>();
    float run[BPR][2];  // maxima of the current pool row's rows so far
    bool have = false;
    // boundaries shared with the neighbouring ranges (counted in at the end)
    const bool start_shared = g > 0 && t0 % a.Ho != 0;
    const bool end_shared = t1 < a.tiles && (t1 - 1) % a.Ho + 1 < a.Ho;
    const __amdgpu_buffer_rsrc_t rout = make_rsrc(pb.out), rside = make_rsrc(pb.side);
    float first[BPR][2];  // this range's part of its first pool row (start_shared)
    bool first_pending = start_shared;
    for (int t = t0, i = 0; t < t1; ++t, ++i) {
        const float* B = lds + (i & 1) * S::BUF;
        f32x4 acc[BPR];
#pragma unroll
        for (int b = 0; b < BPR; ++b) acc[b] = f32x4{0.f, 0.f, 0.f, 0.f};
        float x[BPR];
#pragma unroll
        for (int b = 0; b < BPR; ++b) x[b] = B[koff[0] + 32 * b];
#pragma unroll
        for (int s = 0; s < kStemSteps; ++s) {
            float xn[BPR];
            if (s + 1 < kStemSteps) {
#pragma unroll
                for (int b = 0; b < BPR; ++b) xn[b] = B[koff[s + 1] + 32 * b];
            }
            if (s == kStemSteps - 1 && 4 * s + kq >= kStemK) {
#pragma unroll
                for (int b = 0; b < BPR; ++b) x[b] = 0.f;
            }
#pragma unroll
            for (int b = 0; b < BPR; ++b) acc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(x[b], A[s], acc[b], 0, 0, 0);
            if (s + 1 < kStemSteps) {
#pragma unroll
                for (int b = 0; b < BPR; ++b) x[b] = xn[b];
                __builtin_amdgcn_sched_group_barrier(0x100, (BPR + 1) / 2, 0);
                __builtin_amdgcn_sched_group_barrier(0x008, BPR, 0);
            }
        }
        dma_barrier<0>();
        if (t + 2 < t1) stem_window<BPR>(a, rin, lds + (i & 1) * S::BUF, t + 2, wave, lane);
        const int n = t / a.Ho, y = t - n * a.Ho;
        // bias + relu, then the horizontal maxima
        float h[BPR][2];
        float prev3 = 0.f;  // this lane's last pixel of the previous block (0: the padding column)
#pragma unroll
        for (int b = 0; b < BPR; ++b) {
            // element copies first: bit_cast of an ext-vector element is miscompiled
            const float e0 = acc[b][0], e1 = acc[b][1], e2 = acc[b][2], e3 = acc[b][3];
            const float v0 = activate(e0 + bias, kActRelu), v1 = activate(e1 + bias, kActRelu);
            const float v2 = activate(e2 + bias, kActRelu), v3 = activate(e3 + bias, kActRelu);
            // the pixel left of a lane's four sits in the lane 16 below; the
            // first lane group's in the last group's previous block
            const float left = __shfl(kq == 3 ? prev3 : v3, (lane + 48) & 63);
            prev3 = v3;
            h[b][0] = fmaxf(fmaxf(left, v0), v1);
            h[b][1] = fmaxf(fmaxf(v1, v2), v3);
        }
        if (y == 0) have = false;  // an image's first row
        if ((y & 1) == 0) {
#pragma unroll
            for (int b = 0; b < BPR; ++b)
#pragma unroll
                for (int k = 0; k < 2; ++k) run[b][k] = have ? fmaxf(run[b][k], h[b][k]) : h[b][k];
        } else {
            if (co_a < a.Co) {
                const int64_t oe = (((int64_t)n * a.Co + co_a) * pb.Hp + (y >> 1)) * pb.Wp + 2 * kq;
#pragma unroll
                for (int b = 0; b < BPR; ++b) {
                    const float m0 = have ? fmaxf(run[b][0], h[b][0]) : h[b][0];
                    const float m1 = have ? fmaxf(run[b][1], h[b][1]) : h[b][1];
                    if (first_pending) {  // the shared pool row: for the finishing range
                        first[b][0] = m0;
                        first[b][1] = m1;
                        store_partial(rout, (uint32_t)(oe + 8 * b) * 4u, m0);
                        store_partial(rout, (uint32_t)(oe + 8 * b + 1) * 4u, m1);
                    } else {
                        *reinterpret_cast<float2*>(pb.out + oe + 8 * b) = make_float2(m0, m1);
                    }
                }
            }
            first_pending = false;
#pragma unroll
            for (int b = 0; b < BPR; ++b)
#pragma unroll
                for (int k = 0; k < 2; ++k) run[b][k] = h[b][k];  // row 2p+1 also starts pool row p+1
        }
        have = true;
    }
    // the range's last maxima: the rows the next range's first pool row
    // lacks (device-scope stores: the next range may read them in-kernel)
    if (end_shared && co_a < a.Co) {
        const uint32_t se = (uint32_t)(((int64_t)g * a.Co + co_a) * pb.Wp + 2 * kq) * 4u;
#pragma unroll
        for (int b = 0; b < BPR; ++b) {
            store_partial(rside, se + 32u * b, run[b][0]);
            store_partial(rside, se + 32u * b + 4u, run[b][1]);
        }
    }
    bool last_start, last_end;
    finish_arrive_pair(pb.cnt + g, start_shared, pb.cnt + g + 1, end_shared, last_start, last_end);
    if (co_a >= a.Co) return;
    // every load of a finish before its stores (the next range's part is
    // read from, and its max written to, the same addresses)
    if (last_start) {  // this range's first pool row with the previous range's last maxima
        const int n = t0 / a.Ho;
        const int64_t oe = (((int64_t)n * a.Co + co_a) * pb.Hp + ((t0 % a.Ho) >> 1)) * pb.Wp + 2 * kq;
        const uint32_t se = (uint32_t)(((int64_t)(g - 1) * a.Co + co_a) * pb.Wp + 2 * kq) * 4u;
        float sv[BPR][2];
#pragma unroll
        for (int b = 0; b < BPR; ++b) {
            sv[b][0] = load_partial(rside, se + 32u * b);
            sv[b][1] = load_partial(rside, se + 32u * b + 4u);
        }
#pragma unroll
        for (int b = 0; b < BPR; ++b)
            *reinterpret_cast<float2*>(pb.out + oe + 8 * b) =
                make_float2(fmaxf(first[b][0], sv[b][0]), fmaxf(first[b][1], sv[b][1]));
    }
    if (last_end) {  // the next range's first pool row with this range's last maxima
        const int n = t1 / a.Ho;
        const int64_t oe = (((int64_t)n * a.Co + co_a) * pb.Hp + ((t1 % a.Ho) >> 1)) * pb.Wp + 2 * kq;
        float pv[BPR][2];
#pragma unroll
        for (int b = 0; b < BPR; ++b) {
            pv[b][0] = load_partial(rout, (uint32_t)(oe + 8 * b) * 4u);
            pv[b][1] = load_partial(rout, (uint32_t)(oe + 8 * b + 1) * 4u);
        }
#pragma unroll
        for (int b = 0; b < BPR; ++b)
            *reinterpret_cast<float2*>(pb.out + oe + 8 * b) =
                make_float2(fmaxf(run[b][0], pv[b][0]), fmaxf(run[b][1], pv[b][1]));
    }
}

template <class T>
static void launch_conv_stem(ConvArgs& a, const char* entry) {
    a.tiles_m = (int)ceil_div(a.Co, T::BM);
    a.tiles_n = (int)ceil_div(a.Npix, T::BN);
    char name[64];
    snprintf(name, sizeof name, "conv_igemm_%dx%d_k7x7c3_dma", T::BM, T::BN);
    launch_conv_dma_t<T, DmaSmallC<T, 7, 7, 3>>(a, entry, name);
}

// `dma`: weights tap-major [Co][kh][kw][Ci] (or 1x1), Ci % 32 == 0, kernel
// 1x1 or 3x3, weights 16-byte aligned; checked by the caller.
template <class T>
static void launch_conv(ConvArgs& a, bool avec, bool dma, const char* entry) {
    if (dma && launch_conv_ws<false>(a, entry)) return;
    a.tiles_m = (int)ceil_div(a.Co, T::BM);
    a.tiles_n = (int)ceil_div(a.Npix, T::BN);
    if (dma) {
        if (a.kh == 3) return launch_conv_dma<T, 3, 3>(a, entry);
        return launch_conv_dma<T, 1, 1>(a, entry);
    }
#define NNC_CONV_KS(KH, KW)                                                 \
    if (avec) launch_conv_t<T, KH, KW, true>(a, entry);                     \
    else launch_conv_t<T, KH, KW, false>(a, entry);                         \
    return;
    if (a.kh == 1 && a.kw == 1) { NNC_CONV_KS(1, 1) }
    if (a.kh == 3 && a.kw == 3) { NNC_CONV_KS(3, 3) }
    if (a.kh == 7 && a.kw == 7) { NNC_CONV_KS(7, 7) }
    NNC_CONV_KS(0, 0)
#undef NNC_CONV_KS
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

// nnc_hip_conv_packed: weights [Co][kh][kw][Ci] or [Co][Kp]
static bool conv_check_packed(Tensor* in, Tensor* w, Tensor* out, const char* name) {
    if (w && w->shape && w->ndim == 2) {
        int64_t shape4[4] = {w->shape[0], w->shape[1], 1, 1};
        Tensor w4 = *w;
        w4.ndim = 4;
        w4.shape = shape4;
        return conv_check(in, &w4, out, name);
    }
    return conv_check(in, w, out, name);
}

// `packed`: the weights are [Co][kh][kw][Ci] (nnc_hip_conv_packed)
static void conv_run(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw,
                     int ph, int pw, int act, const char* name, Tensor* res = nullptr, bool packed = false) {
    ConvArgs a{};
    a.res = res ? (const float*)res->data : nullptr;
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
    if (res && numel(res) < (int64_t)a.N * a.Co * out->shape[2] * out->shape[3])
        return fail(NNC_HIP_EINVAL, name, "residual smaller than the output");
    const int64_t K = (int64_t)a.Ci * kh * kw;
    const int64_t npix = (int64_t)a.N * a.Ho * a.Wo;
    // the kernels address input and weights with 32-bit byte offsets
    const int64_t in_bytes = (int64_t)a.N * a.Ci * a.H * a.W * 4;
    const int64_t w_bytes = (int64_t)a.Co * K * 4;
    if (K >= (1 << 30) || npix >= (1 << 30) || in_bytes >= ((int64_t)1 << 31) || w_bytes >= ((int64_t)1 << 31))
        return fail(NNC_HIP_EUNSUPP, name, "input or weights of 2 GiB or more");
    a.K = (int)K;
    a.ldw = (int)K;
    a.Npix = (int)npix;
    a.vec_out = aligned16(a.out) && (!a.res || aligned16(a.res));
    a.out32 = (int64_t)a.N * a.Co * a.Ho * a.Wo * 4 < ((int64_t)1 << 31);
    // direct-to-LDS kernels: tap-major weights (1x1 weights already are)
    const bool dma_ok = a.Ci % 32 == 0 && aligned16(a.w) && ((kh == 3 && kw == 3) || (kh == 1 && kw == 1));
    bool stem = false;
    if (packed && w->ndim == 2) {
        // [Co][Kp], K padded with zeros to a multiple of 32: the RGB 7x7 stem
        const int64_t kp = (K + 31) / 32 * 32;
        if (w->shape[1] != kp) return fail(NNC_HIP_EINVAL, name, "packed weight row is not K rounded up to 32");
        if (!(kh == 7 && kw == 7 && a.Ci == 3 && aligned16(a.w)))
            return fail(NNC_HIP_EUNSUPP, name, "[Co][Kp] packed weights need a 7x7 kernel, 3 channels, alignment");
        if (a.Co * kp * 4 >= ((int64_t)1 << 31)) return fail(NNC_HIP_EUNSUPP, name, "weights of 2 GiB or more");
        if (kp > 256) return fail(NNC_HIP_EUNSUPP, name, "[Co][Kp] packed rows longer than 256");
        a.ldw = (int)kp;
        stem = true;
    } else if (packed) {
        if (w->shape[1] != kh || w->shape[2] != kw || w->shape[3] != a.Ci)
            return fail(NNC_HIP_EINVAL, name, "packed weight shape is not [Co][kh][kw][Ci]");
        if (!dma_ok)
            return fail(NNC_HIP_EUNSUPP, name,
                        "packed weights need Ci % 32 == 0, a 1x1 or 3x3 kernel and 16-byte alignment");
    }
    bool dma = dma_ok && (packed || (kh == 1 && kw == 1));
    if (a.N == 0 || a.Co == 0 || a.Ho <= 0 || a.Wo <= 0) return;
    // reference-layout 3x3 weights of a large convolution: a tap-major copy
    // (one small transpose kernel) pays for itself on the direct-to-LDS path
    if (dma_ok && !packed && kh == 3 && 2.0 * a.Co * (double)a.Npix * a.K >= kRepackMinFlops) {
        float* wp = repack_buffer((size_t)a.Co * a.K * sizeof(float));
        if (wp) {
            const int64_t n = (int64_t)a.Co * a.K;
            set_work(0.0, 8.0 * (double)n);
            launch("conv_repack_taps", repack_taps_k, dim3((unsigned)ceil_div(n, 256)), dim3(256), 0, a.w, wp, a.Ci,
                   kh * kw, n);
            a.w = wp;
            dma = true;
        }
    }
    if (stem) {
        if (conv_stem_rows(a, name)) return;
        // 64x128 tiles only once there are plenty of them (batch 32: 3136)
        if (a.Co <= 64 && a.Npix >= 65536)
            return launch_conv_stem<ConvT64>(a, name);
        return launch_conv_stem<ConvTSmall>(a, name);
    }
    const bool avec = (a.K % 4 == 0) && aligned16(a.w);
    // Tile choice (measured on ResNet-18 layers at batch 1 and 32): big tiles
    // pay off only for long contractions with enough output tiles; short
    // ones (1x1, the 3-channel stem) and small images run best on 64x64
    // tiles, whose shorter per-tile latency and larger tile count fill the
    // GPU.
    if (a.K >= 512 && a.Co >= 128 && a.Npix >= 1024)
        launch_conv<ConvT128>(a, avec, dma, name);
    else if (a.K >= 512 && a.Co <= 64 && a.Npix >= 4096)
        launch_conv<ConvT64>(a, avec, dma, name);
    else
        launch_conv<ConvTSmall>(a, avec, dma, name);
}

// nnc_hip_conv_maxpool: maxpool3x3/s2/p1(relu(conv(in, w) + b)) for the
// packed 3-channel stem ([Co][Kp] rows, Co <= 64) with conv rows of at most
// 128 pixels and even conv output sizes.
template <int BPR>
static void launch_conv_stem_pool(const ConvArgs& c, float* out, int Hp, int Wp, const char* entry) {
    auto kernel = conv_stem_pool_k<BPR>;
    static const int ok = hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                              kStemLdsBytes) == hipSuccess;
    if (!ok) return fail(NNC_HIP_EDEVICE, entry, "hipFuncSetAttribute failed");
    const int rows = c.N * c.Ho;
    const StemArgs a{c.in, c.w, c.bias, nullptr, c.N, c.H, c.W, c.Co, c.Ho, c.Wo, c.ldw, kActRelu, rows};
    // two workgroups on every CU, ranges of two or more rows
    const int G = std::min(2 * cu_count(), rows / 2);
    PoolBand pb{};
    pb.out = out;
    pb.Wr = c.Wo, pb.Hp = Hp, pb.Wp = Wp;
    const size_t side_bytes = (size_t)G * c.Co * Wp * sizeof(float);
    pb.side = workspace(side_bytes);
    if (!pb.side) return partials_fail(entry, side_bytes);
    // boundary counters: the ranges finish the shared pool rows themselves
    // (every thread state holds far more counters than G from its creation)
    pb.cnt = tile_counters((size_t)G);
    if (!pb.cnt) return fail(NNC_HIP_ENOMEM, entry, "no %d range-boundary counters", G);
    if (ts().fixed)
        launch("zero_tile_counters", zero_counters_k, dim3((unsigned)ceil_div(G, 256)), dim3(256), 0, pb.cnt, G);
    set_work(2.0 * c.Co * (double)rows * c.Wo * kStemK, 0.0);
    char name[64];
    snprintf(name, sizeof name, "conv_stem_pool_w%d", 16 * BPR);
    launch(name, kernel, dim3((unsigned)G), dim3(256), kStemLdsBytes, a, pb);
}

static void conv_maxpool_run(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph,
                             int pw, const char* name) {
    typedef ConvT64 T;
    typedef DmaSmallC<T, 7, 7, 3> L;
    if (!ready(name)) return;
    if (!has_data(in) || !has_data(w) || !has_data(out)) return fail(NNC_HIP_EINVAL, name, "NULL tensor or data");
    if (in->ndim != 4 || w->ndim != 2 || out->ndim != 4) return fail(NNC_HIP_EINVAL, name, "expected 4D in/out, [Co][Kp] w");
    ConvArgs a{};
    a.in = (const float*)in->data;
    a.w = (const float*)w->data;
    a.bias = (b && b->data) ? (const float*)b->data : nullptr;
    a.N = (int)in->shape[0];
    a.Ci = (int)in->shape[1];
    a.H = (int)in->shape[2];
    a.W = (int)in->shape[3];
    a.Co = (int)w->shape[0];
    a.kh = kh, a.kw = kw, a.sh = sh, a.sw = sw, a.ph = ph, a.pw = pw;
    a.act = kActRelu;
    if (!(kh == 7 && kw == 7 && a.Ci == 3)) return fail(NNC_HIP_EUNSUPP, name, "only the 3-channel 7x7 stem");
    if (sh <= 0 || sw <= 0 || ph < 0 || pw < 0) return fail(NNC_HIP_EINVAL, name, "bad stride/pad");
    const int Ho = (a.H + 2 * ph - kh) / sh + 1, Wr = (a.W + 2 * pw - kw) / sw + 1;
    const int64_t K = (int64_t)a.Ci * kh * kw, kp = (K + 31) / 32 * 32;
    if (w->shape[1] != kp) return fail(NNC_HIP_EINVAL, name, "packed weight row is not K rounded up to 32");
    if (a.Co < 1 || a.Co > 64 || Ho < 2 || Wr < 2 || Ho % 2 || Wr % 2 || Wr > 128)
        return fail(NNC_HIP_EUNSUPP, name, "needs Co <= 64 and even conv output sizes with rows of at most 128");
    const int Hp = Ho / 2, Wp = Wr / 2;
    if (out->shape[0] != a.N || out->shape[1] != a.Co || out->shape[2] != Hp || out->shape[3] != Wp)
        return fail(NNC_HIP_EINVAL, name, "output is not [N][Co][%d][%d]", Hp, Wp);
    if (a.bias && numel(b) < a.Co) return fail(NNC_HIP_EINVAL, name, "bias smaller than Co");
    if (!aligned16(a.w)) return fail(NNC_HIP_EUNSUPP, name, "weights not 16-byte aligned");
    const int64_t in_bytes = (int64_t)a.N * a.Ci * a.H * a.W * 4;
    const int64_t npix = (int64_t)a.N * Ho * 128;
    if (in_bytes >= ((int64_t)1 << 31) || npix >= (1 << 30)) return fail(NNC_HIP_EUNSUPP, name, "input of 2 GiB or more");
    if (a.N == 0) return;
    // where the unfused stem runs its row kernel, the pool folds into that
    // (the same convolution bits)
    if (sh == 2 && sw == 2 && ph == 3 && pw == 3 && a.H == 2 * Ho && a.W == 2 * Wr && (Wr == 112 || Wr == 32) &&
        aligned16(a.in) && aligned16(out->data) && kp >= 4 * kStemSteps && (int64_t)a.N * Ho >= 2 * cu_count() &&
        (int64_t)a.N * a.Co * Hp * Wp * 4 < ((int64_t)1 << 31)) {
        ConvArgs c = a;
        c.Ho = Ho;
        c.Wo = Wr;
        c.ldw = (int)kp;
        if (Wr == 112) return launch_conv_stem_pool<7>(c, (float*)out->data, Hp, Wp, name);
        return launch_conv_stem_pool<2>(c, (float*)out->data, Hp, Wp, name);
    }
    a.Ho = Ho;
    a.Wo = 128;  // rows of 128 pixels: one tile per conv row
    a.K = (int)K;
    a.ldw = (int)kp;
    a.Npix = (int)npix;
    auto kernel = conv_pool_k<T, L>;
    const size_t lds = (size_t)(DmaStage<T>::LDS_FLOATS + L::EXTRA_LDS_FLOATS) * sizeof(float);
    static const int slots = [&] {
        if (hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
            return -1;
        return resident_groups(kernel, lds, T::THREADS);
    }();
    if (slots < 0) return fail(NNC_HIP_EDEVICE, name, "hipFuncSetAttribute failed");
    PoolBand pb{};
    pb.out = (float*)out->data;
    pb.Wr = Wr, pb.Hp = Hp, pb.Wp = Wp;
    pb.pairs = a.N * Hp;
    const int G = slots < pb.pairs ? slots : pb.pairs;
    const size_t side_bytes = (size_t)G * a.Co * Wp * sizeof(float);
    pb.side = workspace(side_bytes);
    if (!pb.side) return partials_fail(name, side_bytes);
    set_work(2.0 * a.Co * (double)a.N * Ho * Wr * K, 0.0);
    launch("conv_igemm_64x128_k7x7c3_pool", kernel, dim3((unsigned)G), dim3(T::THREADS), lds, a, pb);
    if (G > 1) {
        set_work(0.0, 12.0 * (double)(G - 1) * a.Co * Wp);
        launch("conv_pool_fixup", conv_pool_fixup_k, dim3((unsigned)ceil_div((int64_t)a.Co * Wp, 256), G - 1),
               dim3(256), 0, pb, a.Co, Ho, G);
    }
}

template <class T>
static void launch_conv_proj(ConvArgs& a, const char* entry) {
    a.tiles_m = (int)ceil_div(a.Co, T::BM);
    a.tiles_n = (int)ceil_div(a.Npix, T::BN);
    char name[64];
    snprintf(name, sizeof name, "conv_igemm_%dx%d_k3x3p_dma", T::BM, T::BN);
    launch_conv_dma_t<T, DmaProj<T, 3, 3>>(a, entry, name);
}

// nnc_hip_conv_proj: act(conv3x3(in, w[:, :9*Ci]) + conv1x1(x, w[:, 9*Ci:],
// stride psh x psw) + bias); w packed [Co][9*Ci + Cx].
static void conv_proj_run(Tensor* in, Tensor* w, Tensor* b, Tensor* x, Tensor* out, int kh, int kw, int sh, int sw,
                          int ph, int pw, int psh, int psw, int act, const char* name) {
    if (!conv_check(in, x, out, name)) return;
    if (!w || !w->data || !w->shape || w->ndim != 2) return fail(NNC_HIP_EINVAL, name, "weights must be [Co][K]");
    if (!(kh == 3 && kw == 3)) return fail(NNC_HIP_EUNSUPP, name, "only 3x3 convolutions take a projection");
    if (sh <= 0 || sw <= 0 || ph < 0 || pw < 0 || psh <= 0 || psw <= 0)
        return fail(NNC_HIP_EINVAL, name, "bad stride/pad");
    ConvArgs a{};
    a.in = (const float*)in->data;
    a.w = (const float*)w->data;
    a.bias = (b && b->data) ? (const float*)b->data : nullptr;
    a.out = (float*)out->data;
    a.pin = (const float*)x->data;
    a.N = (int)in->shape[0];
    a.Ci = (int)in->shape[1];
    a.H = (int)in->shape[2];
    a.W = (int)in->shape[3];
    a.Co = (int)out->shape[1];
    a.Ho = (int)out->shape[2];
    a.Wo = (int)out->shape[3];
    a.pci = (int)x->shape[1];
    a.pH = (int)x->shape[2];
    a.pW = (int)x->shape[3];
    a.kh = kh;
    a.kw = kw;
    a.sh = sh;
    a.sw = sw;
    a.ph = ph;
    a.pw = pw;
    a.psh = psh;
    a.psw = psw;
    a.act = act;
    const int64_t K = (int64_t)a.Ci * kh * kw + a.pci;
    if (w->shape[0] != a.Co || w->shape[1] != K) return fail(NNC_HIP_EINVAL, name, "weights are not [Co][9*Ci + Cx]");
    if (x->shape[0] != a.N) return fail(NNC_HIP_EINVAL, name, "projection input batch differs");
    if (out->shape[0] != a.N) return fail(NNC_HIP_EINVAL, name, "output batch differs");
    // every projection tap (oh * psh, ow * psw) inside the projection input
    if ((int64_t)(a.Ho - 1) * psh >= a.pH || (int64_t)(a.Wo - 1) * psw >= a.pW)
        return fail(NNC_HIP_EINVAL, name, "output larger than the strided projection input");
    if (a.bias && numel(b) < a.Co) return fail(NNC_HIP_EINVAL, name, "bias smaller than Co");
    if (a.Ci % 32 != 0 || a.pci % 32 != 0 || !aligned16(a.w))
        return fail(NNC_HIP_EUNSUPP, name, "needs Ci and Cx multiples of 32 and 16-byte aligned weights");
    const int64_t npix = (int64_t)a.N * a.Ho * a.Wo;
    const int64_t in_bytes = (int64_t)a.N * a.Ci * a.H * a.W * 4, x_bytes = numel(x) * 4;
    if (K >= (1 << 30) || npix >= (1 << 30) || in_bytes >= ((int64_t)1 << 31) || x_bytes >= ((int64_t)1 << 31) ||
        (int64_t)a.Co * K * 4 >= ((int64_t)1 << 31))
        return fail(NNC_HIP_EUNSUPP, name, "inputs or weights of 2 GiB or more");
    a.K = (int)K;
    a.ldw = (int)K;
    a.Npix = (int)npix;
    a.vec_out = aligned16(a.out);
    a.out32 = (int64_t)a.N * a.Co * a.Ho * a.Wo * 4 < ((int64_t)1 << 31);
    if (a.N == 0 || a.Co == 0 || a.Ho <= 0 || a.Wo <= 0) return;
    if (launch_conv_ws<true>(a, name)) return;
    // the tile choice of conv_run
    if (a.K >= 512 && a.Co >= 128 && a.Npix >= 1024) return launch_conv_proj<ConvT128>(a, name);
    if (a.K >= 512 && a.Co <= 64 && a.Npix >= 4096) return launch_conv_proj<ConvT64>(a, name);
    launch_conv_proj<ConvTSmall>(a, name);
}

// ---------------------------------------------------------------------------
// Scratch of the allocation-free entry point (nnc_hip_conv_packed_noalloc)
// ---------------------------------------------------------------------------
// Its stream-K partial tiles and tile counters live in `scratch`, a static
// device array of which every GPU the library runs on holds its own copy
// until the process ends: 64 MiB of partials (two 128x128 fp32 slots for each
// of up to 512 resident workgroups, the largest persistent grid of any conv
// tile on MI355X's 256 CUs), then 16384 tile counters. Host code never uses
// the array's name as an address (on the host it is only a stand-in):
// nnc_hip_init looks up each device's address once, with that device
// current, and calls take it from there.
static constexpr size_t kStaticPartialBytes = (size_t)64 << 20;
static constexpr size_t kStaticCounters = 16384;
static __device__ __align__(256) unsigned char scratch[kStaticPartialBytes + kStaticCounters * sizeof(int)];
static constexpr int kMaxDevices = 64;
static unsigned char* g_scratch_addr[kMaxDevices] = {};
// per device: recorded after each call's last launch; the next call's
// stream waits on it first, so calls on one device run one after another
// whatever thread or stream issued them
static hipEvent_t g_scratch_done[kMaxDevices] = {};
static std::mutex g_scratch_mutex;
// held while a call enqueues its wait, launches and record: the calls'
// order on the device is the order in which they take it
static std::mutex g_scratch_order;

int conv_static_scratch_setup(int device) {
    if (device < 0 || device >= kMaxDevices) {
        fail(NNC_HIP_EINVAL, "nnc_hip_init", "device %d beyond the %d the static scratch covers", device, kMaxDevices);
        return NNC_HIP_EINVAL;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_addr[device]) return NNC_HIP_OK;
    void* p = nullptr;
    if (!hip_ok(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "nnc_hip_init", "hipGetSymbolAddress(scratch)"))
        return NNC_HIP_EDEVICE;
    hipEvent_t ev = nullptr;
    if (!hip_ok(hipEventCreateWithFlags(&ev, hipEventDisableTiming), "nnc_hip_init", "hipEventCreate(scratch order)"))
        return NNC_HIP_EDEVICE;
    g_scratch_done[device] = ev;
    g_scratch_addr[device] = static_cast<unsigned char*>(p);
    return NNC_HIP_OK;
}

}  // namespace nnc

using namespace nnc;

extern "C" {

#define NNC_CONV_ENTRY(fname, act)                                                                \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw,      \
               int ph, int pw) {                                                                  \
        if (!conv_check(in, w, out, #fname)) return;                                              \
        conv_run(in, w, b, out, kh, kw, sh, sw, ph, pw, act, #fname);                              \
    }
NNC_CONV_ENTRY(nnc_conv, kActNone)
NNC_CONV_ENTRY(nnc_conv_relu, kActRelu)
NNC_CONV_ENTRY(nnc_conv_sigmoid, kActSigmoid)

#define NNC_CONV1X1_ENTRY(fname, act)                                                              \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int sh, int sw, int ph, int pw) {     \
        if (!conv_check(in, w, out, #fname)) return;                                               \
        conv_run(in, w, b, out, 1, 1, sh, sw, ph, pw, act, #fname);                                 \
    }
NNC_CONV1X1_ENTRY(nnc_conv1x1, kActNone)
NNC_CONV1X1_ENTRY(nnc_conv_relu1x1, kActRelu)

// ops.c:1089-1093: the 3x3 s1 entry requires a same-size output and
// otherwise leaves the output untouched.
#define NNC_CONV3X3_ENTRY(fname, act)                                                  \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {                        \
        if (!conv_check(in, w, out, #fname)) return;                                   \
        if (out->shape[2] != in->shape[2] || out->shape[3] != in->shape[3])            \
            return fail(NNC_HIP_EINVAL, #fname, "expected same-padding output shape"); \
        conv_run(in, w, b, out, 3, 3, 1, 1, 1, 1, act, #fname);                         \
    }
NNC_CONV3X3_ENTRY(nnc_conv3x3_s1, kActNone)
NNC_CONV3X3_ENTRY(nnc_conv_relu3x3_s1, kActRelu)

// ops.c:1310-1311, 1403: stride 2 with the pad fixed at 3.
#define NNC_CONV7X7_ENTRY(fname, act)                                   \
    void fname(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {         \
        if (!conv_check(in, w, out, #fname)) return;                    \
        conv_run(in, w, b, out, 7, 7, 2, 2, 3, 3, act, #fname);          \
    }
NNC_CONV7X7_ENTRY(nnc_conv7x7_s2, kActNone)
NNC_CONV7X7_ENTRY(nnc_conv_relu7x7_s2, kActRelu)

// Not in the reference ABI: Conv -> Add(residual) -> Relu as one kernel,
// emitted by the mi355x target at O3 for residual blocks. out = relu(conv(in,
// w) + bias + res), with the sum taken in the order of nnc_conv followed by
// nnc_add_relu(conv_out, res). `res` may be the same buffer as `out`.
void nnc_hip_conv_add_relu(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh,
                           int sw, int ph, int pw) {
    const char* name = "nnc_hip_conv_add_relu";
    if (!conv_check(in, w, out, name)) return;
    if (!res || !res->data || !res->shape) return fail(NNC_HIP_EINVAL, name, "NULL residual");
    conv_run(in, w, b, out, kh, kw, sh, sw, ph, pw, kActRelu, name, res);
}

// No reference counterpart: a residual block's 3x3 convolution with its 1x1
// projection shortcut folded into the same contraction. Each weight row is
// [Co][9*Ci + Cx]: the 3x3 taps tap-major over `in`, then the Cx projection
// weights over `x` read at (oh*psh, ow*psw). out = act(conv3x3(in) +
// conv1x1(x) + b), b the sum of both biases (may be NULL); no residual
// argument. Ci and Cx multiples of 32.
void nnc_hip_conv_proj(Tensor* in, Tensor* w, Tensor* b, Tensor* x, Tensor* out, int kh, int kw, int sh, int sw,
                       int ph, int pw, int psh, int psw, int act) {
    const char* name = "nnc_hip_conv_proj";
    if (act < kActNone || act > kActSigmoid) return fail(NNC_HIP_EINVAL, name, "act must be 0, 1 or 2");
    conv_proj_run(in, w, b, x, out, kh, kw, sh, sw, ph, pw, psh, psw, act, name);
}

// No reference counterpart: convolution with weights packed tap-major,
// emitted by the mi355x target at O3 (the compiler packs the constant):
// [Co][kh][kw][Ci] with Ci % 32 == 0 and a 1x1 or 3x3 kernel, or [Co][Kp]
// for the 3-channel 7x7 stem (k = tap * Ci + ci, zero up to Kp = K rounded
// up to 32). out = act(conv(in, w) + bias (+ res)), act 0 none, 1 relu, 2
// sigmoid; `b` and `res` may be NULL, `res` may be the same buffer as `out`
// but not as `in`. Weights 16-byte aligned; other shapes give NNC_HIP_EUNSUPP.
void nnc_hip_conv_packed(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh, int sw,
                         int ph, int pw, int act) {
    const char* name = "nnc_hip_conv_packed";
    if (!conv_check_packed(in, w, out, name)) return;
    if (res && (!res->data || !res->shape)) return fail(NNC_HIP_EINVAL, name, "NULL residual data");
    if (act < kActNone || act > kActSigmoid) return fail(NNC_HIP_EINVAL, name, "act must be 0, 1 or 2");
    conv_run(in, w, b, out, kh, kw, sh, sw, ph, pw, act, name, res, true);
}

// No reference counterpart: ResNet's stem convolution (packed [Co][Kp]
// rows, 3 channels, 7x7) with its relu and the 3x3 / stride 2 / pad 1 max
// pool that follows, in one kernel (conv_pool_k) plus a small fixup; the
// convolution output never reaches HBM. out = maxpool(relu(conv(in, w) +
// b)) of shape [N][Co][Ho/2][Wo/2]; Co <= 64, Ho and Wo even, Wo <= 128.
void nnc_hip_conv_maxpool(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph,
                          int pw) {
    conv_maxpool_run(in, w, b, out, kh, kw, sh, sw, ph, pw, "nnc_hip_conv_maxpool");
}

// No reference counterpart: nnc_hip_conv_packed for callers that cannot
// allocate (code under graph capture, serving loops). Same arguments, the
// same kernels and stream-K plan (same results to the bit), but partials and
// counters in the device's static scratch (64 MiB + 16384 counters) instead
// of the grow-only workspace; shapes needing more fail with NNC_HIP_EUNSUPP
// before anything is launched. The counters a launch uses are cleared by a
// fill kernel just before it; calls are not timed in the profiling table.
// Calls on one device share the one array, so they are ordered on the
// device: each call's stream first waits for the previous call's work (an
// event recorded after every call, whichever thread or stream made it).
// Inside a graph capture the captured calls are ordered by the graph
// instead; a replay is not ordered against calls made outside it. The
// calling thread must already have its library state (nnc_hip_init or any
// earlier call on that thread), which this entry point never creates
// (NNC_HIP_ESTATE otherwise).
void nnc_hip_conv_packed_noalloc(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh,
                                 int sw, int ph, int pw, int act) {
    const char* name = "nnc_hip_conv_packed_noalloc";
    if (!thread_ready()) return fail(NNC_HIP_ESTATE, name, "no library state on this thread: call nnc_hip_init first");
    const int d = dev().device;
    unsigned char* base = d >= 0 && d < kMaxDevices ? g_scratch_addr[d] : nullptr;
    if (!base) return fail(NNC_HIP_ESTATE, name, "static scratch not set up on device %d", d);
    if (!conv_check_packed(in, w, out, name)) return;
    if (res && (!res->data || !res->shape)) return fail(NNC_HIP_EINVAL, name, "NULL residual data");
    if (act < kActNone || act > kActSigmoid) return fail(NNC_HIP_EINVAL, name, "act must be 0, 1 or 2");
    FixedScratch fs;
    fs.ws = reinterpret_cast<float*>(base);
    fs.ws_bytes = kStaticPartialBytes;
    fs.cnt = reinterpret_cast<int*>(base + kStaticPartialBytes);
    fs.cnt_n = kStaticCounters;
    ThreadState& t = ts();
    std::lock_guard<std::mutex> order(g_scratch_order);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (!hip_ok(hipStreamIsCapturing(t.stream(), &cap), name, "hipStreamIsCapturing")) return;
    const bool ordered = cap == hipStreamCaptureStatusNone;
    if (ordered && !hip_ok(hipStreamWaitEvent(t.stream(), g_scratch_done[d], 0), name, "hipStreamWaitEvent")) return;
    t.fixed = &fs;
    conv_run(in, w, b, out, kh, kw, sh, sw, ph, pw, act, name, res, true);
    t.fixed = nullptr;
    if (ordered) hip_ok(hipEventRecord(g_scratch_done[d], t.stream()), name, "hipEventRecord");
}

}  // extern "C"
