// libnnc_costmodel.so: the nnc_* ABI as an analytic MI355X timeline.
//
// Counterpart of the reference's runtime/x86/costmodel.c (4 simulated compute
// units sharing one memory port, fixed elements per cycle per op class,
// costmodel.c:15-24, 253-320). Here every call is turned into the kernels
// libnnc_hip.so launches for it - its conv/GEMM tile choice (conv.hip
// conv_run, gemm.hip gemm_run) and the stream-K plan it shares through
// plan.h - and each kernel is priced on MI355X:
//
//   MFMA kernels: a workgroup runs slices of BM x BN x 32 MACs; r of them
//   share a CU (r = ceil(G / 256)); a slice takes
//       max(r * 2*BM*BN*32 / (157.3 TFLOP/s / 256 * eff), lat)
//   (eff: the fraction of a CU's fp32 MFMA rate the kernel's main loop
//   reaches when the CU is full; lat: one slice's latency when alone), the
//   kernel max(slices of the busiest workgroup * slice, HBM time) + launch.
//   Stream-K fixups and the in-kernel finish move the partial tiles.
//   Bandwidth kernels: bytes that must cross HBM / (8 TB/s * eff) + launch.
//
// eff, lat and launch are fitted to rocprofv3 kernel durations of this
// library on MI355X (ResNet-18 at batch 1, 8 and 32); occupancies (resident
// workgroups per CU) are the compiler's resource report for each kernel.
// Kernels on the two streams (nnc_hip_stream_fork/select/join) overlap on
// the timeline as if each had the GPU to itself; the join takes the later.
//
// No tensor data is read or written by the nnc_* calls; the lifecycle calls
// keep host memory so generated programs run unchanged.

#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <string>
#include <vector>

#include "nnc_costmodel.h"
#include "nnc_hip.h"
#include "nnc_ops.h"
#include "ew_chains.h"
#include "plan.h"

namespace {

// ---------------------------------------------------------------------------
// the device
// ---------------------------------------------------------------------------
constexpr int kCUs = 256;
constexpr double kMfmaF32 = 157.3e12;  // dense fp32 MFMA, FLOP/s
constexpr double kHbm = 8.0e12;        // B/s
constexpr double kStreamEff = 0.72;    // large streaming kernels (copy, element-wise, pools)
constexpr double kLaunchUs = 4.0;      // per kernel in a graph replay: dispatch, ramp, drain
constexpr double kMinBodyUs = 0.8;     // a bandwidth kernel's body is at least one HBM round trip
constexpr int kBK = 32;

struct MfmaKind {
    const char* tag;
    int bm, bn, per_cu;  // tile, resident workgroups per CU
    double eff, lat_us;  // main loop: fraction of a CU's MFMA rate, slice latency alone
};
// Fitted to 97 launches of ResNet-18 at batch 1, 8 and 32 (rocprofv3 kernel
// trace, hipGraph replay; rms error 11% per launch, 2-6% per step).
// direct-to-LDS conv kernels (packed 3x3 / 1x1), the 3-channel stem; the
// register-staged conv kernels (reference-layout weights) and GEMM tiles
// are priced like the direct-to-LDS ones of their tile shape, the gather
// kernels 20% slower.
const MfmaKind kConv128 = {"conv_dma_128", 128, 128, 2, 0.75, 0.47};
const MfmaKind kConv64x128 = {"conv_dma_64x128", 64, 128, 3, 0.65, 4.0};
const MfmaKind kConv64 = {"conv_dma_64", 64, 64, 4, 0.60, 1.0};
const MfmaKind kStem64x128 = {"stem_64x128", 64, 128, 3, 0.50, 1.26};  // with the in-kernel finish
const MfmaKind kStem64 = {"stem_64", 64, 64, 4, 0.30, 1.43};
const MfmaKind kGather128 = {"conv_gather_128", 128, 128, 2, 0.60, 0.6};
const MfmaKind kGather64x128 = {"conv_gather_64x128", 64, 128, 3, 0.52, 4.0};
const MfmaKind kGather64 = {"conv_gather_64", 64, 64, 4, 0.48, 1.2};
const MfmaKind kGemm128 = {"gemm_128", 128, 128, 2, 0.75, 0.47};  // direct-to-LDS, two stages
const MfmaKind kGemmDma64 = {"gemm_dma_64", 64, 64, 2, 0.60, 1.0};  // direct-to-LDS, four stages
const MfmaKind kGemm64 = {"gemm_64", 64, 64, 4, 0.60, 1.0};         // register-staged
// the stem's row kernel (input window in LDS): fraction of a CU's MFMA rate
// over its 64 channels x Wo pixels x 148 k per row, fitted to ResNet-18's
// stem at batch 8 and 32
constexpr double kStemRowsEff = 0.55;
constexpr double kColdUsPerMB = 0.061;  // weights (B operand) arriving from HBM, per MB
constexpr double kFixupUsPerMB = 0.073; // fixup kernel: partial tiles read + finished tiles written, per MB
constexpr double kFixupUsPerPart = 0.069; // fixup kernel: each partial summed into a tile (sequential)
// conv_ws_k (short convolutions, plan_ws): one wave slice (32 x 32 x 32 MACs
// and its operands' arrival) and the in-kernel finish of a split tile
// (partial stores, counter, partial loads), fitted to ResNet-18 at batch 1
constexpr double kWsSliceUs = 0.88;
constexpr double kWsFinishUs = 1.9, kWsFinishUsPerPart = 0.2;

// ---------------------------------------------------------------------------
// the timeline and the per-kernel table
// ---------------------------------------------------------------------------
struct Stat {
    std::string name;
    int64_t launches = 0;
    double us = 0, flops = 0, bytes = 0;
};

struct Model {
    double ready[2] = {0, 0};  // per stream: time its last kernel ends
    int cur = 0;
    int64_t n = 0;
    std::vector<Stat> stats;
    bool quiet = getenv("NNC_COSTMODEL_QUIET") != nullptr;
    bool summary_registered = false;
};
Model g_model;

// host memory standing in for the arena and the spill pool
char* g_arena = nullptr;
size_t g_arena_bytes = 0;
char* g_spill = nullptr;
size_t g_spill_bytes = 0;
int g_error = 0;
char g_msg[256] = "";

void summary() {
    Model& m = g_model;
    if (!m.n || m.quiet) return;
    double total = 0;
    for (auto& s : m.stats) total += s.us;
    printf("[costmodel] summary kernels=%lld elapsed_us=%.1f kernel_us=%.1f\n", (long long)m.n,
           m.ready[0] > m.ready[1] ? m.ready[0] : m.ready[1], total);
    for (auto& s : m.stats)
        printf("[costmodel] summary kernel=%s launches=%lld us=%.1f share=%.1f%%\n", s.name.c_str(),
               (long long)s.launches, s.us, total > 0 ? 100.0 * s.us / total : 0.0);
}

void record(const char* op, const char* kernel, double us, double flops, double bytes) {
    Model& m = g_model;
    if (!m.summary_registered) {
        m.summary_registered = true;
        atexit(summary);
    }
    const double start = m.ready[m.cur];
    m.ready[m.cur] = start + us;
    ++m.n;
    Stat* s = nullptr;
    for (auto& st : m.stats)
        if (st.name == kernel) { s = &st; break; }
    if (!s) {
        m.stats.push_back(Stat{kernel});
        s = &m.stats.back();
    }
    s->launches += 1;
    s->us += us;
    s->flops += flops;
    s->bytes += bytes;
    if (!m.quiet)
        printf("[costmodel] #%lld op=%s kernel=%s stream=%d start=%.2f end=%.2f us=%.2f flops=%.0f bytes=%.0f\n",
               (long long)m.n, op, kernel, m.cur, start, start + us, us, flops, bytes);
}

int64_t numel(const Tensor* t) {
    if (!t || !t->shape) return 0;
    int64_t n = 1;
    for (int d = 0; d < t->ndim; ++d) n *= t->shape[d];
    return n;
}
double nbytes(const Tensor* t) { return t ? (double)t->nbytes : 0.0; }
int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// a bandwidth kernel moving `bytes` through HBM
void stream_kernel(const char* op, const char* kernel, double bytes, double eff = kStreamEff,
                   double min_body_us = kMinBodyUs) {
    record(op, kernel, kLaunchUs + fmax(bytes / (kHbm * eff) * 1e6, min_body_us), 0.0, bytes);
}

// ---------------------------------------------------------------------------
// MFMA kernels: stream-K grid of one tile kind
// ---------------------------------------------------------------------------
struct MfmaResult {
    nnc::StreamK sk;
    double us;
};

// `slots`: the persistent grid's cap (0: k.per_cu workgroups per CU)
MfmaResult mfma_kernel(const MfmaKind& k, int tiles, int64_t K, double hbm_bytes, double weight_bytes,
                       int slots = 0) {
    const int iters = K > 0 ? (int)ceil_div(K, kBK) : 1;
    const nnc::StreamK sk =
        nnc::plan_streamk(tiles, iters, slots > 0 ? slots : k.per_cu * kCUs, nnc::fixup_slices_for(k.bm, k.bn));
    const int G = sk.G < 1 ? 1 : sk.G;
    const int r = (int)ceil_div(G, kCUs);
    const double cu_rate = kMfmaF32 / kCUs;
    const double slice = fmax(r * 2.0 * k.bm * k.bn * kBK / (cu_rate * k.eff) * 1e6, k.lat_us);
    const int64_t dp_tiles = sk.tiles - sk.sk_tiles;
    const double slices = (double)ceil_div(sk.total(), G) + (double)ceil_div(dp_tiles, G) * iters;
    double partial = 0;
    if (sk.needs_fixup()) partial = 2.0 * G * k.bm * k.bn * 4;  // each workgroup: at most two partial tiles
    const double mem = (hbm_bytes + partial) / (kHbm * kStreamEff) * 1e6;
    return {sk, kLaunchUs + fmax(slices * slice, mem) + kColdUsPerMB * weight_bytes * 1e-6};
}

// finishing shared tiles: the fixup kernel reads every partial tile and
// writes the finished tiles
double fixup_us(const MfmaKind& k, const nnc::StreamK& sk) {
    const double bytes = (2.0 * sk.G + sk.sk_tiles) * k.bm * k.bn * 4;
    const double parts = (double)sk.G / (sk.sk_tiles > 0 ? sk.sk_tiles : 1) + 1.0;
    return kLaunchUs + kFixupUsPerMB * bytes * 1e-6 + kFixupUsPerPart * parts;
}

// conv.hip conv_ws_k: each workgroup's waves run NS slices side by side;
// a split tile adds the finish
bool ws_kernel(const char* op, int kh, int kw, bool proj, int64_t Co, int64_t npix, int64_t K, double flops,
               double bytes, double weight_bytes) {
    nnc::WsPlan p;
    if (!nnc::plan_ws(Co, npix, K, p)) return false;
    char name[64];
    snprintf(name, sizeof name, "conv_ws_32x32_k%dx%d%s", kh, kw, proj ? "p" : "");
    const int r = (int)ceil_div(p.tiles * p.S, kCUs);  // workgroups sharing a CU
    double us = kLaunchUs + r * p.NS * kWsSliceUs + kColdUsPerMB * weight_bytes * 1e-6;
    if (p.S > 1) us += kWsFinishUs + kWsFinishUsPerPart * p.S;
    us = fmax(us, kLaunchUs + bytes / (kHbm * kStreamEff) * 1e6);
    record(op, name, us, flops, bytes);
    return true;
}

// ---------------------------------------------------------------------------
// convolution: conv.hip conv_run's choices
// ---------------------------------------------------------------------------
constexpr double kRepackMinFlops = 1e9;
constexpr int kMaxInKernelParts = 4;

void conv(const char* op, Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, bool packed) {
    if (!in || !w || !out || !in->shape || !w->shape || !out->shape || in->ndim != 4 || out->ndim != 4) return;
    const int64_t N = in->shape[0], Ci = in->shape[1], Co = w->shape[0];
    const int64_t Ho = out->shape[2], Wo = out->shape[3];
    const int64_t K = Ci * kh * kw, npix = N * Ho * Wo;
    if (N == 0 || Co == 0 || Ho <= 0 || Wo <= 0) return;
    const double flops = 2.0 * Co * (double)npix * K;
    const double bytes = nbytes(in) + nbytes(w) + nbytes(b) + nbytes(out) + (res ? nbytes(res) : 0.0);
    const bool stem = packed && w->ndim == 2;
    const bool dma_ok = Ci % 32 == 0 && ((kh == 3 && kw == 3) || (kh == 1 && kw == 1));
    bool dma = dma_ok && (packed || (kh == 1 && kw == 1));
    if (dma_ok && !packed && kh == 3 && flops >= kRepackMinFlops) {
        stream_kernel(op, "conv_repack_taps", 8.0 * Co * K);
        dma = true;
    }
    const MfmaKind* k;
    char name[64];
    const int64_t H = in->shape[2], W = in->shape[3];
    if (stem && H == 2 * Ho && W == 2 * Wo && Co <= 64 && !res && (Wo == 112 || Wo == 32) && N * Ho >= 2 * kCUs) {
        // conv.hip conv_stem_rows (a 7x7 stem with H == 2 Ho is stride 2,
        // pad 3): two workgroups per CU, each taking every G-th output row
        const int64_t rows = N * Ho, G = rows < 2 * kCUs ? rows : 2 * kCUs;
        const double per_cu = (double)ceil_div(rows, G) * (G > kCUs ? 2 : 1);
        const double row_flops = 2.0 * 64 * Wo * 148;
        snprintf(name, sizeof name, "conv_stem_rows_w%d", (int)Wo);
        record(op, name, kLaunchUs + per_cu * row_flops / (kMfmaF32 / kCUs * kStemRowsEff) * 1e6, flops, bytes);
        return;
    }
    if (stem) {
        k = (Co <= 64 && npix >= 65536) ? &kStem64x128 : &kStem64;
        snprintf(name, sizeof name, "conv_igemm_%dx%d_k7x7c3_dma", k->bm, k->bn);
    } else {
        if (dma && ws_kernel(op, kh, kw, false, Co, npix, K, flops, bytes, nbytes(w))) return;
        const int tile = (K >= 512 && Co >= 128 && npix >= 1024) ? 2 : (K >= 512 && Co <= 64 && npix >= 4096) ? 1 : 0;
        if (dma) {
            k = tile == 2 ? &kConv128 : tile == 1 ? &kConv64x128 : &kConv64;
            snprintf(name, sizeof name, "conv_igemm_%dx%d_k%dx%d_dma", k->bm, k->bn, kh, kw);
        } else {
            k = tile == 2 ? &kGather128 : tile == 1 ? &kGather64x128 : &kGather64;
            const bool known = (kh == 1 && kw == 1) || (kh == 3 && kw == 3) || (kh == 7 && kw == 7);
            const char* vec = K % 4 == 0 ? "v4" : "s1";
            if (known) snprintf(name, sizeof name, "conv_igemm_%dx%d_k%dx%d_%s", k->bm, k->bn, kh, kw, vec);
            else snprintf(name, sizeof name, "conv_igemm_%dx%d_kany_%s", k->bm, k->bn, vec);
        }
    }
    const int tiles = (int)(ceil_div(Co, k->bm) * ceil_div(npix, k->bn));
    // the stem's K is padded to a multiple of 32 with zeros
    MfmaResult m = mfma_kernel(*k, tiles, K, bytes, nbytes(w));
    record(op, name, m.us, flops, bytes);
    if (!m.sk.needs_fixup()) return;
    // the 64x128 direct-to-LDS kernels finish a shared tile in the kernel
    // when at most kMaxInKernelParts workgroups share it
    const bool fin = (dma && !stem && k == &kConv64x128) || k == &kStem64x128;
    const int64_t per = m.sk.total() / m.sk.G;
    // (its cost is inside the kernel's fitted efficiency)
    if (fin && (m.sk.iters + per - 1) / per + 1 <= kMaxInKernelParts) return;
    record(op, "conv_streamk_fixup", fixup_us(*k, m.sk), 0.0, 0.0);
}

// ---------------------------------------------------------------------------
// GEMM: gemm.hip gemm_run's choices (operands 16-byte aligned)
// ---------------------------------------------------------------------------
void gemm(const char* op, int M, int N, int K, int batches, bool a_kc, bool b_kc, double bytes, double b_bytes) {
    if (M <= 0 || N <= 0 || batches <= 0) return;
    const double flops = 2.0 * M * (double)N * K * batches;
    if (K <= 0) return stream_kernel(op, op, 4.0 * M * N);
    if (batches == 1 && M == 1 && !b_kc && N % 4 == 0) {
        // gemm.hip gemv_fin_k: one launch, its K splits finished in the
        // kernel by the last of each column block's workgroups (a round trip
        // for the partials when split)
        const int col_blocks = (int)ceil_div(N, 64);
        int splits = (int)ceil_div(4 * kCUs, col_blocks);
        if (splits > 16) splits = 16;
        if (splits > K) splits = K;
        const double b = 4.0 * ((double)K * N + K + N);
        record(op, "gemv_v4", kLaunchUs + b / (kHbm * kStreamEff) * 1e6 + (splits > 1 ? 1.0 : 0.0), flops, b);
        return;
    }
    if (batches == 1 && M == 1 && !b_kc) {
        const int col_blocks = (int)ceil_div(N, 256);
        int splits = (int)ceil_div(4 * kCUs, col_blocks);
        if (splits > ceil_div(K, 16)) splits = (int)ceil_div(K, 16);
        if (splits < 1) splits = 1;
        record(op, "gemv_xc_s1",
               kLaunchUs + 4.0 * ((double)K * N + K + (double)N * splits) / (kHbm * kStreamEff) * 1e6, flops,
               4.0 * K * N);
        return stream_kernel(op, "gemv_reduce", 4.0 * N * (splits + 1));
    }
    if (batches == 1 && a_kc && b_kc && (M == 1 || N == 1 || (int64_t)M * N <= 64)) {
        const double b = 4.0 * ((double)M * K + (double)N * K + (double)M * N);
        record(op, K % 4 == 0 ? "dot_rows_v4" : "dot_rows_s1", kLaunchUs + b / (kHbm * kStreamEff) * 1e6, flops, b);
        return;
    }
    if (batches == 1 && a_kc && b_kc && M <= 32 && K <= 1024 && K % 4 == 0) {
        // gemm.hip gemm_skinny_nt_k: 16 columns per workgroup, all rows, K
        // over 8 waves; latency-bound: the first round trip of every wave's
        // loads (0.5 us past the launch ramp; traced 4.1 us at M = 8, 5.1 us
        // at M = 32, K = 512, N = 1000), then its chunks' 16x16x4 MFMAs
        // (32 cycles each at 2.1 GHz)
        const double b = 4.0 * ((double)M * K + (double)N * K + (double)M * N);
        const double chain_us = (double)ceil_div(ceil_div(K, 16), 8) * 4 * (M > 16 ? 2 : 1) * 32 / 2100.0;
        record(op, M > 16 ? "gemm_skinny_nt_32" : "gemm_skinny_nt_16",
               kLaunchUs + 0.5 + chain_us + b / (kHbm * kStreamEff) * 1e6, flops, b);
        return;
    }
    {
        // gemm.hip gemm_ws_k (plan_gemm_ws): k-contiguous operands need K % 4
        // == 0 (16-byte rows), x-contiguous ones take any layout
        nnc::WsPlan p;
        if ((!a_kc || K % 4 == 0) && (!b_kc || K % 4 == 0) && nnc::plan_gemm_ws(M, N, K, batches, p)) {
            char name[48];
            snprintf(name, sizeof name, "gemm_ws_32x32_%s%s", a_kc ? "k4" : "x1", b_kc ? "k4" : "x1");
            const int r = (int)ceil_div(p.tiles * p.S, kCUs);  // workgroups sharing a CU
            double us = kLaunchUs + r * p.NS * kWsSliceUs + kColdUsPerMB * b_bytes * 1e-6;
            if (p.S > 1) us += kWsFinishUs + kWsFinishUsPerPart * p.S;
            record(op, name, fmax(us, kLaunchUs + bytes / (kHbm * kStreamEff) * 1e6), flops, bytes);
            return;
        }
    }
    const bool a4 = a_kc ? K % 4 == 0 : M % 4 == 0;  // 16-byte loads along the contiguous axis
    const bool b4 = b_kc ? K % 4 == 0 : N % 4 == 0;
    const bool big = (int64_t)M * N * batches >= (int64_t)128 * 128 * 2 * kCUs / 4 && M >= 128 && N >= 128;
    static const char* kinds[4] = {"k4", "k1", "x4", "x1"};
    const int ak = a_kc ? (a4 ? 0 : 1) : (a4 ? 2 : 3), bk = b_kc ? (b4 ? 0 : 1) : (b4 ? 2 : 3);
    char name[64];
    if (a4 && b4) {
        // direct-to-LDS: 128x128 or 64x64 tiles (one workgroup per CU over
        // 16 or more K slices); shared tiles of at most four partials are
        // finished in-kernel
        const MfmaKind& k = big ? kGemm128 : kGemmDma64;
        snprintf(name, sizeof name, "gemm_dma_%dx%d_%s%s", k.bm, k.bn, kinds[ak], kinds[bk]);
        const int tiles = (int)(ceil_div(M, k.bm) * ceil_div(N, k.bn) * batches);
        const int iters = (int)ceil_div(K, kBK);
        MfmaResult m = mfma_kernel(k, tiles, K, bytes, b_bytes, !big && iters >= 16 ? kCUs : 0);
        record(op, name, m.us, flops, bytes);
        if (!m.sk.needs_fixup()) return;
        const int64_t per = m.sk.total() / m.sk.G;
        if ((m.sk.iters + per - 1) / per + 1 <= kMaxInKernelParts) return;
        return record(op, "gemm_streamk_fixup", fixup_us(k, m.sk), 0.0, 0.0);
    }
    const MfmaKind& k = kGemm64;
    snprintf(name, sizeof name, "gemm_mfma_%dx%d_%s%s", k.bm, k.bn, kinds[ak], kinds[bk]);
    const int tiles = (int)(ceil_div(M, k.bm) * ceil_div(N, k.bn) * batches);
    MfmaResult m = mfma_kernel(k, tiles, K, bytes, b_bytes);
    record(op, name, m.us, flops, bytes);
    if (m.sk.needs_fixup()) record(op, "gemm_streamk_fixup", fixup_us(k, m.sk), 0.0, 0.0);
}

void matmul(const char* op, Tensor* a, Tensor* b, Tensor* bias, Tensor* out) {
    if (!a || !b || !out || !a->shape || !b->shape || !out->shape) return;
    const double bytes = nbytes(a) + nbytes(b) + nbytes(bias) + nbytes(out);
    const int an = a->ndim, bn = b->ndim, on = out->ndim;
    if (an == 2 && bn == 2)
        return gemm(op, (int)a->shape[0], (int)b->shape[1], (int)a->shape[1], 1, true, false, bytes, nbytes(b));
    if (an == 1 && bn == 2) return gemm(op, 1, (int)b->shape[1], (int)a->shape[0], 1, true, false, bytes, nbytes(b));
    if (an == 2 && bn == 1) return gemm(op, (int)a->shape[0], 1, (int)a->shape[1], 1, true, true, bytes, nbytes(b));
    if (an >= 2 && bn >= 2) {
        int64_t batches = 1;
        for (int d = 0; d < on - 2; ++d) batches *= out->shape[d];
        return gemm(op, (int)out->shape[on - 2], (int)out->shape[on - 1], (int)a->shape[an - 1], (int)batches, true,
                    false, bytes, nbytes(b));
    }
}

// a copy kernel of libnnc_hip.so; nothing when source and destination coincide
void copy(const char* op, const Tensor* in, const Tensor* out) {
    if (!in || !out || in->data == out->data) return;
    stream_kernel(op, op, nbytes(in) + nbytes(out));
}

void unary(const char* op, Tensor* in, Tensor* out) {
    if (in && out && numel(out) > 0) stream_kernel(op, op, nbytes(in) + nbytes(out));
}

void binary(const char* op, Tensor* a, Tensor* b, Tensor* out) {
    if (a && b && out && numel(out) > 0) stream_kernel(op, op, nbytes(a) + nbytes(b) + nbytes(out));
}

}  // namespace

extern "C" {

// ---- queries ----------------------------------------------------------------
void nnc_costmodel_reset(void) {
    g_model.ready[0] = g_model.ready[1] = 0;
    g_model.cur = 0;
    g_model.n = 0;
    g_model.stats.clear();
}
double nnc_costmodel_elapsed_us(void) { return g_model.ready[0] > g_model.ready[1] ? g_model.ready[0] : g_model.ready[1]; }
int nnc_costmodel_kernel_count(void) { return (int)g_model.stats.size(); }
int nnc_costmodel_kernel(int i, char* name, int cap, int64_t* launches, double* us, double* flops, double* bytes) {
    if (i < 0 || i >= (int)g_model.stats.size()) return NNC_HIP_EINVAL;
    const Stat& s = g_model.stats[i];
    if (name && cap > 0) {
        strncpy(name, s.name.c_str(), (size_t)cap - 1);
        name[cap - 1] = '\0';
    }
    if (launches) *launches = s.launches;
    if (us) *us = s.us;
    if (flops) *flops = s.flops;
    if (bytes) *bytes = s.bytes;
    return 0;
}

// ---- lifecycle (host memory) --------------------------------------------------
int nnc_hip_init(int device) { return device == 0 ? 0 : NNC_HIP_EDEVICE; }
void nnc_hip_shutdown(void) {
    free(g_arena);
    free(g_spill);
    g_arena = g_spill = nullptr;
    g_arena_bytes = g_spill_bytes = 0;
}
static int reserve(char** pool, size_t* have, size_t bytes) {
    if (*pool && bytes <= *have) return 0;
    free(*pool);
    *pool = (char*)aligned_alloc(256, (bytes + 255) / 256 * 256 + 256);
    *have = *pool ? bytes : 0;
    return *pool ? 0 : NNC_HIP_ENOMEM;
}
int nnc_hip_arena_reserve(size_t bytes) { return reserve(&g_arena, &g_arena_bytes, bytes); }
void* nnc_hip_arena_base(void) { return g_arena; }
size_t nnc_hip_arena_size(void) { return g_arena_bytes; }
int nnc_hip_bind(Tensor* t, size_t offset) {
    if (!t || !g_arena || offset + (size_t)t->nbytes > g_arena_bytes) return NNC_HIP_EINVAL;
    t->data = g_arena + offset;
    return 0;
}
int nnc_hip_spill_reserve(size_t bytes) { return reserve(&g_spill, &g_spill_bytes, bytes); }
void* nnc_hip_spill_base(void) { return g_spill; }
int nnc_hip_bind_spill(Tensor* t, size_t offset) {
    if (!t || !g_spill || offset + (size_t)t->nbytes > g_spill_bytes) return NNC_HIP_EINVAL;
    t->data = g_spill + offset;
    return 0;
}
void* nnc_hip_malloc(size_t bytes) { return aligned_alloc(256, (bytes + 255) / 256 * 256 + 256); }
void nnc_hip_free(void* p) { free(p); }
void* nnc_hip_host_malloc(size_t bytes) { return aligned_alloc(256, (bytes + 255) / 256 * 256 + 256); }
void nnc_hip_host_free(void* p) { free(p); }
int nnc_hip_upload(Tensor* t, const void* src) {
    if (!t || !t->data || !src) return NNC_HIP_EINVAL;
    memcpy(t->data, src, (size_t)t->nbytes);
    return 0;
}
int nnc_hip_download(const Tensor* t, void* dst) {
    if (!t || !t->data || !dst) return NNC_HIP_EINVAL;
    memcpy(dst, t->data, (size_t)t->nbytes);
    return 0;
}
int nnc_hip_memcpy_h2d(void* d, const void* s, size_t n) { memcpy(d, s, n); return 0; }
int nnc_hip_memcpy_d2h(void* d, const void* s, size_t n) { memcpy(d, s, n); return 0; }
int nnc_hip_sync(void) { return 0; }
void* nnc_hip_stream(void) { return nullptr; }
int nnc_hip_last_error(void) { return g_error; }
const char* nnc_hip_last_error_message(void) { return g_msg; }
void nnc_hip_clear_error(void) {
    g_error = 0;
    g_msg[0] = '\0';
}
int nnc_hip_stream_fork(void) {
    if (g_model.ready[1] < g_model.ready[0]) g_model.ready[1] = g_model.ready[0];
    return 0;
}
int nnc_hip_stream_select(int slot) {
    if (slot != 0 && slot != 1) return NNC_HIP_EINVAL;
    g_model.cur = slot;
    return 0;
}
int nnc_hip_stream_join(void) {
    if (g_model.ready[0] < g_model.ready[1]) g_model.ready[0] = g_model.ready[1];
    return 0;
}
// the per-kernel table of libnnc_hip.so: the model's table
void nnc_hip_profile_enable(int on) { (void)on; }
void nnc_hip_profile_reset(void) { nnc_costmodel_reset(); }
int nnc_hip_profile_count(void) { return nnc_costmodel_kernel_count(); }
int nnc_hip_profile_entry(int i, char* name, int cap, int64_t* launches, double* total_ms) {
    double us = 0;
    const int rc = nnc_costmodel_kernel(i, name, cap, launches, &us, nullptr, nullptr);
    if (total_ms) *total_ms = us * 1e-3;
    return rc;
}
int nnc_hip_profile_work(int i, double* flops, double* bytes) {
    return nnc_costmodel_kernel(i, nullptr, 0, nullptr, nullptr, flops, bytes);
}
// no graphs: generated programs take their node-by-node path, priced as a
// graph replay (kLaunchUs per kernel)
int nnc_hip_graph_begin(void) { return NNC_HIP_EUNSUPP; }
int nnc_hip_graph_end(void) { return NNC_HIP_EUNSUPP; }
int nnc_hip_graph_launch(void) { return NNC_HIP_EUNSUPP; }
void nnc_hip_graph_destroy(void) {}
int nnc_hip_debug_dump(const Tensor* t, const char* name, int node_idx, void* file) {
    (void)t;
    (void)name;
    (void)node_idx;
    (void)file;
    return NNC_HIP_EUNSUPP;
}
void nnc_hip_transfer(Tensor* src, Tensor* dst) {
    if (!src || !dst) return;
    // one PCIe Gen5 x16 copy: about 50 GB/s each way
    record("nnc_hip_transfer", "nnc_hip_transfer", kLaunchUs + nbytes(src) / 50e9 * 1e6, 0.0, nbytes(src));
}

// ---- convolutions -------------------------------------------------------------
void nnc_conv(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    conv("nnc_conv", in, w, b, nullptr, out, kh, kw, false);
}
void nnc_conv1x1(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int sh, int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    conv("nnc_conv1x1", in, w, b, nullptr, out, 1, 1, false);
}
void nnc_conv3x3_s1(Tensor* in, Tensor* w, Tensor* b, Tensor* out) { conv("nnc_conv3x3_s1", in, w, b, nullptr, out, 3, 3, false); }
void nnc_conv7x7_s2(Tensor* in, Tensor* w, Tensor* b, Tensor* out) { conv("nnc_conv7x7_s2", in, w, b, nullptr, out, 7, 7, false); }
void nnc_conv_relu(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    conv("nnc_conv_relu", in, w, b, nullptr, out, kh, kw, false);
}
void nnc_conv_relu1x1(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int sh, int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    conv("nnc_conv_relu1x1", in, w, b, nullptr, out, 1, 1, false);
}
void nnc_conv_relu3x3_s1(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {
    conv("nnc_conv_relu3x3_s1", in, w, b, nullptr, out, 3, 3, false);
}
void nnc_conv_relu7x7_s2(Tensor* in, Tensor* w, Tensor* b, Tensor* out) {
    conv("nnc_conv_relu7x7_s2", in, w, b, nullptr, out, 7, 7, false);
}
void nnc_conv_sigmoid(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    conv("nnc_conv_sigmoid", in, w, b, nullptr, out, kh, kw, false);
}
void nnc_hip_conv_add_relu(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh,
                           int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    conv("nnc_hip_conv_add_relu", in, w, b, res, out, kh, kw, false);
}
// conv.hip conv_proj_run: one direct-to-LDS kernel over K = 9*Ci + Cx
void nnc_hip_conv_proj(Tensor* in, Tensor* w, Tensor* b, Tensor* x, Tensor* out, int kh, int kw, int sh, int sw,
                       int ph, int pw, int psh, int psw, int act) {
    (void)kh, (void)kw, (void)sh, (void)sw, (void)ph, (void)pw, (void)psh, (void)psw, (void)act;
    const char* op = "nnc_hip_conv_proj";
    if (!in || !w || !x || !out || !in->shape || !w->shape || !out->shape || w->ndim != 2 || out->ndim != 4) return;
    const int64_t N = out->shape[0], Co = out->shape[1], npix = N * out->shape[2] * out->shape[3];
    const int64_t K = w->shape[1];
    if (N == 0 || Co == 0 || npix == 0) return;
    const double flops = 2.0 * Co * (double)npix * K;
    const double bytes = nbytes(in) + nbytes(x) + nbytes(w) + nbytes(b) + nbytes(out);
    if (ws_kernel(op, 3, 3, true, Co, npix, K, flops, bytes, nbytes(w))) return;
    const MfmaKind* k = (K >= 512 && Co >= 128 && npix >= 1024) ? &kConv128
                        : (K >= 512 && Co <= 64 && npix >= 4096) ? &kConv64x128 : &kConv64;
    char name[64];
    snprintf(name, sizeof name, "conv_igemm_%dx%d_k3x3p_dma", k->bm, k->bn);
    const int tiles = (int)(ceil_div(Co, k->bm) * ceil_div(npix, k->bn));
    MfmaResult m = mfma_kernel(*k, tiles, K, bytes, nbytes(w));
    record(op, name, m.us, flops, bytes);
    if (!m.sk.needs_fixup()) return;
    const int64_t per = m.sk.total() / m.sk.G;
    if (k == &kConv64x128 && (m.sk.iters + per - 1) / per + 1 <= kMaxInKernelParts) return;
    record(op, "conv_streamk_fixup", fixup_us(*k, m.sk), 0.0, 0.0);
}
void nnc_hip_conv_packed(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh, int sw,
                         int ph, int pw, int act) {
    (void)sh, (void)sw, (void)ph, (void)pw, (void)act;
    conv("nnc_hip_conv_packed", in, w, b, res, out, kh, kw, true);
}
// the stem streamed into its max pool: bands of whole conv rows (64 x 128
// tiles of which the row's pixels are used, no stream-K split), two
// workgroups per CU, then the band-boundary fixup
const MfmaKind kStemPool = {"stem_pool_64x128", 64, 128, 2, 0.50, 1.26};
void nnc_hip_conv_maxpool(Tensor* in, Tensor* w, Tensor* b, Tensor* out, int kh, int kw, int sh, int sw, int ph,
                          int pw) {
    if (!in || !w || !out || !in->shape || !w->shape || !out->shape || in->ndim != 4 || out->ndim != 4) return;
    if (sh <= 0 || sw <= 0) return;
    const int64_t N = in->shape[0], Ci = in->shape[1], Co = w->shape[0];
    const int64_t Ho = (in->shape[2] + 2 * ph - kh) / sh + 1, Wo = (in->shape[3] + 2 * pw - kw) / sw + 1;
    const int64_t K = Ci * kh * kw, Hp = out->shape[2], Wp = out->shape[3];
    if (N == 0 || Co == 0 || Ho <= 0 || Wo <= 0) return;
    const double bytes = nbytes(in) + nbytes(w) + nbytes(b) + nbytes(out);
    if (sh == 2 && sw == 2 && ph == 3 && pw == 3 && in->shape[2] == 2 * Ho && in->shape[3] == 2 * Wo &&
        (Wo == 112 || Wo == 32) && N * Ho >= 2 * kCUs) {
        // conv.hip launch_conv_stem_pool: the stem's row kernel over
        // contiguous ranges of rows (two workgroups per CU); neighbouring
        // ranges finish the pool row they share in-kernel, over counters
        const int64_t rows = N * Ho, G = rows / 2 < 2 * kCUs ? rows / 2 : 2 * kCUs;
        const double per_cu = (double)ceil_div(rows, G) * (G > kCUs ? 2 : 1);
        const double row_flops = 2.0 * 64 * Wo * 148;
        char name[64];
        snprintf(name, sizeof name, "conv_stem_pool_w%d", (int)Wo);
        record("nnc_hip_conv_maxpool", name, kLaunchUs + per_cu * row_flops / (kMfmaF32 / kCUs * kStemRowsEff) * 1e6,
               2.0 * Co * (double)rows * Wo * K, bytes);
        return;
    }
    const int tiles = (int)(N * Ho);  // one conv row per tile: whole tiles, one band's rows per workgroup
    const int iters = (int)ceil_div(K, kBK);
    const double cu_rate = kMfmaF32 / kCUs;
    const int slots = kStemPool.per_cu * kCUs;
    int R = 1;
    for (int c : {14, 8, 7, 4, 2, 1})
        if (N * ceil_div(Hp, c) >= slots) {
            R = c;
            break;
        }
    const int64_t bands = N * ceil_div(Hp, R);
    const double rows_per_cu = (double)ceil_div(bands, kCUs) * 2.0 * R;
    const double slice = kStemPool.per_cu * 2.0 * kStemPool.bm * kStemPool.bn * kBK / (cu_rate * kStemPool.eff) * 1e6;
    const double us = kLaunchUs + fmax(rows_per_cu / kStemPool.per_cu * iters * slice,
                                       bytes / (kHbm * kStreamEff) * 1e6);
    record("nnc_hip_conv_maxpool", "conv_igemm_64x128_k7x7c3_pool", us, 2.0 * Co * (double)N * Ho * Wo * K, bytes);
    (void)tiles;
    if (bands > N) stream_kernel("nnc_hip_conv_maxpool", "conv_pool_fixup", 12.0 * (double)(bands - N) * Co * Wp);
}

// the allocation-free variant launches the same kernels (plus a counter fill
// where the in-kernel finish runs, priced as free here)
void nnc_hip_conv_packed_noalloc(Tensor* in, Tensor* w, Tensor* b, Tensor* res, Tensor* out, int kh, int kw, int sh,
                                 int sw, int ph, int pw, int act) {
    (void)sh, (void)sw, (void)ph, (void)pw, (void)act;
    conv("nnc_hip_conv_packed_noalloc", in, w, b, res, out, kh, kw, true);
}

// ---- GEMM ---------------------------------------------------------------------
void nnc_matmul(Tensor* a, Tensor* b, Tensor* out) { matmul("nnc_matmul", a, b, nullptr, out); }
void nnc_matmul_relu(Tensor* a, Tensor* b, Tensor* bias, Tensor* out) { matmul("nnc_matmul_relu", a, b, bias, out); }
void nnc_gemm(Tensor* a, Tensor* b, Tensor* c, Tensor* out, float alpha, float beta, int ta, int tb) {
    (void)alpha, (void)beta;
    if (!a || !b || !out || !a->shape || !b->shape) return;
    const double bytes = nbytes(a) + nbytes(b) + nbytes(c) + nbytes(out);
    if (a->ndim == 2 && b->ndim == 2) {
        const int M = (int)(ta ? a->shape[1] : a->shape[0]), K = (int)(ta ? a->shape[0] : a->shape[1]);
        const int N = (int)(tb ? b->shape[0] : b->shape[1]);
        return gemm("nnc_gemm", M, N, K, 1, !ta, tb != 0, bytes, nbytes(b));
    }
    if (a->ndim == 1 && b->ndim == 2)
        return gemm("nnc_gemm", 1, (int)b->shape[1], (int)a->shape[0], 1, true, false, bytes, nbytes(b));
    if (a->ndim == 2 && b->ndim == 1)
        return gemm("nnc_gemm", (int)a->shape[0], 1, (int)a->shape[1], 1, true, true, bytes, nbytes(b));
}
void nnc_gemm_nt(Tensor* a, Tensor* b, Tensor* c, Tensor* out, float alpha, float beta) {
    (void)alpha, (void)beta;
    if (!a || !b || !out || !a->shape || !b->shape) return;
    const double bytes = nbytes(a) + nbytes(b) + nbytes(c) + nbytes(out);
    int M = 1, K = (int)numel(a), N = b->ndim == 2 ? (int)b->shape[0] : (int)numel(b);
    if (a->ndim == 2 && b->ndim == 2) M = (int)a->shape[0], K = (int)a->shape[1];
    else if (a->ndim == 1 && b->ndim == 2) K = (int)a->shape[0];
    gemm("nnc_gemm_nt", M, N, K, 1, true, true, bytes, nbytes(b));
}

// ---- pools ----------------------------------------------------------------------
void nnc_maxpool2d(Tensor* in, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    (void)kh, (void)kw, (void)sh, (void)sw, (void)ph, (void)pw;
    // streaming (MI355X: 4.7 us at ResNet-18 batch 1, 8.4 at batch 8, 26.4 at
    // batch 32)
    if (in && out && numel(out) > 0)
        stream_kernel("nnc_maxpool2d", "nnc_maxpool2d", nbytes(in) + nbytes(out), kStreamEff, 1.0);
}
void nnc_avgpool2d(Tensor* in, Tensor* out, int kh, int kw, int sh, int sw, int ph, int pw) {
    (void)sh, (void)sw, (void)ph, (void)pw;
    if (!in || !out || !in->shape || numel(out) <= 0) return;
    const bool global = in->ndim == 4 && kh == in->shape[2] && kw == in->shape[3];
    stream_kernel("nnc_avgpool2d", global ? "nnc_avgpool2d_global" : "nnc_avgpool2d", nbytes(in) + nbytes(out), 0.5);
}

// the global average pool streamed into the classifier: one launch whose
// time is its bytes (input planes, w read by every image group) at a low
// streaming efficiency, or its sequential per-lane dot products, whichever
// is longer (about 2 us for 512 channels)
void nnc_hip_gap_gemm_nt(Tensor* in, Tensor* w, Tensor* c, Tensor* out, float alpha, float beta) {
    (void)alpha, (void)beta;
    if (!in || !w || !out || !in->shape || !w->shape || in->ndim != 4 || w->ndim != 2) return;
    const double groups = (double)ceil_div(in->shape[0], 4);
    const double bytes = nbytes(in) + nbytes(w) * groups + nbytes(c) + nbytes(out);
    const double dot_us = 4.0e-3 * (double)w->shape[1];
    record("nnc_hip_gap_gemm_nt", "nnc_hip_gap_gemm_nt", kLaunchUs + fmax(bytes / (kHbm * 0.25) * 1e6, dot_us),
           2.0 * (double)in->shape[0] * (double)w->shape[0] * (double)w->shape[1], bytes);
}

// ---- element-wise -----------------------------------------------------------------
void nnc_add(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_add", a, b, out); }
void nnc_mul(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_mul", a, b, out); }
void nnc_sub(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_sub", a, b, out); }
void nnc_div(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_div", a, b, out); }
void nnc_equal(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_equal", a, b, out); }
void nnc_and(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_and", a, b, out); }
void nnc_greater(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_greater", a, b, out); }
void nnc_or(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_or", a, b, out); }
void nnc_add_relu(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_add_relu", a, b, out); }
void nnc_add_sigmoid(Tensor* a, Tensor* b, Tensor* out) { binary("nnc_add_sigmoid", a, b, out); }
void nnc_not(Tensor* in, Tensor* out) { unary("nnc_not", in, out); }
void nnc_relu(Tensor* in, Tensor* out) { unary("nnc_relu", in, out); }
void nnc_sigmoid(Tensor* in, Tensor* out) { unary("nnc_sigmoid", in, out); }
void nnc_tanh(Tensor* in, Tensor* out) { unary("nnc_tanh", in, out); }
void nnc_clip(Tensor* in, Tensor* out, float lo, float hi) {
    (void)lo, (void)hi;
    unary("nnc_clip", in, out);
}
// norm.hip nnc_hip_add_layernorm: nnc_layernorm's row kernel reading a
// second addend
void nnc_hip_add_layernorm(Tensor* a, Tensor* b, Tensor* scale, Tensor* bias, Tensor* out, int axis, float eps) {
    (void)axis, (void)eps;
    if (!a || !b || !out) return;
    stream_kernel("nnc_hip_add_layernorm", "nnc_hip_add_layernorm",
                  nbytes(a) + nbytes(b) + nbytes(out) + nbytes(scale) + nbytes(bias));
}
// movement.hip nnc_hip_transpose_slice: nnc_transpose's gather reading a
// column block of the unsplit tensor
void nnc_hip_transpose_slice(Tensor* in, Tensor* out, int64_t* perm, int ndim, int col0, int width) {
    (void)in, (void)perm, (void)ndim, (void)col0, (void)width;
    if (out && numel(out) > 0)
        stream_kernel("nnc_hip_transpose_slice", "nnc_hip_transpose_slice", 2.0 * nbytes(out), 0.6);
}
// norm.hip nnc_hip_scaled_softmax: nnc_softmax's row kernel dividing on load
void nnc_hip_scaled_softmax(Tensor* in, Tensor* div, Tensor* out, int axis) {
    (void)axis;
    if (in && div && out && numel(out) > 0)
        stream_kernel("nnc_hip_scaled_softmax", "nnc_hip_scaled_softmax", nbytes(in) + nbytes(out), 0.40);
}
// attention.hip nnc_hip_attention: one workgroup per (batch, head, 16 query
// rows) for heads of 64 (attention16_k), 32 rows for heads of 32
// (attention_k), each on its own CU staging Q, K and V and running two
// MFMA products; the body fitted to the transformer encoder at batch 8,
// sequence 128
constexpr double kAttnBodyUs = 2.7;
void nnc_hip_attention(Tensor* qkv, Tensor* div, Tensor* out, int batch, int seq, int heads, int head_dim, int q_col,
                       int k_col, int v_col) {
    (void)q_col, (void)k_col, (void)v_col;
    if (!qkv || !div || !out || batch <= 0 || seq <= 0 || heads <= 0) return;
    const int64_t blocks = (int64_t)batch * heads * (head_dim == 64 ? (seq + 15) / 16 : (seq + 31) / 32);
    const double flops = 4.0 * batch * heads * (double)seq * seq * head_dim;
    record("nnc_hip_attention", head_dim == 64 ? "attention16_d64" : "attention32_d32",
           kLaunchUs + kAttnBodyUs * ceil_div(blocks, kCUs), flops,
           nbytes(qkv) + nbytes(out));
}
// eltwise.hip nnc_hip_fused_eltwise: one streaming pass, each input read and
// the output written once
void nnc_hip_fused_eltwise(Tensor** ins, int n_in, const int* prog, int n_steps, const float* consts, Tensor* out) {
    (void)prog, (void)n_steps, (void)consts;
    if (!ins || !out || n_in < 1) return;
    double bytes = nbytes(out);
    for (int i = 0; i < n_in; ++i) bytes += nbytes(ins[i]);
    stream_kernel("nnc_hip_fused_eltwise", "nnc_hip_fused_eltwise", bytes);
}
int nnc_hip_ew_chain_specialized(int n_in, const int* prog, int n_steps) {
    return nnc::ew_chain_index(n_in, prog, n_steps) >= 0 ? 1 : 0;
}
void nnc_sqrt(Tensor* in, Tensor* out) { unary("nnc_sqrt", in, out); }
void nnc_pow(Tensor* in, Tensor* out) { unary("nnc_pow", in, out); }
void nnc_exp(Tensor* in, Tensor* out) { unary("nnc_exp", in, out); }
void nnc_log(Tensor* in, Tensor* out) { unary("nnc_log", in, out); }
void nnc_abs(Tensor* in, Tensor* out) { unary("nnc_abs", in, out); }
void nnc_neg(Tensor* in, Tensor* out) { unary("nnc_neg", in, out); }
void nnc_cast(Tensor* in, Tensor* out, int to) {
    (void)to;
    unary("nnc_cast", in, out);
}

// ---- rows: softmax, layernorm, reductions (one wave per row) ----------------------
void nnc_softmax(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    if (in && out && numel(out) > 0) stream_kernel("nnc_softmax", "nnc_softmax", nbytes(in) + nbytes(out), 0.40);
}
void nnc_layernorm(Tensor* in, Tensor* s, Tensor* b, Tensor* out, int axis, float eps) {
    (void)axis, (void)eps;
    if (in && out && numel(out) > 0)
        stream_kernel("nnc_layernorm", "nnc_layernorm", nbytes(in) + nbytes(s) + nbytes(b) + nbytes(out), 0.55);
}
void nnc_reducemean(Tensor* in, Tensor* out, int axis, int keepdims) {
    (void)axis, (void)keepdims;
    if (in && out && numel(out) > 0) stream_kernel("nnc_reducemean", "nnc_reducemean", nbytes(in) + nbytes(out), 0.6);
}
void nnc_reducesum(Tensor* in, Tensor* out, int axis, int keepdims) {
    (void)axis, (void)keepdims;
    if (in && out && numel(out) > 0) stream_kernel("nnc_reducesum", "nnc_reducesum", nbytes(in) + nbytes(out), 0.6);
}
void nnc_batchnorm(Tensor* in, Tensor* s, Tensor* b, Tensor* mean, Tensor* var, Tensor* out, float eps, int momentum) {
    (void)s, (void)b, (void)mean, (void)var, (void)eps, (void)momentum;
    unary("nnc_batchnorm", in, out);
}

// ---- data movement -------------------------------------------------------------------
void nnc_reshape(Tensor* in, Tensor* out, int64_t* shape, int ndim) {
    (void)shape, (void)ndim;
    copy("nnc_reshape", in, out);
}
void nnc_flatten(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    copy("nnc_flatten", in, out);
}
void nnc_squeeze(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    copy("nnc_squeeze", in, out);
}
void nnc_unsqueeze(Tensor* in, Tensor* out, int axis) {
    (void)axis;
    copy("nnc_unsqueeze", in, out);
}
void nnc_identity(Tensor* in, Tensor* out) { copy("nnc_identity", in, out); }
void nnc_transpose(Tensor* in, Tensor* out, int64_t* perm, int ndim) {
    (void)perm, (void)ndim;
    if (in && out && numel(out) > 0) stream_kernel("nnc_transpose", "nnc_transpose", nbytes(in) + nbytes(out), 0.6);
}
void nnc_tile(Tensor* in, Tensor* out, int64_t* repeats, int ndim) {
    (void)repeats, (void)ndim;
    unary("nnc_tile", in, out);
}
void nnc_expand(Tensor* in, Tensor* out, int64_t* shape, int ndim) {
    (void)shape, (void)ndim;
    unary("nnc_expand", in, out);
}
// one slab copy per part
void nnc_concat(Tensor** ins, Tensor* out, int n, int axis) {
    (void)axis;
    for (int i = 0; ins && out && i < n; ++i)
        if (ins[i] && numel(ins[i]) > 0) stream_kernel("nnc_concat", "nnc_concat", 2.0 * nbytes(ins[i]), 0.66);
}
void nnc_split(Tensor* in, Tensor** outs, int n, int axis) {
    (void)axis;
    for (int i = 0; in && outs && i < n; ++i)
        if (outs[i] && numel(outs[i]) > 0) stream_kernel("nnc_split", "nnc_split", 2.0 * nbytes(outs[i]), 0.66);
}
void nnc_shape(Tensor* in, Tensor* out, int64_t* shape_data, int ndim) {
    (void)in, (void)shape_data, (void)ndim;
    if (out) record("nnc_shape", "nnc_shape", kLaunchUs, 0.0, nbytes(out));
}
void nnc_constantofshape(Tensor* out, float value, int ndim) {
    (void)value, (void)ndim;
    if (out && numel(out) > 0) stream_kernel("nnc_constantofshape", "nnc_constantofshape", nbytes(out));
}
void nnc_gather(Tensor* data, Tensor* idx, Tensor* out, int axis, int dtype) {
    (void)data, (void)axis, (void)dtype;
    if (out && numel(out) > 0) stream_kernel("nnc_gather", "nnc_gather", 2.0 * nbytes(out) + nbytes(idx), 0.5);
}

// ---- LSTM: one workgroup, sequential over time ---------------------------------------
void nnc_lstm(Tensor* X, Tensor* W, Tensor* R, Tensor* B, Tensor* Y, Tensor* Yh, Tensor* Yc, int direction,
              int hidden) {
    (void)B, (void)Y, (void)Yh, (void)Yc, (void)direction;
    if (!X || !X->shape || X->ndim < 1 || hidden <= 0) return;
    // each step: 4*hidden x (input + hidden) MACs on one CU's VALUs (64 lanes x 4 SIMDs x 2.4 GHz)
    const double steps = (double)X->shape[0];
    const double macs = steps * 4.0 * hidden * ((double)numel(W) / (4.0 * hidden) + (double)numel(R) / (4.0 * hidden));
    record("nnc_lstm", "nnc_lstm", kLaunchUs + macs / (256 * 2.4e9) * 1e6 + steps * 2.0, 2.0 * macs, 0.0);
}

}  // extern "C"
