// Host-side launch planning of the MFMA tile engine, shared by
// libnnc_hip.so and the cost-model runtime (compiled without HIP there).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define NNC_HD __host__ __device__
#else
#define NNC_HD
#endif

namespace nnc {

// ---------------------------------------------------------------------------
// stream-K bookkeeping. The stream-K region holds S = sk_tiles * iters slice
// iterations; workgroup g owns [lo(g), hi(g)) with lo(g) = g*S/G.
// ---------------------------------------------------------------------------
struct StreamK {
    int tiles, iters, G, sk_tiles;
    NNC_HD int64_t total() const { return (int64_t)sk_tiles * iters; }
    NNC_HD int64_t lo(int g) const { return total() * g / G; }
    NNC_HD int64_t hi(int g) const { return total() * (g + 1) / G; }
    // first workgroup whose range reaches into stream-K tile t
    NNC_HD int first_owner(int t) const {
        const int64_t start = (int64_t)t * iters;
        int g = (int)(start * G / total());
        while (g > 0 && hi(g - 1) > start) --g;
        while (hi(g) <= start) ++g;
        return g;
    }
    // true if some stream-K tile is shared (a range boundary inside a tile)
    bool needs_fixup() const {
        if (sk_tiles == 0 || iters == 1) return false;
        return !(total() % G == 0 && (total() / G) % iters == 0);
    }
};

// Host: choose the grid and the stream-K region for `tiles` tiles of
// `iters` slices on `slots` resident workgroups. `fixup_slices` is what
// finishing the shared tiles costs, in slice times of this tile shape (the
// fixup kernel's launch and partial traffic).
//  - few slices per tile (< 4): splitting costs more than the tail; plain
//    round-robin over min(tiles, slots) workgroups
//  - otherwise round-robin (every tile whole) unless stream-K's estimated
//    time, ceil(tiles * iters / G) + fixup_slices, is shorter than
//    round-robin's ceil(tiles / slots) * iters
//  - stream-K with tiles >= slots: all but the last full round plus the
//    partial round are split, so every workgroup ends at the same time
//  - stream-K with tiles < slots: everything is split, each workgroup
//    taking at least 4 slices (fewer workgroups for short problems)
inline StreamK plan_streamk(int tiles, int iters, int slots, int fixup_slices) {
    StreamK sk{};
    sk.tiles = tiles;
    sk.iters = iters;
    const int kMinSplitIters = 4, kMinRangeIters = 4;
    const int64_t total = (int64_t)tiles * iters;
    const int64_t dp_time = (int64_t)((tiles + slots - 1) / slots) * iters;
    if (iters < kMinSplitIters) {
        sk.G = tiles < slots ? tiles : slots;
        sk.sk_tiles = 0;
        return sk;
    }
    if (tiles >= slots) {
        const int rem = tiles % slots;
        sk.G = slots;
        const int64_t sk_time = (total + slots - 1) / slots + fixup_slices;
        sk.sk_tiles = (rem == 0 || sk_time >= dp_time) ? 0 : tiles - (tiles / slots - 1) * slots;
        return sk;
    }
    int64_t G = total / kMinRangeIters;
    if (G > slots) G = slots;
    if (G < tiles) G = tiles;
    const int64_t sk_time = (total + G - 1) / G + fixup_slices;
    if (sk_time >= dp_time) {
        sk.G = tiles;
        sk.sk_tiles = 0;
        return sk;
    }
    sk.G = (int)G;
    sk.sk_tiles = tiles;
    return sk;
}

// ---------------------------------------------------------------------------
// Short convolutions (conv.hip conv_ws_k): 32 x 32 output tiles, the four
// waves of a workgroup splitting each tile's K range, S workgroups sharing a
// tile (the last to arrive finishes it in the kernel), at most kWsMaxSlices
// slices of 32 k per wave held in registers (NS).
// Taken for convolutions with fewer 64 x 64 tiles than kWsMaxTiles64 and
// at most kWsMaxFlops of work (ResNet-18 at batch 1 and 2, and the stride-2
// convolutions at batch 4), where the 64 x 64 stream-K plan splits nearly
// every tile and needs a fixup launch. Bigger ones keep the LDS-shared
// tiles, whose waves share their operands: measured on ResNet-18, this
// kernel up to 0.5 GFLOP per convolution gives batch 1 0.262 -> 0.198 ms,
// batch 2 0.346 -> 0.286 ms, batch 4 0.436 -> 0.435 ms; up to 1 GFLOP batch
// 4 0.435 -> 0.466 ms and batch 8 0.570 -> 0.597 ms (its stride-2
// convolutions); and ResNet-18's layer 4 at batch 32 (7.4 GFLOP on 200
// tiles of 64 x 64) 25.8k -> 19.2k images/s.
// S: the smallest power of two that leaves a wave at most kWsMaxSlices
// slices; a split tile costs the finish's round trips (partial stores, the
// counter, partial loads: several slice times), so a tile that fits one
// workgroup stays whole, and a split one is split further while the grid
// stays within kWsGroups workgroups (one per CU) and each keeps at least 8
// slices.
// ---------------------------------------------------------------------------
constexpr int kWsMaxSlices = 6;
constexpr int kWsMaxSplit = 16;
constexpr int kWsMaxTiles64 = 256;
constexpr double kWsMaxFlops = 5e8;
constexpr int kWsGroups = 256;

struct WsPlan {
    int64_t tiles;  // 32 x 32 tiles
    int iters;      // slices of 32 k
    int S, NS;
};

// false: conv_ws_k does not take this convolution (K a multiple of 32 and
// the tap-major layout are the caller's to check)
inline bool plan_ws(int64_t Co, int64_t Npix, int64_t K, WsPlan& p) {
    if (K <= 0 || K % 32 != 0 || Co <= 0 || Npix <= 0) return false;
    if (((Co + 63) / 64) * ((Npix + 63) / 64) >= kWsMaxTiles64 || 2.0 * Co * (double)Npix * K > kWsMaxFlops)
        return false;
    p.tiles = ((Co + 31) / 32) * ((Npix + 31) / 32);
    p.iters = (int)(K / 32);
    int S = 1;
    while (S < kWsMaxSplit && (p.iters + S - 1) / S > 4 * kWsMaxSlices) S *= 2;
    if (S > 1)
        while (S < kWsMaxSplit && p.tiles * 2 * S <= kWsGroups && p.iters / (2 * S) >= 8) S *= 2;
    const int per = (p.iters + S - 1) / S;
    if (per > 4 * kWsMaxSlices) return false;
    p.S = S;
    p.NS = (per + 3) / 4;
    return true;
}

// Short GEMMs (gemm.hip gemm_ws_k, the GEMM form of conv_ws_k): products of
// at most kGwsMaxFlops (a transformer encoder's projections and FFN2 at
// batch 8, sequence 128), on 32 x 32 tiles of every batch with the same
// split rule, while a wave holds at most kGwsMaxSlices slices (longer K
// splits over more workgroups) and the grid stays below kGwsMaxGroups.
// Measured on MI355X against the 64 x 64 direct-to-LDS tiles (rocprofv3,
// one kernel per product): 1024x256x256 5.8 vs 9.7 us, 512^3 7.0 vs 14.3,
// 1024x768x256 11.0 vs 11.5, 1024x256x1024 (split in two) 15.1 vs 16.1;
// the tile kernel ahead at 1024 workgroups (1024x1024x256: 12.2-12.8 vs
// 11.3-11.5 us) and with six slices per wave (768^3: 28.1 vs 22.4 us).
constexpr double kGwsMaxFlops = 1e9;
constexpr int kGwsMaxSlices = 4, kGwsMaxGroups = 1024;

inline bool plan_gemm_ws(int64_t M, int64_t N, int64_t K, int64_t batches, WsPlan& p) {
    if (M <= 0 || N <= 0 || K <= 0 || batches <= 0) return false;
    if (2.0 * M * (double)N * K * batches > kGwsMaxFlops) return false;
    p.tiles = ((M + 31) / 32) * ((N + 31) / 32) * batches;
    p.iters = (int)((K + 31) / 32);
    int S = 1;
    while (S < kWsMaxSplit && (p.iters + S - 1) / S > 4 * kGwsMaxSlices) S *= 2;
    if (S > 1)
        while (S < kWsMaxSplit && p.tiles * 2 * S <= kWsGroups && p.iters / (2 * S) >= 8) S *= 2;
    const int per = (p.iters + S - 1) / S;
    if (per > 4 * kGwsMaxSlices || p.tiles * S >= kGwsMaxGroups) return false;
    p.S = S;
    p.NS = (per + 3) / 4;
    return true;
}

// Fixup cost in slice times of a BM x BN tile: about one slice for 128x128
// tiles, scaled by tile area for smaller tiles (shorter slices).
constexpr int fixup_slices_for(int bm, int bn) { return (128 * 128) / (bm * bn); }

}  // namespace nnc
