// mm_plan.h -- launch planning of the byte-plane products (gemm_mfma2.h):
// block shapes, tile counts, the K split, grid and LDS sizes.  Plain C++
// with no HIP dependency: the launchers call these functions, and a host
// build of them runs under AddressSanitizer and UndefinedBehaviorSanitizer
// in the CPU tests (tests/test_launch_plan.py).
#pragma once

#include <algorithm>
#include <cstddef>
#include <cstdint>

namespace myl {

// Block shape of an mm2 launch: MB x NB 32 x 32 accumulators per wave,
// WM_ x WN_ waves, STAGES LDS stages of KS bytes of K.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS>
struct Mm2Dims {
    static_assert(KS == 64 || KS == 128, "stage width");
    static constexpr int kThreads = WM_ * WN_ * 64;
    static constexpr int BR = 32 * MB * WM_;   // A' rows per block (2 per token)
    static constexpr int BN = 32 * NB * WN_;   // weight rows per block
    static constexpr int kCpr = KS / 16;       // 16-byte chunks per stage row
    static constexpr int kRowsPerLoad = 64 / kCpr;
    static constexpr int kSwzRows = 256 / KS;  // rows sharing one swizzle slot
    static constexpr int kStageBytes = (BR + BN) * KS;
    static constexpr size_t kLds = (size_t)STAGES * kStageBytes;
    // 1 KiB wave loads per stage, dealt round-robin to the waves: every wave
    // issues kLoadsMin or kLoadsMax of them
    static constexpr int kGroups = (BR + BN) / kRowsPerLoad;
    static constexpr int kLoadsMin = kGroups / (kThreads / 64);
    static constexpr int kLoadsMax = (kGroups + kThreads / 64 - 1) / (kThreads / 64);
    static_assert((BR + BN) % kRowsPerLoad == 0, "whole 1 KiB loads");
};

// Grid of a launch over `items` work items: a multiple of 8 (the XCD count),
// so block b's XCD is b % 8 for every tile-order computation.
inline int mm2_grid_of(int items) { return 8 * ((items + 7) / 8); }

// The K split of a product over M activation rows (A' = 2M plane rows), N
// weight rows and K (a multiple of KS): with fewer tiles than `fill` and
// room for the M x N i64 partial sums, K is cut into ns slices of kslice
// bytes (a multiple of KS, at least 512 bytes of K per slice, about two
// items per CU), else one slice covers K.
struct Mm2SplitPlan {
    int tiles_r = 0, ntiles = 0;  // row tiles, all output tiles
    int ks = 1;                   // requested split
    int kslice = 0, ns = 1;       // bytes of K per slice, slices
    int nitems = 0, grid = 0;     // work items (tiles x slices), blocks
    bool split = false;
};

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS>
inline Mm2SplitPlan mm2_split_plan(int M, int N, int K, int cus, size_t acc_elems, int fill) {
    using S = Mm2Dims<MB, NB, WM_, WN_, STAGES, KS>;
    Mm2SplitPlan p;
    const int R2 = 2 * M;
    p.tiles_r = (R2 + S::BR - 1) / S::BR;
    p.ntiles = p.tiles_r * ((N + S::BN - 1) / S::BN);
    const int nkb = K / KS;
    if (p.ntiles < fill && (size_t)M * (size_t)N <= acc_elems)
        p.ks = std::max(1, std::min((2 * cus + p.ntiles - 1) / p.ntiles, nkb / (512 / KS)));
    p.split = p.ks > 1;
    p.kslice = p.split ? ((nkb + p.ks - 1) / p.ks) * KS : K;
    p.ns = p.split ? (K + p.kslice - 1) / p.kslice : 1;
    p.nitems = p.ntiles * p.ns;
    p.grid = mm2_grid_of(p.nitems);
    return p;
}

}  // namespace myl
