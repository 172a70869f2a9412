// mm_plan.h -- launch planning of the byte-plane products (gemm_mfma2.h) and
// of the fragment-major products of decode batches (gemm_frag.h): block
// shapes, tile counts, the K split, grid and LDS sizes.  Plain C++
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

// ---- the fragment-major products of decode batches (gemm_frag.h) ----------

constexpr int kFragWaves = 8;
constexpr int kFragMaxRows = 32;  // token rows: 64 plane rows, RT = 4

// Plane-row tiles for R token rows (0: too many rows).
inline int frag_rt(int R) { return R <= 8 ? 1 : (R <= 16 ? 2 : (R <= kFragMaxRows ? 4 : 0)); }

// The LDS a launch needs: the reduction of ngb row groups and, for the
// staged epilogue, R x 16 ngb int16.  At least 81 KiB, so that one block
// runs per CU (the grid has one block per CU).
inline size_t frag_lds(int rt, int ngb, int R, bool staged) {
    const size_t red = (size_t)ngb * (rt * 256 + 16) * 4;
    const size_t stage = staged ? (size_t)R * 16 * ngb * 2 : 0;
    return std::max<size_t>(red + stage, 81 * 1024);
}
constexpr size_t kFragLdsMax = 160 * 1024;

// One K slice, the whole sum to the staged epilogue (gate/up with its SiLU):
// K <= 8 x 8 KiB (KT <= 64), N % 16 == 0.
inline bool frag_full_ok(int R, int K, int N, int cus) {
    if (frag_rt(R) == 0 || R < 1 || K <= 0 || K % 64 != 0 || K / 64 > kFragWaves * 8 || N <= 0 || N % 16 != 0) return false;
    const int NG = N / 16, ngb = (NG + cus - 1) / cus;
    return 16 * ngb <= kFragWaves * 64 && frag_lds(frag_rt(R), ngb, R, true) <= kFragLdsMax;
}

// Split-K plan: KPW K tiles per wave (8 or 5), S = ceil(KT / (8 KPW)) K
// slices of 8 KPW tiles, P = cus / S row parts; the plan whose busiest wave
// streams the fewest tiles (ceil(NG / P) row groups x KPW).  For the 7B down
// product (296 K tiles, 224 row groups): 5 x 8 slices, 7 row groups per block
// (the busiest wave 35 tiles; 8 tiles a wave in 5 slices: 40).
struct FragSplit {
    int kpw = 0, S = 0, P = 0, ngb = 0;
};
inline FragSplit frag_split_plan(int K, int N, int cus) {
    FragSplit best;
    const int KT = K / 64, NG = (N + 15) / 16;
    for (int kpw : {8, 5}) {
        const int S = (KT + kFragWaves * kpw - 1) / (kFragWaves * kpw);
        if (S > cus) continue;
        const int P = std::max(1, cus / S), ngb = (NG + P - 1) / P;
        if (best.kpw == 0 || ngb * kpw < best.ngb * best.kpw) best = FragSplit{kpw, S, P, ngb};
    }
    return best;
}

// The output policies map the block's 16 ngb columns onto its 512 threads
// (FragCols), so a plan needs 16 ngb <= 512.
inline bool frag_split_ok(int R, int K, int N, int cus, size_t acc_elems) {
    if (frag_rt(R) == 0 || R < 1 || K <= 0 || K % 64 != 0 || N <= 0 || (size_t)R * (size_t)N > acc_elems) return false;
    const FragSplit sp = frag_split_plan(K, N, cus);
    return sp.kpw != 0 && 16 * sp.ngb <= kFragWaves * 64 && frag_lds(frag_rt(R), sp.ngb, R, false) <= kFragLdsMax;
}

}  // namespace myl
