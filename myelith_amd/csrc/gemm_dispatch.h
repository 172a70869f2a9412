// gemm_dispatch.h -- shape dispatch of the W8A16 / W16A16 products: the
// GEMV kernels for one activation row, the int8 matrix cores for more
// rows.  Shared by the op launchers (kernels.hip) and the batched forward
// (batch.hip), which plug in their own epilogues.
//
// An epilogue type provides
//   one(n, m, acc)              the output of weight row n, activation row m
//   apply<R, MT>(...)           the GEMV form (see gemv.h)
//   offset_m(m0)                the same epilogue shifted by m0 activation rows
#pragma once

#include "gemm_mfma.h"
#include "gemm_mfma2.h"
#include "gemv.h"
#include "gemv_stream.h"
#include "internal.h"

#include <algorithm>
#include <cstdlib>

namespace myl {

// ---------------------------------------------------------------------------
// GEMV dispatch
// ---------------------------------------------------------------------------

inline int xvec_ok(const int16_t* x, int ldx) { return (((uintptr_t)x & 15) == 0) && (ldx % 8 == 0); }

template <int R, int MT, int U, class Epi>
inline hipError_t launch_i8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
                            hipStream_t st) {
    // K-chunk staged in LDS per pass: both byte planes of MT rows fit 64 KiB.
    const int kc = min(kGemvLdsBytes / (2 * MT), ((K + 15) / 16) * 16);
    const int rows_per_block = R * kGemvWaves;
    const int blocks = (N + rows_per_block - 1) / rows_per_block;
    gemv_i8_kernel<R, MT, U, Epi><<<blocks, kGemvThreads, (size_t)2 * MT * kc, st>>>(x, M, ldx, W, N, K, kc,
                                                                                   xvec_ok(x, ldx), epi);
    return hipGetLastError();
}

template <int R, int MT, int U, class Epi>
inline hipError_t launch_i16(const int16_t* x, int M, int ldx, const int16_t* W, int N, int K, const Epi& epi,
                             hipStream_t st) {
    const int kc = min(kGemvLdsBytes / (4 * MT), ((K + 7) / 8) * 8);
    const int rows_per_block = R * kGemvWaves;
    const int blocks = (N + rows_per_block - 1) / rows_per_block;
    gemv_i16_kernel<R, MT, U, Epi><<<blocks, kGemvThreads, (size_t)4 * MT * kc, st>>>(x, M, ldx, W, N, K, kc,
                                                                                    xvec_ok(x, ldx), epi);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Matrix-core path (M > 1 activation rows)
// ---------------------------------------------------------------------------

// Tile shapes (activation rows x weight rows per block).
enum MmTile { MM_128x128 = 0, MM_128x64 = 1, MM_64x128 = 2, MM_64x64 = 3 };

// Overrides for tile sweeps: MYL_MM_TILE (an MmTile) and MYL_MM_KSPLIT.
inline int mm_env(const char* name) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : -1;
}

template <int WM, int WN, int WAVES_M, int WAVES_N, class Epi>
inline hipError_t mm_launch(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
                            int ksplit, const MmCtx* mm, hipStream_t st) {
    using S = MmShape<WM, WN, WAVES_M, WAVES_N>;
    const int tiles_m = (M + S::BM - 1) / S::BM, tiles_n = (N + S::BN - 1) / S::BN;
    const int ntiles = tiles_m * tiles_n;
    if (ksplit <= 1) {
        const int grid = 8 * ((ntiles + 7) / 8);
        mm_w8_kernel<WM, WN, WAVES_M, WAVES_N, Epi><<<grid, S::kThreads, S::kLds, st>>>(
            x, M, ldx, W, N, K, Divider::of((uint32_t)tiles_m), ntiles, epi);
        return hipGetLastError();
    }
    const int nkb = (K + kMmBK - 1) / kMmBK;
    const int kslice = ((nkb + ksplit - 1) / ksplit) * kMmBK;
    const int ns = (K + kslice - 1) / kslice;
    const int nitems = ntiles * ns;
    const int grid = 8 * ((nitems + 7) / 8);
    mm_w8_splitk_kernel<WM, WN, WAVES_M, WAVES_N><<<grid, S::kThreads, S::kLds, st>>>(
        x, M, ldx, W, N, K, Divider::of((uint32_t)tiles_m), Divider::of((uint32_t)ntiles), nitems, kslice, mm->acc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int colb = (N + 255) / 256;
    const int rows = std::max(1, std::min(M, (mm->cus * 8 + colb - 1) / colb));
    mm_splitk_finish_kernel<Epi><<<dim3(colb, rows), 256, 0, st>>>(mm->acc, M, N, epi);
    return hipGetLastError();
}

// Whether the W8A16 product of M rows over K runs on byte planes (and a
// producer may write them directly): every M >= 2 with K a multiple of 64
// and room in the context's plane buffer.
inline bool mm_planes_ok(int M, int K, const MmCtx* mm) {
    return M >= 2 && K % 64 == 0 && mm && mm->planes && mm->acc && (size_t)2 * M * K <= mm->planes_bytes &&
           mm_env("MYL_MM_TILE") < 0;
}

// Row tiles per group of the tile order of 256 x 256 tiles (TileOrder): the
// 32 blocks an XCD runs at one time cover 4 row tiles x 8 weight tiles.
// MYL_MM_GROUP overrides it for sweeps (0: the plain order).
inline int mm_group() {
    static const int g = [] {
        const int v = mm_env("MYL_MM_GROUP");
        return v >= 0 ? v : 4;
    }();
    return g;
}

// Whether 256 x 256 tiles with 128-byte K stages fill the chip well enough
// (mm_planes).
inline bool mm_wide_tiles(int M, int N, int K, int cus) {
    return K % 128 == 0 && mm2_tiles<2, 2, 4, 4, 2, 128>(M, N) >= cus + cus / 2;
}

// The product on planes Ap [2M x K] (mm_planes_ok): few rows stream the
// weights once in 64 or 128 plane-row tiles (K split until the chip is
// full, or half full past 32 rows).  More rows take 256 x 256 block tiles of
// 16 waves with 128-byte K stages (128 KB of LDS, one block per CU) when the
// grid holds at least 1.5 such tiles per CU: 12-25% faster than the
// alternative on MI355X for 2048-4096 rows of the 7B projections.  Smaller
// grids, where the last partial wave of big tiles costs more than the stage
// width gains (about 15% slower at 1.2 tiles per CU), take 256 x 128 tiles
// with 64-byte stages (72 KB of LDS, two blocks per CU) when those give
// every CU a tile.
template <class Epi>
inline hipError_t mm_planes(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi, const MmCtx* mm,
                            hipStream_t st) {
    const int cus = mm->cus;
    // few rows: partial sums cost little, so K is split until every CU has
    // work (up to 16 tokens: one 32-row plane tile with 128-byte K stages, 64
    // weight rows per tile, or 128 when that alone gives two tiles per CU;
    // K split for up to two items per CU: 20-25% faster on MI355X than
    // 64-byte stages for the 7B gate/up and LM head shapes at 8 rows)
    if (M <= 16 && K % 128 == 0) {
        if (N >= 256 * cus) return mm2_launch_splitk<1, 1, 1, 4, 3, 128>(Ap, M, W, N, K, epi, mm, 2 * cus, st);
        return mm2_launch_splitk<1, 1, 1, 2, 4, 128>(Ap, M, W, N, K, epi, mm, 2 * cus, st);
    }
    if (M <= 16) return mm2_launch_splitk<1, 1, 1, 4, 4>(Ap, M, W, N, K, epi, mm, 2 * cus, st);
    // up to 32 / 64 tokens: 128-byte stages on 64- / 128-row plane tiles
    // (5-20% faster than 64-byte stages on the 7B shapes)
    if (M <= 32 && K % 128 == 0) return mm2_launch_splitk<2, 1, 1, 4, 2, 128>(Ap, M, W, N, K, epi, mm, 2 * cus, st);
    if (M <= 32) return mm2_launch_splitk<2, 1, 1, 4, 4>(Ap, M, W, N, K, epi, mm, cus, st);
    if (M <= 64 && K % 128 == 0) return mm2_launch_splitk<1, 1, 4, 2, 3, 128>(Ap, M, W, N, K, epi, mm, cus, st);
    if (M > 64 && mm_wide_tiles(M, N, K, cus)) return mm2_launch<2, 2, 4, 4, 2, 128>(Ap, M, W, N, K, epi, st, mm_group());
    if (M > 64 && mm2_tiles<2, 2, 4, 2, 3>(M, N) >= cus) return mm2_launch<2, 2, 4, 2, 3>(Ap, M, W, N, K, epi, st);
    return mm2_launch_splitk<2, 1, 2, 4, 4>(Ap, M, W, N, K, epi, mm, cus / 2, st);
}

// mm_planes with a custom finish of split products (mm2_launch_splitk_fin):
// for up to 64 rows the same tiles and splits, and *split tells whether fin
// ran; more rows take mm_planes (no split, *split = false).
template <class Epi, class Fin>
inline hipError_t mm_planes_fin(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi, const MmCtx* mm,
                                hipStream_t st, const Fin& fin, bool* split) {
    const int cus = mm->cus;
    *split = false;
    if (M <= 16 && K % 128 == 0) {
        if (N >= 256 * cus)
            return mm2_launch_splitk_fin<1, 1, 1, 4, 3, 128>(Ap, M, W, N, K, epi, mm, 2 * cus, st, fin, split);
        return mm2_launch_splitk_fin<1, 1, 1, 2, 4, 128>(Ap, M, W, N, K, epi, mm, 2 * cus, st, fin, split);
    }
    if (M <= 16) return mm2_launch_splitk_fin<1, 1, 1, 4, 4>(Ap, M, W, N, K, epi, mm, 2 * cus, st, fin, split);
    if (M <= 32 && K % 128 == 0)
        return mm2_launch_splitk_fin<2, 1, 1, 4, 2, 128>(Ap, M, W, N, K, epi, mm, 2 * cus, st, fin, split);
    if (M <= 32) return mm2_launch_splitk_fin<2, 1, 1, 4, 4>(Ap, M, W, N, K, epi, mm, cus, st, fin, split);
    if (M <= 64 && K % 128 == 0)
        return mm2_launch_splitk_fin<1, 1, 4, 2, 3, 128>(Ap, M, W, N, K, epi, mm, cus, st, fin, split);
    if (M <= 64) return mm2_launch_splitk_fin<2, 1, 2, 4, 4>(Ap, M, W, N, K, epi, mm, cus / 2, st, fin, split);
    return mm_planes(Ap, M, W, N, K, epi, mm, st);
}

// The gate/up product with the staged epilogue (EpiGUSiluPlanes), N % 16 ==
// 0, without a K split: up to 64 rows, 32/64/128-row plane tiles x 64 weight
// rows with 128-byte stages (K % 128 == 0: enough tiles without a split for
// the 7B gate/up; the batched forward uses it up to 16 rows); more rows, the
// tiles of mm_planes.
template <class Epi>
inline hipError_t mm_planes_staged(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi,
                                   const MmCtx* mm, hipStream_t st) {
    if (M < 2 || N % 16 != 0 || K % 64 != 0) return hipErrorInvalidValue;
    if (M <= 64 && K % 128 != 0) return hipErrorInvalidValue;
    if (M <= 16) return mm2_staged_launch<1, 1, 1, 2, 4, 128>(Ap, M, W, N, K, epi, st);
    if (M <= 32) return mm2_staged_launch<2, 1, 1, 2, 4, 128>(Ap, M, W, N, K, epi, st);
    if (M <= 64) return mm2_staged_launch<2, 1, 2, 2, 4, 128>(Ap, M, W, N, K, epi, st);
    if (mm_wide_tiles(M, N, K, mm->cus)) return mm2_staged_launch<2, 2, 4, 4, 2, 128>(Ap, M, W, N, K, epi, st, mm_group());
    return mm2_staged_launch<2, 2, 4, 2, 3, 64>(Ap, M, W, N, K, epi, st);
}

// Tile and K split, from a sweep of the W8A16 shapes on MI355X: 64-row tiles
// (two waves per SIMD) beat 128-row tiles at every M; 64 x 128 wins once M
// is large.  K is split (slices of >= 1024 bytes) only when the tiles alone
// leave CUs idle.
template <class Epi>
inline hipError_t mm_i8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
                        const MmCtx* mm, hipStream_t st) {
    const int cus = mm ? mm->cus : 256;
    // The activations split once into byte planes, then the pipelined int8
    // product (gemm_mfma2.h).
    if (mm_planes_ok(M, K, mm)) {
        hipError_t e = split_planes(x, M, ldx, K, mm->planes, st);
        if (e != hipSuccess) return e;
        return mm_planes(mm->planes, M, W, N, K, epi, mm, st);
    }
    int tile = mm_env("MYL_MM_TILE");
    if (tile < 0 || tile > 3) tile = M <= 512 ? MM_64x64 : MM_64x128;
    const int bm = (tile == MM_128x128 || tile == MM_128x64) ? 128 : 64;
    const int bn = (tile == MM_128x128 || tile == MM_64x128) ? 128 : 64;
    const int ntiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const bool can_split = mm && mm->acc && (size_t)M * (size_t)N <= mm->acc_elems;
    int ks = mm_env("MYL_MM_KSPLIT");
    if (ks < 1) {
        ks = 1;
        if (ntiles < cus) ks = std::min((cus + ntiles - 1) / ntiles, std::max(1, K / 1024));
    }
    if (!can_split) ks = 1;
    switch (tile) {
        case MM_128x128: return mm_launch<2, 2, 2, 2>(x, M, ldx, W, N, K, epi, ks, mm, st);
        case MM_128x64: return mm_launch<2, 1, 2, 2>(x, M, ldx, W, N, K, epi, ks, mm, st);
        case MM_64x128: return mm_launch<1, 2, 2, 2>(x, M, ldx, W, N, K, epi, ks, mm, st);
        default: return mm_launch<1, 1, 2, 2>(x, M, ldx, W, N, K, epi, ks, mm, st);
    }
}

template <class Epi>
inline hipError_t gemv_i8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
                          hipStream_t st, const MmCtx* mm) {
    const bool fast = (K % 16 == 0) && (((uintptr_t)W & 15) == 0) && K < 131072;
    if (!fast) {
        dim3 grid((N + 255) / 256, M);
        gemv_generic_kernel<int8_t, Epi><<<grid, 256, 0, st>>>(x, M, ldx, W, N, K, epi);
        return hipGetLastError();
    }
    // More than one activation row: the int8 matrix cores (16-byte aligned
    // rows).  Up to 64 rows are one tile row, so the weights stream once; the
    // multi-row GEMV below reached only ~0.6 TB/s at 8 rows on MI355X.
    if (M > 1 && xvec_ok(x, ldx)) return mm_i8(x, M, ldx, W, N, K, epi, mm, st);
    // One row: the persistent streaming kernel of the decode step.
    if (M == 1 && xvec_ok(x, ldx)) {
        const int cus = mm ? mm->cus : 256;
        if (const int shape = stream_rows_shape(N, K, cus)) return stream_rows_i8(shape, x, W, N, K, epi, st, cus);
    }
    // Activation rows in groups of at most 8.
    for (int m0 = 0; m0 < M; m0 += 8) {
        const int mm_rows = min(8, M - m0);
        Epi e = epi.offset_m(m0);
        hipError_t rc;
        const int16_t* xm = x + (size_t)m0 * ldx;
        // Few rows: one row per wave so that the grid still fills the chip.
        const bool few = N < 8192;
        if (mm_rows == 1) rc = few ? launch_i8<1, 1, 4>(xm, mm_rows, ldx, W, N, K, e, st) : launch_i8<2, 1, 4>(xm, mm_rows, ldx, W, N, K, e, st);
        else if (mm_rows == 2) rc = launch_i8<2, 2, 4>(xm, mm_rows, ldx, W, N, K, e, st);
        else if (mm_rows <= 4) rc = launch_i8<2, 4, 2>(xm, mm_rows, ldx, W, N, K, e, st);
        else rc = launch_i8<1, 8, 2>(xm, mm_rows, ldx, W, N, K, e, st);
        if (rc != hipSuccess) return rc;
    }
    return hipSuccess;
}

template <class Epi>
inline hipError_t gemv_i16(const int16_t* x, int M, int ldx, const int16_t* W, int N, int K, const Epi& epi,
                           hipStream_t st) {
    const bool fast = (K % 8 == 0) && (((uintptr_t)W & 15) == 0) && K <= 8192;
    if (!fast) {
        dim3 grid((N + 255) / 256, M);
        gemv_generic_kernel<int16_t, Epi><<<grid, 256, 0, st>>>(x, M, ldx, W, N, K, epi);
        return hipGetLastError();
    }
    // More than one activation row: the int8 matrix cores, four byte-plane products.
    if (M > 1 && xvec_ok(x, ldx) && K < 65536) {
        using S = Mm16Shape<1, 1, 2, 2>;
        const int tiles_m = (M + S::BM - 1) / S::BM, ntiles = tiles_m * ((N + S::BN - 1) / S::BN);
        mm_w16_kernel<1, 1, 2, 2, Epi><<<8 * ((ntiles + 7) / 8), S::kThreads, S::kLds, st>>>(
            x, M, ldx, W, N, K, Divider::of((uint32_t)tiles_m), ntiles, epi);
        return hipGetLastError();
    }
    for (int m0 = 0; m0 < M; m0 += 4) {
        const int mm = min(4, M - m0);
        Epi e = epi.offset_m(m0);
        hipError_t rc;
        const int16_t* xm = x + (size_t)m0 * ldx;
        if (mm == 1) rc = launch_i16<2, 1, 4>(xm, mm, ldx, W, N, K, e, st);
        else rc = launch_i16<1, 4, 2>(xm, mm, ldx, W, N, K, e, st);
        if (rc != hipSuccess) return rc;
    }
    return hipSuccess;
}

}  // namespace myl
