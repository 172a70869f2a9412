// gemm_mfma2.h -- the large-M W8A16 product on the int8 matrix cores.
//
// y[m][n] = epilogue(n, m, sum_k W[n][k] * x[m][k])  (exact i64 sums)
//
// The activations are split once, before the product, into byte planes laid
// out as interleaved rows of an int8 matrix A' [2M x K]: row 2m = hi(x_m) =
// x_m >> 8, row 2m + 1 = lo'(x_m) = (x_m & 255) - 128.  The product is then a
// plain int8 GEMM over 2M rows, C' = A' . W^T, and
//   sum_k w*x = 256 * C'[2m][n] + C'[2m+1][n] + 128 * sum_k W[n][k]
// with the row sums of W taken by v_dot4 on the B fragments.  In the 32x32
// accumulator layout rows 2m and 2m+1 land in registers r and r+1 of the same
// lane, so the combination needs no data movement.
//
// Tiling (gfx950, 160 KB LDS): a block of WM x WN waves owns BR = 32*MB*WM
// rows of A' and BN = 32*NB*WN weight rows; K advances KS = 64 or 128 bytes
// per stage through STAGES LDS buffers filled by direct global-to-LDS loads
// (global_load_lds_dwordx4: each wave instruction writes 1 KiB = 1024/KS rows
// x KS bytes), issued STAGES-1 stages ahead and awaited with an explicit
// vmcnt.  128-byte stages read whole cache lines of every row per load
// instruction and halve the barriers per K; they pay off for grids of many
// large tiles.  The KS/16 chunks of LDS row r sit at slot
// chunk ^ ((r / (256/KS)) % (KS/16)), so the 16-byte fragment reads of 16
// consecutive rows cover all 64 banks once.  K must be a multiple of KS; rows
// past the matrix clamp to its last row (their outputs are discarded), so
// every load stays in bounds.
#pragma once

#include "gemm_mfma.h"
#include "internal.h"
#include "mm_plan.h"
#include "wave.h"

#include <algorithm>

namespace myl {

typedef __attribute__((address_space(3))) void lds_void;

// x int16 [M x K] -> Ap int8 [2M x K]: row 2m = hi(x_m), row 2m+1 = lo'(x_m).
template <int = 0>
__global__ __launch_bounds__(256) void split_planes_kernel(const int16_t* __restrict__ x, int M, int ldx, int K, int8_t* __restrict__ Ap) {
    const int m = blockIdx.y;
    const int c = blockIdx.x * blockDim.x + threadIdx.x;  // 8-element chunk
    if (m >= M || c * 8 >= K) return;
    const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)m * ldx + c * 8);
    uint2 h, l;
    split_planes8(v, h, l);
    *reinterpret_cast<uint2*>(Ap + (size_t)(2 * m) * K + c * 8) = h;
    *reinterpret_cast<uint2*>(Ap + (size_t)(2 * m + 1) * K + c * 8) = l;
}

__device__ inline constexpr int waitcnt_vm(int v) { return (v & 0xF) | (0x7 << 4) | (0xF << 8) | (((v >> 4) & 0x3) << 14); }

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64>
struct Mm2 : Mm2Dims<MB, NB, WM_, WN_, STAGES, KS> {
    using D = Mm2Dims<MB, NB, WM_, WN_, STAGES, KS>;
    __device__ static int slot(int row, int chunk) { return chunk ^ ((row / D::kSwzRows) & (D::kCpr - 1)); }
};

// Order of a product's output tiles over the grid.  mm_tile_index gives each
// XCD a contiguous range of tile numbers; here tile numbers run over groups
// of G row tiles (the row-tile count padded to a multiple of G, padding
// tiles exit at once), the row tile fastest inside a group.  G = tiles_r is
// the plain order (all row tiles of one weight tile, then the next weight
// tile): the blocks an XCD runs at one time share one weight tile and read
// as many distinct A' tiles.  A small G makes them cover G row tiles x
// (blocks / G) weight tiles, so both operands are shared in the XCD's L2.
struct TileOrder {
    Divider span;  // G * tiles_n
    Divider g;     // G
    uint32_t tiles_r;
    static TileOrder of(int tiles_r, int tiles_n, int G) {
        if (G < 1 || G > tiles_r) G = tiles_r;
        return TileOrder{Divider::of((uint32_t)(G * tiles_n)), Divider::of((uint32_t)G), (uint32_t)tiles_r};
    }
    // tile numbers the grid must cover
    int count(int tiles_n) const { return (int)(((tiles_r + g.d - 1) / g.d) * g.d) * tiles_n; }
    __device__ inline bool decode(uint32_t t, uint32_t& tn, uint32_t& tr) const {
        uint32_t grp, in, r;
        span.divmod(t, grp, in);
        g.divmod(in, tn, r);
        tr = grp * g.d + r;
        return tr < tiles_r;
    }
};

// LDS layout of a stage: BR A' rows then BN weight rows, KS bytes each, the
// chunks of each row at Mm2::slot.
// The pipelined main loop: acc[i][j] = A' tile i x W tile j over K in
// [kb, ke) (multiples of KS); rs[j] = the lane's weight-row sum (summed over
// the lane pair l, l + 32 only after the loop).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64>
__device__ inline void mm2_main(const int8_t* __restrict__ Ap, int R2, const int8_t* __restrict__ W, int N, int K,
                                int kb, int ke, int r0, int n0, int8_t* lds, v16i32_t (&acc)[MB][NB],
                                int32_t (&rs)[NB]) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM_, wn = wave / WM_;
    const int nk = (ke - kb) / KS;
    // Each wave-level load moves 1 KiB (64 lanes x 16 bytes) of 1024/KS rows:
    // lane l takes row l / (KS/16) of the group and the global chunk whose
    // swizzled slot is l % (KS/16) (the swizzle is its own inverse).
    auto issue = [&](int kt, int buf) {
        int8_t* st = lds + buf * S::kStageBytes;
#pragma unroll
        for (int i = 0; i < S::kLoadsMax; ++i) {
            const int grp = wave + i * (S::kThreads / 64);   // 1 KiB row-group index in the stage
            if (i >= S::kLoadsMin && grp >= S::kGroups) break;  // wave-uniform
            const int row = grp * S::kRowsPerLoad + lane / S::kCpr;  // stage row: A' rows first
            const int chunk = S::slot(row, lane & (S::kCpr - 1));
            const int8_t* src;
            if (row < S::BR) {
                const int gr = min(r0 + row, R2 - 1);
                src = Ap + (size_t)gr * K + kb + kt * KS + chunk * 16;
            } else {
                const int gn = min(n0 + row - S::BR, N - 1);
                src = W + (size_t)gn * K + kb + kt * KS + chunk * 16;
            }
            __builtin_amdgcn_global_load_lds((const void*)src, (lds_void*)(st + grp * 1024), 16, 0, 0);
        }
    };
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
#pragma unroll
    for (int j = 0; j < NB; ++j) rs[j] = 0;

#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s)
        if (s < nk) issue(s, s);
    for (int kt = 0; kt < nk; ++kt) {
        // stage kt complete: later stages may still be in flight (loads
        // retire in order; a wave with kLoadsMax loads per stage waits for
        // a few of the next stage's too)
        if (kt + STAGES - 2 < nk) __builtin_amdgcn_s_waitcnt(waitcnt_vm(S::kLoadsMin * (STAGES - 2)));
        else __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
        __syncthreads();
        if (kt + STAGES - 1 < nk) issue(kt + STAGES - 1, (kt + STAGES - 1) % STAGES);
        const int8_t* st = lds + (kt % STAGES) * S::kStageBytes;
#pragma unroll
        for (int s = 0; s < KS / 32; ++s) {
            const int chunk = 2 * s + (lane >> 5);
            v4i32_t a[MB], b[NB];
#pragma unroll
            for (int j = 0; j < NB; ++j) {
                const int row = S::BR + (wn * NB + j) * 32 + (lane & 31);
                b[j] = *reinterpret_cast<const v4i32_t*>(st + row * KS + (S::slot(row, chunk) << 4));
            }
#pragma unroll
            for (int i = 0; i < MB; ++i) {
                const int row = (wm * MB + i) * 32 + (lane & 31);
                a[i] = *reinterpret_cast<const v4i32_t*>(st + row * KS + (S::slot(row, chunk) << 4));
            }
#pragma unroll
            for (int j = 0; j < NB; ++j) {
#pragma unroll
                for (int i = 0; i < MB; ++i) acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], acc[i][j], 0, 0, 0);
                rs[j] = sdot4((uint32_t)b[j][0], 0x01010101u, rs[j]);
                rs[j] = sdot4((uint32_t)b[j][1], 0x01010101u, rs[j]);
                rs[j] = sdot4((uint32_t)b[j][2], 0x01010101u, rs[j]);
                rs[j] = sdot4((uint32_t)b[j][3], 0x01010101u, rs[j]);
            }
        }
    }
}

// K runs over [kb, ke) (multiples of KS).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Sink>
__device__ inline void mm2_tile(const int8_t* __restrict__ Ap, int R2, const int8_t* __restrict__ W, int N, int K,
                                int kb, int ke, int r0, int n0, int8_t* lds, const Sink& sink) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % WM_, wn = wave / WM_;
    v16i32_t acc[MB][NB];
    int32_t rs[NB];
    mm2_main<MB, NB, WM_, WN_, STAGES, KS>(Ap, R2, W, N, K, kb, ke, r0, n0, lds, acc, rs);
#pragma unroll
    for (int j = 0; j < NB; ++j) rs[j] += __shfl_xor(rs[j], 32);
    // accumulator rows 8*(r/4) + 4*(lane/32) + r%4: registers (r, r+1), r even,
    // hold the hi and lo' rows of one token.
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int n = n0 + (wn * NB + j) * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int arow = r0 + (wm * MB + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int m = arow >> 1;
                if (arow < R2 && n < N)
                    sink(n, m, (int64_t)acc[i][j][r] * 256 + (int64_t)acc[i][j][r + 1] + (int64_t)rs[j] * 128);
            }
        }
}

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Epi>
__global__ __launch_bounds__(WM_ * WN_ * 64) void mm2_kernel(const int8_t* __restrict__ Ap, int R2, const int8_t* __restrict__ W,
                                                             int N, int K, TileOrder ord, int ntiles, Epi epi) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(ntiles);
    if (t < 0) return;
    uint32_t tn, tr;
    if (!ord.decode((uint32_t)t, tn, tr)) return;
    mm2_tile<MB, NB, WM_, WN_, STAGES, KS>(Ap, R2, W, N, K, 0, K, (int)tr * S::BR, (int)tn * S::BN, lds, SinkEpi<Epi>{epi});
}

// As mm2_kernel, with a staged epilogue for products whose output columns
// pair up (2i, 2i+1 -> element i of an output row): every accumulator value
// is first reduced to an int16 by Epi::stage(n, sum) and parked in LDS as a
// [BR/2 x BN] tile (the K stages are free by then); the block then hands
// Epi::emit(m, i0, v) the 16 staged values of columns 2 i0 .. 2 i0 + 15 of
// row m, for 8-column chunks of N / 2 (N % 16 == 0), so the outputs leave in
// whole 8-byte pieces.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Epi>
__global__ __launch_bounds__(WM_ * WN_ * 64) void mm2_staged_kernel(const int8_t* __restrict__ Ap, int R2,
                                                                    const int8_t* __restrict__ W, int N, int K,
                                                                    TileOrder ord, int ntiles, Epi epi) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    static_assert((size_t)(S::BR / 2) * S::BN * 2 <= S::kLds, "staged tile fits the stage buffers");
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(ntiles);
    if (t < 0) return;
    uint32_t tn, tr;
    if (!ord.decode((uint32_t)t, tn, tr)) return;
    const int r0 = (int)tr * S::BR, n0 = (int)tn * S::BN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % WM_, wn = wave / WM_;
    v16i32_t acc[MB][NB];
    int32_t rs[NB];
    mm2_main<MB, NB, WM_, WN_, STAGES, KS>(Ap, R2, W, N, K, 0, K, r0, n0, lds, acc, rs);
#pragma unroll
    for (int j = 0; j < NB; ++j) rs[j] += __shfl_xor(rs[j], 32);
    __syncthreads();  // every wave is past its last stage read
    int16_t* tile = reinterpret_cast<int16_t*>(lds);  // [BR / 2][BN]
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int nl = (wn * NB + j) * 32 + (lane & 31);
            const int n = n0 + nl;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int arl = (wm * MB + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                int16_t v = 0;
                if (r0 + arl < R2 && n < N)
                    v = epi.stage(n, (int64_t)acc[i][j][r] * 256 + (int64_t)acc[i][j][r + 1] + (int64_t)rs[j] * 128);
                tile[(arl >> 1) * S::BN + nl] = v;
            }
        }
    __syncthreads();
    constexpr int kChunks = S::BN / 16;  // 8-column output chunks per tile row
    const int m0 = r0 >> 1, i00 = n0 >> 1;
    for (int c = threadIdx.x; c < (S::BR / 2) * kChunks; c += S::kThreads) {
        const int ml = c / kChunks, ic = c % kChunks;  // powers of two
        const int m = m0 + ml, i0 = i00 + ic * 8;
        if (2 * m >= R2 || 2 * i0 >= N) continue;
        const uint4* src = reinterpret_cast<const uint4*>(tile + ml * S::BN + ic * 16);
        epi.emit(m, i0, src[0], src[1]);
    }
}

// group: row tiles per group of the tile order (TileOrder; 0: the plain order).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Epi>
hipError_t mm2_staged_launch(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi, hipStream_t st,
                             int group = 0) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    const int R2 = 2 * M;
    const int tiles_r = (R2 + S::BR - 1) / S::BR, tiles_n = (N + S::BN - 1) / S::BN;
    const TileOrder ord = TileOrder::of(tiles_r, tiles_n, group);
    const int ntiles = ord.count(tiles_n);
    auto kern = mm2_staged_kernel<MB, NB, WM_, WN_, STAGES, KS, Epi>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
    if (e != hipSuccess) return e;
    kern<<<8 * ((ntiles + 7) / 8), S::kThreads, S::kLds, st>>>(Ap, R2, W, N, K, ord, ntiles, epi);
    return hipGetLastError();
}

// int16 weights as byte planes: Wp [2N x K] with row 2n = hi(w_n), row
// 2n+1 = lo'(w_n), and wsum[n] = sum_k w_n[k]; likewise xsum[m] for the
// activations.  One int8 product over 2M x 2N plane rows yields the four
// plane products of each (m, n): in the 32x32 accumulator layout rows 2m and
// 2m+1 sit in registers r, r+1 of one lane and columns 2n, 2n+1 in lanes
// l, l^1, so a DPP swap of lane pairs assembles
//   x.w = 65536*hh + 256*(h lo' + lo' h) + lo' lo' + 128*(xsum + wsum) - 16384*K.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Sink>
__device__ inline void mm2w16_tile(const int8_t* __restrict__ Ap, int R2, const int8_t* __restrict__ Wp, int N2,
                                   int K, const int32_t* __restrict__ xsum, const int32_t* __restrict__ wsum, int r0,
                                   int n0, int8_t* lds, const Sink& sink) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % WM_, wn = wave / WM_;
    v16i32_t acc[MB][NB];
    int32_t rs[NB];
    mm2_main<MB, NB, WM_, WN_, STAGES, KS>(Ap, R2, Wp, N2, K, 0, K, r0, n0, lds, acc, rs);
    const int64_t kterm = 16384 * (int64_t)K;
    const bool even = (lane & 1) == 0;
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int np = n0 + (wn * NB + j) * 32 + (lane & 31);
            const int n = np >> 1;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int32_t a0 = acc[i][j][r], a1 = acc[i][j][r + 1];
                const int32_t b0 = dpp_mov<dpp::kXor1>(a0), b1 = dpp_mov<dpp::kXor1>(a1);
                const int arow = r0 + (wm * MB + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int m = arow >> 1;
                if (even && arow < R2 && np < N2)
                    sink(n, m, 65536 * (int64_t)a0 + 256 * ((int64_t)a1 + (int64_t)b0) + (int64_t)b1 +
                                   128 * ((int64_t)xsum[m] + (int64_t)wsum[n]) - kterm);
            }
        }
}

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Epi>
__global__ __launch_bounds__(WM_ * WN_ * 64) void mm2w16_kernel(const int8_t* __restrict__ Ap, int R2,
                                                                const int8_t* __restrict__ Wp, int N2, int K,
                                                                const int32_t* __restrict__ xsum,
                                                                const int32_t* __restrict__ wsum, TileOrder ord,
                                                                int ntiles, Epi epi) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(ntiles);
    if (t < 0) return;
    uint32_t tn, tr;
    if (!ord.decode((uint32_t)t, tn, tr)) return;
    mm2w16_tile<MB, NB, WM_, WN_, STAGES, KS>(Ap, R2, Wp, N2, K, xsum, wsum, (int)tr * S::BR, (int)tn * S::BN, lds,
                                          SinkEpi<Epi>{epi});
}

// x int16 [M x K] -> planes as split_planes_kernel, plus xsum[m] = sum_k x[m][k].
// One block per row.
template <int = 0>
__global__ __launch_bounds__(256) void split_planes_sum_kernel(const int16_t* __restrict__ x, int ldx, int K,
                                                               int8_t* __restrict__ Ap, int32_t* __restrict__ xsum) {
    __shared__ int32_t red[4];
    const int m = blockIdx.x;
    int32_t s = 0;
    for (int c = threadIdx.x; c * 8 < K; c += 256) {
        const uint4 v = *reinterpret_cast<const uint4*>(x + (size_t)m * ldx + c * 8);
        uint2 h, l;
        split_planes8(v, h, l);
        *reinterpret_cast<uint2*>(Ap + (size_t)(2 * m) * K + c * 8) = h;
        *reinterpret_cast<uint2*>(Ap + (size_t)(2 * m + 1) * K + c * 8) = l;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) s += (int32_t)(int16_t)(w[q] & 0xFFFFu) + (int32_t)(int16_t)(w[q] >> 16);
    }
    s = wave_sum_i32(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) xsum[m] = red[0] + red[1] + red[2] + red[3];
}

// Plane rows and sums of int16 rows (the weights of mm2w16, or activations).
inline hipError_t split_planes_sum(const int16_t* x, int M, int ldx, int K, int8_t* Ap, int32_t* xsum, hipStream_t st) {
    split_planes_sum_kernel<><<<M, 256, 0, st>>>(x, ldx, K, Ap, xsum);
    return hipGetLastError();
}

// The int16-weight product for two rows or more: A' and xsum from
// split_planes_sum, Wp and wsum prepared once the same way.  Up to 64 rows:
// 32- or 64-row plane tiles x 128 W' rows (the weight planes stream once);
// more: 256 A' rows x 256 W' rows with 128-byte stages when the grid holds
// at least four tiles per CU (and K % 128 == 0), else 256 x 128 tiles.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class Epi>
hipError_t mm2w16_launch_cfg(const int8_t* Ap, const int32_t* xsum, int M, const int8_t* Wp, const int32_t* wsum,
                             int N, int K, const Epi& epi, hipStream_t st, int group = 0) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    const int R2 = 2 * M, N2 = 2 * N;
    const int tiles_r = (R2 + S::BR - 1) / S::BR, tiles_n = (N2 + S::BN - 1) / S::BN;
    const TileOrder ord = TileOrder::of(tiles_r, tiles_n, group);
    const int ntiles = ord.count(tiles_n);
    auto kern = mm2w16_kernel<MB, NB, WM_, WN_, STAGES, KS, Epi>;
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
    if (e != hipSuccess) return e;
    kern<<<8 * ((ntiles + 7) / 8), S::kThreads, S::kLds, st>>>(Ap, R2, Wp, N2, K, xsum, wsum, ord, ntiles, epi);
    return hipGetLastError();
}

template <class Epi>
hipError_t mm2w16_launch(const int8_t* Ap, const int32_t* xsum, int M, const int8_t* Wp, const int32_t* wsum, int N,
                         int K, const Epi& epi, int cus, hipStream_t st) {
    // few rows: one plane-row tile streams the weight planes once
    if (M <= 16 && K % 128 == 0) return mm2w16_launch_cfg<1, 1, 1, 4, 3, 128>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    if (M <= 16) return mm2w16_launch_cfg<1, 1, 1, 4, 4, 64>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    if (M <= 32 && K % 128 == 0) return mm2w16_launch_cfg<2, 1, 1, 4, 2, 128>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    if (M <= 32) return mm2w16_launch_cfg<2, 1, 1, 4, 4, 64>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    if (M <= 64 && K % 128 == 0) return mm2w16_launch_cfg<2, 1, 2, 2, 3, 128>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    if (M <= 64) return mm2w16_launch_cfg<2, 1, 2, 4, 4, 64>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    using W = Mm2<2, 2, 4, 4, 2, 128>;
    const int wide_tiles = ((2 * M + W::BR - 1) / W::BR) * ((2 * N + W::BN - 1) / W::BN);
    if (K % 128 == 0 && wide_tiles >= 4 * cus)
        return mm2w16_launch_cfg<2, 2, 4, 4, 2, 128>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
    return mm2w16_launch_cfg<2, 2, 4, 2, 3, 64>(Ap, xsum, M, Wp, wsum, N, K, epi, st);
}

// Split-K form: item t -> (slice t / ntiles, tile t % ntiles); the exact
// partial sums of each slice are added into acc [M x N] (i64, zero-kept; the
// finish kernel applies the epilogue and clears it).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64>
__global__ __launch_bounds__(WM_ * WN_ * 64) void mm2_splitk_kernel(const int8_t* __restrict__ Ap, int R2,
                                                                    const int8_t* __restrict__ W, int N, int K,
                                                                    Divider tiles_r, Divider ntiles, int nitems,
                                                                    int kslice, unsigned long long* __restrict__ acc) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(nitems);
    if (t < 0) return;
    uint32_t ks, tile, tn, tr;
    ntiles.divmod((uint32_t)t, ks, tile);
    tiles_r.divmod(tile, tn, tr);
    const int kb = (int)ks * kslice, ke = min(K, kb + kslice);
    if (kb >= ke) return;
    mm2_tile<MB, NB, WM_, WN_, STAGES, KS>(Ap, R2, W, N, K, kb, ke, (int)tr * S::BR, (int)tn * S::BN, lds,
                                           SinkAtomic{acc, N});
}

// Work item of this block when the item count n is in device memory (written
// by an earlier kernel; grid = 8 ceil(max / 8) for an upper bound max): XCD x
// takes items [x per, (x + 1) per) with per = ceil(n / 8), as mm_tile_index
// does for a count known at launch; the other blocks get -1.
__device__ inline int mm_dyn_tile_index(const int* __restrict__ nwork) {
    const int n = __builtin_amdgcn_readfirstlane(*nwork);
    const int b = blockIdx.x, per = (n + 7) >> 3;
    const int t = (b & 7) * per + (b >> 3);
    return (b >> 3) < per && t < n ? t : -1;
}

// Grouped products (MoE experts): work item t = (expert e, token tile m0,
// weight tile n0) of the work table; expert e's rows are the byte-plane rows
// [2 offsets[e], 2 offsets[e+1]) of Ap and its weights W + e * w_stride
// [N x K].  The epilogue receives (e, n, row, sum) with row the activation
// row in Ap's token order (SinkGrouped).  The item count is read from
// *nwork on the device (the work table is built there); the grid covers
// maxwork items.  K % KS == 0.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class EpiG>
__global__ __launch_bounds__(WM_ * WN_ * 64) void mm2_grouped_kernel(const int8_t* __restrict__ Ap,
                                                                     const int8_t* __restrict__ W, size_t w_stride,
                                                                     int N, int K, const int* __restrict__ offsets,
                                                                     const MmWork* __restrict__ work,
                                                                     const int* __restrict__ nwork, EpiG epi) {
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_dyn_tile_index(nwork);
    if (t < 0) return;
    const MmWork wk = work[t];
    const int row0 = offsets[wk.e];
    const int Me = offsets[wk.e + 1] - row0;
    mm2_tile<MB, NB, WM_, WN_, STAGES, KS>(Ap + (size_t)2 * row0 * K, 2 * Me, W + (size_t)wk.e * w_stride, N, K, 0, K,
                                           2 * wk.m0, wk.n0, lds, SinkGrouped<EpiG>{epi, wk.e, row0});
}

// mm2_grouped_kernel with the staged epilogue of mm2_staged_kernel: every
// sum is reduced by EpiG::stage(e, n, sum) to an int16 parked in LDS, then
// EpiG::emit(e, row, i0, v) takes the 16 values of columns 2 i0 .. 2 i0 + 15
// of activation row `row` (Ap's token order) for 8-column chunks of N / 2
// (N % 16 == 0).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class EpiG>
__global__ __launch_bounds__(WM_ * WN_ * 64) void mm2_grouped_staged_kernel(
    const int8_t* __restrict__ Ap, const int8_t* __restrict__ W, size_t w_stride, int N, int K,
    const int* __restrict__ offsets, const MmWork* __restrict__ work, const int* __restrict__ nwork, EpiG epi) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    static_assert((size_t)(S::BR / 2) * S::BN * 2 <= S::kLds, "staged tile fits the stage buffers");
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_dyn_tile_index(nwork);
    if (t < 0) return;
    const MmWork wk = work[t];
    const int row0 = offsets[wk.e];
    const int R2 = 2 * (offsets[wk.e + 1] - row0);
    const int r0 = 2 * wk.m0, n0 = wk.n0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave % WM_, wn = wave / WM_;
    v16i32_t acc[MB][NB];
    int32_t rs[NB];
    mm2_main<MB, NB, WM_, WN_, STAGES, KS>(Ap + (size_t)row0 * 2 * K, R2, W + (size_t)wk.e * w_stride, N, K, 0, K, r0,
                                           n0, lds, acc, rs);
#pragma unroll
    for (int j = 0; j < NB; ++j) rs[j] += __shfl_xor(rs[j], 32);
    __syncthreads();  // every wave is past its last stage read
    int16_t* tile = reinterpret_cast<int16_t*>(lds);  // [BR / 2][BN]
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int j = 0; j < NB; ++j) {
            const int nl = (wn * NB + j) * 32 + (lane & 31);
            const int n = n0 + nl;
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const int arl = (wm * MB + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                int16_t v = 0;
                if (r0 + arl < R2 && n < N)
                    v = epi.stage(wk.e, n,
                                  (int64_t)acc[i][j][r] * 256 + (int64_t)acc[i][j][r + 1] + (int64_t)rs[j] * 128);
                tile[(arl >> 1) * S::BN + nl] = v;
            }
        }
    __syncthreads();
    constexpr int kChunks = S::BN / 16;  // 8-column output chunks per tile row
    const int m0 = r0 >> 1, i00 = n0 >> 1;
    for (int c = threadIdx.x; c < (S::BR / 2) * kChunks; c += S::kThreads) {
        const int ml = c / kChunks, ic = c % kChunks;  // powers of two
        const int m = m0 + ml, i0 = i00 + ic * 8;
        if (2 * m >= R2 || 2 * i0 >= N) continue;
        const uint4* src = reinterpret_cast<const uint4*>(tile + ml * S::BN + ic * 16);
        epi.emit(wk.e, row0 + m, i0, src[0], src[1]);
    }
}

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class EpiG>
hipError_t mm2_grouped_staged_launch(const int8_t* Ap, const int8_t* W, size_t w_stride, int N, int K,
                                     const int* offsets, const MmWork* work, const int* nwork, int maxwork,
                                     const EpiG& epi, hipStream_t st) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    if (K % KS != 0 || N % 16 != 0) return hipErrorInvalidValue;
    if (maxwork <= 0) return hipSuccess;
    auto kern = mm2_grouped_staged_kernel<MB, NB, WM_, WN_, STAGES, KS, EpiG>;
    if (S::kLds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
        if (e != hipSuccess) return e;
    }
    kern<<<8 * ((maxwork + 7) / 8), S::kThreads, S::kLds, st>>>(Ap, W, w_stride, N, K, offsets, work, nwork, epi);
    return hipGetLastError();
}

// Token rows and weight rows of one grouped work item (for the work table).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS>
struct Mm2GroupedShape {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    static constexpr int kTokens = S::BR / 2;
    static constexpr int kRows = S::BN;
};

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS, class EpiG>
hipError_t mm2_grouped_launch(const int8_t* Ap, const int8_t* W, size_t w_stride, int N, int K, const int* offsets,
                              const MmWork* work, const int* nwork, int maxwork, const EpiG& epi, hipStream_t st) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    if (K % KS != 0) return hipErrorInvalidValue;
    if (maxwork <= 0) return hipSuccess;
    auto kern = mm2_grouped_kernel<MB, NB, WM_, WN_, STAGES, KS, EpiG>;
    if (S::kLds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
        if (e != hipSuccess) return e;
    }
    kern<<<8 * ((maxwork + 7) / 8), S::kThreads, S::kLds, st>>>(Ap, W, w_stride, N, K, offsets, work, nwork, epi);
    return hipGetLastError();
}

// K % KS == 0.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64, class Epi>
hipError_t mm2_launch(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi, hipStream_t st,
                      int group = 0) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    const int R2 = 2 * M;
    const int tiles_r = (R2 + S::BR - 1) / S::BR, tiles_n = (N + S::BN - 1) / S::BN;
    const TileOrder ord = TileOrder::of(tiles_r, tiles_n, group);
    const int ntiles = ord.count(tiles_n);
    auto kern = mm2_kernel<MB, NB, WM_, WN_, STAGES, KS, Epi>;
    if (S::kLds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
        if (e != hipSuccess) return e;
    }
    kern<<<8 * ((ntiles + 7) / 8), S::kThreads, S::kLds, st>>>(Ap, R2, W, N, K, ord, ntiles, epi);
    return hipGetLastError();
}

// Weights stream once per row tile; K split across blocks when there are
// fewer tiles than `fill` (slices of at least 512 bytes), partial sums
// through the i64 accumulator.  A split product ends with fin(acc, st) (the
// finish kernel that applies the epilogue and clears acc) and sets *split;
// otherwise the tiles apply epi themselves.  K % KS == 0.
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64, class Epi, class Fin>
hipError_t mm2_launch_splitk_fin(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi,
                                 const MmCtx* mm, int fill, hipStream_t st, const Fin& fin, bool* split) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    const Mm2SplitPlan p = mm2_split_plan<MB, NB, WM_, WN_, STAGES, KS>(M, N, K, mm->cus, mm->acc_elems, fill);
    *split = p.split;
    if (!p.split) return mm2_launch<MB, NB, WM_, WN_, STAGES, KS>(Ap, M, W, N, K, epi, st);
    auto kern = mm2_splitk_kernel<MB, NB, WM_, WN_, STAGES, KS>;
    if (S::kLds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)S::kLds);
        if (e != hipSuccess) return e;
    }
    kern<<<p.grid, S::kThreads, S::kLds, st>>>(Ap, 2 * M, W, N, K, Divider::of((uint32_t)p.tiles_r),
                                               Divider::of((uint32_t)p.ntiles), p.nitems, p.kslice, mm->acc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return fin(mm->acc, st);
}

template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64, class Epi>
hipError_t mm2_launch_splitk(const int8_t* Ap, int M, const int8_t* W, int N, int K, const Epi& epi, const MmCtx* mm,
                             int fill, hipStream_t st) {
    bool split = false;
    auto fin = [&](unsigned long long* acc, hipStream_t s) {
        const int colb = (N + 255) / 256;
        const int rows = std::max(1, std::min(M, (mm->cus * 8 + colb - 1) / colb));
        mm_splitk_finish_kernel<Epi><<<dim3(colb, rows), 256, 0, s>>>(acc, M, N, epi);
        return hipGetLastError();
    };
    return mm2_launch_splitk_fin<MB, NB, WM_, WN_, STAGES, KS>(Ap, M, W, N, K, epi, mm, fill, st, fin, &split);
}

// Block tiles of a launch shape (for the dispatch's tile count).
template <int MB, int NB, int WM_, int WN_, int STAGES, int KS = 64>
inline int mm2_tiles(int M, int N) {
    using S = Mm2<MB, NB, WM_, WN_, STAGES, KS>;
    return ((2 * M + S::BR - 1) / S::BR) * ((N + S::BN - 1) / S::BN);
}


inline hipError_t split_planes(const int16_t* x, int M, int ldx, int K, int8_t* Ap, hipStream_t st) {
    split_planes_kernel<><<<dim3((K / 8 + 255) / 256, M), 256, 0, st>>>(x, M, ldx, K, Ap);
    return hipGetLastError();
}

}  // namespace myl
