// gemm_mfma.h -- W8A16 matrix-matrix products on the int8 matrix cores (gfx950).
//
// y[m][n] = epilogue(n, m, sum_k W[n][k] * x[m][k])   (exact i64 sums)
//
// The same sum as the GEMV (dot.rs:141-147), for M activation rows at once.
// The int16 activation is split x = 256*hi + lo' + 128 (hi = x >> 8 and
// lo' = (x & 255) - 128, both signed bytes), so
//   sum w*x = 256 * sum(w*hi) + sum(w*lo') + 128 * sum(w)
// The first two sums are v_mfma_i32_32x32x32_i8 products (A = activation
// plane, B = weight rows); the weight row sums come from v_dot4 on the B
// fragments the wave already holds, issued between the matrix instructions.
// Each i32 accumulator is exact: |w*hi|, |w*lo'| <= 128*128, so a K range
// below 131072 stays below 2^31 (128*128*131072 = 2^31).
//
// Tiling: a block of WAVES_M x WAVES_N waves owns a BM x BN output tile
// (BM = 32*WM*WAVES_M activation rows, BN = 32*WN*WAVES_N weight rows), each
// wave a (32*WM) x (32*WN) sub-tile.  K advances 64 bytes per stage through
// two LDS buffers (global loads of stage s+1 are in flight while stage s is
// multiplied).  LDS rows are padded to 80 bytes: the 16-byte reads of 8
// consecutive rows then fall on disjoint banks.
//
// Split K: with ksplit > 1 the K range is cut into ksplit slices (multiples of
// 64); each block adds its exact partial sum into an i64 [M x N] accumulator
// with 64-bit atomics (order-free), and a second kernel applies the epilogue
// and clears the accumulator for the next call.
//
// XCD-aware order: workgroups go to the 8 XCDs round robin, so block b is
// given tile (b % 8) * (grid / 8) + b / 8 -- each XCD works on one contiguous
// run of tiles, activation rows fastest, so consecutive tiles on one XCD read
// the same weight rows from that XCD's L2.
#pragma once

#include "gemv.h"

namespace myl {

typedef int v4i32_t __attribute__((ext_vector_type(4)));
typedef int v16i32_t __attribute__((ext_vector_type(16)));

constexpr int kMmBK = 64;           // K bytes per stage
constexpr int kMmStride = kMmBK + 16;  // LDS row stride (bytes)

template <int WM, int WN, int WAVES_M, int WAVES_N>
struct MmShape {
    static constexpr int kThreads = WAVES_M * WAVES_N * 64;
    static constexpr int BM = 32 * WM * WAVES_M;
    static constexpr int BN = 32 * WN * WAVES_N;
    static constexpr int kPlaneA = BM * kMmStride;
    static constexpr int kPlaneB = BN * kMmStride;
    static constexpr int kStage = 2 * kPlaneA + kPlaneB;
    static constexpr size_t kLds = 2 * (size_t)kStage;
    static constexpr int XCH = BM * kMmBK / 8;   // 16-byte chunks of x (8 int16) per stage
    static constexpr int WCH = BN * kMmBK / 16;  // 16-byte chunks of W per stage
    static constexpr int XPT = (XCH + kThreads - 1) / kThreads;
    static constexpr int WPT = (WCH + kThreads - 1) / kThreads;
};

// 8 int16 (one uint4) -> 8 hi bytes and 8 lo' bytes.
__device__ inline void split_planes8(const uint4 v, uint2& h, uint2& l) {
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    uint32_t hh[2], ll[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t d0 = d[2 * t], d1 = d[2 * t + 1];
        hh[t] = ((d0 >> 8) & 0xFFu) | ((d0 >> 16) & 0xFF00u) | ((d1 << 8) & 0xFF0000u) | (d1 & 0xFF000000u);
        ll[t] = ((d0 & 0xFFu) | ((d0 >> 8) & 0xFF00u) | ((d1 << 16) & 0xFF0000u) | ((d1 << 8) & 0xFF000000u)) ^ 0x80808080u;
    }
    h = make_uint2(hh[0], hh[1]);
    l = make_uint2(ll[0], ll[1]);
}

// Exact sums of one block tile over k in [kb, ke) (kb, ke multiples of 64, or
// ke = K).  Calls sink(n, m, sum) for every in-range (m, n) of the tile.
template <int WM, int WN, int WAVES_M, int WAVES_N, class Sink>
__device__ inline void mm_w8_tile(const int16_t* __restrict__ x, int M, int ldx, const int8_t* __restrict__ W,
                                  int N, int K, int m0, int n0, int kb, int ke, int8_t* lds, const Sink& sink) {
    using S = MmShape<WM, WN, WAVES_M, WAVES_N>;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;

    uint4 xr[S::XPT], wr[S::WPT];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < S::XPT; ++i) {
            const int c = tid + i * S::kThreads;
            const int row = c / (kMmBK / 8), kc = c % (kMmBK / 8);
            const int gm = m0 + row, gk = k0 + kc * 8;
            xr[i] = (c < S::XCH && gm < M && gk < ke) ? *reinterpret_cast<const uint4*>(x + (size_t)gm * ldx + gk)
                                                      : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < S::WPT; ++i) {
            const int c = tid + i * S::kThreads;
            const int row = c / (kMmBK / 16), kc = c % (kMmBK / 16);
            const int gn = n0 + row, gk = k0 + kc * 16;
            wr[i] = (c < S::WCH && gn < N && gk < ke) ? *reinterpret_cast<const uint4*>(W + (size_t)gn * K + gk)
                                                      : make_uint4(0, 0, 0, 0);
        }
    };
    auto swrite = [&](int8_t* st) {
        int8_t* ah = st;
        int8_t* al = st + S::kPlaneA;
        int8_t* bw = st + 2 * S::kPlaneA;
#pragma unroll
        for (int i = 0; i < S::XPT; ++i) {
            const int c = tid + i * S::kThreads;
            if (c < S::XCH) {
                const int row = c / (kMmBK / 8), kc = c % (kMmBK / 8);
                uint2 h, l;
                split_planes8(xr[i], h, l);
                *reinterpret_cast<uint2*>(ah + row * kMmStride + kc * 8) = h;
                *reinterpret_cast<uint2*>(al + row * kMmStride + kc * 8) = l;
            }
        }
#pragma unroll
        for (int i = 0; i < S::WPT; ++i) {
            const int c = tid + i * S::kThreads;
            if (c < S::WCH) {
                const int row = c / (kMmBK / 16), kc = c % (kMmBK / 16);
                *reinterpret_cast<uint4*>(bw + row * kMmStride + kc * 16) = wr[i];
            }
        }
    };

    v16i32_t acc_h[WM][WN], acc_l[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) { acc_h[i][j][r] = 0; acc_l[i][j][r] = 0; }
    int32_t rs[WN];
#pragma unroll
    for (int j = 0; j < WN; ++j) rs[j] = 0;

    auto compute = [&](const int8_t* st) {
        const int8_t* ah = st;
        const int8_t* al = st + S::kPlaneA;
        const int8_t* bw = st + 2 * S::kPlaneA;
#pragma unroll
        for (int s = 0; s < kMmBK / 32; ++s) {
            const int koff = s * 32 + (lane >> 5) * 16;
            v4i32_t a_h[WM], a_l[WM], b[WN];
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int row = (wn * WN + j) * 32 + (lane & 31);
                b[j] = *reinterpret_cast<const v4i32_t*>(bw + row * kMmStride + koff);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int row = (wm * WM + i) * 32 + (lane & 31);
                a_h[i] = *reinterpret_cast<const v4i32_t*>(ah + row * kMmStride + koff);
                a_l[i] = *reinterpret_cast<const v4i32_t*>(al + row * kMmStride + koff);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    acc_h[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_h[i], b[j], acc_h[i][j], 0, 0, 0);
                    acc_l[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_l[i], b[j], acc_l[i][j], 0, 0, 0);
                }
                rs[j] = sdot4((uint32_t)b[j][0], 0x01010101u, rs[j]);
                rs[j] = sdot4((uint32_t)b[j][1], 0x01010101u, rs[j]);
                rs[j] = sdot4((uint32_t)b[j][2], 0x01010101u, rs[j]);
                rs[j] = sdot4((uint32_t)b[j][3], 0x01010101u, rs[j]);
            }
        }
    };

    const int nk = (ke - kb + kMmBK - 1) / kMmBK;
    gload(kb);
    swrite(lds);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        int8_t* cur = lds + (kt & 1) * S::kStage;
        const bool more = kt + 1 < nk;
        if (more) gload(kb + (kt + 1) * kMmBK);
        compute(cur);
        if (more) swrite(lds + ((kt + 1) & 1) * S::kStage);
        __syncthreads();
    }

    // Row sums: lanes l and l ^ 32 hold the two 16-byte halves of each k-step.
#pragma unroll
    for (int j = 0; j < WN; ++j) rs[j] += __shfl_xor(rs[j], 32);
    // 32x32 accumulator layout: lane l holds column l % 32 (a weight row) and
    // rows 8 * (r / 4) + 4 * (l / 32) + r % 4 (activation rows) in register r.
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int n = n0 + (wn * WN + j) * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int m = m0 + (wm * WM + i) * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (m < M && n < N)
                    sink(n, m, (int64_t)acc_h[i][j][r] * 256 + (int64_t)acc_l[i][j][r] + (int64_t)rs[j] * 128);
            }
        }
}

// ---- int16 weights (the LM head of model.rs:285-296) --------------------------
//
// Both operands are split: x = Xa + 128 with Xa = 256*xh + xl', and likewise
// w = Wa + 128.  Then per k
//   x*w = 65536*xh*wh + 256*(xh*wl' + xl'*wh) + xl'*wl' + 128*Wa + 128*Xa + 16384
// so four int8 products per tile plus the row sums of Wa (from the B
// fragments) and of Xa (from the A fragments).  A zero-padded slot (x = w = 0,
// i.e. Xa = Wa = -128) contributes exactly 0, so the constant term counts
// every processed slot.  Partial sums stay exact in i32 for K < 65536
// (|Wa|, |Xa| <= 32768).

template <int WM, int WN, int WAVES_M, int WAVES_N>
struct Mm16Shape {
    static constexpr int kThreads = WAVES_M * WAVES_N * 64;
    static constexpr int BM = 32 * WM * WAVES_M;
    static constexpr int BN = 32 * WN * WAVES_N;
    static constexpr int kPlaneA = BM * kMmStride;
    static constexpr int kPlaneB = BN * kMmStride;
    static constexpr int kStage = 2 * kPlaneA + 2 * kPlaneB;
    static constexpr size_t kLds = 2 * (size_t)kStage;
    static constexpr int XCH = BM * kMmBK / 8;
    static constexpr int WCH = BN * kMmBK / 8;
    static constexpr int XPT = (XCH + kThreads - 1) / kThreads;
    static constexpr int WPT = (WCH + kThreads - 1) / kThreads;
};

template <int WM, int WN, int WAVES_M, int WAVES_N, class Sink>
__device__ inline void mm_w16_tile(const int16_t* __restrict__ x, int M, int ldx, const int16_t* __restrict__ W,
                                   int N, int K, int m0, int n0, int kb, int ke, int8_t* lds, const Sink& sink) {
    using S = Mm16Shape<WM, WN, WAVES_M, WAVES_N>;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WAVES_M, wn = wave / WAVES_M;

    uint4 xr[S::XPT], wr[S::WPT];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < S::XPT; ++i) {
            const int c = tid + i * S::kThreads;
            const int row = c / (kMmBK / 8), kc = c % (kMmBK / 8);
            const int gm = m0 + row, gk = k0 + kc * 8;
            xr[i] = (c < S::XCH && gm < M && gk < ke) ? *reinterpret_cast<const uint4*>(x + (size_t)gm * ldx + gk)
                                                      : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < S::WPT; ++i) {
            const int c = tid + i * S::kThreads;
            const int row = c / (kMmBK / 8), kc = c % (kMmBK / 8);
            const int gn = n0 + row, gk = k0 + kc * 8;
            wr[i] = (c < S::WCH && gn < N && gk < ke) ? *reinterpret_cast<const uint4*>(W + (size_t)gn * K + gk)
                                                      : make_uint4(0, 0, 0, 0);
        }
    };
    auto swrite = [&](int8_t* st) {
        int8_t* ah = st;
        int8_t* al = st + S::kPlaneA;
        int8_t* bh = st + 2 * S::kPlaneA;
        int8_t* bl = bh + S::kPlaneB;
#pragma unroll
        for (int i = 0; i < S::XPT; ++i) {
            const int c = tid + i * S::kThreads;
            if (c < S::XCH) {
                const int row = c / (kMmBK / 8), kc = c % (kMmBK / 8);
                uint2 h, l;
                split_planes8(xr[i], h, l);
                *reinterpret_cast<uint2*>(ah + row * kMmStride + kc * 8) = h;
                *reinterpret_cast<uint2*>(al + row * kMmStride + kc * 8) = l;
            }
        }
#pragma unroll
        for (int i = 0; i < S::WPT; ++i) {
            const int c = tid + i * S::kThreads;
            if (c < S::WCH) {
                const int row = c / (kMmBK / 8), kc = c % (kMmBK / 8);
                uint2 h, l;
                split_planes8(wr[i], h, l);
                *reinterpret_cast<uint2*>(bh + row * kMmStride + kc * 8) = h;
                *reinterpret_cast<uint2*>(bl + row * kMmStride + kc * 8) = l;
            }
        }
    };

    v16i32_t hh[WM][WN], hl[WM][WN], lh[WM][WN], ll[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) { hh[i][j][r] = 0; hl[i][j][r] = 0; lh[i][j][r] = 0; ll[i][j][r] = 0; }
    int32_t ws[WN], xs[WM];
#pragma unroll
    for (int j = 0; j < WN; ++j) ws[j] = 0;
#pragma unroll
    for (int i = 0; i < WM; ++i) xs[i] = 0;
    auto sum16 = [](const v4i32_t& h, const v4i32_t& l, int32_t acc) {
        int32_t sh = 0, sl = 0;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            sh = sdot4((uint32_t)h[t], 0x01010101u, sh);
            sl = sdot4((uint32_t)l[t], 0x01010101u, sl);
        }
        return acc + sh * 256 + sl;
    };

    auto compute = [&](const int8_t* st) {
        const int8_t* ah = st;
        const int8_t* al = st + S::kPlaneA;
        const int8_t* bh = st + 2 * S::kPlaneA;
        const int8_t* bl = bh + S::kPlaneB;
#pragma unroll
        for (int s = 0; s < kMmBK / 32; ++s) {
            const int koff = s * 32 + (lane >> 5) * 16;
            v4i32_t a_h[WM], a_l[WM], b_h[WN], b_l[WN];
#pragma unroll
            for (int j = 0; j < WN; ++j) {
                const int row = (wn * WN + j) * 32 + (lane & 31);
                b_h[j] = *reinterpret_cast<const v4i32_t*>(bh + row * kMmStride + koff);
                b_l[j] = *reinterpret_cast<const v4i32_t*>(bl + row * kMmStride + koff);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i) {
                const int row = (wm * WM + i) * 32 + (lane & 31);
                a_h[i] = *reinterpret_cast<const v4i32_t*>(ah + row * kMmStride + koff);
                a_l[i] = *reinterpret_cast<const v4i32_t*>(al + row * kMmStride + koff);
            }
#pragma unroll
            for (int j = 0; j < WN; ++j) {
#pragma unroll
                for (int i = 0; i < WM; ++i) {
                    hh[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_h[i], b_h[j], hh[i][j], 0, 0, 0);
                    hl[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_h[i], b_l[j], hl[i][j], 0, 0, 0);
                    lh[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_l[i], b_h[j], lh[i][j], 0, 0, 0);
                    ll[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_l[i], b_l[j], ll[i][j], 0, 0, 0);
                }
                ws[j] = sum16(b_h[j], b_l[j], ws[j]);
            }
#pragma unroll
            for (int i = 0; i < WM; ++i) xs[i] = sum16(a_h[i], a_l[i], xs[i]);
        }
    };

    const int nk = (ke - kb + kMmBK - 1) / kMmBK;
    gload(kb);
    swrite(lds);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        int8_t* cur = lds + (kt & 1) * S::kStage;
        const bool more = kt + 1 < nk;
        if (more) gload(kb + (kt + 1) * kMmBK);
        compute(cur);
        if (more) swrite(lds + ((kt + 1) & 1) * S::kStage);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < WN; ++j) ws[j] += __shfl_xor(ws[j], 32);
#pragma unroll
    for (int i = 0; i < WM; ++i) xs[i] += __shfl_xor(xs[i], 32);
    const int64_t cterm = (int64_t)16384 * (int64_t)nk * kMmBK;
#pragma unroll
    for (int i = 0; i < WM; ++i)
#pragma unroll
        for (int j = 0; j < WN; ++j) {
            const int n = n0 + (wn * WN + j) * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int ml = 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                const int32_t xsum = __shfl(xs[i], ml);  // row ml's sum lives in lane ml
                const int m = m0 + (wm * WM + i) * 32 + ml;
                const int64_t v = (int64_t)hh[i][j][r] * 65536 + ((int64_t)hl[i][j][r] + (int64_t)lh[i][j][r]) * 256 +
                                  (int64_t)ll[i][j][r] + ((int64_t)ws[j] + (int64_t)xsum) * 128 + cterm;
                if (m < M && n < N) sink(n, m, v);
            }
        }
}

// Tile index of this block (XCD-aware order, see above); -1 when idle.
__device__ inline int mm_tile_index(int ntiles) {
    const int b = blockIdx.x;
    const int t = (b & 7) * (int)(gridDim.x >> 3) + (b >> 3);
    return t < ntiles ? t : -1;
}

template <class Epi>
struct SinkEpi {
    const Epi& e;
    __device__ inline void operator()(int n, int m, int64_t v) const { e.one(n, m, v); }
};
struct SinkAtomic {
    unsigned long long* acc;
    int ldn;
    __device__ inline void operator()(int n, int m, int64_t v) const {
        atomicAdd(acc + (size_t)m * ldn + n, (unsigned long long)v);
    }
};

// Unsigned n / d and n % d with the host-computed reciprocal of d (fixed.h):
// index arithmetic without the float-reciprocal sequence of a plain `/`.
struct Divider {
    uint32_t d;
    uint64_t m;
    static Divider of(uint32_t d) { return Divider{d, recip32(d)}; }
    __device__ inline void divmod(uint32_t n, uint32_t& q, uint32_t& r) const { udivmod32(n, d, m, &q, &r); }
};

// grid = 8 * ceil(tiles / 8); tile t -> (t % tiles_m, t / tiles_m).
template <int WM, int WN, int WAVES_M, int WAVES_N, class Epi>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void mm_w8_kernel(const int16_t* __restrict__ x, int M, int ldx,
                                                                      const int8_t* __restrict__ W, int N, int K,
                                                                      Divider tiles_m, int ntiles, Epi epi) {
    using S = MmShape<WM, WN, WAVES_M, WAVES_N>;
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(ntiles);
    if (t < 0) return;
    uint32_t tn, tm;
    tiles_m.divmod((uint32_t)t, tn, tm);
    mm_w8_tile<WM, WN, WAVES_M, WAVES_N>(x, M, ldx, W, N, K, (int)tm * S::BM, (int)tn * S::BN, 0, K, lds,
                                         SinkEpi<Epi>{epi});
}

// Split-K variant: work item t covers tile t % ntiles_mn and K slice
// t / ntiles_mn (slices of kslice bytes, a multiple of 64).
template <int WM, int WN, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void mm_w8_splitk_kernel(
    const int16_t* __restrict__ x, int M, int ldx, const int8_t* __restrict__ W, int N, int K, Divider tiles_m,
    Divider ntiles_mn, int nitems, int kslice, unsigned long long* __restrict__ acc) {
    using S = MmShape<WM, WN, WAVES_M, WAVES_N>;
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(nitems);
    if (t < 0) return;
    uint32_t ks, tile, tn, tm;
    ntiles_mn.divmod((uint32_t)t, ks, tile);
    tiles_m.divmod(tile, tn, tm);
    const int kb = (int)ks * kslice, ke = min(K, kb + kslice);
    if (kb >= ke) return;
    mm_w8_tile<WM, WN, WAVES_M, WAVES_N>(x, M, ldx, W, N, K, (int)tm * S::BM, (int)tn * S::BN, kb, ke, lds,
                                         SinkAtomic{acc, N});
}

template <int WM, int WN, int WAVES_M, int WAVES_N, class Epi>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void mm_w16_kernel(const int16_t* __restrict__ x, int M,
                                                                       int ldx, const int16_t* __restrict__ W, int N,
                                                                       int K, Divider tiles_m, int ntiles, Epi epi) {
    using S = Mm16Shape<WM, WN, WAVES_M, WAVES_N>;
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(ntiles);
    if (t < 0) return;
    uint32_t tn, tm;
    tiles_m.divmod((uint32_t)t, tn, tm);
    mm_w16_tile<WM, WN, WAVES_M, WAVES_N>(x, M, ldx, W, N, K, (int)tm * S::BM, (int)tn * S::BN, 0, K, lds,
                                          SinkEpi<Epi>{epi});
}

// ---- grouped products (MoE experts) ------------------------------------------
//
// One launch covers every expert: work item t = (expert e, row tile m0,
// column tile n0) of a table built from the experts' row counts.  Expert e
// owns activation rows [offsets[e], offsets[e + 1]) of x and the weight
// matrix W + e * w_stride; the epilogue gets (e, n, global row, sum).
struct MmWork { int e, m0, n0, pad; };

template <class EpiG>
struct SinkGrouped {
    const EpiG& epi;
    int e, row0;
    __device__ inline void operator()(int n, int m, int64_t v) const { epi.one(e, n, row0 + m, v); }
};

template <int WM, int WN, int WAVES_M, int WAVES_N, class EpiG>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void mm_w8_grouped_kernel(
    const int16_t* __restrict__ x, int ldx, const int8_t* __restrict__ W, size_t w_stride, int N, int K,
    const int* __restrict__ offsets, const MmWork* __restrict__ work, int nwork, EpiG epi) {
    extern __shared__ __align__(16) int8_t lds[];
    const int t = mm_tile_index(nwork);
    if (t < 0) return;
    const MmWork wk = work[t];
    const int row0 = offsets[wk.e];
    const int Me = offsets[wk.e + 1] - row0;
    mm_w8_tile<WM, WN, WAVES_M, WAVES_N>(x + (size_t)row0 * ldx, Me, ldx, W + (size_t)wk.e * w_stride, N, K, wk.m0,
                                         wk.n0, 0, K, lds, SinkGrouped<EpiG>{epi, wk.e, row0});
}

// Epilogue over the split-K accumulator; clears it for the next call.
// grid (ceil(N / 256), rows): block (x, y) handles columns x * 256 .. of rows
// y, y + gridDim.y, ...
template <class Epi>
__global__ __launch_bounds__(256) void mm_splitk_finish_kernel(unsigned long long* __restrict__ acc, int M, int N,
                                                              Epi epi) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    if (n >= N) return;
    for (int m = blockIdx.y; m < M; m += gridDim.y) {
        unsigned long long* p = acc + (size_t)m * N + n;
        const int64_t v = (int64_t)*p;
        *p = 0;
        epi.one(n, m, v);
    }
}

}  // namespace myl
