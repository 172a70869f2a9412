// gemm_frag.h -- the few-row W8A16 product of the decode batches (2 to 32
// token rows) on fragment-major weights.
//
// y[m][n] = sum_k W[n][k] * x[m][k] exactly, x split into the byte planes of
// gemm_mfma2.h (A' [2M x K], row 2m = hi(x_m), row 2m+1 = lo'(x_m)):
//   sum_k w*x = 256 * C'[2m][n] + C'[2m+1][n] + 128 * sum_k W[n][k].
//
// Weights: a second copy of W in the operand order of
// v_mfma_i32_16x16x64_i8.  Tile (g, t) holds weight rows 16g .. 16g+15 and K
// bytes 64t .. 64t+63 as 1 KiB in lane order: lane l's 16 bytes are row
// 16g + l % 16, bytes 64t + 16 (l / 16) .. +15 (rows past N are zero).  Tiles
// are stored row group by row group (g, then t), so a wave's 16-byte load
// of one tile is one contiguous KiB and lands in the B-operand registers.
//
// Launch: one block of 8 waves per CU (S P <= CUs blocks).  Block b takes K
// slice s = b / P and the row groups of part p = b % P; wave w of the block
// owns the KPW K tiles [s 8 KPW + w KPW, + KPW) and keeps their A' fragments
// in registers for the whole kernel (RT tiles of 16 plane rows each), then
// streams the weight tiles (g, its K tiles) of every row group g of the
// block: the eight waves read each row group's KT KiB side by side, so a
// block sweeps its weight range in order.  The batches of KPW tiles of two
// row groups alternate in two register buffers.  Each wave adds its partial
// sums of a row group into LDS (exact i32 plane sums); after the stream the
// block hands every exact sum of its rows to the output policy: the whole
// product's epilogue when there is one K slice, the split-K accumulator
// otherwise.
//
// Bounds: |plane sum| <= 128 * 128 * K < 2^31 for K < 2^17.
#pragma once

#include "bufload.h"
#include "gemm_mfma.h"
#include "internal.h"
#include "mm_plan.h"
#include "wave.h"

#include <algorithm>

namespace myl {

constexpr int kFragWeightCpol = 2;  // streaming (read once per product)

// Bytes of the fragment copy of an N x K weight matrix (K % 64 == 0).
inline size_t frag_bytes(int N, int K) { return (size_t)((N + 15) / 16) * (size_t)(K / 64) * 1024; }

// Row-major W [N x K] -> the fragment copy.  One wave per tile: grid
// (ceil(KT / 4), NG), tile (g = blockIdx.y, t = 4 blockIdx.x + wave).
__global__ __launch_bounds__(256) void frag_relayout_kernel(const int8_t* __restrict__ W, int N, int K,
                                                            int8_t* __restrict__ Wf) {
    const int KT = K / 64;
    const int g = blockIdx.y, t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= KT) return;
    const int l = threadIdx.x & 63;
    const int n = 16 * g + (l & 15);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (n < N) v = *reinterpret_cast<const uint4*>(W + (size_t)n * K + 64 * t + 16 * (l >> 4));
    *reinterpret_cast<uint4*>(Wf + ((size_t)g * KT + t) * 1024 + l * 16) = v;
}

inline hipError_t frag_relayout(const int8_t* W, int N, int K, int8_t* Wf, hipStream_t st) {
    if (N <= 0 || K <= 0 || K % 64 != 0 || (N + 15) / 16 > 65535) return hipErrorInvalidValue;
    frag_relayout_kernel<<<dim3((K / 64 + 3) / 4, (N + 15) / 16), 256, 0, st>>>(W, N, K, Wf);
    return hipGetLastError();
}

// The exact sums of a block's rows, read back from the LDS reduction.
template <int RT>
struct FragSums {
    const int32_t* red;  // [ngb][RT * 16][16] plane sums
    const int32_t* rsl;  // [ngb][16] weight row sums
    __device__ inline int64_t operator()(int gg, int m, int c) const {
        const int32_t* rg = red + (size_t)gg * RT * 256;
        return 256ll * rg[(2 * m) * 16 + c] + (int64_t)rg[(2 * m + 1) * 16 + c] + 128ll * rsl[gg * 16 + c];
    }
};

// Output policies:
//   Pre; pre(g0, ngb, R, N)          per thread at kernel start: loads of the
//                                     operands its outputs need that do not
//                                     depend on the sums (in registers during
//                                     the stream, so the tail waits for none)
//   run(pre, sums, g0, ngb, R, N, lds_free)   whole block, after the reduction
//                                     (lds_free: at least R x 16 ngb int16)
// Threads take fixed output columns (FragCols): the block's columns rounded
// up to a power of two w <= 512, thread t on column t % w and rows t / w,
// + 512 / w, ... (shifts and masks: no division in the kernels).
struct FragCols {
    int lg, w, slices;
    __device__ static inline FragCols of(int cols) {
        const int lg = cols <= 1 ? 0 : 32 - __builtin_clz((unsigned)(cols - 1));
        return FragCols{lg, 1 << lg, max(1, (kFragWaves * 64) >> lg)};
    }
    __device__ inline int col() const { return (int)threadIdx.x & (w - 1); }
    __device__ inline int row0() const { return (int)threadIdx.x >> lg; }
};

// Split-K partial sums into acc [M x N] (u64, zero-kept).
struct FragOutAtomic {
    unsigned long long* acc;
    struct Pre {};
    __device__ inline Pre pre(int, int, int, int) const { return Pre{}; }
    template <int RT>
    __device__ inline void run(const Pre&, const FragSums<RT>& s, int g0, int ngb, int R, int N, int8_t*) const {
        const int ncol = 16 * ngb;
        const FragCols fc = FragCols::of(ncol);
        const int c = fc.col(), n = 16 * g0 + c;
        if (c >= ncol || n >= N) return;
        for (int m = fc.row0(); m < R; m += fc.slices)
            atomicAdd(acc + (size_t)m * N + n, (unsigned long long)s(c >> 4, m, c & 15));
    }
};

// The staged epilogue of mm2_staged_kernel (EpiGUSiluPlanes): the int16 of
// every output (Epi::stage_with(op(n), n, sum), op(n) fetched before the
// stream), then Epi::emit(m, i0, ...) for the 16 staged values of columns
// 2 i0 .. 2 i0 + 15.  N % 16 == 0, 16 ngb <= 512.
template <class Epi>
struct FragOutStaged {
    Epi epi;
    struct Pre { typename Epi::Op op; };
    __device__ inline Pre pre(int g0, int ngb, int, int N) const {
        const int c = FragCols::of(16 * ngb).col();
        return Pre{epi.op(min(16 * g0 + c, N - 1))};
    }
    template <int RT>
    __device__ inline void run(const Pre& pr, const FragSums<RT>& s, int g0, int ngb, int R, int N,
                               int8_t* lds_free) const {
        int16_t* tile = reinterpret_cast<int16_t*>(lds_free);  // [R][16 ngb]
        const int ld = 16 * ngb;
        const FragCols fc = FragCols::of(ld);
        const int c = fc.col(), n = 16 * g0 + c;
        if (c < ld)
            for (int m = fc.row0(); m < R; m += fc.slices)
                tile[m * ld + c] = n < N ? epi.stage_with(pr.op, n, s(c >> 4, m, c & 15)) : (int16_t)0;
        __syncthreads();
        const FragCols fe = FragCols::of(ngb);  // one emit per (row group, row)
        const int gg = fe.col();
        if (gg >= ngb || 16 * (g0 + gg) >= N) return;
        for (int m = fe.row0(); m < R; m += fe.slices) {
            const uint4* src = reinterpret_cast<const uint4*>(tile + m * ld + 16 * gg);
            epi.emit(m, 8 * (g0 + gg), src[0], src[1]);
        }
    }
};

template <int RT, int KPW, class Out>
__global__ __launch_bounds__(kFragWaves * 64) void frag_mm_kernel(const int8_t* __restrict__ Ap, int R2, int K,
                                                                  const int8_t* __restrict__ Wf, int N, int NG,
                                                                  Divider P, Out out) {
    extern __shared__ __align__(16) int8_t lds[];
    const int KT = K >> 6;
    uint32_t s, p, g0u, g1u, rem;
    P.divmod(blockIdx.x, s, p);
    P.divmod(p * (uint32_t)NG, g0u, rem);  // p NG < 2^32: P <= 256 CUs, NG < 2^16
    P.divmod((p + 1) * (uint32_t)NG, g1u, rem);
    const int g0 = (int)g0u, g1 = (int)g1u;
    const int ngb = g1 - g0;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int kb = ((int)s * kFragWaves + wave) * KPW;  // first K tile of the wave
    const int kn = max(0, min(KPW, KT - kb));           // K tiles it owns (0 past K)
    int32_t* red = reinterpret_cast<int32_t*>(lds);
    int32_t* rsl = red + (size_t)ngb * RT * 256;
    // A' fragments of the wave's K tiles (clamped into the matrix; tiles past
    // kn are never used)
    v4i32_t a[KPW][RT];
#pragma unroll
    for (int j = 0; j < KPW; ++j) {
        const int t = min(kb + j, KT - 1);
#pragma unroll
        for (int i = 0; i < RT; ++i) {
            const int row = min(16 * i + (lane & 15), R2 - 1);
            a[j][i] = *reinterpret_cast<const v4i32_t*>(Ap + (size_t)row * K + 64 * t + 16 * (lane >> 4));
        }
    }
    for (int i = threadIdx.x; i < ngb * (RT * 256 + 16); i += kFragWaves * 64) red[i] = 0;
    // Weight loads go through a buffer descriptor over the block's row groups
    // (streaming cache policy): they keep their order around the scheduling
    // barriers below, and a load past the block's tiles (the batches after
    // the last row group) returns zeros without touching memory.
    const uint32_t bbytes = (uint32_t)ngb * (uint32_t)KT * 1024u;
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(Wf + (size_t)g0 * KT * 1024, bbytes);
    const uint32_t wlane = (uint32_t)lane * 16u + (uint32_t)kb * 1024u;
    auto load = [&](v4i32_t (&buf)[KPW], int g) {
        const uint32_t base = (uint32_t)g * (uint32_t)KT * 1024u + wlane;
#pragma unroll
        for (int j = 0; j < KPW; ++j) {
            // tiles past the wave's K range or the block's row groups read as zeros
            const uint32_t off = (g < ngb && j < kn) ? base + (uint32_t)j * 1024u : bbytes;
            buf[j] = __builtin_amdgcn_raw_buffer_load_b128(wr, (int)off, 0, kFragWeightCpol);
        }
    };
    v4i32_t bA[KPW], bB[KPW];
    const bool any = kn > 0 && ngb > 0;
    if (any) {
        load(bA, 0);
        load(bB, 1);
    }
    const typename Out::Pre pre = out.pre(g0, ngb, R2 >> 1, N);
    __syncthreads();  // red cleared
    auto compute = [&](const v4i32_t (&buf)[KPW], int g) {
        v4i32_t acc[RT];
#pragma unroll
        for (int i = 0; i < RT; ++i) acc[i] = v4i32_t{0, 0, 0, 0};
        int32_t rs = 0;
#pragma unroll
        for (int j = 0; j < KPW; ++j) {
            const v4i32_t w = buf[j];
#pragma unroll
            for (int i = 0; i < RT; ++i) acc[i] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[j][i], w, acc[i], 0, 0, 0);
            rs = sdot4((uint32_t)w[0], 0x01010101u, rs);
            rs = sdot4((uint32_t)w[1], 0x01010101u, rs);
            rs = sdot4((uint32_t)w[2], 0x01010101u, rs);
            rs = sdot4((uint32_t)w[3], 0x01010101u, rs);
        }
        // accumulator row 4 (l / 16) + r of tile i, column l % 16
        int32_t* rg = red + (size_t)g * RT * 256;
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) atomicAdd(rg + (16 * i + 4 * (lane >> 4) + r) * 16 + (lane & 15), acc[i][r]);
        atomicAdd(rsl + g * 16 + (lane & 15), rs);
    };
    // (the loads of a batch stay where they are issued: the scheduler would
    // otherwise sink them below the next batch's multiplies, whose wait then
    // drains every load in flight)
    if (any) {
        for (int g = 0; g < ngb; g += 2) {
            compute(bA, g);
            load(bA, g + 2);
            __builtin_amdgcn_sched_barrier(0);
            if (g + 1 < ngb) compute(bB, g + 1);
            load(bB, g + 3);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    __syncthreads();
    out.template run<RT>(pre, FragSums<RT>{red, rsl}, g0, ngb, R2 >> 1, N,
                         reinterpret_cast<int8_t*>(rsl + (size_t)ngb * 16));
}

// ---- launches ---------------------------------------------------------------

template <int RT, int KPW, class Out>
hipError_t frag_launch(const int8_t* Ap, int R, int K, const int8_t* Wf, int N, int S, int P, size_t lds, const Out& out,
                       hipStream_t st) {
    auto kern = frag_mm_kernel<RT, KPW, Out>;
    // set on every launch, as the other product launchers do: the attribute
    // belongs to the current device
    hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    kern<<<S * P, kFragWaves * 64, lds, st>>>(Ap, 2 * R, K, Wf, N, (N + 15) / 16, Divider::of((uint32_t)P), out);
    return hipGetLastError();
}

// One K slice: every sum of a block's rows goes to the output policy (the
// staged epilogue needs its LDS tile: staged = true).
template <class Out>
hipError_t frag_mm_full(const int8_t* Ap, int R, int K, const int8_t* Wf, int N, const Out& out, bool staged, int cus,
                        hipStream_t st) {
    if (!frag_full_ok(R, K, N, cus)) return hipErrorInvalidValue;
    const int KT = K / 64, NG = N / 16, rt = frag_rt(R);
    const int ngb = (NG + cus - 1) / cus;
    const size_t lds = frag_lds(rt, ngb, R, staged);
    const bool k7 = KT <= kFragWaves * 7;  // seven K tiles per wave suffice
    switch (rt) {
    case 1: return k7 ? frag_launch<1, 7>(Ap, R, K, Wf, N, 1, cus, lds, out, st) : frag_launch<1, 8>(Ap, R, K, Wf, N, 1, cus, lds, out, st);
    case 2: return k7 ? frag_launch<2, 7>(Ap, R, K, Wf, N, 1, cus, lds, out, st) : frag_launch<2, 8>(Ap, R, K, Wf, N, 1, cus, lds, out, st);
    default: return k7 ? frag_launch<4, 7>(Ap, R, K, Wf, N, 1, cus, lds, out, st) : frag_launch<4, 8>(Ap, R, K, Wf, N, 1, cus, lds, out, st);
    }
}

template <class Epi>
hipError_t frag_mm_staged(const int8_t* Ap, int R, int K, const int8_t* Wf, int N, const Epi& epi, int cus,
                          hipStream_t st) {
    return frag_mm_full(Ap, R, K, Wf, N, FragOutStaged<Epi>{epi}, true, cus, st);
}

// The K-sliced product: each slice's partial sums added into acc [R x N].
inline hipError_t frag_mm_split(const int8_t* Ap, int R, int K, const int8_t* Wf, int N, unsigned long long* acc,
                                int cus, size_t acc_elems, hipStream_t st) {
    if (!frag_split_ok(R, K, N, cus, acc_elems)) return hipErrorInvalidValue;
    const FragSplit sp = frag_split_plan(K, N, cus);
    const int rt = frag_rt(R);
    const size_t lds = frag_lds(rt, sp.ngb, R, false);
    const FragOutAtomic out{acc};
    if (sp.kpw == 5) {
        switch (rt) {
        case 1: return frag_launch<1, 5>(Ap, R, K, Wf, N, sp.S, sp.P, lds, out, st);
        case 2: return frag_launch<2, 5>(Ap, R, K, Wf, N, sp.S, sp.P, lds, out, st);
        default: return frag_launch<4, 5>(Ap, R, K, Wf, N, sp.S, sp.P, lds, out, st);
        }
    }
    switch (rt) {
    case 1: return frag_launch<1, 8>(Ap, R, K, Wf, N, sp.S, sp.P, lds, out, st);
    case 2: return frag_launch<2, 8>(Ap, R, K, Wf, N, sp.S, sp.P, lds, out, st);
    default: return frag_launch<4, 8>(Ap, R, K, Wf, N, sp.S, sp.P, lds, out, st);
    }
}

}  // namespace myl
