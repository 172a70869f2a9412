// gemv_stream.h -- persistent, wave-streaming M = 1 GEMV for the decode step.
//
// The activation vector is staged once per block (the Src policy decides how:
// plain int16, RMS-normalised on the fly, or reduced from the attention
// accumulator), then every wave walks its own sequence of row groups
//   g = wave_global, wave_global + waves_total, ...
// with no further block-level synchronisation.  A group's weights are read in
// batches of U steps of 1 KiB per row (int8) or 8 weights per lane (int16);
// two register buffers alternate, so the loads of the next batch are in flight
// while the current batch is multiplied.  The sums are exact (see gemv.h for
// the byte-split bounds).
//
// The streaming loop touches global memory only through the weight loads.
// vmcnt is one in-order counter for loads and stores alike, so any other
// global access inside the loop (an epilogue operand, a LUT lookup, a store)
// would make the next wait drain the prefetched batch.  Each finished group
// therefore leaves its R exact sums, reduced to wave-uniform values with DPP,
// in a per-wave LDS record; after the stream every lane applies the epilogue
// to one recorded group, so all epilogue loads and stores of a wave overlap.
//
// Staging interface (Src):
//   Pre; pre(K, kpad, nthr)                      per thread, first thing in the kernel
//   stage_i8(pre, hi, lo, K, kpad, nthr)         whole block, after the first weight loads
// nthr is the block size as a compile-time constant of the kernel: blockDim
// is read from the dispatch packet, a load that would delay the first loads
// and (issued behind the weights) make the staging wait for them.
// pre() issues the source's own loads (activations, scales, norm sums) ahead of
// every weight load: loads complete in issue order, so staging then waits for
// its operands without waiting for a weight batch.
//
// Epilogue interface:
//   State; begin(State&)                        per thread, before the stream
//   prefetch(State&, row0, N)                    per lane, right after the first
//                                                weight batch: the per-row operands
//                                                of the lane's first group (rows
//                                                row0 ..), in registers by the end
//   group(State&, row0, N, const int64_t (&)[R]) per lane, one group each
//   finish(State&)                               whole block, after the stream
//                                                (may synchronise the block)
#pragma once

#include "bufload.h"
#include "gemv.h"

#include <algorithm>
#include <cstdlib>
#include <type_traits>

namespace myl {

// Weight loads are non-temporal (cache-policy bit nt): each weight byte is
// read once per step, and on MI355X the streaming kernels ran 5-12 % faster
// with them (decode step 2.29 -> 2.13 ms, int16 LM head 188 -> 165 us).
constexpr int kWeightCpol = 2;
__device__ inline uint4 bload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kWeightCpol);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}

// The staging operands load through cload16 / cload8 (bufload.h), issued
// ahead of the first weight batch: past num_records a load returns zero, so
// no branch guards it.

// ---- staging sources ----------------------------------------------------------

// 8-element chunks of the staged vector a thread loads in pre(): chunks
// threadIdx.x + j * nthr, j < kPreChunks; the rest load during staging.
constexpr int kPreChunks = 5;

// Each staged plane is followed by kStageSlack spare elements: chunk index
// n8 = kpad / 8 is a dump slot, so the chunks loaded ahead of the weights are
// staged without a branch (a thread past the end writes its zeros there).
// A branch would let the compiler sink those loads behind the weight batch.
constexpr int kStageSlack = 16;
__device__ inline int stage_slot(int i, int n8) { return i < n8 ? i : n8; }

// Eight int16 values -> their signed byte planes (hi = x >> 8, lo' = (x & 255) - 128).
__device__ inline void put_x8_planes(const uint4 v, int8_t* hi, int8_t* lo) {
    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
    uint32_t h[2], l[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t d0 = d[2 * t], d1 = d[2 * t + 1];
        h[t] = ((d0 >> 8) & 0xFFu) | ((d0 >> 16) & 0xFF00u) | ((d1 << 8) & 0xFF0000u) | (d1 & 0xFF000000u);
        l[t] = ((d0 & 0xFFu) | ((d0 >> 8) & 0xFF00u) | ((d1 << 16) & 0xFF0000u) | ((d1 << 8) & 0xFF000000u)) ^ 0x80808080u;
    }
    *reinterpret_cast<uint2*>(hi) = make_uint2(h[0], h[1]);
    *reinterpret_cast<uint2*>(lo) = make_uint2(l[0], l[1]);
}

// Plain int16 activations (K % 8 == 0), converted to the two signed byte planes.
struct SrcPlain {
    const int16_t* x;
    struct Pre {
        uint4 x[kPreChunks];
    };
    __device__ inline Pre pre(int K, int kpad, int nthr) const {
        Pre p;
        const __amdgpu_buffer_rsrc_t r = weight_rsrc(x, 2u * (uint32_t)K);
#pragma unroll
        for (int j = 0; j < kPreChunks; ++j) p.x[j] = cload16(r, (threadIdx.x + j * nthr) * 16u);
        return p;
    }
    __device__ inline void stage_i8(const Pre& p, int8_t* hi, int8_t* lo, int K, int kpad, int nthr) const {
        const int n8 = kpad >> 3;
#pragma unroll
        for (int j = 0; j < kPreChunks; ++j) {
            const int i = stage_slot(threadIdx.x + j * nthr, n8);
            put_x8_planes(p.x[j], hi + i * 8, lo + i * 8);
        }
        for (int i = threadIdx.x + kPreChunks * nthr; i < n8; i += nthr) {
            const uint4 v = i * 8 < K ? *reinterpret_cast<const uint4*>(x + i * 8) : make_uint4(0, 0, 0, 0);
            put_x8_planes(v, hi + i * 8, lo + i * 8);
        }
    }
};

// LDS bytes of a stream launch: the two activation planes plus the records.
__host__ __device__ inline size_t stream_lds_bytes(int K, int elem, int waves, int gpw, int R) {
    const size_t step = elem == 1 ? 16 : 8;
    const size_t kpad = (((size_t)K + step - 1) / step) * step;
    return 2 * (kpad + kStageSlack) * (size_t)elem + (size_t)waves * gpw * R * 8;
}

template <int R, class Epi>
__device__ inline void stream_epilogue(const int64_t* rec, int g0, int nw, int cnt, int N, int lane, Epi& epi,
                                       typename Epi::State& es) {
    for (int k = lane; k < cnt; k += kWave) {
        int64_t tot[R];
#pragma unroll
        for (int r = 0; r < R; ++r) tot[r] = rec[k * R + r];
        epi.group(es, (g0 + k * nw) * R, N, tot);
    }
}

// gpw: the most groups any wave of the grid handles, ceil(ceil(N/R) / waves);
// the launcher sizes the records from it.
// PF2: both register buffers are loaded before the activations are staged, so
// two batches stream while a slow staging source (RMSNorm) runs.
template <int R, int U, int WAVES, class Src, class Epi, bool PF2 = false>
__global__ __launch_bounds__(WAVES * 64) void gemv_i8_stream(Src src, const int8_t* __restrict__ W, int N, int K,
                                                            int gpw, Epi epi) {
    extern __shared__ __align__(16) int8_t lds[];
    const int kpad = ((K + 15) >> 4) << 4;
    int8_t* hi_plane = lds;
    int8_t* lo_plane = lds + kpad + kStageSlack;
    const int lane = threadIdx.x & (kWave - 1);
    // wave-uniform by construction; readfirstlane lets the compiler keep the
    // loop control in scalar registers (a vector loop would end every
    // iteration with a full vmcnt drain)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    int64_t* rec = reinterpret_cast<int64_t*>(lds + 2 * (kpad + kStageSlack)) + (size_t)wave * gpw * R;
    const int nw = gridDim.x * WAVES;
    const int ngroups = (N + R - 1) / R;
    const int nit = (K + kWave * 16 - 1) / (kWave * 16);  // 1 KiB steps per row
    const int nb = (nit + U - 1) / U;                      // batches per group
    constexpr int kThreads = WAVES * kWave;
    const typename Src::Pre pre = src.pre(K, kpad, kThreads);
    typename Epi::State es;
    epi.begin(es);
    // the staging loads above go out before the first weight batch below
    // (the scheduler would otherwise interleave them, and loads complete in
    // issue order)
    __builtin_amdgcn_sched_barrier(0);

    const uint32_t wbytes = (uint32_t)N * (uint32_t)K;  // < 2^32 (checked by the launcher)
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(W, wbytes);
    auto load = [&](uint4 (&buf)[U][R], int g, int kb) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = (kb * U + u) * (kWave * 16) + lane * 16;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = g * R + r;
                const bool ok = k < K && row < N;
                buf[u][r] = bload16(wr, ok ? (uint32_t)row * (uint32_t)K + (uint32_t)k : wbytes);
            }
        }
    };
    int32_t ahi[R], alo[R], aws[R];
    auto reset = [&]() {
#pragma unroll
        for (int r = 0; r < R; ++r) { ahi[r] = 0; alo[r] = 0; aws[r] = 0; }
    };
    // Out-of-range slots hold zero weights, so they may read any staged
    // column: the LDS offset is clamped into the planes.
    auto compute = [&](const uint4 (&buf)[U][R], int kb) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min((kb * U + u) * (kWave * 16) + lane * 16, kpad - 16);
            const uint4 h = *reinterpret_cast<const uint4*>(hi_plane + k);
            const uint4 l = *reinterpret_cast<const uint4*>(lo_plane + k);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                ahi[r] = sdot4(buf[u][r].x, h.x, ahi[r]);
                ahi[r] = sdot4(buf[u][r].y, h.y, ahi[r]);
                ahi[r] = sdot4(buf[u][r].z, h.z, ahi[r]);
                ahi[r] = sdot4(buf[u][r].w, h.w, ahi[r]);
                alo[r] = sdot4(buf[u][r].x, l.x, alo[r]);
                alo[r] = sdot4(buf[u][r].y, l.y, alo[r]);
                alo[r] = sdot4(buf[u][r].z, l.z, alo[r]);
                alo[r] = sdot4(buf[u][r].w, l.w, alo[r]);
                aws[r] = sdot4(buf[u][r].x, 0x01010101u, aws[r]);
                aws[r] = sdot4(buf[u][r].y, 0x01010101u, aws[r]);
                aws[r] = sdot4(buf[u][r].z, 0x01010101u, aws[r]);
                aws[r] = sdot4(buf[u][r].w, 0x01010101u, aws[r]);
            }
        }
    };
    // The three partial sums are exact in i32 over the whole row (K < 131072),
    // so each is reduced in i32 and widened once.
    int cnt = 0;
    auto finish_group = [&]() {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t t = (int64_t)wave_sum_i32(ahi[r]) * 256 + (int64_t)wave_sum_i32(alo[r]) +
                              (int64_t)wave_sum_i32(aws[r]) * 128;
            if (lane == 0) rec[cnt * R + r] = t;
        }
        ++cnt;
        reset();
    };

    // Batch sequence of this wave: (g, kb) for g = g0, g0 + nw, ... and
    // kb = 0 .. nb-1, taken two at a time; the loads of the batch after next
    // are issued unconditionally (past the end they fall outside the buffer
    // and return zeros), so the only branch inside the loop is uniform.
    uint4 A[U][R], B[U][R];
    const int g0 = blockIdx.x * WAVES + wave;
    int g = g0, kb = 0;
    auto advance = [&](int& gg, int& kk) {
        if (++kk == nb) { kk = 0; gg += nw; }
    };
    if (PF2) {
        // A and B both in flight during staging; each round consumes A then
        // B and reloads both two batches ahead.
        int g1 = g, kb1 = kb;
        advance(g1, kb1);
        load(A, g, 0);
        epi.prefetch(es, (g0 + lane * nw) * R, N);
        load(B, g1, kb1);
        src.stage_i8(pre, hi_plane, lo_plane, K, kpad, kThreads);
        __syncthreads();
        reset();
        while (g < ngroups) {
            compute(A, kb);
            if (kb == nb - 1) finish_group();
            int g2 = g1, kb2 = kb1;
            advance(g2, kb2);
            load(A, g2, kb2);
            if (g1 < ngroups) {
                compute(B, kb1);
                if (kb1 == nb - 1) finish_group();
            }
            int g3 = g2, kb3 = kb2;
            advance(g3, kb3);
            load(B, g3, kb3);
            g = g2;
            kb = kb2;
            g1 = g3;
            kb1 = kb3;
        }
    } else {
        load(A, g, 0);
        epi.prefetch(es, (g0 + lane * nw) * R, N);
        src.stage_i8(pre, hi_plane, lo_plane, K, kpad, kThreads);
        __syncthreads();
        reset();
        while (g < ngroups) {
            int g1 = g, kb1 = kb;
            advance(g1, kb1);
            load(B, g1, kb1);
            compute(A, kb);
            if (kb == nb - 1) finish_group();
            int g2 = g1, kb2 = kb1;
            advance(g2, kb2);
            load(A, g2, kb2);
            if (g1 < ngroups) {
                compute(B, kb1);
                if (kb1 == nb - 1) finish_group();
            }
            g = g2;
            kb = kb2;
        }
    }
    stream_epilogue<R>(rec, g0, nw, cnt, N, lane, epi, es);
    epi.finish(es);
}

// int16 weights (LM head path A): planes of int16 hi = x >> 8 and lo = x & 255.
template <int R, int U, int WAVES, class Src16, class Epi>
__global__ __launch_bounds__(WAVES * 64) void gemv_i16_stream(Src16 src, const int16_t* __restrict__ W, int N,
                                                             int K, int gpw, Epi epi) {
    extern __shared__ __align__(16) int8_t lds_raw[];
    const int kpad = ((K + 7) >> 3) << 3;
    int16_t* hi_plane = reinterpret_cast<int16_t*>(lds_raw);
    int16_t* lo_plane = hi_plane + kpad + kStageSlack;
    const int lane = threadIdx.x & (kWave - 1);
    // wave-uniform by construction; readfirstlane lets the compiler keep the
    // loop control in scalar registers (a vector loop would end every
    // iteration with a full vmcnt drain)
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    int64_t* rec = reinterpret_cast<int64_t*>(lds_raw + 4 * (kpad + kStageSlack)) + (size_t)wave * gpw * R;
    const int nw = gridDim.x * WAVES;
    const int ngroups = (N + R - 1) / R;
    const int nit = (K + kWave * 8 - 1) / (kWave * 8);
    const int nb = (nit + U - 1) / U;
    typedef short __attribute__((ext_vector_type(2))) s2;
    constexpr int kThreads = WAVES * kWave;
    const typename Src16::Pre pre = src.pre(K, kpad, kThreads);
    typename Epi::State es;
    epi.begin(es);
    __builtin_amdgcn_sched_barrier(0);  // staging loads before the first weight batch

    const uint32_t wbytes = 2u * (uint32_t)N * (uint32_t)K;  // < 2^32 (checked by the launcher)
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(W, wbytes);
    auto load = [&](uint4 (&buf)[U][R], int g, int kb) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = (kb * U + u) * (kWave * 8) + lane * 8;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int row = g * R + r;
                const bool ok = k < K && row < N;
                buf[u][r] = bload16(wr, ok ? 2u * ((uint32_t)row * (uint32_t)K + (uint32_t)k) : wbytes);
            }
        }
    };
    int32_t ahi[R], alo[R];
    auto reset = [&]() {
#pragma unroll
        for (int r = 0; r < R; ++r) { ahi[r] = 0; alo[r] = 0; }
    };
    auto d2 = [](uint32_t a, uint32_t b, int32_t c) {
        return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, b), c, false);
    };
    auto compute = [&](const uint4 (&buf)[U][R], int kb) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = min((kb * U + u) * (kWave * 8) + lane * 8, kpad - 8);
            const uint4 h = *reinterpret_cast<const uint4*>(hi_plane + k);
            const uint4 l = *reinterpret_cast<const uint4*>(lo_plane + k);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                ahi[r] = d2(buf[u][r].x, h.x, ahi[r]);
                ahi[r] = d2(buf[u][r].y, h.y, ahi[r]);
                ahi[r] = d2(buf[u][r].z, h.z, ahi[r]);
                ahi[r] = d2(buf[u][r].w, h.w, ahi[r]);
                alo[r] = d2(buf[u][r].x, l.x, alo[r]);
                alo[r] = d2(buf[u][r].y, l.y, alo[r]);
                alo[r] = d2(buf[u][r].z, l.z, alo[r]);
                alo[r] = d2(buf[u][r].w, l.w, alo[r]);
            }
        }
    };
    // Per lane the partials are below 2^31 (K <= 8192); across the wave they
    // need 64 bits.
    int cnt = 0;
    auto finish_group = [&]() {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t t = wave_sum_i64((int64_t)ahi[r] * 256 + (int64_t)alo[r]);
            if (lane == 0) rec[cnt * R + r] = t;
        }
        ++cnt;
        reset();
    };

    // Batch sequence of this wave: (g, kb) for g = g0, g0 + nw, ... and
    // kb = 0 .. nb-1, taken two at a time; the loads of the batch after next
    // are issued unconditionally (past the end they fall outside the buffer
    // and return zeros), so the only branch inside the loop is uniform.
    uint4 A[U][R], B[U][R];
    const int g0 = blockIdx.x * WAVES + wave;
    int g = g0, kb = 0;
    auto advance = [&](int& gg, int& kk) {
        if (++kk == nb) { kk = 0; gg += nw; }
    };
    load(A, g, 0);
    epi.prefetch(es, (g0 + lane * nw) * R, N);
    src.stage_i16(pre, hi_plane, lo_plane, K, kpad, kThreads);
    __syncthreads();
    reset();
    while (g < ngroups) {
        int g1 = g, kb1 = kb;
        advance(g1, kb1);
        load(B, g1, kb1);
        compute(A, kb);
        if (kb == nb - 1) finish_group();
        int g2 = g1, kb2 = kb1;
        advance(g2, kb2);
        load(A, g2, kb2);
        if (g1 < ngroups) {
            compute(B, kb1);
            if (kb1 == nb - 1) finish_group();
        }
        g = g2;
        kb = kb2;
    }
    stream_epilogue<R>(rec, g0, nw, cnt, N, lane, epi, es);
    epi.finish(es);
}

// Short rows (K a multiple of 128, K <= 2048: the 0.5B-shape LM head at K =
// 896): a wave load of 1 KiB covers eight rows, 128 bytes each, so every lane
// carries 16 bytes, and the eight rows reduce together with three DPP steps
// over their 8-lane groups, instead of one whole-wave reduction per row
// (which dominated at one 1 KiB step per row).  A group is 8 rows (lane l:
// row 8 g + l / 8, bytes 16 (l % 8) of each 128-byte step), all K / 128 steps
// of the group in one batch; two batches alternate.  Records hold the rows'
// exact sums; the epilogue runs on row pairs (Epi::group<2>).
template <int STEPS, int WAVES, class Src, class Epi>
__global__ __launch_bounds__(WAVES * 64) void gemv_i8_stream8(Src src, const int8_t* __restrict__ W, int N, int K,
                                                              int gpw, Epi epi) {
    extern __shared__ __align__(16) int8_t lds[];
    constexpr int kRows = 8;  // rows per group
    const int kpad = ((K + 15) >> 4) << 4;
    int8_t* hi_plane = lds;
    int8_t* lo_plane = lds + kpad + kStageSlack;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    int64_t* rec = reinterpret_cast<int64_t*>(lds + 2 * (kpad + kStageSlack)) + (size_t)wave * gpw * kRows;
    const int nw = gridDim.x * WAVES;
    const int ngroups = (N + kRows - 1) / kRows;
    constexpr int kThreads = WAVES * kWave;
    const typename Src::Pre pre = src.pre(K, kpad, kThreads);
    typename Epi::State es;
    epi.begin(es);
    __builtin_amdgcn_sched_barrier(0);  // staging loads before the first weight batch

    const uint32_t wbytes = (uint32_t)N * (uint32_t)K;  // < 2^32 (checked by the launcher)
    const __amdgpu_buffer_rsrc_t wr = weight_rsrc(W, wbytes);
    const int sub = lane & 7, rin = lane >> 3;
    auto load = [&](uint4 (&buf)[STEPS], int g) {
        const int row = g * kRows + rin;
        const uint32_t base = (uint32_t)row * (uint32_t)K + (uint32_t)sub * 16u;
#pragma unroll
        for (int u = 0; u < STEPS; ++u) buf[u] = bload16(wr, row < N ? base + (uint32_t)u * 128u : wbytes);
    };
    int cnt = 0;
    auto group = [&](const uint4 (&buf)[STEPS]) {
        int32_t ahi = 0, alo = 0, aws = 0;
#pragma unroll
        for (int u = 0; u < STEPS; ++u) {
            const int k = u * 128 + sub * 16;
            const uint4 h = *reinterpret_cast<const uint4*>(hi_plane + k);
            const uint4 l = *reinterpret_cast<const uint4*>(lo_plane + k);
            ahi = sdot4(buf[u].x, h.x, ahi);
            ahi = sdot4(buf[u].y, h.y, ahi);
            ahi = sdot4(buf[u].z, h.z, ahi);
            ahi = sdot4(buf[u].w, h.w, ahi);
            alo = sdot4(buf[u].x, l.x, alo);
            alo = sdot4(buf[u].y, l.y, alo);
            alo = sdot4(buf[u].z, l.z, alo);
            alo = sdot4(buf[u].w, l.w, alo);
            aws = sdot4(buf[u].x, 0x01010101u, aws);
            aws = sdot4(buf[u].y, 0x01010101u, aws);
            aws = sdot4(buf[u].z, 0x01010101u, aws);
            aws = sdot4(buf[u].w, 0x01010101u, aws);
        }
        // each partial is exact in i32 over the row (K <= 2048); the row's 8
        // lanes reduce together, every lane of the group gets the totals
        ahi = row_sum8_i32(ahi);
        alo = row_sum8_i32(alo);
        aws = row_sum8_i32(aws);
        if (sub == 0) rec[cnt * kRows + rin] = (int64_t)ahi * 256 + (int64_t)alo + (int64_t)aws * 128;
        ++cnt;
    };
    uint4 A[STEPS], B[STEPS];
    const int g0 = blockIdx.x * WAVES + wave;
    load(A, g0);
    // the lane's first row pair (pairs q = lane: group q / 4, rows 2 (q % 4) ..)
    epi.prefetch(es, (g0 + (lane >> 2) * nw) * kRows + 2 * (lane & 3), N);
    src.stage_i8(pre, hi_plane, lo_plane, K, kpad, kThreads);
    __syncthreads();
    for (int g = g0; g < ngroups; g += 2 * nw) {
        load(B, g + nw);  // past the end: zeros
        group(A);
        load(A, g + 2 * nw);
        if (g + nw < ngroups) group(B);
    }
    // row pairs: pair q of the wave's records is rows 2 (q % 4), + 1 of group q / 4
    for (int q = lane; q < cnt * (kRows / 2); q += kWave) {
        const int j = q >> 2, p = q & 3;
        const int64_t tot[2] = {rec[j * kRows + 2 * p], rec[j * kRows + 2 * p + 1]};
        epi.group(es, (g0 + j * nw) * kRows + 2 * p, N, tot);
    }
    epi.finish(es);
}

// ---- launchers ------------------------------------------------------------------

// Blocks of a kernel that fit on one CU at `lds` bytes of dynamic LDS.  The
// answer is cached per kernel (the last LDS size asked), so a launch of a few
// microseconds does not wait for the runtime query.
template <class Kern>
int stream_occupancy(Kern kern, int threads, size_t lds) {
    static thread_local Kern last_kern = nullptr;
    static thread_local size_t last_lds = ~(size_t)0;
    static thread_local int last_occ = 1;
    if (kern != last_kern || lds != last_lds) {
        int occ = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kern, threads, lds) != hipSuccess || occ < 1) occ = 1;
        last_kern = kern;
        last_lds = lds;
        last_occ = occ;
    }
    return last_occ;
}

// Persistent grid: as many blocks as fit on the device (at most occ_cap per
// CU when occ_cap > 0), shrunk so that every wave gets the same number of row
// groups (no tail of half-filled rounds).  Returns the grid and, in gpw, the
// most groups one wave handles.
template <class Kern>
int stream_grid(Kern kern, int waves_per_block, size_t lds, int ngroups, int cus, int* gpw, int occ_cap = 0) {
    int occ = stream_occupancy(kern, waves_per_block * 64, lds);
    if (occ_cap > 0) occ = std::min(occ, occ_cap);
    const int waves_cap = occ * cus * waves_per_block;
    const int per_wave = (ngroups + waves_cap - 1) / waves_cap;
    const int waves = (ngroups + per_wave - 1) / per_wave;
    const int grid = (waves + waves_per_block - 1) / waves_per_block;
    const int nw = grid * waves_per_block;
    *gpw = (ngroups + nw - 1) / nw;
    return grid;
}

// Records are sized for up to kGpwReserve groups per wave when the occupancy
// is computed; larger counts still run correctly (the LDS grows to fit).
constexpr int kGpwReserve = 16;
constexpr size_t kStreamLdsMax = 64 * 1024;

// occ_cap: at most this many blocks per CU (0: as many as fit).  Fewer waves
// in flight streamed matrices of about 70 MB faster on MI355X (the N = 18944
// x K = 3584 product at one block per CU: 16.9 -> 14.6 us).
template <int R, int U, int WAVES, bool PF2 = false, class Src, class Epi>
hipError_t stream_i8(const Src& src, const int8_t* W, int N, int K, const Epi& e, hipStream_t s, int cus,
                     int occ_cap = 0) {
    // one buffer descriptor; i32 partial sums exact for K < 131072
    if ((uint64_t)N * (uint64_t)K > 0xFFFFFF00ull || K >= 131072 || N < 1 || K < 1) return hipErrorInvalidValue;
    auto kern = gemv_i8_stream<R, U, WAVES, Src, Epi, PF2>;
    int gpw = 0;
    const int grid = stream_grid(kern, WAVES, stream_lds_bytes(K, 1, WAVES, kGpwReserve, R), (N + R - 1) / R, cus, &gpw,
                                 occ_cap);
    const size_t lds = stream_lds_bytes(K, 1, WAVES, gpw, R);
    if (lds > kStreamLdsMax) return hipErrorInvalidValue;
    kern<<<grid, WAVES * 64, lds, s>>>(src, W, N, K, gpw, e);
    return hipGetLastError();
}

// The 8-row short-row stream (gemv_i8_stream8) for K = 128 STEPS.
template <int STEPS, int WAVES, class Src, class Epi>
hipError_t stream_i8_rows8(const Src& src, const int8_t* W, int N, int K, const Epi& e, hipStream_t s, int cus,
                           int occ_cap = 0) {
    if ((uint64_t)N * (uint64_t)K > 0xFFFFFF00ull || K != 128 * STEPS || N < 1) return hipErrorInvalidValue;
    auto kern = gemv_i8_stream8<STEPS, WAVES, Src, Epi>;
    int gpw = 0;
    const int grid = stream_grid(kern, WAVES, stream_lds_bytes(K, 1, WAVES, kGpwReserve, 8), (N + 7) / 8, cus, &gpw,
                                 occ_cap);
    const size_t lds = stream_lds_bytes(K, 1, WAVES, gpw, 8);
    if (lds > kStreamLdsMax) return hipErrorInvalidValue;
    kern<<<grid, WAVES * 64, lds, s>>>(src, W, N, K, gpw, e);
    return hipGetLastError();
}

template <int R, int U, int WAVES, class Src, class Epi>
hipError_t stream_i16(const Src& src, const int16_t* W, int N, int K, const Epi& e, hipStream_t s, int cus) {
    // one buffer descriptor; per-lane i32 partials exact for K <= 8192
    if (2ull * (uint64_t)N * (uint64_t)K > 0xFFFFFF00ull || K > 8192 || N < 1 || K < 1) return hipErrorInvalidValue;
    auto kern = gemv_i16_stream<R, U, WAVES, Src, Epi>;
    int gpw = 0;
    const int grid = stream_grid(kern, WAVES, stream_lds_bytes(K, 2, WAVES, kGpwReserve, R), (N + R - 1) / R, cus, &gpw);
    const size_t lds = stream_lds_bytes(K, 2, WAVES, gpw, R);
    if (lds > kStreamLdsMax) return hipErrorInvalidValue;
    kern<<<grid, WAVES * 64, lds, s>>>(src, W, N, K, gpw, e);
    return hipGetLastError();
}

// ---- row-wise epilogues in the streaming interface ------------------------------

struct NoState {};

// Drives an epilogue of the row-wise form one(n, m, acc) (gemv.h, rows_epi.h)
// for one activation row.
template <class Epi>
struct StreamOne {
    Epi e;
    using State = NoState;
    __device__ inline void begin(State&) const {}
    __device__ inline void prefetch(State&, int, int) const {}
    __device__ inline void finish(State&) const {}
    template <int R>
    __device__ inline void group(State&, int row0, int N, const int64_t (&tot)[R]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < N) e.one(row0 + r, 0, tot[r]);
    }
};

// The same for epilogues whose per-row operands are tables (Epi::Ops,
// ops(n), one_ops): the lane's first group's operands load right after the
// first weight batch, so they are in registers when the stream ends.
template <class Epi>
struct StreamOneOps {
    Epi e;
    struct State {
        typename Epi::Ops o[2];
        int row0;
    };
    __device__ inline void begin(State& s) const { s.row0 = -1; }
    __device__ inline void prefetch(State& s, int row0, int N) const {
        s.o[0] = e.ops(min(row0, N - 1));
        s.o[1] = e.ops(min(row0 + 1, N - 1));
        s.row0 = row0;
    }
    __device__ inline void finish(State&) const {}
    template <int R>
    __device__ inline void group(State& s, int row0, int N, const int64_t (&tot)[R]) const {
        static_assert(R <= 2, "two prefetched rows per group");
        const bool pre = s.row0 == row0;
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (row0 + r < N) e.one_ops(row0 + r, 0, tot[r], pre ? s.o[r] : e.ops(row0 + r));
    }
};

template <class Epi, class = void>
struct StreamEpiOf {
    using type = StreamOne<Epi>;
};
template <class Epi>
struct StreamEpiOf<Epi, std::void_t<typename Epi::Ops>> {
    using type = StreamOneOps<Epi>;
};

// Whether stream_i8<R, U, WAVES> takes N rows of K int8 weights: one buffer
// descriptor, exact i32 partials, and the LDS of the widest grid stream_grid
// can choose (at least one block per CU, so at most
// ceil(ceil(N / R) / (cus * WAVES)) groups per wave).
template <int R, int WAVES>
inline bool stream_fits(int N, int K, int cus) {
    if (N < 1 || K < 1 || K % 16 != 0 || K >= 131072 || (uint64_t)N * (uint64_t)K > 0xFFFFFF00ull || cus < 1)
        return false;
    const int ngroups = (N + R - 1) / R;
    const int gpw = (ngroups + cus * WAVES - 1) / (cus * WAVES);
    return stream_lds_bytes(K, 1, WAVES, gpw, R) <= kStreamLdsMax;
}

// Launch shape of one activation row through the streaming kernel, the
// decode step's shape for a product of the same kind: many rows (gate/up,
// LM head) two rows per wave and 8-wave blocks; a long K (down) one row per
// wave; short K and few rows (o_proj) 16-wave blocks.  0: the stream does
// not take the shape.
inline int stream_rows_shape(int N, int K, int cus) {
    if (N >= 8192) return stream_fits<2, 8>(N, K, cus) ? 1 : 0;
    if (K >= 8192) return stream_fits<1, 8>(N, K, cus) ? 2 : 0;
    return stream_fits<1, 16>(N, K, cus) ? 3 : 0;
}

// One activation row x (16-byte aligned) of a W8A16 product with a row-wise
// epilogue, in the shape stream_rows_shape chose (nonzero).
template <class Epi>
hipError_t stream_rows_i8(int shape, const int16_t* x, const int8_t* W, int N, int K, const Epi& epi, hipStream_t st,
                          int cus) {
    const SrcPlain src{x};
    const typename StreamEpiOf<Epi>::type e{epi};
    // one block per CU for 32-100 MB of weights (measured faster for the
    // 68 MB shapes), as many as fit otherwise (12.8 MB: 5.5 against 6.0 us;
    // the 545 MB LM-head shape).  Many rows at 32-100 MB: one row per wave
    // group (18944 x 3584 on MI355X: 12.9 us against 14.3-14.7 us with two;
    // the 545 MB shape is the same either way)
    const uint64_t wb = (uint64_t)N * (uint64_t)K;
    const int occ = wb >= (32ull << 20) && wb <= (100ull << 20) ? 1 : 0;
    switch (shape) {
        case 1:
            return occ ? stream_i8<1, 4, 8>(src, W, N, K, e, st, cus, occ)
                       : stream_i8<2, 4, 8>(src, W, N, K, e, st, cus, occ);
        case 2: return stream_i8<1, 4, 8>(src, W, N, K, e, st, cus, occ);
        case 3: return stream_i8<1, 2, 16>(src, W, N, K, e, st, cus, occ);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace myl
