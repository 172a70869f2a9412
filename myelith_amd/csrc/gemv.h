// gemv.h -- W8A16 / W16A16 matrix-vector kernels with pluggable epilogues.
//
// y[m][r] = epilogue(r, m, sum_k W[r][k] * x[m][k])   (exact i64 sums)
//
// The sum is the reference dot product (INTEGER_LLM/kernels/src/dot.rs:141-147),
// computed in a different order; exact integer addition makes every order
// equal (dot.rs:19-36).
//
// int8 weights: the int16 activation is split x = 256*hi + lo' + 128 with
// hi = x >> 8 (signed byte) and lo' = (x & 255) - 128 (signed byte), so
//   sum w*x = 256*sum(w*hi) + sum(w*lo') + 128*sum(w)
// and each of the three sums is a chain of v_dot4_i32_i8 (4 int8 MACs per
// instruction).  Per lane and in total each partial is bounded by
// 128*128*K < 2^31 for K < 131072, so the i32 partials are exact and are
// widened to i64 only once, after the cross-lane reduction.
//
// int16 weights (LM head, model.rs:285-296): x = 256*hi + lo with lo in
// [0, 255]; v_dot2_i32_i16 on (w, hi) and (w, lo).  Per lane the partials stay
// below 2^31 for K <= 8192.
//
// Layout: W row-major [N][K] with K % 16 == 0 and 16-byte aligned rows.  A
// wave owns R consecutive rows; its 64 lanes read 64 x 16 B = 1 KiB of one row
// per step (fully coalesced dwordx4 loads).  x is staged once per block into
// LDS as the two byte planes.
#pragma once

#include "fixed.h"
#include "wave.h"

namespace myl {

constexpr int kWave = 64;
constexpr int kGemvThreads = 256;
constexpr int kGemvWaves = kGemvThreads / kWave;
constexpr int kGemvLdsBytes = 64 * 1024;

__device__ inline int32_t sdot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// Stage x[m][k0 .. k0+len) of M rows into two signed byte planes (len is a
// multiple of 16, zero-padded past K: hi = 0, lo' = -128 with w = 0 there).
// With xvec, each thread converts 8 activations from one 16-byte load: the
// high bytes of the int16 lanes form the hi plane, the low bytes XOR 0x80
// (i.e. lo - 128) form the lo' plane.
__device__ inline void stage_x_planes(const int16_t* __restrict__ x, int M, int ldx, int K, int k0,
                                      int len, int8_t* hi, int8_t* lo, bool xvec) {
    if (xvec) {
        const int n8 = len >> 3;
        for (int m = 0; m < M; ++m) {
            for (int i = threadIdx.x; i < n8; i += blockDim.x) {
                const int kk = k0 + i * 8;
                uint4 v = make_uint4(0, 0, 0, 0);
                if (kk < K) v = *reinterpret_cast<const uint4*>(x + (size_t)m * ldx + kk);
                const uint32_t d[4] = {v.x, v.y, v.z, v.w};
                uint32_t h[2], l[2];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    const uint32_t d0 = d[2 * t], d1 = d[2 * t + 1];
                    h[t] = ((d0 >> 8) & 0xFFu) | ((d0 >> 16) & 0xFF00u) | ((d1 << 8) & 0xFF0000u) | (d1 & 0xFF000000u);
                    l[t] = ((d0 & 0xFFu) | ((d0 >> 8) & 0xFF00u) | ((d1 << 16) & 0xFF0000u) | ((d1 << 8) & 0xFF000000u))
                           ^ 0x80808080u;
                }
                *reinterpret_cast<uint2*>(hi + m * len + i * 8) = make_uint2(h[0], h[1]);
                *reinterpret_cast<uint2*>(lo + m * len + i * 8) = make_uint2(l[0], l[1]);
            }
        }
        return;
    }
    for (int m = 0; m < M; ++m) {
        for (int k = threadIdx.x; k < len; k += blockDim.x) {
            const int kk = k0 + k;
            const int16_t v = kk < K ? x[(size_t)m * ldx + kk] : (int16_t)0;
            hi[m * len + k] = (int8_t)(v >> 8);
            lo[m * len + k] = (int8_t)((int)(v & 255) - 128);
        }
    }
}

// Core of the int8 kernel: the exact row sums of R rows x MT activation rows
// for one wave, left in every lane of the wave.  The wave walks its rows in
// batches of U steps of 1 KiB per row: all U*R weight loads of a batch are
// issued before any of them is consumed, and the first batch is issued before
// the activations are staged, so the staging overlaps the weight stream.
template <int R, int MT, int U>
__device__ inline void gemv_i8_rows(const int16_t* __restrict__ x, int M, int ldx,
                                    const int8_t* __restrict__ W, int N, int K, int row0,
                                    int8_t* hi_plane, int8_t* lo_plane, int kc, bool xvec,
                                    int64_t (&tot)[R][MT]) {
    const int lane = threadIdx.x & (kWave - 1);
    int32_t ahi[R][MT], alo[R][MT], aws[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        aws[r] = 0;
#pragma unroll
        for (int m = 0; m < MT; ++m) { ahi[r][m] = 0; alo[r][m] = 0; }
    }
    const int8_t* wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) wrow[r] = W + (size_t)min(row0 + r, N - 1) * K;
    bool rok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) rok[r] = row0 + r < N;

    for (int k0 = 0; k0 < K; k0 += kc) {
        const int len = min(kc, K - k0);
        uint4 w[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = u * (kWave * 16) + lane * 16;
#pragma unroll
            for (int r = 0; r < R; ++r)
                w[u][r] = (k < len && rok[r]) ? *reinterpret_cast<const uint4*>(wrow[r] + k0 + k) : make_uint4(0, 0, 0, 0);
        }
        __syncthreads();
        stage_x_planes(x, M, ldx, K, k0, len, hi_plane, lo_plane, xvec);
        __syncthreads();
        for (int kb = 0; kb < len; kb += U * kWave * 16) {
            if (kb > 0) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int k = kb + u * (kWave * 16) + lane * 16;
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        w[u][r] = (k < len && rok[r]) ? *reinterpret_cast<const uint4*>(wrow[r] + k0 + k)
                                                      : make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = kb + u * (kWave * 16) + lane * 16;
                if (k < len) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m < M) {
                            const uint4 h = *reinterpret_cast<const uint4*>(hi_plane + m * len + k);
                            const uint4 l = *reinterpret_cast<const uint4*>(lo_plane + m * len + k);
#pragma unroll
                            for (int r = 0; r < R; ++r) {
                                ahi[r][m] = sdot4(w[u][r].x, h.x, ahi[r][m]);
                                ahi[r][m] = sdot4(w[u][r].y, h.y, ahi[r][m]);
                                ahi[r][m] = sdot4(w[u][r].z, h.z, ahi[r][m]);
                                ahi[r][m] = sdot4(w[u][r].w, h.w, ahi[r][m]);
                                alo[r][m] = sdot4(w[u][r].x, l.x, alo[r][m]);
                                alo[r][m] = sdot4(w[u][r].y, l.y, alo[r][m]);
                                alo[r][m] = sdot4(w[u][r].z, l.z, alo[r][m]);
                                alo[r][m] = sdot4(w[u][r].w, l.w, alo[r][m]);
                            }
                        }
                    }
#pragma unroll
                    for (int r = 0; r < R; ++r) {
                        aws[r] = sdot4(w[u][r].x, 0x01010101u, aws[r]);
                        aws[r] = sdot4(w[u][r].y, 0x01010101u, aws[r]);
                        aws[r] = sdot4(w[u][r].z, 0x01010101u, aws[r]);
                        aws[r] = sdot4(w[u][r].w, 0x01010101u, aws[r]);
                    }
                }
            }
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            int64_t v = (int64_t)ahi[r][m] * 256 + (int64_t)alo[r][m] + (int64_t)aws[r] * 128;
            tot[r][m] = wave_sum_i64(v);
        }
    }
}

// One block = 4 waves x R rows.  The epilogue sees all R x MT sums of its wave.
template <int R, int MT, int U, class Epi>
__global__ __launch_bounds__(kGemvThreads) void gemv_i8_kernel(const int16_t* __restrict__ x, int M, int ldx,
                                                              const int8_t* __restrict__ W, int N, int K,
                                                              int kc, int xvec, Epi epi) {
    extern __shared__ __align__(16) int8_t lds[];
    const int wave = threadIdx.x / kWave;
    const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
    int64_t tot[R][MT];
    gemv_i8_rows<R, MT, U>(x, M, ldx, W, N, K, row0, lds, lds + MT * kc, kc, xvec != 0, tot);
    epi.apply(row0, N, M, threadIdx.x & (kWave - 1), tot);
}

// int16-weight kernel (LM head path A).  Planes are int16: hi = x >> 8,
// lo = x & 255; each lane reads 8 weights (16 B) per step.
template <int R, int MT, int U, class Epi>
__global__ __launch_bounds__(kGemvThreads) void gemv_i16_kernel(const int16_t* __restrict__ x, int M, int ldx,
                                                               const int16_t* __restrict__ W, int N, int K,
                                                               int kc, int xvec, Epi epi) {
    extern __shared__ __align__(16) int8_t lds_raw[];
    int16_t* hi_plane = reinterpret_cast<int16_t*>(lds_raw);
    int16_t* lo_plane = hi_plane + MT * kc;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int row0 = (blockIdx.x * kGemvWaves + wave) * R;
    typedef short __attribute__((ext_vector_type(2))) s2;
    int32_t ahi[R][MT], alo[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m) { ahi[r][m] = 0; alo[r][m] = 0; }
    const int16_t* wrow[R];
    bool rok[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        wrow[r] = W + (size_t)min(row0 + r, N - 1) * K;
        rok[r] = row0 + r < N;
    }
    for (int k0 = 0; k0 < K; k0 += kc) {
        const int len = min(kc, K - k0);
        uint4 w[U][R];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = u * (kWave * 8) + lane * 8;
#pragma unroll
            for (int r = 0; r < R; ++r)
                w[u][r] = (k < len && rok[r]) ? *reinterpret_cast<const uint4*>(wrow[r] + k0 + k) : make_uint4(0, 0, 0, 0);
        }
        __syncthreads();
        if (xvec) {
            const int n8 = len >> 3;
            for (int m = 0; m < M; ++m) {
                for (int i = threadIdx.x; i < n8; i += blockDim.x) {
                    const int kk = k0 + i * 8;
                    uint4 v = make_uint4(0, 0, 0, 0);
                    if (kk < K) v = *reinterpret_cast<const uint4*>(x + (size_t)m * ldx + kk);
                    const uint32_t d[4] = {v.x, v.y, v.z, v.w};
                    uint32_t h[4], l[4];
#pragma unroll
                    for (int t = 0; t < 4; ++t) {
                        h[t] = (((uint32_t)((int32_t)(d[t] << 16) >> 24)) & 0xFFFFu) | ((uint32_t)((int32_t)d[t] >> 24) << 16);
                        l[t] = d[t] & 0x00FF00FFu;
                    }
                    *reinterpret_cast<uint4*>(hi_plane + m * len + i * 8) = make_uint4(h[0], h[1], h[2], h[3]);
                    *reinterpret_cast<uint4*>(lo_plane + m * len + i * 8) = make_uint4(l[0], l[1], l[2], l[3]);
                }
            }
        } else {
            for (int m = 0; m < M; ++m) {
                for (int k = threadIdx.x; k < len; k += blockDim.x) {
                    const int kk = k0 + k;
                    const int16_t v = kk < K ? x[(size_t)m * ldx + kk] : (int16_t)0;
                    hi_plane[m * len + k] = (int16_t)(v >> 8);
                    lo_plane[m * len + k] = (int16_t)(v & 255);
                }
            }
        }
        __syncthreads();
        for (int kb = 0; kb < len; kb += U * kWave * 8) {
            if (kb > 0) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int k = kb + u * (kWave * 8) + lane * 8;
#pragma unroll
                    for (int r = 0; r < R; ++r)
                        w[u][r] = (k < len && rok[r]) ? *reinterpret_cast<const uint4*>(wrow[r] + k0 + k)
                                                      : make_uint4(0, 0, 0, 0);
                }
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = kb + u * (kWave * 8) + lane * 8;
                if (k < len) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        if (m < M) {
                            const uint4 h = *reinterpret_cast<const uint4*>(hi_plane + m * len + k);
                            const uint4 l = *reinterpret_cast<const uint4*>(lo_plane + m * len + k);
#pragma unroll
                            for (int r = 0; r < R; ++r) {
                                auto d2 = [](uint32_t a, uint32_t b, int32_t c) {
                                    return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, b), c, false);
                                };
                                ahi[r][m] = d2(w[u][r].x, h.x, ahi[r][m]);
                                ahi[r][m] = d2(w[u][r].y, h.y, ahi[r][m]);
                                ahi[r][m] = d2(w[u][r].z, h.z, ahi[r][m]);
                                ahi[r][m] = d2(w[u][r].w, h.w, ahi[r][m]);
                                alo[r][m] = d2(w[u][r].x, l.x, alo[r][m]);
                                alo[r][m] = d2(w[u][r].y, l.y, alo[r][m]);
                                alo[r][m] = d2(w[u][r].z, l.z, alo[r][m]);
                                alo[r][m] = d2(w[u][r].w, l.w, alo[r][m]);
                            }
                        }
                    }
                }
            }
        }
    }
    int64_t tot[R][MT];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int m = 0; m < MT; ++m)
            tot[r][m] = wave_sum_i64((int64_t)ahi[r][m] * 256 + (int64_t)alo[r][m]);
    epi.apply(row0, N, M, lane, tot);
}

// Exact fallback for shapes the fast kernels do not take (K % 16 != 0,
// unaligned rows, K beyond the i32-partial bound): one thread per (m, row),
// plain i64 accumulation.  Grid: x over rows, y over activation rows.
template <typename WT, class Epi>
__global__ __launch_bounds__(256) void gemv_generic_kernel(const int16_t* __restrict__ x, int M, int ldx,
                                                          const WT* __restrict__ W, int N, int K, Epi epi) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    const int m = blockIdx.y;
    if (r >= N || m >= M) return;
    uint64_t acc = 0;
    const WT* w = W + (size_t)r * K;
    const int16_t* xr = x + (size_t)m * ldx;
    for (int k = 0; k < K; ++k) acc += (uint64_t)((int64_t)w[k] * (int64_t)xr[k]);
    epi.one(r, m, (int64_t)acc);
}

// ---- standard epilogues ------------------------------------------------------

// linear.rs:61-68 / :110-117: clamp_i16(rescale_i64(acc, w_shift + act_frac, out_frac)).
struct EpiShift {
    const uint8_t* w_shifts;
    const uint8_t* out_frac_pc;  // per channel (linear_w8a16_pc) or null
    uint8_t act_frac, out_frac;
    int16_t* out; int ldo;
    EpiShift offset_m(int m0) const { EpiShift e = *this; e.out += (size_t)m0 * ldo; return e; }
    // the per-row operands, loadable ahead of the sums
    struct Ops {
        uint8_t ws, of;
    };
    __device__ inline Ops ops(int r) const { return Ops{w_shifts[r], out_frac_pc ? out_frac_pc[r] : out_frac}; }
    __device__ inline void one_ops(int r, int m, int64_t acc, const Ops& o) const {
        out[(size_t)m * ldo + r] = clamp_i16_i64(rescale64(acc, (uint8_t)(o.ws + act_frac), o.of));
    }
    __device__ inline void one(int r, int m, int64_t acc) const { one_ops(r, m, acc, ops(r)); }
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (lane == r * MT + m && row0 + r < N && m < M) one(row0 + r, m, tot[r][m]);
    }
};

// Build-defined multiplier requant: clamp_i16(rshift_round_i128(acc * mult, shift)).
struct EpiMult {
    const int32_t* mult;
    const uint8_t* shift;
    int16_t* out; int ldo;
    EpiMult offset_m(int m0) const { EpiMult e = *this; e.out += (size_t)m0 * ldo; return e; }
    struct Ops {
        int32_t mult;
        uint8_t shift;
    };
    __device__ inline Ops ops(int r) const { return Ops{mult[r], shift[r]}; }
    __device__ inline void one_ops(int r, int m, int64_t acc, const Ops& o) const {
        myl_i128 p = (myl_i128)acc * (myl_i128)o.mult;
        myl_i128 y = rshift_round128(p, o.shift);
        out[(size_t)m * ldo + r] = y < -32768 ? (int16_t)-32768 : (y > 32767 ? (int16_t)32767 : (int16_t)y);
    }
    __device__ inline void one(int r, int m, int64_t acc) const { one_ops(r, m, acc, ops(r)); }
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (lane == r * MT + m && row0 + r < N && m < M) one(row0 + r, m, tot[r][m]);
    }
};

// model.rs:293-295: logits = clamp_i32(rescale_i64(acc, row_shift + norm_frac, logit_frac)).
struct EpiLogits {
    const uint8_t* row_shifts;
    uint8_t norm_frac, logit_frac;
    int32_t* out; int ldo;
    EpiLogits offset_m(int m0) const { EpiLogits e = *this; e.out += (size_t)m0 * ldo; return e; }
    __device__ inline void one(int r, int m, int64_t acc) const {
        out[(size_t)m * ldo + r] = clamp_i32_i64(rescale64(acc, (uint8_t)(row_shifts[r] + norm_frac), logit_frac));
    }
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (lane == r * MT + m && row0 + r < N && m < M) one(row0 + r, m, tot[r][m]);
    }
};

// Raw i64 sums (for tests and for consumers with their own epilogue).
struct EpiRaw {
    int64_t* out; int ldo;
    EpiRaw offset_m(int m0) const { EpiRaw e = *this; e.out += (size_t)m0 * ldo; return e; }
    __device__ inline void one(int r, int m, int64_t acc) const { out[(size_t)m * ldo + r] = acc; }
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MT; ++m)
                if (lane == r * MT + m && row0 + r < N && m < M) one(row0 + r, m, tot[r][m]);
    }
};

}  // namespace myl
