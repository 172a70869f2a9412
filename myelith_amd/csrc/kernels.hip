// kernels.hip -- launchers for the GEMV and the op kernels of the integer
// forward path (gfx950).  Host-side shape checks live in abi.cpp; everything
// here assumes validated arguments.
#include "internal.h"
#include "gemm_mfma.h"
#include "gemv.h"
#include "ops.h"

#include <cstdlib>

namespace myl {

// ---------------------------------------------------------------------------
// GEMV dispatch
// ---------------------------------------------------------------------------

inline int xvec_ok(const int16_t* x, int ldx) { return (((uintptr_t)x & 15) == 0) && (ldx % 8 == 0); }

template <int R, int MT, int U, class Epi>
static hipError_t launch_i8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
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
static hipError_t launch_i16(const int16_t* x, int M, int ldx, const int16_t* W, int N, int K, const Epi& epi,
                             hipStream_t st) {
    const int kc = min(kGemvLdsBytes / (4 * MT), ((K + 7) / 8) * 8);
    const int rows_per_block = R * kGemvWaves;
    const int blocks = (N + rows_per_block - 1) / rows_per_block;
    gemv_i16_kernel<R, MT, U, Epi><<<blocks, kGemvThreads, (size_t)4 * MT * kc, st>>>(x, M, ldx, W, N, K, kc,
                                                                                    xvec_ok(x, ldx), epi);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Matrix-core path (M > 8 activation rows)
// ---------------------------------------------------------------------------

// Tile shapes (activation rows x weight rows per block).
enum MmTile { MM_128x128 = 0, MM_128x64 = 1, MM_64x128 = 2, MM_64x64 = 3 };

// Overrides for tile sweeps: MYL_MM_TILE (an MmTile) and MYL_MM_KSPLIT.
static int mm_env(const char* name) {
    const char* v = std::getenv(name);
    return v && *v ? std::atoi(v) : -1;
}

template <int WM, int WN, int WAVES_M, int WAVES_N, class Epi>
static hipError_t mm_launch(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
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

// Tile and K split, from a sweep of the W8A16 shapes on MI355X: 64-row tiles
// (two waves per SIMD) beat 128-row tiles at every M; 64 x 128 wins once M
// is large.  K is split (slices of >= 1024 bytes) only when the tiles alone
// leave CUs idle.
template <class Epi>
static hipError_t mm_i8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
                        const MmCtx* mm, hipStream_t st) {
    const int cus = mm ? mm->cus : 256;
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
static hipError_t gemv_i8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const Epi& epi,
                          hipStream_t st, const MmCtx* mm) {
    const bool fast = (K % 16 == 0) && (((uintptr_t)W & 15) == 0) && K < 131072;
    if (!fast) {
        dim3 grid((N + 255) / 256, M);
        gemv_generic_kernel<int8_t, Epi><<<grid, 256, 0, st>>>(x, M, ldx, W, N, K, epi);
        return hipGetLastError();
    }
    // More than 8 activation rows: the int8 matrix cores (16-byte aligned rows).
    if (M > 8 && xvec_ok(x, ldx)) return mm_i8(x, M, ldx, W, N, K, epi, mm, st);
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
static hipError_t gemv_i16(const int16_t* x, int M, int ldx, const int16_t* W, int N, int K, const Epi& epi,
                           hipStream_t st) {
    const bool fast = (K % 8 == 0) && (((uintptr_t)W & 15) == 0) && K <= 8192;
    if (!fast) {
        dim3 grid((N + 255) / 256, M);
        gemv_generic_kernel<int16_t, Epi><<<grid, 256, 0, st>>>(x, M, ldx, W, N, K, epi);
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

hipError_t linear_w8a16(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const uint8_t* w_shifts,
                        uint8_t act_frac, uint8_t out_frac, const uint8_t* out_frac_pc, int16_t* out, int ldo,
                        hipStream_t st, const MmCtx* mm) {
    EpiShift e{w_shifts, out_frac_pc, act_frac, out_frac, out, ldo};
    return gemv_i8(x, M, ldx, W, N, K, e, st, mm);
}

hipError_t linear_w8a16_mult(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const int32_t* mult,
                             const uint8_t* shift, int16_t* out, int ldo, hipStream_t st, const MmCtx* mm) {
    EpiMult e{mult, shift, out, ldo};
    return gemv_i8(x, M, ldx, W, N, K, e, st, mm);
}

hipError_t logits_w8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const uint8_t* row_shifts,
                     uint8_t norm_frac, uint8_t logit_frac, int32_t* out, int ldo, hipStream_t st, const MmCtx* mm) {
    EpiLogits e{row_shifts, norm_frac, logit_frac, out, ldo};
    return gemv_i8(x, M, ldx, W, N, K, e, st, mm);
}

hipError_t logits_w16(const int16_t* x, int M, int ldx, const int16_t* W, int N, int K, const uint8_t* row_shifts,
                      uint8_t norm_frac, uint8_t logit_frac, int32_t* out, int ldo, hipStream_t st, const MmCtx* mm) {
    EpiLogits e{row_shifts, norm_frac, logit_frac, out, ldo};
    return gemv_i16(x, M, ldx, W, N, K, e, st);
}

hipError_t dot_raw_w8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, int64_t* out, int ldo,
                      hipStream_t st, const MmCtx* mm) {
    EpiRaw e{out, ldo};
    return gemv_i8(x, M, ldx, W, N, K, e, st, mm);
}

// ---------------------------------------------------------------------------
// RMSNorm (rmsnorm.rs:61-161): one block per row.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void rmsnorm_kernel(const int16_t* __restrict__ x, int ldx,
                                                        const uint8_t* __restrict__ xs, const int8_t* __restrict__ g,
                                                        const uint8_t* __restrict__ gs, int n, RmsParams p,
                                                        uint8_t out_frac, int16_t* __restrict__ out, int ldo) {
    __shared__ myl_i128 red128[kBlock];
    __shared__ int32_t red32[kBlock / 64];
    const int16_t* xr = x + (size_t)blockIdx.x * ldx;
    const RmsFactor f = rms_factor(xr, xs, n, p, red128, red32);
    int16_t* o = out + (size_t)blockIdx.x * ldo;
    for (int i = threadIdx.x; i < n; i += blockDim.x) o[i] = rms_out(xr[i], xs[i], g[i], gs[i], f, out_frac);
}

// Rows of up to kRmsThreads * kRmsPer elements: every element is loaded once,
// before the reductions, and stays in registers.
constexpr int kRmsThreads = 1024;
constexpr int kRmsPer = 4;
__global__ __launch_bounds__(kRmsThreads) void rmsnorm_fast_kernel(const int16_t* __restrict__ x, int ldx,
                                                                  const uint8_t* __restrict__ xs,
                                                                  const int8_t* __restrict__ g,
                                                                  const uint8_t* __restrict__ gs, int n, RmsParams p,
                                                                  uint8_t out_frac, int16_t* __restrict__ out, int ldo) {
    __shared__ myl_i128 red128[kRmsThreads / 64];
    __shared__ int32_t red32[kRmsThreads / 64];
    const int16_t* xr = x + (size_t)blockIdx.x * ldx;
    int16_t xv[kRmsPer];
    uint8_t sv[kRmsPer];
    int8_t gv[kRmsPer];
    uint8_t gsv[kRmsPer];
#pragma unroll
    for (int t = 0; t < kRmsPer; ++t) {
        const int i = threadIdx.x + t * kRmsThreads;
        const bool ok = i < n;
        xv[t] = ok ? xr[i] : (int16_t)0;
        sv[t] = ok ? xs[i] : (uint8_t)0;
        gv[t] = ok ? g[i] : (int8_t)0;
        gsv[t] = ok ? gs[i] : (uint8_t)0;
    }
    const RmsFactor f = rms_factor_regs<kRmsPer>(xv, sv, p, red128, red32);
    int16_t* o = out + (size_t)blockIdx.x * ldo;
#pragma unroll
    for (int t = 0; t < kRmsPer; ++t) {
        const int i = threadIdx.x + t * kRmsThreads;
        if (i < n) o[i] = rms_out(xv[t], sv[t], gv[t], gsv[t], f, out_frac);
    }
}

hipError_t rmsnorm(const int16_t* x, int M, int ldx, const uint8_t* xs, const int8_t* g, const uint8_t* gs, int n,
                   const int16_t* lut, int lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                   int64_t inv_n_q20, uint8_t out_frac, int16_t* out, int ldo, hipStream_t st) {
    RmsParams p{lut, lut_len, lut_input_shift, lut_output_frac, inv_n_q20};
    if (n <= kRmsThreads * kRmsPer)
        rmsnorm_fast_kernel<<<M, kRmsThreads, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo);
    else
        rmsnorm_kernel<<<M, kBlock, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Softmax (softmax.rs:24-64): one block per row.
// ---------------------------------------------------------------------------

__device__ inline void softmax_row(const int32_t* __restrict__ z, int n, const int16_t* __restrict__ lut,
                                   uint32_t lut_len, uint8_t lut_shift, uint8_t frac_bits, int32_t* __restrict__ out,
                                   int32_t* red32, uint32_t* redu) {
    const int32_t one = shl32(1, frac_bits);
    const int32_t lut_one = lut_len > 0 ? (int32_t)lut[0] : 1;
    int32_t mx = INT32_MIN;
    for (int i = threadIdx.x; i < n; i += blockDim.x) mx = max(mx, z[i]);
    const int32_t m = n > 0 ? block_max_i32(mx, red32) : 0;
    uint32_t s = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x)
        s += (uint32_t)exp_lookup(sat_sub32(m, z[i]), lut, lut_len, lut_shift, lut_one);
    const int32_t S = (int32_t)block_sum_u32(s, redu);
    if (S == 0) {
        // softmax.rs:42-48: uniform with the remainder on the lowest indices.
        // one / n without a divide: n * q <= one < n * (q + 1) by long division.
        uint32_t un = (uint32_t)n;
        uint32_t q = 0, r = 0;
        if (un) {
            uint64_t recip = recip32(un);
            uint32_t uone = one < 0 ? 0u - (uint32_t)one : (uint32_t)one;
            udivmod32(uone, un, recip, &q, &r);
        }
        int32_t base = one < 0 ? -(int32_t)q : (int32_t)q;
        int32_t rem = wsub32(one, wmul32(base, (int32_t)n));
        for (int i = threadIdx.x; i < n; i += blockDim.x)
            out[i] = base + (((uint64_t)i < (uint64_t)(int64_t)rem) ? 1 : 0);
        return;
    }
    const uint32_t us = S < 0 ? 0u - (uint32_t)S : (uint32_t)S;
    const uint64_t recip = recip32(us);
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int32_t e = exp_lookup(sat_sub32(m, z[i]), lut, lut_len, lut_shift, lut_one);
        out[i] = softmax_div_round(wmul32(e, one), S, recip);
    }
}

__global__ __launch_bounds__(kBlock) void softmax_kernel(const int32_t* __restrict__ z, int n, int ldz,
                                                        const int16_t* __restrict__ lut, uint32_t lut_len,
                                                        uint8_t lut_shift, uint8_t frac_bits, int32_t* __restrict__ out,
                                                        int ldo) {
    __shared__ int32_t red32[kBlock / 64];
    __shared__ uint32_t redu[kBlock / 64];
    softmax_row(z + (size_t)blockIdx.x * ldz, n, lut, lut_len, lut_shift, frac_bits, out + (size_t)blockIdx.x * ldo,
                red32, redu);
}

hipError_t softmax(const int32_t* z, int M, int n, int ldz, const int16_t* lut, int lut_len, uint8_t lut_shift,
                   uint8_t frac_bits, int32_t* out, int ldo, hipStream_t st) {
    softmax_kernel<<<M, kBlock, 0, st>>>(z, n, ldz, lut, (uint32_t)lut_len, lut_shift, frac_bits, out, ldo);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Generic attention (attention.rs:42-90): one block per query row.
// scratch holds q_len x kv_len i32 scores followed by as many i32 probs.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kBlock) void attn_scores_kernel(const int16_t* __restrict__ q, const int16_t* __restrict__ k,
                                                            const uint8_t* __restrict__ mask, int kv_len, int hd,
                                                            int64_t score_mult, uint8_t score_shift,
                                                            int32_t* __restrict__ scores) {
    const int i = blockIdx.y;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j >= kv_len) return;
    int32_t s;
    if (!mask || mask[(size_t)i * kv_len + j]) {
        const int16_t* qi = q + (size_t)i * hd;
        const int16_t* kj = k + (size_t)j * hd;
        uint64_t acc = 0;
        for (int d = 0; d < hd; ++d) acc += (uint64_t)((int64_t)qi[d] * (int64_t)kj[d]);
        s = (int32_t)rshift_round64(wmul64((int64_t)acc, score_mult), score_shift);
    } else {
        s = INT32_MIN;
    }
    scores[(size_t)i * kv_len + j] = s;
}

__global__ __launch_bounds__(kBlock) void attn_pv_kernel(const int32_t* __restrict__ probs, const int16_t* __restrict__ v,
                                                        int kv_len, int hd, uint8_t prob_frac,
                                                        int16_t* __restrict__ out) {
    const int i = blockIdx.y;
    const int d = blockIdx.x * blockDim.x + threadIdx.x;
    if (d >= hd) return;
    const int32_t* p = probs + (size_t)i * kv_len;
    uint64_t acc = 0;
    for (int j = 0; j < kv_len; ++j) acc += (uint64_t)((int64_t)p[j] * (int64_t)v[(size_t)j * hd + d]);
    out[(size_t)i * hd + d] = clamp_i16_i64(rshift_round64((int64_t)acc, prob_frac));
}

hipError_t attention_generic(const int16_t* q, const int16_t* k, const int16_t* v, const uint8_t* mask, int q_len,
                             int kv_len, int hd, int64_t score_mult, uint8_t score_shift, const int16_t* lut,
                             int lut_len, uint8_t lut_shift, uint8_t prob_frac, int32_t* scratch, int16_t* out,
                             hipStream_t st) {
    int32_t* scores = scratch;
    int32_t* probs = scratch + (size_t)q_len * kv_len;
    attn_scores_kernel<<<dim3((kv_len + kBlock - 1) / kBlock, q_len), kBlock, 0, st>>>(q, k, mask, kv_len, hd,
                                                                                         score_mult, score_shift, scores);
    hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) return rc;
    rc = softmax(scores, q_len, kv_len, kv_len, lut, lut_len, lut_shift, prob_frac, probs, kv_len, st);
    if (rc != hipSuccess) return rc;
    attn_pv_kernel<<<dim3((hd + kBlock - 1) / kBlock, q_len), kBlock, 0, st>>>(probs, v, kv_len, hd, prob_frac, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RoPE (rope.rs:17-59): one thread per (row, pair); rows[] holds pos % n_pos.
// ---------------------------------------------------------------------------

__global__ void rope_kernel(int16_t* __restrict__ q, int16_t* __restrict__ k, int n, int hd,
                            const int16_t* __restrict__ cos_lut, const int16_t* __restrict__ sin_lut,
                            const int32_t* __restrict__ rows, uint8_t frac_bits) {
    const int half = hd >> 1;
    const int j = blockIdx.x * blockDim.x + threadIdx.x;
    const int i = blockIdx.y;
    if (j >= half || i >= n) return;
    const int32_t c = cos_lut[(size_t)rows[i] * half + j];
    const int32_t s = sin_lut[(size_t)rows[i] * half + j];
    for (int t = 0; t < 2; ++t) {
        int16_t* vec = (t == 0 ? q : k) + (size_t)i * hd;
        const int32_t x0 = vec[j], x1 = vec[j + half];
        vec[j] = clamp_i16(rshift_round32(wsub32(wmul32(x0, c), wmul32(x1, s)), frac_bits));
        vec[j + half] = clamp_i16(rshift_round32(wadd32(wmul32(x1, c), wmul32(x0, s)), frac_bits));
        if ((hd & 1) && j == 0) vec[hd - 1] = 0;
    }
}

hipError_t rope(int16_t* q, int16_t* k, int n, int hd, const int16_t* cos_lut, const int16_t* sin_lut,
                const int32_t* rows, uint8_t frac_bits, hipStream_t st) {
    const int half = hd >> 1;
    rope_kernel<<<dim3((half + 127) / 128, n), 128, 0, st>>>(q, k, n, hd, cos_lut, sin_lut, rows, frac_bits);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Bias (linear.rs:132-145), SiLU gating (mlp.rs:55-65), argmax (sampling.rs:8-18)
// ---------------------------------------------------------------------------

__global__ void bias_kernel(int16_t* __restrict__ out, const int16_t* __restrict__ b, const uint8_t* __restrict__ bs,
                            int n, uint8_t out_frac) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const int32_t br = rescale32((int32_t)b[i], bs[i], out_frac);
    out[i] = clamp_i16_i64((int64_t)out[i] + (int64_t)br);
}

hipError_t add_bias(int16_t* out, const int16_t* b, const uint8_t* bs, int n, uint8_t out_frac, hipStream_t st) {
    bias_kernel<<<(n + 255) / 256, 256, 0, st>>>(out, b, bs, n, out_frac);
    return hipGetLastError();
}

__device__ inline int16_t silu_gate(int16_t g, int16_t u, const int16_t* silu, uint32_t silu_len, uint8_t gate_frac,
                                    uint8_t up_frac, uint8_t down_in_frac, uint8_t silu_in_frac, int16_t silu_off,
                                    uint8_t silu_out_frac) {
    const int32_t g_dom = rescale32((int32_t)g, gate_frac, silu_in_frac);
    const int16_t act = lut_lookup_i16((int16_t)g_dom, silu, silu_len, silu_off);
    const int64_t prod = (int64_t)act * (int64_t)u;
    return clamp_i16_i64(rescale64(prod, (uint8_t)(silu_out_frac + up_frac), down_in_frac));
}

__global__ void silu_gate_kernel(const int16_t* __restrict__ gate, const int16_t* __restrict__ up, int n,
                                 const int16_t* __restrict__ silu, uint32_t silu_len, uint8_t gate_frac, uint8_t up_frac,
                                 uint8_t down_in_frac, uint8_t silu_in_frac, int16_t silu_off, uint8_t silu_out_frac,
                                 int16_t* __restrict__ h) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    h[i] = silu_gate(gate[i], up[i], silu, silu_len, gate_frac, up_frac, down_in_frac, silu_in_frac, silu_off,
                     silu_out_frac);
}

hipError_t silu_gate(const int16_t* gate, const int16_t* up, int n, const int16_t* silu, int silu_len,
                     uint8_t gate_frac, uint8_t up_frac, uint8_t down_in_frac, uint8_t silu_in_frac, int16_t silu_off,
                     uint8_t silu_out_frac, int16_t* h, hipStream_t st) {
    silu_gate_kernel<<<(n + 255) / 256, 256, 0, st>>>(gate, up, n, silu, (uint32_t)silu_len, gate_frac, up_frac,
                                                      down_in_frac, silu_in_frac, silu_off, silu_out_frac, h);
    return hipGetLastError();
}

// First maximum wins: the key orders by value, then by the smaller index.
__device__ inline uint64_t argmax_key(int32_t v, uint32_t idx) {
    return ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__global__ __launch_bounds__(kBlock) void argmax_kernel(const int32_t* __restrict__ v, int n, int ldv,
                                                       int64_t* __restrict__ out) {
    __shared__ uint64_t red[kBlock];
    const int32_t* row = v + (size_t)blockIdx.x * ldv;
    uint64_t best = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint64_t key = argmax_key(row[i], (uint32_t)i);
        best = key > best ? key : best;
    }
    red[threadIdx.x] = best;
    __syncthreads();
    for (int s = blockDim.x >> 1; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x] > red[threadIdx.x + s] ? red[threadIdx.x] : red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = (int64_t)(0xFFFFFFFFu - (uint32_t)(red[0] & 0xFFFFFFFFu));
}

hipError_t argmax(const int32_t* v, int M, int n, int ldv, int64_t* out, hipStream_t st) {
    argmax_kernel<<<M, kBlock, 0, st>>>(v, n, ldv, out);
    return hipGetLastError();
}

}  // namespace myl
