// kernels.hip -- launchers for the GEMV and the op kernels of the integer
// forward path (gfx950).  Host-side shape checks live in abi.cpp; everything
// here assumes validated arguments.
#include "gemm_dispatch.h"
#include "../../include/myl_theta_v.h"
#include "ops.h"
#include "wave.h"

namespace myl {

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
                                                                  uint8_t out_frac, int16_t* __restrict__ out, int ldo,
                                                                  int8_t* __restrict__ planes) {
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
    if (planes) {
        // byte planes of the output row: hi at row 2m, lo' at row 2m + 1
        int8_t* ph = planes + (size_t)(2 * blockIdx.x) * n;
#pragma unroll
        for (int t = 0; t < kRmsPer; ++t) {
            const int i = threadIdx.x + t * kRmsThreads;
            if (i < n) {
                const int32_t y = rms_out(xv[t], sv[t], gv[t], gsv[t], f, out_frac);
                ph[i] = (int8_t)(y >> 8);
                ph[n + i] = (int8_t)((y & 255) - 128);
            }
        }
        return;
    }
    int16_t* o = out + (size_t)blockIdx.x * ldo;
#pragma unroll
    for (int t = 0; t < kRmsPer; ++t) {
        const int i = threadIdx.x + t * kRmsThreads;
        if (i < n) o[i] = rms_out(xv[t], sv[t], gv[t], gsv[t], f, out_frac);
    }
}

// 256 threads per row, each thread owning PER chunks of 8
// consecutive elements loaded as one 16-byte (x) and 8-byte (shifts, gamma)
// vector each; rows of n % 8 == 0 elements, 16-byte aligned.  The sum of
// squares stays in 64 bits for elements at the largest shift (align 0) and
// takes the exact 128-bit path only for the others.
constexpr int kRowsThreads = 256;

__device__ inline uint8_t byte_of(const uint2& v, int q) {
    return (uint8_t)(((q < 4 ? v.x : v.y) >> (8 * (q & 3))) & 0xFFu);
}

template <int PER>
__global__ __launch_bounds__(kRowsThreads) void rmsnorm_rows_kernel(const int16_t* __restrict__ x, int ldx,
                                                                    const uint8_t* __restrict__ xs,
                                                                    const int8_t* __restrict__ g,
                                                                    const uint8_t* __restrict__ gs, int n,
                                                                    RmsParams p, uint8_t out_frac,
                                                                    int16_t* __restrict__ out, int ldo,
                                                                    int8_t* __restrict__ planes) {
    __shared__ myl_i128 red128[kRowsThreads / 64];
    __shared__ int32_t red32[kRowsThreads / 64];
    const int16_t* xr = x + (size_t)blockIdx.x * ldx;
    const int nc = n >> 3;
    uint4 xv[PER];
    uint2 sv[PER], gv[PER], gsv[PER];  // gamma and its shifts load with x
    int32_t mx = 0;
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int c = threadIdx.x + t * kRowsThreads;
        xv[t] = make_uint4(0, 0, 0, 0);
        sv[t] = gv[t] = gsv[t] = make_uint2(0, 0);
        if (c < nc) {
            xv[t] = *reinterpret_cast<const uint4*>(xr + 8 * c);
            sv[t] = *reinterpret_cast<const uint2*>(xs + 8 * c);
            gv[t] = *reinterpret_cast<const uint2*>(g + 8 * c);
            gsv[t] = *reinterpret_cast<const uint2*>(gs + 8 * c);
        }
    }
#pragma unroll
    for (int t = 0; t < PER; ++t)
#pragma unroll
        for (int q = 0; q < 8; ++q) mx = max(mx, (int32_t)byte_of(sv[t], q));
    const uint8_t ref = (uint8_t)block_max_i32(mx, red32);
    uint64_t acc64 = 0;
    myl_i128 acc = 0;
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const uint32_t w[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int32_t xi = (int32_t)(int16_t)((w[q >> 1] >> (16 * (q & 1))) & 0xFFFFu);
            const uint32_t sq = (uint32_t)(xi * xi);   // <= 2^30
            const uint32_t align = 2u * (uint32_t)(uint8_t)(ref - byte_of(sv[t], q));
            if (align == 0) acc64 += sq;
            else acc = (myl_i128)((myl_u128)acc + (myl_u128)shl128((myl_i128)sq, align));
        }
    }
    // all lanes at the largest shift (the usual case): a 64-bit DPP sum
    // (each lane < 2^34, so the wave total < 2^40); else the 128-bit one
    if (__any(acc != 0)) acc = wave_sum_i128((myl_i128)((myl_u128)acc + (myl_u128)acc64));
    else acc = (myl_i128)wave_sum_u64(acc64);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red128[threadIdx.x >> 6] = acc;
    __syncthreads();
    acc = 0;
#pragma unroll
    for (int i = 0; i < kRowsThreads / 64; ++i) acc = (myl_i128)((myl_u128)acc + (myl_u128)red128[i]);
    const RmsFactor f = rms_factor_of(acc, ref, p);
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int c = threadIdx.x + t * kRowsThreads;
        if (c >= nc) continue;
        const uint32_t w[4] = {xv[t].x, xv[t].y, xv[t].z, xv[t].w};
        int32_t y[8];
#pragma unroll
        for (int q = 0; q < 8; ++q)
            y[q] = rms_out((int16_t)((w[q >> 1] >> (16 * (q & 1))) & 0xFFFFu), byte_of(sv[t], q),
                           (int8_t)byte_of(gv[t], q), byte_of(gsv[t], q), f, out_frac);
        if (planes) {
            uint32_t h[2] = {0, 0}, l[2] = {0, 0};
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                h[q >> 2] |= ((uint32_t)(y[q] >> 8) & 0xFFu) << (8 * (q & 3));
                l[q >> 2] |= ((uint32_t)((y[q] & 255) - 128) & 0xFFu) << (8 * (q & 3));
            }
            int8_t* ph = planes + (size_t)(2 * blockIdx.x) * n + 8 * c;
            *reinterpret_cast<uint2*>(ph) = make_uint2(h[0], h[1]);
            *reinterpret_cast<uint2*>(ph + n) = make_uint2(l[0], l[1]);
        } else {
            uint32_t o[4];
#pragma unroll
            for (int q = 0; q < 4; ++q)
                o[q] = ((uint32_t)y[2 * q] & 0xFFFFu) | ((uint32_t)y[2 * q + 1] << 16);
            *reinterpret_cast<uint4*>(out + (size_t)blockIdx.x * ldo + 8 * c) = make_uint4(o[0], o[1], o[2], o[3]);
        }
    }
}

// The row kernel's PER for n elements (0: not applicable).
inline int rms_rows_per(int n) {
    if (n % 8 != 0) return 0;
    const int nc = n / 8;
    return nc <= kRowsThreads ? 1 : nc <= 2 * kRowsThreads ? 2 : nc <= 4 * kRowsThreads ? 4 : 0;
}

// Row kernel launch when the layout allows it.
bool rmsnorm_rows(const int16_t* x, int M, int ldx, const uint8_t* xs, const int8_t* g, const uint8_t* gs, int n,
                  const RmsParams& p, uint8_t out_frac, int16_t* out, int ldo, int8_t* planes, hipStream_t st) {
    const int per = rms_rows_per(n);
    const bool aligned = ((uintptr_t)x % 16 == 0) && ldx % 8 == 0 && ((uintptr_t)xs % 8 == 0) &&
                         ((uintptr_t)g % 8 == 0) && ((uintptr_t)gs % 8 == 0) &&
                         (planes ? (uintptr_t)planes % 8 == 0 : ((uintptr_t)out % 16 == 0 && ldo % 8 == 0));
    if (M < 1 || per == 0 || !aligned) return false;
    if (per == 1)
        rmsnorm_rows_kernel<1><<<M, kRowsThreads, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo, planes);
    else if (per == 2)
        rmsnorm_rows_kernel<2><<<M, kRowsThreads, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo, planes);
    else
        rmsnorm_rows_kernel<4><<<M, kRowsThreads, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo, planes);
    return true;
}

hipError_t rmsnorm(const int16_t* x, int M, int ldx, const uint8_t* xs, const int8_t* g, const uint8_t* gs, int n,
                   const int16_t* lut, int lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                   int64_t inv_n_q20, uint8_t out_frac, int16_t* out, int ldo, hipStream_t st) {
    RmsParams p{lut, lut_len, lut_input_shift, lut_output_frac, inv_n_q20};
    if (rmsnorm_rows(x, M, ldx, xs, g, gs, n, p, out_frac, out, ldo, nullptr, st)) return hipGetLastError();
    if (n <= kRmsThreads * kRmsPer)
        rmsnorm_fast_kernel<<<M, kRmsThreads, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo, nullptr);
    else
        rmsnorm_kernel<<<M, kBlock, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, out, ldo);
    return hipGetLastError();
}

bool rmsnorm_planes_ok(int n) { return n <= kRmsThreads * kRmsPer; }

hipError_t rmsnorm_planes(const int16_t* x, int M, int ldx, const uint8_t* xs, const int8_t* g, const uint8_t* gs,
                          int n, const int16_t* lut, int lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                          int64_t inv_n_q20, uint8_t out_frac, int8_t* planes, hipStream_t st) {
    if (!rmsnorm_planes_ok(n)) return hipErrorInvalidValue;
    RmsParams p{lut, lut_len, lut_input_shift, lut_output_frac, inv_n_q20};
    if (rmsnorm_rows(x, M, ldx, xs, g, gs, n, p, out_frac, nullptr, 0, planes, st)) return hipGetLastError();
    rmsnorm_fast_kernel<<<M, kRmsThreads, 0, st>>>(x, ldx, xs, g, gs, n, p, out_frac, nullptr, 0, planes);
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

// Integer log-softmax of one row at its target (build-defined, see fixed.h):
//   m = max z;  S = sum_j lut[(m - z_j) << 2] (0 past the table; logits are
//   Q6 and the exp LUT's input is Q8);  lp = (z_target - m) * 2^10 - ln_q16(S)
// in Q16.  One block per row; targets < 0 give 0.
constexpr int kLogsoftmaxLds = 4096;  // exp-table entries a block copies to LDS (8 KB)
__global__ __launch_bounds__(kBlock) void logsoftmax_kernel(const int32_t* __restrict__ z, int n, int ldz,
                                                           const int16_t* __restrict__ lut, uint32_t lut_len,
                                                           const int64_t* __restrict__ targets,
                                                           int64_t* __restrict__ out) {
    __shared__ int32_t red32[kBlock / 64];
    __shared__ uint64_t red64[kBlock / 64];
    __shared__ int16_t elut[kLogsoftmaxLds];
    const int32_t* row = z + (size_t)blockIdx.x * ldz;
    // the table's first entries in LDS (the exp table is zero past a short
    // prefix, so nearly every lookup is served there); the rest from memory
    const int nl = (int)min(lut_len, (uint32_t)kLogsoftmaxLds);
    for (int i = threadIdx.x; i < nl; i += kBlock) elut[i] = lut[i];
    // 16-byte loads over the aligned part of the row, four in flight per thread
    const int n4 = ((uintptr_t)row & 15) == 0 ? n >> 2 : 0;
    const int4* row4 = reinterpret_cast<const int4*>(row);
    int32_t mx = INT32_MIN;
#pragma unroll 4
    for (int i = threadIdx.x; i < n4; i += kBlock) {
        const int4 v = row4[i];
        mx = max(mx, max(max(v.x, v.y), max(v.z, v.w)));
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += kBlock) mx = max(mx, row[i]);
    const int32_t m = block_max_i32(mx, red32);  // its barrier also publishes elut
    constexpr uint32_t sh = MYL_TV_EXP_INPUT_FRAC - MYL_TV_LOGIT_FRAC_BITS;
    auto term = [&](int32_t zi) -> int64_t {
        const uint64_t d = (uint64_t)((int64_t)m - (int64_t)zi) << sh;
        if (d < (uint64_t)nl) return (int64_t)elut[d];
        return d < lut_len ? (int64_t)lut[d] : 0;
    };
    int64_t s = 0;
#pragma unroll 4
    for (int i = threadIdx.x; i < n4; i += kBlock) {
        const int4 v = row4[i];
        s += term(v.x) + term(v.y) + term(v.z) + term(v.w);
    }
    for (int i = 4 * n4 + threadIdx.x; i < n; i += kBlock) s += term(row[i]);
    s = wave_sum_i64(s);
    if ((threadIdx.x & 63) == 0) red64[threadIdx.x >> 6] = (uint64_t)s;
    __syncthreads();
    if (threadIdx.x == 0) {
        int64_t S = 0;
        for (int w = 0; w < (int)(blockDim.x >> 6); ++w) S += (int64_t)red64[w];
        const int64_t t = targets[blockIdx.x];
        int64_t lp = 0;
        if (t >= 0 && t < n)
            lp = ((int64_t)row[t] - (int64_t)m) * 1024 - ln_q16_of_sum(S < 1 ? 1u : (uint64_t)S);
        out[blockIdx.x] = lp;
    }
}

hipError_t logsoftmax(const int32_t* z, int M, int n, int ldz, const int16_t* lut, int lut_len, const int64_t* targets,
                      int64_t* out, hipStream_t st) {
    logsoftmax_kernel<<<M, kBlock, 0, st>>>(z, n, ldz, lut, (uint32_t)lut_len, targets, out);
    return hipGetLastError();
}

hipError_t argmax(const int32_t* v, int M, int n, int ldv, int64_t* out, hipStream_t st) {
    argmax_kernel<<<M, kBlock, 0, st>>>(v, n, ldv, out);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Integer CDF sampling (sampling.rs:20-46): one block per row.
// ---------------------------------------------------------------------------

// SplitMix64 (prng.rs:7-14): advances the state, returns the output.
__device__ inline uint64_t splitmix64_next(uint64_t& state) {
    state += 0x9E3779B97F4A7C15ull;
    uint64_t z = state;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// n % d by binary long division (no hardware divide); d < 2^63.
__device__ inline uint64_t umod64(uint64_t n, uint64_t d) {
    uint64_t r = 0;
    for (int i = 63; i >= 0; --i) {
        r = (r << 1) | ((n >> i) & 1u);
        if (r >= d) r -= d;
    }
    return r;
}

__device__ inline int64_t shfl_up_i64(int64_t v, int d) {
    const uint32_t lo = (uint32_t)__shfl_up((int)(uint32_t)v, d, 64);
    const uint32_t hi = (uint32_t)__shfl_up((int)(uint32_t)((uint64_t)v >> 32), d, 64);
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Exclusive prefix sum of one i64 per thread over the block (wrapping),
// and the block's total.  wt needs one slot per wave.
__device__ inline int64_t block_scan_i64(int64_t v, int64_t* wt, int64_t& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    int64_t inc = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t o = shfl_up_i64(inc, d);
        if (lane >= d) inc = (int64_t)((uint64_t)inc + (uint64_t)o);
    }
    if (lane == 63) wt[w] = inc;
    __syncthreads();
    int64_t before = 0, all = 0;
    for (int k = 0; k < nw; ++k) {
        const int64_t t = wt[k];
        if (k < w) before = (int64_t)((uint64_t)before + (uint64_t)t);
        all = (int64_t)((uint64_t)all + (uint64_t)t);
    }
    total = all;
    return (int64_t)((uint64_t)before + (uint64_t)inc - (uint64_t)v);
}

// sample_integer_cdf (sampling.rs:27-46) of row blockIdx.x at state
// states[row]: weights w_i = z_i - min z + 1 (logits_to_weights,
// sampling.rs:20-24; i32 arithmetic, wrapping as the reference's release
// build does), total = sum w_i as i64; total <= 0 gives token 0 and the state
// unchanged; otherwise (state', r) = splitmix64(state), threshold = r % total
// and the token is the first i with threshold < w_0 + ... + w_i (the last
// index when there is none).  The running sums are scanned over tiles of
// 4 x kSampleThreads positions in order, so the first such i is exact also
// when wrapped weights make the sums non-monotone.
constexpr int kSampleThreads = 1024;
__global__ __launch_bounds__(kSampleThreads) void sample_cdf_kernel(const int32_t* __restrict__ z, int n, int ldz,
                                                                   const uint64_t* __restrict__ states,
                                                                   int64_t* __restrict__ tokens,
                                                                   uint64_t* __restrict__ new_states) {
    __shared__ int32_t redm[kSampleThreads / 64];
    __shared__ int32_t redc[kSampleThreads / 64];
    __shared__ int64_t wt[kSampleThreads / 64];
    __shared__ int64_t s_thr;
    const int32_t* row = z + (size_t)blockIdx.x * ldz;
    const int tid = threadIdx.x;
    // the minimum as ~max(~z) (bitwise not reverses the signed order)
    int32_t nm = INT32_MIN;
    for (int i = tid; i < n; i += kSampleThreads) nm = max(nm, ~row[i]);
    const int32_t m = ~block_max_i32_dpp(nm, redm);
    auto weight = [&](int32_t zi) -> int64_t { return (int64_t)(int32_t)((uint32_t)zi - (uint32_t)m + 1u); };
    int64_t part = 0;
    for (int i = tid; i < n; i += kSampleThreads) part += weight(row[i]);
    int64_t total = 0;
    (void)block_scan_i64(part, wt, total);
    uint64_t state = states[blockIdx.x];
    if (total <= 0) {  // uniform: an empty or non-positive total keeps the state
        if (tid == 0) {
            tokens[blockIdx.x] = 0;
            new_states[blockIdx.x] = state;
        }
        return;
    }
    if (tid == 0) {
        const uint64_t r = splitmix64_next(state);
        s_thr = (int64_t)umod64(r, (uint64_t)total);  // total < 2^62: n < 2^31 weights below 2^31
        new_states[blockIdx.x] = state;
    }
    __syncthreads();
    const int64_t thr = s_thr;
    int64_t base = 0;
    int pick = n - 1;
    for (int t0 = 0; t0 < n; t0 += 4 * kSampleThreads) {
        const int i0 = t0 + 4 * tid;
        int64_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = i0 + e < n ? weight(row[i0 + e]) : 0;
        const int64_t loc = w[0] + w[1] + w[2] + w[3];
        int64_t tile = 0;
        int64_t acc = base + block_scan_i64(loc, wt, tile);
        int cand = INT32_MAX;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            acc += w[e];
            if (i0 + e < n && thr < acc && cand == INT32_MAX) cand = i0 + e;
        }
        // the first candidate of the tile: a block minimum as ~max(~x)
        const int first = ~block_max_i32_dpp(~cand, redc);
        if (first != INT32_MAX) {  // uniform
            pick = first;
            break;
        }
        base += tile;
    }
    if (tid == 0) tokens[blockIdx.x] = pick;
}

hipError_t sample_cdf(const int32_t* z, int M, int n, int ldz, const uint64_t* states, int64_t* tokens,
                      uint64_t* new_states, hipStream_t st) {
    sample_cdf_kernel<<<M, kSampleThreads, 0, st>>>(z, n, ldz, states, tokens, new_states);
    return hipGetLastError();
}

// Best key of chunk blockIdx.x of row blockIdx.y.
__global__ __launch_bounds__(kBlock) void argmax_part_kernel(const int32_t* __restrict__ v, int n, int ldv,
                                                            uint64_t* __restrict__ part, int nch) {
    __shared__ uint64_t red[kBlock];
    const int32_t* row = v + (size_t)blockIdx.y * ldv;
    const int i0 = blockIdx.x * kArgChunk, i1 = min(n, i0 + kArgChunk);
    uint64_t best = 0;
    // 16-byte loads when the chunk starts aligned (kArgChunk is a multiple
    // of 4), the chunk's last partial quad and unaligned rows one by one
    const int q1 = ((uintptr_t)(row + i0) & 15) == 0 ? i0 + ((i1 - i0) & ~3) : i0;
#pragma unroll 4
    for (int i = i0 + 4 * (int)threadIdx.x; i < q1; i += 4 * kBlock) {
        const int4 q = *reinterpret_cast<const int4*>(row + i);
        const uint64_t k0 = argmax_key(q.x, (uint32_t)i), k1 = argmax_key(q.y, (uint32_t)i + 1);
        const uint64_t k2 = argmax_key(q.z, (uint32_t)i + 2), k3 = argmax_key(q.w, (uint32_t)i + 3);
        const uint64_t a = k0 > k1 ? k0 : k1, b = k2 > k3 ? k2 : k3, c = a > b ? a : b;
        best = c > best ? c : best;
    }
    for (int i = q1 + threadIdx.x; i < i1; i += kBlock) {
        const uint64_t key = argmax_key(row[i], (uint32_t)i);
        best = key > best ? key : best;
    }
    red[threadIdx.x] = best;
    __syncthreads();
    for (int s = blockDim.x >> 1; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = red[threadIdx.x] > red[threadIdx.x + s] ? red[threadIdx.x] : red[threadIdx.x + s];
        __syncthreads();
    }
    if (threadIdx.x == 0) part[(size_t)blockIdx.y * nch + blockIdx.x] = red[0];
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const uint64_t* __restrict__ part, int nch,
                                                         int64_t* __restrict__ out) {
    uint64_t best = 0;
    for (int c = threadIdx.x; c < nch; c += 64) best = max(best, part[(size_t)blockIdx.x * nch + c]);
    best = wave_max_u64(best);
    if (threadIdx.x == 0) out[blockIdx.x] = (int64_t)(0xFFFFFFFFu - (uint32_t)(best & 0xFFFFFFFFu));
}

// One pass over `bytes` (a multiple of 16) of device memory: nontemporal
// 16-byte loads, four in flight per thread, grid-stride.  The thread's XOR of
// its words is stored only when it equals one arbitrary constant, so the
// loads cannot be dropped and at most a word is written.
__global__ __launch_bounds__(512) void read_probe_kernel(const uint4* __restrict__ p, size_t n16,
                                                         uint32_t* __restrict__ out) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const size_t tid = blockIdx.x * (size_t)blockDim.x + threadIdx.x;
    const size_t nthr = (size_t)gridDim.x * blockDim.x;
    uint32_t acc = 0;
    size_t i = tid;
    for (; i + 3 * nthr < n16; i += 4 * nthr) {
        v4u v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p + i + u * nthr));
#pragma unroll
        for (int u = 0; u < 4; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    for (; i < n16; i += nthr) {
        const uint4 v = p[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) out[0] = acc;
}

hipError_t read_probe(const void* p, size_t bytes, uint32_t* out, int cus, hipStream_t st) {
    read_probe_kernel<<<cus, 512, 0, st>>>(reinterpret_cast<const uint4*>(p), bytes / 16, out);
    return hipGetLastError();
}

hipError_t argmax_rows(const int32_t* v, int M, int n, int ldv, int64_t* out, uint64_t* part, hipStream_t st) {
    const int nch = (n + kArgChunk - 1) / kArgChunk;
    argmax_part_kernel<<<dim3(nch, M), kBlock, 0, st>>>(v, n, ldv, part, nch);
    argmax_final_kernel<<<M, 64, 0, st>>>(part, nch, out);
    return hipGetLastError();
}

}  // namespace myl
