// ops.h -- integer kernels of the forward path other than the GEMV.
//
// Each kernel restates one reference function (cited at the kernel) and is
// exact: results equal the reference bit for bit, whatever the launch shape.
#pragma once

#include "fixed.h"
#include "wave.h"

namespace myl {

constexpr int kBlock = 256;

// ---- block reductions -------------------------------------------------------

// The slots are read in parallel (lane l, slot l) and reduced again across
// the wave, not one LDS read and wait per slot.
__device__ inline int32_t block_max_i32(int32_t v, int32_t* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    v = l < nw ? red[l] : INT32_MIN;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ inline uint32_t block_sum_u32(uint32_t v, uint32_t* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, 64);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6, l = threadIdx.x & 63;
    __syncthreads();
    if (l == 0) red[w] = v;
    __syncthreads();
    v = l < nw ? red[l] : 0u;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += (uint32_t)__shfl_xor((int)v, off, 64);
    return v;
}

// Exact i128 sum over the block (tree in LDS; red holds blockDim.x entries).
__device__ inline myl_i128 block_sum_i128(myl_i128 v, myl_i128* red) {
    __syncthreads();
    red[threadIdx.x] = v;
    __syncthreads();
    for (int s = blockDim.x >> 1; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) red[threadIdx.x] = (myl_i128)((myl_u128)red[threadIdx.x] + (myl_u128)red[threadIdx.x + s]);
        __syncthreads();
    }
    return red[0];
}

// ---- rmsnorm.rs:61-161 --------------------------------------------------------

struct RmsParams {
    const int16_t* lut; int lut_len;
    uint8_t lut_input_shift, lut_output_frac;
    int64_t inv_n_q20;
    // nonzero: every table entry equals rsqrt_closed(x, lut_output_frac,
    // lut_input_shift) (checked on the host when the table is set), so the
    // entry is computed instead of loaded
    uint8_t closed = 0;
};

// The closed form of the rsqrt table, round(2^f / sqrt(x / 2^s)) for x >= 1
// and 2^f at x = 0 (luts.py:32-49), in integer arithmetic: the result is the
// largest v >= 0 with v - 1/2 <= 2^f sqrt(2^s / x), i.e. with
// (2v - 1)^2 x <= 2^(2f + s + 2), found by bisection.  Exact ties (where the
// reference's half-even rounding would decide) need x = 2^(2f + s + 2) with
// v = 1; the host check against the table covers them.  f + s / 2 <= 20.
MYL_FN int32_t rsqrt_closed(uint32_t x, uint32_t f, uint32_t s) {
    if (x == 0) return (int32_t)(1u << f);
    const uint32_t e = 2u * f + s + 2u;
    uint32_t lo = 0, hi = (1u << (f + (s + 1u) / 2u)) + 1u;  // v(lo) holds, v(hi) fails
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        const uint64_t t = 2ull * mid - 1ull;
        if (t * t * (uint64_t)x <= (1ull << e)) lo = mid; else hi = mid;
    }
    return (int32_t)lo;
}

__device__ inline int64_t rms_lut_value(const RmsParams& p, int idx) {
    return p.closed ? (int64_t)rsqrt_closed((uint32_t)idx, p.lut_output_frac, p.lut_input_shift) : (int64_t)p.lut[idx];
}

// Norm factor of one row: everything except the per-channel output.
struct RmsFactor { bool zero; uint8_t ref_shift; int64_t lut_val; uint32_t norm_frac; };

__device__ inline uint32_t bitlen128(myl_u128 v) {
    const uint64_t hi = (uint64_t)(v >> 64), lo = (uint64_t)v;
    return hi ? 128u - (uint32_t)__builtin_clzll(hi) : (lo ? 64u - (uint32_t)__builtin_clzll(lo) : 0u);
}

// Where a row's rsqrt-table entry comes from: the table index of the mean
// square, and the even scale q that brought it into the table's range
// (rmsnorm.rs:96-126: mean = acc * inv_n >> 20, scaled down by the smallest
// even q until it indexes the table).
struct RmsIdx { bool zero; uint32_t q; int idx; };

// The same index in 64-bit arithmetic when the sum and m = (sum * inv_n) >> 20
// fit (always, for int16 inputs with fractional-bit spreads below 16): the
// i128 emulation is the slow part of the serial setup every block runs.
__device__ inline bool rms_index_u64(myl_i128 acc, const RmsParams& p, RmsIdx& r) {
    const uint64_t hi = (uint64_t)((myl_u128)acc >> 64), lo = (uint64_t)acc;
    if (hi != 0 || (lo >> 63) != 0) return false;
    const uint64_t ph = __umul64hi(lo, (uint64_t)p.inv_n_q20), pl = lo * (uint64_t)p.inv_n_q20;
    if ((ph >> 20) != 0 || p.inv_n_q20 < 0) return false;
    r.zero = lo == 0;
    r.q = 0;
    r.idx = 0;
    if (!r.zero) {
        const uint64_t m = (ph << 44) | (pl >> 20);
        const uint64_t max_idx = (uint64_t)(p.lut_len - 1);
        uint32_t q = 0;
        if (m > 0) {
            const uint32_t bm = 64u - (uint32_t)__builtin_clzll(m), bi = 64u - (uint32_t)__builtin_clzll(max_idx | 1u);
            if (bm > bi + 2) q = (bm - bi - 2) & ~1u;
        }
        while ((m >> q) > max_idx) q += 2;
        int64_t idx = rshift_round64((int64_t)m, (uint8_t)q);
        if (idx > (int64_t)max_idx) idx = (int64_t)max_idx;
        r.q = q;
        r.idx = (int)idx;
    }
    return true;
}

__device__ inline RmsIdx rms_index(myl_i128 acc, const RmsParams& p) {
    RmsIdx r;
    if (rms_index_u64(acc, p, r)) return r;
    r.zero = acc == 0;
    r.q = 0;
    r.idx = 0;
    if (!r.zero) {
        const myl_i128 m = shr128((myl_i128)((myl_u128)acc * (myl_u128)(myl_i128)p.inv_n_q20), 20);
        const myl_i128 max_idx = (myl_i128)(p.lut_len - 1);
        // rmsnorm.rs:121-123 searches the smallest even q with m >> q <= max_idx.
        // Every q below bitlen(m) - bitlen(max_idx) fails the test, so the
        // search may start just under that bound (same q, few iterations).
        uint32_t q = 0;
        if (m > 0) {
            const uint32_t bm = bitlen128((myl_u128)m), bi = bitlen128((myl_u128)max_idx);
            if (bm > bi + 2) q = (bm - bi - 2) & ~1u;
        }
        while (shr128(m, q) > max_idx) q += 2;
        myl_i128 idx = rshift_round128(m, q);
        if (idx > max_idx) idx = max_idx;
        if (idx < 0) idx = 0;
        r.q = q;
        r.idx = (int)idx;
    }
    return r;
}

__device__ inline RmsFactor rms_factor_at(const RmsIdx& r, uint8_t ref, const RmsParams& p, int64_t lut_val) {
    RmsFactor f;
    f.ref_shift = ref;
    f.zero = r.zero;
    f.lut_val = r.zero ? 0 : lut_val;
    f.norm_frac = r.zero ? 0u : (uint32_t)p.lut_output_frac + (uint32_t)p.lut_input_shift / 2u + r.q / 2u;
    return f;
}

// The factor from the aligned sum of squares acc and the largest input
// shift ref (rmsnorm.rs:96-126).
__device__ inline RmsFactor rms_factor_of(myl_i128 acc, uint8_t ref, const RmsParams& p) {
    const RmsIdx r = rms_index(acc, p);
    return rms_factor_at(r, ref, p, r.zero ? 0 : rms_lut_value(p, r.idx));
}

// rsqrt_closed computed by a whole wave: each round the 64 lanes test 64
// evenly spaced candidates of the remaining range [lo, hi) (v(lo) holds,
// v(hi) fails; the test is monotone in v), and the ballot's count moves lo
// and hi to the last holding and first failing candidate: three rounds for
// the theta_v table's 4097-wide range instead of twelve bisection steps.
// x, f, s uniform over the wave; every lane active.
__device__ inline int32_t rsqrt_closed_wave(uint32_t x, uint32_t f, uint32_t s) {
    if (x == 0) return (int32_t)(1u << f);
    const uint32_t e = 2u * f + s + 2u;
    const uint32_t lane = threadIdx.x & 63u;
    uint32_t lo = 0, hi = (1u << (f + (s + 1u) / 2u)) + 1u;
    while (hi - lo > 1u) {
        const uint32_t step = (hi - lo + 63u) >> 6;
        const uint32_t c = lo + step * (lane + 1u);
        const uint64_t t = 2ull * c - 1ull;
        const bool ok = c < hi && t * t * (uint64_t)x <= (1ull << e);
        const uint32_t k = (uint32_t)__popcll(__ballot(ok));
        const uint32_t nlo = lo + step * k;
        hi = min(hi, nlo + step);
        lo = nlo;
    }
    return (int32_t)lo;
}

// rms_factor_of computed by a whole wave (every lane active, acc uniform):
// the closed-form table entry by rsqrt_closed_wave.  Every lane gets the factor.
__device__ inline RmsFactor rms_factor_wave(myl_i128 acc, uint8_t ref, const RmsParams& p) {
    const RmsIdx r = rms_index(acc, p);
    int64_t v = 0;
    if (!r.zero)
        v = p.closed ? (int64_t)rsqrt_closed_wave((uint32_t)r.idx, p.lut_output_frac, p.lut_input_shift)
                     : (int64_t)p.lut[r.idx];
    return rms_factor_at(r, ref, p, v);
}

// Must be called by the whole block.  red128 needs blockDim.x entries.
__device__ inline RmsFactor rms_factor(const int16_t* x, const uint8_t* xs, int n, const RmsParams& p,
                                       myl_i128* red128, int32_t* red32) {
    int32_t mx = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) mx = max(mx, (int32_t)xs[i]);
    const uint8_t ref = (uint8_t)block_max_i32(mx, red32);
    myl_i128 acc = 0;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t align = 2u * (uint32_t)(uint8_t)(ref - xs[i]);
        const myl_i128 sq = (myl_i128)x[i] * (myl_i128)x[i];
        acc = (myl_i128)((myl_u128)acc + (myl_u128)shl128(sq, align));
    }
    acc = block_sum_i128(acc, red128);
    return rms_factor_of(acc, ref, p);
}

// RNE(v / 2^s) for 0 <= s <= 62 and |v| < 2^62, equal to rshift_round64 there:
// with v = q 2^s + r (0 <= r < 2^s), adding 2^(s-1) - 1 plus q's lowest bit
// carries into q exactly when r is above one half, or equal to it with q odd.
// About a quarter of rshift_round64's instructions (no remainder compares,
// no shift-range selects): the normalisation of a whole activation vector in
// every block of the decode products runs it per element.
MYL_FN int64_t rne_shift64_small(int64_t v, uint32_t s) {
    const int64_t lsb = (v >> s) & 1;
    const int64_t half = (int64_t)((1ull << s) >> 1);
    return (v + (s ? half - 1 + lsb : 0)) >> s;
}

// Per-channel output of rmsnorm.rs:130-159.  |x * lut * gamma| < 2^37, so for
// 0 <= shift <= 62 and for left shifts up to 25 bits the i64 computation is the
// i128 one bit for bit; other shifts take the i128 path.  (Branches: a lane
// computes only the form its shift needs; computing both and selecting
// measured slower in the decode staging.)
__device__ inline int16_t rms_out(int16_t x, uint8_t xs, int8_t g, uint8_t gs, const RmsFactor& f, uint8_t out_frac) {
    if (f.zero) return 0;
    const int32_t total = (int32_t)f.norm_frac + (int32_t)gs + ((int32_t)xs - (int32_t)f.ref_shift);
    const int32_t shift = total - (int32_t)out_frac;
    // |x * g| < 2^22 and the LUT value is an int16: one 32 x 32 -> 64 product
    const int64_t p64 = (int64_t)((int32_t)x * (int32_t)g) * (int64_t)(int32_t)f.lut_val;
    // clamp to i32 then to i16 is the clamp to i16
    if (shift >= 0 && shift <= 62) return clamp_i16_i64(rne_shift64_small(p64, (uint32_t)shift));
    if (shift < 0 && shift >= -25) return clamp_i16_i64(clamp_i32_i64(p64 << (-shift)));
    const myl_i128 prod = (myl_i128)p64;
    const myl_i128 s = shift >= 0 ? rshift_round128(prod, (uint32_t)shift) : shl128(prod, (uint32_t)(-shift));
    const int32_t c = s < (myl_i128)INT32_MIN ? INT32_MIN : (s > (myl_i128)INT32_MAX ? INT32_MAX : (int32_t)s);
    return clamp_i16(c);
}

// The aligned square x^2 << 2 (ref - xs) of rmsnorm.rs:96-110 split into
// three 42-bit limbs added to l: each limb of up to 2^22 terms fits a u64,
// so sums stay exact with 64-bit reductions, and the value mod 2^128 is
// l0 + l1 2^42 + l2 2^84 (limbs_value).
constexpr uint64_t kSqLimbMask = (1ull << 42) - 1;
__device__ inline void add_sq_limbs(int16_t x, uint8_t xs, uint8_t ref, uint64_t (&l)[3]) {
    const uint32_t align = 2u * (uint32_t)(uint8_t)(ref - xs);
    const myl_u128 t = (myl_u128)shl128((myl_i128)((int64_t)x * (int64_t)x), align);
    l[0] += (uint64_t)t & kSqLimbMask;
    l[1] += (uint64_t)(t >> 42) & kSqLimbMask;
    l[2] += (uint64_t)(t >> 84);
}
__device__ inline myl_i128 limbs_value(const uint64_t (&l)[3]) {
    return (myl_i128)((myl_u128)l[0] + ((myl_u128)l[1] << 42) + ((myl_u128)l[2] << 84));
}

// Exact i128 sum over a wave: 64-bit halves exchanged by shuffles, carry kept.
__device__ inline myl_i128 wave_sum_i128(myl_i128 v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const uint64_t lo = (uint64_t)(myl_u128)v, hi = (uint64_t)((myl_u128)v >> 64);
        const uint32_t l0 = (uint32_t)__shfl_xor((int)(uint32_t)lo, off, 64);
        const uint32_t l1 = (uint32_t)__shfl_xor((int)(uint32_t)(lo >> 32), off, 64);
        const uint32_t h0 = (uint32_t)__shfl_xor((int)(uint32_t)hi, off, 64);
        const uint32_t h1 = (uint32_t)__shfl_xor((int)(uint32_t)(hi >> 32), off, 64);
        const myl_u128 o = ((myl_u128)(((uint64_t)h1 << 32) | h0) << 64) | (((uint64_t)l1 << 32) | l0);
        v = (myl_i128)((myl_u128)v + o);
    }
    return v;
}

// Norm factor for blocks of up to 1024 threads where each thread holds PER
// elements (x, x_shift) in registers (invalid slots carry x = 0, xs = 0).
template <int PER>
__device__ inline RmsFactor rms_factor_regs(const int16_t (&x)[PER], const uint8_t (&xs)[PER], const RmsParams& p,
                                            myl_i128* red128, int32_t* red32) {
    int32_t mx = 0;
#pragma unroll
    for (int t = 0; t < PER; ++t) mx = max(mx, (int32_t)xs[t]);
    const uint8_t ref = (uint8_t)block_max_i32(mx, red32);
    myl_i128 acc = 0;
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const uint32_t align = 2u * (uint32_t)(uint8_t)(ref - xs[t]);
        const int64_t sq = (int64_t)x[t] * (int64_t)x[t];
        acc = (myl_i128)((myl_u128)acc + (myl_u128)shl128((myl_i128)sq, align));
    }
    acc = wave_sum_i128(acc);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red128[w] = acc;
    __syncthreads();
    acc = 0;
    for (int i = 0; i < nw; ++i) acc = (myl_i128)((myl_u128)acc + (myl_u128)red128[i]);
    return rms_factor_of(acc, ref, p);
}

// The same factor when the row's largest input shift ref is known (a
// per-layer constant of the channel scales): limb sums with 64-bit wave
// reductions instead of the i128 shuffles and the block maximum (one
// 1024-thread row finish on MI355X: 9.8 -> 7.2 us).  red: blockDim.x / 64
// entries, sf: one entry, both in LDS.  Whole block.
template <int PER>
__device__ inline RmsFactor rms_factor_limbs(const int16_t (&x)[PER], const uint8_t (&xs)[PER], uint8_t ref,
                                             const RmsParams& p, uint64_t (*red)[3], RmsFactor* sf) {
    uint64_t l[3] = {0, 0, 0};
#pragma unroll
    for (int t = 0; t < PER; ++t) add_sq_limbs(x[t], xs[t], ref, l);
#pragma unroll
    for (int j = 0; j < 3; ++j) l[j] = wave_sum_u64(l[j]);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
    if ((threadIdx.x & 63) == 0)
        for (int j = 0; j < 3; ++j) red[w][j] = l[j];
    __syncthreads();
    if (threadIdx.x < 64) {  // wave 0, every lane: the table entry is a wave-wide search
#pragma unroll
        for (int j = 0; j < 3; ++j) l[j] = wave_sum_u64((int)threadIdx.x < nw ? red[threadIdx.x][j] : 0);
        const RmsFactor f = rms_factor_wave(limbs_value(l), ref, p);
        if (threadIdx.x == 0) *sf = f;
    }
    __syncthreads();
    return *sf;
}

// ---- softmax.rs:12-64 ----------------------------------------------------------

__device__ inline int32_t exp_lookup(int32_t x, const int16_t* lut, uint32_t len, uint8_t shift, int32_t one) {
    if (x <= 0) return one;
    const uint32_t idx = (uint32_t)x >> (shift & 31u);
    if (idx >= len) return 0;
    return (int32_t)lut[idx];
}

__device__ inline int32_t sat_sub32(int32_t a, int32_t b) {
    const int64_t d = (int64_t)a - (int64_t)b;
    return d > INT32_MAX ? INT32_MAX : (d < INT32_MIN ? INT32_MIN : (int32_t)d);
}

}  // namespace myl
