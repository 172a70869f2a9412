// fixed.h -- integer fixed-point primitives of the theta_v numeric contract,
// for device (and host) code of the HIP library.
//
// Semantics are those of the reference Rust kernels compiled in release mode
// (INTEGER_LLM/kernels/src/fixed_point.rs): + - * wrap, `as` truncates and
// shift amounts are masked to the operand width.  Nothing here uses floating
// point: integer division is done by shift-and-subtract or by a reciprocal
// computed that way, so no v_rcp_f32 sequence enters an integer kernel.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define MYL_FN __host__ __device__ static inline

typedef __int128 myl_i128;
typedef unsigned __int128 myl_u128;

MYL_FN int32_t shl32(int32_t v, uint32_t s) { return (int32_t)((uint32_t)v << (s & 31u)); }
MYL_FN int32_t shr32(int32_t v, uint32_t s) { return v >> (s & 31u); }
MYL_FN int64_t shl64(int64_t v, uint32_t s) { return (int64_t)((uint64_t)v << (s & 63u)); }
MYL_FN int64_t shr64(int64_t v, uint32_t s) { return v >> (s & 63u); }
MYL_FN myl_i128 shl128(myl_i128 v, uint32_t s) { return (myl_i128)((myl_u128)v << (s & 127u)); }
MYL_FN myl_i128 shr128(myl_i128 v, uint32_t s) { return v >> (s & 127u); }
MYL_FN int32_t wadd32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
MYL_FN int32_t wsub32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
MYL_FN int32_t wmul32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
MYL_FN int64_t wadd64(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
MYL_FN int64_t wmul64(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }

// fixed_point.rs:15-35
MYL_FN int16_t clamp_i16(int32_t x) { return x < -32768 ? (int16_t)-32768 : (x > 32767 ? (int16_t)32767 : (int16_t)x); }
MYL_FN int16_t clamp_i16_i64(int64_t x) { return x < -32768 ? (int16_t)-32768 : (x > 32767 ? (int16_t)32767 : (int16_t)x); }
MYL_FN int32_t clamp_i32_i64(int64_t x) { return x < (int64_t)INT32_MIN ? INT32_MIN : (x > (int64_t)INT32_MAX ? INT32_MAX : (int32_t)x); }

// fixed_point.rs:39-53: arithmetic right shift, round half to even.
MYL_FN int32_t rshift_round32(int32_t value, uint8_t shift) {
    if (shift == 0) return value;
    int32_t mask = wsub32(shl32(1, shift), 1);
    int32_t half = shl32(1, (uint8_t)(shift - 1));
    int32_t q = shr32(value, shift);
    int32_t r = value & mask;
    return (r > half || (r == half && (q & 1))) ? wadd32(q, 1) : q;
}

// fixed_point.rs:57-71
MYL_FN int64_t rshift_round64(int64_t value, uint8_t shift) {
    if (shift == 0) return value;
    int64_t mask = (int64_t)((uint64_t)shl64(1, shift) - 1u);
    int64_t half = shl64(1, (uint8_t)(shift - 1));
    int64_t q = shr64(value, shift);
    int64_t r = value & mask;
    return (r > half || (r == half && (q & 1))) ? wadd64(q, 1) : q;
}

// fixed_point.rs:155-169
MYL_FN myl_i128 rshift_round128(myl_i128 value, uint32_t shift) {
    if (shift == 0) return value;
    myl_i128 mask = (myl_i128)((myl_u128)shl128(1, shift) - 1u);
    myl_i128 half = shl128(1, shift - 1u);
    myl_i128 q = shr128(value, shift);
    myl_i128 r = value & mask;
    return (r > half || (r == half && (q & 1))) ? (myl_i128)((myl_u128)q + 1u) : q;
}

// fixed_point.rs:173-191: shift = in_frac as i8 - out_frac as i8 (wrapping);
// a negative shift is an unrounded, wrapping left shift.
MYL_FN int32_t rescale32(int32_t acc, uint8_t in_frac, uint8_t out_frac) {
    int8_t sh = (int8_t)(uint8_t)((int8_t)in_frac - (int8_t)out_frac);
    return sh >= 0 ? rshift_round32(acc, (uint8_t)sh) : shl32(acc, (uint8_t)(-(int32_t)sh));
}
MYL_FN int64_t rescale64(int64_t acc, uint8_t in_frac, uint8_t out_frac) {
    int8_t sh = (int8_t)(uint8_t)((int8_t)in_frac - (int8_t)out_frac);
    return sh >= 0 ? rshift_round64(acc, (uint8_t)sh) : shl64(acc, (uint8_t)(-(int32_t)sh));
}

// floor(2^32 / d) for d >= 1 (2^33 - 1 for d = 0), by restoring long
// division (integer only).  The dividend 2^32 has its only set bit at
// position 32, so the quotient bits above position 32 - ceil(log2 d) are zero
// and the remainder entering that position is 2^(ceil(log2 d) - 1): the loop
// starts there (33 - ceil(log2 d) steps instead of 33).  For d >= 2 the
// quotient fits 32 bits and the remainder stays below d, so each step runs
// on 32-bit words: the doubled remainder's 33rd bit is the old top bit, and
// when it is set the difference 2r - d (below d) is exact modulo 2^32.
MYL_FN uint64_t recip32(uint32_t d) {
    if (d <= 1) return d == 0 ? 0x1FFFFFFFFull : 0x100000000ull;
    const int c = 32 - __builtin_clz(d - 1u);  // ceil(log2 d), 1..32
    uint32_t q = 0, r = 1u << (c - 1);
    for (int bit = 32 - c; bit >= 0; --bit) {
        const bool carry = (int32_t)r < 0;
        const uint32_t r2 = r << 1;
        const bool take = carry || r2 >= d;
        r = take ? r2 - d : r2;
        q = (q << 1) | (take ? 1u : 0u);
    }
    return q;
}

// Unsigned n / d with the reciprocal m = recip32(d): at most one correction
// (m = 2^32/d - e with 0 <= e < 1 and n < 2^32 put n*m/2^32 in (n/d - 1, n/d]).
MYL_FN void udivmod32(uint32_t n, uint32_t d, uint64_t m, uint32_t* q, uint32_t* r) {
    uint64_t q0 = ((uint64_t)n * m) >> 32;
    uint64_t rem = (uint64_t)n - q0 * (uint64_t)d;
    if (rem >= d) { q0 += 1; rem -= d; }
    *q = (uint32_t)q0;
    *r = (uint32_t)rem;
}

// softmax.rs:50-63 for one element: Rust i32 `/` and `%` (truncating), then
// round to nearest, ties to even.  recip = recip32(|s|).
MYL_FN int32_t softmax_div_round(int32_t num, int32_t s, uint64_t recip) {
    uint32_t un = num < 0 ? 0u - (uint32_t)num : (uint32_t)num;
    uint32_t us = s < 0 ? 0u - (uint32_t)s : (uint32_t)s;
    uint32_t uq, ur;
    udivmod32(un, us, recip, &uq, &ur);
    bool neg_q = (num < 0) != (s < 0);
    int32_t q = neg_q ? (int32_t)(0u - uq) : (int32_t)uq;
    int32_t r = num < 0 ? (int32_t)(0u - ur) : (int32_t)ur;
    int32_t ra = r < 0 ? (int32_t)(0u - (uint32_t)r) : r;
    int32_t twice = wmul32(ra, 2);
    int32_t den_abs = (int32_t)us;
    if (twice > den_abs || (twice == den_abs && (q & 1)))
        return ((num > 0) == (s > 0)) ? wadd32(q, 1) : wsub32(q, 1);
    return q;
}

// softmax_div_round for 0 <= num < 2^31 and s >= 1 with one 32-bit reciprocal
// m = min(floor(2^32 / s), 2^32 - 1): q0 = (num * m) >> 32 is q or q - 1
// (num * m / 2^32 > num / s - 1 for num < 2^32), one correction gives the
// truncating quotient and remainder, then the same half-even step with the
// same wrapping i32 doubling of the remainder.
MYL_FN uint32_t recip32_u32(uint32_t s) {
    const uint64_t m = recip32(s);
    return m > 0xFFFFFFFFull ? 0xFFFFFFFFu : (uint32_t)m;
}
MYL_FN int32_t softmax_div_round_pos(int32_t num, int32_t s, uint32_t m) {
    const uint32_t un = (uint32_t)num, us = (uint32_t)s;
    uint32_t q = (uint32_t)(((uint64_t)un * m) >> 32);
    uint32_t r = un - q * us;
    if (r >= us) {
        q += 1;
        r -= us;
    }
    const int32_t twice = wmul32((int32_t)r, 2);
    if (twice > s || (twice == s && (q & 1u))) return wadd32((int32_t)q, 1);
    return (int32_t)q;
}

// Unsigned 32-bit n % d without a hardware divide (small loops only: LUT row
// selection pos % n_pos, done once per launch).
MYL_FN uint32_t umod32_slow(uint32_t n, uint32_t d) {
    uint64_t m = recip32(d);
    uint32_t q, r;
    udivmod32(n, d, m, &q, &r);
    return r;
}

// integer_math.rs:44-48 with shift 0: index arithmetic in i16 (wrapping).
MYL_FN int16_t lut_lookup_i16(int16_t x, const int16_t* lut, uint32_t len, int16_t offset) {
    int16_t idx = (int16_t)(uint16_t)((uint16_t)x + (uint16_t)offset);
    int16_t hi = (int16_t)(uint16_t)((uint16_t)len - 1u);
    if (idx < 0) idx = 0;
    if (idx > hi) idx = hi;
    return lut[(uint16_t)idx];
}

// ---- integer log-softmax (build-defined; the reference computes it in f64,
// runtime/src/bin/perplexity_probe.rs:55-67) ------------------------------------
//
// log2(S) for S >= 1 as (e, f): e = floor(log2 S) and f the first 16 fraction
// bits of log2(S / 2^e), by repeated squaring of the Q62 mantissa (the binary
// logarithm algorithm: squaring doubles the logarithm, an overflow past 2
// emits a 1 bit).  Integer only; the same on every machine.
MYL_FN void log2_q16(uint64_t S, int32_t* e_out, uint32_t* f_out) {
    if (S == 0) S = 1;
    int32_t e = 63;
    while (!(S >> e)) --e;
    uint64_t x = S << (62 - e);  // S < 2^63, so e <= 62: x in [2^62, 2^63)
    uint32_t f = 0;
    for (int i = 0; i < 16; ++i) {
        x = (uint64_t)(((myl_u128)x * (myl_u128)x) >> 62);  // in [2^62, 2^64)
        f <<= 1;
        if (x >> 63) { x >>= 1; f |= 1u; }
    }
    *e_out = e;
    *f_out = f;
}

// ln(S / 2^14) in Q16: RNE((((e - 14) << 16) + f) * round(ln 2 * 2^30), 30).
#define MYL_LN2_Q30 744261118LL
MYL_FN int64_t ln_q16_of_sum(uint64_t S) {
    int32_t e;
    uint32_t f;
    log2_q16(S, &e, &f);
    const int64_t v = (int64_t)(e - 14) * 65536 + (int64_t)f;
    return rshift_round64(wmul64(v, MYL_LN2_Q30), 30);
}

