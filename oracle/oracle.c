/*
 * oracle.c -- CPU restatement of the INTEGER_LLM integer forward path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker; see oracle.h).  Plain C99 + gcc's
 * __int128.  Release-mode Rust semantics throughout:
 *   - i32/i64/i128 + - * wrap (computed in unsigned arithmetic here),
 *   - `x << s` / `x >> s` mask s to the operand width (s & 31, & 63, & 127),
 *   - `as` truncates,
 *   - i8 differences of fractional bits wrap.
 */
#include "oracle.h"
#include "../include/myl_synth.h"

#include <stdlib.h>
#include <string.h>

typedef __int128 i128;
typedef unsigned __int128 u128;

static int g_threads = 1;
void or_set_threads(int n) { g_threads = n < 1 ? 1 : n; }

/* Dot-product form: 0 = the scalar i64 loop of dot.rs:141-147 (the reference
 * backend), 1 = i32 blocks drained to i64 (the cpu-simd backend's scheme,
 * dot.rs:175-221).  Both are exact, so every result is the same. */
static int g_simd = 1;
void or_set_simd(int on) { g_simd = on != 0; }

/* ---- release-mode shift helpers ---------------------------------------- */
static inline int32_t shl32(int32_t v, uint32_t s) { return (int32_t)((uint32_t)v << (s & 31u)); }
static inline int32_t shr32(int32_t v, uint32_t s) { return v >> (s & 31u); }
static inline int64_t shl64(int64_t v, uint32_t s) { return (int64_t)((uint64_t)v << (s & 63u)); }
static inline int64_t shr64(int64_t v, uint32_t s) { return v >> (s & 63u); }
static inline i128 shl128(i128 v, uint32_t s) { return (i128)((u128)v << (s & 127u)); }
static inline i128 shr128(i128 v, uint32_t s) { return v >> (s & 127u); }
static inline int32_t add32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a + (uint32_t)b); }
static inline int32_t sub32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a - (uint32_t)b); }
static inline int32_t mul32(int32_t a, int32_t b) { return (int32_t)((uint32_t)a * (uint32_t)b); }
static inline int64_t add64(int64_t a, int64_t b) { return (int64_t)((uint64_t)a + (uint64_t)b); }
static inline int64_t mul64(int64_t a, int64_t b) { return (int64_t)((uint64_t)a * (uint64_t)b); }

/* ---- fixed_point.rs ----------------------------------------------------- */

/* fixed_point.rs:7-11 */
int8_t or_clamp_i8(int32_t x) { return x < -128 ? -128 : (x > 127 ? 127 : (int8_t)x); }
/* fixed_point.rs:15-19 */
int16_t or_clamp_i16(int32_t x) { return x < -32768 ? -32768 : (x > 32767 ? 32767 : (int16_t)x); }
/* fixed_point.rs:23-27 */
int16_t or_clamp_i16_from_i64(int64_t x) { return x < -32768 ? -32768 : (x > 32767 ? 32767 : (int16_t)x); }
/* fixed_point.rs:31-35 */
int32_t or_clamp_i32(int64_t x) { return x < INT32_MIN ? INT32_MIN : (x > INT32_MAX ? INT32_MAX : (int32_t)x); }

/* fixed_point.rs:39-53: arithmetic right shift, round half to even. */
int32_t or_rshift_round(int32_t value, uint8_t shift) {
    if (shift == 0) return value;
    int32_t mask = sub32(shl32(1, shift), 1);
    int32_t half = shl32(1, (uint8_t)(shift - 1));
    int32_t q = shr32(value, shift);
    int32_t r = value & mask;
    if (r > half || (r == half && (q & 1) != 0)) return add32(q, 1);
    return q;
}

/* fixed_point.rs:57-71 */
int64_t or_rshift_round_i64(int64_t value, uint8_t shift) {
    if (shift == 0) return value;
    int64_t mask = (int64_t)((uint64_t)shl64(1, shift) - 1u);
    int64_t half = shl64(1, (uint8_t)(shift - 1));
    int64_t q = shr64(value, shift);
    int64_t r = value & mask;
    if (r > half || (r == half && (q & 1) != 0)) return add64(q, 1);
    return q;
}

/* fixed_point.rs:155-169 */
static i128 rshift_round_i128(i128 value, uint32_t shift) {
    if (shift == 0) return value;
    i128 mask = (i128)((u128)shl128(1, shift) - 1u);
    i128 half = shl128(1, shift - 1u);
    i128 q = shr128(value, shift);
    i128 r = value & mask;
    if (r > half || (r == half && (q & 1) != 0)) return (i128)((u128)q + 1u);
    return q;
}

void or_rshift_round_i128(int64_t hi, uint64_t lo, uint32_t shift, int64_t* out_hi, uint64_t* out_lo) {
    i128 v = (i128)(((u128)(uint64_t)hi << 64) | (u128)lo);
    i128 r = rshift_round_i128(v, shift);
    *out_hi = (int64_t)(r >> 64);
    *out_lo = (uint64_t)r;
}

/* fixed_point.rs:173-180: shift = in_frac as i8 - out_frac as i8. */
int32_t or_rescale(int32_t acc, uint8_t in_frac, uint8_t out_frac) {
    int8_t shift = (int8_t)(uint8_t)((int8_t)in_frac - (int8_t)out_frac);
    if (shift >= 0) return or_rshift_round(acc, (uint8_t)shift);
    return shl32(acc, (uint8_t)(-(int32_t)shift));
}

/* fixed_point.rs:184-191 */
int64_t or_rescale_i64(int64_t acc, uint8_t in_frac, uint8_t out_frac) {
    int8_t shift = (int8_t)(uint8_t)((int8_t)in_frac - (int8_t)out_frac);
    if (shift >= 0) return or_rshift_round_i64(acc, (uint8_t)shift);
    return shl64(acc, (uint8_t)(-(int32_t)shift));
}

/* fixed_point.rs:117-146: Newton with monotone stop, then round. */
uint64_t or_isqrt_round(uint64_t n) {
    if (n == 0) return 0;
    uint64_t r = n;
    uint64_t next = n / 2 + (n & 1);
    while (next < r) {
        r = next;
        next = (r + n / r) / 2;
    }
    while (r > 0 && r > n / r) r -= 1;
    while ((r + 1) <= n / (r + 1)) r += 1;
    uint64_t below = n - r * r;
    uint64_t above = (r + 1) * (r + 1) - n;
    return above < below ? r + 1 : r;
}

/* fixed_point.rs:102-107 */
int64_t or_inv_sqrt_q15(size_t head_dim) {
    if (head_dim == 0) return -1;
    return (int64_t)or_isqrt_round((1ULL << 30) / (uint64_t)head_dim);
}

/* ---- dot.rs / linear.rs ------------------------------------------------- */

/* dot.rs:175-221: products summed in i32 over blocks of 256 elements, then
 * widened.  |w| <= 128 and |x| <= 32768 bound a block by 2^30 < 2^31, so no
 * i32 sum wraps and the total equals the scalar loop's (dot.rs:266-296). */
static int64_t dot_i8_i16_blocks(const int8_t* w, const int16_t* x, size_t n) {
    int64_t acc = 0;
    for (size_t i = 0; i < n; i += 256) {
        size_t e = n - i < 256 ? n : i + 256;
        int32_t s = 0;
        for (size_t j = i; j < e; ++j) s += (int32_t)w[j] * (int32_t)x[j];
        acc += s;
    }
    return acc;
}

/* dot.rs:141-147 (the numeric contract; any summation order is equal). */
int64_t or_dot_i8_i16(const int8_t* w, const int16_t* x, size_t n) {
    if (g_simd) return dot_i8_i16_blocks(w, x, n);
    uint64_t acc = 0;
    for (size_t i = 0; i < n; ++i) acc += (uint64_t)((int64_t)w[i] * (int64_t)x[i]);
    return (int64_t)acc;
}

/* linear.rs:43-70 */
int or_linear_w8a16(const int16_t* x, const int8_t* W, size_t in_features,
                    const uint8_t* w_shifts, size_t out_features,
                    uint8_t act_frac, uint8_t out_frac, int16_t* out) {
    if (in_features == 0) return -1; /* chunks_exact(0) panics */
    long long N = (long long)out_features;
#pragma omp parallel for if (g_threads > 1 && N > 64) num_threads(g_threads) schedule(static)
    for (long long r = 0; r < N; ++r) {
        int64_t acc = or_dot_i8_i16(W + (size_t)r * in_features, x, in_features);
        int64_t y = or_rescale_i64(acc, (uint8_t)(w_shifts[r] + act_frac), out_frac);
        out[r] = or_clamp_i16_from_i64(y);
    }
    return 0;
}

/* linear.rs:87-119 */
int or_linear_w8a16_pc(const int16_t* x, const int8_t* W, size_t in_features,
                       const uint8_t* w_shifts, size_t out_features,
                       uint8_t act_frac, const uint8_t* out_frac, int16_t* out) {
    if (in_features == 0) return -1;
    long long N = (long long)out_features;
#pragma omp parallel for if (g_threads > 1 && N > 64) num_threads(g_threads) schedule(static)
    for (long long r = 0; r < N; ++r) {
        int64_t acc = or_dot_i8_i16(W + (size_t)r * in_features, x, in_features);
        int64_t y = or_rescale_i64(acc, (uint8_t)(w_shifts[r] + act_frac), out_frac[r]);
        out[r] = or_clamp_i16_from_i64(y);
    }
    return 0;
}

/* linear.rs:132-145 */
int or_add_bias_i16(int16_t* out, const int16_t* bias, const uint8_t* bias_shifts,
                    size_t n, uint8_t out_frac) {
    for (size_t i = 0; i < n; ++i) {
        int32_t b = or_rescale((int32_t)bias[i], bias_shifts[i], out_frac);
        out[i] = or_clamp_i16_from_i64((int64_t)out[i] + (int64_t)b);
    }
    return 0;
}

int or_linear_w8a16_batch(const int16_t* x, size_t M, const int8_t* W, size_t N, size_t K,
                          const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac,
                          const uint8_t* out_frac_pc, int16_t* out) {
    for (size_t m = 0; m < M; ++m) {
        int rc = out_frac_pc
            ? or_linear_w8a16_pc(x + m * K, W, K, w_shifts, N, act_frac, out_frac_pc, out + m * N)
            : or_linear_w8a16(x + m * K, W, K, w_shifts, N, act_frac, out_frac, out + m * N);
        if (rc) return rc;
    }
    return 0;
}

/* Build-defined multiplier requant of one sum: clamp16(RNE(acc * mult, shift))
 * in 128 bits.  With mult = 2^k and shift = k + s_ref it equals
 * linear_w8a16's rescale by s_ref >= 0 (the identity proved by
 * fixed_point.rs:364-379). */
static int16_t requant_mult(int64_t acc, int32_t mult, uint8_t shift) {
    i128 y = rshift_round_i128((i128)acc * (i128)mult, shift);
    return y < -32768 ? -32768 : (y > 32767 ? 32767 : (int16_t)y);
}

int or_linear_w8a16_mult(const int16_t* x, size_t M, const int8_t* W, size_t N, size_t K,
                         const int32_t* mult, const uint8_t* shift, int16_t* out) {
    if (K == 0) return -1;
    for (size_t m = 0; m < M; ++m) {
        long long NN = (long long)N;
#pragma omp parallel for if (g_threads > 1 && NN > 64) num_threads(g_threads) schedule(static)
        for (long long r = 0; r < NN; ++r)
            out[m * N + (size_t)r] = requant_mult(or_dot_i8_i16(W + (size_t)r * K, x + m * K, K), mult[r], shift[r]);
    }
    return 0;
}

/* The requant step of linear_w8a16 (linear.rs:61-68) and of the multiplier
 * form on sums computed elsewhere: acc [M x N] exact i64 dot products. */
int or_requant_shift(const int64_t* acc, size_t M, size_t N, const uint8_t* w_shifts, uint8_t act_frac,
                     uint8_t out_frac, int16_t* out) {
    long long n = (long long)(M * N);
#pragma omp parallel for if (g_threads > 1 && n > 4096) num_threads(g_threads) schedule(static)
    for (long long i = 0; i < n; ++i) {
        size_t r = (size_t)i % N;
        out[i] = or_clamp_i16_from_i64(or_rescale_i64(acc[i], (uint8_t)(w_shifts[r] + act_frac), out_frac));
    }
    return 0;
}

int or_requant_mult(const int64_t* acc, size_t M, size_t N, const int32_t* mult, const uint8_t* shift, int16_t* out) {
    long long n = (long long)(M * N);
#pragma omp parallel for if (g_threads > 1 && n > 4096) num_threads(g_threads) schedule(static)
    for (long long i = 0; i < n; ++i) {
        size_t r = (size_t)i % N;
        out[i] = requant_mult(acc[i], mult[r], shift[r]);
    }
    return 0;
}

/* ---- rmsnorm.rs --------------------------------------------------------- */

/* rmsnorm.rs:20-23 */
int64_t or_inv_n_q20(size_t n) {
    if (n == 0) return -1;
    return ((1LL << 20) + (int64_t)n / 2) / (int64_t)n;
}

/* rmsnorm.rs:61-161 */
int or_rmsnorm_i16(const int16_t* x, const uint8_t* x_shifts, const int8_t* gamma,
                   const uint8_t* gamma_shifts, size_t n, const int16_t* rsqrt_lut,
                   size_t lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                   int64_t inv_n_q20, uint8_t out_frac, int16_t* out) {
    if (n == 0) return -1;                    /* max() of empty x_shifts panics (:96) */
    if (lut_input_shift % 2 != 0) return -1;  /* :76 */
    if (lut_len < 2) return -1;               /* the even-shift search needs max_idx >= 1 */
    uint8_t ref_shift = 0;
    for (size_t i = 0; i < n; ++i) if (x_shifts[i] > ref_shift) ref_shift = x_shifts[i];

    i128 acc = 0;
    for (size_t i = 0; i < n; ++i) {
        uint32_t align = 2u * (uint32_t)(uint8_t)(ref_shift - x_shifts[i]);
        i128 sq = (i128)x[i] * (i128)x[i];
        acc = (i128)((u128)acc + (u128)shl128(sq, align));
    }
    if (acc == 0) {
        memset(out, 0, n * sizeof(int16_t));
        return 0;
    }
    i128 m = shr128((i128)((u128)acc * (u128)(i128)inv_n_q20), 20);
    i128 max_idx = (i128)(lut_len - 1);
    uint32_t q = 0;
    while (shr128(m, q) > max_idx) q += 2;
    i128 idx = rshift_round_i128(m, q);
    if (idx > max_idx) idx = max_idx;
    if (idx < 0) idx = 0;
    int64_t lut_val = (int64_t)rsqrt_lut[(size_t)idx];
    uint32_t norm_frac = (uint32_t)lut_output_frac + (uint32_t)lut_input_shift / 2u + q / 2u;

    for (size_t i = 0; i < n; ++i) {
        int32_t total_frac = (int32_t)norm_frac + (int32_t)gamma_shifts[i]
                           + ((int32_t)x_shifts[i] - (int32_t)ref_shift);
        int32_t shift = total_frac - (int32_t)out_frac;
        i128 prod = (i128)x[i] * (i128)lut_val * (i128)gamma[i];
        i128 s = shift >= 0 ? rshift_round_i128(prod, (uint32_t)shift)
                            : shl128(prod, (uint32_t)(-shift));
        int32_t c = s < (i128)INT32_MIN ? INT32_MIN : (s > (i128)INT32_MAX ? INT32_MAX : (int32_t)s);
        out[i] = or_clamp_i16(c);
    }
    return 0;
}

/* ---- rope.rs ------------------------------------------------------------ */

/* rope.rs:17-31: half-split pairs (x_j, x_{j+half}), i32 arithmetic. */
int or_rotate_half_split_i16(const int16_t* vec, size_t head_dim, const int16_t* cos_row,
                             const int16_t* sin_row, uint8_t frac_bits, int16_t* out) {
    size_t half = head_dim / 2;
    for (size_t j = 0; j < half; ++j) {
        int32_t c = cos_row[j], s = sin_row[j];
        int32_t x0 = vec[j], x1 = vec[j + half];
        out[j] = or_clamp_i16(or_rshift_round(sub32(mul32(x0, c), mul32(x1, s)), frac_bits));
        out[j + half] = or_clamp_i16(or_rshift_round(add32(mul32(x1, c), mul32(x0, s)), frac_bits));
    }
    if (head_dim & 1) out[head_dim - 1] = 0; /* vec![0; len]: an odd tail stays 0 */
    return 0;
}

/* rope.rs:36-59: LUT row = pos % n_pos, n_pos = lut_len / half. */
int or_apply_rope_i16(const int16_t* q, const int16_t* k, size_t n, size_t head_dim,
                      const int16_t* cos_lut, const int16_t* sin_lut, size_t lut_len,
                      const uint64_t* positions, uint8_t frac_bits,
                      int16_t* q_out, int16_t* k_out) {
    size_t half = head_dim / 2;
    if (half == 0) return -1;
    size_t n_pos = lut_len / half;
    if (n_pos == 0) return -1;
    for (size_t i = 0; i < n; ++i) {
        size_t idx = (size_t)(positions[i] % n_pos);
        or_rotate_half_split_i16(q + i * head_dim, head_dim, cos_lut + idx * half, sin_lut + idx * half, frac_bits, q_out + i * head_dim);
        or_rotate_half_split_i16(k + i * head_dim, head_dim, cos_lut + idx * half, sin_lut + idx * half, frac_bits, k_out + i * head_dim);
    }
    return 0;
}

/* ---- softmax.rs --------------------------------------------------------- */

/* softmax.rs:12-21 */
int32_t or_exp_lut_lookup(int32_t x, const int16_t* lut, size_t len, uint8_t lut_shift, int32_t one) {
    if (x <= 0) return one;
    uint32_t idx = (uint32_t)x >> (lut_shift & 31u);
    if ((size_t)idx >= len) return 0;
    return (int32_t)lut[idx];
}

static int32_t sat_sub32(int32_t a, int32_t b) {
    int64_t d = (int64_t)a - (int64_t)b;
    return d > INT32_MAX ? INT32_MAX : (d < INT32_MIN ? INT32_MIN : (int32_t)d);
}

/* Rust i32 `/` and `%` truncate toward zero; i32::MIN / -1 panics. */
static int softmax_div_round(int32_t num, int32_t s, int32_t* out) {
    if (s == 0 || (num == INT32_MIN && s == -1)) return -1;
    int32_t q = num / s;
    int32_t r = num % s;
    int32_t ra = r < 0 ? (int32_t)(0u - (uint32_t)r) : r;      /* abs wraps in release */
    int32_t twice = mul32(ra, 2);
    int32_t den_abs = s < 0 ? (int32_t)(0u - (uint32_t)s) : s;
    if (twice > den_abs || (twice == den_abs && (q & 1) != 0)) {
        *out = ((num > 0) == (s > 0)) ? add32(q, 1) : sub32(q, 1);
    } else {
        *out = q;
    }
    return 0;
}

/* softmax.rs:24-64 */
int or_softmax_int(const int32_t* logits, size_t n, const int16_t* exp_lut, size_t lut_len,
                   uint8_t lut_shift, uint8_t frac_bits, int32_t* out) {
    int32_t one = shl32(1, frac_bits);
    int32_t lut_one = lut_len > 0 ? (int32_t)exp_lut[0] : 1;
    int32_t m = 0;
    if (n > 0) { m = logits[0]; for (size_t i = 1; i < n; ++i) if (logits[i] > m) m = logits[i]; }
    int32_t s = 0;
    int32_t* e = (int32_t*)malloc((n ? n : 1) * sizeof(int32_t));
    if (!e) return -3;
    for (size_t i = 0; i < n; ++i) {
        e[i] = or_exp_lut_lookup(sat_sub32(m, logits[i]), exp_lut, lut_len, lut_shift, lut_one);
        s = add32(s, e[i]);
    }
    int rc = 0;
    if (s == 0) {
        if (n == 0) { free(e); return -1; } /* one / 0 panics */
        int32_t base = one / (int32_t)n;
        int32_t rem = sub32(one, mul32(base, (int32_t)n));
        for (size_t i = 0; i < n; ++i) out[i] = base + ((uint64_t)i < (uint64_t)(int64_t)rem ? 1 : 0);
    } else {
        for (size_t i = 0; i < n && rc == 0; ++i) rc = softmax_div_round(mul32(e[i], one), s, &out[i]);
    }
    free(e);
    return rc;
}

/* ---- attention.rs ------------------------------------------------------- */

/* attention.rs:21-27 */
int64_t or_dot_int(const int16_t* a, const int16_t* b, size_t n) {
    uint64_t acc = 0;
    for (size_t i = 0; i < n; ++i) acc += (uint64_t)((int64_t)a[i] * (int64_t)b[i]);
    return (int64_t)acc;
}

/* attention.rs:42-90 */
int or_attention_int(const int16_t* q, const int16_t* k, const int16_t* v,
                     const uint8_t* mask, size_t q_len, size_t kv_len, size_t head_dim,
                     int64_t score_mult, uint8_t score_shift, const int16_t* exp_lut,
                     size_t lut_len, uint8_t lut_shift, uint8_t prob_frac_bits,
                     int16_t* out) {
    if (kv_len == 0) return -1; /* v[0] panics */
    int32_t* scores = (int32_t*)malloc(kv_len * sizeof(int32_t));
    int32_t* probs = (int32_t*)malloc(kv_len * sizeof(int32_t));
    int64_t* row = (int64_t*)malloc((head_dim ? head_dim : 1) * sizeof(int64_t));
    if (!scores || !probs || !row) { free(scores); free(probs); free(row); return -3; }
    int rc = 0;
    for (size_t i = 0; i < q_len && rc == 0; ++i) {
        for (size_t j = 0; j < kv_len; ++j) {
            if (!mask || mask[i * kv_len + j]) {
                int64_t s = mul64(or_dot_int(q + i * head_dim, k + j * head_dim, head_dim), score_mult);
                scores[j] = (int32_t)or_rshift_round_i64(s, score_shift); /* `as i32` truncates */
            } else {
                scores[j] = INT32_MIN;
            }
        }
        rc = or_softmax_int(scores, kv_len, exp_lut, lut_len, lut_shift, prob_frac_bits, probs);
        if (rc) break;
        for (size_t d = 0; d < head_dim; ++d) row[d] = 0;
        for (size_t j = 0; j < kv_len; ++j) {
            if (probs[j] == 0) continue;
            for (size_t d = 0; d < head_dim; ++d)
                row[d] = add64(row[d], (int64_t)probs[j] * (int64_t)v[j * head_dim + d]);
        }
        for (size_t d = 0; d < head_dim; ++d)
            out[i * head_dim + d] = or_clamp_i16_from_i64(or_rshift_round_i64(row[d], prob_frac_bits));
    }
    free(scores); free(probs); free(row);
    return rc;
}

/* ---- integer_math.rs / mlp.rs / sampling.rs / prng.rs ------------------ */

/* integer_math.rs:44-48: index arithmetic in i16 (wrapping add). */
int16_t or_lut_lookup(int16_t x, const int16_t* lut, size_t len, uint8_t shift, int16_t offset) {
    int16_t idx = (int16_t)(uint16_t)((uint16_t)(int16_t)(x >> (shift & 15u)) + (uint16_t)offset);
    int16_t hi = (int16_t)(uint16_t)((uint16_t)(int16_t)(uint16_t)len - 1u);
    if (idx < 0) idx = 0;
    if (idx > hi) idx = hi;
    return lut[(size_t)(uint16_t)idx];
}

/* mlp.rs:28-74 */
int or_mlp_int(const int16_t* x, const int8_t* W_gate, const int8_t* W_up, const int8_t* W_down,
               size_t hidden, size_t inter, const uint8_t* gate_w_shifts,
               const uint8_t* up_w_shifts, const uint8_t* down_w_shifts,
               const int16_t* silu_lut, size_t silu_len, uint8_t in_frac,
               uint8_t gate_out_frac, uint8_t up_out_frac, uint8_t down_in_frac,
               uint8_t silu_in_frac, int16_t silu_lut_offset, uint8_t silu_out_frac,
               const uint8_t* out_frac, int16_t* out) {
    int16_t* gate = (int16_t*)malloc(inter * sizeof(int16_t));
    int16_t* up = (int16_t*)malloc(inter * sizeof(int16_t));
    int16_t* h = (int16_t*)malloc(inter * sizeof(int16_t));
    if (!gate || !up || !h) { free(gate); free(up); free(h); return -3; }
    int rc = or_linear_w8a16(x, W_gate, hidden, gate_w_shifts, inter, in_frac, gate_out_frac, gate);
    if (!rc) rc = or_linear_w8a16(x, W_up, hidden, up_w_shifts, inter, in_frac, up_out_frac, up);
    if (!rc) {
        for (size_t i = 0; i < inter; ++i) {
            int32_t g_dom = or_rescale((int32_t)gate[i], gate_out_frac, silu_in_frac);
            int16_t act = or_lut_lookup((int16_t)g_dom, silu_lut, silu_len, 0, silu_lut_offset);
            int64_t prod = (int64_t)act * (int64_t)up[i];
            h[i] = or_clamp_i16_from_i64(or_rescale_i64(prod, (uint8_t)(silu_out_frac + up_out_frac), down_in_frac));
        }
        rc = or_linear_w8a16_pc(h, W_down, inter, down_w_shifts, hidden, down_in_frac, out_frac, out);
    }
    free(gate); free(up); free(h);
    return rc;
}

/* sampling.rs:8-18: the first maximum wins. */
int64_t or_argmax_int(const int32_t* v, size_t n) {
    if (n == 0) return -1;
    size_t best = 0;
    int32_t bv = v[0];
    for (size_t i = 1; i < n; ++i) if (v[i] > bv) { bv = v[i]; best = i; }
    return (int64_t)best;
}

/* prng.rs:7-14 */
void or_splitmix64(uint64_t state, uint64_t* new_state, uint64_t* out) {
    uint64_t s = state + MYL_SM_GAMMA;
    *new_state = s;
    *out = myl_mix64(s);
}

/* sampling.rs:20-46: logits_to_weights (w_i = z_i - min + 1, i32 arithmetic
 * that wraps as in the reference's release build; no logits: min 0), the
 * total as i64, (token 0, state) when total <= 0, else one SplitMix64 draw r,
 * threshold r % total and the first i whose running sum exceeds it (the last
 * index when none does). */
void or_sample_integer_cdf(const int32_t* z, size_t n, uint64_t state, int64_t* token, uint64_t* new_state) {
    int32_t m = 0;
    if (n > 0) {
        m = z[0];
        for (size_t i = 1; i < n; ++i) if (z[i] < m) m = z[i];
    }
    int64_t total = 0;
    for (size_t i = 0; i < n; ++i) total += (int64_t)(int32_t)((uint32_t)z[i] - (uint32_t)m + 1u);
    if (total <= 0) {
        *token = 0;
        *new_state = state;
        return;
    }
    uint64_t r;
    or_splitmix64(state, new_state, &r);
    const int64_t threshold = (int64_t)(r % (uint64_t)total);
    int64_t acc = 0;
    for (size_t i = 0; i < n; ++i) {
        acc += (int64_t)(int32_t)((uint32_t)z[i] - (uint32_t)m + 1u);
        if (threshold < acc) {
            *token = (int64_t)i;
            return;
        }
    }
    *token = (int64_t)n - 1;
}

/* ---- integer log-softmax (build-defined) --------------------------------
 * The binary logarithm by repeated squaring: with x = S / 2^e in [1, 2),
 * log2(x^2) = 2 log2(x), so each squaring shifts the next fraction bit of
 * log2(x) into the integer part; a square >= 2 means that bit is 1 and is
 * halved back into [1, 2).  x is held in Q62 and each square truncated. */
void or_log2_q16(uint64_t S, int32_t* e_out, uint32_t* f_out) {
    if (S == 0) S = 1;
    int32_t e = 0;
    for (uint64_t t = S; t > 1; t >>= 1) ++e;
    uint64_t x = S << (62 - e);
    uint32_t f = 0;
    for (int i = 0; i < 16; ++i) {
        u128 sq = (u128)x * (u128)x;
        x = (uint64_t)(sq >> 62);
        f <<= 1;
        if (x >= (1ULL << 63)) { x >>= 1; f |= 1u; }
    }
    *e_out = e;
    *f_out = f;
}

int64_t or_ln_q16(uint64_t S) {
    int32_t e;
    uint32_t f;
    or_log2_q16(S, &e, &f);
    int64_t v = (int64_t)(e - 14) * 65536 + (int64_t)f;
    return or_rshift_round_i64(mul64(v, 744261118LL), 30);
}

int64_t or_logsoftmax_at(const int32_t* z, size_t n, const int16_t* exp_lut, size_t lut_len, int64_t target) {
    if (n == 0 || target < 0 || (uint64_t)target >= n) return 0;
    int32_t m = z[0];
    for (size_t j = 1; j < n; ++j) if (z[j] > m) m = z[j];
    int64_t S = 0;
    for (size_t j = 0; j < n; ++j) {
        uint64_t d = (uint64_t)((int64_t)m - (int64_t)z[j]) << 2;  /* Q6 logits -> Q8 LUT input */
        if (d < lut_len) S += exp_lut[d];
    }
    return ((int64_t)z[target] - (int64_t)m) * 1024 - or_ln_q16(S < 1 ? 1u : (uint64_t)S);
}

/* ---- model.rs / kv_cache.rs -------------------------------------------- */

typedef struct {
    int8_t *in_gamma, *post_gamma;
    uint8_t *in_gamma_shifts, *post_gamma_shifts;
    int8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    uint8_t *sq, *sk, *sv, *so, *sg, *su, *sd;
    int16_t *bq, *bk, *bv;
    uint8_t *bq_s, *bk_s, *bv_s;
    myl_layer_fracs f;
    uint8_t *res_in_frac, *res_mid_frac;
} or_layer;

struct or_model {
    myl_synth_spec spec;
    int8_t* emb; uint8_t* emb_shifts;
    int16_t* lm16; uint8_t* lm16_shifts;
    int8_t* final_gamma; uint8_t* final_gamma_shifts;
    uint8_t final_norm_frac; uint8_t* final_res_frac;
    int16_t *rsqrt, *silu, *exp_lut, *cos_lut, *sin_lut;
    size_t rsqrt_len, silu_len, exp_len, rope_len;
    int64_t inv_n_q20;
    or_layer* layers;
    int16_t *kcache, *vcache; /* [layer][kv_head][max_pos][head_dim] */
    uint32_t n_cached;
};

static void* xalloc(size_t bytes) { return malloc(bytes ? bytes : 1); }

static int8_t* gen_w8(uint64_t seed, uint32_t layer, uint32_t role, size_t n) {
    int8_t* p = (int8_t*)xalloc(n);
    if (!p) return NULL;
    uint64_t ts = myl_tensor_seed(seed, layer, role);
    long long nn = (long long)n;
#pragma omp parallel for schedule(static) if (nn > (1 << 20))
    for (long long i = 0; i < nn; ++i) p[i] = myl_synth_w8(ts, (uint64_t)i);
    return p;
}

static uint8_t* gen_wshift(uint64_t seed, uint32_t layer, uint32_t role, size_t rows, size_t K) {
    uint8_t* p = (uint8_t*)xalloc(rows);
    if (!p) return NULL;
    uint64_t ts = myl_tensor_seed(seed, layer, role);
    for (size_t r = 0; r < rows; ++r) p[r] = myl_synth_wshift(ts, r, K);
    return p;
}

static uint8_t* gen_small_u8(uint64_t seed, uint32_t layer, uint32_t role, size_t n) {
    uint8_t* p = (uint8_t*)xalloc(n);
    if (!p) return NULL;
    for (size_t i = 0; i < n; ++i) p[i] = (uint8_t)myl_synth_small(seed, layer, role, i);
    return p;
}

static int16_t* gen_small_i16(uint64_t seed, uint32_t layer, uint32_t role, size_t n) {
    int16_t* p = (int16_t*)xalloc(n * sizeof(int16_t));
    if (!p) return NULL;
    for (size_t i = 0; i < n; ++i) p[i] = (int16_t)myl_synth_small(seed, layer, role, i);
    return p;
}

static int16_t* dup16(const int16_t* src, size_t n) {
    int16_t* p = (int16_t*)xalloc(n * sizeof(int16_t));
    if (p && n) memcpy(p, src, n * sizeof(int16_t));
    return p;
}

void or_model_destroy(or_model* m) {
    if (!m) return;
    if (m->layers) {
        for (uint32_t l = 0; l < m->spec.layers; ++l) {
            or_layer* L = &m->layers[l];
            free(L->in_gamma); free(L->post_gamma); free(L->in_gamma_shifts); free(L->post_gamma_shifts);
            free(L->wq); free(L->wk); free(L->wv); free(L->wo); free(L->wg); free(L->wu); free(L->wd);
            free(L->sq); free(L->sk); free(L->sv); free(L->so); free(L->sg); free(L->su); free(L->sd);
            free(L->bq); free(L->bk); free(L->bv); free(L->bq_s); free(L->bk_s); free(L->bv_s);
            free(L->res_in_frac); free(L->res_mid_frac);
        }
        free(m->layers);
    }
    free(m->emb); free(m->emb_shifts); free(m->lm16); free(m->lm16_shifts);
    free(m->final_gamma); free(m->final_gamma_shifts); free(m->final_res_frac);
    free(m->rsqrt); free(m->silu); free(m->exp_lut); free(m->cos_lut); free(m->sin_lut);
    free(m->kcache); free(m->vcache);
    free(m);
}

or_model* or_model_create_synthetic(const myl_synth_spec* spec, const myl_luts* luts) {
    const myl_synth_spec s = *spec;
    if (!s.hidden || !s.layers || !s.heads || !s.kv_heads || !s.head_dim || !s.inter || !s.vocab) return NULL;
    if (s.heads % s.kv_heads != 0 || s.heads * s.head_dim != s.hidden || s.head_dim % 2) return NULL;
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    if (!m) return NULL;
    m->spec = s;
    const uint64_t seed = s.seed;
    const size_t H = s.hidden, I = s.inter, V = s.vocab, hd = s.head_dim;
    const size_t qN = (size_t)s.heads * hd, kvN = (size_t)s.kv_heads * hd;

    m->emb = gen_w8(seed, 0, MYL_R_EMB, V * H);
    m->emb_shifts = gen_small_u8(seed, 0, MYL_R_EMB_SHIFT, V);
    if (s.lm_head_int16) {
        m->lm16 = (int16_t*)xalloc(V * H * sizeof(int16_t));
        uint64_t ts = myl_tensor_seed(seed, 0, MYL_R_LM16);
        if (m->lm16) {
            long long n = (long long)(V * H);
#pragma omp parallel for schedule(static) if (n > (1 << 20))
            for (long long i = 0; i < n; ++i) m->lm16[i] = myl_synth_w16(ts, (uint64_t)i);
        }
        m->lm16_shifts = gen_small_u8(seed, 0, MYL_R_LM16_SHIFT, V);
    }
    m->final_gamma = gen_w8(seed, 0, MYL_R_FINAL_GAMMA, H);
    m->final_gamma_shifts = gen_small_u8(seed, 0, MYL_R_FINAL_GAMMA_SHIFT, H);
    m->final_norm_frac = myl_synth_final_norm_frac(seed);
    m->final_res_frac = (uint8_t*)xalloc(H);
    if (m->final_res_frac) {
        uint64_t ts = myl_tensor_seed(seed, 0, MYL_R_FINAL_RES_FRAC);
        for (size_t i = 0; i < H; ++i) m->final_res_frac[i] = myl_synth_res_frac(ts, i);
    }
    m->rsqrt = dup16(luts->rsqrt, luts->rsqrt_len); m->rsqrt_len = luts->rsqrt_len;
    m->silu = dup16(luts->silu, luts->silu_len); m->silu_len = luts->silu_len;
    m->exp_lut = dup16(luts->exp, luts->exp_len); m->exp_len = luts->exp_len;
    m->cos_lut = dup16(luts->cos, luts->rope_len); m->sin_lut = dup16(luts->sin, luts->rope_len);
    m->rope_len = luts->rope_len;
    m->inv_n_q20 = or_inv_n_q20(H);

    m->layers = (or_layer*)calloc(s.layers, sizeof(or_layer));
    if (!m->layers) { or_model_destroy(m); return NULL; }
    for (uint32_t l = 0; l < s.layers; ++l) {
        or_layer* L = &m->layers[l];
        L->in_gamma = gen_w8(seed, l, MYL_R_IN_GAMMA, H);
        L->in_gamma_shifts = gen_small_u8(seed, l, MYL_R_IN_GAMMA_SHIFT, H);
        L->post_gamma = gen_w8(seed, l, MYL_R_POST_GAMMA, H);
        L->post_gamma_shifts = gen_small_u8(seed, l, MYL_R_POST_GAMMA_SHIFT, H);
        L->wq = gen_w8(seed, l, MYL_R_WQ, qN * H);  L->sq = gen_wshift(seed, l, MYL_R_SQ, qN, H);
        L->wk = gen_w8(seed, l, MYL_R_WK, kvN * H); L->sk = gen_wshift(seed, l, MYL_R_SK, kvN, H);
        L->wv = gen_w8(seed, l, MYL_R_WV, kvN * H); L->sv = gen_wshift(seed, l, MYL_R_SV, kvN, H);
        L->wo = gen_w8(seed, l, MYL_R_WO, H * qN);  L->so = gen_wshift(seed, l, MYL_R_SO, H, qN);
        L->wg = gen_w8(seed, l, MYL_R_WG, I * H);   L->sg = gen_wshift(seed, l, MYL_R_SG, I, H);
        L->wu = gen_w8(seed, l, MYL_R_WU, I * H);   L->su = gen_wshift(seed, l, MYL_R_SU, I, H);
        L->wd = gen_w8(seed, l, MYL_R_WD, H * I);   L->sd = gen_wshift(seed, l, MYL_R_SD, H, I);
        if (s.attention_bias) {
            L->bq = gen_small_i16(seed, l, MYL_R_BQ, qN);
            L->bk = gen_small_i16(seed, l, MYL_R_BK, kvN);
            L->bv = gen_small_i16(seed, l, MYL_R_BV, kvN);
            L->bq_s = gen_small_u8(seed, l, MYL_R_BQ_SHIFT, qN);
            L->bk_s = gen_small_u8(seed, l, MYL_R_BK_SHIFT, kvN);
            L->bv_s = gen_small_u8(seed, l, MYL_R_BV_SHIFT, kvN);
        }
        L->f = myl_synth_layer_fracs(seed, l);
        L->res_in_frac = (uint8_t*)xalloc(H);
        L->res_mid_frac = (uint8_t*)xalloc(H);
        if (L->res_in_frac && L->res_mid_frac) {
            uint64_t ti = myl_tensor_seed(seed, l, MYL_R_RES_IN), tm = myl_tensor_seed(seed, l, MYL_R_RES_MID);
            for (size_t i = 0; i < H; ++i) {
                L->res_in_frac[i] = myl_synth_res_frac(ti, i);
                L->res_mid_frac[i] = myl_synth_res_frac(tm, i);
            }
        }
    }
    size_t kv_elems = (size_t)s.layers * s.kv_heads * (size_t)s.max_pos * hd;
    m->kcache = (int16_t*)calloc(kv_elems ? kv_elems : 1, sizeof(int16_t));
    m->vcache = (int16_t*)calloc(kv_elems ? kv_elems : 1, sizeof(int16_t));
    if (!m->emb || !m->kcache || !m->vcache || (s.lm_head_int16 && !m->lm16)) { or_model_destroy(m); return NULL; }
    return m;
}

void or_model_reset(or_model* m) { m->n_cached = 0; }

static inline int16_t* kv_at(int16_t* base, const myl_synth_spec* s, uint32_t layer, uint32_t kvh, uint32_t pos) {
    return base + ((((size_t)layer * s->kv_heads + kvh) * s->max_pos + pos) * s->head_dim);
}

/* model.rs:401-674 (forward_layer). */
static int forward_layer(or_model* m, uint32_t l, const int16_t* hidden, uint32_t pos,
                         const uint8_t* out_res_frac, int16_t* out) {
    const myl_synth_spec* s = &m->spec;
    const or_layer* L = &m->layers[l];
    const myl_layer_fracs* sc = &L->f;
    const size_t hs = s->hidden, hd = s->head_dim, qN = (size_t)s->heads * hd, kvN = (size_t)s->kv_heads * hd;
    const size_t I = s->inter;
    int rc = 0;
    int16_t* norm = (int16_t*)xalloc(hs * 2);
    int16_t* qf = (int16_t*)xalloc(qN * 2);
    int16_t* kf = (int16_t*)xalloc(kvN * 2);
    int16_t* vf = (int16_t*)xalloc(kvN * 2);
    int16_t* qr = (int16_t*)xalloc(qN * 2);
    int16_t* attn = (int16_t*)xalloc(hs * 2);
    int16_t* o = (int16_t*)xalloc(hs * 2);
    int16_t* resid = (int16_t*)xalloc(hs * 2);
    int16_t* mlp = (int16_t*)xalloc(hs * 2);
    uint8_t* acc_attn = (uint8_t*)xalloc(hs);
    uint8_t* acc_mlp = (uint8_t*)xalloc(hs);
    if (!norm || !qf || !kf || !vf || !qr || !attn || !o || !resid || !mlp || !acc_attn || !acc_mlp) { rc = -3; goto done; }

    /* input_layernorm (:416-426) */
    rc = or_rmsnorm_i16(hidden, L->res_in_frac, L->in_gamma, L->in_gamma_shifts, hs, m->rsqrt, m->rsqrt_len,
                        MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, sc->norm_attn_frac, norm);
    if (rc) goto done;
    /* q/k/v projections (:438-440) + biases (:445-453) */
    or_linear_w8a16(norm, L->wq, hs, L->sq, qN, sc->norm_attn_frac, sc->q_frac, qf);
    or_linear_w8a16(norm, L->wk, hs, L->sk, kvN, sc->norm_attn_frac, sc->k_frac, kf);
    or_linear_w8a16(norm, L->wv, hs, L->sv, kvN, sc->norm_attn_frac, sc->v_frac, vf);
    if (s->attention_bias) {
        or_add_bias_i16(qf, L->bq, L->bq_s, qN, sc->q_frac);
        or_add_bias_i16(kf, L->bk, L->bk_s, kvN, sc->k_frac);
        or_add_bias_i16(vf, L->bv, L->bv_s, kvN, sc->v_frac);
    }
    /* RoPE row pos % n_pos (:469-479) */
    {
        size_t half = hd / 2, n_pos = m->rope_len / half, idx = pos % n_pos;
        const int16_t* cr = m->cos_lut + idx * half;
        const int16_t* sr = m->sin_lut + idx * half;
        for (uint32_t h = 0; h < s->heads; ++h)
            or_rotate_half_split_i16(qf + h * hd, hd, cr, sr, MYL_TV_ROPE_FRAC_BITS, qr + h * hd);
        /* KV write without rescale (:500-503) */
        for (uint32_t h = 0; h < s->kv_heads; ++h) {
            or_rotate_half_split_i16(kf + h * hd, hd, cr, sr, MYL_TV_ROPE_FRAC_BITS, kv_at(m->kcache, s, l, h, pos));
            memcpy(kv_at(m->vcache, s, l, h, pos), vf + h * hd, hd * 2);
        }
    }
    /* attention per query head, GQA kv head h / group (:508-558) */
    {
        uint32_t group = s->heads / s->kv_heads;
        int64_t score_mult = or_inv_sqrt_q15(hd);
        uint32_t ss = (uint32_t)sc->q_frac + sc->k_frac + 15u;
        uint8_t score_shift = (uint8_t)(ss > MYL_TV_SCORE_FRAC_BITS ? ss - MYL_TV_SCORE_FRAC_BITS : 0);
        uint8_t lut_shift = MYL_TV_SCORE_FRAC_BITS > MYL_TV_EXP_INPUT_FRAC ? MYL_TV_SCORE_FRAC_BITS - MYL_TV_EXP_INPUT_FRAC : 0;
        /* heads are independent: each writes its own slice of attn */
        int bad = 0;
        long long nh = (long long)s->heads;
#pragma omp parallel for if (g_threads > 1 && pos >= 64) num_threads(g_threads) schedule(static) reduction(| : bad)
        for (long long h = 0; h < nh; ++h) {
            uint32_t kvh = (uint32_t)h / group;
            bad |= or_attention_int(qr + h * hd, kv_at(m->kcache, s, l, kvh, 0), kv_at(m->vcache, s, l, kvh, 0),
                                    NULL, 1, (size_t)pos + 1, hd, score_mult, score_shift, m->exp_lut, m->exp_len,
                                    lut_shift, MYL_TV_PROB_FRAC_BITS, attn + h * hd) != 0;
        }
        if (bad) { rc = -3; goto done; }
    }
    /* v_frac -> attn_out_frac (:563-567) */
    if (sc->attn_out_frac != sc->v_frac)
        for (size_t i = 0; i < hs; ++i) attn[i] = or_clamp_i16(or_rescale(attn[i], sc->v_frac, sc->attn_out_frac));
    /* o_proj at min(res_in, res_mid) per channel (:576-582) */
    for (size_t i = 0; i < hs; ++i) acc_attn[i] = L->res_in_frac[i] < L->res_mid_frac[i] ? L->res_in_frac[i] : L->res_mid_frac[i];
    or_linear_w8a16_pc(attn, L->wo, qN, L->so, hs, sc->attn_out_frac, acc_attn, o);
    /* residual add 1 (:588-593) */
    for (size_t i = 0; i < hs; ++i) {
        int64_t hh = or_rescale_i64(hidden[i], L->res_in_frac[i], acc_attn[i]);
        int64_t sum = add64(hh, o[i]);
        resid[i] = or_clamp_i16_from_i64(or_rescale_i64(sum, acc_attn[i], L->res_mid_frac[i]));
    }
    /* post_attention_layernorm (:596-606) */
    rc = or_rmsnorm_i16(resid, L->res_mid_frac, L->post_gamma, L->post_gamma_shifts, hs, m->rsqrt, m->rsqrt_len,
                        MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, sc->norm_mlp_frac, norm);
    if (rc) goto done;
    /* MLP (:612-637) */
    for (size_t i = 0; i < hs; ++i) acc_mlp[i] = L->res_mid_frac[i] < out_res_frac[i] ? L->res_mid_frac[i] : out_res_frac[i];
    rc = or_mlp_int(norm, L->wg, L->wu, L->wd, hs, I, L->sg, L->su, L->sd, m->silu, m->silu_len,
                    sc->norm_mlp_frac, sc->gate_frac, sc->up_frac, sc->down_in_frac,
                    MYL_TV_SILU_IN_FRAC, MYL_TV_SILU_LUT_OFFSET, MYL_TV_SILU_OUT_FRAC, acc_mlp, mlp);
    if (rc) goto done;
    /* residual add 2 (:666-671) */
    for (size_t i = 0; i < hs; ++i) {
        int64_t r = or_rescale_i64(resid[i], L->res_mid_frac[i], acc_mlp[i]);
        int64_t sum = add64(r, mlp[i]);
        out[i] = or_clamp_i16_from_i64(or_rescale_i64(sum, acc_mlp[i], out_res_frac[i]));
    }
done:
    free(norm); free(qf); free(kf); free(vf); free(qr); free(attn); free(o); free(resid); free(mlp);
    free(acc_attn); free(acc_mlp);
    return rc;
}

/* model.rs:323-331 */
int or_model_embed_token(const or_model* m, uint32_t token, int16_t* hidden) {
    if (token >= m->spec.vocab) return -1;
    const size_t H = m->spec.hidden;
    const uint8_t* first = m->layers[0].res_in_frac;
    const int8_t* row = m->emb + (size_t)token * H;
    uint8_t sh = m->emb_shifts[token];
    for (size_t i = 0; i < H; ++i) hidden[i] = or_clamp_i16(or_rescale((int32_t)row[i], sh, first[i]));
    return 0;
}

/* model.rs:339-356 */
int or_model_run_layers(or_model* m, int16_t* hidden, uint32_t pos, uint32_t layer_start, uint32_t layer_end) {
    if (pos >= m->spec.max_pos || layer_end > m->spec.layers) return -1;
    int16_t* tmp = (int16_t*)xalloc(m->spec.hidden * 2);
    if (!tmp) return -3;
    int rc = 0;
    for (uint32_t l = layer_start; l < layer_end && !rc; ++l) {
        const uint8_t* of = (l + 1 < m->spec.layers) ? m->layers[l + 1].res_in_frac : m->final_res_frac;
        rc = forward_layer(m, l, hidden, pos, of, tmp);
        memcpy(hidden, tmp, m->spec.hidden * 2);
    }
    free(tmp);
    return rc;
}

/* model.rs:360-399: final RMSNorm + LM head (path A int16 / path B int8). */
int or_model_head_logits(const or_model* m, const int16_t* hidden, int32_t* logits) {
    const size_t H = m->spec.hidden;
    long long V = (long long)m->spec.vocab;
    int16_t* normed = (int16_t*)xalloc(H * 2);
    if (!normed) return -3;
    int rc = or_rmsnorm_i16(hidden, m->final_res_frac, m->final_gamma, m->final_gamma_shifts, H, m->rsqrt,
                            m->rsqrt_len, MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20,
                            m->final_norm_frac, normed);
    if (rc) { free(normed); return rc; }
#pragma omp parallel for if (g_threads > 1) num_threads(g_threads) schedule(static)
    for (long long row = 0; row < V; ++row) {
        uint64_t acc = 0;
        uint8_t sh;
        if (m->spec.lm_head_int16) {
            const int16_t* w = m->lm16 + (size_t)row * H;
            for (size_t d = 0; d < H; ++d) acc += (uint64_t)((int64_t)w[d] * (int64_t)normed[d]);
            sh = m->lm16_shifts[row];
        } else {
            const int8_t* w = m->emb + (size_t)row * H;
            for (size_t d = 0; d < H; ++d) acc += (uint64_t)((int64_t)w[d] * (int64_t)normed[d]);
            sh = m->emb_shifts[row];
        }
        int64_t y = or_rescale_i64((int64_t)acc, (uint8_t)(sh + m->final_norm_frac), MYL_TV_LOGIT_FRAC_BITS);
        logits[row] = or_clamp_i32(y);
    }
    free(normed);
    return 0;
}

/* model.rs:229-311 */
int or_model_forward_token(or_model* m, uint32_t token, uint32_t pos, int32_t* logits) {
    if (pos > m->n_cached) return -1; /* positions are written contiguously from 0 */
    int16_t* hidden = (int16_t*)xalloc(m->spec.hidden * 2);
    if (!hidden) return -3;
    int rc = or_model_embed_token(m, token, hidden);
    if (!rc) rc = or_model_run_layers(m, hidden, pos, 0, m->spec.layers);
    if (!rc && pos + 1 > m->n_cached) m->n_cached = pos + 1;
    if (!rc && logits) rc = or_model_head_logits(m, hidden, logits);
    free(hidden);
    return rc;
}

/* KVCache::write for positions [0, n_pos) of one (layer, KV head), and the
 * cached length: continues a run whose cache another implementation built
 * (kv_cache.rs:38-52). */
int or_model_write_kv(or_model* m, uint32_t layer, uint32_t kv_head, uint32_t n_pos, const int16_t* k,
                      const int16_t* v) {
    const myl_synth_spec* s = &m->spec;
    if (layer >= s->layers || kv_head >= s->kv_heads || n_pos > s->max_pos) return -1;
    size_t n = (size_t)n_pos * s->head_dim * 2;
    memcpy(kv_at(m->kcache, s, layer, kv_head, 0), k, n);
    memcpy(kv_at(m->vcache, s, layer, kv_head, 0), v, n);
    return 0;
}

int or_model_set_cached(or_model* m, uint32_t n_pos) {
    if (n_pos > m->spec.max_pos) return -1;
    m->n_cached = n_pos;
    return 0;
}

int or_model_read_kv(const or_model* m, uint32_t layer, uint32_t kv_head, uint32_t n_pos,
                     int16_t* k_out, int16_t* v_out) {
    const myl_synth_spec* s = &m->spec;
    if (layer >= s->layers || kv_head >= s->kv_heads || n_pos > s->max_pos) return -1;
    size_t n = (size_t)n_pos * s->head_dim * 2;
    memcpy(k_out, kv_at(m->kcache, s, layer, kv_head, 0), n);
    memcpy(v_out, kv_at(m->vcache, s, layer, kv_head, 0), n);
    return 0;
}

const void* or_model_tensor(const or_model* m, const char* name, uint32_t layer, size_t* bytes) {
    const myl_synth_spec* s = &m->spec;
    const size_t H = s->hidden, I = s->inter, V = s->vocab, hd = s->head_dim;
    const size_t qN = (size_t)s->heads * hd, kvN = (size_t)s->kv_heads * hd;
    if (layer >= s->layers) return NULL;
    const or_layer* L = &m->layers[layer];
#define T(nm, ptr, n) if (!strcmp(name, nm)) { *bytes = (n); return (ptr); }
    T("emb", m->emb, V * H) T("emb_shifts", m->emb_shifts, V)
    T("lm16", m->lm16, s->lm_head_int16 ? V * H * 2 : 0) T("lm16_shifts", m->lm16_shifts, s->lm_head_int16 ? V : 0)
    T("final_gamma", m->final_gamma, H) T("final_gamma_shifts", m->final_gamma_shifts, H)
    T("final_res_frac", m->final_res_frac, H)
    T("in_gamma", L->in_gamma, H) T("in_gamma_shifts", L->in_gamma_shifts, H)
    T("post_gamma", L->post_gamma, H) T("post_gamma_shifts", L->post_gamma_shifts, H)
    T("wq", L->wq, qN * H) T("wk", L->wk, kvN * H) T("wv", L->wv, kvN * H) T("wo", L->wo, H * qN)
    T("wg", L->wg, I * H) T("wu", L->wu, I * H) T("wd", L->wd, H * I)
    T("sq", L->sq, qN) T("sk", L->sk, kvN) T("sv", L->sv, kvN) T("so", L->so, H)
    T("sg", L->sg, I) T("su", L->su, I) T("sd", L->sd, H)
    T("bq", L->bq, s->attention_bias ? qN * 2 : 0) T("bk", L->bk, s->attention_bias ? kvN * 2 : 0)
    T("bv", L->bv, s->attention_bias ? kvN * 2 : 0)
    T("bq_s", L->bq_s, s->attention_bias ? qN : 0) T("bk_s", L->bk_s, s->attention_bias ? kvN : 0)
    T("bv_s", L->bv_s, s->attention_bias ? kvN : 0)
    T("res_in_frac", L->res_in_frac, H) T("res_mid_frac", L->res_mid_frac, H)
    T("layer_fracs", &L->f, sizeof(myl_layer_fracs))
#undef T
    if (!strcmp(name, "final_norm_frac")) { *bytes = 1; return &m->final_norm_frac; }
    return NULL;
}

/* ---- integer MoE layer (build-defined; the reference has no MoE) ---------
 * The definition the GPU layer implements (include/myl_hip.h, section 4),
 * restated with the reference primitives above: router logits by the LM-head
 * requant plus an integer bias, top-k by repeated first maxima, softmax_int
 * gates, mlp_int experts, one i64 weighted sum and one rounding. */
struct or_moe {
    myl_moe_spec spec;
    int8_t* wr;          /* [E x H] */
    int32_t* bias;       /* [E] */
    int8_t *wg, *wu, *wd;          /* per expert and shared (index E): [I x H], [I x H], [H x I] */
    uint8_t *sg, *su, *sd;
    size_t* woff;        /* element offset of expert x's gate/up and down matrices */
    size_t* soff;        /* offset of expert x's gate/up shifts; down shifts at x * H */
    uint8_t* out_frac;   /* [H] */
    int16_t* silu; size_t silu_len;
    int16_t* exp_lut; size_t exp_len;
};

static void moe_fill_w8(int8_t* dst, size_t rows, size_t K, uint64_t tseed) {
    size_t n = rows * K;
#pragma omp parallel for schedule(static) if (n > (1 << 20))
    for (size_t i = 0; i < n; ++i) dst[i] = myl_synth_w8(tseed, i);
}

void or_moe_destroy(or_moe* m) {
    if (!m) return;
    free(m->wr); free(m->bias); free(m->wg); free(m->wu); free(m->wd);
    free(m->sg); free(m->su); free(m->sd); free(m->woff); free(m->soff);
    free(m->out_frac); free(m->silu); free(m->exp_lut);
    free(m);
}

or_moe* or_moe_create_synthetic(const myl_moe_spec* spec, const int32_t* router_bias, const myl_luts* luts) {
    const size_t H = spec->hidden, E = spec->n_experts, I = spec->inter, S = spec->shared_inter;
    if (!H || !E || !I || !S || !spec->top_k || spec->top_k > E) return NULL;
    /* the route's per-token scratch (or_moe_route: z[256], sel[16]) bounds
       the expert count and top-k, as the device layer's checks do */
    if (E > 256 || spec->top_k > 16) return NULL;
    or_moe* m = (or_moe*)calloc(1, sizeof(or_moe));
    if (!m) return NULL;
    m->spec = *spec;
    const uint64_t seed = spec->seed;
    size_t wtot = 0, stot = 0;
    m->woff = (size_t*)malloc((E + 1) * sizeof(size_t));
    m->soff = (size_t*)malloc((E + 1) * sizeof(size_t));
    for (size_t x = 0; x <= E; ++x) {
        const size_t inter = x == E ? S : I;
        m->woff[x] = wtot;
        m->soff[x] = stot;
        wtot += inter * H;
        stot += inter;
    }
    m->wr = (int8_t*)malloc(E * H);
    m->bias = (int32_t*)malloc(E * sizeof(int32_t));
    m->wg = (int8_t*)malloc(wtot);
    m->wu = (int8_t*)malloc(wtot);
    m->wd = (int8_t*)malloc(wtot);
    m->sg = (uint8_t*)malloc(stot);
    m->su = (uint8_t*)malloc(stot);
    m->sd = (uint8_t*)malloc((E + 1) * H);
    m->out_frac = (uint8_t*)malloc(H);
    m->silu = (int16_t*)malloc(luts->silu_len * sizeof(int16_t));
    m->exp_lut = (int16_t*)malloc(luts->exp_len * sizeof(int16_t));
    if (!m->woff || !m->soff || !m->wr || !m->bias || !m->wg || !m->wu || !m->wd || !m->sg || !m->su || !m->sd ||
        !m->out_frac || !m->silu || !m->exp_lut) {
        or_moe_destroy(m);
        return NULL;
    }
    memcpy(m->bias, router_bias, E * sizeof(int32_t));
    memcpy(m->silu, luts->silu, luts->silu_len * sizeof(int16_t));
    memcpy(m->exp_lut, luts->exp, luts->exp_len * sizeof(int16_t));
    m->silu_len = luts->silu_len;
    m->exp_len = luts->exp_len;
    moe_fill_w8(m->wr, E, H, myl_tensor_seed(seed, 0, MYL_R_ROUTER));
    for (size_t i = 0; i < H; ++i) m->out_frac[i] = myl_synth_moe_out_frac(seed, i);
    for (size_t x = 0; x <= E; ++x) {
        const size_t inter = x == E ? S : I;
        moe_fill_w8(m->wg + m->woff[x], inter, H, myl_tensor_seed(seed, (uint32_t)x, MYL_R_WG));
        moe_fill_w8(m->wu + m->woff[x], inter, H, myl_tensor_seed(seed, (uint32_t)x, MYL_R_WU));
        moe_fill_w8(m->wd + m->woff[x], H, inter, myl_tensor_seed(seed, (uint32_t)x, MYL_R_WD));
        const uint64_t tg = myl_tensor_seed(seed, (uint32_t)x, MYL_R_SG), tu = myl_tensor_seed(seed, (uint32_t)x, MYL_R_SU),
                       td = myl_tensor_seed(seed, (uint32_t)x, MYL_R_SD);
        for (size_t r = 0; r < inter; ++r) {
            m->sg[m->soff[x] + r] = myl_synth_wshift(tg, r, H);
            m->su[m->soff[x] + r] = myl_synth_wshift(tu, r, H);
        }
        for (size_t r = 0; r < H; ++r) m->sd[x * H + r] = myl_synth_wshift(td, r, inter);
    }
    return m;
}

void or_moe_synth_input(const or_moe* m, uint32_t T, int16_t* x) {
    const size_t n = (size_t)T * m->spec.hidden;
    const uint64_t ts = myl_tensor_seed(m->spec.seed, 0, MYL_R_ACT);
#pragma omp parallel for schedule(static) if (n > (1 << 16))
    for (size_t i = 0; i < n; ++i) x[i] = myl_synth_gauss16(ts, i, 2000);
}

/* Router, top-k and gates of every token; counts, offsets and the stable
 * expert-major token lists.  Any output may be NULL except ids and gates. */
int or_moe_route(const or_moe* m, const int16_t* x, uint32_t T, int32_t* ids, int32_t* gates, int32_t* counts,
                 int32_t* offsets, int32_t* list_tok) {
    const size_t H = m->spec.hidden, E = m->spec.n_experts, K = m->spec.top_k;
    int rc = 0;
#pragma omp parallel for schedule(static) if (g_threads > 1) num_threads(g_threads)
    for (uint32_t t = 0; t < T; ++t) {
        const int16_t* xt = x + (size_t)t * H;
        int32_t z[256], sel[16], g[16];
        int taken[256];
        for (size_t e = 0; e < E; ++e) {
            int64_t d = or_dot_i8_i16(m->wr + e * H, xt, H);
            int32_t r = or_clamp_i32(or_rescale_i64(d, MYL_MOE_ROUTER_SHIFT + MYL_MOE_X_FRAC, MYL_MOE_ROUTER_FRAC));
            z[e] = or_clamp_i32((int64_t)r + (int64_t)m->bias[e]);
            taken[e] = 0;
        }
        for (size_t k = 0; k < K; ++k) {
            size_t best = E;
            for (size_t e = 0; e < E; ++e)
                if (!taken[e] && (best == E || z[e] > z[best])) best = e;
            taken[best] = 1;
            sel[k] = z[best];
            ids[(size_t)t * K + k] = (int32_t)best;
        }
        if (or_softmax_int(sel, K, m->exp_lut, m->exp_len, 0, MYL_TV_PROB_FRAC_BITS, g)) rc = -1;
        for (size_t k = 0; k < K; ++k) gates[(size_t)t * K + k] = g[k];
    }
    if (rc) return rc;
    if (counts || offsets || list_tok) {
        int32_t* c = (int32_t*)calloc(E, sizeof(int32_t));
        if (!c) return -3;
        for (size_t i = 0; i < (size_t)T * K; ++i) c[ids[i]]++;
        if (counts) memcpy(counts, c, E * sizeof(int32_t));
        int32_t run = 0;
        for (size_t e = 0; e < E; ++e) {
            if (offsets) offsets[e] = run;
            if (list_tok)
                for (uint32_t t = 0; t < T; ++t)
                    for (size_t k = 0; k < K; ++k)
                        if ((size_t)ids[(size_t)t * K + k] == e) list_tok[run++] = (int32_t)t;
            if (!list_tok) run += c[e];
        }
        if (offsets) offsets[E] = run;
        free(c);
    }
    return 0;
}

/* The layer's output for one token given its route (ids, gates). */
int or_moe_token(const or_moe* m, const int16_t* xt, const int32_t* ids_t, const int32_t* gates_t, int16_t* out) {
    const size_t H = m->spec.hidden, E = m->spec.n_experts, K = m->spec.top_k;
    int16_t* y = (int16_t*)malloc(H * sizeof(int16_t));
    int64_t* acc = (int64_t*)malloc(H * sizeof(int64_t));
    if (!y || !acc) { free(y); free(acc); return -3; }
    int rc = 0;
    for (size_t k = 0; k <= K && !rc; ++k) {  /* k == K: the shared expert */
        const size_t x = k == K ? E : (size_t)ids_t[k];
        const size_t inter = x == E ? m->spec.shared_inter : m->spec.inter;
        rc = or_mlp_int(xt, m->wg + m->woff[x], m->wu + m->woff[x], m->wd + m->woff[x], H, inter,
                        m->sg + m->soff[x], m->su + m->soff[x], m->sd + x * H, m->silu, m->silu_len, MYL_MOE_X_FRAC,
                        MYL_MOE_GATE_FRAC, MYL_MOE_UP_FRAC, MYL_MOE_DOWN_IN_FRAC, MYL_TV_SILU_IN_FRAC,
                        MYL_TV_SILU_LUT_OFFSET, MYL_TV_SILU_OUT_FRAC, m->out_frac, y);
        for (size_t c = 0; c < H && !rc; ++c) {
            const int64_t w = k == K ? (int64_t)1 << MYL_TV_PROB_FRAC_BITS : (int64_t)gates_t[k];
            const int64_t term = mul64(w, (int64_t)y[c]);
            acc[c] = k == 0 ? term : add64(acc[c], term);
        }
    }
    if (!rc)
        for (size_t c = 0; c < H; ++c) out[c] = or_clamp_i16_from_i64(or_rshift_round_i64(acc[c], MYL_TV_PROB_FRAC_BITS));
    free(y); free(acc);
    return rc;
}

/* One expert's mlp_int output (x == n_experts: the shared expert), for tests. */
int or_moe_expert(const or_moe* m, const int16_t* xt, uint32_t expert, int16_t* out) {
    const size_t H = m->spec.hidden, E = m->spec.n_experts;
    if (expert > E) return -1;
    const size_t inter = expert == E ? m->spec.shared_inter : m->spec.inter;
    return or_mlp_int(xt, m->wg + m->woff[expert], m->wu + m->woff[expert], m->wd + m->woff[expert], H, inter,
                      m->sg + m->soff[expert], m->su + m->soff[expert], m->sd + expert * H, m->silu, m->silu_len,
                      MYL_MOE_X_FRAC, MYL_MOE_GATE_FRAC, MYL_MOE_UP_FRAC, MYL_MOE_DOWN_IN_FRAC, MYL_TV_SILU_IN_FRAC,
                      MYL_TV_SILU_LUT_OFFSET, MYL_TV_SILU_OUT_FRAC, m->out_frac, out);
}

/* Router logits (after the bias) of one token, for tests. */
void or_moe_router_logits(const or_moe* m, const int16_t* xt, int32_t* z) {
    const size_t H = m->spec.hidden, E = m->spec.n_experts;
    for (size_t e = 0; e < E; ++e) {
        int64_t d = or_dot_i8_i16(m->wr + e * H, xt, H);
        int32_t r = or_clamp_i32(or_rescale_i64(d, MYL_MOE_ROUTER_SHIFT + MYL_MOE_X_FRAC, MYL_MOE_ROUTER_FRAC));
        z[e] = or_clamp_i32((int64_t)r + (int64_t)m->bias[e]);
    }
}
