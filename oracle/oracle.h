/*
 * oracle.h -- CPU restatement of the INTEGER_LLM integer forward path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker that the HIP path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function restates a function of the reference Rust crates
 * (INTEGER_LLM/kernels, INTEGER_LLM/runtime) in release-mode Rust semantics:
 * + - * wrap, `as` truncates, shift amounts are masked to the operand width,
 * and the i128 arithmetic of rmsnorm uses gcc's __int128.  Citations are
 * file:line in the reference tree.
 *
 * Where the reference would panic (assert!, empty slices, division by zero)
 * the oracle returns a negative status instead.
 */
#ifndef MYL_ORACLE_H
#define MYL_ORACLE_H

#include <stdint.h>
#include <stddef.h>
#include "../include/myl_theta_v.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- fixed_point.rs ---------------------------------------------------- */
int8_t  or_clamp_i8(int32_t x);                      /* fixed_point.rs:7-11   */
int16_t or_clamp_i16(int32_t x);                     /* fixed_point.rs:15-19  */
int16_t or_clamp_i16_from_i64(int64_t x);            /* fixed_point.rs:23-27  */
int32_t or_clamp_i32(int64_t x);                     /* fixed_point.rs:31-35  */
int32_t or_rshift_round(int32_t value, uint8_t shift);      /* :39-53  */
int64_t or_rshift_round_i64(int64_t value, uint8_t shift);  /* :57-71  */
/* rshift_round_i128 (:155-169) on a value given as hi:lo 64-bit halves. */
void    or_rshift_round_i128(int64_t hi, uint64_t lo, uint32_t shift, int64_t* out_hi, uint64_t* out_lo);
int32_t or_rescale(int32_t acc, uint8_t in_frac, uint8_t out_frac);      /* :173-180 */
int64_t or_rescale_i64(int64_t acc, uint8_t in_frac, uint8_t out_frac);  /* :184-191 */
int64_t or_inv_sqrt_q15(size_t head_dim);            /* fixed_point.rs:102-107 */
uint64_t or_isqrt_round(uint64_t n);                 /* fixed_point.rs:117-146 */

/* ---- dot.rs / linear.rs ------------------------------------------------ */
int64_t or_dot_i8_i16(const int8_t* w, const int16_t* x, size_t n);   /* dot.rs:141-147 */
int or_linear_w8a16(const int16_t* x, const int8_t* W, size_t in_features,
                    const uint8_t* w_shifts, size_t out_features,
                    uint8_t act_frac, uint8_t out_frac, int16_t* out);   /* linear.rs:43-70 */
int or_linear_w8a16_pc(const int16_t* x, const int8_t* W, size_t in_features,
                       const uint8_t* w_shifts, size_t out_features,
                       uint8_t act_frac, const uint8_t* out_frac, int16_t* out); /* linear.rs:87-119 */
int or_add_bias_i16(int16_t* out, const int16_t* bias, const uint8_t* bias_shifts,
                    size_t n, uint8_t out_frac);                         /* linear.rs:132-145 */
/* Batched form used by the M-row sweep: M independent linear_w8a16 calls
 * (x is [M x K], out is [M x N]).  out_frac_pc may be NULL (scalar out_frac). */
int or_linear_w8a16_batch(const int16_t* x, size_t M, const int8_t* W, size_t N, size_t K,
                          const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac,
                          const uint8_t* out_frac_pc, int16_t* out);
/* Build-defined multiplier requant (no reference counterpart):
 * y[m][r] = clamp_i16(rshift_round_i128(dot(W[r], x[m]) * mult[r], shift[r])). */
int or_linear_w8a16_mult(const int16_t* x, size_t M, const int8_t* W, size_t N, size_t K,
                         const int32_t* mult, const uint8_t* shift, int16_t* out);
/* The two requant steps on precomputed exact sums acc [M x N]:
 * clamp_i16(rescale_i64(acc, w_shifts[r] + act_frac, out_frac)) (linear.rs:61-68)
 * and the multiplier form above. */
int or_requant_shift(const int64_t* acc, size_t M, size_t N, const uint8_t* w_shifts, uint8_t act_frac,
                     uint8_t out_frac, int16_t* out);
int or_requant_mult(const int64_t* acc, size_t M, size_t N, const int32_t* mult, const uint8_t* shift, int16_t* out);

/* ---- rmsnorm.rs -------------------------------------------------------- */
int64_t or_inv_n_q20(size_t n);                                          /* rmsnorm.rs:20-23 */
int or_rmsnorm_i16(const int16_t* x, const uint8_t* x_shifts, const int8_t* gamma,
                   const uint8_t* gamma_shifts, size_t n, const int16_t* rsqrt_lut,
                   size_t lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                   int64_t inv_n_q20, uint8_t out_frac, int16_t* out);   /* rmsnorm.rs:61-161 */

/* ---- rope.rs ----------------------------------------------------------- */
int or_rotate_half_split_i16(const int16_t* vec, size_t head_dim, const int16_t* cos_row,
                             const int16_t* sin_row, uint8_t frac_bits, int16_t* out); /* rope.rs:17-31 */
int or_apply_rope_i16(const int16_t* q, const int16_t* k, size_t n, size_t head_dim,
                      const int16_t* cos_lut, const int16_t* sin_lut, size_t lut_len,
                      const uint64_t* positions, uint8_t frac_bits,
                      int16_t* q_out, int16_t* k_out);                    /* rope.rs:36-59 */

/* ---- softmax.rs / attention.rs ---------------------------------------- */
int32_t or_exp_lut_lookup(int32_t x, const int16_t* lut, size_t len, uint8_t lut_shift, int32_t one); /* softmax.rs:12-21 */
int or_softmax_int(const int32_t* logits, size_t n, const int16_t* exp_lut, size_t lut_len,
                   uint8_t lut_shift, uint8_t frac_bits, int32_t* out);  /* softmax.rs:24-64 */
int64_t or_dot_int(const int16_t* a, const int16_t* b, size_t n);        /* attention.rs:21-27 */
/* mask is [q_len x kv_len] bytes (nonzero = attend) or NULL for all-true. */
int or_attention_int(const int16_t* q, const int16_t* k, const int16_t* v,
                     const uint8_t* mask, size_t q_len, size_t kv_len, size_t head_dim,
                     int64_t score_mult, uint8_t score_shift, const int16_t* exp_lut,
                     size_t lut_len, uint8_t lut_shift, uint8_t prob_frac_bits,
                     int16_t* out);                                      /* attention.rs:42-90 */

/* ---- integer_math.rs / mlp.rs / sampling.rs / prng.rs ----------------- */
int16_t or_lut_lookup(int16_t x, const int16_t* lut, size_t len, uint8_t shift, int16_t offset); /* integer_math.rs:44-48 */
int or_mlp_int(const int16_t* x, const int8_t* W_gate, const int8_t* W_up, const int8_t* W_down,
               size_t hidden, size_t inter, const uint8_t* gate_w_shifts,
               const uint8_t* up_w_shifts, const uint8_t* down_w_shifts,
               const int16_t* silu_lut, size_t silu_len, uint8_t in_frac,
               uint8_t gate_out_frac, uint8_t up_out_frac, uint8_t down_in_frac,
               uint8_t silu_in_frac, int16_t silu_lut_offset, uint8_t silu_out_frac,
               const uint8_t* out_frac, int16_t* out);                   /* mlp.rs:28-74 */
int64_t or_argmax_int(const int32_t* v, size_t n);                       /* sampling.rs:8-18 */
void or_splitmix64(uint64_t state, uint64_t* new_state, uint64_t* out);  /* prng.rs:7-14 */
void or_sample_integer_cdf(const int32_t* z, size_t n, uint64_t state, int64_t* token,
                           uint64_t* new_state);                        /* sampling.rs:20-46 */

/* ---- integer log-softmax (build-defined; no reference counterpart: the
 * reference's perplexity probe works in f64, perplexity_probe.rs:55-67) --- */
/* floor(log2 S) and 16 fraction bits of log2(S / 2^e) by repeated squaring
 * of the Q62 mantissa; S = 0 is taken as 1. */
void or_log2_q16(uint64_t S, int32_t* e, uint32_t* f);
/* ln(S / 2^14) in Q16: RNE((((e - 14) << 16) + f) * 744261118, 30). */
int64_t or_ln_q16(uint64_t S);
/* (z[t] - max z) * 2^10 - ln_q16(sum_j exp_lut[(max z - z_j) << 2]), Q16. */
int64_t or_logsoftmax_at(const int32_t* z, size_t n, const int16_t* exp_lut, size_t lut_len, int64_t target);

/* ---- model.rs / kv_cache.rs ------------------------------------------- */
typedef struct or_model or_model;
/* Builds the seeded synthetic model of include/myl_synth.h on the host. */
or_model* or_model_create_synthetic(const myl_synth_spec* spec, const myl_luts* luts);
void or_model_destroy(or_model* m);
void or_model_reset(or_model* m);                   /* empty KV cache */
void or_set_threads(int n);                          /* rows of a GEMV split over n threads (results unchanged) */
void or_set_simd(int on);                            /* 1: i32-block dot (dot.rs:175-221), 0: scalar i64 loop; results unchanged */
/* model.rs:229-311; logits has vocab entries. */
int or_model_forward_token(or_model* m, uint32_t token, uint32_t pos, int32_t* logits);
/* model.rs:323-331 */
int or_model_embed_token(const or_model* m, uint32_t token, int16_t* hidden);
/* model.rs:339-356 (hidden in/out, in place) */
int or_model_run_layers(or_model* m, int16_t* hidden, uint32_t pos, uint32_t layer_start, uint32_t layer_end);
/* model.rs:360-399 */
int or_model_head_logits(const or_model* m, const int16_t* hidden, int32_t* logits);
/* kv_cache.rs:43-52 for one (layer, kv head): positions [0, n_pos). */
int or_model_read_kv(const or_model* m, uint32_t layer, uint32_t kv_head, uint32_t n_pos,
                     int16_t* k_out, int16_t* v_out);
/* kv_cache.rs:38-52 writes of positions [0, n_pos) of one (layer, kv head), and
 * the cached length: a run continues from a cache another implementation built. */
int or_model_write_kv(or_model* m, uint32_t layer, uint32_t kv_head, uint32_t n_pos, const int16_t* k,
                      const int16_t* v);
int or_model_set_cached(or_model* m, uint32_t n_pos);
/* Raw tensor access for tests (NULL if the name is unknown). */
const void* or_model_tensor(const or_model* m, const char* name, uint32_t layer, size_t* bytes);

/* ---- integer MoE layer (build-defined; include/myl_hip.h section 4) ---- */
typedef struct or_moe or_moe;
or_moe* or_moe_create_synthetic(const myl_moe_spec* spec, const int32_t* router_bias, const myl_luts* luts);
void or_moe_destroy(or_moe* m);
void or_moe_synth_input(const or_moe* m, uint32_t T, int16_t* x);
int or_moe_route(const or_moe* m, const int16_t* x, uint32_t T, int32_t* ids, int32_t* gates, int32_t* counts,
                 int32_t* offsets, int32_t* list_tok);
int or_moe_token(const or_moe* m, const int16_t* xt, const int32_t* ids_t, const int32_t* gates_t, int16_t* out);
int or_moe_expert(const or_moe* m, const int16_t* xt, uint32_t expert, int16_t* out);
void or_moe_router_logits(const or_moe* m, const int16_t* xt, int32_t* z);

#ifdef __cplusplus
}
#endif

#endif
