/*
 * myl_synth.h -- the seeded synthetic workload shared by the HIP library and
 * the CPU oracle.
 *
 * There are no real checkpoints on the machines this code runs on, so every
 * model and matrix is drawn from a SplitMix64 stream.  The stream is the
 * reference PRNG (INTEGER_LLM/kernels/src/prng.rs:7-14): state += gamma, then
 * the mix below.  Element i of a stream seeded with s is therefore
 * mix(s + (i + 1) * gamma), which a GPU thread can evaluate on its own.
 *
 * Everything here is integer-only and header-only.  Under hipcc the functions
 * are __host__ __device__, under gcc they are plain static inline C.
 */
#ifndef MYL_SYNTH_H
#define MYL_SYNTH_H

#include <stdint.h>
#include <stddef.h>

#include "myl_theta_v.h"

#if defined(__HIPCC__)
#define MYL_HD __host__ __device__ static inline
#else
#define MYL_HD static inline
#endif

#ifdef __cplusplus
extern "C" {
#endif

#define MYL_SM_GAMMA 0x9E3779B97F4A7C15ULL

/* SplitMix64 output function (prng.rs:11-13). */
MYL_HD uint64_t myl_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

/* i-th output (0-based) of the SplitMix64 stream whose state starts at seed. */
MYL_HD uint64_t myl_splitmix_at(uint64_t seed, uint64_t i) {
    return myl_mix64(seed + (i + 1) * MYL_SM_GAMMA);
}

/* Unbiased-enough map of a 64-bit draw onto [lo, hi] (Lemire multiply-shift on
 * the high 32 bits; the span is < 2^32). */
MYL_HD int32_t myl_draw_range(uint64_t z, int32_t lo, int32_t hi) {
    uint64_t span = (uint64_t)((int64_t)hi - (int64_t)lo + 1);
    return (int32_t)((int64_t)lo + (int64_t)(((z >> 32) * span) >> 32));
}

/* Per-tensor stream seed: model seed and a tensor tag (layer, role). */
MYL_HD uint64_t myl_tensor_seed(uint64_t model_seed, uint32_t layer, uint32_t role) {
    return myl_mix64(model_seed ^ myl_mix64(((uint64_t)layer << 16) ^ (uint64_t)role ^ 0xA5A5000000000000ULL));
}

/* Tensor roles (the tag in myl_tensor_seed). */
enum myl_role {
    MYL_R_EMB = 1, MYL_R_EMB_SHIFT, MYL_R_LM16, MYL_R_LM16_SHIFT,
    MYL_R_FINAL_GAMMA, MYL_R_FINAL_GAMMA_SHIFT, MYL_R_FINAL_RES_FRAC,
    MYL_R_IN_GAMMA, MYL_R_IN_GAMMA_SHIFT, MYL_R_POST_GAMMA, MYL_R_POST_GAMMA_SHIFT,
    MYL_R_WQ, MYL_R_WK, MYL_R_WV, MYL_R_WO, MYL_R_WG, MYL_R_WU, MYL_R_WD,
    MYL_R_SQ, MYL_R_SK, MYL_R_SV, MYL_R_SO, MYL_R_SG, MYL_R_SU, MYL_R_SD,
    MYL_R_BQ, MYL_R_BK, MYL_R_BV, MYL_R_BQ_SHIFT, MYL_R_BK_SHIFT, MYL_R_BV_SHIFT,
    MYL_R_RES_IN, MYL_R_RES_MID, MYL_R_LAYER_FRACS, MYL_R_MODEL_FRACS,
    MYL_R_MAT, MYL_R_MAT_SHIFT, MYL_R_MAT_MULT, MYL_R_ACT,
    MYL_R_ROUTER, MYL_R_ROUTER_SHIFT, MYL_R_MOE_OUT_FRAC
};

/* int8 weight element, uniform in [-127, 127] (the benchmark models' weight distribution). */
MYL_HD int8_t myl_synth_w8(uint64_t tseed, uint64_t i) {
    return (int8_t)myl_draw_range(myl_splitmix_at(tseed, i), -127, 127);
}

/* int16 LM-head element, uniform in [-32767, 32767]. */
MYL_HD int16_t myl_synth_w16(uint64_t tseed, uint64_t i) {
    return (int16_t)myl_draw_range(myl_splitmix_at(tseed, i), -32767, 32767);
}

/* Approximately Gaussian int16 activation with standard deviation sigma: an
 * integer Irwin-Hall draw.  Each of the 12 uniforms lies in [-4096, 4095]
 * (sd 8192/sqrt(12)), so their sum has sd 8192; it is scaled by sigma/8192
 * and clipped to +-32767 (the benchmark sweep's activation distribution). */
MYL_HD int16_t myl_synth_gauss16(uint64_t tseed, uint64_t i, int32_t sigma) {
    int64_t s = 0;
    for (int t = 0; t < 12; ++t)
        s += myl_draw_range(myl_splitmix_at(tseed, i * 12u + (uint64_t)t), -4096, 4095);
    int64_t v = (s * (int64_t)sigma) / 8192;
    if (v > 32767) v = 32767;
    if (v < -32767) v = -32767;
    return (int16_t)v;
}

/* floor(log2(v)) for v > 0. */
MYL_HD int myl_ilog2_u64(uint64_t v) {
    int r = -1;
    while (v) { v >>= 1; ++r; }
    return r;
}

/* Integer floor(sqrt(v)). */
MYL_HD uint64_t myl_isqrt_floor(uint64_t v) {
    uint64_t r = 0, bit = 1ULL << 62;
    while (bit > v) bit >>= 2;
    while (bit) {
        if (v >= r + bit) { v -= r + bit; r = (r >> 1) + bit; }
        else r >>= 1;
        bit >>= 2;
    }
    return r;
}

/* Per-row weight shift for an int8 matrix with K inputs: uniform int8 has
 * standard deviation ~73, so a dot with K unit-scale inputs grows by
 * 73*sqrt(K); the shift removes that growth (plus a 0/1 jitter per row so rows
 * carry different scales). */
MYL_HD uint8_t myl_synth_wshift(uint64_t tseed, uint64_t row, uint64_t K) {
    int base = myl_ilog2_u64(73ULL * myl_isqrt_floor(K) + 1);
    return (uint8_t)(base + (int)(myl_splitmix_at(tseed, row) & 1u));
}

/* Per-layer activation fractional bits of the synthetic model. */
MYL_HD myl_layer_fracs myl_synth_layer_fracs(uint64_t model_seed, uint32_t layer) {
    uint64_t s = myl_tensor_seed(model_seed, layer, MYL_R_LAYER_FRACS);
    myl_layer_fracs f;
    f.norm_attn_frac = (uint8_t)myl_draw_range(myl_splitmix_at(s, 0), 10, 11);
    f.q_frac        = (uint8_t)myl_draw_range(myl_splitmix_at(s, 1), 9, 10);
    f.k_frac        = (uint8_t)myl_draw_range(myl_splitmix_at(s, 2), 8, 9);
    f.v_frac        = (uint8_t)myl_draw_range(myl_splitmix_at(s, 3), 10, 11);
    f.attn_out_frac = (uint8_t)myl_draw_range(myl_splitmix_at(s, 4), 10, 12);
    f.norm_mlp_frac = (uint8_t)myl_draw_range(myl_splitmix_at(s, 5), 10, 11);
    f.gate_frac     = (uint8_t)myl_draw_range(myl_splitmix_at(s, 6), 10, 11);
    f.up_frac       = (uint8_t)myl_draw_range(myl_splitmix_at(s, 7), 10, 11);
    f.down_in_frac  = (uint8_t)myl_draw_range(myl_splitmix_at(s, 8), 10, 12);
    return f;
}

/* Per-channel residual-stream fractional bits (input/mid segments and the
 * final segment): 7..10, i.e. a real range of +-256 down to +-32. */
MYL_HD uint8_t myl_synth_res_frac(uint64_t tseed, uint64_t ch) {
    return (uint8_t)myl_draw_range(myl_splitmix_at(tseed, ch), 7, 10);
}

/* Small per-row / per-element tensors: value i of (layer, role) is uniform in
 * the role's range.  One table, so the device generator and the oracle agree. */
MYL_HD void myl_synth_small_range(uint32_t role, int32_t* lo, int32_t* hi) {
    switch (role) {
    case MYL_R_EMB_SHIFT:         *lo = 7;     *hi = 9;    break; /* int8 row scale 2^-7..2^-9 */
    case MYL_R_LM16_SHIFT:        *lo = 17;    *hi = 19;   break;
    case MYL_R_FINAL_GAMMA_SHIFT:
    case MYL_R_IN_GAMMA_SHIFT:
    case MYL_R_POST_GAMMA_SHIFT:  *lo = 6;     *hi = 7;    break;
    case MYL_R_BQ: case MYL_R_BK: case MYL_R_BV:
                                  *lo = -3000; *hi = 3000; break; /* int16 biases */
    case MYL_R_BQ_SHIFT: case MYL_R_BK_SHIFT: case MYL_R_BV_SHIFT:
                                  *lo = 10;    *hi = 13;   break;
    default:                      *lo = 0;     *hi = 0;    break;
    }
}

MYL_HD int32_t myl_synth_small(uint64_t model_seed, uint32_t layer, uint32_t role, uint64_t i) {
    int32_t lo, hi;
    myl_synth_small_range(role, &lo, &hi);
    return myl_draw_range(myl_splitmix_at(myl_tensor_seed(model_seed, layer, role), i), lo, hi);
}

/* ---- the synthetic MoE layer (myl_moe_spec) ---------------------------------
 * Expert e's gate/up/down weights and row shifts use the model roles
 * MYL_R_WG/WU/WD and MYL_R_SG/SU/SD with `layer` = e; the shared expert uses
 * layer = n_experts.  The router is [n_experts x hidden] (MYL_R_ROUTER); the
 * input is Gaussian int16 with sd 2000 (MYL_R_ACT, element t * hidden + i). */
#define MYL_MOE_X_FRAC        8   /* input fractional bits */
#define MYL_MOE_ROUTER_FRAC   8   /* router logits: the exp LUT's input frac */
#define MYL_MOE_ROUTER_SHIFT  15  /* router row shift: logit sd ~0.8 at sd-2000 inputs */
#define MYL_MOE_GATE_FRAC     10
#define MYL_MOE_UP_FRAC       10
#define MYL_MOE_DOWN_IN_FRAC  11

/* Per-channel output fractional bits of every expert (and the layer). */
MYL_HD uint8_t myl_synth_moe_out_frac(uint64_t model_seed, uint64_t ch) {
    return myl_synth_res_frac(myl_tensor_seed(model_seed, 0, MYL_R_MOE_OUT_FRAC), ch);
}

/* Model-wide scalars. */
MYL_HD uint8_t myl_synth_final_norm_frac(uint64_t model_seed) {
    return (uint8_t)myl_draw_range(myl_splitmix_at(myl_tensor_seed(model_seed, 0, MYL_R_MODEL_FRACS), 0), 9, 10);
}

#ifdef __cplusplus
}
#endif

#endif /* MYL_SYNTH_H */
