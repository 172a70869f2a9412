/*
 * myl_theta_v.h -- the numeric-contract constants of theta_v 0.17.0 that the
 * integer forward path consumes, and the LUT bundle type.
 *
 * Values follow INTEGER_LLM/theta_v/spec.json as read by
 * INTEGER_LLM/runtime/src/loader.rs:654-682 (spec_model_params):
 *   score_frac_bits   = nonlinear.softmax.exp_lut_frac_bits   = 14
 *   exp_input_frac    = nonlinear.softmax.exp_input_frac_bits = 8
 *   prob_frac_bits    = nonlinear.softmax.prob_frac_bits      = 14
 *   rope_frac_bits    = nonlinear.rope.frac_bits              = 8
 *   silu_in_frac      = nonlinear.silu.input_frac_bits        = 6
 *   silu_lut_offset   = -nonlinear.silu.input_range[0]        = 8192
 *   silu_out_frac     = nonlinear.silu.output_frac_bits       = 8
 *   rsqrt_input_shift = nonlinear.rsqrt.input_shift           = 8
 *   rsqrt_output_frac = nonlinear.rsqrt.output_frac_bits      = 8
 *   logit_frac_bits   = 6 (loader.rs:681)
 * LUT lengths: rsqrt 32768, silu 16384, exp 16385, cos/sin 2048 x head_dim/2.
 */
#ifndef MYL_THETA_V_H
#define MYL_THETA_V_H

#include <stdint.h>
#include <stddef.h>

#define MYL_TV_SCORE_FRAC_BITS   14
#define MYL_TV_EXP_INPUT_FRAC    8
#define MYL_TV_PROB_FRAC_BITS    14
#define MYL_TV_ROPE_FRAC_BITS    8
#define MYL_TV_SILU_IN_FRAC      6
#define MYL_TV_SILU_LUT_OFFSET   8192
#define MYL_TV_SILU_OUT_FRAC     8
#define MYL_TV_RSQRT_INPUT_SHIFT 8
#define MYL_TV_RSQRT_OUTPUT_FRAC 8
#define MYL_TV_LOGIT_FRAC_BITS   6
#define MYL_TV_ROPE_ROWS         2048

/* The theta_v version this numeric contract is (spec.json theta_v.version);
 * an artifact calibrated under another version is refused
 * (loader.rs:56-72, verify_version_against_spec). */
#define MYL_TV_VERSION "0.17.0"

#define MYL_TV_RSQRT_LEN 32768
#define MYL_TV_SILU_LEN  16384
#define MYL_TV_EXP_LEN   16385

#ifdef __cplusplus
extern "C" {
#endif

/* The five lookup tables of an artifact (loader.rs:509, model.rs:149-155).
 * cos/sin are flat row-major [rope_rows x head_dim/2]; rope_len is the element
 * count of each. */
typedef struct myl_luts {
    const int16_t* rsqrt; size_t rsqrt_len;
    const int16_t* silu;  size_t silu_len;
    const int16_t* exp;   size_t exp_len;
    const int16_t* cos;
    const int16_t* sin;   size_t rope_len;
} myl_luts;

/* The nine scalar activation fractional bits of one layer, in the order of
 * LayerScales (runtime/src/model.rs; filled by loader.rs:784-797 from the
 * scales.json keys <p>.input_layernorm, <p>.self_attn.{q,k,v}_proj,
 * <p>.self_attn, <p>.post_attention_layernorm, <p>.mlp.{gate,up}_proj and
 * <p>.mlp.down_proj.input). */
typedef struct myl_layer_fracs {
    uint8_t norm_attn_frac, q_frac, k_frac, v_frac, attn_out_frac;
    uint8_t norm_mlp_frac, gate_frac, up_frac, down_in_frac;
} myl_layer_fracs;

/* Dimensions of an artifact's model (model_config.json, loader.rs:240-275,
 * ModelDims) plus the LM-head form the artifact carries.  lm_head_int16 = 1:
 * an int16 LM head with per-row shifts (loader.rs:304-352, model.rs:285-296);
 * 0: the int8 head (lm_head.weight, or the embedding when tied;
 * model.rs:297-307). */
typedef struct myl_model_dims {
    uint32_t vocab, hidden, layers, heads, kv_heads, head_dim, inter;
    uint32_t max_context;
    int32_t  tie_word_embeddings;
    int32_t  attention_bias;
    int32_t  lm_head_int16;
} myl_model_dims;

/* Shape and seed of a synthetic integer model (Qwen2.5 layout, model.rs:94-163).
 * lm_head_int16 = 1 selects the int16 LM head (model.rs:285-296, path A);
 * 0 selects the tied int8 embedding (model.rs:297-307, path B). */
typedef struct myl_synth_spec {
    uint64_t seed;
    uint32_t vocab, hidden, layers, heads, kv_heads, head_dim, inter;
    uint32_t max_pos;        /* KV-cache capacity in positions */
    int32_t  lm_head_int16;
    int32_t  attention_bias; /* Qwen2.5 carries q/k/v biases (loader.rs:751-781) */
} myl_synth_spec;

/* Shape and seed of a synthetic integer MoE layer (Qwen1.5-MoE-A2.7B shape:
 * hidden 2048, 60 routed experts of intermediate 1408, top-4, one shared
 * expert of intermediate 5632).  The reference has no MoE; the layer's
 * integer semantics are the build's own, composed from reference primitives
 * (include/myl_hip.h, myl_moe_forward). */
typedef struct myl_moe_spec {
    uint64_t seed;
    uint32_t hidden, n_experts, inter, top_k, shared_inter;
} myl_moe_spec;

#ifdef __cplusplus
}
#endif

#endif /* MYL_THETA_V_H */
