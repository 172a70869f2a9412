/*
 * myl_hip.h -- C ABI of libmyl_hip.so, the MI355X (gfx950) backend of the
 * INTEGER_LLM integer forward path.
 *
 * Plain C types only (pointers, sizes, fixed-width integers): this is the
 * surface a Rust `RocmBackend` (INTEGER_LLM/kernels/src/backends/rocm.rs)
 * binds through `extern "C"`, replacing the delegating stub.  Every compute
 * entry point is bit-identical to the reference Rust kernel it names.
 *
 * Sections:
 *   1. Backend-trait mirror (host slices in, host slices out), one function per
 *      method of `trait Backend` (INTEGER_LLM/kernels/src/backend.rs:23-127) and
 *      per free function that runtime/src/model.rs calls directly
 *      (model.rs:16-22).  Slices are copied to and from the device per call,
 *      like the reference passes weights per call (linear.rs:43-50).
 *   2. Device-pointer forms (`*_dev`): the same arithmetic on device buffers,
 *      asynchronous on the context's stream, with a batch dimension M.
 *   3. A device-resident model (`myl_model_*`): forward_token / run_layers /
 *      head_logits of runtime/src/model.rs:229-399 with weights uploaded once
 *      and the KV cache of runtime/src/kv_cache.rs held in HBM; batched rows
 *      over per-sequence KV caches.
 *   4. An integer MoE layer (`myl_moe_*`, build-defined).
 *   5. The reference's artifact directory format (`myl_artifact_*`,
 *      runtime/src/loader.rs) and tensor uploads into a device model.
 *
 * Status codes: 0 = ok; MYL_E_INVALID where the reference panics (assert!,
 * empty slices, length mismatches); MYL_E_HIP for runtime failures;
 * MYL_E_NOMEM; MYL_E_UNSUPPORTED.  myl_last_error() returns the message of the
 * last failure on a context.
 *
 * Threading: one context per device; calls on one context must be serialised
 * by the caller (the trait's `&self` methods map onto a Mutex in the shim).
 */
#ifndef MYL_HIP_H
#define MYL_HIP_H

#include <stddef.h>
#include <stdint.h>

#include "myl_theta_v.h"

#ifdef __cplusplus
extern "C" {
#endif

#define MYL_OK 0
#define MYL_E_INVALID (-1)
#define MYL_E_HIP (-2)
#define MYL_E_NOMEM (-3)
#define MYL_E_UNSUPPORTED (-4)

typedef struct myl_ctx myl_ctx;
typedef struct myl_model myl_model;
typedef struct myl_moe myl_moe;

/* ---- backend identity: rocm.rs:71-82 (name / hardware_family / feature_tag) */
const char* myl_backend_name(void);     /* "rocm"    */
const char* myl_hardware_family(void);  /* "amd-gpu" */
const char* myl_feature_tag(void);      /* "rocm"    */

/* ---- context: RocmBackend::init(device_id) -> Result<Self, String> (rocm.rs:54-59) */
int myl_init(int device_id, myl_ctx** out);
void myl_destroy(myl_ctx* ctx);
const char* myl_last_error(const myl_ctx* ctx);
/* The real gcnArchName (e.g. "gfx950:sramecc+:xnack-") in place of the stub's
 * hard-coded "gfx90a" (rocm.rs:58); cu_count / hbm_bytes may be NULL. */
int myl_device_info(const myl_ctx* ctx, char* gcn_arch, size_t cap, int* cu_count, uint64_t* hbm_bytes);
int myl_synchronize(myl_ctx* ctx);
void* myl_stream(myl_ctx* ctx); /* the hipStream_t all *_dev calls use */
/* Use the caller's stream (hipStream_t) for all later calls; NULL restores the
 * context's own stream.  The caller keeps ownership. */
int myl_set_stream(myl_ctx* ctx, void* stream);

/* ---- device memory for callers without their own allocator ------------- */
/* No counterpart in the reference: a measurement of the achievable read rate
 * for the roofline figures.  Enqueues one pass of 16-byte nontemporal loads
 * (the cache policy of the GEMV weight streams) over
 * `bytes` of device memory at p (16-byte aligned, bytes % 16 == 0), one block
 * of 512 threads per CU; `out` (one device word) receives at most one
 * word. */
int myl_read_probe(myl_ctx* ctx, const void* p, size_t bytes, uint32_t* out);
int myl_malloc(myl_ctx* ctx, size_t bytes, void** dptr);
int myl_free(myl_ctx* ctx, void* dptr);
int myl_memcpy_htod(myl_ctx* ctx, void* dst, const void* src, size_t bytes);
int myl_memcpy_dtoh(myl_ctx* ctx, void* dst, const void* src, size_t bytes);

/* ======================================================================
 * 1. Backend-trait mirror (host slices)
 * ==================================================================== */

/* Backend::linear_w8a16 (backend.rs:39-49) == linear.rs:43-70.
 * W is flat row-major [out_features x in_features]. */
int myl_linear_w8a16(myl_ctx* ctx, const int16_t* x, const int8_t* W, int16_t* out, size_t in_features,
                     size_t out_features, const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac);

/* linear.rs:87-119 (o_proj / down_proj, per-channel output scale; model.rs:582,618). */
int myl_linear_w8a16_pc(myl_ctx* ctx, const int16_t* x, const int8_t* W, int16_t* out, size_t in_features,
                        size_t out_features, const uint8_t* w_shifts, uint8_t act_frac, const uint8_t* out_frac);

/* linear.rs:132-145 (in place on out). */
int myl_add_bias_i16(myl_ctx* ctx, int16_t* out, const int16_t* bias, const uint8_t* bias_shifts, size_t n,
                     uint8_t out_frac);

/* Backend::rmsnorm (backend.rs:54-66) == rmsnorm.rs:61-161. */
int myl_rmsnorm(myl_ctx* ctx, const int16_t* x, const uint8_t* x_shifts, const int8_t* gamma,
                const uint8_t* gamma_shifts, size_t n, const int16_t* rsqrt_lut, size_t lut_len,
                uint8_t lut_input_shift, uint8_t lut_output_frac, int64_t inv_n_q20, int16_t* out, uint8_t out_frac);

/* Backend::softmax (backend.rs:69-75) == softmax.rs:24-64. */
int myl_softmax(myl_ctx* ctx, const int32_t* logits, int32_t* out, size_t n, const int16_t* exp_lut,
                size_t lut_len, uint8_t lut_shift, uint8_t frac_bits);

/* Backend::attention (backend.rs:79-91) == attention.rs:42-90.  The Vec<Vec<i16>>
 * arguments are flattened: q/out [q_len x head_dim], k/v [kv_len x head_dim];
 * mask is [q_len x kv_len] bytes (nonzero = attend) or NULL for all-true. */
int myl_attention(myl_ctx* ctx, const int16_t* q, const int16_t* k, const int16_t* v, int16_t* out,
                  size_t q_len, size_t kv_len, size_t head_dim, const uint8_t* mask, int64_t score_mult,
                  uint8_t score_shift, const int16_t* exp_lut, size_t lut_len, uint8_t lut_shift, uint8_t prob_frac);

/* Backend::rope (backend.rs:94-101) == rope.rs:36-59, in place on q and k
 * ([n x head_dim] each); LUT row = positions[i] % (lut_len / (head_dim/2)). */
int myl_rope(myl_ctx* ctx, int16_t* q, int16_t* k, size_t n, size_t head_dim, const int16_t* cos_lut,
             const int16_t* sin_lut, size_t lut_len, const uint64_t* positions, uint8_t frac_bits);

/* Backend::mlp (backend.rs:107-126) == mlp.rs:28-74; intermediate size is
 * inferred from the slice lengths as in rocm.rs:183-186 (given explicitly here). */
int myl_mlp(myl_ctx* ctx, const int16_t* x, const int8_t* W_gate, const int8_t* W_up, const int8_t* W_down,
            int16_t* out, size_t hidden, size_t inter, const uint8_t* gate_w_shifts, const uint8_t* up_w_shifts,
            const uint8_t* down_w_shifts, const int16_t* silu_lut, size_t silu_len, uint8_t in_frac,
            uint8_t gate_out_frac, uint8_t up_out_frac, uint8_t down_in_frac, uint8_t silu_in_frac,
            int16_t silu_lut_offset, uint8_t silu_out_frac, const uint8_t* out_frac);

/* sampling.rs:8-18 (first maximum wins); *out_index receives the token id. */
int myl_argmax_int(myl_ctx* ctx, const int32_t* values, size_t n, int64_t* out_index);

/* sample_integer_cdf (sampling.rs:27-46, called by IntegerModel::sample_next,
 * model.rs:785-787): weights z - min z + 1 (i32, wrapping), SplitMix64
 * (prng.rs:7-14) draw r, threshold r % total, the first token whose running
 * weight sum exceeds it; total <= 0 (or no logits) gives token 0 and the
 * state unchanged.  *token and *new_state receive the result. */
int myl_sample_integer_cdf(myl_ctx* ctx, const int32_t* logits, size_t n, uint64_t state, int64_t* token,
                           uint64_t* new_state);

/* ======================================================================
 * 2. Device-pointer forms (asynchronous on myl_stream(ctx))
 * ==================================================================== */

/* M independent linear_w8a16 / linear_w8a16_pc calls: x [M x K] (row stride
 * ldx), W [N x K], out [M x N] (row stride ldo).  out_frac_pc = NULL selects
 * the scalar out_frac (linear.rs:43-70), else per channel (linear.rs:87-119). */
int myl_linear_w8a16_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N,
                         size_t K, const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac,
                         const uint8_t* out_frac_pc, int16_t* out, size_t ldo);

/* Multiplier + shift requantization (no reference counterpart: a superset of
 * linear.rs's power-of-two rescale): out = clamp_i16(RNE(dot * mult[r], shift[r]))
 * in 128-bit arithmetic.  mult = 2^k, shift = k + w_shift + act_frac - out_frac
 * reproduces myl_linear_w8a16_dev exactly whenever that shift is >= 0. */
int myl_linear_w8a16_mult_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N,
                              size_t K, const int32_t* mult, const uint8_t* shift, int16_t* out, size_t ldo);

/* No counterpart in the reference: myl_linear_w8a16_dev for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  Same arguments and results; it
 * calls no hipMalloc / hipFree.  Its scratch (activation byte planes and
 * split-K partial sums) is one fixed device array per GPU of
 * myl_noalloc_scratch_bytes() bytes, held until the process ends: 2 * M * K
 * must not exceed 4 MiB when M >= 2 (MYL_E_INVALID otherwise; one row needs
 * no scratch).  Calls that overlap on one GPU share that array and race; the
 * caller orders them. */
int myl_linear_w8a16_dev_noalloc(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N,
                                 size_t K, const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac,
                                 const uint8_t* out_frac_pc, int16_t* out, size_t ldo);
/* Bytes of the per-GPU scratch array of myl_linear_w8a16_dev_noalloc. */
size_t myl_noalloc_scratch_bytes(void);

/* LM head (model.rs:284-308): logits[m][r] = clamp_i32(rescale_i64(W[r].x[m],
 * row_shifts[r] + norm_frac, logit_frac)); w_bits = 16 for the int16 head
 * (path A), 8 for the tied int8 embedding (path B). */
int myl_logits_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const void* W, int w_bits, size_t N,
                   size_t K, const uint8_t* row_shifts, uint8_t norm_frac, uint8_t logit_frac, int32_t* out,
                   size_t ldo);

/* Exact i64 dot products (dot.rs:141-147) of M activation rows with N weight rows. */
int myl_dot_i8_i16_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N, size_t K,
                       int64_t* out, size_t ldo);

/* M rows of rmsnorm_i16 (rmsnorm.rs:61-161), shared x_shifts / gamma. */
int myl_rmsnorm_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const uint8_t* x_shifts,
                    const int8_t* gamma, const uint8_t* gamma_shifts, size_t n, const int16_t* rsqrt_lut,
                    size_t lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac, int64_t inv_n_q20,
                    uint8_t out_frac, int16_t* out, size_t ldo);

/* M rows of softmax_int (softmax.rs:24-64). */
int myl_softmax_dev(myl_ctx* ctx, const int32_t* logits, size_t M, size_t n, size_t ldz, const int16_t* exp_lut,
                    size_t lut_len, uint8_t lut_shift, uint8_t frac_bits, int32_t* out, size_t ldo);

/* M rows of argmax_int (sampling.rs:8-18). */
int myl_argmax_dev(myl_ctx* ctx, const int32_t* values, size_t M, size_t n, size_t ldv, int64_t* out_index);

/* M rows of sample_integer_cdf (sampling.rs:27-46): row m at states[m] gives
 * tokens[m] and new_states[m] (all device pointers). */
int myl_sample_dev(myl_ctx* ctx, const int32_t* logits, size_t M, size_t n, size_t ldz, const uint64_t* states,
                   int64_t* tokens, uint64_t* new_states);

/* Integer log-softmax at a target token per row (no reference counterpart:
 * the reference evaluates perplexity in f64, runtime/src/bin/perplexity_probe.rs:55-67).
 * For logits z (Q6, model.rs:284-308) and target t:
 *   m = max z;  S = sum_j exp_lut[(m - z_j) << 2] (0 past the table);
 *   out = (z_t - m) * 2^10 - ln_q16(S)   (Q16, int64)
 * where ln_q16(S) = RNE((((e - 14) << 16) + f) * 744261118, 30) with
 * e = floor(log2 S) and f the first 16 fraction bits of log2(S / 2^e) by
 * repeated squaring of the Q62 mantissa.  targets[m] < 0 gives 0. */
int myl_logsoftmax_dev(myl_ctx* ctx, const int32_t* logits, size_t M, size_t n, size_t ldz, const int16_t* exp_lut,
                       size_t lut_len, const int64_t* targets, int64_t* out);

/* ======================================================================
 * 3. Device-resident model (runtime/src/model.rs, kv_cache.rs)
 * ==================================================================== */

/* Builds the seeded synthetic model of include/myl_synth.h directly in HBM
 * (weights are generated on the device; the LUTs are uploaded). */
int myl_model_create_synthetic(myl_ctx* ctx, const myl_synth_spec* spec, const myl_luts* luts, myl_model** out);
void myl_model_destroy(myl_model* m);
/* Empties the KV cache (KVCache::new, kv_cache.rs:14-16). */
int myl_model_reset(myl_model* m);
/* IntegerModel::forward_token (model.rs:229-311) for one token at position pos.
 * logits (host, vocab entries) may be NULL; argmax (host) may be NULL.
 * Positions must be written contiguously from 0 (the generate loop,
 * generate.rs:28-50). */
int myl_model_forward_token(myl_model* m, uint32_t token, uint32_t pos, int32_t* logits, int64_t* argmax);
/* Greedy decode: n_steps tokens after `token` at `pos` (generate.rs:38-50),
 * each step's argmax feeding the next without a host round trip.  tokens_out
 * (host, n_steps) receives the chosen ids; logits_out (host, n_steps x vocab)
 * may be NULL. */
int myl_model_decode_greedy(myl_model* m, uint32_t token, uint32_t pos, uint32_t n_steps, int64_t* tokens_out,
                            int32_t* logits_out);
/* The prompt loop of generate.rs:28-32: tokens[i] at position pos0 + i, the
 * KV cache filled exactly as by n forward_token calls.  Only the last
 * position's logits are computed (earlier ones are discarded by the
 * reference's loop); last_logits (host, vocab) may be NULL. */
int myl_model_prefill(myl_model* m, const uint32_t* tokens, uint32_t n, uint32_t pos0, int32_t* last_logits);
/* Greedy steps after the first replay one captured HIP graph (default on);
 * enable = 0 launches every kernel from the host instead. */
int myl_model_set_graphs(myl_model* m, int enable);
/* No counterpart in the reference: a measurement hook for callers that time a
 * kernel class inside the captured decode step.  Launches the class's kernel
 * `times` (1-4, at most the number of layers) times per layer and step: the
 * first as usual, each repeat with the same launch shape over the weights of
 * layer l + 1, l + 2, ... (wrapping to the first layers: weights the step read
 * at least a layer's traffic earlier, which no longer sit in the caches) into
 * scratch output rows, so every output of the step is unchanged.  Only the
 * gate/up class (kclass 5 of the timing order below) is accepted;
 * myl_model_timing does not count the repeats.  The next greedy decode
 * recaptures its step graph. */
int myl_model_set_kernel_repeat(myl_model* m, int kclass, int times);
/* Per-kernel-class timing with HIP events around each launch (eager launches,
 * no graphs while enabled).  enable = 1 starts; enable = 0 stops and returns
 * per class the summed milliseconds and launch counts in the order embed,
 * rmsnorm, qkv, attention, o_proj, gate_up, down, lm_head (8 entries each). */
int myl_model_timing(myl_model* m, int enable, double* ms_out, uint64_t* counts_out);
/* IntegerModel::embed_token (model.rs:323-331): hidden (host, hidden entries). */
int myl_model_embed_token(myl_model* m, uint32_t token, int16_t* hidden);
/* IntegerModel::run_layers (model.rs:339-356), hidden in/out on the host. */
int myl_model_run_layers(myl_model* m, int16_t* hidden, uint32_t pos, uint32_t layer_start, uint32_t layer_end);
/* IntegerModel::head_logits (model.rs:360-399). */
int myl_model_head_logits(myl_model* m, const int16_t* hidden, int32_t* logits);
/* KVCache::read (kv_cache.rs:43-52) for positions [0, n_pos): k/v [n_pos x head_dim]. */
int myl_model_read_kv(myl_model* m, uint32_t layer, uint32_t kv_head, uint32_t n_pos, int16_t* k_out,
                      int16_t* v_out);
/* Device copy of a named weight tensor (the synthetic generator's output),
 * for verification; same names as the oracle's tensor table. */
int myl_model_read_tensor(myl_model* m, const char* name, uint32_t layer, void* host_out, size_t bytes);

/* ---- batched forward: rows of (sequence, position, token) -------------------
 * Generalises the prompt loop of generate.rs:28-32 to many sequences with
 * their own KV caches; row r computes what IntegerModel::forward_token
 * (model.rs:229-311) computes for token[r] at pos[r] on sequence seq[r].
 * The row path splits attention probabilities into bytes, so it returns
 * MYL_E_UNSUPPORTED for models with more than 16 query heads per KV head, an
 * exp table with negative entries, or one whose sum over max_pos positions
 * could pass 2^31 - 1 (myl_model_prefill then runs the token loop). */

/* Allocates KV caches for n_seqs sequences (max_pos positions each, separate
 * from the single-sequence cache) and empties them. */
int myl_model_batch_begin(myl_model* m, uint32_t n_seqs);
/* One forward over n_rows rows.  Per sequence the rows' positions must be
 * distinct, contiguous and start at or before its cached length (a re-run
 * position overwrites, as KVCache::write does).  logits (host, n_rows x vocab)
 * and argmax_out (host, n_rows; first maximum, sampling.rs:8-18) may be NULL. */
int myl_model_forward_batch(myl_model* m, uint32_t n_rows, const uint32_t* seq, const uint32_t* pos,
                            const uint32_t* tokens, int32_t* logits, int64_t* argmax_out);
/* Device pointer of the last batch's logits ([n_rows x vocab] int32), valid
 * until the next batched call. */
int myl_model_batch_logits_dev(myl_model* m, const int32_t** logits_dev);
/* Greedy decode of n_rows sequences in lock step (generate.rs:38-50 per
 * sequence): step 0 consumes tokens[r] at pos[r], step i the argmax of step
 * i-1 at pos[r] + i.  tokens_out (host, n_steps x n_rows) gets the argmax of
 * every step. */
int myl_model_batch_decode_greedy(myl_model* m, uint32_t n_rows, const uint32_t* seq, const uint32_t* pos,
                                  const uint32_t* tokens, uint32_t n_steps, int64_t* tokens_out);
/* KVCache::read (kv_cache.rs:43-52) of one batch sequence. */
int myl_model_batch_read_kv(myl_model* m, uint32_t seq, uint32_t layer, uint32_t kv_head, uint32_t n_pos,
                            int16_t* k_out, int16_t* v_out);

/* ======================================================================
 * 4. Integer MoE layer (no reference counterpart: the reference is dense,
 *    README/Whitepaper/myelith-whitepaper-v0.3-en.md:662).  Semantics, each
 *    step a reference primitive:
 *      router   r_e = clamp_i32(clamp_i32(rescale_i64(W_r[e] . x, 15 + 8, 8)) + bias_e)
 *               (LM-head requant, model.rs:284-308; Q8 logits)
 *      top-k    k first maxima, lowest index on ties (sampling.rs:8-18)
 *      gates    softmax_int of the k logits, shift 0, frac 14 (softmax.rs:24-64)
 *      dispatch per expert, its tokens in ascending token order
 *      experts  mlp_int (mlp.rs:28-74); shared expert likewise
 *      combine  clamp_i16(RNE(sum_k g_k y_k + 2^14 s, 14)) in i64
 * ==================================================================== */

/* Builds the seeded synthetic layer of include/myl_synth.h in HBM;
 * router_bias holds n_experts Q8 biases. */
int myl_moe_create_synthetic(myl_ctx* ctx, const myl_moe_spec* spec, const int32_t* router_bias, const myl_luts* luts,
                             myl_moe** out);
void myl_moe_destroy(myl_moe* m);
/* The layer's synthetic input for n_tokens tokens (device, [n_tokens x hidden]). */
int myl_moe_synth_input(myl_moe* m, uint32_t n_tokens, int16_t* x_dev);
/* out_dev [n_tokens x hidden] = the layer on x_dev [n_tokens x hidden] (device,
 * 16-byte aligned).  When hidden and the intermediate widths are multiples of
 * 64 the whole layer is planned on the device (expert offsets and the grouped
 * products' work tables from the token counts) and nothing waits for the
 * host; other widths synchronise once with the host, whose work tables size
 * the grouped products. */
int myl_moe_forward(myl_moe* m, const int16_t* x_dev, uint32_t n_tokens, int16_t* out_dev);
/* Routing of the last forward (host arrays, any may be NULL): ids and gates
 * [n_tokens x top_k] (descending logit, lowest expert first on ties), counts
 * [n_experts], offsets [n_experts + 1], list_tok [n_tokens x top_k] (expert-
 * major, ascending token order within an expert). */
int myl_moe_read_route(myl_moe* m, uint32_t n_tokens, int32_t* ids, int32_t* gates, int32_t* counts, int32_t* offsets,
                       int32_t* list_tok);

/* ====================================================================
 * 5. Artifacts: the reference's model directory format and the uploader
 *
 * An artifact directory (runtime/src/loader.rs:322-600) holds theta_v.json,
 * model_config.json, weights_manifest.json with one raw little-endian file
 * per tensor (+ a _shifts.bin of one u8 per row), scales.json and luts.json
 * with its *.lut.bin tables.  myl_artifact_open() performs every check of
 * load_model (loader.rs:611-636) and build_model (:712-849) that does not
 * need the tensor bytes: theta_v version against MYL_TV_VERSION, the SHA-256
 * of the three manifest files against theta_v.json, model_config.json
 * dimensions, manifest dtype / shape / file size rules, shift ranges,
 * scale = 2^-shift, per-channel shift lengths, the LUT tables (read and
 * hashed), and the presence of every tensor, scale and LUT the model consumes.
 * Tensor files are hashed by myl_artifact_verify() or while
 * myl_model_load_artifact() streams them to the device; a mismatch refuses
 * the artifact, as load_weights does (loader.rs:364-372).
 * ==================================================================== */

typedef struct myl_artifact myl_artifact;

/* Opens and checks an artifact directory.  On failure *out is NULL and the
 * message is written to err (err_cap bytes, may be 0). */
int myl_artifact_open(const char* dir, myl_artifact** out, char* err, size_t err_cap);
void myl_artifact_close(myl_artifact* a);
const char* myl_artifact_last_error(const myl_artifact* a);
int myl_artifact_dims(const myl_artifact* a, myl_model_dims* out);
/* Reads every tensor and shifts file of the manifest and checks its SHA-256
 * (loader.rs:364-399); host only. */
int myl_artifact_verify(myl_artifact* a);
/* A LUT by its luts.json key (cos, sin, exp, silu, rsqrt); *len = its length.
 * out may be NULL to query the length. */
int myl_artifact_lut(const myl_artifact* a, const char* name, int16_t* out, size_t cap, size_t* len);
/* The activation scales of one layer (loader.rs:784-797): nine scalar fracs
 * and the per-channel residual segments res_in / res_mid [hidden] (either may
 * be NULL). */
int myl_artifact_layer_scales(const myl_artifact* a, uint32_t layer, myl_layer_fracs* fracs, uint8_t* res_in,
                              uint8_t* res_mid);
/* model.norm (final_norm_frac) and model.norm.input [hidden] (loader.rs:737-742). */
int myl_artifact_final_scales(const myl_artifact* a, uint8_t* final_norm_frac, uint8_t* final_res);

/* SHA-256 of n bytes as 64 lowercase hex digits plus NUL (loader.rs:600-605). */
int myl_sha256_hex(const void* data, size_t n, char out[65]);

/* Builds the device model of an opened artifact with a KV cache of max_pos
 * positions (0 = model_config max_context): the tensors are streamed from
 * their files through pinned staging buffers to HBM and hashed on the way.
 * The model is ready for every myl_model_* call. */
int myl_model_load_artifact(myl_ctx* ctx, const myl_artifact* a, uint32_t max_pos, myl_model** out);

/* An empty device model of the given dimensions and LUTs (the shape of
 * build_model, loader.rs:712-849), filled by the calls below and sealed by
 * myl_model_finalize().  This is the path for a host that loads artifacts
 * itself (the Rust loader.rs) and hands over the tensors of its IntegerModel. */
int myl_model_create(myl_ctx* ctx, const myl_model_dims* dims, uint32_t max_pos, const myl_luts* luts,
                     myl_model** out);
/* Uploads one tensor by its reference name (the HF original_name of the
 * manifest): model.embed_tokens.weight, model.norm.weight, lm_head.weight
 * (bits 8: the untied int8 head; bits 16: the int16 head),
 * model.layers.<l>.{input_layernorm,post_attention_layernorm}.weight,
 * model.layers.<l>.self_attn.{q,k,v,o}_proj.weight,
 * model.layers.<l>.mlp.{gate,up,down}_proj.weight and, with attention_bias,
 * model.layers.<l>.self_attn.{q,k,v}_proj.bias (int16).  data is the
 * row-major tensor (int8, or int16 for bits 16), shape its dimensions, and
 * shifts one u8 per row (per element for 1-D tensors), n_shifts = shape[0].
 * The int8 lm_head.weight of an artifact that also carries the int16 head is
 * accepted and not stored (model.rs:285 reads only the int16 head then). */
int myl_model_upload_tensor(myl_model* m, const char* name, const void* data, int bits, const uint64_t* shape,
                            uint32_t ndim, const uint8_t* shifts, size_t n_shifts);
/* The inverse: the tensor in the reference layout and its per-row shifts
 * (bytes = element count * bits / 8; shifts may be NULL). */
int myl_model_download_tensor(myl_model* m, const char* name, int bits, void* data, size_t bytes, uint8_t* shifts,
                              size_t n_shifts);
/* LayerScales of one layer (loader.rs:784-797) and the final segment. */
int myl_model_set_layer_scales(myl_model* m, uint32_t layer, const myl_layer_fracs* fracs, const uint8_t* res_in,
                               const uint8_t* res_mid);
int myl_model_set_final_scales(myl_model* m, uint8_t final_norm_frac, const uint8_t* final_res);
/* Reads the scales back (either array may be NULL). */
int myl_model_get_layer_scales(myl_model* m, uint32_t layer, myl_layer_fracs* fracs, uint8_t* res_in,
                               uint8_t* res_mid);
int myl_model_get_final_scales(myl_model* m, uint8_t* final_norm_frac, uint8_t* final_res);
/* Checks that every tensor and scale has arrived (the require_* checks of
 * loader.rs:690-710, naming the first missing item) and derives the
 * per-channel accumulation scales.  Forward calls fail until it succeeds. */
int myl_model_finalize(myl_model* m);

#ifdef __cplusplus
}
#endif

#endif /* MYL_HIP_H */
