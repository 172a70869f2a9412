// model_internal.h -- the device-resident model object shared by the decode
// step (model.hip) and the batched forward (batch.hip).
#pragma once

#include "abi_internal.h"
#include "../../include/myl_synth.h"

#include <string>
#include <utility>
#include <vector>

namespace myl {

// Per-step state of the single-sequence decode, in device memory.
struct DecodeState {
    uint64_t argmax_key;  // packed (value, ~index) of the best logit so far
    int32_t token;
    int32_t pos;
    int32_t rope_row;     // pos % rope rows
    int32_t step;         // decode steps taken since the last set
};

// Exact sum of squares of a residual-stream vector for the next RMSNorm,
// as 42-bit limbs in u64 spread over 64 slots.
constexpr int kNormSlots = 64;
constexpr uint64_t kLimbMask = (1ull << 42) - 1;
struct NormAcc { unsigned long long v[kNormSlots][3]; };

struct LayerDev {
    int8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;
    // fragment-major copies of wqkv, wgu and wd for the decode-batch
    // products (gemm_frag.h), built on first use
    int8_t *wqkv_f = nullptr, *wgu_f = nullptr, *wd_f = nullptr;
    uint8_t *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sd = nullptr;
    int16_t* bqkv = nullptr;
    uint8_t* bsqkv = nullptr;
    int8_t *in_gamma = nullptr, *post_gamma = nullptr;
    uint8_t *in_gamma_s = nullptr, *post_gamma_s = nullptr;
    uint8_t *res_in = nullptr, *res_mid = nullptr, *acc_attn = nullptr, *acc_mlp = nullptr;
    const uint8_t* res_out = nullptr;  // next layer's res_in or the final segment
    uint8_t ref_in = 0, ref_mid = 0, ref_out = 0;  // max of res_in / res_mid / res_out (rmsnorm.rs:96)
    myl_layer_fracs f{};
};

struct BatchState;  // batch.hip
void batch_free(BatchState* b);
// A prompt of n >= kPromptRows tokens at positions pos0.. as one batch of
// rows over the model's own KV cache (batch.hip); writes the last logits to
// the model's logits.  Returns MYL_E_UNSUPPORTED when the row path cannot
// take this model (then the caller runs the tokens one at a time).
constexpr uint32_t kPromptRows = 16;
int prompt_rows(myl_model* m, const uint32_t* tokens, uint32_t n, uint32_t pos0);

// What a model receives before it is sealed: model-wide tensors, then
// kLayerSlots tensors per layer (index kModelSlots + layer * kLayerSlots + slot).
enum ModelSlot { SLOT_EMB, SLOT_LM8, SLOT_LM16, SLOT_FINAL_GAMMA, kModelSlots };
enum LayerSlot {
    SLOT_IN_GAMMA, SLOT_POST_GAMMA, SLOT_Q, SLOT_K, SLOT_V, SLOT_O, SLOT_GATE, SLOT_UP, SLOT_DOWN,
    SLOT_BQ, SLOT_BK, SLOT_BV, kLayerSlots
};

}  // namespace myl

using myl::DecodeState;
using myl::LayerDev;
using myl::NormAcc;

struct myl_model {
    myl_ctx* ctx = nullptr;
    myl_synth_spec spec{};
    int H = 0, I = 0, V = 0, hd = 0, hd_log = 0, G = 0, nq = 0, nkv = 0, max_pos = 0;
    uint32_t rope_rows = 0;
    std::vector<void*> allocs;
    std::vector<LayerDev> layers;
    // model-wide tensors
    int8_t* emb = nullptr;
    uint8_t* emb_shifts = nullptr;
    int16_t* lm16 = nullptr;
    uint8_t* lm16_shifts = nullptr;
    // byte planes of lm16 [2V x H] and its row sums, for the many-row head
    // product; built on first use, invalidated by an upload of the head
    int8_t* lm16_planes = nullptr;
    int32_t* lm16_wsum = nullptr;
    bool lm16_planes_ok = false;
    // the layers' fragment-major q/k/v, gate/up and down copies: 0 not built (or a
    // weight upload since), 1 current, -1 not available (shapes or memory)
    int frag_state = 0;
    int8_t* final_gamma = nullptr;
    uint8_t* final_gamma_s = nullptr;
    uint8_t* final_res = nullptr;
    uint8_t final_norm_frac = 0;
    // the int8 LM head (model.rs:297-307): the embedding when tied, else its own
    bool tied = true;
    int8_t* lm8 = nullptr;
    uint8_t* lm8_shifts = nullptr;
    // stored row of each logical output row (q/k/v pair-ordered, gate/up interleaved)
    std::vector<int32_t> qkv_map, gu_map;
    int32_t *qkv_map_dev = nullptr, *gu_map_dev = nullptr;
    // host copies of the per-channel residual scales, and what has arrived
    std::vector<std::vector<uint8_t>> h_res_in, h_res_mid;
    std::vector<uint8_t> h_final_res;
    std::vector<uint8_t> have;         // per ModelSlot / LayerSlot
    std::vector<uint8_t> scales_have;  // per layer
    bool final_have = false;
    bool ready = false;                // sealed by myl::model_finalize
    void* io = nullptr;                // upload staging (model_io.hip) while tensors arrive
    void (*io_free)(void*) = nullptr;
    int16_t *rsqrt = nullptr, *silu = nullptr, *exp_lut = nullptr, *cos_lut = nullptr, *sin_lut = nullptr;
    int rsqrt_len = 0, silu_len = 0, exp_len = 0;
    uint8_t rsqrt_closed = 0;  // the rsqrt table equals its closed form (RmsParams::closed)
    int exp_nz = 0;  // exp-table entries up to its last nonzero one
    bool pv32 = false;  // decode P.V by the wide-chunk kernel in i32 (attn_acc holds int32 sums)
    int gu_repeat = 1;  // launches of each layer's gate/up GEMV per step (myl_model_set_kernel_repeat)
    int16_t* h_scratch = nullptr;  // output rows of the repeated launches
    int64_t inv_n_q20 = 0;
    int64_t score_mult = 0;
    // caches and activations
    int16_t *kcache = nullptr, *vcache = nullptr;
    int16_t *hidden = nullptr, *norm = nullptr, *q = nullptr, *attn = nullptr, *resid = nullptr, *h = nullptr;
    int32_t* logits = nullptr;
    int32_t* scores = nullptr;  // [heads][score_ld] decode attention scores
    int score_ld = 0;           // max_pos rounded up to 4 (16-byte aligned rows)
    unsigned long long* attn_acc = nullptr;  // [nq] exact P.V sums (i64, or i32 when pv32), cleared after each use
    NormAcc* norm_a = nullptr;               // input-norm / final-norm sums of squares
    NormAcc* norm_b = nullptr;               // post-attention-norm sums of squares
    uint8_t ref_final = 0;
    int cus = 0;
    DecodeState* state = nullptr;
    int16_t* rope_cur = nullptr;  // the step's RoPE row: cos [hd / 2] then sin [hd / 2]
    int64_t* tokens_dev = nullptr;
    uint32_t tokens_cap = 0;
    uint32_t n_cached = 0;
    // decode step captured as a HIP graph (replayed per greedy step)
    bool use_graphs = true;
    hipGraph_t step_graph = nullptr;
    hipGraphExec_t step_exec = nullptr;
    const int64_t* graph_tokens = nullptr;
    // per-kernel-class event timing (eager launches only)
    bool timing = false;
    std::vector<hipEvent_t> ev_pool;
    size_t ev_used = 0;
    std::vector<std::pair<int, size_t>> marks;  // (class, index of the start event; end = +1)

    template <class T> T* dalloc(size_t count) {
        void* p = nullptr;
        if (hipMalloc(&p, count * sizeof(T) ? count * sizeof(T) : 1) != hipSuccess) return nullptr;
        allocs.push_back(p);
        return (T*)p;
    }
    myl::BatchState* batch = nullptr;  // per-sequence KV caches and row buffers
    myl::BatchState* prompt = nullptr; // row buffers of batched prompts (KV: kcache / vcache)
    int prompt_ok = -1;                // row path usable for prompts: -1 not yet checked

    // MYL_OK when the model is sealed, else the error of a forward call.
    int not_ready() {
        return ready ? 0 : ctx->fail(MYL_E_INVALID, "model: not finalized (tensors or scales missing)");
    }
    ~myl_model() {
        if (ctx) (void)hipStreamSynchronize(ctx->stream);
        if (step_exec) (void)hipGraphExecDestroy(step_exec);
        if (step_graph) (void)hipGraphDestroy(step_graph);
        for (hipEvent_t e : ev_pool) (void)hipEventDestroy(e);
        if (batch) myl::batch_free(batch);
        if (prompt) myl::batch_free(prompt);
        if (io) io_free(io);
        for (void* p : allocs) (void)hipFree(p);
    }
};


namespace myl {

// Validates the dimensions, allocates the model and its buffers (model.hip).
int model_setup(myl_ctx* ctx, const myl_synth_spec& s, bool tied, const myl_luts* luts, myl_model** out);
// Checks completeness and derives the accumulation scales (model.hip).
int model_finalize(myl_model* m);

inline bool slot_required(const myl_model* m, size_t i) {
    if (i < (size_t)kModelSlots) {
        if (i == SLOT_LM8) return !m->tied && !m->spec.lm_head_int16;
        if (i == SLOT_LM16) return m->spec.lm_head_int16 != 0;
        return true;
    }
    const int t = (int)((i - kModelSlots) % kLayerSlots);
    return t < SLOT_BQ || m->spec.attention_bias;
}

// The reference name of a slot (the HF original_name of the manifest).
inline std::string slot_name(const myl_model* m, size_t i) {
    static const char* model_names[kModelSlots] = {"model.embed_tokens.weight", "lm_head.weight", "lm_head.weight",
                                                    "model.norm.weight"};
    static const char* layer_names[kLayerSlots] = {
        "input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
        "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.o_proj.weight", "mlp.gate_proj.weight",
        "mlp.up_proj.weight", "mlp.down_proj.weight", "self_attn.q_proj.bias", "self_attn.k_proj.bias",
        "self_attn.v_proj.bias"};
    (void)m;
    if (i < (size_t)kModelSlots) return model_names[i];
    const size_t l = (i - kModelSlots) / kLayerSlots, t = (i - kModelSlots) % kLayerSlots;
    return "model.layers." + std::to_string(l) + "." + layer_names[t];
}

}  // namespace myl
