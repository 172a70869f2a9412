// model_internal.h -- the device-resident model object shared by the decode
// step (model.hip) and the batched forward (batch.hip).
#pragma once

#include "abi_internal.h"
#include "../../include/myl_synth.h"

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
    int8_t* final_gamma = nullptr;
    uint8_t* final_gamma_s = nullptr;
    uint8_t* final_res = nullptr;
    uint8_t final_norm_frac = 0;
    int16_t *rsqrt = nullptr, *silu = nullptr, *exp_lut = nullptr, *cos_lut = nullptr, *sin_lut = nullptr;
    int rsqrt_len = 0, silu_len = 0, exp_len = 0;
    int64_t inv_n_q20 = 0;
    int64_t score_mult = 0;
    // caches and activations
    int16_t *kcache = nullptr, *vcache = nullptr;
    int16_t *hidden = nullptr, *norm = nullptr, *q = nullptr, *attn = nullptr, *resid = nullptr, *h = nullptr;
    int32_t* logits = nullptr;
    int32_t* scores = nullptr;
    unsigned long long* attn_acc = nullptr;  // [nq] exact P.V sums, cleared after each use
    NormAcc* norm_a = nullptr;               // input-norm / final-norm sums of squares
    NormAcc* norm_b = nullptr;               // post-attention-norm sums of squares
    uint8_t ref_final = 0;
    int cus = 0;
    DecodeState* state = nullptr;
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
    ~myl_model() {
        if (ctx) (void)hipStreamSynchronize(ctx->stream);
        if (step_exec) (void)hipGraphExecDestroy(step_exec);
        if (step_graph) (void)hipGraphDestroy(step_graph);
        for (hipEvent_t e : ev_pool) (void)hipEventDestroy(e);
        if (batch) myl::batch_free(batch);
        for (void* p : allocs) (void)hipFree(p);
    }
};

