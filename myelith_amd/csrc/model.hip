// model.hip -- the device-resident integer model: IntegerModel::forward_token
// (INTEGER_LLM/runtime/src/model.rs:229-311, forward_layer :401-674) with the
// KV cache of runtime/src/kv_cache.rs held in HBM.
//
// One decode step is a fixed sequence of kernels on the context stream whose
// per-step inputs (token, position, LUT row) live in a device-side state word,
// so a greedy decode chains steps without host round trips:
//
//   embed          state <- token/pos; hidden = rescale(E[tok]) (model.rs:241-248)
//   per layer:
//     rmsnorm      input_layernorm                                 (:416-426)
//     gemv qkv     q/k/v rows + bias + RoPE, K/V appended to cache (:438-503)
//     attn_scores  s_j = (i32)RNE(q.k_j * mult, shift)             (attention.rs:66-67)
//     attn_stats   max, sum of exp-LUT, reciprocal of the sum      (softmax.rs:32-48)
//     attn_pv      p_j = RNE(e_j * 2^14 / S), partial sum p_j v_j  (softmax.rs:50-63, attention.rs:75-81)
//     attn_reduce  RNE(., 14), clamp, rescale v -> attn_out        (attention.rs:84-86, model.rs:563-567)
//     gemv o       o_proj + residual add 1                         (:576-593)
//     rmsnorm      post_attention_layernorm                        (:596-606)
//     gemv gate/up gate, up interleaved, SiLU-LUT product           (mlp.rs:55-65)
//     gemv down    down_proj + residual add 2                      (:612-671)
//   rmsnorm        final norm                                      (:264-274)
//   gemv lm head   logits + first-maximum argmax                   (:284-308, sampling.rs:8-18)
//
// Weight layout in HBM (chosen for the GEMV, not copied from the artifact):
//   Wqkv  [(nq + 2 nkv) x H]: q, k, v rows, each head's rows reordered so that
//         rows 2i, 2i+1 are the RoPE pair (j, j + head_dim/2): one wave owns a
//         pair and rotates it in its epilogue.
//   Wgu   [2 I x H]: gate row r at 2r, up row r at 2r+1 (a wave owns both).
//   Wo [H x nq], Wd [H x I], LM head [V x H] (int8 tied embedding or int16).
#include "abi_internal.h"
#include "gemv.h"
#include "ops.h"
#include "../../include/myl_synth.h"

#include <cstring>
#include <new>
#include <string>
#include <vector>

using namespace myl;

namespace {

constexpr int kChunk = 256;          // attention positions per block
constexpr int kChunkLog = 8;
constexpr int kMaxGroup = 8;         // query heads per KV head handled by one block

struct DecodeState {
    uint64_t argmax_key;  // packed (value, ~index) of the best logit so far
    int32_t token;
    int32_t pos;
    int32_t rope_row;     // pos % rope rows
    int32_t step;         // decode steps taken since the last set
};

struct AttnStat {
    int32_t m;        // max score
    int32_t S;        // sum of exp-LUT values (wrapping i32)
    uint64_t recip;   // recip32(|S|) or recip32(L) when S == 0
    int32_t base, rem;
};

__device__ inline uint64_t argmax_key(int32_t v, uint32_t idx) {
    return ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}
__host__ __device__ inline int32_t key_index(uint64_t key) { return (int32_t)(0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFu)); }

// ---------------------------------------------------------------------------
// synthetic weights, generated in place (include/myl_synth.h)
// ---------------------------------------------------------------------------

__global__ void gen_w8_kernel(int8_t* __restrict__ dst, const int32_t* __restrict__ dst_row, int row0, int K,
                              uint64_t tseed) {
    const int r = row0 + blockIdx.y;
    const int dr = dst_row ? dst_row[r] : r;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < K; k += gridDim.x * blockDim.x)
        dst[(size_t)dr * K + k] = myl_synth_w8(tseed, (uint64_t)r * K + k);
}

__global__ void gen_w16_kernel(int16_t* __restrict__ dst, int row0, int K, uint64_t tseed) {
    const int r = row0 + blockIdx.y;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < K; k += gridDim.x * blockDim.x)
        dst[(size_t)r * K + k] = myl_synth_w16(tseed, (uint64_t)r * K + k);
}

// ---------------------------------------------------------------------------
// embedding + step state (model.rs:241-248, 323-331)
// ---------------------------------------------------------------------------

// mode 0: token/pos from the arguments; mode 1: greedy continuation (token =
// argmax of the previous step, pos + 1).  Resets the argmax key for this step.
__global__ __launch_bounds__(1024) void embed_kernel(DecodeState* st, int mode, int token_arg, int pos_arg,
                                                     uint32_t rope_rows, int vocab, const int8_t* __restrict__ E,
                                                     const uint8_t* __restrict__ emb_shifts,
                                                     const uint8_t* __restrict__ res_frac0, int H,
                                                     int64_t* __restrict__ tokens_out, int16_t* __restrict__ hidden) {
    __shared__ int32_t s_tok;
    if (threadIdx.x == 0) {
        int32_t tok, pos;
        if (mode == 0) {
            tok = token_arg;
            pos = pos_arg;
            st->step = 0;
        } else {
            tok = key_index(st->argmax_key);
            if (tok < 0 || tok >= vocab) tok = 0;  // a step without an LM head leaves no key
            pos = st->pos + 1;
            if (tokens_out) tokens_out[st->step] = tok;
            st->step = st->step + 1;
        }
        st->token = tok;
        st->pos = pos;
        st->rope_row = (int32_t)umod32_slow((uint32_t)pos, rope_rows);
        st->argmax_key = 0;
        s_tok = tok;
    }
    __syncthreads();
    const int tok = s_tok;
    const int8_t* row = E + (size_t)tok * H;
    const uint8_t sh = emb_shifts[tok];
    for (int i = threadIdx.x; i < H; i += blockDim.x)
        hidden[i] = clamp_i16(rescale32((int32_t)row[i], sh, res_frac0[i]));
}

// ---------------------------------------------------------------------------
// fused GEMV epilogues
// ---------------------------------------------------------------------------

// q/k/v projection rows (pair-ordered) -> bias -> RoPE -> q buffer / KV cache.
struct EpiQKV {
    const uint8_t* shifts;    // per device row
    const int16_t* bias;      // per device row, or null
    const uint8_t* bias_sh;
    uint8_t act_frac, q_frac, k_frac, v_frac;
    int nq, nkv, hd_log, max_pos;
    const int16_t* cos_lut;
    const int16_t* sin_lut;
    const DecodeState* st;
    int16_t* q_out;           // [nq]
    int16_t* kc;              // layer base [kv_heads][max_pos][hd]
    int16_t* vc;
    EpiQKV offset_m(int) const { return *this; }
    __device__ inline void one(int, int, int64_t) const {}
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
        static_assert(R == 2, "the RoPE pair needs two rows per wave");
        if (lane != 0 || row0 >= N) return;
        const int seg = row0 < nq ? 0 : (row0 < nq + nkv ? 1 : 2);
        const int e = row0 - (seg == 0 ? 0 : (seg == 1 ? nq : nq + nkv));
        const uint8_t frac = seg == 0 ? q_frac : (seg == 1 ? k_frac : v_frac);
        const int hd = 1 << hd_log, half = hd >> 1;
        const int head = e >> hd_log;
        const int p = (e & (hd - 1)) >> 1;
        int16_t y[2];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const int d = row0 + t;
            int16_t v = clamp_i16_i64(rescale64(tot[t][0], (uint8_t)(shifts[d] + act_frac), frac));
            if (bias) v = clamp_i16_i64((int64_t)v + (int64_t)rescale32((int32_t)bias[d], bias_sh[d], frac));
            y[t] = v;
        }
        const int pos = st->pos;
        if (seg < 2) {
            const int32_t c = cos_lut[(size_t)st->rope_row * half + p];
            const int32_t s = sin_lut[(size_t)st->rope_row * half + p];
            const int32_t x0 = y[0], x1 = y[1];
            y[0] = clamp_i16(rshift_round32(wsub32(wmul32(x0, c), wmul32(x1, s)), MYL_TV_ROPE_FRAC_BITS));
            y[1] = clamp_i16(rshift_round32(wadd32(wmul32(x1, c), wmul32(x0, s)), MYL_TV_ROPE_FRAC_BITS));
        }
        int16_t* dst;
        if (seg == 0) dst = q_out + (size_t)head * hd;
        else dst = (seg == 1 ? kc : vc) + ((size_t)head * max_pos + pos) * hd;
        dst[p] = y[0];
        dst[p + half] = y[1];
    }
};

// o_proj / down_proj + residual add (model.rs:576-593, 612-671):
//   o = clamp(rescale(acc, w_shift + act, acc_frac)); h = rescale(res_in, res_frac, acc_frac)
//   out = clamp(rescale(h + o, acc_frac, out_frac))
struct EpiResid {
    const uint8_t* shifts;
    uint8_t act_frac;
    const uint8_t* acc_frac;   // min(res_frac, out_frac) per channel
    const uint8_t* res_frac;
    const uint8_t* out_frac;
    const int16_t* res_in;
    int16_t* out;
    EpiResid offset_m(int) const { return *this; }
    __device__ inline void one(int r, int, int64_t acc) const {
        const uint8_t af = acc_frac[r];
        const int16_t o = clamp_i16_i64(rescale64(acc, (uint8_t)(shifts[r] + act_frac), af));
        const int64_t h = rescale64((int64_t)res_in[r], res_frac[r], af);
        out[r] = clamp_i16_i64(rescale64(wadd64(h, (int64_t)o), af, out_frac[r]));
    }
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
#pragma unroll
        for (int r = 0; r < R; ++r)
            if (lane == r && row0 + r < N) one(row0 + r, 0, tot[r][0]);
    }
};

// gate row 2r and up row 2r+1 -> h[r] (mlp.rs:46-65).
struct EpiSilu {
    const uint8_t* shifts;    // interleaved like the rows
    uint8_t act_frac, gate_frac, up_frac, down_in_frac;
    const int16_t* silu; uint32_t silu_len;
    int16_t* h;
    EpiSilu offset_m(int) const { return *this; }
    __device__ inline void one(int, int, int64_t) const {}
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
        static_assert(R == 2, "gate and up share a wave");
        if (lane != 0 || row0 >= N) return;
        const int16_t g = clamp_i16_i64(rescale64(tot[0][0], (uint8_t)(shifts[row0] + act_frac), gate_frac));
        const int16_t u = clamp_i16_i64(rescale64(tot[1][0], (uint8_t)(shifts[row0 + 1] + act_frac), up_frac));
        const int32_t g_dom = rescale32((int32_t)g, gate_frac, MYL_TV_SILU_IN_FRAC);
        const int16_t act = lut_lookup_i16((int16_t)g_dom, silu, silu_len, (int16_t)MYL_TV_SILU_LUT_OFFSET);
        const int64_t prod = (int64_t)act * (int64_t)u;
        h[row0 >> 1] = clamp_i16_i64(rescale64(prod, (uint8_t)(MYL_TV_SILU_OUT_FRAC + up_frac), down_in_frac));
    }
};

// LM head logits (model.rs:284-308) + first-maximum argmax (sampling.rs:8-18).
struct EpiHead {
    const uint8_t* shifts;
    uint8_t norm_frac;
    int32_t* logits;
    DecodeState* st;
    EpiHead offset_m(int) const { return *this; }
    __device__ inline void one(int r, int, int64_t acc) const {
        const int32_t v = clamp_i32_i64(rescale64(acc, (uint8_t)(shifts[r] + norm_frac), MYL_TV_LOGIT_FRAC_BITS));
        logits[r] = v;
        atomicMax((unsigned long long*)&st->argmax_key, (unsigned long long)argmax_key(v, (uint32_t)r));
    }
    template <int R, int MT>
    __device__ inline void apply(int row0, int N, int M, int lane, const int64_t (&tot)[R][MT]) const {
        uint64_t best = 0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r < N) {
                const int32_t v = clamp_i32_i64(rescale64(tot[r][0], (uint8_t)(shifts[row0 + r] + norm_frac),
                                                          MYL_TV_LOGIT_FRAC_BITS));
                if (lane == r) logits[row0 + r] = v;
                const uint64_t k = argmax_key(v, (uint32_t)(row0 + r));
                best = k > best ? k : best;
            }
        }
        if (lane == 0 && best) atomicMax((unsigned long long*)&st->argmax_key, (unsigned long long)best);
    }
};

template <int R, class Epi>
hipError_t gemv_model(const int16_t* x, const int8_t* W, int N, int K, const Epi& e, hipStream_t s) {
    const int kc = std::min(((K + 15) / 16) * 16, kGemvLdsBytes / 2);
    const int blocks = (N + R * kGemvWaves - 1) / (R * kGemvWaves);
    gemv_i8_kernel<R, 1, Epi><<<blocks, kGemvThreads, (size_t)2 * kc, s>>>(x, 1, K, W, N, K, kc, e);
    return hipGetLastError();
}

template <int R, class Epi>
hipError_t gemv_model16(const int16_t* x, const int16_t* W, int N, int K, const Epi& e, hipStream_t s) {
    const int kc = std::min(((K + 7) / 8) * 8, kGemvLdsBytes / 4);
    const int blocks = (N + R * kGemvWaves - 1) / (R * kGemvWaves);
    gemv_i16_kernel<R, 1, Epi><<<blocks, kGemvThreads, (size_t)4 * kc, s>>>(x, 1, K, W, N, K, kc, e);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// decode attention over the KV cache (attention.rs:42-90), GQA (model.rs:508-511)
// ---------------------------------------------------------------------------

// scores[h][j] for the G query heads of KV head g, positions j of one chunk.
// LPP = HD/8 lanes read one 16-byte slice each of a K row (coalesced rows).
template <int HD>
__global__ __launch_bounds__(256) void attn_scores_kernel(const DecodeState* __restrict__ st,
                                                         const int16_t* __restrict__ q, const int16_t* __restrict__ kc,
                                                         int max_pos, int G, int64_t score_mult, uint8_t score_shift,
                                                         int32_t* __restrict__ scores) {
    constexpr int LPP = HD / 8;
    constexpr int PPW = 64 / LPP;
    const int L = st->pos + 1;
    const int g = blockIdx.y;
    const int base = blockIdx.x * kChunk;
    if (base >= L) return;
    __shared__ __align__(16) int16_t qhi[kMaxGroup][HD];
    __shared__ __align__(16) int16_t qlo[kMaxGroup][HD];
    for (int i = threadIdx.x; i < G * HD; i += blockDim.x) {
        const int h = i / HD, d = i - h * HD;  // HD is a compile-time power of two
        const int16_t v = q[(size_t)(g * G + h) * HD + d];
        qhi[h][d] = (int16_t)(v >> 8);
        qlo[h][d] = (int16_t)(v & 255);
    }
    __syncthreads();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPP, slot = lane / LPP;
    const int16_t* kg = kc + (size_t)g * max_pos * HD;
    typedef short __attribute__((ext_vector_type(2))) s2;
    for (int it = 0; it < kChunk / 4 / PPW; ++it) {
        const int j = base + wave * (kChunk / 4) + it * PPW + slot;
        uint4 kv = make_uint4(0, 0, 0, 0);
        if (j < L) kv = *reinterpret_cast<const uint4*>(kg + (size_t)j * HD + sub * 8);
        for (int h = 0; h < G; ++h) {
            const uint4 qh = *reinterpret_cast<const uint4*>(&qhi[h][sub * 8]);
            const uint4 ql = *reinterpret_cast<const uint4*>(&qlo[h][sub * 8]);
            int32_t ahi = 0, alo = 0;
            ahi = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.x), __builtin_bit_cast(s2, qh.x), ahi, false);
            ahi = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.y), __builtin_bit_cast(s2, qh.y), ahi, false);
            ahi = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.z), __builtin_bit_cast(s2, qh.z), ahi, false);
            ahi = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.w), __builtin_bit_cast(s2, qh.w), ahi, false);
            alo = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.x), __builtin_bit_cast(s2, ql.x), alo, false);
            alo = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.y), __builtin_bit_cast(s2, ql.y), alo, false);
            alo = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.z), __builtin_bit_cast(s2, ql.z), alo, false);
            alo = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, kv.w), __builtin_bit_cast(s2, ql.w), alo, false);
#pragma unroll
            for (int off = LPP / 2; off > 0; off >>= 1) {
                ahi += __shfl_xor(ahi, off, 64);
                alo += __shfl_xor(alo, off, 64);
            }
            if (sub == 0 && j < L) {
                const int64_t dot = (int64_t)ahi * 256 + (int64_t)alo;
                scores[(size_t)(g * G + h) * max_pos + j] =
                    (int32_t)rshift_round64(wmul64(dot, score_mult), score_shift);
            }
        }
    }
}

// Per query head: max score, sum of exp-LUT values, reciprocal of the divisor.
__global__ __launch_bounds__(256) void attn_stats_kernel(const DecodeState* __restrict__ st,
                                                        const int32_t* __restrict__ scores, int max_pos,
                                                        const int16_t* __restrict__ lut, uint32_t lut_len,
                                                        uint8_t lut_shift, AttnStat* __restrict__ stats) {
    __shared__ int32_t red32[4];
    __shared__ uint32_t redu[4];
    const int L = st->pos + 1;
    const int32_t* z = scores + (size_t)blockIdx.x * max_pos;
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    const int32_t lut_one = lut_len > 0 ? (int32_t)lut[0] : 1;
    int32_t mx = INT32_MIN;
    for (int j = threadIdx.x; j < L; j += blockDim.x) mx = max(mx, z[j]);
    const int32_t m = block_max_i32(mx, red32);
    uint32_t s = 0;
    for (int j = threadIdx.x; j < L; j += blockDim.x) s += (uint32_t)exp_lookup(sat_sub32(m, z[j]), lut, lut_len, lut_shift, lut_one);
    const int32_t S = (int32_t)block_sum_u32(s, redu);
    if (threadIdx.x == 0) {
        AttnStat a;
        a.m = m;
        a.S = S;
        a.base = 0;
        a.rem = 0;
        if (S == 0) {
            uint32_t qq, rr;
            a.recip = recip32((uint32_t)L);
            udivmod32((uint32_t)one, (uint32_t)L, a.recip, &qq, &rr);
            a.base = (int32_t)qq;
            a.rem = wsub32(one, wmul32(a.base, L));
        } else {
            a.recip = recip32(S < 0 ? 0u - (uint32_t)S : (uint32_t)S);
        }
        stats[blockIdx.x] = a;
    }
}

// Probabilities of one chunk and their partial products with V, for the G
// heads of KV head g: partial[chunk][h][d] (i64, exact).
template <int HD>
__global__ __launch_bounds__(256) void attn_pv_kernel(const DecodeState* __restrict__ st,
                                                     const int32_t* __restrict__ scores, const AttnStat* __restrict__ stats,
                                                     const int16_t* __restrict__ vc, int max_pos, int G,
                                                     const int16_t* __restrict__ lut, uint32_t lut_len, uint8_t lut_shift,
                                                     int64_t* __restrict__ partial, int nq) {
    constexpr int TPR = HD / 2;           // threads per V row (one dim pair each)
    constexpr int STREAMS = 256 / TPR;    // position streams per block
    const int L = st->pos + 1;
    const int g = blockIdx.y;
    const int base = blockIdx.x * kChunk;
    if (base >= L) return;
    const int n = min(kChunk, L - base);
    __shared__ int32_t p[kMaxGroup][kChunk];
    __shared__ int64_t red[STREAMS][2 * TPR];
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    const int32_t lut_one = lut_len > 0 ? (int32_t)lut[0] : 1;
    for (int h = 0; h < G; ++h) {
        const AttnStat a = stats[g * G + h];
        const int32_t* z = scores + (size_t)(g * G + h) * max_pos + base;
        for (int t = threadIdx.x; t < n; t += blockDim.x) {
            int32_t pv;
            if (a.S == 0) {
                pv = a.base + (((uint64_t)(base + t) < (uint64_t)(int64_t)a.rem) ? 1 : 0);
            } else {
                const int32_t e = exp_lookup(sat_sub32(a.m, z[t]), lut, lut_len, lut_shift, lut_one);
                pv = softmax_div_round(wmul32(e, one), a.S, a.recip);
            }
            p[h][t] = pv;
        }
    }
    __syncthreads();
    const int dp = threadIdx.x % TPR, stream = threadIdx.x / TPR;
    int64_t acc0[kMaxGroup], acc1[kMaxGroup];
#pragma unroll
    for (int h = 0; h < kMaxGroup; ++h) { acc0[h] = 0; acc1[h] = 0; }
    const int16_t* vg = vc + (size_t)g * max_pos * HD;
    for (int t = stream; t < n; t += STREAMS) {
        const uint32_t pair = *reinterpret_cast<const uint32_t*>(vg + (size_t)(base + t) * HD + 2 * dp);
        const int64_t v0 = (int16_t)(pair & 0xFFFFu), v1 = (int16_t)(pair >> 16);
#pragma unroll
        for (int h = 0; h < kMaxGroup; ++h) {
            if (h < G) {
                const int64_t pv = p[h][t];
                acc0[h] = wadd64(acc0[h], pv * v0);
                acc1[h] = wadd64(acc1[h], pv * v1);
            }
        }
    }
    for (int h = 0; h < G; ++h) {
        __syncthreads();
        red[stream][2 * dp] = acc0[h];
        red[stream][2 * dp + 1] = acc1[h];
        __syncthreads();
        if (threadIdx.x < HD) {
            int64_t s = 0;
            for (int k = 0; k < STREAMS; ++k) s = wadd64(s, red[k][threadIdx.x]);
            partial[(size_t)blockIdx.x * nq + (size_t)(g * G + h) * HD + threadIdx.x] = s;
        }
    }
}

// attn_out[i] = clamp(rescale(clamp(RNE(sum_c partial[c][i], 14)), v_frac, attn_out_frac)).
__global__ void attn_reduce_kernel(const DecodeState* __restrict__ st, const int64_t* __restrict__ partial, int nq,
                                   uint8_t v_frac, uint8_t attn_out_frac, int16_t* __restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nq) return;
    const int L = st->pos + 1;
    const int chunks = (L + kChunk - 1) >> kChunkLog;
    int64_t s = 0;
    for (int c = 0; c < chunks; ++c) s = wadd64(s, partial[(size_t)c * nq + i]);
    const int16_t a = clamp_i16_i64(rshift_round64(s, MYL_TV_PROB_FRAC_BITS));
    out[i] = clamp_i16(rescale32((int32_t)a, v_frac, attn_out_frac));
}

// ---------------------------------------------------------------------------
// host-side model
// ---------------------------------------------------------------------------

struct LayerDev {
    int8_t *wqkv = nullptr, *wo = nullptr, *wgu = nullptr, *wd = nullptr;
    uint8_t *sqkv = nullptr, *so = nullptr, *sgu = nullptr, *sd = nullptr;
    int16_t* bqkv = nullptr;
    uint8_t* bsqkv = nullptr;
    int8_t *in_gamma = nullptr, *post_gamma = nullptr;
    uint8_t *in_gamma_s = nullptr, *post_gamma_s = nullptr;
    uint8_t *res_in = nullptr, *res_mid = nullptr, *acc_attn = nullptr, *acc_mlp = nullptr;
    const uint8_t* res_out = nullptr;  // next layer's res_in or the final segment
    myl_layer_fracs f{};
};

}  // namespace

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
    AttnStat* stats = nullptr;
    int64_t* partial = nullptr;
    DecodeState* state = nullptr;
    int64_t* tokens_dev = nullptr;
    uint32_t tokens_cap = 0;
    uint32_t n_cached = 0;

    template <class T> T* dalloc(size_t count) {
        void* p = nullptr;
        if (hipMalloc(&p, count * sizeof(T) ? count * sizeof(T) : 1) != hipSuccess) return nullptr;
        allocs.push_back(p);
        return (T*)p;
    }
    ~myl_model() {
        if (ctx) (void)hipStreamSynchronize(ctx->stream);
        for (void* p : allocs) (void)hipFree(p);
    }
};

namespace {

int ilog2_exact(int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return (1 << l) == v ? l : -1;
}

template <class T>
int upload(myl_model* m, T* dst, const std::vector<T>& src) {
    return m->ctx->hip(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice, m->ctx->stream),
                       "upload");
}

std::vector<uint8_t> small_u8(uint64_t seed, uint32_t layer, uint32_t role, size_t n) {
    std::vector<uint8_t> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (uint8_t)myl_synth_small(seed, layer, role, i);
    return v;
}
std::vector<int16_t> small_i16(uint64_t seed, uint32_t layer, uint32_t role, size_t n) {
    std::vector<int16_t> v(n);
    for (size_t i = 0; i < n; ++i) v[i] = (int16_t)myl_synth_small(seed, layer, role, i);
    return v;
}
std::vector<uint8_t> wshifts(uint64_t seed, uint32_t layer, uint32_t role, size_t rows, size_t K) {
    std::vector<uint8_t> v(rows);
    const uint64_t ts = myl_tensor_seed(seed, layer, role);
    for (size_t r = 0; r < rows; ++r) v[r] = myl_synth_wshift(ts, r, K);
    return v;
}

hipError_t gen_w8(myl_model* m, int8_t* dst, const int32_t* dst_row, int rows, int K, uint64_t tseed) {
    for (int r0 = 0; r0 < rows; r0 += 65535) {
        const int nr = std::min(65535, rows - r0);
        dim3 grid((unsigned)std::min((K + 255) / 256, 64), (unsigned)nr);
        gen_w8_kernel<<<grid, 256, 0, m->ctx->stream>>>(dst, dst_row, r0, K, tseed);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

hipError_t gen_w16(myl_model* m, int16_t* dst, int rows, int K, uint64_t tseed) {
    for (int r0 = 0; r0 < rows; r0 += 65535) {
        const int nr = std::min(65535, rows - r0);
        dim3 grid((unsigned)std::min((K + 255) / 256, 64), (unsigned)nr);
        gen_w16_kernel<<<grid, 256, 0, m->ctx->stream>>>(dst, r0, K, tseed);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Device row of original row o within a pair-ordered segment (heads of hd rows).
int pair_row(int o, int hd) {
    const int head = o / hd, w = o % hd, half = hd / 2;
    return head * hd + (w < half ? 2 * w : 2 * (w - half) + 1);
}

int build(myl_model* m, const myl_luts* luts) {
    myl_ctx* c = m->ctx;
    const myl_synth_spec& s = m->spec;
    const uint64_t seed = s.seed;
    const int H = m->H, I = m->I, V = m->V, hd = m->hd, nq = m->nq, nkv = m->nkv;
    const int nqkv = nq + 2 * nkv;

    // LUTs
    m->rsqrt_len = (int)luts->rsqrt_len;
    m->silu_len = (int)luts->silu_len;
    m->exp_len = (int)luts->exp_len;
    m->rope_rows = (uint32_t)(luts->rope_len / (size_t)(hd / 2));
    m->rsqrt = m->dalloc<int16_t>(luts->rsqrt_len);
    m->silu = m->dalloc<int16_t>(luts->silu_len);
    m->exp_lut = m->dalloc<int16_t>(luts->exp_len);
    m->cos_lut = m->dalloc<int16_t>(luts->rope_len);
    m->sin_lut = m->dalloc<int16_t>(luts->rope_len);
    if (!m->rsqrt || !m->silu || !m->exp_lut || !m->cos_lut || !m->sin_lut) return c->fail(MYL_E_NOMEM, "LUT allocation");
    int rc = 0;
    rc |= upload(m, m->rsqrt, std::vector<int16_t>(luts->rsqrt, luts->rsqrt + luts->rsqrt_len));
    rc |= upload(m, m->silu, std::vector<int16_t>(luts->silu, luts->silu + luts->silu_len));
    rc |= upload(m, m->exp_lut, std::vector<int16_t>(luts->exp, luts->exp + luts->exp_len));
    rc |= upload(m, m->cos_lut, std::vector<int16_t>(luts->cos, luts->cos + luts->rope_len));
    rc |= upload(m, m->sin_lut, std::vector<int16_t>(luts->sin, luts->sin + luts->rope_len));
    if (rc) return MYL_E_HIP;
    m->inv_n_q20 = ((1LL << 20) + H / 2) / H;  // rmsnorm.rs:20-23
    {
        // inv_sqrt_q15 (fixed_point.rs:102-146): rounded integer sqrt of 2^30 / hd.
        uint64_t n = (1ULL << 30) / (uint64_t)hd, r = 0;
        while ((r + 1) * (r + 1) <= n) ++r;
        const uint64_t below = n - r * r, above = (r + 1) * (r + 1) - n;
        m->score_mult = (int64_t)(above < below ? r + 1 : r);
    }

    // embedding / LM head / final norm
    m->emb = m->dalloc<int8_t>((size_t)V * H);
    m->emb_shifts = m->dalloc<uint8_t>(V);
    m->final_gamma = m->dalloc<int8_t>(H);
    m->final_gamma_s = m->dalloc<uint8_t>(H);
    m->final_res = m->dalloc<uint8_t>(H);
    if (!m->emb || !m->emb_shifts || !m->final_gamma || !m->final_gamma_s || !m->final_res)
        return c->fail(MYL_E_NOMEM, "embedding allocation");
    if (gen_w8(m, m->emb, nullptr, V, H, myl_tensor_seed(seed, 0, MYL_R_EMB)) != hipSuccess) return MYL_E_HIP;
    rc |= upload(m, m->emb_shifts, small_u8(seed, 0, MYL_R_EMB_SHIFT, V));
    if (s.lm_head_int16) {
        m->lm16 = m->dalloc<int16_t>((size_t)V * H);
        m->lm16_shifts = m->dalloc<uint8_t>(V);
        if (!m->lm16 || !m->lm16_shifts) return c->fail(MYL_E_NOMEM, "LM head allocation");
        if (gen_w16(m, m->lm16, V, H, myl_tensor_seed(seed, 0, MYL_R_LM16)) != hipSuccess) return MYL_E_HIP;
        rc |= upload(m, m->lm16_shifts, small_u8(seed, 0, MYL_R_LM16_SHIFT, V));
    }
    if (gen_w8(m, m->final_gamma, nullptr, 1, H, myl_tensor_seed(seed, 0, MYL_R_FINAL_GAMMA)) != hipSuccess) return MYL_E_HIP;
    rc |= upload(m, m->final_gamma_s, small_u8(seed, 0, MYL_R_FINAL_GAMMA_SHIFT, H));
    std::vector<uint8_t> final_res(H);
    {
        const uint64_t ts = myl_tensor_seed(seed, 0, MYL_R_FINAL_RES_FRAC);
        for (int i = 0; i < H; ++i) final_res[i] = myl_synth_res_frac(ts, i);
    }
    rc |= upload(m, m->final_res, final_res);
    m->final_norm_frac = myl_synth_final_norm_frac(seed);

    // layers
    std::vector<int32_t> qkv_rows(nqkv);
    for (int o = 0; o < nq; ++o) qkv_rows[o] = pair_row(o, hd);
    for (int o = 0; o < nkv; ++o) qkv_rows[nq + o] = nq + pair_row(o, hd);
    for (int o = 0; o < nkv; ++o) qkv_rows[nq + nkv + o] = nq + nkv + pair_row(o, hd);
    int32_t* qkv_rows_dev = m->dalloc<int32_t>(nqkv);
    std::vector<int32_t> gu_rows(2 * (size_t)I);
    for (int r = 0; r < I; ++r) { gu_rows[r] = 2 * r; gu_rows[I + r] = 2 * r + 1; }
    int32_t* gu_rows_dev = m->dalloc<int32_t>(2 * (size_t)I);
    if (!qkv_rows_dev || !gu_rows_dev) return c->fail(MYL_E_NOMEM, "row tables");
    rc |= upload(m, qkv_rows_dev, qkv_rows);
    rc |= upload(m, gu_rows_dev, gu_rows);

    std::vector<std::vector<uint8_t>> res_in(s.layers), res_mid(s.layers);
    for (uint32_t l = 0; l < s.layers; ++l) {
        res_in[l].resize(H);
        res_mid[l].resize(H);
        const uint64_t ti = myl_tensor_seed(seed, l, MYL_R_RES_IN), tm = myl_tensor_seed(seed, l, MYL_R_RES_MID);
        for (int i = 0; i < H; ++i) {
            res_in[l][i] = myl_synth_res_frac(ti, i);
            res_mid[l][i] = myl_synth_res_frac(tm, i);
        }
    }
    m->layers.resize(s.layers);
    for (uint32_t l = 0; l < s.layers; ++l) {
        LayerDev& L = m->layers[l];
        L.f = myl_synth_layer_fracs(seed, l);
        L.wqkv = m->dalloc<int8_t>((size_t)nqkv * H);
        L.wo = m->dalloc<int8_t>((size_t)H * nq);
        L.wgu = m->dalloc<int8_t>((size_t)2 * I * H);
        L.wd = m->dalloc<int8_t>((size_t)H * I);
        L.sqkv = m->dalloc<uint8_t>(nqkv);
        L.so = m->dalloc<uint8_t>(H);
        L.sgu = m->dalloc<uint8_t>(2 * (size_t)I);
        L.sd = m->dalloc<uint8_t>(H);
        L.in_gamma = m->dalloc<int8_t>(H);
        L.post_gamma = m->dalloc<int8_t>(H);
        L.in_gamma_s = m->dalloc<uint8_t>(H);
        L.post_gamma_s = m->dalloc<uint8_t>(H);
        L.res_in = m->dalloc<uint8_t>(H);
        L.res_mid = m->dalloc<uint8_t>(H);
        L.acc_attn = m->dalloc<uint8_t>(H);
        L.acc_mlp = m->dalloc<uint8_t>(H);
        if (s.attention_bias) {
            L.bqkv = m->dalloc<int16_t>(nqkv);
            L.bsqkv = m->dalloc<uint8_t>(nqkv);
            if (!L.bqkv || !L.bsqkv) return c->fail(MYL_E_NOMEM, "bias allocation");
        }
        if (!L.wqkv || !L.wo || !L.wgu || !L.wd || !L.sqkv || !L.so || !L.sgu || !L.sd || !L.in_gamma ||
            !L.post_gamma || !L.in_gamma_s || !L.post_gamma_s || !L.res_in || !L.res_mid || !L.acc_attn || !L.acc_mlp)
            return c->fail(MYL_E_NOMEM, "layer allocation");
        hipError_t e = gen_w8(m, L.wqkv, qkv_rows_dev, nq, H, myl_tensor_seed(seed, l, MYL_R_WQ));
        if (e == hipSuccess) e = gen_w8(m, L.wqkv, qkv_rows_dev + nq, nkv, H, myl_tensor_seed(seed, l, MYL_R_WK));
        if (e == hipSuccess) e = gen_w8(m, L.wqkv, qkv_rows_dev + nq + nkv, nkv, H, myl_tensor_seed(seed, l, MYL_R_WV));
        if (e == hipSuccess) e = gen_w8(m, L.wo, nullptr, H, nq, myl_tensor_seed(seed, l, MYL_R_WO));
        if (e == hipSuccess) e = gen_w8(m, L.wgu, gu_rows_dev, I, H, myl_tensor_seed(seed, l, MYL_R_WG));
        if (e == hipSuccess) e = gen_w8(m, L.wgu, gu_rows_dev + I, I, H, myl_tensor_seed(seed, l, MYL_R_WU));
        if (e == hipSuccess) e = gen_w8(m, L.wd, nullptr, H, I, myl_tensor_seed(seed, l, MYL_R_WD));
        if (e == hipSuccess) e = gen_w8(m, L.in_gamma, nullptr, 1, H, myl_tensor_seed(seed, l, MYL_R_IN_GAMMA));
        if (e == hipSuccess) e = gen_w8(m, L.post_gamma, nullptr, 1, H, myl_tensor_seed(seed, l, MYL_R_POST_GAMMA));
        if (e != hipSuccess) return c->hip(e, "weight generation");
        // per-row tables, permuted like the rows
        auto sq = wshifts(seed, l, MYL_R_SQ, nq, H), sk = wshifts(seed, l, MYL_R_SK, nkv, H),
             sv = wshifts(seed, l, MYL_R_SV, nkv, H);
        std::vector<uint8_t> sqkv(nqkv);
        for (int o = 0; o < nq; ++o) sqkv[qkv_rows[o]] = sq[o];
        for (int o = 0; o < nkv; ++o) sqkv[qkv_rows[nq + o]] = sk[o];
        for (int o = 0; o < nkv; ++o) sqkv[qkv_rows[nq + nkv + o]] = sv[o];
        rc |= upload(m, L.sqkv, sqkv);
        if (s.attention_bias) {
            auto bq = small_i16(seed, l, MYL_R_BQ, nq), bk = small_i16(seed, l, MYL_R_BK, nkv),
                 bv = small_i16(seed, l, MYL_R_BV, nkv);
            auto bqs = small_u8(seed, l, MYL_R_BQ_SHIFT, nq), bks = small_u8(seed, l, MYL_R_BK_SHIFT, nkv),
                 bvs = small_u8(seed, l, MYL_R_BV_SHIFT, nkv);
            std::vector<int16_t> b(nqkv);
            std::vector<uint8_t> bs(nqkv);
            for (int o = 0; o < nq; ++o) { b[qkv_rows[o]] = bq[o]; bs[qkv_rows[o]] = bqs[o]; }
            for (int o = 0; o < nkv; ++o) { b[qkv_rows[nq + o]] = bk[o]; bs[qkv_rows[nq + o]] = bks[o]; }
            for (int o = 0; o < nkv; ++o) {
                b[qkv_rows[nq + nkv + o]] = bv[o];
                bs[qkv_rows[nq + nkv + o]] = bvs[o];
            }
            rc |= upload(m, L.bqkv, b);
            rc |= upload(m, L.bsqkv, bs);
        }
        rc |= upload(m, L.so, wshifts(seed, l, MYL_R_SO, H, nq));
        auto sg = wshifts(seed, l, MYL_R_SG, I, H), su = wshifts(seed, l, MYL_R_SU, I, H);
        std::vector<uint8_t> sgu(2 * (size_t)I);
        for (int r = 0; r < I; ++r) { sgu[2 * r] = sg[r]; sgu[2 * r + 1] = su[r]; }
        rc |= upload(m, L.sgu, sgu);
        rc |= upload(m, L.sd, wshifts(seed, l, MYL_R_SD, H, I));
        rc |= upload(m, L.in_gamma_s, small_u8(seed, l, MYL_R_IN_GAMMA_SHIFT, H));
        rc |= upload(m, L.post_gamma_s, small_u8(seed, l, MYL_R_POST_GAMMA_SHIFT, H));
        const std::vector<uint8_t>& out_frac = (l + 1 < s.layers) ? res_in[l + 1] : final_res;
        std::vector<uint8_t> acc_a(H), acc_m(H);
        for (int i = 0; i < H; ++i) {
            acc_a[i] = std::min(res_in[l][i], res_mid[l][i]);   // model.rs:576-581
            acc_m[i] = std::min(res_mid[l][i], out_frac[i]);    // model.rs:612-617
        }
        rc |= upload(m, L.res_in, res_in[l]);
        rc |= upload(m, L.res_mid, res_mid[l]);
        rc |= upload(m, L.acc_attn, acc_a);
        rc |= upload(m, L.acc_mlp, acc_m);
        if (rc) return MYL_E_HIP;
    }
    for (uint32_t l = 0; l < s.layers; ++l)
        m->layers[l].res_out = (l + 1 < s.layers) ? m->layers[l + 1].res_in : m->final_res;

    // caches, activations, scratch
    const size_t kv = (size_t)s.layers * s.kv_heads * (size_t)m->max_pos * hd;
    m->kcache = m->dalloc<int16_t>(kv);
    m->vcache = m->dalloc<int16_t>(kv);
    m->hidden = m->dalloc<int16_t>(H);
    m->norm = m->dalloc<int16_t>(H);
    m->q = m->dalloc<int16_t>(nq);
    m->attn = m->dalloc<int16_t>(nq);
    m->resid = m->dalloc<int16_t>(H);
    m->h = m->dalloc<int16_t>(I);
    m->logits = m->dalloc<int32_t>(V);
    m->scores = m->dalloc<int32_t>((size_t)s.heads * m->max_pos);
    m->stats = m->dalloc<AttnStat>(s.heads);
    const int max_chunks = (m->max_pos + kChunk - 1) / kChunk;
    m->partial = m->dalloc<int64_t>((size_t)max_chunks * nq);
    m->state = m->dalloc<DecodeState>(1);
    if (!m->kcache || !m->vcache || !m->hidden || !m->norm || !m->q || !m->attn || !m->resid || !m->h ||
        !m->logits || !m->scores || !m->stats || !m->partial || !m->state)
        return c->fail(MYL_E_NOMEM, "activation allocation");
    if (hipMemsetAsync(m->kcache, 0, kv * 2, c->stream) != hipSuccess ||
        hipMemsetAsync(m->vcache, 0, kv * 2, c->stream) != hipSuccess ||
        hipMemsetAsync(m->state, 0, sizeof(DecodeState), c->stream) != hipSuccess)
        return MYL_E_HIP;
    return c->hip(hipStreamSynchronize(c->stream), "model build");
}

hipError_t rms(myl_model* m, const int16_t* x, const uint8_t* xs, const int8_t* g, const uint8_t* gs, uint8_t out_frac,
               int16_t* out) {
    return rmsnorm(x, 1, m->H, xs, g, gs, m->H, m->rsqrt, m->rsqrt_len, MYL_TV_RSQRT_INPUT_SHIFT,
                   MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, out_frac, out, m->H, m->ctx->stream);
}

// One transformer layer on m->hidden (model.rs:401-674); the result replaces m->hidden.
hipError_t layer_step(myl_model* m, int l) {
    const LayerDev& L = m->layers[l];
    const myl_layer_fracs& f = L.f;
    hipStream_t st = m->ctx->stream;
    const int H = m->H, I = m->I, nq = m->nq, nkv = m->nkv, hd = m->hd, G = m->G;
    const int kvh = (int)m->spec.kv_heads;
    hipError_t e = rms(m, m->hidden, L.res_in, L.in_gamma, L.in_gamma_s, f.norm_attn_frac, m->norm);
    if (e != hipSuccess) return e;
    {
        const size_t layer_kv = (size_t)l * kvh * m->max_pos * hd;
        EpiQKV q{L.sqkv, L.bqkv, L.bsqkv, f.norm_attn_frac, f.q_frac, f.k_frac, f.v_frac, nq, nkv, m->hd_log,
                 m->max_pos, m->cos_lut, m->sin_lut, m->state, m->q, m->kcache + layer_kv, m->vcache + layer_kv};
        e = gemv_model<2>(m->norm, L.wqkv, nq + 2 * nkv, H, q, st);
        if (e != hipSuccess) return e;
        const uint32_t ss = (uint32_t)f.q_frac + f.k_frac + 15u;
        const uint8_t score_shift = (uint8_t)(ss > MYL_TV_SCORE_FRAC_BITS ? ss - MYL_TV_SCORE_FRAC_BITS : 0);
        const uint8_t lut_shift = MYL_TV_SCORE_FRAC_BITS - MYL_TV_EXP_INPUT_FRAC;
        const int chunks = (m->max_pos + kChunk - 1) / kChunk;
        const int16_t* kc = m->kcache + layer_kv;
        const int16_t* vc = m->vcache + layer_kv;
        if (hd == 128) {
            attn_scores_kernel<128><<<dim3(chunks, kvh), 256, 0, st>>>(m->state, m->q, kc, m->max_pos, G, m->score_mult,
                                                                     score_shift, m->scores);
        } else {
            attn_scores_kernel<64><<<dim3(chunks, kvh), 256, 0, st>>>(m->state, m->q, kc, m->max_pos, G, m->score_mult,
                                                                    score_shift, m->scores);
        }
        attn_stats_kernel<<<m->spec.heads, 256, 0, st>>>(m->state, m->scores, m->max_pos, m->exp_lut,
                                                         (uint32_t)m->exp_len, lut_shift, m->stats);
        if (hd == 128) {
            attn_pv_kernel<128><<<dim3(chunks, kvh), 256, 0, st>>>(m->state, m->scores, m->stats, vc, m->max_pos, G,
                                                                 m->exp_lut, (uint32_t)m->exp_len, lut_shift,
                                                                 m->partial, nq);
        } else {
            attn_pv_kernel<64><<<dim3(chunks, kvh), 256, 0, st>>>(m->state, m->scores, m->stats, vc, m->max_pos, G,
                                                                m->exp_lut, (uint32_t)m->exp_len, lut_shift,
                                                                m->partial, nq);
        }
        attn_reduce_kernel<<<(nq + 255) / 256, 256, 0, st>>>(m->state, m->partial, nq, f.v_frac, f.attn_out_frac,
                                                            m->attn);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    {
        EpiResid o{L.so, f.attn_out_frac, L.acc_attn, L.res_in, L.res_mid, m->hidden, m->resid};
        e = gemv_model<2>(m->attn, L.wo, H, nq, o, st);
        if (e != hipSuccess) return e;
    }
    e = rms(m, m->resid, L.res_mid, L.post_gamma, L.post_gamma_s, f.norm_mlp_frac, m->norm);
    if (e != hipSuccess) return e;
    {
        EpiSilu s{L.sgu, f.norm_mlp_frac, f.gate_frac, f.up_frac, f.down_in_frac, m->silu, (uint32_t)m->silu_len, m->h};
        e = gemv_model<2>(m->norm, L.wgu, 2 * I, H, s, st);
        if (e != hipSuccess) return e;
        EpiResid d{L.sd, f.down_in_frac, L.acc_mlp, L.res_mid, L.res_out, m->resid, m->hidden};
        e = gemv_model<2>(m->h, L.wd, H, I, d, st);
    }
    return e;
}

hipError_t head_step(myl_model* m) {
    hipStream_t st = m->ctx->stream;
    hipError_t e = rms(m, m->hidden, m->final_res, m->final_gamma, m->final_gamma_s, m->final_norm_frac, m->norm);
    if (e != hipSuccess) return e;
    if (m->spec.lm_head_int16) {
        EpiHead hd{m->lm16_shifts, m->final_norm_frac, m->logits, m->state};
        return gemv_model16<2>(m->norm, m->lm16, m->V, m->H, hd, st);
    }
    EpiHead hd{m->emb_shifts, m->final_norm_frac, m->logits, m->state};
    return gemv_model<2>(m->norm, m->emb, m->V, m->H, hd, st);
}

hipError_t embed_step(myl_model* m, int mode, int token, int pos, int64_t* tokens_dev) {
    embed_kernel<<<1, 1024, 0, m->ctx->stream>>>(m->state, mode, token, pos, m->rope_rows, m->V, m->emb, m->emb_shifts,
                                                  m->layers[0].res_in, m->H, tokens_dev, m->hidden);
    return hipGetLastError();
}

hipError_t full_step(myl_model* m, int mode, int token, int pos, int64_t* tokens_dev) {
    hipError_t e = embed_step(m, mode, token, pos, tokens_dev);
    for (int l = 0; e == hipSuccess && l < (int)m->spec.layers; ++l) e = layer_step(m, l);
    if (e == hipSuccess) e = head_step(m);
    return e;
}

}  // namespace

extern "C" {

int myl_model_create_synthetic(myl_ctx* ctx, const myl_synth_spec* spec, const myl_luts* luts, myl_model** out) {
    if (!ctx || !spec || !luts || !out) return MYL_E_INVALID;
    *out = nullptr;
    const myl_synth_spec& s = *spec;
    if (!s.hidden || !s.layers || !s.heads || !s.kv_heads || !s.head_dim || !s.inter || !s.vocab || !s.max_pos)
        return ctx->fail(MYL_E_INVALID, "model: every dimension must be > 0");
    if (s.heads % s.kv_heads || s.heads * s.head_dim != s.hidden)
        return ctx->fail(MYL_E_INVALID, "model: heads must divide evenly into KV heads and tile hidden");
    if (s.head_dim != 64 && s.head_dim != 128)
        return ctx->fail(MYL_E_UNSUPPORTED, "model: the fused decode path takes head_dim 64 or 128");
    if (s.heads / s.kv_heads > kMaxGroup) return ctx->fail(MYL_E_UNSUPPORTED, "model: more than 8 query heads per KV head");
    if (s.hidden % 16 || s.inter % 16) return ctx->fail(MYL_E_UNSUPPORTED, "model: hidden and intermediate must be multiples of 16");
    if (!luts->rsqrt || luts->rsqrt_len < 2 || !luts->silu || !luts->silu_len || !luts->exp || !luts->cos ||
        !luts->sin || luts->rope_len < s.head_dim / 2)
        return ctx->fail(MYL_E_INVALID, "model: incomplete LUT set");
    if ((uint64_t)s.vocab * s.hidden > (uint64_t)INT32_MAX * 16)
        return ctx->fail(MYL_E_UNSUPPORTED, "model: embedding too large");
    (void)hipSetDevice(ctx->device);
    myl_model* m = new (std::nothrow) myl_model();
    if (!m) return MYL_E_NOMEM;
    m->ctx = ctx;
    m->spec = s;
    m->H = (int)s.hidden;
    m->I = (int)s.inter;
    m->V = (int)s.vocab;
    m->hd = (int)s.head_dim;
    m->hd_log = ilog2_exact(m->hd);
    m->G = (int)(s.heads / s.kv_heads);
    m->nq = (int)(s.heads * s.head_dim);
    m->nkv = (int)(s.kv_heads * s.head_dim);
    m->max_pos = (int)s.max_pos;
    int rc = build(m, luts);
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return MYL_OK;
}

void myl_model_destroy(myl_model* m) { delete m; }

int myl_model_reset(myl_model* m) {
    if (!m) return MYL_E_INVALID;
    m->n_cached = 0;
    return MYL_OK;
}

int myl_model_forward_token(myl_model* m, uint32_t token, uint32_t pos, int32_t* logits, int64_t* argmax_out) {
    if (!m) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (token >= (uint32_t)m->V) return c->fail(MYL_E_INVALID, "forward_token: token id out of range");
    if (pos >= (uint32_t)m->max_pos) return c->fail(MYL_E_INVALID, "forward_token: position beyond the KV capacity");
    if (pos > m->n_cached) return c->fail(MYL_E_INVALID, "forward_token: positions must be contiguous from 0");
    int rc = c->hip(full_step(m, 0, (int)token, (int)pos, nullptr), "forward_token");
    if (rc) return rc;
    if (pos + 1 > m->n_cached) m->n_cached = pos + 1;
    if (logits) {
        rc = c->hip(hipMemcpyAsync(logits, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, c->stream), "logits");
        if (rc) return rc;
    }
    if (argmax_out) {
        DecodeState s;
        rc = c->hip(hipMemcpyAsync(&s, m->state, sizeof(s), hipMemcpyDeviceToHost, c->stream), "state");
        if (rc) return rc;
        rc = c->hip(hipStreamSynchronize(c->stream), "forward_token");
        if (rc) return rc;
        *argmax_out = key_index(s.argmax_key);
        return MYL_OK;
    }
    return c->hip(hipStreamSynchronize(c->stream), "forward_token");
}

int myl_model_decode_greedy(myl_model* m, uint32_t token, uint32_t pos, uint32_t n_steps, int64_t* tokens_out,
                            int32_t* logits_out) {
    if (!m) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (n_steps == 0) return MYL_OK;
    if (token >= (uint32_t)m->V) return c->fail(MYL_E_INVALID, "decode: token id out of range");
    if ((uint64_t)pos + n_steps > (uint64_t)m->max_pos)
        return c->fail(MYL_E_INVALID, "decode: positions beyond the KV capacity");
    if (pos > m->n_cached) return c->fail(MYL_E_INVALID, "decode: positions must be contiguous from 0");
    if (n_steps > m->tokens_cap) {
        int64_t* t = m->dalloc<int64_t>(n_steps);
        if (!t) return c->fail(MYL_E_NOMEM, "decode: token buffer");
        m->tokens_dev = t;
        m->tokens_cap = n_steps;
    }
    // Step 0 consumes the given token; step i >= 1 consumes step i-1's argmax.
    // The argmax of the last step is the next token, reported by tokens_out.
    hipError_t e = full_step(m, 0, (int)token, (int)pos, nullptr);
    for (uint32_t i = 0; e == hipSuccess && i < n_steps; ++i) {
        if (logits_out)
            e = hipMemcpyAsync(logits_out + (size_t)i * m->V, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost,
                               c->stream);
        if (e == hipSuccess && i + 1 < n_steps) e = full_step(m, 1, 0, 0, m->tokens_dev);
    }
    int rc = c->hip(e, "decode");
    if (rc) return rc;
    m->n_cached = std::max(m->n_cached, pos + n_steps);
    // tokens_dev[0..n_steps-2] were written by steps 1..n-1; the last argmax is in the state.
    std::vector<int64_t> toks(n_steps);
    DecodeState s;
    if (n_steps > 1) {
        rc = c->hip(hipMemcpyAsync(toks.data(), m->tokens_dev, (size_t)(n_steps - 1) * 8, hipMemcpyDeviceToHost,
                                   c->stream), "tokens");
        if (rc) return rc;
    }
    rc = c->hip(hipMemcpyAsync(&s, m->state, sizeof(s), hipMemcpyDeviceToHost, c->stream), "state");
    if (rc) return rc;
    rc = c->hip(hipStreamSynchronize(c->stream), "decode");
    if (rc) return rc;
    toks[n_steps - 1] = key_index(s.argmax_key);
    if (tokens_out) std::memcpy(tokens_out, toks.data(), (size_t)n_steps * 8);
    return MYL_OK;
}

int myl_model_embed_token(myl_model* m, uint32_t token, int16_t* hidden) {
    if (!m || !hidden) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (token >= (uint32_t)m->V) return c->fail(MYL_E_INVALID, "embed_token: token id out of range");
    int rc = c->hip(embed_step(m, 0, (int)token, 0, nullptr), "embed_token");
    if (rc) return rc;
    rc = c->hip(hipMemcpyAsync(hidden, m->hidden, (size_t)m->H * 2, hipMemcpyDeviceToHost, c->stream), "hidden");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "embed_token");
}

int myl_model_run_layers(myl_model* m, int16_t* hidden, uint32_t pos, uint32_t layer_start, uint32_t layer_end) {
    if (!m || !hidden) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (layer_end > m->spec.layers || layer_start > layer_end || pos >= (uint32_t)m->max_pos)
        return c->fail(MYL_E_INVALID, "run_layers: bad layer range or position");
    DecodeState s{};
    s.pos = (int32_t)pos;
    s.rope_row = (int32_t)(pos % m->rope_rows);
    int rc = c->hip(hipMemcpyAsync(m->state, &s, sizeof(s), hipMemcpyHostToDevice, c->stream), "state");
    if (rc) return rc;
    rc = c->hip(hipMemcpyAsync(m->hidden, hidden, (size_t)m->H * 2, hipMemcpyHostToDevice, c->stream), "hidden");
    hipError_t e = hipSuccess;
    for (uint32_t l = layer_start; !rc && e == hipSuccess && l < layer_end; ++l) e = layer_step(m, (int)l);
    if (!rc) rc = c->hip(e, "run_layers");
    if (rc) return rc;
    rc = c->hip(hipMemcpyAsync(hidden, m->hidden, (size_t)m->H * 2, hipMemcpyDeviceToHost, c->stream), "hidden");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "run_layers");
}

int myl_model_head_logits(myl_model* m, const int16_t* hidden, int32_t* logits) {
    if (!m || !hidden || !logits) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    int rc = c->hip(hipMemcpyAsync(m->hidden, hidden, (size_t)m->H * 2, hipMemcpyHostToDevice, c->stream), "hidden");
    if (rc) return rc;
    rc = c->hip(head_step(m), "head_logits");
    if (rc) return rc;
    rc = c->hip(hipMemcpyAsync(logits, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, c->stream), "logits");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "head_logits");
}

int myl_model_read_kv(myl_model* m, uint32_t layer, uint32_t kv_head, uint32_t n_pos, int16_t* k_out,
                      int16_t* v_out) {
    if (!m) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (layer >= m->spec.layers || kv_head >= m->spec.kv_heads || n_pos > (uint32_t)m->max_pos)
        return c->fail(MYL_E_INVALID, "read_kv: out of range");
    const size_t off = (((size_t)layer * m->spec.kv_heads + kv_head) * m->max_pos) * m->hd;
    const size_t bytes = (size_t)n_pos * m->hd * 2;
    int rc = 0;
    if (k_out) rc = c->hip(hipMemcpyAsync(k_out, m->kcache + off, bytes, hipMemcpyDeviceToHost, c->stream), "k");
    if (!rc && v_out) rc = c->hip(hipMemcpyAsync(v_out, m->vcache + off, bytes, hipMemcpyDeviceToHost, c->stream), "v");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "read_kv");
}

int myl_model_read_tensor(myl_model* m, const char* name, uint32_t layer, void* host_out, size_t bytes) {
    if (!m || !name || !host_out) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (layer >= m->spec.layers) return c->fail(MYL_E_INVALID, "read_tensor: layer out of range");
    const LayerDev& L = m->layers[layer];
    const void* src = nullptr;
    size_t n = 0;
    const size_t H = m->H, I = m->I, V = m->V, nq = m->nq, nkv = m->nkv;
    const std::string s(name);
    if (s == "emb") { src = m->emb; n = V * H; }
    else if (s == "lm16") { src = m->lm16; n = m->lm16 ? V * H * 2 : 0; }
    else if (s == "wqkv") { src = L.wqkv; n = (nq + 2 * nkv) * H; }
    else if (s == "wo") { src = L.wo; n = H * nq; }
    else if (s == "wgu") { src = L.wgu; n = 2 * I * H; }
    else if (s == "wd") { src = L.wd; n = H * I; }
    else if (s == "in_gamma") { src = L.in_gamma; n = H; }
    else if (s == "final_gamma") { src = m->final_gamma; n = H; }
    if (!src) return c->fail(MYL_E_INVALID, "read_tensor: unknown tensor " + s);
    if (bytes != n) return c->fail(MYL_E_INVALID, "read_tensor: byte count mismatch");
    int rc = c->hip(hipMemcpyAsync(host_out, src, n, hipMemcpyDeviceToHost, c->stream), "read_tensor");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "read_tensor");
}

}  // extern "C"
