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
//     attn_pv      max, sum of exp-LUT, reciprocal of the sum      (softmax.rs:32-48)
//                  p_j = RNE(e_j * 2^14 / S), partial sum p_j v_j  (softmax.rs:50-63, attention.rs:75-81)
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
#include "gemv_stream.h"
#include "ops.h"
#include "dec_attn.h"
#include "../../include/myl_synth.h"
#include "model_internal.h"

#include <cstring>
#include <new>
#include <string>
#include <vector>

using namespace myl;

namespace {




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
// RMSNorm fused across kernels (rmsnorm.rs:61-161)
//
// The producer of a residual-stream vector (embed, o_proj, down_proj) adds the
// exact terms x_i^2 << 2(ref - x_shift_i) of the next RMSNorm into a
// NormAcc: each 128-bit term is split into 42-bit limbs summed in u64 (no
// limb sum can overflow for n < 2^10 * 2^10), spread over 64 slots to keep
// atomic contention low.  The consumer GEMV rebuilds the 128-bit sum modulo
// 2^128 (the reference's wrapping i128 additions), derives the LUT factor and
// normalises the vector while staging it.
// ---------------------------------------------------------------------------



// Block-level sum of per-thread limbs; the first wave (thread 0 among it)
// gets the totals, reading the per-wave slots in parallel.
__device__ inline void block_sum_limbs(uint64_t (&l)[3], uint64_t* red /* [16][3] */) {
#pragma unroll
    for (int j = 0; j < 3; ++j) l[j] = wave_sum_u64(l[j]);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0)
        for (int j = 0; j < 3; ++j) red[w * 3 + j] = l[j];
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int j = 0; j < 3; ++j) l[j] = wave_sum_u64(lane < nw ? red[lane * 3 + j] : 0ull);
    }
}

// Writes the norm sum of an n-vector computed by one block into slot 0 of acc
// (the other slots are cleared): used where one block sees the whole vector.
__device__ inline void block_seed_norm(const int16_t* x, const uint8_t* xs, uint8_t ref, int n, NormAcc* acc) {
    __shared__ uint64_t red[16 * 3];
    uint64_t l[3] = {0, 0, 0};
    for (int i = threadIdx.x; i < n; i += blockDim.x) add_sq_limbs(x[i], xs[i], ref, l);
    block_sum_limbs(l, red);
    for (int i = threadIdx.x; i < kNormSlots * 3; i += blockDim.x) (&acc->v[0][0])[i] = 0;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int j = 0; j < 3; ++j) acc->v[0][j] = l[j];
}

__global__ __launch_bounds__(1024) void norm_seed_kernel(const int16_t* __restrict__ x, const uint8_t* __restrict__ xs,
                                                         uint8_t ref, int n, NormAcc* acc) {
    block_seed_norm(x, xs, ref, n, acc);
}

// int16 values -> the two signed byte planes (hi = v >> 8, lo' = (v & 255) - 128).
__device__ inline void put_planes_i8(const int16_t (&v)[8], int8_t* hi, int8_t* lo) {
    uint32_t h[2], l[2];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
        const uint32_t d0 = (uint32_t)(uint16_t)v[4 * t] | ((uint32_t)(uint16_t)v[4 * t + 1] << 16);
        const uint32_t d1 = (uint32_t)(uint16_t)v[4 * t + 2] | ((uint32_t)(uint16_t)v[4 * t + 3] << 16);
        h[t] = ((d0 >> 8) & 0xFFu) | ((d0 >> 16) & 0xFF00u) | ((d1 << 8) & 0xFF0000u) | (d1 & 0xFF000000u);
        l[t] = ((d0 & 0xFFu) | ((d0 >> 8) & 0xFF00u) | ((d1 << 16) & 0xFF0000u) | ((d1 << 8) & 0xFF000000u)) ^ 0x80808080u;
    }
    *reinterpret_cast<uint2*>(hi) = make_uint2(h[0], h[1]);
    *reinterpret_cast<uint2*>(lo) = make_uint2(l[0], l[1]);
}

// int16 values -> int16 planes (hi = v >> 8, lo = v & 255) for int16 weights.
__device__ inline void put_planes_i16(const int16_t (&v)[8], int16_t* hi, int16_t* lo) {
    int16_t h[8], l[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) { h[t] = (int16_t)(v[t] >> 8); l[t] = (int16_t)(v[t] & 255); }
    *reinterpret_cast<uint4*>(hi) = *reinterpret_cast<const uint4*>(h);
    *reinterpret_cast<uint4*>(lo) = *reinterpret_cast<const uint4*>(l);
}

// Staging source: RMSNorm of x (x_shifts xs, gamma g/gs) from a NormAcc.
constexpr int kNormPre = 1;

struct SrcNorm {
    const int16_t* x;
    const uint8_t* xs;
    const int8_t* g;
    const uint8_t* gs;
    RmsParams p;
    uint8_t ref, out_frac;
    const NormAcc* acc;

    // the norm-sum words (threads < 64) and the first kNormPre chunks of x,
    // its shifts, gamma and gamma's shifts (one: every launch has K <= 8 x
    // its threads)
    struct Pre {
        uint64_t a[3];
        uint4 xv[kNormPre];
        uint2 sv[kNormPre], gv[kNormPre], gsv[kNormPre];
    };
    __device__ inline Pre pre(int K, int kpad, int nthr) const {
        Pre q;
        const __amdgpu_buffer_rsrc_t ra = weight_rsrc(acc, sizeof(NormAcc));
        const uint2 a01 = cload8(ra, threadIdx.x * 24u), a2 = cload8(ra, threadIdx.x * 24u + 8u);
        q.a[0] = ((uint64_t)a01.y << 32) | a01.x;
        q.a[1] = ((uint64_t)a2.y << 32) | a2.x;
        const uint2 a3 = cload8(ra, threadIdx.x * 24u + 16u);
        q.a[2] = ((uint64_t)a3.y << 32) | a3.x;
        const __amdgpu_buffer_rsrc_t rx = weight_rsrc(x, 2u * (uint32_t)K), rs = weight_rsrc(xs, (uint32_t)K),
                                     rg = weight_rsrc(g, (uint32_t)K), rgs = weight_rsrc(gs, (uint32_t)K);
#pragma unroll
        for (int j = 0; j < kNormPre; ++j) {
            const uint32_t k0 = (threadIdx.x + j * nthr) * 8u;
            q.xv[j] = cload16(rx, 2u * k0);
            q.sv[j] = cload8(rs, k0);
            q.gv[j] = cload8(rg, k0);
            q.gsv[j] = cload8(rgs, k0);
        }
        return q;
    }
    __device__ inline RmsFactor factor(const Pre& q) const {
        __shared__ RmsFactor sf;
        // every wave reduces (the words past thread 63 are zero): the
        // reduction has no branch to sink the norm-sum loads into
        uint64_t l[3];
#pragma unroll
        for (int j = 0; j < 3; ++j) l[j] = wave_sum_u64(q.a[j]);
        if (threadIdx.x < 64) {  // wave 0, every lane: the table entry is a wave-wide search
            const myl_i128 a = (myl_i128)((myl_u128)l[0] + ((myl_u128)l[1] << 42) + ((myl_u128)l[2] << 84));
            const RmsFactor f = rms_factor_wave(a, ref, p);
            if (threadIdx.x == 0) sf = f;
        }
        __syncthreads();
        return sf;
    }
    __device__ inline void values8(const RmsFactor& f, uint4 xv, uint2 sv, uint2 gv, uint2 gsv,
                                   int16_t (&v)[8]) const {
        const int16_t* xe = reinterpret_cast<const int16_t*>(&xv);
        const uint8_t* se = reinterpret_cast<const uint8_t*>(&sv);
        const int8_t* ge = reinterpret_cast<const int8_t*>(&gv);
        const uint8_t* gse = reinterpret_cast<const uint8_t*>(&gsv);
#pragma unroll
        for (int t = 0; t < 8; ++t) v[t] = rms_out(xe[t], se[t], ge[t], gse[t], f, out_frac);
    }
    // chunk i (k0 = 8 i) of the normalised vector; zeros past K
    template <class Put>
    __device__ inline void stage(const Pre& q, int K, int kpad, int nthr, const Put& put) const {
        const RmsFactor f = factor(q);
        const int n8 = kpad >> 3;
#pragma unroll
        for (int j = 0; j < kNormPre; ++j) {
            // zero operands past K give zero outputs
            int16_t v[8];
            values8(f, q.xv[j], q.sv[j], q.gv[j], q.gsv[j], v);
            put(stage_slot(threadIdx.x + j * nthr, n8), v);
        }
        for (int i = threadIdx.x + kNormPre * nthr; i < n8; i += nthr) {
            int16_t v[8];
            const int k0 = i * 8;
            if (k0 < K) {
                values8(f, *reinterpret_cast<const uint4*>(x + k0), *reinterpret_cast<const uint2*>(xs + k0),
                        *reinterpret_cast<const uint2*>(g + k0), *reinterpret_cast<const uint2*>(gs + k0), v);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) v[t] = 0;
            }
            put(i, v);
        }
    }
    __device__ inline void stage_i8(const Pre& q, int8_t* hi, int8_t* lo, int K, int kpad, int nthr) const {
        stage(q, K, kpad, nthr, [&](int i, const int16_t (&v)[8]) { put_planes_i8(v, hi + i * 8, lo + i * 8); });
    }
    __device__ inline void stage_i16(const Pre& q, int16_t* hi, int16_t* lo, int K, int kpad, int nthr) const {
        stage(q, K, kpad, nthr, [&](int i, const int16_t (&v)[8]) { put_planes_i16(v, hi + i * 8, lo + i * 8); });
    }
};

// Staging source: attention output from the exact P.V accumulator
// (attention.rs:84-86 then model.rs:563-567): i64 sums (Acc = unsigned long
// long, the general P.V kernel) or i32 sums (Acc = int32_t, the GQA kernel,
// exact where it runs).
template <class Acc>
struct SrcAttn {
    const Acc* acc;
    uint8_t v_frac, out_frac;
    static constexpr int kPieces = (int)sizeof(Acc) / 2;  // 16-byte pieces of 8 accumulators
    // the first chunk of each thread: 8 accumulators
    struct Pre {
        uint4 a[kPieces];
    };
    __device__ inline Pre pre(int K, int kpad, int nthr) const {
        Pre q;
        const __amdgpu_buffer_rsrc_t r = weight_rsrc(acc, (uint32_t)sizeof(Acc) * (uint32_t)K);
#pragma unroll
        for (int t = 0; t < kPieces; ++t) q.a[t] = cload16(r, threadIdx.x * (8u * (uint32_t)sizeof(Acc)) + 16u * t);
        return q;
    }
    __device__ inline void values8(const uint4 (&a4)[kPieces], int16_t (&v)[8]) const {
        int64_t a[8];
#pragma unroll
        for (int t = 0; t < kPieces; ++t) {
            if (sizeof(Acc) == 8) {
                a[2 * t] = (int64_t)(((uint64_t)a4[t].y << 32) | a4[t].x);
                a[2 * t + 1] = (int64_t)(((uint64_t)a4[t].w << 32) | a4[t].z);
            } else {
                a[4 * t] = (int32_t)a4[t].x;
                a[4 * t + 1] = (int32_t)a4[t].y;
                a[4 * t + 2] = (int32_t)a4[t].z;
                a[4 * t + 3] = (int32_t)a4[t].w;
            }
        }
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int16_t r = clamp_i16_i64(rshift_round64(a[t], MYL_TV_PROB_FRAC_BITS));
            v[t] = clamp_i16(rescale32((int32_t)r, v_frac, out_frac));
        }
    }
    __device__ inline void stage_i8(const Pre& q, int8_t* hi, int8_t* lo, int K, int kpad, int nthr) const {
        const int n8 = kpad >> 3;
        {
            // zero accumulators past K give zero outputs
            int16_t v[8];
            values8(q.a, v);
            const int i = stage_slot(threadIdx.x, n8);
            put_planes_i8(v, hi + i * 8, lo + i * 8);
        }
        for (int i = threadIdx.x + nthr; i < n8; i += nthr) {
            int16_t v[8];
            const int k0 = i * 8;
            if (k0 < K) {
                const uint4* a4 = reinterpret_cast<const uint4*>(acc + k0);
                uint4 w[kPieces];
#pragma unroll
                for (int t = 0; t < kPieces; ++t) w[t] = a4[t];
                values8(w, v);
            } else {
#pragma unroll
                for (int t = 0; t < 8; ++t) v[t] = 0;
            }
            put_planes_i8(v, hi + i * 8, lo + i * 8);
        }
    }
};

// ---------------------------------------------------------------------------
// embedding + step state (model.rs:241-248, 323-331)
// ---------------------------------------------------------------------------

// mode 0: token/pos from the arguments; mode 1: greedy continuation (token =
// argmax of the previous step, pos + 1).  Resets the argmax key for this step,
// copies the step's RoPE row (cos then sin, half entries each) to rope_cur
// and seeds the first layer's input-norm accumulator.
__global__ __launch_bounds__(1024) void embed_kernel(DecodeState* st, int mode, int token_arg, int pos_arg,
                                                     uint32_t rope_rows, int vocab, const int8_t* __restrict__ E,
                                                     const uint8_t* __restrict__ emb_shifts,
                                                     const uint8_t* __restrict__ res_frac0, uint8_t ref0, int H,
                                                     int64_t* __restrict__ tokens_out, int16_t* __restrict__ hidden,
                                                     NormAcc* norm_acc, const int16_t* __restrict__ cos_lut,
                                                     const int16_t* __restrict__ sin_lut, int half,
                                                     int16_t* __restrict__ rope_cur) {
    __shared__ int32_t s_tok, s_row;
    __shared__ uint64_t red[16 * 3];
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
        const int32_t row = (int32_t)umod32_slow((uint32_t)pos, rope_rows);
        st->token = tok;
        st->pos = pos;
        st->rope_row = row;
        st->argmax_key = 0;
        s_tok = tok;
        s_row = row;
    }
    __syncthreads();
    const int tok = s_tok;
    if ((int)threadIdx.x < 2 * half) {
        const bool c = (int)threadIdx.x < half;
        const int i = c ? (int)threadIdx.x : (int)threadIdx.x - half;  // no integer division
        rope_cur[threadIdx.x] = (c ? cos_lut : sin_lut)[(size_t)s_row * half + i];
    }
    const int8_t* row = E + (size_t)tok * H;
    const uint8_t sh = emb_shifts[tok];
    uint64_t l[3] = {0, 0, 0};
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const int16_t v = clamp_i16(rescale32((int32_t)row[i], sh, res_frac0[i]));
        hidden[i] = v;
        add_sq_limbs(v, res_frac0[i], ref0, l);
    }
    block_sum_limbs(l, red);
    for (int i = threadIdx.x; i < kNormSlots * 3; i += blockDim.x) (&norm_acc->v[0][0])[i] = 0;
    __syncthreads();
    if (threadIdx.x == 0)
        for (int j = 0; j < 3; ++j) norm_acc->v[0][j] = l[j];
}

// ---------------------------------------------------------------------------
// fused GEMV epilogues (streaming interface: begin / group per lane / finish)
// ---------------------------------------------------------------------------

// q/k/v projection rows (pair-ordered) -> bias -> RoPE -> q buffer / KV cache.
// The step's RoPE row is in rope (cos [hd / 2] then sin [hd / 2], written by
// the embedding kernel), so the rotation's operands are loads that depend on
// nothing.  The per-row operands load in group(): prefetching them after the
// first weight batch measured 0.46 us slower per launch on MI355X.
struct EpiQKV {
    const uint8_t* shifts;    // per device row
    const int16_t* bias;      // per device row, or null
    const uint8_t* bias_sh;
    uint8_t act_frac, q_frac, k_frac, v_frac;
    int nq, nkv, hd_log, max_pos;
    const int16_t* rope;
    const DecodeState* st;
    int16_t* q_out;           // [nq]
    int16_t* kc;              // layer base [kv_heads][max_pos][hd]
    int16_t* vc;
    using State = NoState;
    __device__ inline void begin(State&) const {}
    __device__ inline void prefetch(State&, int, int) const {}
    __device__ inline void finish(State&) const {}
    template <int R>
    __device__ inline void group(State&, int row0, int N, const int64_t (&tot)[R]) const {
        static_assert(R == 2, "the RoPE pair needs two rows per group");
        if (row0 >= N) return;
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
            int16_t v = clamp_i16_i64(rescale64(tot[t], (uint8_t)(shifts[d] + act_frac), frac));
            if (bias) v = clamp_i16_i64((int64_t)v + (int64_t)rescale32((int32_t)bias[d], bias_sh[d], frac));
            y[t] = v;
        }
        const int pos = st->pos;
        if (seg < 2) {
            const int32_t c = rope[p];
            const int32_t sn = rope[half + p];
            const int32_t x0 = y[0], x1 = y[1];
            y[0] = clamp_i16(rshift_round32(wsub32(wmul32(x0, c), wmul32(x1, sn)), MYL_TV_ROPE_FRAC_BITS));
            y[1] = clamp_i16(rshift_round32(wadd32(wmul32(x1, c), wmul32(x0, sn)), MYL_TV_ROPE_FRAC_BITS));
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
// plus the next RMSNorm's sum of squares of `out` into sum_out, and clearing
// of a NormAcc whose consumer has already run.
struct EpiResid {
    const uint8_t* shifts;
    uint8_t act_frac;
    const uint8_t* acc_frac;   // min(res_frac, out_frac) per channel
    const uint8_t* res_frac;
    const uint8_t* out_frac;
    const int16_t* res_in;
    int16_t* out;
    NormAcc* sum_out;
    uint8_t ref_out;           // max over out_frac
    NormAcc* clear;            // may be null
    // the norm partial sums, and the per-row operands of the lane's first
    // group (up to two rows)
    struct State {
        uint64_t l[3];
        int row0;
        uint8_t sh[2], af[2], rf[2], of[2];
        int16_t res[2];
    };
    __device__ inline void begin(State& s) const {
        s.l[0] = s.l[1] = s.l[2] = 0;
        s.row0 = -1;
    }
    __device__ inline void prefetch(State& s, int row0, int N) const {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int i = min(row0 + r, N - 1);
            s.sh[r] = shifts[i];
            s.af[r] = acc_frac[i];
            s.rf[r] = res_frac[i];
            s.of[r] = out_frac[i];
            s.res[r] = res_in[i];
        }
        s.row0 = row0;
    }
    template <int R>
    __device__ inline void group(State& s, int row0, int N, const int64_t (&tot)[R]) const {
        static_assert(R <= 2, "two prefetched rows per group");
        const bool pre = s.row0 == row0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r < N) {
                const int i = row0 + r;
                const uint8_t af = pre ? s.af[r] : acc_frac[i];
                const uint8_t sh = pre ? s.sh[r] : shifts[i];
                const int16_t ri = pre ? s.res[r] : res_in[i];
                const uint8_t rf = pre ? s.rf[r] : res_frac[i];
                const int16_t o = clamp_i16_i64(rescale64(tot[r], (uint8_t)(sh + act_frac), af));
                const int64_t h = rescale64((int64_t)ri, rf, af);
                const uint8_t of = pre ? s.of[r] : out_frac[i];
                const int16_t v = clamp_i16_i64(rescale64(wadd64(h, (int64_t)o), af, of));
                out[i] = v;
                add_sq_limbs(v, of, ref_out, s.l);
            }
        }
    }
    __device__ inline void finish(State& s) const {
        if (clear && blockIdx.x == 0)
            for (int i = threadIdx.x; i < kNormSlots * 3; i += blockDim.x) (&clear->v[0][0])[i] = 0;
        __shared__ uint64_t red[16 * 3];
        block_sum_limbs(s.l, red);
        if (threadIdx.x == 0) {
            const int slot = blockIdx.x & (kNormSlots - 1);
            for (int j = 0; j < 3; ++j)
                if (s.l[j]) atomicAdd(&sum_out->v[slot][j], (unsigned long long)s.l[j]);
        }
    }
};

// gate row 2r and up row 2r+1 -> h[r] (mlp.rs:46-65); clears the attention
// accumulator (its reader, o_proj, has finished).
struct EpiSilu {
    const uint8_t* shifts;    // interleaved like the rows
    uint8_t act_frac, gate_frac, up_frac, down_in_frac;
    const int16_t* silu; uint32_t silu_len;
    int16_t* h;
    unsigned long long* clear; int clear_n;
    using State = NoState;
    __device__ inline void begin(State&) const {}
    // two shift bytes: loading them early measured slower
    __device__ inline void prefetch(State&, int, int) const {}
    __device__ inline void finish(State&) const {
        for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < clear_n; i += gridDim.x * blockDim.x) clear[i] = 0;
    }
    template <int R>
    __device__ inline void group(State&, int row0, int N, const int64_t (&tot)[R]) const {
        static_assert(R == 2, "gate and up share a group");
        if (row0 >= N) return;
        const int16_t g = clamp_i16_i64(rescale64(tot[0], (uint8_t)(shifts[row0] + act_frac), gate_frac));
        const int16_t u = clamp_i16_i64(rescale64(tot[1], (uint8_t)(shifts[row0 + 1] + act_frac), up_frac));
        const int32_t g_dom = rescale32((int32_t)g, gate_frac, MYL_TV_SILU_IN_FRAC);
        const int16_t act = lut_lookup_i16((int16_t)g_dom, silu, silu_len, (int16_t)MYL_TV_SILU_LUT_OFFSET);
        const int64_t prod = (int64_t)act * (int64_t)u;
        h[row0 >> 1] = clamp_i16_i64(rescale64(prod, (uint8_t)(MYL_TV_SILU_OUT_FRAC + up_frac), down_in_frac));
    }
};

// LM head logits (model.rs:284-308) + first-maximum argmax (sampling.rs:8-18):
// each lane keeps the best key of its rows; the block's maximum (waves, then
// the block through LDS) goes to one atomic, issued only when it beats the
// current key.  Every atomic of a launch targets one word, so they serialise:
// one per block rather than one per wave.
struct EpiHead {
    const uint8_t* shifts;
    uint8_t norm_frac;
    int32_t* logits;
    DecodeState* st;
    struct State {
        uint64_t best;
        int row0;
        uint8_t sh[2];
    };
    __device__ inline void begin(State& s) const {
        s.best = 0;
        s.row0 = -1;
    }
    __device__ inline void prefetch(State& s, int row0, int N) const {
        s.sh[0] = shifts[min(row0, N - 1)];
        s.sh[1] = shifts[min(row0 + 1, N - 1)];
        s.row0 = row0;
    }
    template <int R>
    __device__ inline void group(State& s, int row0, int N, const int64_t (&tot)[R]) const {
        static_assert(R <= 2, "two prefetched rows per group");
        const bool pre = s.row0 == row0;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r < N) {
                const uint8_t sh = pre ? s.sh[r] : shifts[row0 + r];
                const int32_t v = clamp_i32_i64(rescale64(tot[r], (uint8_t)(sh + norm_frac),
                                                          MYL_TV_LOGIT_FRAC_BITS));
                logits[row0 + r] = v;
                const uint64_t k = argmax_key(v, (uint32_t)(row0 + r));
                s.best = k > s.best ? k : s.best;
            }
        }
    }
    __device__ inline void finish(State& s) const {
        __shared__ uint64_t wbest[16];
        const uint64_t best = wave_max_u64(s.best);
        const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6, lane = threadIdx.x & 63;
        if (lane == 0) wbest[w] = best;
        __syncthreads();
        if (w == 0) {
            const uint64_t b = wave_max_u64(lane < nw ? wbest[lane] : 0ull);
            if (lane == 0 && b) {
                const uint64_t cur = __hip_atomic_load(&st->argmax_key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (b > cur) atomicMax((unsigned long long*)&st->argmax_key, (unsigned long long)b);
            }
        }
    }
};

// ---------------------------------------------------------------------------
// decode attention over the KV cache (attention.rs:42-90), GQA (model.rs:508-511)
// ---------------------------------------------------------------------------

// Launch shape of the attention kernels, one query head per block.  Workgroups
// are dispatched to the 8 XCDs round robin in linear-id order, and each XCD
// has its own L2.  With kv_heads dividing 8 (xs_log = log2(8 / kv_heads)):
// grid 8 * G * ceil(chunks / 2^xs_log); block x, with k = x >> 3 (the XCD's
// k-th block), works on query head k % G of KV head (x & 7) >> xs_log and on
// position chunk (k / G) 2^xs_log + (x & (2^xs_log - 1)), so each KV head's
// chunks stay on its 2^xs_log XCDs and the G heads of a chunk run there
// back to back: a chunk's K or V rows are read into one L2 for the heads that
// share them, and a head's score row into 2^xs_log L2s rather than all 8.
// Otherwise (xs_log < 0): grid dim3(8 * G, ceil(chunks / 8),
// kv_heads); block (x, y, z) works on query head x >> 3 of KV head z and on
// chunk y * 8 + (x & 7), the G head blocks of a chunk on one XCD.
struct AttnBlock {
    int h, c, g;
    __device__ AttnBlock(int xs_log, int G, uint32_t ginv) {
        if (xs_log >= 0) {
            const int xcd = (int)blockIdx.x & 7, k = (int)blockIdx.x >> 3;
            const int cc = (int)(((uint64_t)(uint32_t)k * ginv) >> 24);  // k / G: ginv = ceil(2^24 / G), k G < 2^24
            h = k - cc * G;
            g = xcd >> xs_log;
            c = (cc << xs_log) + (xcd & ((1 << xs_log) - 1));
        } else {
            h = (int)blockIdx.x >> 3;
            c = (int)blockIdx.y * 8 + ((int)blockIdx.x & 7);
            g = (int)blockIdx.z;
        }
    }
};

template <int HD>
__global__ __launch_bounds__(256) void attn_scores_kernel(const DecodeState* __restrict__ st,
                                                         const int16_t* __restrict__ q, const int16_t* __restrict__ kc,
                                                         int max_pos, int G, int chunks, int64_t score_mult,
                                                         uint8_t score_shift, int32_t* __restrict__ scores,
                                                         int score_ld, int xs_log, uint32_t ginv) {
    const AttnBlock b(xs_log, G, ginv);
    if (b.c >= chunks) return;
    const int L = st->pos + 1;
    const int base = b.c * kChunk;
    if (base >= L) return;
    const int head = b.g * G + b.h;
    dec_scores<HD>(L, base, q + (size_t)head * HD, kc + (size_t)b.g * max_pos * HD, score_mult, score_shift,
                   scores + (size_t)head * score_ld);
}

// P.V of one query head over kPvWide positions (dec_pv_wide), i32 partials
// into acc.  512 threads; AttnBlock over chunks of kPvWide positions.
template <int HD>
__global__ __launch_bounds__(512) void attn_pv_wide_kernel(const DecodeState* __restrict__ st,
                                                          const int32_t* __restrict__ scores,
                                                          const int16_t* __restrict__ vc, int max_pos, int score_ld,
                                                          int G, int chunks, const int16_t* __restrict__ lut,
                                                          uint32_t lut_len, uint8_t lut_shift, int exp_lds,
                                                          int32_t* __restrict__ acc, int xs_log, uint32_t ginv) {
    const AttnBlock b(xs_log, G, ginv);
    if (b.c >= chunks) return;
    const int L = st->pos + 1;
    const int base = b.c * kPvWide;
    if (base >= L) return;
    const int head = b.g * G + b.h;
    dec_pv_wide<HD>(L, base, scores + (size_t)head * score_ld, score_ld, vc + (size_t)b.g * max_pos * HD, lut,
                    lut_len, lut_shift, exp_lds, acc + (size_t)head * HD);
}

// The whole attention of one query head per block (dec_attn_short) for
// contexts of at most dec_short_max<HD>() positions: grid (G, kv_heads),
// block (h, g) works on query head g G + h; the head's i32 output is stored
// to acc.  512 threads.
template <int HD>
__global__ __launch_bounds__(512) void attn_short_kernel(const DecodeState* __restrict__ st,
                                                        const int16_t* __restrict__ q, const int16_t* __restrict__ kc,
                                                        const int16_t* __restrict__ vc, int max_pos, int G,
                                                        int64_t score_mult, uint8_t score_shift,
                                                        const int16_t* __restrict__ lut, uint32_t lut_len,
                                                        uint8_t lut_shift, int exp_lds, int32_t* __restrict__ acc) {
    const int L = st->pos + 1;
    if (L > dec_short_max<HD>()) return;  // the launcher bounds max_pos
    const int g = (int)blockIdx.y, head = g * G + (int)blockIdx.x;
    const size_t kv = (size_t)g * max_pos * HD;
    dec_attn_short<HD>(L, q + (size_t)head * HD, kc + kv, vc + kv, score_mult, score_shift, lut, lut_len, lut_shift,
                       exp_lds, acc + (size_t)head * HD);
}

// The general P.V kernel (dec_pv): one query head and kChunk positions, i64
// partials into acc.
template <int HD>
__global__ __launch_bounds__(256) void attn_pv_kernel(const DecodeState* __restrict__ st,
                                                     const int32_t* __restrict__ scores,
                                                     const int16_t* __restrict__ vc, int max_pos, int score_ld, int G,
                                                     int chunks, const int16_t* __restrict__ lut, uint32_t lut_len,
                                                     uint8_t lut_shift, int exp_lds,
                                                     unsigned long long* __restrict__ acc, int xs_log,
                                                     uint32_t ginv) {
    const AttnBlock b(xs_log, G, ginv);
    if (b.c >= chunks) return;
    const int L = st->pos + 1;
    const int base = b.c * kChunk;
    if (base >= L) return;
    const int head = b.g * G + b.h;
    dec_pv<HD>(L, base, scores + (size_t)head * score_ld, score_ld, vc + (size_t)b.g * max_pos * HD, lut, lut_len,
               lut_shift, exp_lds, acc + (size_t)head * HD);
}

// ---------------------------------------------------------------------------
// host-side model
// ---------------------------------------------------------------------------

}  // namespace

namespace {

// Kernel classes of one decode step, for the per-class event timing.
enum KClass { K_EMBED = 0, K_RMS, K_QKV, K_ATTN, K_O, K_GU, K_DOWN, K_HEAD, K_COUNT };

struct TimedScope {
    myl_model* m;
    int cls;
    size_t idx = 0;
    TimedScope(myl_model* mm, int c) : m(mm), cls(c) {
        if (!m->timing) return;
        while (m->ev_pool.size() < m->ev_used + 2) {
            hipEvent_t e;
            if (hipEventCreate(&e) != hipSuccess) { m->timing = false; return; }
            m->ev_pool.push_back(e);
        }
        idx = m->ev_used;
        m->ev_used += 2;
        (void)hipEventRecord(m->ev_pool[idx], m->ctx->stream);
    }
    ~TimedScope() {
        if (!m->timing || m->ev_used < idx + 2) return;
        (void)hipEventRecord(m->ev_pool[idx + 1], m->ctx->stream);
        m->marks.push_back({cls, idx});
    }
};

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

// Allocates every device buffer of a model of m's dimensions, uploads the
// LUTs and the row maps, and clears the caches.  Tensors and scales are
// written afterwards by the synthetic generator (synth_fill) or the uploader
// (model_io.hip); model_finalize() seals the model.
int alloc_impl(myl_model* m, const myl_luts* luts) {
    myl_ctx* c = m->ctx;
    const myl_synth_spec& s = m->spec;
    const int H = m->H, I = m->I, V = m->V, hd = m->hd, nq = m->nq, nkv = m->nkv;
    const int nqkv = nq + 2 * nkv;

    // LUTs
    m->rsqrt_len = (int)luts->rsqrt_len;
    m->silu_len = (int)luts->silu_len;
    m->exp_len = (int)luts->exp_len;
    m->exp_nz = 0;
    for (int i = m->exp_len - 1; i >= 0; --i)
        if (luts->exp[i] != 0) {
            m->exp_nz = i + 1;
            break;
        }
    // the wide P.V kernel accumulates in i32: exact for a table without
    // negative entries (dec_attn.h) whose nonzero prefix fits its LDS copy
    m->pv32 = m->exp_nz <= kDecExpLds && m->max_pos <= 65536;
    for (size_t i = 0; i < luts->exp_len && m->pv32; ++i)
        if (luts->exp[i] < 0) m->pv32 = false;
    // a table equal to its closed form at every entry is computed in the
    // norm setup instead of read: the read is a dependent load that waits
    // behind the weight stream the kernel has already issued
    m->rsqrt_closed = MYL_TV_RSQRT_OUTPUT_FRAC + (MYL_TV_RSQRT_INPUT_SHIFT + 1) / 2 <= 20;
    for (size_t i = 0; i < luts->rsqrt_len && m->rsqrt_closed; ++i)
        if (luts->rsqrt[i] != rsqrt_closed((uint32_t)i, MYL_TV_RSQRT_OUTPUT_FRAC, MYL_TV_RSQRT_INPUT_SHIFT))
            m->rsqrt_closed = 0;
    m->rope_rows = (uint32_t)(luts->rope_len / (size_t)(hd / 2));
    m->rsqrt = m->dalloc<int16_t>(luts->rsqrt_len);
    m->silu = m->dalloc<int16_t>(luts->silu_len);
    const size_t exp_pad = (luts->exp_len + 7) & ~(size_t)7;  // whole 16-byte pieces (dec_pv)
    m->exp_lut = m->dalloc<int16_t>(exp_pad ? exp_pad : 8);
    m->cos_lut = m->dalloc<int16_t>(luts->rope_len);
    m->sin_lut = m->dalloc<int16_t>(luts->rope_len);
    if (!m->rsqrt || !m->silu || !m->exp_lut || !m->cos_lut || !m->sin_lut) return c->fail(MYL_E_NOMEM, "LUT allocation");
    int rc = 0;
    rc |= upload(m, m->rsqrt, std::vector<int16_t>(luts->rsqrt, luts->rsqrt + luts->rsqrt_len));
    rc |= upload(m, m->silu, std::vector<int16_t>(luts->silu, luts->silu + luts->silu_len));
    std::vector<int16_t> exp_host(luts->exp, luts->exp + luts->exp_len);
    exp_host.resize(exp_pad, 0);
    rc |= upload(m, m->exp_lut, exp_host);
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

    // embedding / LM heads / final norm
    m->emb = m->dalloc<int8_t>((size_t)V * H);
    m->emb_shifts = m->dalloc<uint8_t>(V);
    m->final_gamma = m->dalloc<int8_t>(H);
    m->final_gamma_s = m->dalloc<uint8_t>(H);
    m->final_res = m->dalloc<uint8_t>(H);
    if (!m->emb || !m->emb_shifts || !m->final_gamma || !m->final_gamma_s || !m->final_res)
        return c->fail(MYL_E_NOMEM, "embedding allocation");
    if (s.lm_head_int16) {
        m->lm16 = m->dalloc<int16_t>((size_t)V * H);
        m->lm16_shifts = m->dalloc<uint8_t>(V);
        if (!m->lm16 || !m->lm16_shifts) return c->fail(MYL_E_NOMEM, "LM head allocation");
    } else if (!m->tied) {
        m->lm8 = m->dalloc<int8_t>((size_t)V * H);
        m->lm8_shifts = m->dalloc<uint8_t>(V);
        if (!m->lm8 || !m->lm8_shifts) return c->fail(MYL_E_NOMEM, "LM head allocation");
    }
    if (m->tied) {
        m->lm8 = m->emb;
        m->lm8_shifts = m->emb_shifts;
    }

    // Stored row of each logical output row: q/k/v heads pair-ordered for the
    // fused RoPE, gate and up rows interleaved for the fused SiLU product.
    m->qkv_map.resize(nqkv);
    for (int o = 0; o < nq; ++o) m->qkv_map[o] = pair_row(o, hd);
    for (int o = 0; o < nkv; ++o) m->qkv_map[nq + o] = nq + pair_row(o, hd);
    for (int o = 0; o < nkv; ++o) m->qkv_map[nq + nkv + o] = nq + nkv + pair_row(o, hd);
    m->gu_map.resize(2 * (size_t)I);
    for (int r = 0; r < I; ++r) { m->gu_map[r] = 2 * r; m->gu_map[I + r] = 2 * r + 1; }
    m->qkv_map_dev = m->dalloc<int32_t>(nqkv);
    m->gu_map_dev = m->dalloc<int32_t>(2 * (size_t)I);
    if (!m->qkv_map_dev || !m->gu_map_dev) return c->fail(MYL_E_NOMEM, "row tables");
    rc |= upload(m, m->qkv_map_dev, m->qkv_map);
    rc |= upload(m, m->gu_map_dev, m->gu_map);
    if (rc) return MYL_E_HIP;

    m->layers.resize(s.layers);
    for (uint32_t l = 0; l < s.layers; ++l) {
        LayerDev& L = m->layers[l];
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
    }
    m->h_res_in.assign(s.layers, std::vector<uint8_t>(H, 0));
    m->h_res_mid.assign(s.layers, std::vector<uint8_t>(H, 0));
    m->h_final_res.assign(H, 0);
    m->have.assign(myl::kModelSlots + (size_t)myl::kLayerSlots * s.layers, 0);
    m->scales_have.assign(s.layers, 0);
    m->final_have = false;
    m->ready = false;

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
    m->score_ld = (m->max_pos + 3) & ~3;
    m->scores = m->dalloc<int32_t>((size_t)s.heads * m->score_ld);
    m->attn_acc = m->dalloc<unsigned long long>((size_t)nq);
    m->norm_a = m->dalloc<NormAcc>(1);
    m->norm_b = m->dalloc<NormAcc>(1);
    m->state = m->dalloc<DecodeState>(1);
    m->rope_cur = m->dalloc<int16_t>(hd);
    if (!m->rope_cur) return c->fail(MYL_E_NOMEM, "activation allocation");
    if (!m->kcache || !m->vcache || !m->hidden || !m->norm || !m->q || !m->attn || !m->resid || !m->h ||
        !m->logits || !m->scores || !m->attn_acc || !m->state || !m->norm_a || !m->norm_b)
        return c->fail(MYL_E_NOMEM, "activation allocation");
    if (hipMemsetAsync(m->kcache, 0, kv * 2, c->stream) != hipSuccess ||
        hipMemsetAsync(m->vcache, 0, kv * 2, c->stream) != hipSuccess ||
        hipMemsetAsync(m->state, 0, sizeof(DecodeState), c->stream) != hipSuccess ||
        hipMemsetAsync(m->attn_acc, 0, (size_t)nq * 8, c->stream) != hipSuccess ||
        hipMemsetAsync(m->norm_a, 0, sizeof(NormAcc), c->stream) != hipSuccess ||
        hipMemsetAsync(m->norm_b, 0, sizeof(NormAcc), c->stream) != hipSuccess)
        return MYL_E_HIP;
    return c->hip(hipStreamSynchronize(c->stream), "model allocation");
}

// Checks that every tensor and scale has arrived, derives the accumulation
// scales of the two residual adds, min(res_in, res_mid) and
// min(res_mid, res_out) per channel (model.rs:576-581,612-617), and the
// per-segment maxima the RMSNorm reference shift takes (rmsnorm.rs:96).
int finalize_impl(myl_model* m) {
    myl_ctx* c = m->ctx;
    const myl_synth_spec& s = m->spec;
    const int H = m->H;
    for (size_t i = 0; i < m->have.size(); ++i) {
        if (m->have[i] || !myl::slot_required(m, i)) continue;
        return c->fail(MYL_E_INVALID, "model: missing tensor " + myl::slot_name(m, i));
    }
    for (uint32_t l = 0; l < s.layers; ++l)
        if (!m->scales_have[l])
            return c->fail(MYL_E_INVALID, "model: missing activation scales of layer " + std::to_string(l));
    if (!m->final_have) return c->fail(MYL_E_INVALID, "model: missing final norm scales (model.norm)");
    auto vmax = [](const std::vector<uint8_t>& v) { uint8_t r = 0; for (uint8_t x : v) r = std::max(r, x); return r; };
    int rc = upload(m, m->final_res, m->h_final_res);
    m->ref_final = vmax(m->h_final_res);
    for (uint32_t l = 0; l < s.layers && !rc; ++l) {
        LayerDev& L = m->layers[l];
        const std::vector<uint8_t>& in = m->h_res_in[l];
        const std::vector<uint8_t>& mid = m->h_res_mid[l];
        const std::vector<uint8_t>& out = (l + 1 < s.layers) ? m->h_res_in[l + 1] : m->h_final_res;
        std::vector<uint8_t> acc_a(H), acc_m(H);
        for (int i = 0; i < H; ++i) {
            acc_a[i] = std::min(in[i], mid[i]);
            acc_m[i] = std::min(mid[i], out[i]);
        }
        rc |= upload(m, L.res_in, in);
        rc |= upload(m, L.res_mid, mid);
        rc |= upload(m, L.acc_attn, acc_a);
        rc |= upload(m, L.acc_mlp, acc_m);
        // The uploads read host vectors that live until the synchronisation below.
        rc |= c->hip(hipStreamSynchronize(c->stream), "model finalize");
        L.res_out = (l + 1 < s.layers) ? m->layers[l + 1].res_in : m->final_res;
        L.ref_in = vmax(in);
        L.ref_mid = vmax(mid);
        L.ref_out = vmax(out);
    }
    if (rc) return MYL_E_HIP;
    // A captured decode step holds the previous scales as kernel arguments.
    if (m->step_exec) (void)hipGraphExecDestroy(m->step_exec);
    if (m->step_graph) (void)hipGraphDestroy(m->step_graph);
    m->step_exec = nullptr;
    m->step_graph = nullptr;
    int r = c->hip(hipStreamSynchronize(c->stream), "model finalize");
    if (!r) m->ready = true;
    return r;
}

// The seeded synthetic model of include/myl_synth.h, generated in place.
int synth_fill(myl_model* m) {
    myl_ctx* c = m->ctx;
    const myl_synth_spec& s = m->spec;
    const uint64_t seed = s.seed;
    const int H = m->H, I = m->I, V = m->V, nq = m->nq, nkv = m->nkv;
    const int nqkv = nq + 2 * nkv;
    const std::vector<int32_t>& qkv_rows = m->qkv_map;
    int rc = 0;
    if (gen_w8(m, m->emb, nullptr, V, H, myl_tensor_seed(seed, 0, MYL_R_EMB)) != hipSuccess) return MYL_E_HIP;
    rc |= upload(m, m->emb_shifts, small_u8(seed, 0, MYL_R_EMB_SHIFT, V));
    if (s.lm_head_int16) {
        if (gen_w16(m, m->lm16, V, H, myl_tensor_seed(seed, 0, MYL_R_LM16)) != hipSuccess) return MYL_E_HIP;
        rc |= upload(m, m->lm16_shifts, small_u8(seed, 0, MYL_R_LM16_SHIFT, V));
    }
    if (gen_w8(m, m->final_gamma, nullptr, 1, H, myl_tensor_seed(seed, 0, MYL_R_FINAL_GAMMA)) != hipSuccess) return MYL_E_HIP;
    rc |= upload(m, m->final_gamma_s, small_u8(seed, 0, MYL_R_FINAL_GAMMA_SHIFT, H));
    {
        const uint64_t ts = myl_tensor_seed(seed, 0, MYL_R_FINAL_RES_FRAC);
        for (int i = 0; i < H; ++i) m->h_final_res[i] = myl_synth_res_frac(ts, i);
    }
    m->final_norm_frac = myl_synth_final_norm_frac(seed);
    for (uint32_t l = 0; l < s.layers; ++l) {
        const uint64_t ti = myl_tensor_seed(seed, l, MYL_R_RES_IN), tm = myl_tensor_seed(seed, l, MYL_R_RES_MID);
        for (int i = 0; i < H; ++i) {
            m->h_res_in[l][i] = myl_synth_res_frac(ti, i);
            m->h_res_mid[l][i] = myl_synth_res_frac(tm, i);
        }
    }
    const int32_t* qkv_rows_dev = m->qkv_map_dev;
    const int32_t* gu_rows_dev = m->gu_map_dev;
    for (uint32_t l = 0; l < s.layers; ++l) {
        LayerDev& L = m->layers[l];
        L.f = myl_synth_layer_fracs(seed, l);
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
        if (rc) return MYL_E_HIP;
    }
    std::fill(m->have.begin(), m->have.end(), 1);
    std::fill(m->scales_have.begin(), m->scales_have.end(), 1);
    m->final_have = true;
    return finalize_impl(m);
}

RmsParams rms_params(const myl_model* m) {
    return RmsParams{m->rsqrt, m->rsqrt_len, MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20,
                     m->rsqrt_closed};
}

// One transformer layer on m->hidden (model.rs:401-674); the result replaces
// m->hidden and its input-norm sum is left in norm_a for the next consumer.
//   qkv   : RMSNorm(hidden) staged from norm_a            -> q, KV cache
//   attn  : scores, then softmax + P.V into attn_acc
//   o     : attn_acc staged, residual 1 -> resid; sum -> norm_b; clears norm_a
//   gu    : RMSNorm(resid) staged from norm_b             -> h; clears attn_acc
//   down  : h, residual 2 -> hidden; sum -> norm_a; clears norm_b
hipError_t layer_step(myl_model* m, int l) {
    const LayerDev& L = m->layers[l];
    const myl_layer_fracs& f = L.f;
    hipStream_t st = m->ctx->stream;
    const int H = m->H, I = m->I, nq = m->nq, nkv = m->nkv, hd = m->hd, G = m->G, cus = m->cus;
    const int kvh = (int)m->spec.kv_heads;
    const RmsParams rp = rms_params(m);
    hipError_t e;
    {
        const size_t layer_kv = (size_t)l * kvh * m->max_pos * hd;
        EpiQKV q{L.sqkv, L.bqkv, L.bsqkv, f.norm_attn_frac, f.q_frac, f.k_frac, f.v_frac, nq, nkv, m->hd_log,
                 m->max_pos, m->rope_cur, m->state, m->q, m->kcache + layer_kv, m->vcache + layer_kv};
        SrcNorm src{m->hidden, L.res_in, L.in_gamma, L.in_gamma_s, rp, L.ref_in, f.norm_attn_frac, m->norm_a};
        {
            TimedScope t(m, K_QKV);
            // one 1 KiB step covers a row of a small model (0.5B: K = 896):
            // 4-wave blocks without a second step per batch measured 4 %
            // faster per token there
            e = H <= 1024 ? stream_i8<2, 1, 4>(src, L.wqkv, nq + 2 * nkv, H, q, st, cus)
                          : stream_i8<2, 2, 16>(src, L.wqkv, nq + 2 * nkv, H, q, st, cus);
        }
        if (e != hipSuccess) return e;
        TimedScope ta(m, K_ATTN);
        const uint32_t ss = (uint32_t)f.q_frac + f.k_frac + 15u;
        const uint8_t score_shift = (uint8_t)(ss > MYL_TV_SCORE_FRAC_BITS ? ss - MYL_TV_SCORE_FRAC_BITS : 0);
        const uint8_t lut_shift = MYL_TV_SCORE_FRAC_BITS - MYL_TV_EXP_INPUT_FRAC;
        const int16_t* kc = m->kcache + layer_kv;
        const int16_t* vc = m->vcache + layer_kv;
        int xs_log = -1;  // AttnBlock
        if (kvh <= 8 && 8 % kvh == 0)
            for (xs_log = 0; (kvh << xs_log) < 8;) ++xs_log;
        const uint32_t ginv = ((1u << 24) + (uint32_t)G - 1) / (uint32_t)G;
        auto attn_grid = [&](int chunks, int& xsl) {
            xsl = xs_log;
            if (xsl >= 0 && (int64_t)G * G * ((chunks + (1 << xsl) - 1) >> xsl) >= (1 << 24)) xsl = -1;
            return xsl >= 0 ? dim3(8 * G * ((chunks + (1 << xsl) - 1) >> xsl)) : dim3(8 * G, (chunks + 7) / 8, kvh);
        };
        // a short cache: one kernel, one block per query head
        if (m->pv32 && m->max_pos <= (hd == 128 ? dec_short_max<128>() : dec_short_max<64>())) {
            int32_t* acc = reinterpret_cast<int32_t*>(m->attn_acc);
            if (hd == 128)
                attn_short_kernel<128><<<dim3(G, kvh), 512, 0, st>>>(m->state, m->q, kc, vc, m->max_pos, G,
                                                                     m->score_mult, score_shift, m->exp_lut,
                                                                     (uint32_t)m->exp_len, lut_shift, m->exp_nz, acc);
            else
                attn_short_kernel<64><<<dim3(G, kvh), 512, 0, st>>>(m->state, m->q, kc, vc, m->max_pos, G,
                                                                    m->score_mult, score_shift, m->exp_lut,
                                                                    (uint32_t)m->exp_len, lut_shift, m->exp_nz, acc);
        } else {
            const int chunks = (m->max_pos + kChunk - 1) / kChunk;
            int sxs = -1;
            const dim3 agrid = attn_grid(chunks, sxs);
            if (hd == 128)
                attn_scores_kernel<128><<<agrid, 256, 0, st>>>(m->state, m->q, kc, m->max_pos, G, chunks, m->score_mult,
                                                              score_shift, m->scores, m->score_ld, sxs, ginv);
            else
                attn_scores_kernel<64><<<agrid, 256, 0, st>>>(m->state, m->q, kc, m->max_pos, G, chunks, m->score_mult,
                                                             score_shift, m->scores, m->score_ld, sxs, ginv);
            if (m->pv32) {
                const int wchunks = (m->max_pos + kPvWide - 1) / kPvWide;
                int wxs = -1;
                const dim3 wgrid = attn_grid(wchunks, wxs);
                int32_t* acc = reinterpret_cast<int32_t*>(m->attn_acc);
                if (hd == 128)
                    attn_pv_wide_kernel<128><<<wgrid, 512, 0, st>>>(m->state, m->scores, vc, m->max_pos,
                                                                    m->score_ld, G, wchunks, m->exp_lut,
                                                                    (uint32_t)m->exp_len, lut_shift, m->exp_nz, acc,
                                                                    wxs, ginv);
                else
                    attn_pv_wide_kernel<64><<<wgrid, 512, 0, st>>>(m->state, m->scores, vc, m->max_pos, m->score_ld, G,
                                                                   wchunks, m->exp_lut, (uint32_t)m->exp_len, lut_shift,
                                                                   m->exp_nz, acc, wxs, ginv);
            } else {
                const int exp_lds = m->exp_nz <= kDecExpLds ? m->exp_nz : -1;
                if (hd == 128)
                    attn_pv_kernel<128><<<agrid, 256, 0, st>>>(m->state, m->scores, vc, m->max_pos, m->score_ld, G,
                                                              chunks, m->exp_lut, (uint32_t)m->exp_len, lut_shift,
                                                              exp_lds, m->attn_acc, sxs, ginv);
                else
                    attn_pv_kernel<64><<<agrid, 256, 0, st>>>(m->state, m->scores, vc, m->max_pos, m->score_ld, G,
                                                             chunks, m->exp_lut, (uint32_t)m->exp_len, lut_shift,
                                                             exp_lds, m->attn_acc, sxs, ginv);
            }
        }
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    {
        TimedScope t(m, K_O);
        EpiResid o{L.so, f.attn_out_frac, L.acc_attn, L.res_in, L.res_mid, m->hidden, m->resid, m->norm_b, L.ref_mid,
                   m->norm_a};
        // 8-wave blocks streaming 4 KiB per row per batch, one block per CU:
        // 10.8 -> 9.7 us per launch on MI355X at 7B widths (16-wave blocks,
        // two-step batches, as many blocks as fit: the previous shape)
        auto o_proj = [&](const auto& src) {
            return nq <= 1024 ? stream_i8<1, 1, 4>(src, L.wo, H, nq, o, st, cus)
                              : stream_i8<1, 4, 8>(src, L.wo, H, nq, o, st, cus, 1);
        };
        if (m->pv32)
            e = o_proj(SrcAttn<int32_t>{reinterpret_cast<const int32_t*>(m->attn_acc), f.v_frac, f.attn_out_frac});
        else
            e = o_proj(SrcAttn<unsigned long long>{m->attn_acc, f.v_frac, f.attn_out_frac});
        if (e != hipSuccess) return e;
    }
    {
        SrcNorm src{m->resid, L.res_mid, L.post_gamma, L.post_gamma_s, rp, L.ref_mid, f.norm_mlp_frac, m->norm_b};
        EpiSilu s{L.sgu, f.norm_mlp_frac, f.gate_frac, f.up_frac, f.down_in_frac, m->silu, (uint32_t)m->silu_len, m->h,
                  m->attn_acc, nq};
        {
            TimedScope t(m, K_GU);
            // staging loads go out before the weights, so one register buffer in
            // flight during staging is enough (1.5-2 % faster per decode step on
            // MI355X than two).  Small models: one block per CU, so each block
            // normalises the activation once for 2-3 row groups per wave
            // (0.5B: 0.881 -> 0.826 ms per token against as many blocks as fit)
            e = H <= 1024 ? stream_i8<2, 1, 8>(src, L.wgu, 2 * I, H, s, st, cus, 1)
                          : stream_i8<2, 4, 8>(src, L.wgu, 2 * I, H, s, st, cus);
        }
        // measurement repeats (myl_model_set_kernel_repeat), outside the timed
        // class: the same launch (same shape) over another layer's gate/up
        // weights, l + rep, wrapping to the first layers (read at least a
        // layer's traffic ago, so out of the caches as this layer's are),
        // into scratch rows
        for (int rep = 1; rep < m->gu_repeat && e == hipSuccess; ++rep) {
            const LayerDev& Lr = m->layers[(l + rep) % (int)m->spec.layers];
            EpiSilu sr = s;
            sr.shifts = Lr.sgu;
            sr.h = m->h_scratch;
            e = H <= 1024 ? stream_i8<2, 1, 8>(src, Lr.wgu, 2 * I, H, sr, st, cus, 1)
                          : stream_i8<2, 4, 8>(src, Lr.wgu, 2 * I, H, sr, st, cus);
        }
    }
    if (e != hipSuccess) return e;
    {
        TimedScope t(m, K_DOWN);
        SrcPlain src{m->h};
        EpiResid d{L.sd, f.down_in_frac, L.acc_mlp, L.res_mid, L.res_out, m->resid, m->hidden, m->norm_a, L.ref_out,
                   m->norm_b};
        e = stream_i8<1, 4, 8>(src, L.wd, H, I, d, st, cus);
    }
    return e;
}

// Final RMSNorm (staged from norm_a) + LM head + argmax (model.rs:264-308).
hipError_t head_step(myl_model* m) {
    hipStream_t st = m->ctx->stream;
    TimedScope t(m, K_HEAD);
    SrcNorm src{m->hidden, m->final_res, m->final_gamma, m->final_gamma_s, rms_params(m), m->ref_final,
                m->final_norm_frac, m->norm_a};
    if (m->spec.lm_head_int16) {
        EpiHead hd{m->lm16_shifts, m->final_norm_frac, m->logits, m->state};
        return stream_i16<2, 4, 8>(src, m->lm16, m->V, m->H, hd, st, m->cus);
    }
    EpiHead hd{m->lm8_shifts, m->final_norm_frac, m->logits, m->state};
    // a small model's row is a few 128-byte steps: eight rows per wave load
    // (K = 896, the 0.5B shape), two blocks per CU (one: 23.2 us, two: 22.2 us
    // for the 136 MB head on MI355X)
    if (m->H == 896) return stream_i8_rows8<7, 8>(src, m->lm8, m->V, m->H, hd, st, m->cus, 2);
    // other rows of one 1 KiB step: one-step batches, one block per CU
    if (m->H <= 1024) return stream_i8<2, 1, 8, true>(src, m->lm8, m->V, m->H, hd, st, m->cus, 1);
    return stream_i8<2, 4, 8, true>(src, m->lm8, m->V, m->H, hd, st, m->cus);
}

hipError_t embed_step(myl_model* m, int mode, int token, int pos, int64_t* tokens_dev) {
    TimedScope t(m, K_EMBED);
    embed_kernel<<<1, 1024, 0, m->ctx->stream>>>(m->state, mode, token, pos, m->rope_rows, m->V, m->emb, m->emb_shifts,
                                                  m->layers[0].res_in, m->layers[0].ref_in, m->H, tokens_dev, m->hidden,
                                                  m->norm_a, m->cos_lut, m->sin_lut, m->hd / 2, m->rope_cur);
    return hipGetLastError();
}

// The step's RoPE row for layers run from a host-supplied state.
int set_rope_cur(myl_model* m, int row) {
    const size_t half = (size_t)m->hd / 2;
    myl_ctx* c = m->ctx;
    int rc = c->hip(hipMemcpyAsync(m->rope_cur, m->cos_lut + (size_t)row * half, half * 2, hipMemcpyDeviceToDevice,
                                   c->stream), "rope row");
    if (rc) return rc;
    return c->hip(hipMemcpyAsync(m->rope_cur + half, m->sin_lut + (size_t)row * half, half * 2,
                                 hipMemcpyDeviceToDevice, c->stream), "rope row");
}

// The input-norm accumulator for a hidden vector supplied by the host.
hipError_t seed_norm(myl_model* m, const uint8_t* xs, uint8_t ref) {
    norm_seed_kernel<<<1, 1024, 0, m->ctx->stream>>>(m->hidden, xs, ref, m->H, m->norm_a);
    return hipGetLastError();
}

hipError_t full_step(myl_model* m, int mode, int token, int pos, int64_t* tokens_dev) {
    hipError_t e = embed_step(m, mode, token, pos, tokens_dev);
    for (int l = 0; e == hipSuccess && l < (int)m->spec.layers; ++l) e = layer_step(m, l);
    if (e == hipSuccess) e = head_step(m);
    return e;
}

// Captures one greedy step (mode 1: token and position come from the device
// state) as a graph; replays are valid for any position.
// Capture runs on the context's own stream (the caller's stream may be the
// legacy null stream, which cannot capture); the graph is later launched on
// whichever stream is active.
hipError_t capture_step(myl_model* m) {
    myl_ctx* c = m->ctx;
    if (m->step_exec) { (void)hipGraphExecDestroy(m->step_exec); m->step_exec = nullptr; }
    if (m->step_graph) { (void)hipGraphDestroy(m->step_graph); m->step_graph = nullptr; }
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return e;
    hipStream_t active = c->stream;
    c->stream = c->own_stream;
    e = hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) { c->stream = active; return e; }
    hipError_t le = full_step(m, 1, 0, 0, m->tokens_dev);
    e = hipStreamEndCapture(c->stream, &m->step_graph);
    c->stream = active;
    if (le != hipSuccess) return le;
    if (e != hipSuccess) return e;
    e = hipGraphInstantiate(&m->step_exec, m->step_graph, nullptr, nullptr, 0);
    if (e == hipSuccess) m->graph_tokens = m->tokens_dev;
    return e;
}

}  // namespace

namespace myl {

int model_setup(myl_ctx* ctx, const myl_synth_spec& s, bool tied, const myl_luts* luts, myl_model** out) {
    *out = nullptr;
    if (!s.hidden || !s.layers || !s.heads || !s.kv_heads || !s.head_dim || !s.inter || !s.vocab || !s.max_pos)
        return ctx->fail(MYL_E_INVALID, "model: every dimension must be > 0");
    if (s.heads % s.kv_heads || s.heads * s.head_dim != s.hidden)
        return ctx->fail(MYL_E_INVALID, "model: heads must divide evenly into KV heads and tile hidden");
    if (s.head_dim != 64 && s.head_dim != 128)
        return ctx->fail(MYL_E_UNSUPPORTED, "model: the fused decode path takes head_dim 64 or 128");
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
    m->tied = tied;
    m->H = (int)s.hidden;
    m->I = (int)s.inter;
    m->V = (int)s.vocab;
    m->hd = (int)s.head_dim;
    m->hd_log = ilog2_exact(m->hd);
    m->G = (int)(s.heads / s.kv_heads);
    m->nq = (int)(s.heads * s.head_dim);
    m->nkv = (int)(s.kv_heads * s.head_dim);
    m->max_pos = (int)s.max_pos;
    m->cus = ctx->prop.multiProcessorCount > 0 ? ctx->prop.multiProcessorCount : 1;
    int rc = alloc_impl(m, luts);
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return MYL_OK;
}

int model_finalize(myl_model* m) { return finalize_impl(m); }

}  // namespace myl

extern "C" {

int myl_model_set_kernel_repeat(myl_model* m, int kclass, int times) {
    if (!m || kclass != K_GU || times < 1 || times > 4) return MYL_E_INVALID;
    // each repeat streams another layer's weights; more repeats than layers
    // would re-read weights this step already brought into the caches
    if (times > (int)m->spec.layers)
        return m->ctx->fail(MYL_E_INVALID, "kernel repeat: more repeats than layers");
    (void)hipStreamSynchronize(m->ctx->stream);
    if (times > 1 && !m->h_scratch && !(m->h_scratch = m->dalloc<int16_t>(m->I)))
        return m->ctx->fail(MYL_E_NOMEM, "kernel repeat scratch");
    m->gu_repeat = times;
    // the captured step holds the launch sequence
    if (m->step_exec) { (void)hipGraphExecDestroy(m->step_exec); m->step_exec = nullptr; }
    if (m->step_graph) { (void)hipGraphDestroy(m->step_graph); m->step_graph = nullptr; }
    return MYL_OK;
}

int myl_model_set_graphs(myl_model* m, int enable) {
    if (!m) return MYL_E_INVALID;
    m->use_graphs = enable != 0;
    return MYL_OK;
}

int myl_model_timing(myl_model* m, int enable, double* ms_out, uint64_t* counts_out) {
    if (!m) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (enable) {
        m->timing = true;
        m->ev_used = 0;
        m->marks.clear();
        return MYL_OK;
    }
    int rc = c->hip(hipStreamSynchronize(c->stream), "timing");
    if (rc) return rc;
    std::vector<double> ms(K_COUNT, 0.0);
    std::vector<uint64_t> n(K_COUNT, 0);
    for (auto& mk : m->marks) {
        float t = 0.f;
        if (hipEventElapsedTime(&t, m->ev_pool[mk.second], m->ev_pool[mk.second + 1]) == hipSuccess) {
            ms[mk.first] += t;
            n[mk.first] += 1;
        }
    }
    m->timing = false;
    m->ev_used = 0;
    m->marks.clear();
    for (int k = 0; k < K_COUNT; ++k) {
        if (ms_out) ms_out[k] = ms[k];
        if (counts_out) counts_out[k] = n[k];
    }
    return MYL_OK;
}

int myl_model_create_synthetic(myl_ctx* ctx, const myl_synth_spec* spec, const myl_luts* luts, myl_model** out) {
    if (!ctx || !spec || !luts || !out) return MYL_E_INVALID;
    *out = nullptr;
    myl_model* m = nullptr;
    // The synthetic int8 head is the tied embedding (model.rs:297-307).
    int rc = myl::model_setup(ctx, *spec, /*tied=*/true, luts, &m);
    if (!rc) rc = synth_fill(m);
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
    if (int nr = m->not_ready()) return nr;
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
    if (int nr = m->not_ready()) return nr;
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
    const bool graphs = m->use_graphs && !m->timing && n_steps > 2;
    if (e == hipSuccess && graphs && (!m->step_exec || m->graph_tokens != m->tokens_dev)) e = capture_step(m);
    for (uint32_t i = 0; e == hipSuccess && i < n_steps; ++i) {
        if (logits_out)
            e = hipMemcpyAsync(logits_out + (size_t)i * m->V, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost,
                               c->stream);
        if (e == hipSuccess && i + 1 < n_steps)
            e = graphs ? hipGraphLaunch(m->step_exec, c->stream) : full_step(m, 1, 0, 0, m->tokens_dev);
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

int myl_model_prefill(myl_model* m, const uint32_t* tokens, uint32_t n, uint32_t pos0, int32_t* last_logits) {
    if (!m || (!tokens && n)) return MYL_E_INVALID;
    if (int nr = m->not_ready()) return nr;
    myl_ctx* c = m->ctx;
    if (n == 0) return MYL_OK;
    if ((uint64_t)pos0 + n > (uint64_t)m->max_pos) return c->fail(MYL_E_INVALID, "prefill: beyond the KV capacity");
    if (pos0 > m->n_cached) return c->fail(MYL_E_INVALID, "prefill: positions must be contiguous from 0");
    for (uint32_t i = 0; i < n; ++i)
        if (tokens[i] >= (uint32_t)m->V) return c->fail(MYL_E_INVALID, "prefill: token id out of range");
    // Long prompts run as one batch of rows over this cache (each row equals
    // forward_token at its position); short ones, or models the row path
    // cannot take, token by token as the reference's prompt loop does.
    int rc = MYL_E_UNSUPPORTED;
    if (n >= myl::kPromptRows) {
        rc = myl::prompt_rows(m, tokens, n, pos0);
        if (rc && rc != MYL_E_UNSUPPORTED) return rc;
    }
    if (rc == MYL_E_UNSUPPORTED) {
        hipError_t e = hipSuccess;
        for (uint32_t i = 0; e == hipSuccess && i < n; ++i) {
            e = embed_step(m, 0, (int)tokens[i], (int)(pos0 + i), nullptr);
            for (int l = 0; e == hipSuccess && l < (int)m->spec.layers; ++l) e = layer_step(m, l);
        }
        if (e == hipSuccess) e = head_step(m);
        rc = c->hip(e, "prefill");
        if (rc) return rc;
    }
    m->n_cached = std::max(m->n_cached, pos0 + n);
    if (last_logits) {
        rc = c->hip(hipMemcpyAsync(last_logits, m->logits, (size_t)m->V * 4, hipMemcpyDeviceToHost, c->stream), "logits");
        if (rc) return rc;
    }
    return c->hip(hipStreamSynchronize(c->stream), "prefill");
}

int myl_model_embed_token(myl_model* m, uint32_t token, int16_t* hidden) {
    if (!m || !hidden) return MYL_E_INVALID;
    if (int nr = m->not_ready()) return nr;
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
    if (int nr = m->not_ready()) return nr;
    myl_ctx* c = m->ctx;
    if (layer_end > m->spec.layers || layer_start > layer_end || pos >= (uint32_t)m->max_pos)
        return c->fail(MYL_E_INVALID, "run_layers: bad layer range or position");
    DecodeState s{};
    s.pos = (int32_t)pos;
    s.rope_row = (int32_t)(pos % m->rope_rows);
    int rc = c->hip(hipMemcpyAsync(m->state, &s, sizeof(s), hipMemcpyHostToDevice, c->stream), "state");
    if (rc) return rc;
    rc = set_rope_cur(m, s.rope_row);
    if (rc) return rc;
    rc = c->hip(hipMemcpyAsync(m->hidden, hidden, (size_t)m->H * 2, hipMemcpyHostToDevice, c->stream), "hidden");
    hipError_t e = hipSuccess;
    if (!rc && layer_start < layer_end) e = seed_norm(m, m->layers[layer_start].res_in, m->layers[layer_start].ref_in);
    for (uint32_t l = layer_start; !rc && e == hipSuccess && l < layer_end; ++l) e = layer_step(m, (int)l);
    if (!rc) rc = c->hip(e, "run_layers");
    if (rc) return rc;
    rc = c->hip(hipMemcpyAsync(hidden, m->hidden, (size_t)m->H * 2, hipMemcpyDeviceToHost, c->stream), "hidden");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "run_layers");
}

int myl_model_head_logits(myl_model* m, const int16_t* hidden, int32_t* logits) {
    if (!m || !hidden || !logits) return MYL_E_INVALID;
    if (int nr = m->not_ready()) return nr;
    myl_ctx* c = m->ctx;
    int rc = c->hip(hipMemcpyAsync(m->hidden, hidden, (size_t)m->H * 2, hipMemcpyHostToDevice, c->stream), "hidden");
    if (rc) return rc;
    rc = c->hip(seed_norm(m, m->final_res, m->ref_final), "head_logits");
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
