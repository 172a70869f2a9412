// batch.hip -- the batched forward of the device-resident model: R rows, each
// one (sequence, position, token), through all layers at once.
//
// The reference has no batching: prefill is a loop of forward_token calls
// (INTEGER_LLM/runtime/src/generate.rs:28-32) and each sequence owns a KV
// cache (runtime/src/kv_cache.rs).  Row r of a batch computes exactly what
// forward_token(token[r], pos[r]) computes on sequence seq[r]'s cache, because
// every op is per token except attention, and attention for position p reads
// only cached positions <= p (kv_cache.rs:43-52): the K/V rows of all rows of
// a batch are appended before any row attends.  One batch therefore serves
// teacher-forced prefill (many positions of few sequences, the projections on
// the int8 matrix cores) and batched decode (one position of many sequences).
//
// Per layer (model.rs:401-674):
//   rmsnorm          X -> Xn                                  (rmsnorm.rs:61-161)
//   q/k/v product    Xn -> QKV, requant + bias                (linear.rs:43-70,132-145)
//   rope_scatter     RoPE on q/k pairs, q -> Q, k/v -> caches (rope.rs:17-31, model.rs:458-503)
//   attention        scores, softmax statistics, P.V          (attention.rs:42-90, softmax.rs:12-64)
//   o_proj           A -> X2 with residual 1                  (model.rs:563-593)
//   rmsnorm          X2 -> Xn
//   gate/up product  Xn -> GU; SiLU gating GU -> Hh           (mlp.rs:28-65)
//   down_proj        Hh -> X with residual 2                  (mlp.rs:66-74, model.rs:612-671)
// then the final norm, the LM head over every row (model.rs:264-308) and a
// first-maximum argmax per row (sampling.rs:8-18).
#include "gemm_dispatch.h"
#include "gemm_frag.h"
#include "model_internal.h"
#include "ops.h"
#include "rows_attn.h"
#include "rows_dec.h"
#include "rows_epi.h"
#include "wave.h"

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

using namespace myl;

namespace myl {

struct BatchState {
    int n_seqs = 0;
    std::vector<uint32_t> len;           // cached positions per sequence
    int16_t* kc = nullptr;               // [seq][layer][kv_head][max_pos][head_dim]
    int16_t* vc = nullptr;
    bool owns_kv = true;                 // false: kc / vc are the model's single-sequence caches
    int head_rows = 0;                   // rows the logits buffer holds (0: every row)
    int rows_cap = 0, lmax_cap = 0;
    int32_t* rows = nullptr;             // [4][rows_cap]: seq, pos, rope row, token
    int16_t *X = nullptr, *Xn = nullptr, *X2 = nullptr, *QKV = nullptr, *Q = nullptr, *A = nullptr;
    int16_t *GU = nullptr, *Hh = nullptr;
    int32_t* logits = nullptr;           // [rows_cap][V]
    int64_t* argmax = nullptr;           // [rows_cap]
    int32_t* xsum = nullptr;             // [rows_cap] sums of the final-norm rows (int16 head product)
    uint64_t* argmax_part = nullptr;     // [rows_cap][ceil(V / kArgChunk)] best keys per chunk
    int64_t* tokens_out = nullptr;       // greedy chains: [steps][rows]
    size_t tokens_out_cap = 0;
    int32_t* scores = nullptr;           // [rows_cap][heads][lmax_cap]
    int16_t* probs = nullptr;            // [rows_cap][heads][lmax_cap] softmax probabilities (Q14)
    int64_t* part = nullptr;             // [lmax_cap / 256][rows_cap][nq]: exact P.V per position range
    AttnTile* tiles = nullptr;           // rows grouped by sequence for the attention kernels
    int ntiles = 0, tiles_cap = 0;
    int max_qv = 0;                      // largest query-vector count of a tile (rows x G)
    std::vector<void*> allocs_rows;      // row buffers (regrown together)
    std::vector<void*> allocs_scores;
};

void batch_free(BatchState* b) {
    if (!b) return;
    for (void* p : b->allocs_rows) (void)hipFree(p);
    for (void* p : b->allocs_scores) (void)hipFree(p);
    if (b->owns_kv && b->kc) (void)hipFree(b->kc);
    if (b->owns_kv && b->vc) (void)hipFree(b->vc);
    if (b->tokens_out) (void)hipFree(b->tokens_out);
    if (b->tiles) (void)hipFree(b->tiles);
    delete b;
}

}  // namespace myl

namespace {

// ---------------------------------------------------------------------------
// row kernels
// ---------------------------------------------------------------------------

// model.rs:241-248 per row.
__global__ __launch_bounds__(256) void embed_rows_kernel(const int32_t* __restrict__ tok, const int8_t* __restrict__ E,
                                                         const uint8_t* __restrict__ emb_shifts,
                                                         const uint8_t* __restrict__ res_frac0, int H,
                                                         int16_t* __restrict__ X) {
    const int r = blockIdx.x;
    const int t = tok[r];
    const int8_t* row = E + (size_t)t * H;
    const uint8_t sh = emb_shifts[t];
    for (int i = threadIdx.x; i < H; i += blockDim.x)
        X[(size_t)r * H + i] = clamp_i16(rescale32((int32_t)row[i], sh, res_frac0[i]));
}

// RoPE of the q/k pairs (rope.rs:17-31, LUT row pos % rows, model.rs:469-473),
// q to Q [R x nq] in head-major order, k (post-RoPE) and v to the sequence's
// cache at its position (model.rs:481-503).  Grid (ceil(pairs / 256), R).
__global__ __launch_bounds__(256) void rope_scatter_kernel(const int16_t* __restrict__ qkv, int ldq, const int32_t* __restrict__ rows,
                                                           int rows_cap, int nq, int nkv, int hd_log,
                                                           const int16_t* __restrict__ cos_lut,
                                                           const int16_t* __restrict__ sin_lut, int16_t* __restrict__ Q,
                                                           int16_t* __restrict__ kc, int16_t* __restrict__ vc,
                                                           size_t seq_stride, int kvh, int max_pos);

// RoPE of a q/k pair (rope.rs:17-31) and its destination: q to Q in
// head-major order, k (post-RoPE) and v to the sequence's cache at the row's
// position (model.rs:469-503), for row r at sequence seq and position pos
// with the pair's cos / sin entries c, s (used for q and k).
__device__ inline void rope_store_pair_at(int r, int n0, int16_t y0, int16_t y1, int seq, int pos, int32_t c,
                                          int32_t s, int nq, int nkv, int hd_log, int16_t* __restrict__ Q,
                                          int16_t* __restrict__ kc, int16_t* __restrict__ vc, size_t seq_stride,
                                          int max_pos) {
    const int seg = n0 < nq ? 0 : (n0 < nq + nkv ? 1 : 2);
    const int e = n0 - (seg == 0 ? 0 : (seg == 1 ? nq : nq + nkv));
    const int hd = 1 << hd_log, half = hd >> 1;
    const int head = e >> hd_log;
    const int p = (e & (hd - 1)) >> 1;
    if (seg < 2) {
        const int32_t x0 = y0, x1 = y1;
        y0 = clamp_i16(rshift_round32(wsub32(wmul32(x0, c), wmul32(x1, s)), MYL_TV_ROPE_FRAC_BITS));
        y1 = clamp_i16(rshift_round32(wadd32(wmul32(x1, c), wmul32(x0, s)), MYL_TV_ROPE_FRAC_BITS));
    }
    int16_t* dst;
    if (seg == 0) dst = Q + (size_t)r * nq + (size_t)head * hd;
    else dst = (seg == 1 ? kc : vc) + (size_t)seq * seq_stride + ((size_t)head * max_pos + pos) * hd;
    dst[p] = y0;
    dst[p + half] = y1;
}

// The pair's cos / sin entries for RoPE row rope_row (zero for v rows).
__device__ inline void rope_cs(int n0, int rope_row, int nq, int nkv, int hd_log, const int16_t* __restrict__ cos_lut,
                               const int16_t* __restrict__ sin_lut, int32_t& c, int32_t& s) {
    c = s = 0;
    if (n0 >= nq + nkv) return;
    const int e = n0 - (n0 < nq ? 0 : nq);
    const int half = (1 << hd_log) >> 1, p = (e & ((1 << hd_log) - 1)) >> 1;
    c = cos_lut[(size_t)rope_row * half + p];
    s = sin_lut[(size_t)rope_row * half + p];
}

// rope_store_pair_at with the row's sequence, position and RoPE row read
// from the row table.  Shared by rope_scatter_kernel and the fused finish of
// a split q/k/v product.
__device__ inline void rope_store_pair(int r, int n0, int16_t y0, int16_t y1, const int32_t* __restrict__ rows,
                                       int rows_cap, int nq, int nkv, int hd_log, const int16_t* __restrict__ cos_lut,
                                       const int16_t* __restrict__ sin_lut, int16_t* __restrict__ Q,
                                       int16_t* __restrict__ kc, int16_t* __restrict__ vc, size_t seq_stride,
                                       int max_pos) {
    const int seq = rows[r], pos = rows[rows_cap + r], rope_row = rows[2 * rows_cap + r];
    int32_t c, s;
    rope_cs(n0, rope_row, nq, nkv, hd_log, cos_lut, sin_lut, c, s);
    rope_store_pair_at(r, n0, y0, y1, seq, pos, c, s, nq, nkv, hd_log, Q, kc, vc, seq_stride, max_pos);
}

// The q/k/v product's epilogue on the fragment-major weights (gemm_frag.h):
// requantise with the bias (EpiQKVRows), rotate q/k pairs and store q and
// the KV append (rope_store_pair).  Threads take the block's 8 ngb pair
// columns (FragCols); the pair's operands are fetched before the stream.
struct FragOutQKV {
    EpiQKVRows epi;
    const int32_t* rows;
    int rows_cap, nq, nkv, hd_log;
    const int16_t *cos_lut, *sin_lut;
    int16_t *Q, *kc, *vc;
    size_t seq_stride;
    int max_pos;
    // the pair's operands, and the seq / position / cos / sin of the thread's
    // first row (the only one while 8 ngb x R <= 512)
    struct Pre {
        EpiQKVRows::ValOps o0, o1;
        int seq, pos;
        int32_t c, s;
    };
    __device__ inline Pre pre(int g0, int ngb, int R, int N) const {
        const FragCols fc = FragCols::of(8 * ngb);
        const int n0 = min(16 * g0 + 2 * fc.col(), N - 2);
        const int m = min(fc.row0(), R - 1);
        Pre q{epi.val_ops(n0), epi.val_ops(n0 + 1), rows[m], rows[rows_cap + m], 0, 0};
        rope_cs(n0, rows[2 * rows_cap + m], nq, nkv, hd_log, cos_lut, sin_lut, q.c, q.s);
        return q;
    }
    template <int RT>
    __device__ inline void run(const Pre& pr, const FragSums<RT>& s, int g0, int ngb, int R, int N, int8_t*) const {
        const int np = 8 * ngb;
        const FragCols fc = FragCols::of(np);
        const int c2 = fc.col(), gg = c2 >> 3, cc = 2 * (c2 & 7);
        const int n0 = 16 * (g0 + gg) + cc;
        if (c2 >= np || n0 >= N) return;
        for (int m = fc.row0(); m < R; m += fc.slices) {
            const int16_t y0 = epi.value_with(pr.o0, n0, s(gg, m, cc));
            const int16_t y1 = epi.value_with(pr.o1, n0 + 1, s(gg, m, cc + 1));
            if (m == fc.row0())
                rope_store_pair_at(m, n0, y0, y1, pr.seq, pr.pos, pr.c, pr.s, nq, nkv, hd_log, Q, kc, vc, seq_stride,
                                   max_pos);
            else
                rope_store_pair(m, n0, y0, y1, rows, rows_cap, nq, nkv, hd_log, cos_lut, sin_lut, Q, kc, vc,
                                seq_stride, max_pos);
        }
    }
};

__global__ __launch_bounds__(256) void rope_scatter_kernel(const int16_t* __restrict__ qkv, int ldq, const int32_t* __restrict__ rows,
                                                           int rows_cap, int nq, int nkv, int hd_log,
                                                           const int16_t* __restrict__ cos_lut,
                                                           const int16_t* __restrict__ sin_lut, int16_t* __restrict__ Q,
                                                           int16_t* __restrict__ kc, int16_t* __restrict__ vc,
                                                           size_t seq_stride, int kvh, int max_pos) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    const int npairs = (nq + 2 * nkv) >> 1;
    if (i >= npairs) return;
    const int n0 = 2 * i;
    rope_store_pair(r, n0, qkv[(size_t)r * ldq + n0], qkv[(size_t)r * ldq + n0 + 1], rows, rows_cap, nq, nkv, hd_log,
                    cos_lut, sin_lut, Q, kc, vc, seq_stride, max_pos);
}

// The finish of a split q/k/v product fused with rope_scatter_kernel's work:
// thread (pair i, row r) takes the pair's two exact sums out of the split-K
// accumulator (clearing them), requantises them with the bias (EpiQKVRows),
// rotates q/k pairs and writes q to Q and k, v to the sequence's cache.  The
// q/k/v rows are pair-ordered, so the pair is outputs 2i, 2i + 1.  Grid
// (ceil(pairs / 256), R).
__global__ __launch_bounds__(256) void qkv_finish_rope_kernel(unsigned long long* __restrict__ acc, int N, EpiQKVRows epi,
                                                              const int32_t* __restrict__ rows, int rows_cap, int nq,
                                                              int nkv, int hd_log, const int16_t* __restrict__ cos_lut,
                                                              const int16_t* __restrict__ sin_lut,
                                                              int16_t* __restrict__ Q, int16_t* __restrict__ kc,
                                                              int16_t* __restrict__ vc, size_t seq_stride, int max_pos) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (N >> 1)) return;
    const int n0 = 2 * i;
    unsigned long long* a = acc + (size_t)r * N + n0;
    const int64_t a0 = (int64_t)a[0], a1 = (int64_t)a[1];
    const int16_t y0 = epi.value(n0, a0), y1 = epi.value(n0 + 1, a1);
    a[0] = 0;
    a[1] = 0;
    rope_store_pair(r, n0, y0, y1, rows, rows_cap, nq, nkv, hd_log, cos_lut, sin_lut, Q, kc, vc, seq_stride, max_pos);
}

// softmax.rs:12-64 for one (row, head) over its L scores: m = max, S =
// wrapping i32 sum of the exp LUT values, then every probability
// p_j = RNE(e_j 2^14 / S) (or the uniform split when S == 0) as an int16
// into probs[row][head][j], j < L (the rest of the last 4-position group gets
// 0; later positions are not written, and their readers mask them).
// W waves per (row, head) (pair = row * heads + head), 4 / W pairs per
// 256-thread block; a thread takes 4 positions of each chunk of 256 W.
// Rows of up to 1024 (W = 1) or 4096 (W = 4) positions keep their scores,
// then their exp values, in registers; longer ones read the scores three times.
template <int W>
__global__ __launch_bounds__(256) void rows_probs_kernel(const int32_t* __restrict__ rows, int rows_cap,
                                                         const int32_t* __restrict__ scores, Divider heads, int lcap,
                                                         int npairs, const int16_t* __restrict__ lut, uint32_t lut_len,
                                                         uint8_t lut_shift, int16_t* __restrict__ probs) {
    static_assert(W == 1 || W == 4, "waves per pair");
    constexpr int CW = 256 * W;      // positions per chunk
    constexpr int KPER = 4;  // register-resident chunks (1024 / 4096 positions; 38 VGPRs, 8 waves per SIMD at W = 1)
    __shared__ int32_t redm[4];
    __shared__ uint32_t reds[4];
    const int t = W == 1 ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
    const int pair = W == 1 ? (int)(blockIdx.x * 4 + (threadIdx.x >> 6)) : (int)blockIdx.x;
    if (pair >= npairs) return;  // uniform over the pair's waves: every reduction sees all of them
    uint32_t row, head;
    heads.divmod((uint32_t)pair, row, head);
    const int L = rows[rows_cap + (int)row] + 1;
    const size_t o = (size_t)pair * lcap;
    const int32_t* z = scores + o;
    int16_t* pr = probs + o;
    const int32_t lut_one = lut_len > 0 ? (int32_t)lut[0] : 1;
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    const int nc = (L + CW - 1) / CW;
    const bool regs = nc <= KPER;
    int32_t e[KPER][4];
    int32_t mx = INT32_MIN;
    if (regs) {
#pragma unroll
        for (int c = 0; c < KPER; ++c) {
            const int jb = c * CW + 4 * t;
            int4 v = make_int4(INT32_MIN, INT32_MIN, INT32_MIN, INT32_MIN);
            if (c < nc && jb < L) v = *reinterpret_cast<const int4*>(z + jb);  // jb + 3 < lcap
            e[c][0] = jb < L ? v.x : INT32_MIN;
            e[c][1] = jb + 1 < L ? v.y : INT32_MIN;
            e[c][2] = jb + 2 < L ? v.z : INT32_MIN;
            e[c][3] = jb + 3 < L ? v.w : INT32_MIN;
#pragma unroll
            for (int k = 0; k < 4; ++k) mx = max(mx, e[c][k]);
        }
    } else {
        for (int jb = 4 * t; jb < L; jb += CW) {
            const int4 v = *reinterpret_cast<const int4*>(z + jb);
            const int32_t zz[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (jb + k < L) mx = max(mx, zz[k]);
        }
    }
    mx = W == 1 ? wave_max_i32(mx) : block_max_i32_dpp(mx, redm);
    uint32_t s = 0;
    if (regs) {
#pragma unroll
        for (int c = 0; c < KPER; ++c) {
            const int jb = c * CW + 4 * t;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                e[c][k] = jb + k < L ? exp_lookup(sat_sub32(mx, e[c][k]), lut, lut_len, lut_shift, lut_one) : 0;
                s += (uint32_t)e[c][k];
            }
        }
    } else {
        for (int jb = 4 * t; jb < L; jb += CW) {
            const int4 v = *reinterpret_cast<const int4*>(z + jb);
            const int32_t zz[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int k = 0; k < 4; ++k)
                if (jb + k < L) s += (uint32_t)exp_lookup(sat_sub32(mx, zz[k]), lut, lut_len, lut_shift, lut_one);
        }
    }
    const int32_t S = W == 1 ? wave_sum_i32((int32_t)s) : (int32_t)block_sum_u32_dpp(s, reds);
    int32_t ub = 0, ur = 0;
    uint32_t r32 = 0;
    uint64_t recip = 0;
    if (S > 0) {
        r32 = recip32_u32((uint32_t)S);
    } else if (S < 0) {
        recip = recip32(0u - (uint32_t)S);  // a wrapped sum
    } else {  // the uniform split (softmax.rs:42-48)
        uint32_t qq, rr;
        udivmod32((uint32_t)one, (uint32_t)L, recip32((uint32_t)L), &qq, &rr);
        ub = (int32_t)qq;
        ur = wsub32(one, wmul32((int32_t)qq, L));
    }
    auto emit = [&](int jb, const int32_t (&ev)[4]) {
        uint32_t pw[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int j = jb + k;
            int32_t p = 0;
            if (j < L) {
                if (S == 0) p = ub + (((uint64_t)j < (uint64_t)(int64_t)ur) ? 1 : 0);
                else if (S > 0) p = softmax_div_round_pos(wmul32(ev[k], one), S, r32);
                else p = softmax_div_round(wmul32(ev[k], one), S, recip);
            }
            pw[k] = (uint32_t)p & 0xFFFFu;
        }
        *reinterpret_cast<uint2*>(pr + jb) = make_uint2(pw[0] | (pw[1] << 16), pw[2] | (pw[3] << 16));
    };
    if (regs) {
#pragma unroll
        for (int c = 0; c < KPER; ++c)
            if (c < nc && c * CW + 4 * t < L) emit(c * CW + 4 * t, e[c]);
        return;
    }
    for (int jb = 4 * t; jb < L; jb += CW) {
        const int4 v = *reinterpret_cast<const int4*>(z + jb);
        const int32_t zz[4] = {v.x, v.y, v.z, v.w};
        int32_t ev[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            ev[k] = jb + k < L ? exp_lookup(sat_sub32(mx, zz[k]), lut, lut_len, lut_shift, lut_one) : 0;
        emit(jb, ev);
    }
}

// mlp.rs:55-65 per row: h = clamp(rescale(silu(g) * u, 8 + up_frac, down_in_frac)).
__global__ __launch_bounds__(256) void silu_rows_kernel(const int16_t* __restrict__ GU, int I,
                                                        const int16_t* __restrict__ silu, uint32_t silu_len,
                                                        uint8_t gate_frac, uint8_t up_frac, uint8_t down_in_frac,
                                                        int16_t* __restrict__ Hh) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= I) return;
    const uint32_t gu = *reinterpret_cast<const uint32_t*>(GU + (size_t)r * 2 * I + 2 * i);
    Hh[(size_t)r * I + i] = (int16_t)silu_mul((int16_t)(gu & 0xFFFFu), (int16_t)(gu >> 16), silu, silu_len, gate_frac,
                                              up_frac, down_in_frac);
}

// silu_rows_kernel writing byte planes [2R x I] of h for the down product.
__global__ __launch_bounds__(256) void silu_planes_kernel(const int16_t* __restrict__ GU, int I,
                                                          const int16_t* __restrict__ silu, uint32_t silu_len,
                                                          uint8_t gate_frac, uint8_t up_frac, uint8_t down_in_frac,
                                                          int8_t* __restrict__ planes) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= I) return;
    const uint32_t gu = *reinterpret_cast<const uint32_t*>(GU + (size_t)r * 2 * I + 2 * i);
    const int32_t h = silu_mul((int16_t)(gu & 0xFFFFu), (int16_t)(gu >> 16), silu, silu_len, gate_frac, up_frac,
                               down_in_frac);
    planes[(size_t)(2 * r) * I + i] = (int8_t)(h >> 8);
    planes[(size_t)(2 * r + 1) * I + i] = (int8_t)((h & 255) - 128);
}

// The finish of a split residual product fused with the next RMSNorm
// (rmsnorm.rs:61-161): one block per row m takes the row's exact sums out of
// the split-K accumulator (clearing them), applies the residual epilogue
// (storing the new residual row) and normalises that row into the next
// product's byte planes [2M x N].  1024 threads, PER = ceil(N / 1024).
constexpr int kFinNormThreads = 1024;
template <int PER>
__global__ __launch_bounds__(kFinNormThreads) void finish_resid_norm_kernel(unsigned long long* __restrict__ acc, int N,
                                                                EpiResidRows epi, const uint8_t* __restrict__ xs,
                                                                uint8_t ref, const int8_t* __restrict__ g,
                                                                const uint8_t* __restrict__ gs, RmsParams p,
                                                                uint8_t out_frac, int8_t* __restrict__ planes) {
    __shared__ uint64_t red[kFinNormThreads / 64][3];
    __shared__ RmsFactor sf;
    const int m = blockIdx.x;
    int16_t xv[PER];
    uint8_t sv[PER], gsv[PER];
    int8_t gv[PER];
    // every load of the thread's elements first, then the arithmetic, then
    // the stores (the output row and the accumulator's clearing): one memory
    // latency instead of one per element (6 -> 1.x us on MI355X)
    int64_t av[PER];
    EpiResidRows::FinOps op[PER];
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int n = min((int)threadIdx.x + t * kFinNormThreads, N - 1);  // lanes past N load a valid element, unused
        av[t] = (int64_t)acc[(size_t)m * N + n];
        op[t] = epi.fin_ops(n, m);
        sv[t] = xs[n];
        gv[t] = g[n];
        gsv[t] = gs[n];
    }
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int n = threadIdx.x + t * kFinNormThreads;
        xv[t] = 0;
        if (n < N) {
            xv[t] = epi.value_of(av[t], op[t]);
        } else {
            sv[t] = gsv[t] = 0;
            gv[t] = 0;
        }
    }
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int n = threadIdx.x + t * kFinNormThreads;
        if (n < N) {
            epi.out[(size_t)m * epi.ldo + n] = xv[t];
            acc[(size_t)m * N + n] = 0;
        }
    }
    const RmsFactor f = rms_factor_limbs<PER>(xv, sv, ref, p, red, &sf);
    int8_t* ph = planes + (size_t)(2 * m) * N;
#pragma unroll
    for (int t = 0; t < PER; ++t) {
        const int n = threadIdx.x + t * kFinNormThreads;
        if (n < N) {
            const int32_t y = rms_out(xv[t], sv[t], gv[t], gsv[t], f, out_frac);
            ph[n] = (int8_t)(y >> 8);
            ph[N + n] = (int8_t)((y & 255) - 128);
        }
    }
}

// A residual product (o_proj, down) of R rows followed by the RMSNorm of its
// output rows into planes: fused into the finish of a split product,
// otherwise the product then rmsnorm_planes.  ref is the largest entry of
// the norm's input scales xs (rmsnorm.rs:96).
hipError_t resid_then_norm(const int8_t* Ap, int R, const int8_t* W, int N, int K, const EpiResidRows& epi,
                           const MmCtx* mm, const uint8_t* xs, uint8_t ref, const int8_t* g, const uint8_t* gs,
                           const myl_model* m, uint8_t out_frac, int8_t* planes, hipStream_t st,
                           const int8_t* Wf = nullptr) {
    const RmsParams p{m->rsqrt, m->rsqrt_len, MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20,
                      m->rsqrt_closed};
    auto fin = [&](unsigned long long* acc, hipStream_t s) -> hipError_t {
        if (N <= kFinNormThreads)
            finish_resid_norm_kernel<1><<<R, kFinNormThreads, 0, s>>>(acc, N, epi, xs, ref, g, gs, p, out_frac, planes);
        else
            finish_resid_norm_kernel<4><<<R, kFinNormThreads, 0, s>>>(acc, N, epi, xs, ref, g, gs, p, out_frac, planes);
        return hipGetLastError();
    };
    // fragment-major weights: the K-sliced product into the accumulator, then the same finish
    if (Wf && N <= 4096 && frag_split_ok(R, K, N, mm->cus, mm->acc_elems)) {
        hipError_t e = frag_mm_split(Ap, R, K, Wf, N, mm->acc, mm->cus, mm->acc_elems, st);
        return e != hipSuccess ? e : fin(mm->acc, st);
    }
    bool split = false;
    hipError_t e = N <= 4096 ? mm_planes_fin(Ap, R, W, N, K, epi, mm, st, fin, &split) : mm_planes(Ap, R, W, N, K, epi, mm, st);
    if (e != hipSuccess || split) return e;
    return rmsnorm_planes(epi.out, R, epi.ldo, xs, g, gs, N, m->rsqrt, m->rsqrt_len, MYL_TV_RSQRT_INPUT_SHIFT,
                          MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, out_frac, planes, st);
}

// Greedy continuation: row r's next token is its argmax; positions advance.
__global__ void rows_advance_kernel(int32_t* __restrict__ rows, int rows_cap, int R, const int64_t* __restrict__ am,
                                    uint32_t rope_rows, int64_t* __restrict__ tokens_out) {
    const int r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= R) return;
    const int64_t t = am[r];
    rows[3 * rows_cap + r] = (int32_t)t;
    tokens_out[r] = t;
    const int pos = rows[rows_cap + r] + 1;
    rows[rows_cap + r] = pos;
    rows[2 * rows_cap + r] = (int32_t)umod32_slow((uint32_t)pos, rope_rows);
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

template <class T>
T* balloc(std::vector<void*>& list, size_t count) {
    void* p = nullptr;
    if (hipMalloc(&p, count * sizeof(T) ? count * sizeof(T) : 1) != hipSuccess) return nullptr;
    list.push_back(p);
    return (T*)p;
}

size_t seq_stride(const myl_model* m) {
    return (size_t)m->spec.layers * m->spec.kv_heads * (size_t)m->max_pos * m->hd;
}

int ensure_rows(myl_model* m, BatchState* b, int R) {
    if (R <= b->rows_cap) return MYL_OK;
    myl_ctx* c = m->ctx;
    (void)hipStreamSynchronize(c->stream);
    for (void* p : b->allocs_rows) (void)hipFree(p);
    b->allocs_rows.clear();
    b->rows_cap = 0;
    const size_t H = m->H, I = m->I, V = m->V, nq = m->nq, nqkv = m->nq + 2 * m->nkv;
    auto& L = b->allocs_rows;
    b->rows = balloc<int32_t>(L, 4 * (size_t)R);
    b->X = balloc<int16_t>(L, R * H);
    b->Xn = balloc<int16_t>(L, R * H);
    b->X2 = balloc<int16_t>(L, R * H);
    b->QKV = balloc<int16_t>(L, R * nqkv);
    b->Q = balloc<int16_t>(L, R * nq);
    b->A = balloc<int16_t>(L, R * nq);
    b->GU = balloc<int16_t>(L, R * 2 * I);
    b->Hh = balloc<int16_t>(L, R * I);
    b->logits = balloc<int32_t>(L, (b->head_rows > 0 ? std::min<size_t>(R, b->head_rows) : R) * V);
    b->argmax = balloc<int64_t>(L, R);
    b->xsum = balloc<int32_t>(L, R);
    b->argmax_part = balloc<uint64_t>(L, (size_t)R * ((V + kArgChunk - 1) / kArgChunk));
    for (void* p : L)
        if (!p) return c->fail(MYL_E_NOMEM, "batch: row buffer allocation");
    b->rows_cap = R;
    b->lmax_cap = 0;  // scores are sized by rows too
    return MYL_OK;
}

int ensure_scores(myl_model* m, BatchState* b, int lmax) {
    if (lmax <= b->lmax_cap) return MYL_OK;
    myl_ctx* c = m->ctx;
    (void)hipStreamSynchronize(c->stream);
    for (void* p : b->allocs_scores) (void)hipFree(p);
    b->allocs_scores.clear();
    b->lmax_cap = 0;
    const int cap = ((lmax + kAttnRange - 1) / kAttnRange) * kAttnRange;
    b->scores = balloc<int32_t>(b->allocs_scores, (size_t)b->rows_cap * m->spec.heads * cap);
    b->probs = balloc<int16_t>(b->allocs_scores, (size_t)b->rows_cap * m->spec.heads * cap);
    b->part = balloc<int64_t>(b->allocs_scores, (size_t)(cap / kAttnRange) * b->rows_cap * m->nq);
    if (!b->scores || !b->probs || !b->part) return c->fail(MYL_E_NOMEM, "batch: score buffer allocation");
    b->lmax_cap = cap;
    return MYL_OK;
}

// The decode-batch attention kernels (rows_dec.h) for the query-head group
// sizes they are built for.
constexpr bool rows_dec_ok(int hd, int G) { return (hd == 64 || hd == 128) && (G == 4 || G == 7 || G == 8); }

template <int HD>
hipError_t rows_dec_qk(int G, dim3 grid, hipStream_t st, const int32_t* rows, int rows_cap, const int16_t* Q, int nq,
                       const int16_t* kc, size_t sstride, int max_pos, int64_t mult, uint8_t shift, int32_t* scores,
                       int heads, int lcap) {
#define MYL_DEC_QK(GV)                                                                                              \
    rows_dec_qk_kernel<HD, GV><<<grid, 256, 0, st>>>(rows, rows_cap, Q, nq, kc, sstride, max_pos, mult, shift, scores, \
                                                     heads, lcap)
    switch (G) {
        case 4: MYL_DEC_QK(4); break;
        case 7: MYL_DEC_QK(7); break;
        case 8: MYL_DEC_QK(8); break;
        default: return hipErrorInvalidValue;
    }
#undef MYL_DEC_QK
    return hipGetLastError();
}

template <int HD>
hipError_t rows_dec_pv(int G, dim3 grid, hipStream_t st, const int32_t* rows, int rows_cap, const int16_t* probs,
                       int heads, int lcap, const int16_t* vc, size_t sstride, int max_pos, int64_t* part,
                       size_t part_stride, int nq) {
#define MYL_DEC_PV(GV)                                                                                              \
    rows_dec_pv_kernel<HD, GV><<<grid, 256, 0, st>>>(rows, rows_cap, probs, heads, lcap, vc, sstride, max_pos, part, \
                                                     part_stride, nq)
    switch (G) {
        case 4: MYL_DEC_PV(4); break;
        case 7: MYL_DEC_PV(7); break;
        case 8: MYL_DEC_PV(8); break;
        default: return hipErrorInvalidValue;
    }
#undef MYL_DEC_PV
    return hipGetLastError();
}

// One batched forward over the rows already uploaded to b->rows; lmax is the
// largest position + 1 among them.  The final norm and LM head run over rows
// [h0, R) only, into logits_out [(R - h0) x V] and argmax_out [R - h0].
// Whether the decode-batch products of R rows take the fragment-major q/k/v,
// gate/up and down weights (gemm_frag.h): by default for up to 32 rows when the
// gate/up K (the hidden size) is at least 3 KiB, where they stream the
// weights faster than the tiled products (B = 8 / 32 at the 7B shape on
// MI355X: gate/up 30.4 -> 24.1 us and 50.4 -> 32.4 us with its SiLU, down
// 16.9 -> 14.3 us and 26.3 -> 21.9 us).  MYL_BATCH_FRAG=1 takes them for every
// shape they support, 0 never.  The copies are built on first use (one
// relayout per layer on the stream); false when they cannot be (shapes or
// memory), and the tiled products run.
bool frag_ready(myl_model* m, int R, const MmCtx* mm, hipStream_t st) {
    const char* env = std::getenv("MYL_BATCH_FRAG");
    const int mode = env && *env ? std::atoi(env) : -1;
    if (mode == 0 || m->frag_state < 0 || !mm || R < 2 || R > kFragMaxRows) return false;
    const int H = m->H, I = m->I;
    if (mode < 0 && H < 3072) return false;
    const int nqkv = m->nq + 2 * m->nkv;
    if (!frag_full_ok(R, H, 2 * I, mm->cus) || !frag_split_ok(R, I, H, mm->cus, mm->acc_elems) ||
        !frag_full_ok(R, H, nqkv, mm->cus))
        return false;
    if (m->frag_state == 1) return true;
    for (LayerDev& L : m->layers) {
        if (!L.wqkv_f) L.wqkv_f = m->dalloc<int8_t>(frag_bytes(nqkv, H));
        if (!L.wgu_f) L.wgu_f = m->dalloc<int8_t>(frag_bytes(2 * I, H));
        if (!L.wd_f) L.wd_f = m->dalloc<int8_t>(frag_bytes(H, I));
        if (!L.wqkv_f || !L.wgu_f || !L.wd_f) {
            m->frag_state = -1;
            return false;
        }
        if (frag_relayout(L.wqkv, nqkv, H, L.wqkv_f, st) != hipSuccess ||
            frag_relayout(L.wgu, 2 * I, H, L.wgu_f, st) != hipSuccess || frag_relayout(L.wd, H, I, L.wd_f, st) != hipSuccess) {
            m->frag_state = -1;
            return false;
        }
    }
    m->frag_state = 1;
    return true;
}

hipError_t forward_rows(myl_model* m, BatchState* b, int R, int lmax, int h0, int32_t* logits_out,
                        int64_t* argmax_out) {
    myl_ctx* c = m->ctx;
    hipStream_t st = c->stream;
    const int H = m->H, I = m->I, V = m->V, nq = m->nq, nkv = m->nkv, hd = m->hd, G = m->G;
    const int nqkv = nq + 2 * nkv, heads = (int)m->spec.heads, kvh = (int)m->spec.kv_heads;
    // planes: [2R x max(I, H)] for every product, plus [2R x H] after the
    // first 2R x I bytes for the gate/up input when the SiLU is fused
    const size_t plane_req = R < 2 ? 0 : (size_t)2 * R * ((size_t)I + H);
    const MmCtx* mm = c->mm_ctx((size_t)R * std::max(2 * I, nqkv), plane_req);
    const size_t sstride = seq_stride(m);
    const int ranges = (lmax + kAttnRange - 1) / kAttnRange;
    // producers write the products' byte planes directly when every product
    // of the layer runs on planes
    const bool planes = mm_planes_ok(R, H, mm) && mm_planes_ok(R, I, mm) && mm_planes_ok(R, nq, mm) &&
                        rmsnorm_planes_ok(H) && xvec_ok(b->X, H);
    // the gate/up product applies the SiLU and writes the down product's
    // planes itself (staged epilogue) when its tiles need no K split
    // (17-64 rows: the split gate/up product with its own finish and SiLU
    // measured faster on MI355X than the unsplit fused one)
    const bool frag = planes && frag_ready(m, R, mm, st);
    const bool fuse_silu = planes && I % 8 == 0 && (R > 64 || (R <= 16 && H % 128 == 0) || frag) &&
                           (size_t)2 * R * ((size_t)I + H) <= mm->planes_bytes;
    int8_t* const xin = mm && mm->planes ? mm->planes + (size_t)2 * R * I : nullptr;  // gate/up input planes
    const uint8_t lut_shift = MYL_TV_SCORE_FRAC_BITS - MYL_TV_EXP_INPUT_FRAC;
    hipError_t e;
    embed_rows_kernel<<<R, 256, 0, st>>>(b->rows + 3 * b->rows_cap, m->emb, m->emb_shifts, m->layers[0].res_in, H, b->X);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    // Each residual product's split-K finish also normalises its rows into
    // the next product's planes (resid_then_norm; without a split, the
    // product then rmsnorm_planes).
    const bool norm_in_finish = planes;
    bool in_normed = false;  // this layer's input planes were written by the previous down product
    for (int l = 0; l < (int)m->spec.layers; ++l) {
        const LayerDev& Ld = m->layers[l];
        const myl_layer_fracs& f = Ld.f;
        bool qkv_roped = false;  // the q/k/v finish did RoPE and the KV append
        EpiQKVRows eq{};
        eq.shifts = Ld.sqkv; eq.bias = Ld.bqkv; eq.bias_sh = Ld.bsqkv;
        eq.act_frac = f.norm_attn_frac; eq.q_frac = f.q_frac; eq.k_frac = f.k_frac; eq.v_frac = f.v_frac;
        eq.nq = nq; eq.nkv = nkv; eq.out = b->QKV; eq.ldo = nqkv;
        if (planes) {
            if (!in_normed &&
                (e = rmsnorm_planes(b->X, R, H, Ld.res_in, Ld.in_gamma, Ld.in_gamma_s, H, m->rsqrt, m->rsqrt_len,
                                    MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, f.norm_attn_frac,
                                    mm->planes, st)) != hipSuccess)
                return e;
            if (frag) {
                // fragment-major weights: RoPE and the KV append in the product's epilogue
                const FragOutQKV oq{eq, b->rows, b->rows_cap, nq, nkv, m->hd_log, m->cos_lut, m->sin_lut, b->Q,
                                    b->kc + (size_t)l * kvh * m->max_pos * hd,
                                    b->vc + (size_t)l * kvh * m->max_pos * hd, sstride, m->max_pos};
                if ((e = frag_mm_full(mm->planes, R, H, Ld.wqkv_f, nqkv, oq, false, mm->cus, st)) != hipSuccess) return e;
                qkv_roped = true;
            }
            // a split product finishes with RoPE and the KV append fused in
            auto fin = [&](unsigned long long* acc, hipStream_t s) -> hipError_t {
                qkv_finish_rope_kernel<<<dim3((nqkv / 2 + 255) / 256, R), 256, 0, s>>>(
                    acc, nqkv, eq, b->rows, b->rows_cap, nq, nkv, m->hd_log, m->cos_lut, m->sin_lut, b->Q,
                    b->kc + (size_t)l * kvh * m->max_pos * hd, b->vc + (size_t)l * kvh * m->max_pos * hd, sstride,
                    m->max_pos);
                return hipGetLastError();
            };
            if (!frag && (e = mm_planes_fin(mm->planes, R, Ld.wqkv, nqkv, H, eq, mm, st, fin, &qkv_roped)) != hipSuccess)
                return e;
        } else {
            if ((e = rmsnorm(b->X, R, H, Ld.res_in, Ld.in_gamma, Ld.in_gamma_s, H, m->rsqrt, m->rsqrt_len,
                             MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, f.norm_attn_frac, b->Xn,
                             H, st)) != hipSuccess ||
                (e = gemv_i8(b->Xn, R, H, Ld.wqkv, nqkv, H, eq, st, mm)) != hipSuccess)
                return e;
        }
        int16_t* kc = b->kc + (size_t)l * kvh * m->max_pos * hd;
        int16_t* vc = b->vc + (size_t)l * kvh * m->max_pos * hd;
        if (!qkv_roped) {
            rope_scatter_kernel<<<dim3((nqkv / 2 + 255) / 256, R), 256, 0, st>>>(
                b->QKV, nqkv, b->rows, b->rows_cap, nq, nkv, m->hd_log, m->cos_lut, m->sin_lut, b->Q, kc, vc, sstride,
                kvh, m->max_pos);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        const uint32_t ss = (uint32_t)f.q_frac + f.k_frac + 15u;
        const uint8_t score_shift = (uint8_t)(ss > MYL_TV_SCORE_FRAC_BITS ? ss - MYL_TV_SCORE_FRAC_BITS : 0);
        const dim3 ag(b->ntiles, kvh, ranges);
        const size_t pst = (size_t)b->rows_cap * nq;
        // one row per sequence (decode batches): a block per (row, KV head,
        // range) instead of row tiles
        const bool dec_rows = b->max_qv == G && rows_dec_ok(hd, G);
        const dim3 dg((lmax + kChunk - 1) / kChunk, kvh, R), dpg(ranges, kvh, R);
        if (dec_rows)
            e = hd == 128 ? rows_dec_qk<128>(G, dg, st, b->rows, b->rows_cap, b->Q, nq, kc, sstride, m->max_pos,
                                             m->score_mult, score_shift, b->scores, heads, b->lmax_cap)
                          : rows_dec_qk<64>(G, dg, st, b->rows, b->rows_cap, b->Q, nq, kc, sstride, m->max_pos,
                                            m->score_mult, score_shift, b->scores, heads, b->lmax_cap);
        else if (hd == 128)
            rows_qk_kernel<128><<<ag, kAttnThreads, attn_qk_lds<128>(), st>>>(
                b->tiles, b->rows, b->rows_cap, b->Q, nq, kc, sstride, m->max_pos, G, m->score_mult, score_shift,
                b->scores, heads, b->lmax_cap);
        else
            rows_qk_kernel<64><<<ag, kAttnThreads, attn_qk_lds<64>(), st>>>(
                b->tiles, b->rows, b->rows_cap, b->Q, nq, kc, sstride, m->max_pos, G, m->score_mult, score_shift,
                b->scores, heads, b->lmax_cap);
        if (!dec_rows) e = hipGetLastError();
        if (e != hipSuccess) return e;
        // a wave per (row, head) when there are enough of them to fill the
        // chip, else a block of four waves each
        const int npairs = R * heads;
        const Divider hdiv = Divider::of((uint32_t)heads);
        if (npairs >= 16 * c->prop.multiProcessorCount)
            rows_probs_kernel<1><<<(npairs + 3) / 4, 256, 0, st>>>(b->rows, b->rows_cap, b->scores, hdiv, b->lmax_cap,
                                                                   npairs, m->exp_lut, (uint32_t)m->exp_len, lut_shift,
                                                                   b->probs);
        else
            rows_probs_kernel<4><<<npairs, 256, 0, st>>>(b->rows, b->rows_cap, b->scores, hdiv, b->lmax_cap, npairs,
                                                         m->exp_lut, (uint32_t)m->exp_len, lut_shift, b->probs);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        // Big grids (prefill) loop each block over its tile's ranges and
        // finish the attention output in place; small ones (decode batches)
        // keep a block per range and sum the ranges afterwards.
        const bool loop = !dec_rows && (int64_t)b->ntiles * kvh >= 2 * (int64_t)c->prop.multiProcessorCount;
        const dim3 pg(b->ntiles, kvh, loop ? 1 : ranges);
        int8_t* pplanes = planes ? mm->planes : nullptr;
#define MYL_PV_LAUNCH(HDV, LOOPV, QVMV)                                                                            \
    rows_pv_kernel<HDV, LOOPV, QVMV><<<pg, kAttnThreads, attn_pv_lds<HDV, QVMV>(), st>>>(                          \
        b->tiles, b->rows, b->rows_cap, b->probs, heads, b->lmax_cap, vc, sstride, m->max_pos, G, b->part, pst, nq,  \
        f.v_frac, f.attn_out_frac, b->A, pplanes)
        // tiles of at most 32 query vectors (decode batches) take the
        // narrow variant: 60 KB of LDS, two blocks per CU
        const bool narrow = b->max_qv <= 32;
        if (dec_rows) {
            e = hd == 128 ? rows_dec_pv<128>(G, dpg, st, b->rows, b->rows_cap, b->probs, heads, b->lmax_cap, vc,
                                             sstride, m->max_pos, b->part, pst, nq)
                          : rows_dec_pv<64>(G, dpg, st, b->rows, b->rows_cap, b->probs, heads, b->lmax_cap, vc,
                                            sstride, m->max_pos, b->part, pst, nq);
            if (e != hipSuccess) return e;
        } else if (hd == 128) {
            if (narrow) {
                if (loop) MYL_PV_LAUNCH(128, true, 32);
                else MYL_PV_LAUNCH(128, false, 32);
            } else {
                if (loop) MYL_PV_LAUNCH(128, true, kAttnQV);
                else MYL_PV_LAUNCH(128, false, kAttnQV);
            }
        } else {
            if (narrow) {
                if (loop) MYL_PV_LAUNCH(64, true, 32);
                else MYL_PV_LAUNCH(64, false, 32);
            } else {
                if (loop) MYL_PV_LAUNCH(64, true, kAttnQV);
                else MYL_PV_LAUNCH(64, false, kAttnQV);
            }
        }
#undef MYL_PV_LAUNCH
        if ((e = hipGetLastError()) != hipSuccess) return e;
        if (!loop) {
            rows_attn_out_kernel<<<dim3((nq + 255) / 256, R), 256, 0, st>>>(b->part, pst, b->rows, b->rows_cap, nq,
                                                                            ranges, f.v_frac, f.attn_out_frac, b->A,
                                                                            pplanes);
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
        EpiResidRows eo{};
        eo.shifts = Ld.so; eo.act_frac = f.attn_out_frac; eo.acc_frac = Ld.acc_attn; eo.res_frac = Ld.res_in;
        eo.out_frac = Ld.res_mid; eo.res = b->X; eo.ldr = H; eo.out = b->X2; eo.ldo = H;
        if (norm_in_finish)
            e = resid_then_norm(mm->planes, R, Ld.wo, H, nq, eo, mm, Ld.res_mid, Ld.ref_mid, Ld.post_gamma,
                                Ld.post_gamma_s, m, f.norm_mlp_frac, fuse_silu ? xin : mm->planes, st);
        else
            e = planes ? mm_planes(mm->planes, R, Ld.wo, H, nq, eo, mm, st) : gemv_i8(b->A, R, nq, Ld.wo, H, nq, eo, st, mm);
        if (e != hipSuccess) return e;
        EpiGURows eg{};
        eg.shifts = Ld.sgu; eg.act_frac = f.norm_mlp_frac; eg.gate_frac = f.gate_frac; eg.up_frac = f.up_frac;
        eg.out = b->GU; eg.ldo = 2 * I;
        if (fuse_silu) {
            // the post-attention norm's planes (xin) come from the o_proj finish
            EpiGUSiluPlanes es{Ld.sgu, f.norm_mlp_frac, f.gate_frac, f.up_frac, f.down_in_frac,
                               m->silu, (uint32_t)m->silu_len, mm->planes, I};
            if ((e = frag ? frag_mm_staged(xin, R, H, Ld.wgu_f, 2 * I, es, mm->cus, st)
                          : mm_planes_staged(xin, R, Ld.wgu, 2 * I, H, es, mm, st)) != hipSuccess)
                return e;
        } else if (planes) {
            // the post-attention norm's planes come from the o_proj finish
            if ((e = mm_planes(mm->planes, R, Ld.wgu, 2 * I, H, eg, mm, st)) != hipSuccess) return e;
            silu_planes_kernel<<<dim3((I + 255) / 256, R), 256, 0, st>>>(b->GU, I, m->silu, (uint32_t)m->silu_len,
                                                                         f.gate_frac, f.up_frac, f.down_in_frac,
                                                                         mm->planes);
        } else {
            if ((e = rmsnorm(b->X2, R, H, Ld.res_mid, Ld.post_gamma, Ld.post_gamma_s, H, m->rsqrt, m->rsqrt_len,
                             MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20, f.norm_mlp_frac, b->Xn,
                             H, st)) != hipSuccess ||
                (e = gemv_i8(b->Xn, R, H, Ld.wgu, 2 * I, H, eg, st, mm)) != hipSuccess)
                return e;
            silu_rows_kernel<<<dim3((I + 255) / 256, R), 256, 0, st>>>(b->GU, I, m->silu, (uint32_t)m->silu_len,
                                                                       f.gate_frac, f.up_frac, f.down_in_frac, b->Hh);
        }
        if ((e = hipGetLastError()) != hipSuccess) return e;
        EpiResidRows ed{};
        ed.shifts = Ld.sd; ed.act_frac = f.down_in_frac; ed.acc_frac = Ld.acc_mlp; ed.res_frac = Ld.res_mid;
        ed.out_frac = Ld.res_out; ed.res = b->X2; ed.ldr = H; ed.out = b->X; ed.ldo = H;
        in_normed = norm_in_finish && l + 1 < (int)m->spec.layers;
        if (in_normed) {
            const LayerDev& Ln = m->layers[l + 1];
            e = resid_then_norm(mm->planes, R, Ld.wd, H, I, ed, mm, Ln.res_in, Ln.ref_in, Ln.in_gamma, Ln.in_gamma_s, m,
                                Ln.f.norm_attn_frac, mm->planes, st, frag ? Ld.wd_f : nullptr);
        } else {
            e = planes ? mm_planes(mm->planes, R, Ld.wd, H, I, ed, mm, st) : gemv_i8(b->Hh, R, I, Ld.wd, H, I, ed, st, mm);
        }
        if (e != hipSuccess) return e;
    }
    // final norm and head over rows [h0, R)
    const int HR = R - h0;
    if (HR <= 0) return hipSuccess;
    if ((e = rmsnorm(b->X + (size_t)h0 * H, HR, H, m->final_res, m->final_gamma, m->final_gamma_s, H, m->rsqrt,
                     m->rsqrt_len, MYL_TV_RSQRT_INPUT_SHIFT, MYL_TV_RSQRT_OUTPUT_FRAC, m->inv_n_q20,
                     m->final_norm_frac, b->Xn, H, st)) != hipSuccess)
        return e;
    if (m->spec.lm_head_int16) {
        EpiLogits el{m->lm16_shifts, m->final_norm_frac, MYL_TV_LOGIT_FRAC_BITS, logits_out, V};
        if (HR >= 2 && H % 64 == 0 && mm && mm->planes && (size_t)2 * HR * H <= mm->planes_bytes) {
            // byte planes of both operands, one int8 product
            if (!m->lm16_planes_ok) {
                if (!m->lm16_planes) {
                    m->lm16_planes = m->dalloc<int8_t>((size_t)2 * V * H);
                    m->lm16_wsum = m->dalloc<int32_t>(V);
                    if (!m->lm16_planes || !m->lm16_wsum) return hipErrorOutOfMemory;
                }
                if ((e = split_planes_sum(m->lm16, V, H, H, m->lm16_planes, m->lm16_wsum, st)) != hipSuccess) return e;
                m->lm16_planes_ok = true;
            }
            if ((e = split_planes_sum(b->Xn, HR, H, H, mm->planes, b->xsum, st)) != hipSuccess) return e;
            if ((e = mm2w16_launch(mm->planes, b->xsum, HR, m->lm16_planes, m->lm16_wsum, V, H, el, mm->cus, st)) !=
                hipSuccess)
                return e;
        } else if ((e = gemv_i16(b->Xn, HR, H, m->lm16, V, H, el, st)) != hipSuccess) {
            return e;
        }
    } else {
        EpiLogits el{m->lm8_shifts, m->final_norm_frac, MYL_TV_LOGIT_FRAC_BITS, logits_out, V};
        if ((e = gemv_i8(b->Xn, HR, H, m->lm8, V, H, el, st, mm)) != hipSuccess) return e;
    }
    return argmax_rows(logits_out, HR, V, V, argmax_out, b->argmax_part, st);
}

// Checks the rows against the sequences' cached lengths and uploads them.
// Per sequence the batch's positions must be distinct and fill [p0, p0 + n)
// with p0 <= cached length (a re-run position overwrites, as KVCache::write
// does).  end[s] receives p0 + n (0 for sequences without rows); the caller
// raises the cached lengths to it (commit_len) once the rows have run, so a
// failure leaves no length counting positions whose K/V were never written.
int upload_rows(myl_model* m, BatchState* b, uint32_t R, const uint32_t* seq, const uint32_t* pos, const uint32_t* tok,
                int* lmax, std::vector<uint32_t>* end_out) {
    myl_ctx* c = m->ctx;
    std::vector<std::vector<uint32_t>> per(b->n_seqs);
    int lm = 0;
    for (uint32_t r = 0; r < R; ++r) {
        if (seq[r] >= (uint32_t)b->n_seqs) return c->fail(MYL_E_INVALID, "batch: sequence index out of range");
        if (pos[r] >= (uint32_t)m->max_pos) return c->fail(MYL_E_INVALID, "batch: position beyond the KV capacity");
        if (tok[r] >= (uint32_t)m->V) return c->fail(MYL_E_INVALID, "batch: token id out of range");
        per[seq[r]].push_back(pos[r]);
        lm = std::max(lm, (int)pos[r] + 1);
    }
    std::vector<uint32_t> end(b->n_seqs, 0);
    for (int s = 0; s < b->n_seqs; ++s) {
        std::vector<uint32_t>& p = per[s];
        if (p.empty()) continue;
        std::sort(p.begin(), p.end());
        for (size_t i = 1; i < p.size(); ++i)
            if (p[i] != p[i - 1] + 1)
                return c->fail(MYL_E_INVALID, "batch: positions of a sequence must be distinct and contiguous");
        if (p[0] > b->len[s]) return c->fail(MYL_E_INVALID, "batch: positions must continue the sequence's cache");
        end[s] = p.back() + 1;
    }
    int rc = ensure_rows(m, b, (int)R);
    if (!rc) rc = ensure_scores(m, b, lm);
    if (rc) return rc;
    // attention tiles: each sequence's rows in position order, at most
    // kAttnQV / G rows (and kAttnTileRows) per tile
    const int tr = std::max(1, std::min(kAttnTileRows, kAttnQV / m->G));
    std::vector<std::pair<uint64_t, uint32_t>> order(R);
    for (uint32_t r = 0; r < R; ++r) order[r] = {((uint64_t)seq[r] << 32) | pos[r], r};
    std::sort(order.begin(), order.end());
    std::vector<AttnTile> tiles;
    for (uint32_t i = 0; i < R;) {
        AttnTile t{};
        t.seq = (int32_t)(order[i].first >> 32);
        while (i < R && t.n < tr && (int32_t)(order[i].first >> 32) == t.seq) t.row[t.n++] = (int32_t)order[i++].second;
        tiles.push_back(t);
    }
    // tiles reaching furthest into their caches (the most attention work)
    // first: the row attention kernels schedule them earliest
    {
        std::vector<std::pair<uint32_t, size_t>> key(tiles.size());
        for (size_t i = 0; i < tiles.size(); ++i) {
            uint32_t pm = 0;
            for (int k = 0; k < tiles[i].n; ++k) pm = std::max(pm, pos[tiles[i].row[k]]);
            key[i] = {pm, i};
        }
        std::stable_sort(key.begin(), key.end(), [](const auto& x, const auto& y) { return x.first > y.first; });
        std::vector<AttnTile> sorted(tiles.size());
        for (size_t i = 0; i < tiles.size(); ++i) sorted[i] = tiles[key[i].second];
        tiles.swap(sorted);
    }
    if ((int)tiles.size() > b->tiles_cap) {
        (void)hipStreamSynchronize(c->stream);
        if (b->tiles) (void)hipFree(b->tiles);
        b->tiles = nullptr;
        b->tiles_cap = 0;
        if (hipMalloc(&b->tiles, tiles.size() * sizeof(AttnTile)) != hipSuccess)
            return c->fail(MYL_E_NOMEM, "batch: tile table allocation");
        b->tiles_cap = (int)tiles.size();
    }
    b->ntiles = (int)tiles.size();
    b->max_qv = 0;
    for (const AttnTile& t : tiles) b->max_qv = std::max(b->max_qv, t.n * m->G);
    rc = c->hip(hipMemcpyAsync(b->tiles, tiles.data(), tiles.size() * sizeof(AttnTile), hipMemcpyHostToDevice,
                               c->stream), "batch tiles");
    if (rc) return rc;
    std::vector<int32_t> t(4 * (size_t)b->rows_cap, 0);
    for (uint32_t r = 0; r < R; ++r) {
        t[r] = (int32_t)seq[r];
        t[b->rows_cap + r] = (int32_t)pos[r];
        t[2 * b->rows_cap + r] = (int32_t)(pos[r] % m->rope_rows);
        t[3 * b->rows_cap + r] = (int32_t)tok[r];
    }
    rc = c->hip(hipMemcpyAsync(b->rows, t.data(), t.size() * 4, hipMemcpyHostToDevice, c->stream), "batch rows");
    if (rc) return rc;
    // the pageable source must stay alive until the copy has been consumed
    rc = c->hip(hipStreamSynchronize(c->stream), "batch rows");
    if (rc) return rc;
    *lmax = lm;
    end_out->swap(end);
    return MYL_OK;
}

void commit_len(BatchState* b, const std::vector<uint32_t>& end) {
    for (int s = 0; s < b->n_seqs; ++s) b->len[s] = std::max(b->len[s], end[s]);
}

// Whether the row path can run this model, and its kernels' LDS limits.
int row_path_setup(myl_model* m) {
    myl_ctx* c = m->ctx;
    if (m->G > 16) return c->fail(MYL_E_UNSUPPORTED, "batch: at most 16 query heads per KV head");
    // The matrix-core P.V splits probabilities into bytes; they stay within
    // [0, 2^14] when every exp-table entry is non-negative and no exp sum
    // over max_pos positions wraps (then S >= e_j).
    std::vector<int16_t> lut(m->exp_len);
    int rc = c->hip(hipMemcpy(lut.data(), m->exp_lut, lut.size() * 2, hipMemcpyDeviceToHost), "batch: exp table");
    if (rc) return rc;
    int64_t lut_max = 1;  // an empty table reads as 1 (exp_lookup)
    for (int16_t v : lut) {
        if (v < 0) return c->fail(MYL_E_UNSUPPORTED, "batch: the exp table has negative entries");
        lut_max = std::max<int64_t>(lut_max, v);
    }
    if (lut_max * (int64_t)m->max_pos > (int64_t)INT32_MAX)
        return c->fail(MYL_E_UNSUPPORTED, "batch: exp sums over max_pos positions could wrap");
    const std::pair<const void*, size_t> big[10] = {
        {(const void*)rows_qk_kernel<128>, attn_qk_lds<128>()},
        {(const void*)rows_qk_kernel<64>, attn_qk_lds<64>()},
        {(const void*)rows_pv_kernel<128, false, kAttnQV>, attn_pv_lds<128, kAttnQV>()},
        {(const void*)rows_pv_kernel<128, true, kAttnQV>, attn_pv_lds<128, kAttnQV>()},
        {(const void*)rows_pv_kernel<64, false, kAttnQV>, attn_pv_lds<64, kAttnQV>()},
        {(const void*)rows_pv_kernel<64, true, kAttnQV>, attn_pv_lds<64, kAttnQV>()},
        {(const void*)rows_pv_kernel<128, false, 32>, attn_pv_lds<128, 32>()},
        {(const void*)rows_pv_kernel<128, true, 32>, attn_pv_lds<128, 32>()},
        {(const void*)rows_pv_kernel<64, false, 32>, attn_pv_lds<64, 32>()},
        {(const void*)rows_pv_kernel<64, true, 32>, attn_pv_lds<64, 32>()}};
    for (const auto& k : big)
        if (hipFuncSetAttribute(k.first, hipFuncAttributeMaxDynamicSharedMemorySize, (int)k.second) != hipSuccess)
            return c->fail(MYL_E_HIP, "batch: attention LDS size");
    return MYL_OK;
}

}  // namespace

namespace myl {

// Rows per batched prompt chunk (bounds the row and score buffers).
constexpr uint32_t kPromptChunk = 2048;

int prompt_rows(myl_model* m, const uint32_t* tokens, uint32_t n, uint32_t pos0) {
    myl_ctx* c = m->ctx;
    if (m->prompt_ok < 0) {
        const int rc = row_path_setup(m);
        if (rc && rc != MYL_E_UNSUPPORTED) return rc;
        m->prompt_ok = rc ? 0 : 1;
    }
    if (!m->prompt_ok) return MYL_E_UNSUPPORTED;
    if (!m->prompt) {
        BatchState* b = new (std::nothrow) BatchState();
        if (!b) return MYL_E_NOMEM;
        b->n_seqs = 1;
        b->len.assign(1, 0u);
        b->kc = m->kcache;
        b->vc = m->vcache;
        b->owns_kv = false;
        b->head_rows = 1;
        m->prompt = b;
    }
    BatchState* b = m->prompt;
    b->len[0] = m->n_cached;
    std::vector<uint32_t> seq, pos;
    for (uint32_t i0 = 0; i0 < n; i0 += kPromptChunk) {
        const uint32_t k = std::min(kPromptChunk, n - i0);
        seq.assign(k, 0u);
        pos.resize(k);
        for (uint32_t i = 0; i < k; ++i) pos[i] = pos0 + i0 + i;
        int lmax = 0;
        std::vector<uint32_t> end;
        int rc = upload_rows(m, b, k, seq.data(), pos.data(), tokens + i0, &lmax, &end);
        if (rc) return rc;
        // only the chunk that ends the prompt needs its last row's logits
        const int h0 = i0 + k == n ? (int)k - 1 : (int)k;
        rc = c->hip(forward_rows(m, b, (int)k, lmax, h0, m->logits, b->argmax), "prefill rows");
        if (rc) return rc;
        commit_len(b, end);
    }
    return MYL_OK;
}

}  // namespace myl

extern "C" {

int myl_model_batch_begin(myl_model* m, uint32_t n_seqs) {
    if (!m || n_seqs == 0) return MYL_E_INVALID;
    if (int nr = m->not_ready()) return nr;
    myl_ctx* c = m->ctx;
    if (int rc = row_path_setup(m)) return rc;
    if (m->batch && m->batch->n_seqs == (int)n_seqs) {
        std::fill(m->batch->len.begin(), m->batch->len.end(), 0u);
        return MYL_OK;
    }
    (void)hipStreamSynchronize(c->stream);
    if (m->batch) batch_free(m->batch);
    m->batch = new (std::nothrow) BatchState();
    if (!m->batch) return MYL_E_NOMEM;
    BatchState* b = m->batch;
    b->n_seqs = (int)n_seqs;
    b->len.assign(n_seqs, 0u);
    const size_t bytes = seq_stride(m) * n_seqs * 2;
    if (hipMalloc(&b->kc, bytes) != hipSuccess || hipMalloc(&b->vc, bytes) != hipSuccess) {
        batch_free(b);
        m->batch = nullptr;
        return c->fail(MYL_E_NOMEM, "batch: KV cache allocation");
    }
    if (hipMemsetAsync(b->kc, 0, bytes, c->stream) != hipSuccess || hipMemsetAsync(b->vc, 0, bytes, c->stream) != hipSuccess)
        return c->fail(MYL_E_HIP, "batch: KV cache clear");
    return c->hip(hipStreamSynchronize(c->stream), "batch_begin");
}

int myl_model_forward_batch(myl_model* m, uint32_t n_rows, const uint32_t* seq, const uint32_t* pos,
                            const uint32_t* tokens, int32_t* logits, int64_t* argmax_out) {
    if (!m || !seq || !pos || !tokens) return MYL_E_INVALID;
    if (int nr = m->not_ready()) return nr;
    myl_ctx* c = m->ctx;
    if (!m->batch) return c->fail(MYL_E_INVALID, "forward_batch: call myl_model_batch_begin first");
    if (n_rows == 0) return MYL_OK;
    int lmax = 0;
    BatchState* b = m->batch;
    std::vector<uint32_t> end;
    int rc = upload_rows(m, b, n_rows, seq, pos, tokens, &lmax, &end);
    if (rc) return rc;
    rc = c->hip(forward_rows(m, b, (int)n_rows, lmax, 0, b->logits, b->argmax), "forward_batch");
    if (rc) return rc;
    commit_len(b, end);
    if (logits) {
        rc = c->hip(hipMemcpyAsync(logits, b->logits, (size_t)n_rows * m->V * 4, hipMemcpyDeviceToHost, c->stream),
                    "logits");
        if (rc) return rc;
    }
    if (argmax_out) {
        rc = c->hip(hipMemcpyAsync(argmax_out, b->argmax, (size_t)n_rows * 8, hipMemcpyDeviceToHost, c->stream), "argmax");
        if (rc) return rc;
    }
    return c->hip(hipStreamSynchronize(c->stream), "forward_batch");
}

int myl_model_batch_logits_dev(myl_model* m, const int32_t** logits_dev) {
    if (!m || !logits_dev) return MYL_E_INVALID;
    if (!m->batch || !m->batch->logits) return m->ctx->fail(MYL_E_INVALID, "batch_logits_dev: no batch has run");
    *logits_dev = m->batch->logits;
    return MYL_OK;
}

int myl_model_batch_decode_greedy(myl_model* m, uint32_t n_rows, const uint32_t* seq, const uint32_t* pos,
                                  const uint32_t* tokens, uint32_t n_steps, int64_t* tokens_out) {
    if (!m || !seq || !pos || !tokens) return MYL_E_INVALID;
    if (int nr = m->not_ready()) return nr;
    myl_ctx* c = m->ctx;
    if (!m->batch) return c->fail(MYL_E_INVALID, "batch_decode: call myl_model_batch_begin first");
    if (n_rows == 0 || n_steps == 0) return MYL_OK;
    for (uint32_t r = 0; r < n_rows; ++r)
        if ((uint64_t)pos[r] + n_steps > (uint64_t)m->max_pos)
            return c->fail(MYL_E_INVALID, "batch_decode: positions beyond the KV capacity");
    std::vector<uint32_t> seen(m->batch->n_seqs, 0);
    for (uint32_t r = 0; r < n_rows; ++r) {
        if (seq[r] >= (uint32_t)m->batch->n_seqs) return c->fail(MYL_E_INVALID, "batch_decode: sequence out of range");
        if (seen[seq[r]]++) return c->fail(MYL_E_INVALID, "batch_decode: one row per sequence");
    }
    int lmax = 0;
    BatchState* b = m->batch;
    std::vector<uint32_t> end;
    int rc = upload_rows(m, b, n_rows, seq, pos, tokens, &lmax, &end);
    if (rc) return rc;
    const size_t need = (size_t)n_steps * n_rows;
    if (need > b->tokens_out_cap) {
        (void)hipStreamSynchronize(c->stream);
        if (b->tokens_out) (void)hipFree(b->tokens_out);
        b->tokens_out = nullptr;
        b->tokens_out_cap = 0;
        if (hipMalloc(&b->tokens_out, need * 8) != hipSuccess) return c->fail(MYL_E_NOMEM, "batch_decode: tokens");
        b->tokens_out_cap = need;
    }
    rc = ensure_scores(m, b, lmax + (int)n_steps);
    if (rc) return rc;
    hipError_t e = hipSuccess;
    for (uint32_t s = 0; s < n_steps && e == hipSuccess; ++s) {
        e = forward_rows(m, b, (int)n_rows, lmax + (int)s, 0, b->logits, b->argmax);
        if (e == hipSuccess) {
            rows_advance_kernel<<<(n_rows + 255) / 256, 256, 0, c->stream>>>(b->rows, b->rows_cap, (int)n_rows,
                                                                             b->argmax, m->rope_rows,
                                                                             b->tokens_out + (size_t)s * n_rows);
            e = hipGetLastError();
        }
    }
    rc = c->hip(e, "batch_decode");
    if (rc) return rc;
    for (uint32_t r = 0; r < n_rows; ++r) b->len[seq[r]] = std::max(b->len[seq[r]], pos[r] + n_steps);
    if (tokens_out) {
        rc = c->hip(hipMemcpyAsync(tokens_out, b->tokens_out, need * 8, hipMemcpyDeviceToHost, c->stream), "tokens");
        if (rc) return rc;
    }
    return c->hip(hipStreamSynchronize(c->stream), "batch_decode");
}

int myl_model_batch_read_kv(myl_model* m, uint32_t seq, uint32_t layer, uint32_t kv_head, uint32_t n_pos,
                            int16_t* k_out, int16_t* v_out) {
    if (!m) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (!m->batch || seq >= (uint32_t)m->batch->n_seqs || layer >= m->spec.layers || kv_head >= m->spec.kv_heads ||
        n_pos > (uint32_t)m->max_pos)
        return c->fail(MYL_E_INVALID, "batch_read_kv: out of range");
    const size_t off = seq * seq_stride(m) + (((size_t)layer * m->spec.kv_heads + kv_head) * m->max_pos) * m->hd;
    const size_t bytes = (size_t)n_pos * m->hd * 2;
    int rc = 0;
    if (k_out) rc = c->hip(hipMemcpyAsync(k_out, m->batch->kc + off, bytes, hipMemcpyDeviceToHost, c->stream), "k");
    if (!rc && v_out) rc = c->hip(hipMemcpyAsync(v_out, m->batch->vc + off, bytes, hipMemcpyDeviceToHost, c->stream), "v");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "batch_read_kv");
}

}  // extern "C"
