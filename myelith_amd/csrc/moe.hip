// moe.hip -- an integer mixture-of-experts layer (Qwen1.5-MoE-A2.7B shape) on
// the device: route, dispatch, grouped experts, combine.
//
// The reference has no MoE (its whitepaper chooses dense models), so the
// layer's semantics are defined here from the reference's own primitives, and
// the CPU oracle restates the same definition:
//   router    r_e = clamp_i32(clamp_i32(rescale_i64(W_r[e] . x, 15 + 8, 8)) + bias_e)
//             (the LM-head requant of model.rs:284-308, Q8 logits, plus an
//             integer bias per expert)
//   top-k     k times the first maximum of the remaining logits (argmax_int,
//             sampling.rs:8-18): descending value, lowest index on ties
//   gates     softmax_int over the k selected logits, exp LUT, shift 0,
//             frac 14 (softmax.rs:24-64)
//   dispatch  per expert, its (token, slot) pairs in ascending token order
//   experts   mlp_int (mlp.rs:28-74) with the expert's gate/up/down weights;
//             output per channel at the layer's output fracs
//   shared    mlp_int with the shared expert's weights, same output fracs
//   combine   out = clamp_i16(RNE(sum_k g_k * y_k + 2^14 * s, 14)) in i64
//             (the weighted sum and single rounding of attention.rs:75-86)
//
// Device pipeline: router product (matrix cores) -> top-k + gates + counts ->
// (counts to the host: offsets and the grouped work tables) -> dispatch
// (stable, one block per expert) -> gather -> grouped gate/up product ->
// SiLU gating -> grouped down product -> shared expert (dense products) ->
// combine.
#include "gemm_dispatch.h"
#include "model_internal.h"
#include "ops.h"
#include "rows_epi.h"
#include "wave.h"
#include "../../include/myl_synth.h"

#include <algorithm>
#include <vector>

using namespace myl;

struct myl_moe {
    myl_ctx* ctx = nullptr;
    myl_moe_spec spec{};
    int H = 0, E = 0, I = 0, K = 0, S = 0;
    std::vector<void*> allocs;
    // weights
    int8_t* wr = nullptr;          // [E x H]
    uint8_t* r_shift = nullptr;    // [E]
    int32_t* r_bias = nullptr;     // [E]
    int8_t* wgu = nullptr;         // [E][2I x H], gate row r at 2r, up row r at 2r+1
    uint8_t* sgu = nullptr;        // [E][2I]
    int8_t* wd = nullptr;          // [E][H x I]
    uint8_t* sd = nullptr;         // [E][H]
    int8_t* wgu_s = nullptr;       // shared [2S x H]
    uint8_t* sgu_s = nullptr;
    int8_t* wd_s = nullptr;        // shared [H x S]
    uint8_t* sd_s = nullptr;
    uint8_t* out_frac = nullptr;   // [H]
    int16_t *silu = nullptr, *exp_lut = nullptr;
    int silu_len = 0, exp_len = 0;
    // per-call buffers (grown on demand)
    int cap_t = 0;
    std::vector<void*> bufs;
    int32_t* logits = nullptr;     // [T x E]
    int32_t* ids = nullptr;        // [T x K]
    int32_t* gates = nullptr;      // [T x K]
    int32_t* counts = nullptr;     // [E]
    int32_t* offsets = nullptr;    // [E + 1]
    int32_t* list_tok = nullptr;   // [T x K]
    int32_t* slotpos = nullptr;    // [T x K]
    int16_t *Xg = nullptr, *GU = nullptr, *Hh = nullptr, *Y = nullptr;
    int16_t *GUs = nullptr, *Hs = nullptr, *Sh = nullptr;
    MmWork* work = nullptr;
    int work_cap = 0;
    int32_t* nwork = nullptr;      // [2]: items of the gate/up and down work tables
    std::vector<int32_t> counts_host;

    template <class T> T* dalloc(std::vector<void*>& list, size_t count) {
        void* p = nullptr;
        if (hipMalloc(&p, count * sizeof(T) ? count * sizeof(T) : 1) != hipSuccess) return nullptr;
        list.push_back(p);
        return (T*)p;
    }
    ~myl_moe() {
        if (ctx) (void)hipStreamSynchronize(ctx->stream);
        for (void* p : bufs) (void)hipFree(p);
        for (void* p : allocs) (void)hipFree(p);
        if (work) (void)hipFree(work);
    }
};

namespace {

// ---------------------------------------------------------------------------
// synthetic weights (include/myl_synth.h)
// ---------------------------------------------------------------------------

// dst row (row * rstride + roff) of a [*, K] matrix from stream tseed (row-major).
__global__ void moe_gen_kernel(int8_t* __restrict__ dst, int rows, int K, int rstride, int roff, uint64_t tseed) {
    const int r = blockIdx.y;
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < K; k += gridDim.x * blockDim.x)
        dst[((size_t)r * rstride + roff) * K + k] = myl_synth_w8(tseed, (uint64_t)r * K + k);
}

hipError_t gen(myl_moe* m, int8_t* dst, int rows, int K, int rstride, int roff, uint64_t tseed) {
    for (int r0 = 0; r0 < rows; r0 += 65535) {
        const int nr = std::min(65535, rows - r0);
        moe_gen_kernel<<<dim3((unsigned)std::min((K + 255) / 256, 64), (unsigned)nr), 256, 0, m->ctx->stream>>>(
            dst + (size_t)r0 * rstride * K, nr, K, rstride, roff, tseed);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

__global__ void moe_input_kernel(int16_t* __restrict__ x, size_t n, uint64_t tseed) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] = myl_synth_gauss16(tseed, i, 2000);
}

// ---------------------------------------------------------------------------
// route: bias, top-k, gates, counts
// ---------------------------------------------------------------------------

// The routing of token t by its wave (moe_topk_kernel).
__device__ inline void moe_topk_token(const int32_t* __restrict__ z, int t, int E, int K,
                                      const int32_t* __restrict__ bias, const int16_t* __restrict__ lut,
                                      uint32_t lut_len, int32_t* __restrict__ ids, int32_t* __restrict__ gates,
                                      int32_t* hist, int lane) {
    uint64_t key[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int e = lane + 64 * j;
        key[j] = 0;  // below every real key (their low words are >= 2^32 - 256)
        if (e < E) {
            const int32_t v = clamp_i32_i64((int64_t)z[e] + (int64_t)bias[e]);
            key[j] = ((uint64_t)((uint32_t)v ^ 0x80000000u) << 32) | (0xFFFFFFFFu - (uint32_t)e);
        }
    }
    int32_t sel = 0;
    int sid = 0;
    for (int k = 0; k < K; ++k) {
        const uint64_t b01 = key[0] > key[1] ? key[0] : key[1], b23 = key[2] > key[3] ? key[2] : key[3];
        const uint64_t w = wave_max_u64(b01 > b23 ? b01 : b23);
        const int e = (int)(0xFFFFFFFFu - (uint32_t)w);
#pragma unroll
        for (int j = 0; j < 4; ++j)
            if (lane + 64 * j == e) key[j] = 0;
        if (lane == k) {
            sel = (int32_t)((uint32_t)(w >> 32) ^ 0x80000000u);
            sid = e;
        }
    }
    // softmax.rs:24-64 over the K selected logits (lut_shift 0, frac 14); the
    // first choice is their maximum
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    const int32_t lut_one = lut_len > 0 ? (int32_t)lut[0] : 1;
    const int32_t mx = readlane_i32(sel, 0);
    const int32_t ev = lane < K ? exp_lookup(sat_sub32(mx, sel), lut, lut_len, 0, lut_one) : 0;
    const int32_t S = wave_sum_i32(ev);  // wrapping, as the reference's sum
    if (lane < K) {
        int32_t g;
        if (S == 0) {
            const uint64_t rl = recip32((uint32_t)K);
            uint32_t qq, rr;
            udivmod32((uint32_t)one, (uint32_t)K, rl, &qq, &rr);
            const int32_t base = (int32_t)qq;
            const int32_t rem = wsub32(one, wmul32(base, K));
            g = base + ((int64_t)lane < (int64_t)rem ? 1 : 0);
        } else {
            const uint64_t rs = recip32(S < 0 ? 0u - (uint32_t)S : (uint32_t)S);
            g = softmax_div_round(wmul32(ev, one), S, rs);
        }
        ids[(size_t)t * K + lane] = sid;
        gates[(size_t)t * K + lane] = g;
        atomicAdd(hist + sid, 1);
    }
}

// One wave per token (16 per block).  E <= 256, K <= 16.  Lane l holds
// experts l, l + 64, .. as keys (biased logit ^ 2^31) << 32 | (2^32 - 1 - e):
// the larger key is the larger biased logit, then the lower expert index
// (sampling.rs:8-18's first maximum), so each of the K rounds takes the
// wave's largest key and retires it.  Lane k keeps the k-th choice and
// computes its gate.  The block's choices are counted in LDS first, so a
// popular expert's counter takes one global atomic per block, not one per
// routed token (thousands on one address serialise).
constexpr int kTopkWaves = 16;
__global__ __launch_bounds__(kTopkWaves * 64) void moe_topk_kernel(const int32_t* __restrict__ logits, int T, int E, int K,
                                                       const int32_t* __restrict__ bias,
                                                       const int16_t* __restrict__ lut, uint32_t lut_len,
                                                       int32_t* __restrict__ ids, int32_t* __restrict__ gates,
                                                       int32_t* __restrict__ counts) {
    __shared__ int32_t hist[256];
    for (int e = threadIdx.x; e < E; e += blockDim.x) hist[e] = 0;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * kTopkWaves + (int)(threadIdx.x >> 6);
    if (t < T) moe_topk_token(logits + (size_t)t * E, t, E, K, bias, lut, lut_len, ids, gates, hist, lane);
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x)
        if (hist[e]) atomicAdd(counts + e, hist[e]);
}
// Stable dispatch: block e lists the tokens routed to expert e in ascending
// token order at offsets[e].., and records each (token, slot)'s list position.
__global__ __launch_bounds__(256) void moe_dispatch_kernel(const int32_t* __restrict__ ids, int T, int K,
                                                           const int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ list_tok,
                                                           int32_t* __restrict__ slotpos) {
    __shared__ int32_t wsum[4];
    const int e = blockIdx.x;
    int32_t run = offsets[e];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int base = 0; base < T; base += 256) {
        const int t = base + (int)threadIdx.x;
        int slot = -1;
        if (t < T)
            for (int k = 0; k < K; ++k)
                if (ids[(size_t)t * K + k] == e) slot = k;
        const uint64_t bal = __ballot(slot >= 0);
        const int before = __popcll(bal & ((1ull << lane) - 1ull));
        if (lane == 0) wsum[wave] = __popcll(bal);
        __syncthreads();
        int woff = 0, tot = 0;
        for (int w = 0; w < 4; ++w) {
            if (w < wave) woff += wsum[w];
            tot += wsum[w];
        }
        if (slot >= 0) {
            const int p = run + woff + before;
            list_tok[p] = t;
            slotpos[(size_t)t * K + slot] = p;
        }
        run += tot;
        __syncthreads();
    }
}

// The route's plan on the device (no host round trip): offsets[e] = the
// exclusive prefix of counts, and the work tables of the two grouped
// products in work_table's order (expert, weight tile, token tile), the
// gate/up table at work[0 ..) and the down table at work[max1 ..); their
// sizes go to nwork[0], nwork[1].  Token tiles of 2^bm_log tokens, weight
// tiles of bn rows, nt1 / nt2 weight tiles.  One block of 256 threads, E <= 256;
// thread e writes expert e's items.
__global__ __launch_bounds__(256) void moe_plan_kernel(const int32_t* __restrict__ counts, int E, int bm_log, int bn,
                                                       int nt1, int nt2, int max1, int32_t* __restrict__ offsets,
                                                       MmWork* __restrict__ work, int32_t* __restrict__ nwork) {
    __shared__ int32_t off[257], w1[257], w2[257];
    const int e = threadIdx.x;
    if (e == 0) {
        off[0] = w1[0] = w2[0] = 0;
        for (int x = 0; x < E; ++x) {
            const int c = counts[x], mt = (c + (1 << bm_log) - 1) >> bm_log;
            off[x + 1] = off[x] + c;
            w1[x + 1] = w1[x] + mt * nt1;
            w2[x + 1] = w2[x] + mt * nt2;
        }
        nwork[0] = w1[E];
        nwork[1] = w2[E];
    }
    __syncthreads();
    for (int x = e; x <= E; x += blockDim.x) offsets[x] = off[x];
    if (e < E) {
        const int mt = (off[e + 1] - off[e] + (1 << bm_log) - 1) >> bm_log;
        for (int ni = 0; ni < nt1; ++ni)
            for (int mi = 0; mi < mt; ++mi) work[w1[e] + ni * mt + mi] = MmWork{e, mi << bm_log, ni * bn, 0};
        for (int ni = 0; ni < nt2; ++ni)
            for (int mi = 0; mi < mt; ++mi) work[max1 + w2[e] + ni * mt + mi] = MmWork{e, mi << bm_log, ni * bn, 0};
    }
}

__global__ __launch_bounds__(256) void moe_gather_kernel(const int16_t* __restrict__ x, int H,
                                                         const int32_t* __restrict__ list_tok,
                                                         int16_t* __restrict__ Xg) {
    const int p = blockIdx.x;
    const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)list_tok[p] * H);
    uint4* dst = reinterpret_cast<uint4*>(Xg + (size_t)p * H);
    for (int i = threadIdx.x; i < H / 8; i += 256) dst[i] = src[i];
}

// moe_gather_kernel writing byte planes [2R x H] (rows 2p = hi, 2p + 1 = lo')
// for the grouped byte-plane products.  H % 8 == 0.
__global__ __launch_bounds__(256) void moe_gather_planes_kernel(const int16_t* __restrict__ x, int H,
                                                                const int32_t* __restrict__ list_tok,
                                                                int8_t* __restrict__ Xp) {
    const int p = blockIdx.x;
    const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)list_tok[p] * H);
    int8_t* hi = Xp + (size_t)(2 * p) * H;
    for (int i = threadIdx.x; i < H / 8; i += 256) {
        uint2 h, l;
        split_planes8(src[i], h, l);
        *reinterpret_cast<uint2*>(hi + i * 8) = h;
        *reinterpret_cast<uint2*>(hi + H + i * 8) = l;
    }
}

__device__ inline int16_t moe_silu_one(uint32_t gu, const int16_t* __restrict__ silu, uint32_t silu_len) {
    const int16_t g = (int16_t)(gu & 0xFFFFu), u = (int16_t)(gu >> 16);
    const int32_t g_dom = rescale32((int32_t)g, MYL_MOE_GATE_FRAC, MYL_TV_SILU_IN_FRAC);
    const int16_t act = lut_lookup_i16((int16_t)g_dom, silu, silu_len, (int16_t)MYL_TV_SILU_LUT_OFFSET);
    const int64_t prod = (int64_t)act * (int64_t)u;
    return clamp_i16_i64(rescale64(prod, (uint8_t)(MYL_TV_SILU_OUT_FRAC + MYL_MOE_UP_FRAC), MYL_MOE_DOWN_IN_FRAC));
}

// mlp.rs:55-65 per row, eight outputs per thread (I % 8 == 0).  Grid
// (ceil(I / 2048), R).
__global__ __launch_bounds__(256) void moe_silu_kernel(const int16_t* __restrict__ GU, int I,
                                                       const int16_t* __restrict__ silu, uint32_t silu_len,
                                                       int16_t* __restrict__ Hh) {
    const int r = blockIdx.y;
    const int i0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (i0 >= I) return;
    const uint4* src = reinterpret_cast<const uint4*>(GU + (size_t)r * 2 * I + 2 * i0);
    const uint4 a = src[0], b = src[1];
    const uint32_t gu[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        w[j] = ((uint32_t)(uint16_t)moe_silu_one(gu[2 * j], silu, silu_len)) |
               ((uint32_t)(uint16_t)moe_silu_one(gu[2 * j + 1], silu, silu_len) << 16);
    *reinterpret_cast<uint4*>(Hh + (size_t)r * I + i0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// out = clamp_i16(RNE(sum_k g_k * y_k + 2^14 * s, 14)), eight columns per
// thread (H % 8 == 0, 16-byte rows).  Grid (ceil(H / 2048), T).
__global__ __launch_bounds__(256) void moe_combine_kernel(const int32_t* __restrict__ gates,
                                                          const int32_t* __restrict__ slotpos, int K,
                                                          const int16_t* __restrict__ Y, const int16_t* __restrict__ Sh,
                                                          int H, int16_t* __restrict__ out) {
    const int t = blockIdx.y;
    const int c0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (c0 >= H) return;
    auto unpack = [](uint4 v, int j) { return (int64_t)(int16_t)((j & 1 ? (&v.x)[j >> 1] >> 16 : (&v.x)[j >> 1]) & 0xFFFFu); };
    const uint4 sv = *reinterpret_cast<const uint4*>(Sh + (size_t)t * H + c0);
    int64_t acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = unpack(sv, j) * (int64_t)(1 << MYL_TV_PROB_FRAC_BITS);
    for (int k = 0; k < K; ++k) {
        const int p = slotpos[(size_t)t * K + k];
        const int64_t g = gates[(size_t)t * K + k];
        const uint4 yv = *reinterpret_cast<const uint4*>(Y + (size_t)p * H + c0);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[j] = wadd64(acc[j], g * unpack(yv, j));
    }
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
        w[j] = (uint32_t)(uint16_t)clamp_i16_i64(rshift_round64(acc[2 * j], MYL_TV_PROB_FRAC_BITS)) |
               ((uint32_t)(uint16_t)clamp_i16_i64(rshift_round64(acc[2 * j + 1], MYL_TV_PROB_FRAC_BITS)) << 16);
    *reinterpret_cast<uint4*>(out + (size_t)t * H + c0) = make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------
// grouped epilogues
// ---------------------------------------------------------------------------

struct EpiExpertGU {
    const uint8_t* shifts;  // [E][2I]
    int n2;                 // 2I
    int16_t* out;           // [rows x 2I]
    __device__ inline void one(int e, int n, int row, int64_t acc) const {
        const uint8_t frac = (n & 1) ? MYL_MOE_UP_FRAC : MYL_MOE_GATE_FRAC;
        out[(size_t)row * n2 + n] =
            clamp_i16_i64(rescale64(acc, (uint8_t)(shifts[(size_t)e * n2 + n] + MYL_MOE_X_FRAC), frac));
    }
};

// The grouped gate/up fused with the SiLU gate (mlp.rs:46-65) and the byte-plane
// split of h (mm2_grouped_staged_kernel): gate row 2i and up row 2i+1 of
// expert e requantize to their fracs, then h = silu(g) * u leaves as 8-byte
// pieces of planes rows 2 row (hi) and 2 row + 1 (lo') of the grouped down
// product's operand [2R x I].
struct EpiExpertGUSiluPlanes {
    const uint8_t* shifts;  // [E][2I]
    int n2;                 // 2I
    const int16_t* silu;
    uint32_t silu_len;
    int8_t* planes;         // [2R x I]
    __device__ inline int16_t stage(int e, int n, int64_t acc) const {
        const uint8_t frac = (n & 1) ? MYL_MOE_UP_FRAC : MYL_MOE_GATE_FRAC;
        return clamp_i16_i64(rescale64(acc, (uint8_t)(shifts[(size_t)e * n2 + n] + MYL_MOE_X_FRAC), frac));
    }
    __device__ inline void emit(int, int row, int i0, const uint4& a, const uint4& b) const {
        const uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};  // (g, u) pairs
        uint32_t hi[2] = {0, 0}, lo[2] = {0, 0};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int32_t h = moe_silu_one(w[k], silu, silu_len);
            hi[k >> 2] |= ((uint32_t)(h >> 8) & 0xFFu) << (8 * (k & 3));
            lo[k >> 2] |= ((uint32_t)((h & 255) - 128) & 0xFFu) << (8 * (k & 3));
        }
        const int I = n2 >> 1;
        *reinterpret_cast<uint2*>(planes + (size_t)(2 * row) * I + i0) = make_uint2(hi[0], hi[1]);
        *reinterpret_cast<uint2*>(planes + (size_t)(2 * row + 1) * I + i0) = make_uint2(lo[0], lo[1]);
    }
};

struct EpiExpertDown {
    const uint8_t* shifts;    // [E][H]
    const uint8_t* out_frac;  // [H]
    int H;
    int16_t* out;             // [rows x H]
    __device__ inline void one(int e, int n, int row, int64_t acc) const {
        out[(size_t)row * H + n] = clamp_i16_i64(
            rescale64(acc, (uint8_t)(shifts[(size_t)e * H + n] + MYL_MOE_DOWN_IN_FRAC), out_frac[n]));
    }
};

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------

template <class T>
int upload(myl_moe* m, T* dst, const std::vector<T>& src) {
    return m->ctx->hip(hipMemcpyAsync(dst, src.data(), src.size() * sizeof(T), hipMemcpyHostToDevice, m->ctx->stream),
                       "moe upload");
}

std::vector<uint8_t> shifts_for(uint64_t seed, uint32_t layer, uint32_t role, size_t rows, size_t K) {
    std::vector<uint8_t> v(rows);
    const uint64_t ts = myl_tensor_seed(seed, layer, role);
    for (size_t r = 0; r < rows; ++r) v[r] = myl_synth_wshift(ts, r, K);
    return v;
}

int build(myl_moe* m, const int32_t* router_bias, const myl_luts* luts) {
    myl_ctx* c = m->ctx;
    const uint64_t seed = m->spec.seed;
    const size_t H = m->H, E = m->E, I = m->I, S = m->S;
    auto& A = m->allocs;
    m->wr = m->dalloc<int8_t>(A, E * H);
    m->r_shift = m->dalloc<uint8_t>(A, E);
    m->r_bias = m->dalloc<int32_t>(A, E);
    m->wgu = m->dalloc<int8_t>(A, E * 2 * I * H);
    m->sgu = m->dalloc<uint8_t>(A, E * 2 * I);
    m->wd = m->dalloc<int8_t>(A, E * H * I);
    m->sd = m->dalloc<uint8_t>(A, E * H);
    m->wgu_s = m->dalloc<int8_t>(A, 2 * S * H);
    m->sgu_s = m->dalloc<uint8_t>(A, 2 * S);
    m->wd_s = m->dalloc<int8_t>(A, H * S);
    m->sd_s = m->dalloc<uint8_t>(A, H);
    m->out_frac = m->dalloc<uint8_t>(A, H);
    m->silu = m->dalloc<int16_t>(A, luts->silu_len);
    m->exp_lut = m->dalloc<int16_t>(A, luts->exp_len);
    m->counts = m->dalloc<int32_t>(A, E);
    m->offsets = m->dalloc<int32_t>(A, E + 1);
    m->nwork = m->dalloc<int32_t>(A, 2);
    for (void* p : A)
        if (!p) return c->fail(MYL_E_NOMEM, "moe: weight allocation");
    m->silu_len = (int)luts->silu_len;
    m->exp_len = (int)luts->exp_len;
    int rc = 0;
    rc |= upload(m, m->silu, std::vector<int16_t>(luts->silu, luts->silu + luts->silu_len));
    rc |= upload(m, m->exp_lut, std::vector<int16_t>(luts->exp, luts->exp + luts->exp_len));
    rc |= upload(m, m->r_shift, std::vector<uint8_t>(E, (uint8_t)MYL_MOE_ROUTER_SHIFT));
    rc |= upload(m, m->r_bias, std::vector<int32_t>(router_bias, router_bias + E));
    std::vector<uint8_t> of(H);
    for (size_t i = 0; i < H; ++i) of[i] = myl_synth_moe_out_frac(seed, i);
    rc |= upload(m, m->out_frac, of);
    if (rc) return rc;
    hipError_t e = gen(m, m->wr, (int)E, (int)H, 1, 0, myl_tensor_seed(seed, 0, MYL_R_ROUTER));
    std::vector<uint8_t> sgu(E * 2 * I), sd(E * H);
    for (size_t x = 0; x <= E && e == hipSuccess; ++x) {  // x == E: the shared expert
        const bool shared = x == E;
        const size_t inter = shared ? S : I;
        int8_t* wgu = shared ? m->wgu_s : m->wgu + x * 2 * I * H;
        int8_t* wd = shared ? m->wd_s : m->wd + x * H * I;
        e = gen(m, wgu, (int)inter, (int)H, 2, 0, myl_tensor_seed(seed, (uint32_t)x, MYL_R_WG));
        if (e == hipSuccess) e = gen(m, wgu, (int)inter, (int)H, 2, 1, myl_tensor_seed(seed, (uint32_t)x, MYL_R_WU));
        if (e == hipSuccess) e = gen(m, wd, (int)H, (int)inter, 1, 0, myl_tensor_seed(seed, (uint32_t)x, MYL_R_WD));
        const auto sg = shifts_for(seed, (uint32_t)x, MYL_R_SG, inter, H);
        const auto su = shifts_for(seed, (uint32_t)x, MYL_R_SU, inter, H);
        const auto sdv = shifts_for(seed, (uint32_t)x, MYL_R_SD, H, inter);
        if (shared) {
            std::vector<uint8_t> s2(2 * S);
            for (size_t r = 0; r < S; ++r) { s2[2 * r] = sg[r]; s2[2 * r + 1] = su[r]; }
            rc |= upload(m, m->sgu_s, s2);
            rc |= upload(m, m->sd_s, sdv);
        } else {
            for (size_t r = 0; r < I; ++r) { sgu[x * 2 * I + 2 * r] = sg[r]; sgu[x * 2 * I + 2 * r + 1] = su[r]; }
            std::copy(sdv.begin(), sdv.end(), sd.begin() + x * H);
        }
    }
    if (e != hipSuccess) return c->hip(e, "moe weight generation");
    rc |= upload(m, m->sgu, sgu);
    rc |= upload(m, m->sd, sd);
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "moe build");
}

int ensure(myl_moe* m, int T) {
    if (T <= m->cap_t) return MYL_OK;
    myl_ctx* c = m->ctx;
    (void)hipStreamSynchronize(c->stream);
    for (void* p : m->bufs) (void)hipFree(p);
    m->bufs.clear();
    m->cap_t = 0;
    const size_t TT = T, H = m->H, E = m->E, I = m->I, S = m->S, R = TT * m->K;
    auto& B = m->bufs;
    m->logits = m->dalloc<int32_t>(B, TT * E);
    m->ids = m->dalloc<int32_t>(B, R);
    m->gates = m->dalloc<int32_t>(B, R);
    m->list_tok = m->dalloc<int32_t>(B, R);
    m->slotpos = m->dalloc<int32_t>(B, R);
    m->Xg = m->dalloc<int16_t>(B, R * H);
    m->GU = m->dalloc<int16_t>(B, R * 2 * I);
    m->Hh = m->dalloc<int16_t>(B, R * I);
    m->Y = m->dalloc<int16_t>(B, R * H);
    m->GUs = m->dalloc<int16_t>(B, TT * 2 * S);
    m->Hs = m->dalloc<int16_t>(B, TT * S);
    m->Sh = m->dalloc<int16_t>(B, TT * H);
    for (void* p : B)
        if (!p) return c->fail(MYL_E_NOMEM, "moe: buffer allocation");
    m->cap_t = T;
    return MYL_OK;
}

// Byte-plane tile of the grouped expert products: 0: 128 tokens x 256 weight
// rows (16 waves, 128-byte stages), 1: 128 x 128 (8 waves, 64-byte stages),
// 2: 64 x 128 (8 waves).  The whole 4096-token, 60-expert layer on MI355X
// took 1.42, 1.49 and 1.58 ms with them (1.75 ms with the int16-row tiles of
// mm_w8_grouped_kernel), so 0 when both K are multiples of 128.
// MYL_MOE_TILE overrides the choice for sweeps.
int moe_planes_tile(int H, int I) {
    const bool k128 = H % 128 == 0 && I % 128 == 0;
    const int v = mm_env("MYL_MOE_TILE");
    if (v >= 0 && v <= 2) return (v == 0 && !k128) ? 1 : v;
    return k128 ? 0 : 1;
}
int moe_tile_tokens(int tile) {
    return tile == 0 ? Mm2GroupedShape<2, 2, 4, 4, 2, 128>::kTokens
                     : tile == 1 ? Mm2GroupedShape<2, 2, 4, 2, 3, 64>::kTokens : Mm2GroupedShape<2, 1, 2, 4, 4, 64>::kTokens;
}
int moe_tile_rows(int tile) {
    return tile == 0 ? Mm2GroupedShape<2, 2, 4, 4, 2, 128>::kRows
                     : tile == 1 ? Mm2GroupedShape<2, 2, 4, 2, 3, 64>::kRows : Mm2GroupedShape<2, 1, 2, 4, 4, 64>::kRows;
}
template <class EpiG>
hipError_t moe_grouped(int tile, const int8_t* Ap, const int8_t* W, size_t w_stride, int N, int K, const int* offsets,
                       const MmWork* work, const int* nwork, int maxwork, const EpiG& epi, hipStream_t st) {
    if (tile == 0)
        return mm2_grouped_launch<2, 2, 4, 4, 2, 128>(Ap, W, w_stride, N, K, offsets, work, nwork, maxwork, epi, st);
    if (tile == 1)
        return mm2_grouped_launch<2, 2, 4, 2, 3, 64>(Ap, W, w_stride, N, K, offsets, work, nwork, maxwork, epi, st);
    return mm2_grouped_launch<2, 1, 2, 4, 4, 64>(Ap, W, w_stride, N, K, offsets, work, nwork, maxwork, epi, st);
}

template <class EpiG>
hipError_t moe_grouped_staged(int tile, const int8_t* Ap, const int8_t* W, size_t w_stride, int N, int K,
                              const int* offsets, const MmWork* work, const int* nwork, int maxwork, const EpiG& epi,
                              hipStream_t st) {
    if (tile == 0)
        return mm2_grouped_staged_launch<2, 2, 4, 4, 2, 128>(Ap, W, w_stride, N, K, offsets, work, nwork, maxwork, epi,
                                                             st);
    if (tile == 1)
        return mm2_grouped_staged_launch<2, 2, 4, 2, 3, 64>(Ap, W, w_stride, N, K, offsets, work, nwork, maxwork, epi,
                                                            st);
    return mm2_grouped_staged_launch<2, 1, 2, 4, 4, 64>(Ap, W, w_stride, N, K, offsets, work, nwork, maxwork, epi, st);
}

// Work items of a grouped product over R routed rows of E experts in token
// tiles of bm: sum_e ceil(c_e / bm) <= floor(R / bm) + E token tiles.
int moe_max_items(int R, int E, int bm, int nt) { return (R / bm + E) * nt; }

// Work table of a grouped product: (expert, m-tile, n-tile), m fastest.
void work_table(const std::vector<int32_t>& counts, int bm, int bn, int N, std::vector<MmWork>& out) {
    out.clear();
    for (int e = 0; e < (int)counts.size(); ++e)
        for (int n0 = 0; n0 < N; n0 += bn)
            for (int m0 = 0; m0 < counts[e]; m0 += bm) out.push_back(MmWork{e, m0, n0, 0});
}

}  // namespace

extern "C" {

int myl_moe_create_synthetic(myl_ctx* ctx, const myl_moe_spec* spec, const int32_t* router_bias, const myl_luts* luts,
                             myl_moe** out) {
    if (!ctx || !spec || !router_bias || !luts || !out) return MYL_E_INVALID;
    *out = nullptr;
    const myl_moe_spec& s = *spec;
    if (!s.hidden || !s.n_experts || !s.inter || !s.top_k || !s.shared_inter)
        return ctx->fail(MYL_E_INVALID, "moe: every dimension must be > 0");
    if (s.n_experts > 256 || s.top_k > 16 || s.top_k > s.n_experts)
        return ctx->fail(MYL_E_UNSUPPORTED, "moe: at most 256 experts and top-16");
    if (s.hidden % 16 || s.inter % 16 || s.shared_inter % 16)
        return ctx->fail(MYL_E_UNSUPPORTED, "moe: hidden and intermediate sizes must be multiples of 16");
    if (!luts->silu || !luts->silu_len || !luts->exp || !luts->exp_len) return ctx->fail(MYL_E_INVALID, "moe: LUTs");
    (void)hipSetDevice(ctx->device);
    myl_moe* m = new (std::nothrow) myl_moe();
    if (!m) return MYL_E_NOMEM;
    m->ctx = ctx;
    m->spec = s;
    m->H = (int)s.hidden;
    m->E = (int)s.n_experts;
    m->I = (int)s.inter;
    m->K = (int)s.top_k;
    m->S = (int)s.shared_inter;
    int rc = build(m, router_bias, luts);
    if (rc) {
        delete m;
        return rc;
    }
    *out = m;
    return MYL_OK;
}

void myl_moe_destroy(myl_moe* m) { delete m; }

int myl_moe_synth_input(myl_moe* m, uint32_t n_tokens, int16_t* x_dev) {
    if (!m || !x_dev) return MYL_E_INVALID;
    const size_t n = (size_t)n_tokens * m->H;
    moe_input_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 65535), 256, 0, m->ctx->stream>>>(
        x_dev, n, myl_tensor_seed(m->spec.seed, 0, MYL_R_ACT));
    return m->ctx->hip(hipGetLastError(), "moe_synth_input");
}

int myl_moe_forward(myl_moe* m, const int16_t* x_dev, uint32_t n_tokens, int16_t* out_dev) {
    if (!m || !x_dev || !out_dev) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if (n_tokens == 0) return MYL_OK;
    if (n_tokens > (1u << 24)) return c->fail(MYL_E_INVALID, "moe_forward: too many tokens");
    if (((uintptr_t)x_dev & 15) || ((uintptr_t)out_dev & 15))
        return c->fail(MYL_E_INVALID, "moe_forward: x and out must be 16-byte aligned");
    const int T = (int)n_tokens, H = m->H, E = m->E, I = m->I, K = m->K, S = m->S;
    int rc = ensure(m, T);
    if (rc) return rc;
    hipStream_t st = c->stream;
    const MmCtx* mm = c->mm_ctx((size_t)T * std::max(E, 2 * S), T >= 2 ? (size_t)2 * T * std::max(H, S) : 0);
    hipError_t e;
    // router logits (Q8, the LM-head requant), then top-k, gates and counts
    EpiLogits el{m->r_shift, (uint8_t)MYL_MOE_X_FRAC, (uint8_t)MYL_MOE_ROUTER_FRAC, m->logits, E};
    if ((e = gemv_i8(x_dev, T, H, m->wr, E, H, el, st, mm)) != hipSuccess) return c->hip(e, "moe router");
    if ((e = hipMemsetAsync(m->counts, 0, (size_t)E * 4, st)) != hipSuccess) return c->hip(e, "moe counts");
    moe_topk_kernel<<<(T + kTopkWaves - 1) / kTopkWaves, kTopkWaves * 64, 0, st>>>(m->logits, T, E, K, m->r_bias, m->exp_lut, (uint32_t)m->exp_len,
                                                     m->ids, m->gates, m->counts);
    if ((e = hipGetLastError()) != hipSuccess) return c->hip(e, "moe top-k");
    const int R = T * K;
    const bool planes = H % 64 == 0 && I % 64 == 0;
    if (planes) {
        // byte-plane expert products, planned on the device: offsets and
        // work tables from the counts without a host round trip; the planes
        // [2R x H] and [2R x I] take the bytes of Xg and Hh
        const int tile = moe_planes_tile(H, I);
        const int bm = moe_tile_tokens(tile), bn = moe_tile_rows(tile);
        int bm_log = 0;
        while ((1 << bm_log) < bm) ++bm_log;
        const int nt1 = (2 * I + bn - 1) / bn, nt2 = (H + bn - 1) / bn;
        const int max1 = moe_max_items(R, E, bm, nt1), max2 = moe_max_items(R, E, bm, nt2);
        if (max1 + max2 > m->work_cap) {
            (void)hipStreamSynchronize(st);
            if (m->work) (void)hipFree(m->work);
            m->work = nullptr;
            m->work_cap = 0;
            if (hipMalloc(&m->work, (size_t)(max1 + max2) * sizeof(MmWork)) != hipSuccess)
                return c->fail(MYL_E_NOMEM, "moe work");
            m->work_cap = max1 + max2;
        }
        moe_plan_kernel<<<1, 256, 0, st>>>(m->counts, E, bm_log, bn, nt1, nt2, max1, m->offsets, m->work, m->nwork);
        moe_dispatch_kernel<<<E, 256, 0, st>>>(m->ids, T, K, m->offsets, m->list_tok, m->slotpos);
        int8_t* Xp = reinterpret_cast<int8_t*>(m->Xg);
        int8_t* Hp = reinterpret_cast<int8_t*>(m->Hh);
        moe_gather_planes_kernel<<<R, 256, 0, st>>>(x_dev, H, m->list_tok, Xp);
        if ((e = hipGetLastError()) != hipSuccess) return c->hip(e, "moe dispatch");
        EpiExpertGUSiluPlanes eg{m->sgu, 2 * I, m->silu, (uint32_t)m->silu_len, Hp};
        if ((e = moe_grouped_staged(tile, Xp, m->wgu, (size_t)2 * I * H, 2 * I, H, m->offsets, m->work, m->nwork, max1,
                                    eg, st)) != hipSuccess)
            return c->hip(e, "moe gate/up");
        EpiExpertDown ed{m->sd, m->out_frac, H, m->Y};
        if ((e = moe_grouped(tile, Hp, m->wd, (size_t)H * I, H, I, m->offsets, m->work + max1, m->nwork + 1, max2, ed,
                             st)) != hipSuccess)
            return c->hip(e, "moe down");
    } else {
        // int16-row expert products (K not a multiple of 64): the work tables
        // are built on the host from the counts (the one synchronisation)
        m->counts_host.assign(E, 0);
        rc = c->hip(hipMemcpyAsync(m->counts_host.data(), m->counts, (size_t)E * 4, hipMemcpyDeviceToHost, st),
                    "counts");
        if (!rc) rc = c->hip(hipStreamSynchronize(st), "counts");
        if (rc) return rc;
        std::vector<int32_t> offs(E + 1, 0);
        for (int x = 0; x < E; ++x) offs[x + 1] = offs[x] + m->counts_host[x];
        using GT = MmShape<1, 2, 2, 2>;
        std::vector<MmWork> wgu, wdn;
        work_table(m->counts_host, GT::BM, GT::BN, 2 * I, wgu);
        work_table(m->counts_host, GT::BM, GT::BN, H, wdn);
        const int need = (int)(wgu.size() + wdn.size());
        if (need > m->work_cap) {
            if (m->work) (void)hipFree(m->work);
            m->work = nullptr;
            m->work_cap = 0;
            if (hipMalloc(&m->work, (size_t)need * sizeof(MmWork)) != hipSuccess) return c->fail(MYL_E_NOMEM, "moe work");
            m->work_cap = need;
        }
        std::vector<MmWork> all(wgu);
        all.insert(all.end(), wdn.begin(), wdn.end());
        rc = c->hip(hipMemcpyAsync(m->work, all.data(), all.size() * sizeof(MmWork), hipMemcpyHostToDevice, st), "work");
        if (!rc) rc = c->hip(hipMemcpyAsync(m->offsets, offs.data(), offs.size() * 4, hipMemcpyHostToDevice, st), "offs");
        if (rc) return rc;
        moe_dispatch_kernel<<<E, 256, 0, st>>>(m->ids, T, K, m->offsets, m->list_tok, m->slotpos);
        moe_gather_kernel<<<R, 256, 0, st>>>(x_dev, H, m->list_tok, m->Xg);
        if ((e = hipGetLastError()) != hipSuccess) return c->hip(e, "moe dispatch");
        if (!wgu.empty()) {
            EpiExpertGU eg{m->sgu, 2 * I, m->GU};
            mm_w8_grouped_kernel<1, 2, 2, 2, EpiExpertGU><<<8 * (((int)wgu.size() + 7) / 8), GT::kThreads, GT::kLds,
                                                             st>>>(m->Xg, H, m->wgu, (size_t)2 * I * H, 2 * I, H,
                                                                   m->offsets, m->work, (int)wgu.size(), eg);
            if ((e = hipGetLastError()) != hipSuccess) return c->hip(e, "moe gate/up");
            moe_silu_kernel<<<dim3((I / 8 + 255) / 256, R), 256, 0, st>>>(m->GU, I, m->silu, (uint32_t)m->silu_len,
                                                                          m->Hh);
            EpiExpertDown ed{m->sd, m->out_frac, H, m->Y};
            mm_w8_grouped_kernel<1, 2, 2, 2, EpiExpertDown><<<8 * (((int)wdn.size() + 7) / 8), GT::kThreads, GT::kLds,
                                                               st>>>(m->Hh, I, m->wd, (size_t)H * I, H, I, m->offsets,
                                                                     m->work + wgu.size(), (int)wdn.size(), ed);
            if ((e = hipGetLastError()) != hipSuccess) return c->hip(e, "moe down");
        }
    }
    // shared expert: dense products over every token.  With byte planes the
    // gate/up product's staged epilogue applies the SiLU gate and writes the
    // down product's planes [2T x S] (in the bytes of Hs).
    EpiShift eds{m->sd_s, m->out_frac, (uint8_t)MYL_MOE_DOWN_IN_FRAC, 0, m->Sh, H};
    if (mm_planes_ok(T, H, mm) && mm_planes_ok(T, S, mm) && T > 64) {
        int8_t* Sp = reinterpret_cast<int8_t*>(m->Hs);
        EpiGUSiluPlanes es{m->sgu_s, (uint8_t)MYL_MOE_X_FRAC, (uint8_t)MYL_MOE_GATE_FRAC, (uint8_t)MYL_MOE_UP_FRAC,
                           (uint8_t)MYL_MOE_DOWN_IN_FRAC, m->silu, (uint32_t)m->silu_len, Sp, S};
        if ((e = split_planes(x_dev, T, H, H, mm->planes, st)) != hipSuccess) return c->hip(e, "shared planes");
        if ((e = mm_planes_staged(mm->planes, T, m->wgu_s, 2 * S, H, es, mm, st)) != hipSuccess)
            return c->hip(e, "shared gate/up");
        if ((e = mm_planes(Sp, T, m->wd_s, H, S, eds, mm, st)) != hipSuccess) return c->hip(e, "shared down");
    } else {
        EpiGURows egs{};
        egs.shifts = m->sgu_s; egs.act_frac = MYL_MOE_X_FRAC; egs.gate_frac = MYL_MOE_GATE_FRAC;
        egs.up_frac = MYL_MOE_UP_FRAC; egs.out = m->GUs; egs.ldo = 2 * S;
        if ((e = gemv_i8(x_dev, T, H, m->wgu_s, 2 * S, H, egs, st, mm)) != hipSuccess) return c->hip(e, "shared gate/up");
        moe_silu_kernel<<<dim3((S / 8 + 255) / 256, T), 256, 0, st>>>(m->GUs, S, m->silu, (uint32_t)m->silu_len, m->Hs);
        if ((e = gemv_i8(m->Hs, T, S, m->wd_s, H, S, eds, st, mm)) != hipSuccess) return c->hip(e, "shared down");
    }
    moe_combine_kernel<<<dim3((H / 8 + 255) / 256, T), 256, 0, st>>>(m->gates, m->slotpos, K, m->Y, m->Sh, H, out_dev);
    return c->hip(hipGetLastError(), "moe combine");
}

int myl_moe_read_route(myl_moe* m, uint32_t n_tokens, int32_t* ids, int32_t* gates, int32_t* counts, int32_t* offsets,
                       int32_t* list_tok) {
    if (!m) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    if ((int)n_tokens > m->cap_t) return c->fail(MYL_E_INVALID, "moe_read_route: more tokens than the last call");
    const size_t R = (size_t)n_tokens * m->K;
    hipStream_t st = c->stream;
    int rc = 0;
    if (ids) rc = c->hip(hipMemcpyAsync(ids, m->ids, R * 4, hipMemcpyDeviceToHost, st), "ids");
    if (!rc && gates) rc = c->hip(hipMemcpyAsync(gates, m->gates, R * 4, hipMemcpyDeviceToHost, st), "gates");
    if (!rc && counts) rc = c->hip(hipMemcpyAsync(counts, m->counts, (size_t)m->E * 4, hipMemcpyDeviceToHost, st), "counts");
    if (!rc && offsets)
        rc = c->hip(hipMemcpyAsync(offsets, m->offsets, (size_t)(m->E + 1) * 4, hipMemcpyDeviceToHost, st), "offsets");
    if (!rc && list_tok) rc = c->hip(hipMemcpyAsync(list_tok, m->list_tok, R * 4, hipMemcpyDeviceToHost, st), "list");
    if (rc) return rc;
    return c->hip(hipStreamSynchronize(st), "moe_read_route");
}

}  // extern "C"
