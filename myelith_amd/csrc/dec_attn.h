// dec_attn.h -- integer attention of one query row over a KV cache
// (attention.rs:42-90 with softmax.rs:12-64): the decode step's attention as
// one kernel.
//
// A block takes one KV head, a run of `sub` 64-position chunks of the cache,
// and every query head that shares the KV head (G of them), so each K and V
// row is read from HBM once per step.  softmax_int rounds every probability
// against the head's exp sum, which needs the head's maximum score first, so
// the blocks of a KV head exchange two statistics per query head:
//   1. exact scores of the block's positions (kept in LDS); the block maximum
//      of each head is folded into the head's maximum word with a
//      device-scope atomic max; the block arrives on its KV head's counter (a
//      device-scope atomic), waits for all of the KV head's blocks, then reads
//      the head maxima;
//   2. exp values against the head maximum; each block adds 2^48 + its
//      wrapping exp sum to the head's 64-bit word with one device-scope
//      atomic (bits 48-63 count the blocks, bits 0-47 hold the exact sum of
//      the u32 block sums, whose low 32 bits are the wrapping total) and
//      waits until the count is complete;
//   3. probabilities from the head sum, then the exact P.V of the block's
//      positions added to the head's i64 accumulators with 64-bit atomics.
// Device-scope loads bypass the per-XCD L2 caches for coherence and the
// atomics are performed past them, so the exchange needs no L2 writeback or
// invalidate (a fence-based exchange costs 13-30 us on MI355X).
// Every word that many blocks update sits on its own 64-byte line (atomics of
// every block on one line serialise: about 13 us per step at 7B widths when
// all heads shared two lines).  The waits need every block of a KV head
// resident at once: the host launches at most one block per CU, and every
// wait is bounded: a block that waits longer than kAttnSpinLimit polls
// records a stall in the step state and goes on, so the kernel always ends
// and the host fails the call.
#pragma once

#include "ops.h"
#include "wave.h"

namespace myl {

constexpr int kChunk = 64;          // positions per chunk (one row per lane in the statistics passes)
constexpr int kDecExpLds = 4096;    // exp-table entries held in LDS (8 KB)
constexpr int kAttnMaxSub = 8;      // chunks per block at most (a power of two)
constexpr int kAttnSpinLimit = 1 << 15;
constexpr int kAttnMaxG = 64;      // query heads per KV head (one lane each in the sum wait)

// Synchronisation words of the decode attention, zero between steps (the
// layer's gate/up kernel clears them with the P.V accumulators), u32 units,
// each on its own 64-byte line:
//   arrival counter of KV head g at g * 16,
//   64-bit sum word of query head h at kvh * 16 + h * 16,
//   maximum word of query head h at (kvh + heads) * 16 + h * 16 (u32 of the
//   score ^ 2^31: the cleared value 0 stands for INT32_MIN and unsigned order
//   is signed order).
struct AttnSyncWords {
    __host__ __device__ static int counter(int g) { return g * 16; }
    __host__ __device__ static int sum_word(int kvh, int h) { return kvh * 16 + h * 16; }
    __host__ __device__ static int max_word(int kvh, int heads, int h) { return (kvh + heads) * 16 + h * 16; }
    __host__ __device__ static int count(int kvh, int heads) { return (kvh + 2 * heads) * 16; }
};

// Dynamic LDS of one block: scores / exp values / probabilities [G][sub * 64]
// i32, per-head statistics [4][G] u32, the G query vectors [G][HD] int16, the
// raw dot products of one chunk [G][64] (two i32 each).
__host__ __device__ inline size_t attn_dyn_lds(int G, int sub, int hd) {
    return (size_t)G * ((size_t)sub * kChunk * 4 + 16 + (size_t)hd * 2 + kChunk * 8);
}

__device__ inline void vm_wait_all() { __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8)); }  // vmcnt(0)

// Arrives on a counter and waits (bounded) until it reaches target.
__device__ inline bool attn_arrive_wait(uint32_t* ctr, uint32_t target) {
    uint32_t v = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    for (int polls = 0; v < target; ++polls) {
        if (polls >= kAttnSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
        v = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return true;
}

// int16 pairs -> (hi pair, lo pair) with v = 256 * hi + lo, lo in [0, 255].
__device__ inline void split_pair(uint32_t v, uint32_t& hi, uint32_t& lo) {
    const int32_t a = (int16_t)(v & 0xFFFFu), b = (int16_t)(v >> 16);
    hi = ((uint32_t)(uint16_t)(int16_t)(a >> 8)) | ((uint32_t)(uint16_t)(int16_t)(b >> 8) << 16);
    lo = (v & 0x00FF00FFu);
}

// V rows of one chunk in registers: thread t holds 16 bytes of rows
// t / (HD / 8) + 256 / (HD / 8) * i.
template <int HD>
struct DecVRegs {
    static constexpr int TPR = HD / 8;            // threads per row (16 bytes each)
    static constexpr int PER = kChunk * TPR / 256; // rows per thread
    uint4 v[PER];
};

template <int HD>
__device__ inline void dec_load_v(int L, int base, const int16_t* __restrict__ vg, DecVRegs<HD>& r) {
    const int piece = threadIdx.x % DecVRegs<HD>::TPR, row0 = threadIdx.x / DecVRegs<HD>::TPR;
#pragma unroll
    for (int i = 0; i < DecVRegs<HD>::PER; ++i) {
        const int j = base + row0 + i * (256 / DecVRegs<HD>::TPR);
        r.v[i] = j < L ? *reinterpret_cast<const uint4*>(vg + (size_t)j * HD + piece * 8) : make_uint4(0, 0, 0, 0);
    }
}

template <int HD>
__device__ inline void dec_store_v(const DecVRegs<HD>& r, uint32_t* vl) {
    const int piece = threadIdx.x % DecVRegs<HD>::TPR, row0 = threadIdx.x / DecVRegs<HD>::TPR;
#pragma unroll
    for (int i = 0; i < DecVRegs<HD>::PER; ++i) {
        const int row = row0 + i * (256 / DecVRegs<HD>::TPR);
        *reinterpret_cast<uint4*>(vl + row * (HD / 2) + piece * 4) = r.v[i];
    }
}

// K rows of one chunk in registers: LPP = HD / 8 lanes per row (16 bytes
// each), PPW rows per wave per step, STEPS steps per wave (64 rows per block).
template <int HD>
struct DecKRegs {
    static constexpr int LPP = HD / 8;
    static constexpr int PPW = 64 / LPP;
    static constexpr int STEPS = kChunk / 4 / PPW;
    uint4 k[STEPS];
};

template <int HD>
__device__ inline int dec_k_row(int it) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    return wave * (kChunk / 4) + it * DecKRegs<HD>::PPW + lane / DecKRegs<HD>::LPP;
}

template <int HD>
__device__ inline void dec_load_k(int L, int base, const int16_t* __restrict__ kg, DecKRegs<HD>& r) {
    const int sub = (threadIdx.x & 63) % DecKRegs<HD>::LPP;
#pragma unroll
    for (int it = 0; it < DecKRegs<HD>::STEPS; ++it) {
        const int j = base + dec_k_row<HD>(it);
        r.k[it] = j < L ? *reinterpret_cast<const uint4*>(kg + (size_t)j * HD + sub * 8) : make_uint4(0, 0, 0, 0);
    }
}

// The chunk's raw dot products q . k_j for one query head, as the pair
// (sum(k * q_hi), sum(k * q_lo)) with q . k = 256 * first + second (exact:
// |partials| < 2^31), written to dd[j] for the chunk's rows j < L; the row
// sums over the LPP lanes are DPP moves.  The score (attention.rs:66-67) is
// finished later, once per (head, row): dec_score_of.
template <int HD>
__device__ inline void dec_dots(int L, int base, const int16_t* __restrict__ qh_lds, const DecKRegs<HD>& kr,
                                uint2* __restrict__ dd) {
    constexpr int LPP = DecKRegs<HD>::LPP;
    static_assert(LPP == 8 || LPP == 16, "row sums cover 8 or 16 lanes");
    const int sub = (threadIdx.x & 63) % LPP;
    const uint4 qv = *reinterpret_cast<const uint4*>(qh_lds + sub * 8);
    uint4 qh, ql;
    split_pair(qv.x, qh.x, ql.x);
    split_pair(qv.y, qh.y, ql.y);
    split_pair(qv.z, qh.z, ql.z);
    split_pair(qv.w, qh.w, ql.w);
    typedef short __attribute__((ext_vector_type(2))) s2;
    auto d2 = [](uint32_t a, uint32_t c, int32_t acc) {
        return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, c), acc, false);
    };
#pragma unroll
    for (int it = 0; it < DecKRegs<HD>::STEPS; ++it) {
        const int jj = dec_k_row<HD>(it);
        int32_t ahi = 0, alo = 0;
        ahi = d2(kr.k[it].x, qh.x, ahi);
        ahi = d2(kr.k[it].y, qh.y, ahi);
        ahi = d2(kr.k[it].z, qh.z, ahi);
        ahi = d2(kr.k[it].w, qh.w, ahi);
        alo = d2(kr.k[it].x, ql.x, alo);
        alo = d2(kr.k[it].y, ql.y, alo);
        alo = d2(kr.k[it].z, ql.z, alo);
        alo = d2(kr.k[it].w, ql.w, alo);
        if (LPP == 16) {
            ahi = row_sum16_i32(ahi);
            alo = row_sum16_i32(alo);
        } else {
            ahi = row_sum8_i32(ahi);
            alo = row_sum8_i32(alo);
        }
        if (sub == 0 && base + jj < L) dd[jj] = make_uint2((uint32_t)ahi, (uint32_t)alo);
    }
}

// z = (i32)RNE(q . k * mult, shift) (attention.rs:66-67) from a dec_dots pair.
__device__ inline int32_t dec_score_of(uint2 d, int64_t score_mult, uint8_t score_shift) {
    const int64_t dot = (int64_t)(int32_t)d.x * 256 + (int64_t)(int32_t)d.y;
    return (int32_t)rshift_round64(wmul64(dot, score_mult), score_shift);
}

// Wave 0 waits (bounded) until the sum words of heads h0 .. h0 + G - 1 count
// nb blocks and writes the wrapping sums to red[0 .. G); false on a timeout.
__device__ inline bool attn_wait_sums(const uint64_t* __restrict__ words, int h0, int G, int nb, uint32_t* red) {
    const int lane = threadIdx.x & 63;
    bool done = lane >= G;
    uint64_t v = 0;
    for (int polls = 0;; ++polls) {
        if (!done) {
            v = __hip_atomic_load(words + (size_t)(h0 + lane) * 8, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            done = (int)(v >> 48) >= nb;
        }
        if (__builtin_amdgcn_ballot_w64(!done) == 0) break;
        if (polls >= kAttnSpinLimit) return false;
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane < G) red[lane] = (uint32_t)v;
    return true;
}

// The decode attention of KV head blockIdx.y, positions
// [blockIdx.x * sub * 64, ...) of L = st->pos + 1, for query heads
// [g * G, g * G + G), G <= kAttnMaxG.  acc [heads][HD] i64 and the sync words
// must be zero on entry (acc then holds sum_j p_j v_j exactly).  256 threads;
// grid (ceil(max_pos / (64 sub)), kv_heads), sub a power of two; dynamic LDS
// attn_dyn_lds(G, sub, HD).
// exp_lds >= 0: the table has at least kDecExpLds entries in memory and every
// entry from exp_lds on is zero, so entries [0, kDecExpLds) are read from an
// LDS copy; -1: the table is read in place.  PV16: every exp-table entry is
// >= 0 and max_pos * (largest entry) < 2^31, so every exp value lies in
// [0, S], every probability in [0, 2^14] (an int16, a 15-bit quotient found
// by long division without a reciprocal) and a chunk's sum of p_j v_j within
// +-2^30: P.V runs on v_dot2_i32_i16 with i32 sums; otherwise in i64.
template <int HD, bool PV16>
__device__ inline void dec_attention(DecodeState* __restrict__ st, const int16_t* __restrict__ q,
                                     const int16_t* __restrict__ kc, const int16_t* __restrict__ vc, int max_pos,
                                     int G, int sub, int64_t score_mult, uint8_t score_shift,
                                     const int16_t* __restrict__ lut, uint32_t lut_len, uint8_t lut_shift,
                                     int exp_lds, uint32_t* __restrict__ sync,
                                     unsigned long long* __restrict__ acc) {
    extern __shared__ int32_t dyn[];
    __shared__ int16_t elut[kDecExpLds];
    __shared__ uint32_t vl[kChunk * HD / 2];
    __shared__ int s_ok;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int L = st->pos + 1;
    const int P = sub * kChunk;      // sub is a power of two
    const int nb = (L + P - 1) >> (31 - __builtin_clz((uint32_t)P));  // blocks of this KV head holding positions
    const int c = blockIdx.x, g = blockIdx.y, kvh = gridDim.y;
    if (c >= nb) return;
    const int base = c * P, n = min(P, L - base), h0 = g * G;
    int32_t* z = dyn;                                             // [G][P]
    uint32_t* hs = reinterpret_cast<uint32_t*>(dyn + G * P);      // [4][G]: max, sum, recip lo / hi or uniform split
    int16_t* qs = reinterpret_cast<int16_t*>(hs + 4 * G);         // [G][HD]
    uint2* dd = reinterpret_cast<uint2*>(qs + G * HD);            // [G][64]
    const int16_t* kg = kc + (size_t)g * max_pos * HD;
    const int16_t* vg = vc + (size_t)g * max_pos * HD;
    uint32_t* ctr = sync + AttnSyncWords::counter(g);
    uint64_t* sums = reinterpret_cast<uint64_t*>(sync + AttnSyncWords::sum_word(kvh, 0));
    uint32_t* maxw = sync + AttnSyncWords::max_word(kvh, kvh * G, 0);

    // every global load of the block goes out first: q, K and V of the first
    // chunk, the exp table
    const int qpieces = G * HD / 8;
    uint4 qv = tid < qpieces ? reinterpret_cast<const uint4*>(q + (size_t)h0 * HD)[tid] : make_uint4(0, 0, 0, 0);
    DecKRegs<HD> kr;
    dec_load_k<HD>(L, base, kg, kr);
    DecVRegs<HD> vr;
    dec_load_v<HD>(L, base, vg, vr);
    constexpr int LPT = kDecExpLds / 8 / 256;
    uint4 lv[LPT];
    const bool lds = exp_lds >= 0;
#pragma unroll
    for (int i = 0; i < LPT; ++i) {
        const int e0 = (tid + i * 256) * 8;
        lv[i] = lds && e0 < exp_lds ? *reinterpret_cast<const uint4*>(lut + e0) : make_uint4(0, 0, 0, 0);
    }
    if (tid < qpieces) reinterpret_cast<uint4*>(qs)[tid] = qv;
    for (int i = tid + 256; i < qpieces; i += 256)
        reinterpret_cast<uint4*>(qs)[i] = reinterpret_cast<const uint4*>(q + (size_t)h0 * HD)[i];
    __syncthreads();

    // 1. scores, block maxima, first exchange
    for (int s = 0; s < sub; ++s) {
        const int bs = base + s * kChunk;
        if (bs >= L) break;
        if (s > 0) dec_load_k<HD>(L, bs, kg, kr);
        for (int h = 0; h < G; ++h) dec_dots<HD>(L, bs, qs + h * HD, kr, dd + h * kChunk);
        __syncthreads();
        for (int t = tid; t < G * kChunk; t += 256) {
            const int h = t >> 6, jj = t & (kChunk - 1);
            if (bs + jj < L) z[h * P + s * kChunk + jj] = dec_score_of(dd[t], score_mult, score_shift);
        }
        __syncthreads();
    }
    for (int h = wave; h < G; h += 4) {
        int32_t mx = INT32_MIN;
        for (int j = lane; j < n; j += 64) mx = max(mx, z[h * P + j]);
        mx = wave_max_i32(mx);
        if (lane == 0)
            __hip_atomic_fetch_max(maxw + (size_t)(h0 + h) * 16, (uint32_t)mx ^ 0x80000000u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    vm_wait_all();
    __syncthreads();
    if (tid == 0) s_ok = attn_arrive_wait(ctr, (uint32_t)nb) ? 1 : 0;
    __syncthreads();
    if (tid < G)
        hs[tid] = __hip_atomic_load(maxw + (size_t)(h0 + tid) * 16, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ^
                  0x80000000u;

    // 2. exp values against the head maxima, block sums, second exchange
    if (lds) {
#pragma unroll
        for (int i = 0; i < LPT; ++i) {
            const int e0 = (tid + i * 256) * 8;
            if (e0 < exp_lds) *reinterpret_cast<uint4*>(elut + e0) = lv[i];
        }
    }
    __syncthreads();
    const int32_t lut_one = lut_len > 0 ? (int32_t)lut[0] : 1;
    for (int h = wave; h < G; h += 4) {
        const int32_t mh = (int32_t)hs[h];
        uint32_t s = 0;
        for (int j = lane; j < n; j += 64) {
            // exp_lookup (softmax.rs:12-20) of mh - z with a saturating difference
            const int32_t x = sat_sub32(mh, z[h * P + j]);
            int32_t e;
            if (x <= 0) {
                e = lut_one;
            } else {
                const uint32_t idx = (uint32_t)x >> (lut_shift & 31u);
                e = lds ? (idx < (uint32_t)exp_lds ? (int32_t)elut[idx] : 0) : (idx < lut_len ? (int32_t)lut[idx] : 0);
            }
            z[h * P + j] = e;
            s += (uint32_t)e;
        }
        s = (uint32_t)wave_sum_i32((int32_t)s);
        if (lane == 0)
            __hip_atomic_fetch_add(sums + (size_t)(h0 + h) * 8, (1ull << 48) + s, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    }
    dec_store_v<HD>(vr, vl);
    if (wave == 0) {
        const bool ok = attn_wait_sums(sums, h0, G, nb, hs + G);
        if (lane == 0 && !ok) s_ok = 0;
    }
    __syncthreads();

    // 3. probabilities (softmax.rs:40-63), then P.V (attention.rs:75-81)
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    if (tid < G) {
        const int32_t S = (int32_t)hs[G + tid];
        if (PV16 && S != 0) {
            // the long division below needs no reciprocal
        } else if (S != 0) {
            const uint64_t r = recip32(S < 0 ? 0u - (uint32_t)S : (uint32_t)S);
            hs[2 * G + tid] = (uint32_t)r;
            hs[3 * G + tid] = (uint32_t)(r >> 32);
        } else {
            // every exp value zero: one / L each, the remainder to the first positions
            uint32_t qq, rr;
            udivmod32((uint32_t)one, (uint32_t)L, recip32((uint32_t)L), &qq, &rr);
            hs[2 * G + tid] = qq;
            hs[3 * G + tid] = (uint32_t)wsub32(one, wmul32((int32_t)qq, L));
        }
        if (s_ok == 0 && tid == 0) atomicOr(&st->stalls, 1u);
    }
    __syncthreads();
    // probabilities of the block's positions, zero past its last one (the
    // P.V loop then runs whole chunks); PV16 writes them as int16 in place
    // (element j over the i32 slot j / 2, already read by then)
    for (int h = wave; h < G; h += 4) {
        const int32_t S = (int32_t)hs[G + h];
        const uint64_t r = ((uint64_t)hs[3 * G + h] << 32) | hs[2 * G + h];
        for (int j = lane; j < P; j += 64) {
            int32_t p = 0;
            if (j < n) {
                if (S == 0)
                    p = (int32_t)hs[2 * G + h] +
                        (((uint64_t)(base + j) < (uint64_t)(int64_t)(int32_t)hs[3 * G + h]) ? 1 : 0);
                else if (PV16)
                    p = softmax_div_round_q15(z[h * P + j], S);
                else
                    p = softmax_div_round(wmul32(z[h * P + j], one), S, r);
            }
            if (PV16)
                reinterpret_cast<int16_t*>(z + h * P)[j] = (int16_t)p;
            else
                z[h * P + j] = p;
        }
    }
    __syncthreads();
    for (int s = 0; s < sub; ++s) {
        const int bs = base + s * kChunk;
        if (bs >= L) break;
        if (s > 0) {
            __syncthreads();  // every wave is done with the previous chunk's V
            dec_load_v<HD>(L, bs, vg, vr);
            dec_store_v<HD>(vr, vl);
            __syncthreads();
        }
        // lane: dimensions 2 dp, 2 dp + 1 of positions with pair parity par
        constexpr int DP = HD / 2;                  // dimension pairs
        constexpr int PAR = 64 / DP;                // 1 (HD 128) or 2 (HD 64) interleaved position streams
        const int dp = lane % DP, par = lane / DP;
        for (int h = wave; h < G; h += 4) {
            uint64_t a0 = 0, a1 = 0;
            if (PV16) {
                // positions 2i, 2i + 1 at once: (v_2i, v_2i+1) of one dimension
                // against the probability pair on v_dot2_i32_i16
                typedef short __attribute__((ext_vector_type(2))) s2;
                const uint32_t* pp = reinterpret_cast<const uint32_t*>(z + h * P) + s * (kChunk / 2);
                int32_t b0 = 0, b1 = 0;
#pragma unroll
                for (int i = par; i < kChunk / 2; i += PAR) {
                    const uint32_t p2 = pp[i];
                    const uint32_t va = vl[(2 * i) * DP + dp], vb = vl[(2 * i + 1) * DP + dp];
                    const uint32_t lo = __builtin_amdgcn_perm(vb, va, 0x05040100u);
                    const uint32_t hi = __builtin_amdgcn_perm(vb, va, 0x07060302u);
                    b0 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, lo), __builtin_bit_cast(s2, p2), b0, false);
                    b1 = __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, hi), __builtin_bit_cast(s2, p2), b1, false);
                }
                if (PAR == 2) {
                    b0 += __shfl_xor(b0, 32);
                    b1 += __shfl_xor(b1, 32);
                }
                a0 = (uint64_t)(int64_t)b0;
                a1 = (uint64_t)(int64_t)b1;
            } else {
                const int32_t* ph = z + h * P + s * kChunk;
#pragma unroll 16
                for (int j = par; j < kChunk; j += PAR) {
                    const int64_t p = ph[j];
                    const uint32_t v = vl[j * DP + dp];
                    a0 += (uint64_t)(p * (int64_t)(int16_t)(v & 0xFFFFu));
                    a1 += (uint64_t)(p * (int64_t)(int16_t)(v >> 16));
                }
                if (PAR == 2) {
                    a0 += (uint64_t)__shfl_xor((unsigned long long)a0, 32);
                    a1 += (uint64_t)__shfl_xor((unsigned long long)a1, 32);
                }
            }
            if (par == 0) {
                unsigned long long* out = acc + (size_t)(h0 + h) * HD + 2 * dp;
                atomicAdd(out, (unsigned long long)a0);
                atomicAdd(out + 1, (unsigned long long)a1);
            }
        }
    }
}

}  // namespace myl
