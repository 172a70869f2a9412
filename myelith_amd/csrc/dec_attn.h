// dec_attn.h -- integer attention of one query row per KV cache
// (attention.rs:42-90 with softmax.rs:12-64): the decode step's attention.
//
// Two kernels per layer:
//   scores  (query head, kChunk positions): z_j = (i32)RNE(q . k_j * mult, shift)
//   P.V     (query head, kPvWide positions): the head's max and exp-LUT sum
//           over all L scores, the chunk's probabilities, and the exact
//           partial sum_j p_j v_j of the chunk added to the output with one
//           atomic per dim.
// The query heads of a KV head (GQA, model.rs:508-511) run back to back on
// one XCD, so a chunk's K or V rows come from HBM once into that L2.
// dec_pv_wide accumulates in i32, which is exact when every exp-table entry
// is non-negative: then 0 <= p_j <= 2^14 and sum_j p_j <= 2^14 + L/2, so
// |sum_j p_j v_j| < 2^31 for L <= 65536 and wrapping partial sums add up to
// the exact total.  Other tables take dec_pv (kChunk positions, i64).
#pragma once

#include "bufload.h"
#include "ops.h"
#include "wave.h"

namespace myl {

constexpr int kChunk = 64;  // attention positions per block

// int16 pairs -> (hi pair, lo pair) with v = 256 * hi + lo, lo in [0, 255].
__device__ inline void split_pair(uint32_t v, uint32_t& hi, uint32_t& lo) {
    const int32_t a = (int16_t)(v & 0xFFFFu), b = (int16_t)(v >> 16);
    hi = ((uint32_t)(uint16_t)(int16_t)(a >> 8)) | ((uint32_t)(uint16_t)(int16_t)(b >> 8) << 16);
    lo = (v & 0x00FF00FFu);
}

// The K rows of one chunk as dec_scores holds them: LPP = HD / 8 lanes hold
// 16 bytes of a K row each (a wave reads whole rows, coalesced), the wave's
// kChunk / 4 positions in STEPS steps of PPW rows.
template <int HD>
struct DecK {
    static constexpr int LPP = HD / 8;
    static constexpr int PPW = 64 / LPP;              // positions per wave per step
    static constexpr int STEPS = kChunk / 4 / PPW;    // steps per wave
    static_assert(LPP == 8 || LPP == 16, "row sums cover 8 or 16 lanes");
    uint4 kv[STEPS];
    __device__ static int sub() { return (threadIdx.x & 63) % LPP; }
    __device__ static int pos(int base, int it) {
        return base + (int)(threadIdx.x >> 6) * (kChunk / 4) + it * PPW + (int)(threadIdx.x & 63) / LPP;
    }
    __device__ inline void load(int L, int base, const int16_t* __restrict__ kg) {
#pragma unroll
        for (int it = 0; it < STEPS; ++it) {
            const int j = pos(base, it);
            kv[it] = j < L ? *reinterpret_cast<const uint4*>(kg + (size_t)j * HD + sub() * 8) : make_uint4(0, 0, 0, 0);
        }
    }
    // z_j for the held rows j < L and one head's query piece qv (the lane's
    // 16 bytes of q): q . k is exact as 256 * sum(k * q_hi) + sum(k * q_lo) on
    // v_dot2_i32_i16 (|partials| < 2^31), the row sums over the LPP lanes are
    // DPP moves
    __device__ inline void scores(int L, int base, uint4 qv, int64_t score_mult, uint8_t score_shift,
                                  int32_t* __restrict__ z) const {
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
        for (int it = 0; it < STEPS; ++it) {
            const int j = pos(base, it);
            int32_t ahi = 0, alo = 0;
            ahi = d2(kv[it].x, qh.x, ahi);
            ahi = d2(kv[it].y, qh.y, ahi);
            ahi = d2(kv[it].z, qh.z, ahi);
            ahi = d2(kv[it].w, qh.w, ahi);
            alo = d2(kv[it].x, ql.x, alo);
            alo = d2(kv[it].y, ql.y, alo);
            alo = d2(kv[it].z, ql.z, alo);
            alo = d2(kv[it].w, ql.w, alo);
            if (LPP == 16) {
                ahi = row_sum16_i32(ahi);
                alo = row_sum16_i32(alo);
            } else {
                ahi = row_sum8_i32(ahi);
                alo = row_sum8_i32(alo);
            }
            if (sub() == 0 && j < L) {
                const int64_t dot = (int64_t)ahi * 256 + (int64_t)alo;
                z[j] = (int32_t)rshift_round64(wmul64(dot, score_mult), score_shift);
            }
        }
    }
};

// z_j = (i32)RNE(q . k_j * mult, shift) for j in [base, min(base + kChunk, L))
// (attention.rs:66-67); q is one head's vector, kg the KV head's K rows, z
// the head's score row.  256 threads.
template <int HD>
__device__ inline void dec_scores(int L, int base, const int16_t* __restrict__ q, const int16_t* __restrict__ kg,
                                  int64_t score_mult, uint8_t score_shift, int32_t* __restrict__ z) {
    DecK<HD> k;
    k.load(L, base, kg);
    const uint4 qv = *reinterpret_cast<const uint4*>(q + DecK<HD>::sub() * 8);
    k.scores(L, base, qv, score_mult, score_shift, z);
}

// Exp-table entries a P.V block can hold in LDS (8 KB).
constexpr int kDecExpLds = 4096;

// V pairs of one chunk: threads TPR per V row (one dimension pair each), the
// rows of the chunk dealt over STREAMS position streams.
template <int HD>
struct DecV {
    static constexpr int TPR = HD / 2;           // threads per V row (one dim pair each)
    static constexpr int STREAMS = 256 / TPR;    // position streams per block
    static constexpr int PER = kChunk / STREAMS; // positions per stream
    uint32_t vv[PER];
};

// Rows at L and beyond (past the descriptor's range) read zero.
template <int HD>
__device__ inline void dec_load_v(int L, int base, const int16_t* __restrict__ vg, DecV<HD>& v) {
    const int dp = threadIdx.x % DecV<HD>::TPR, stream = threadIdx.x / DecV<HD>::TPR;
    const __amdgpu_buffer_rsrc_t r = weight_rsrc(vg, (uint32_t)L * HD * 2u);
#pragma unroll
    for (int i = 0; i < DecV<HD>::PER; ++i)
        v.vv[i] = cload4(r, ((uint32_t)(base + stream + i * DecV<HD>::STREAMS) * HD + 2 * dp) * 2u);
}

// The exact partial P.V of one chunk (attention.rs:75-81 with
// softmax.rs:12-64): the head's max m and wrapping exp-LUT sum S over all L
// scores (every block of a head recomputes them; cheap for one row), then
// p_j = RNE(e_j * 2^14 / S) (or the uniform split when S == 0) for the
// chunk's positions and sum_j p_j v_j per dimension in i64, added to
// acc[0 .. HD) with 64-bit atomics (exact, order-free).  exp_lds >= 0: every
// exp-table entry from exp_lds on is zero and entries [0, exp_lds) are read
// from an LDS copy (exp_lds <= kDecExpLds); -1: the table is read in place.
// The table is zero-padded to a multiple of 8 entries; z holds zlen >= L
// entries (a multiple of 4, 16-byte aligned).  Every global load of the
// block is issued before any is used, the table and the scores (needed
// first) ahead of the chunk's V rows, all through buffer descriptors (no
// branch, no clamp: past the range a load reads zero).  Whole block (256
// threads).
template <int HD>
__device__ inline void dec_pv(int L, int base, const int32_t* __restrict__ z, int zlen,
                              const int16_t* __restrict__ vg, const int16_t* __restrict__ lut, uint32_t lut_len,
                              uint8_t lut_shift, int exp_lds, unsigned long long* __restrict__ acc) {
    constexpr int ZV = 4;  // 4-score vectors held in registers per thread (L <= 4096)
    constexpr int LPT = kDecExpLds / 8 / 256;  // 8-entry table pieces per thread
    constexpr int STREAMS = DecV<HD>::STREAMS, PER = DecV<HD>::PER;
    __shared__ int16_t elut[kDecExpLds];
    __shared__ int32_t redm[4];
    __shared__ uint32_t reds[4];
    __shared__ int32_t p[kChunk];
    __shared__ int64_t red[STREAMS][HD];
    const int tid = threadIdx.x;
    const bool lds = exp_lds >= 0;
    // the table's nonzero prefix (pieces past it read zero without a fetch)
    const __amdgpu_buffer_rsrc_t rl = weight_rsrc(lut, lds ? (uint32_t)((exp_lds + 7) & ~7) * 2u : 0u);
    uint4 lv[LPT];
#pragma unroll
    for (int i = 0; i < LPT; ++i) lv[i] = cload16(rl, (uint32_t)(tid + i * 256) * 16u);
    const int32_t lut0 = (int16_t)(cload4(weight_rsrc(lut, ((lut_len + 7u) & ~7u) * 2u), 0) & 0xFFFFu);
    // thread t holds the score vectors t + 256 i (positions 4 (t + 256 i) ..
    // + 3); entries at L and beyond are masked where used
    const bool regs = L <= 1024 * ZV;
    const int nzv = (L + 1023) >> 10;
    const __amdgpu_buffer_rsrc_t rz = weight_rsrc(z, (uint32_t)zlen * 4u);
    int4 zv[ZV];
#pragma unroll
    for (int i = 0; i < ZV; ++i) {
        const uint4 w = cload16(rz, (uint32_t)(tid + 256 * i) * 16u);
        zv[i] = make_int4((int32_t)w.x, (int32_t)w.y, (int32_t)w.z, (int32_t)w.w);
    }
    const int n = min(kChunk, L - base);
    const int32_t zown = (int32_t)cload4(rz, (uint32_t)(base + tid) * 4u);  // used for tid < n
    __builtin_amdgcn_sched_barrier(0);  // the V rows load after all of the above
    DecV<HD> v;
    dec_load_v<HD>(L, base, vg, v);
    // the whole LDS table, unconditionally (a store under a branch would take
    // its load in with it); entries from exp_lds on are never read
#pragma unroll
    for (int i = 0; i < LPT; ++i)
        *reinterpret_cast<uint4*>(elut + (tid + i * 256) * 8) = lv[i];  // read after the max's barrier
    const int32_t lut_one = lut_len > 0 ? lut0 : 1;
    auto zat = [&](int i, int e) { return e == 0 ? zv[i].x : e == 1 ? zv[i].y : e == 2 ? zv[i].z : zv[i].w; };
    int32_t mx = INT32_MIN;
    if (regs) {
#pragma unroll
        for (int i = 0; i < ZV; ++i)
            if (i < nzv) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * (tid + 256 * i) + e < L) mx = max(mx, zat(i, e));
            }
    } else {
        for (int j = tid; j < L; j += 256) mx = max(mx, z[j]);
    }
    mx = block_max_i32_dpp(mx, redm);
    // exp_lookup (softmax.rs:12-20) of the score zj
    auto ex = [&](int32_t zj) -> int32_t {
        const int32_t x = sat_sub32(mx, zj);
        if (x <= 0) return lut_one;
        const uint32_t idx = (uint32_t)x >> (lut_shift & 31u);
        if (lds) return idx < (uint32_t)exp_lds ? (int32_t)elut[idx] : 0;
        return idx < lut_len ? (int32_t)lut[idx] : 0;
    };
    // the same from the LDS copy, straight-line: the table read is issued
    // whatever the entry, then selects (no branch, no wait per entry)
    const uint32_t sh = lut_shift & 31u;
    auto ex_lds = [&](int32_t zj) -> int32_t {
        const int32_t x = sat_sub32(mx, zj);
        const uint32_t idx = (uint32_t)x >> sh;
        const bool in = idx < (uint32_t)exp_lds;
        const int32_t t = elut[in ? idx : 0u];
        return x <= 0 ? lut_one : (in ? t : 0);
    };
    uint32_t s = 0;
    if (regs && lds) {
#pragma unroll
        for (int i = 0; i < ZV; ++i)
            if (i < nzv) {
                // a vector's four table reads issue together, then selects
                int32_t x[4], t[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    x[e] = sat_sub32(mx, zat(i, e));
                    const uint32_t idx = (uint32_t)x[e] >> sh;
                    t[e] = elut[idx < (uint32_t)exp_lds ? idx : 0u];
                }
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const bool in = ((uint32_t)x[e] >> sh) < (uint32_t)exp_lds;
                    const int32_t v = x[e] <= 0 ? lut_one : (in ? t[e] : 0);
                    s += 4 * (tid + 256 * i) + e < L ? (uint32_t)v : 0u;
                }
            }
    } else if (regs) {
#pragma unroll
        for (int i = 0; i < ZV; ++i)
            if (i < nzv) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * (tid + 256 * i) + e < L) s += (uint32_t)ex(zat(i, e));
            }
    } else {
        for (int j = tid; j < L; j += 256) s += (uint32_t)ex(z[j]);
    }
    const int32_t eown = lds ? ex_lds(zown) : ex(zown);  // this entry's numerator, ahead of the sum's barrier
    const int32_t S = (int32_t)block_sum_u32_dpp(s, reds);
    const int dp = tid % DecV<HD>::TPR, stream = tid / DecV<HD>::TPR;
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    if (tid < kChunk) {
        int32_t pv = 0;
        if (tid < n) {
            if (S == 0) {
                const uint64_t rl = recip32((uint32_t)L);
                uint32_t qq, rr;
                udivmod32((uint32_t)one, (uint32_t)L, rl, &qq, &rr);
                const int32_t ubase = (int32_t)qq;
                const int32_t urem = wsub32(one, wmul32(ubase, L));
                pv = ubase + (((uint64_t)(base + tid) < (uint64_t)(int64_t)urem) ? 1 : 0);
            } else {
                const uint64_t rs = recip32(S < 0 ? 0u - (uint32_t)S : (uint32_t)S);
                pv = softmax_div_round(wmul32(eown, one), S, rs);
            }
        }
        p[tid] = pv;
    }
    __syncthreads();
    int64_t a0 = 0, a1 = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i) {
        const int64_t pv = p[stream + i * STREAMS];
        a0 = wadd64(a0, pv * (int64_t)(int16_t)(v.vv[i] & 0xFFFFu));
        a1 = wadd64(a1, pv * (int64_t)(int16_t)(v.vv[i] >> 16));
    }
    red[stream][2 * dp] = a0;
    red[stream][2 * dp + 1] = a1;
    __syncthreads();
    if (tid < HD) {
        int64_t sum = 0;
#pragma unroll
        for (int k = 0; k < STREAMS; ++k) sum = wadd64(sum, red[k][tid]);
        atomicAdd(acc + tid, (unsigned long long)sum);
    }
}

// ---- wide P.V chunks, i32 ----------------------------------------------------

constexpr int kPvWide = 256;  // positions per block of dec_pv_wide

// The exact partial P.V of kPvWide positions for one query head
// (attention.rs:75-81 with softmax.rs:12-64), for exp tables without a
// negative entry whose nonzero prefix fits the LDS copy (exp_lds <=
// kDecExpLds) and L <= 65536.  The block computes the head's max m and
// wrapping exp-LUT sum S over all L scores (every chunk's block recomputes
// them: four or so scores per thread), the chunk's probabilities
// p_j = RNE(e_j 2^14 / S) (the uniform split when S == 0) into LDS, then
// thread (wave w, lane) holds 8 dims of the V rows rg + NRG i of its row
// group rg = RS w + lane / (HD / 8) and takes their products with the
// probabilities on v_dot2_i32_i16, two rows per instruction; the row groups
// are summed in LDS and one 32-bit atomic per dim adds the chunk to acc[0 ..
// HD).  Every global load is issued before any is used, through buffer
// descriptors (past the range a load reads zero).  512 threads.
template <int HD>
__device__ inline void dec_pv_wide(int L, int base, const int32_t* __restrict__ z, int zlen,
                                   const int16_t* __restrict__ vg, const int16_t* __restrict__ lut, uint32_t lut_len,
                                   uint8_t lut_shift, int exp_lds, int32_t* __restrict__ acc) {
    constexpr int C = kPvWide;
    constexpr int OPR = HD / 8;     // lanes per V row, 8 dims each
    constexpr int RS = 64 / OPR;    // rows per wave load
    constexpr int NRG = 8 * RS;     // row groups of the block
    constexpr int PR = C / NRG;     // rows per thread
    constexpr int ZV = 2;           // 4-score vectors per thread in registers (L <= 4096)
    static_assert(PR % 2 == 0 && C <= 512, "row pairs; one probability per thread");
    static_assert(kDecExpLds == 8 * 512, "one 16-byte table piece per thread");
    __shared__ __align__(16) int16_t elut[kDecExpLds];
    __shared__ __align__(16) int16_t plt[NRG][PR];
    __shared__ __align__(16) int32_t red[NRG][HD];
    __shared__ int32_t redm[8];
    __shared__ uint32_t reds[8];
    const int tid = (int)threadIdx.x, lane = tid & 63, w = tid >> 6;
    // loads: the table's nonzero prefix, the scores (all L, and this
    // thread's chunk position), then the chunk's V rows
    const __amdgpu_buffer_rsrc_t rl = weight_rsrc(lut, (uint32_t)((exp_lds + 7) & ~7) * 2u);
    const uint4 lv = cload16(rl, (uint32_t)tid * 16u);
    const int32_t lut0 = (int16_t)(cload4(weight_rsrc(lut, ((lut_len + 7u) & ~7u) * 2u), 0) & 0xFFFFu);
    const __amdgpu_buffer_rsrc_t rz = weight_rsrc(z, (uint32_t)min(zlen, L) * 4u);
    uint4 zv[ZV];
#pragma unroll
    for (int i = 0; i < ZV; ++i) zv[i] = cload16(rz, (uint32_t)(tid + 512 * i) * 16u);
    const int32_t zown = (int32_t)cload4(rz, (uint32_t)(base + tid) * 4u);  // used for tid < C
    __builtin_amdgcn_sched_barrier(0);
    const int oc = lane % OPR, rg = w * RS + lane / OPR;
    const __amdgpu_buffer_rsrc_t rv = weight_rsrc(vg, (uint32_t)L * HD * 2u);
    uint4 vv[PR];
#pragma unroll
    for (int i = 0; i < PR; ++i) vv[i] = cload16(rv, ((uint32_t)(base + rg + NRG * i) * HD + 8 * oc) * 2u);
    *reinterpret_cast<uint4*>(elut + tid * 8) = lv;  // read after the max's barrier
    const int32_t lut_one = lut_len > 0 ? lut0 : 1;
    const uint32_t sh = lut_shift & 31u;
    auto zat = [](const uint4& v, int e) { return (int32_t)(e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w); };
    const bool regs = L <= 2048 * ZV;
    const int nzv = (L + 2047) >> 11;  // score vectors holding positions below L
    int32_t mx = INT32_MIN;
    if (regs) {
#pragma unroll
        for (int i = 0; i < ZV; ++i)
            if (i < nzv) {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (4 * (tid + 512 * i) + e < L) mx = max(mx, zat(zv[i], e));
            }
    } else {
        for (int j = tid; j < L; j += 512) mx = max(mx, z[j]);
    }
    mx = block_max_i32_dpp(mx, redm);  // also makes the table copy visible
    // exp_lookup (softmax.rs:12-20) of a score zj <= mx from the LDS copy:
    // the saturating difference is min(mx - zj, 2^31 - 1) (mx - zj is in
    // [0, 2^32) as an unsigned word), entries from exp_lds on are zero, and
    // the read is issued whatever the entry, then selects
    auto ex = [&](int32_t zj) -> int32_t {
        const uint32_t x = min((uint32_t)mx - (uint32_t)zj, 0x7FFFFFFFu);
        const uint32_t idx = x >> sh;
        const bool in = idx < (uint32_t)exp_lds;
        const int32_t t = elut[in ? idx : 0u];
        return x == 0 ? lut_one : (in ? t : 0);
    };
    uint32_t s = 0;
    if (regs) {
#pragma unroll
        for (int i = 0; i < ZV; ++i)
            if (i < nzv) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t v = (uint32_t)ex(zat(zv[i], e));
                    s += 4 * (tid + 512 * i) + e < L ? v : 0u;
                }
            }
    } else {
        for (int j = tid; j < L; j += 512) s += (uint32_t)ex(z[j]);
    }
    const int32_t eown = ex(zown);  // this thread's numerator (used below L), ahead of the sum's barrier
    // block-uniform: the reciprocal runs on the scalar unit, ahead of the
    // per-thread branch.  S > 0 is a sum of non-negative entries below
    // 2^31; S == 0 takes the uniform split 2^14 = ubase L + urem.
    const int32_t S = __builtin_amdgcn_readfirstlane((int32_t)block_sum_u32_dpp(s, reds));
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    const uint32_t den = S == 0 ? (uint32_t)L : (uint32_t)S;
    const uint32_t rs = recip32_u32(den);
    int32_t ubase = 0, urem = 0;
    if (S == 0) {
        uint32_t qq, rr;
        udivmod32((uint32_t)one, (uint32_t)L, recip32((uint32_t)L), &qq, &rr);
        ubase = (int32_t)qq;
        urem = wsub32(one, wmul32(ubase, L));
    }
    if (tid < C) {
        const int j = base + tid;
        int32_t pv = 0;
        if (j < L)
            pv = S == 0 ? ubase + (((uint64_t)j < (uint64_t)(int64_t)urem) ? 1 : 0)
                        : softmax_div_round_pos(eown << MYL_TV_PROB_FRAC_BITS, S, rs);
        plt[tid % NRG][tid / NRG] = (int16_t)pv;
    }
    __syncthreads();
    typedef short __attribute__((ext_vector_type(2))) s2;
    auto d2 = [](uint32_t a, uint32_t c, int32_t t) {
        return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, c), t, false);
    };
    int32_t a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint32_t* pw = reinterpret_cast<const uint32_t*>(&plt[rg][0]);
#pragma unroll
    for (int k = 0; k < PR / 2; ++k) {
        const uint32_t pp = pw[k];  // probabilities of rows 2k, 2k + 1
        const uint32_t ra[4] = {vv[2 * k].x, vv[2 * k].y, vv[2 * k].z, vv[2 * k].w};
        const uint32_t rb[4] = {vv[2 * k + 1].x, vv[2 * k + 1].y, vv[2 * k + 1].z, vv[2 * k + 1].w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            a[2 * t] = d2(pp, (ra[t] & 0xFFFFu) | (rb[t] << 16), a[2 * t]);
            a[2 * t + 1] = d2(pp, (ra[t] >> 16) | (rb[t] & 0xFFFF0000u), a[2 * t + 1]);
        }
    }
    *reinterpret_cast<int4*>(&red[rg][8 * oc]) = make_int4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<int4*>(&red[rg][8 * oc + 4]) = make_int4(a[4], a[5], a[6], a[7]);
    __syncthreads();
    if (tid < HD) {
        uint32_t t = 0;
#pragma unroll
        for (int r = 0; r < NRG; ++r) t += (uint32_t)red[r][tid];
        atomicAdd(acc + tid, (int)t);
    }
}

// ---- short contexts: one block per query head --------------------------------

// Positions one dec_attn_short block holds: eight 16-byte K and V pieces per
// thread (512 threads, HD / 8 lanes per row).
template <int HD>
constexpr int dec_short_max() { return 8 * 8 * (64 / (HD / 8)); }

// The whole attention of one query head (attention.rs:42-90 with
// softmax.rs:12-64) for L <= dec_short_max<HD>() positions, in one block:
// z_j = (i32)RNE(q . k_j * mult, shift) into LDS, the max m and wrapping
// exp-LUT sum S, p_j = RNE(e_j 2^14 / S) (the uniform split when S == 0),
// and sum_j p_j v_j per dimension stored to out[0 .. HD).  For the tables
// dec_pv_wide takes (no negative entry, nonzero prefix exp_lds <=
// kDecExpLds): the sum is exact in i32.  Thread (wave w, lane) holds the 16
// bytes at dims 8 (lane % (HD / 8)) of K and V rows RPR i + rr (rr = RS w +
// lane / (HD / 8)), i < 8; all K, table and V loads are issued first, in
// that order, through buffer descriptors (rows at L and beyond read zero).
// 512 threads.
template <int HD>
__device__ inline void dec_attn_short(int L, const int16_t* __restrict__ q, const int16_t* __restrict__ kg,
                                      const int16_t* __restrict__ vg, int64_t score_mult, uint8_t score_shift,
                                      const int16_t* __restrict__ lut, uint32_t lut_len, uint8_t lut_shift,
                                      int exp_lds, int32_t* __restrict__ out) {
    constexpr int OPR = HD / 8;        // lanes per row, 8 dims each
    constexpr int RS = 64 / OPR;       // rows per wave load
    constexpr int RPR = 8 * RS;        // rows per block round (also the row groups)
    constexpr int NR = 8;              // rounds
    constexpr int LMAX = RPR * NR;
    static_assert(LMAX == dec_short_max<HD>() && LMAX <= 512, "one score per thread");
    static_assert(kDecExpLds == 8 * 512, "one 16-byte table piece per thread");
    __shared__ __align__(16) int16_t elut[kDecExpLds];
    __shared__ __align__(16) int32_t zs[LMAX];
    __shared__ __align__(16) int16_t plt[RPR][NR];
    __shared__ __align__(16) int32_t red[RPR][HD];
    __shared__ int32_t redm[8];
    __shared__ uint32_t reds[8];
    const int tid = (int)threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int oc = lane % OPR, rr = w * RS + lane / OPR;
    const uint32_t kvbytes = (uint32_t)L * HD * 2u;
    const __amdgpu_buffer_rsrc_t rk = weight_rsrc(kg, kvbytes);
    const __amdgpu_buffer_rsrc_t rv = weight_rsrc(vg, kvbytes);
    const uint4 qv = *reinterpret_cast<const uint4*>(q + 8 * oc);
    uint4 kv[NR], vv[NR];
#pragma unroll
    for (int i = 0; i < NR; ++i) kv[i] = cload16(rk, ((uint32_t)(RPR * i + rr) * HD + 8 * oc) * 2u);
    const __amdgpu_buffer_rsrc_t rl = weight_rsrc(lut, (uint32_t)((exp_lds + 7) & ~7) * 2u);
    const uint4 lv = cload16(rl, (uint32_t)tid * 16u);
    const int32_t lut0 = (int16_t)(cload4(weight_rsrc(lut, ((lut_len + 7u) & ~7u) * 2u), 0) & 0xFFFFu);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NR; ++i) vv[i] = cload16(rv, ((uint32_t)(RPR * i + rr) * HD + 8 * oc) * 2u);
    __builtin_amdgcn_sched_barrier(0);
    // scores: q . k = 256 sum(k q_hi) + sum(k q_lo) on v_dot2_i32_i16
    // (|partials| < 2^31), row sums over the row's OPR lanes by DPP
    uint4 qh, ql;
    split_pair(qv.x, qh.x, ql.x);
    split_pair(qv.y, qh.y, ql.y);
    split_pair(qv.z, qh.z, ql.z);
    split_pair(qv.w, qh.w, ql.w);
    typedef short __attribute__((ext_vector_type(2))) s2;
    auto d2 = [](uint32_t a, uint32_t c, int32_t t) {
        return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, c), t, false);
    };
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        int32_t ahi = 0, alo = 0;
        ahi = d2(kv[i].x, qh.x, ahi);
        ahi = d2(kv[i].y, qh.y, ahi);
        ahi = d2(kv[i].z, qh.z, ahi);
        ahi = d2(kv[i].w, qh.w, ahi);
        alo = d2(kv[i].x, ql.x, alo);
        alo = d2(kv[i].y, ql.y, alo);
        alo = d2(kv[i].z, ql.z, alo);
        alo = d2(kv[i].w, ql.w, alo);
        if (OPR == 16) {
            ahi = row_sum16_i32(ahi);
            alo = row_sum16_i32(alo);
        } else {
            ahi = row_sum8_i32(ahi);
            alo = row_sum8_i32(alo);
        }
        if (oc == 0) {
            const int64_t dot = (int64_t)ahi * 256 + (int64_t)alo;
            zs[RPR * i + rr] = (int32_t)rshift_round64(wmul64(dot, score_mult), score_shift);
        }
    }
    *reinterpret_cast<uint4*>(elut + tid * 8) = lv;
    __syncthreads();  // the scores and the table copy
    const bool live = tid < L;
    const int32_t zj = live ? zs[tid] : INT32_MIN;
    const int32_t mx = block_max_i32_dpp(zj, redm);
    // exp_lookup (softmax.rs:12-20) from the LDS copy, as in dec_pv_wide
    const uint32_t sh = lut_shift & 31u;
    const int32_t lut_one = lut_len > 0 ? lut0 : 1;
    const uint32_t x = min((uint32_t)mx - (uint32_t)zj, 0x7FFFFFFFu);
    const uint32_t idx = x >> sh;
    const bool in = idx < (uint32_t)exp_lds;
    const int32_t t = elut[in ? idx : 0u];
    const int32_t e = live ? (x == 0 ? lut_one : (in ? t : 0)) : 0;
    const int32_t S = __builtin_amdgcn_readfirstlane((int32_t)block_sum_u32_dpp((uint32_t)e, reds));
    const int32_t one = 1 << MYL_TV_PROB_FRAC_BITS;
    const uint32_t den = S == 0 ? (uint32_t)L : (uint32_t)S;
    const uint32_t rs = recip32_u32(den);
    int32_t ubase = 0, urem = 0;
    if (S == 0) {
        uint32_t qq, rr2;
        udivmod32((uint32_t)one, (uint32_t)L, recip32((uint32_t)L), &qq, &rr2);
        ubase = (int32_t)qq;
        urem = wsub32(one, wmul32(ubase, L));
    }
    if (tid < LMAX) {
        int32_t pv = 0;
        if (live)
            pv = S == 0 ? ubase + (((uint64_t)tid < (uint64_t)(int64_t)urem) ? 1 : 0)
                        : softmax_div_round_pos(e << MYL_TV_PROB_FRAC_BITS, S, rs);
        plt[tid % RPR][tid / RPR] = (int16_t)pv;
    }
    __syncthreads();
    // P.V: rows RPR 2k + rr and RPR (2k + 1) + rr per v_dot2
    int32_t a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint32_t* pw = reinterpret_cast<const uint32_t*>(&plt[rr][0]);
#pragma unroll
    for (int k = 0; k < NR / 2; ++k) {
        const uint32_t pp = pw[k];
        const uint32_t ra[4] = {vv[2 * k].x, vv[2 * k].y, vv[2 * k].z, vv[2 * k].w};
        const uint32_t rb[4] = {vv[2 * k + 1].x, vv[2 * k + 1].y, vv[2 * k + 1].z, vv[2 * k + 1].w};
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            a[2 * u] = d2(pp, (ra[u] & 0xFFFFu) | (rb[u] << 16), a[2 * u]);
            a[2 * u + 1] = d2(pp, (ra[u] >> 16) | (rb[u] & 0xFFFF0000u), a[2 * u + 1]);
        }
    }
    *reinterpret_cast<int4*>(&red[rr][8 * oc]) = make_int4(a[0], a[1], a[2], a[3]);
    *reinterpret_cast<int4*>(&red[rr][8 * oc + 4]) = make_int4(a[4], a[5], a[6], a[7]);
    __syncthreads();
    if (tid < HD) {
        uint32_t sum = 0;
#pragma unroll
        for (int r = 0; r < RPR; ++r) sum += (uint32_t)red[r][tid];
        out[tid] = (int32_t)sum;
    }
}

}  // namespace myl
