// rows_dec.h -- attention of decode batches (attention.rs:42-90 with
// softmax.rs:12-64 per row): each row attends its own sequence's KV cache up
// to its position, and a block covers one (row, KV head, position range) for
// the G query heads that share the KV head, so the range's K or V rows are
// read once for all of them.
//   rows_dec_qk_kernel   scores[row][head][j] = (i32)RNE(q . k_j * mult, shift)
//                        (attention.rs:66-67), 64-position chunks
//   rows_probs_kernel    (batch.hip) the probabilities, as for row tiles
//   rows_dec_pv_kernel   part[range][row][q dim] = sum_j p_j v_j over the
//                        range's 256 positions, the layout rows_pv_kernel
//                        writes and rows_attn_out_kernel sums
// The row tiles of rows_qk_kernel / rows_pv_kernel put up to 32 rows of one
// sequence on the matrix cores; a decode batch has one row per sequence, so
// those tiles run nearly empty and re-read each row's cache per tile.
#pragma once

#include "bufload.h"
#include "dec_attn.h"
#include "rows_attn.h"

namespace myl {

// A block-uniform pointer kept in scalar registers: a descriptor built from a
// copy in vector registers makes every buffer load a loop over the lanes.
template <class T>
__device__ inline const T* uniform_ptr(const T* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const T*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// Grid (ceil(lmax / kChunk), KV heads, rows); 256 threads.  Chunks at or
// past a row's length return at once.  A wave takes 16 positions on
// v_mfma_i32_16x16x64_i8: lane l holds position (column) l % 16 and query
// head (row) l % 16, each the 16-dimension block l / 16 of every 64-dimension
// step, split into byte planes x = 256 hi + lo' + 128 (lo' = lo - 128), so
//   q . k = 65536 hh + 256 (hl + lh) + ll + 128 sum(q) + 128 sum(k) - 16384 HD
// with hh = sum(q_hi k_hi) and so on, every plane sum exact in i32 (at most
// 2^15 HD in magnitude).  Rows G .. 14 of the query tile are padding; row 15
// holds ones, so the hh and ll products' row 15 are sum(k_hi) and sum(k_lo')
// of each position, which give sum(k) = 256 sum(k_hi) + sum(k_lo') + 128 HD.
// Loads past the row's length read zero (the K descriptor ends there).
template <int HD, int G>
__global__ __launch_bounds__(256) void rows_dec_qk_kernel(const int32_t* __restrict__ rows, int rows_cap,
                                                          const int16_t* __restrict__ Q, int nq,
                                                          const int16_t* __restrict__ kc, size_t seq_stride,
                                                          int max_pos, int64_t score_mult, uint8_t score_shift,
                                                          int32_t* __restrict__ scores, int heads, int lcap) {
    static_assert(G < 16, "row 15 of the query tile holds the ones of the K sums");
    static_assert(kChunk == 64, "four waves of 16 positions");
    constexpr int NS = HD / 64;  // 64-dimension steps
    const int r = blockIdx.z, g = blockIdx.y, base = blockIdx.x * kChunk;
    const int L = __builtin_amdgcn_readfirstlane(rows[rows_cap + r] + 1);
    if (base >= L) return;
    const int seq = __builtin_amdgcn_readfirstlane(rows[r]);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int c = lane & 15, kb = lane >> 4;
    const int j = base + 16 * wave + c;
    const __amdgpu_buffer_rsrc_t rk = weight_rsrc(uniform_ptr(kc + (size_t)seq * seq_stride + (size_t)g * max_pos * HD),
                                                  (uint32_t)L * HD * 2u);
    // the G query vectors are contiguous in the row's q; rows G and beyond read zero
    const __amdgpu_buffer_rsrc_t rq = weight_rsrc(uniform_ptr(Q + (size_t)r * nq + (size_t)g * G * HD), G * HD * 2u);
    uint4 kx[NS][2], qx[NS][2];
#pragma unroll
    for (int s = 0; s < NS; ++s)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const uint32_t d = 64u * s + 16u * kb + 8u * t;
            kx[s][t] = cload16(rk, ((uint32_t)j * HD + d) * 2u);
            qx[s][t] = cload16(rq, ((uint32_t)c * HD + d) * 2u);
        }
    v4i32_t ah[NS], al[NS], bh[NS], bl[NS];
    int32_t qsum = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        uint2 h0, l0, h1, l1;
        split_planes8(kx[s][0], h0, l0);
        split_planes8(kx[s][1], h1, l1);
        bh[s] = v4i32_t{(int)h0.x, (int)h0.y, (int)h1.x, (int)h1.y};
        bl[s] = v4i32_t{(int)l0.x, (int)l0.y, (int)l1.x, (int)l1.y};
        split_planes8(qx[s][0], h0, l0);
        split_planes8(qx[s][1], h1, l1);
        const bool ones = c == 15;
        const int one4 = 0x01010101;
        ah[s] = ones ? v4i32_t{one4, one4, one4, one4} : v4i32_t{(int)h0.x, (int)h0.y, (int)h1.x, (int)h1.y};
        al[s] = ones ? v4i32_t{one4, one4, one4, one4} : v4i32_t{(int)l0.x, (int)l0.y, (int)l1.x, (int)l1.y};
        qsum += sum8_i16(qx[s][0]) + sum8_i16(qx[s][1]);
    }
    v4i32_t hh = {0, 0, 0, 0}, mid = {0, 0, 0, 0}, ll = {0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        hh = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[s], bh[s], hh, 0, 0, 0);
        mid = __builtin_amdgcn_mfma_i32_16x16x64_i8(ah[s], bl[s], mid, 0, 0, 0);
        mid = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[s], bh[s], mid, 0, 0, 0);
        ll = __builtin_amdgcn_mfma_i32_16x16x64_i8(al[s], bl[s], ll, 0, 0, 0);
    }
    // head c's sum over the four dimension blocks, then sum(k) of column c
    // from row 15 (register 3 of lanes 48-63)
    qsum += __shfl_xor(qsum, 16, 64);
    qsum += __shfl_xor(qsum, 32, 64);
    const int32_t ksum = __shfl(256 * hh[3] + ll[3] + 128 * HD, 48 + c, 64);
    const int64_t kterm = 128 * (int64_t)ksum - 16384 * (int64_t)HD;
    int32_t* z = scores + ((size_t)r * heads + (size_t)g * G) * lcap;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        // lane l holds rows (heads) 4 (l / 16) + rr of column (position) l % 16
        const int h = 4 * kb + rr;
        const int32_t qs = __shfl(qsum, h, 64);
        if (h < G && j < L) {
            const int64_t dot = 65536 * (int64_t)hh[rr] + 256 * (int64_t)mid[rr] + (int64_t)ll[rr] +
                                128 * (int64_t)qs + kterm;
            z[(size_t)h * lcap + j] = (int32_t)rshift_round64(wmul64(dot, score_mult), score_shift);
        }
    }
}

// Grid (ceil(lmax / kAttnRange), KV heads, rows); 256 threads.  Thread t holds
// the dimension pair t % (HD / 2) of the positions of stream t / (HD / 2);
// the G heads' probabilities of the range sit in LDS (zero at L and beyond).
// The sums are exact in i32: the probabilities are non-negative (the row path
// admits only a non-negative exp table whose sums do not wrap) and a range's
// add up to at most 2^14 + 128 (each rounding adds at most 1/2), so any
// partial sum is below (2^14 + 128) 2^15 < 2^30 in magnitude.
template <int HD, int G>
__global__ __launch_bounds__(256) void rows_dec_pv_kernel(const int32_t* __restrict__ rows, int rows_cap,
                                                          const int16_t* __restrict__ probs, int heads, int lcap,
                                                          const int16_t* __restrict__ vc, size_t seq_stride,
                                                          int max_pos, int64_t* __restrict__ part, size_t part_stride,
                                                          int nq) {
    constexpr int TPR = HD / 2;                // threads per V row (one dimension pair each)
    constexpr int STREAMS = 256 / TPR;         // position streams per block
    constexpr int PER = kAttnRange / STREAMS;  // positions per stream
    constexpr int PIECES = G * kAttnRange / 8; // 16-byte pieces of the G probability rows
    static_assert(PIECES <= 256, "one probability piece per thread");
    __shared__ __align__(16) int16_t ps[G][kAttnRange];
    __shared__ int32_t red[STREAMS][G][HD];
    const int r = blockIdx.z, g = blockIdx.y, j0 = blockIdx.x * kAttnRange;
    const int L = __builtin_amdgcn_readfirstlane(rows[rows_cap + r] + 1);
    if (j0 >= L) return;
    const int seq = __builtin_amdgcn_readfirstlane(rows[r]);  // the V descriptor lives in scalar registers
    const int tid = threadIdx.x, dp = tid % TPR, stream = tid / TPR;
    // the probabilities first (needed first), then the V rows; rows at L
    // and beyond read zero (past the descriptor's range)
    uint4 pw = make_uint4(0, 0, 0, 0);
    const int ph = tid / (kAttnRange / 8), pc = tid % (kAttnRange / 8);
    if (tid < PIECES)  // within the row's lcap entries (lcap is a multiple of kAttnRange)
        pw = *reinterpret_cast<const uint4*>(probs + ((size_t)r * heads + (size_t)g * G + ph) * lcap + j0 + pc * 8);
    const __amdgpu_buffer_rsrc_t rv = weight_rsrc(uniform_ptr(vc + (size_t)seq * seq_stride + (size_t)g * max_pos * HD),
                                                  (uint32_t)L * HD * 2u);
    uint32_t vv[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) vv[i] = cload4(rv, ((uint32_t)(j0 + stream * PER + i) * HD + 2 * dp) * 2u);
    if (tid < PIECES) {
        // entries at L and beyond are not probabilities of this row
        uint32_t w[4] = {pw.x, pw.y, pw.z, pw.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (j0 + pc * 8 + e >= L) w[e >> 1] &= (e & 1) ? 0x0000FFFFu : 0xFFFF0000u;
        *reinterpret_cast<uint4*>(&ps[ph][pc * 8]) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    __syncthreads();
    // positions in pairs, once for all heads: wl[k] = (v_2k[2 dp], v_2k+1[2 dp]),
    // wh[k] the same of dimension 2 dp + 1, against the heads' probability
    // pairs on v_dot2_i32_i16
    uint32_t wl[PER / 2], wh[PER / 2];
#pragma unroll
    for (int k = 0; k < PER / 2; ++k) {
        wl[k] = __builtin_amdgcn_perm(vv[2 * k + 1], vv[2 * k], 0x05040100u);
        wh[k] = __builtin_amdgcn_perm(vv[2 * k + 1], vv[2 * k], 0x07060302u);
    }
    typedef short __attribute__((ext_vector_type(2))) s2;
    auto d2 = [](uint32_t a, uint32_t c, int32_t acc) {
        return __builtin_amdgcn_sdot2(__builtin_bit_cast(s2, a), __builtin_bit_cast(s2, c), acc, false);
    };
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const uint32_t* pp = reinterpret_cast<const uint32_t*>(&ps[h][stream * PER]);
        int32_t a0 = 0, a1 = 0;
#pragma unroll
        for (int k = 0; k < PER / 2; ++k) {
            a0 = d2(wl[k], pp[k], a0);
            a1 = d2(wh[k], pp[k], a1);
        }
        red[stream][h][2 * dp] = a0;
        red[stream][h][2 * dp + 1] = a1;
    }
    __syncthreads();
    int64_t* out = part + (size_t)blockIdx.x * part_stride + (size_t)r * nq + (size_t)g * G * HD;
    for (int i = tid; i < G * HD; i += 256) {
        const int h = i / HD, d = i % HD;
        int32_t sum = 0;
#pragma unroll
        for (int k = 0; k < STREAMS; ++k) sum += red[k][h][d];
        out[i] = sum;
    }
}

}  // namespace myl
