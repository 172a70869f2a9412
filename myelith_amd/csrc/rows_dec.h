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
#include "qk_planes.h"
#include "rows_attn.h"

namespace myl {

// Grid (ceil(lmax / kChunk), KV heads, rows); 256 threads: wave w takes the
// 16 positions from base + 16 w of its row's chunk (qk_planes_wave).  Chunks
// at or past a row's length return at once.
template <int HD, int G>
__global__ __launch_bounds__(256) void rows_dec_qk_kernel(const int32_t* __restrict__ rows, int rows_cap,
                                                          const int16_t* __restrict__ Q, int nq,
                                                          const int16_t* __restrict__ kc, size_t seq_stride,
                                                          int max_pos, int64_t score_mult, uint8_t score_shift,
                                                          int32_t* __restrict__ scores, int heads, int lcap) {
    static_assert(G < 16, "row 15 of the query tile holds the ones of the K sums");
    static_assert(kChunk == 64, "four waves of 16 positions");
    const int r = blockIdx.z, g = blockIdx.y, base = blockIdx.x * kChunk;
    const int L = __builtin_amdgcn_readfirstlane(rows[rows_cap + r] + 1);
    if (base >= L) return;
    const int seq = __builtin_amdgcn_readfirstlane(rows[r]);
    const int wave = threadIdx.x >> 6;
    qk_planes_wave<HD>(L, base + 16 * wave, kc + (size_t)seq * seq_stride + (size_t)g * max_pos * HD,
                       Q + (size_t)r * nq + (size_t)g * G * HD, G, score_mult, score_shift,
                       scores + ((size_t)r * heads + (size_t)g * G) * lcap, (size_t)lcap);
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
