// qk_planes.h -- exact attention scores of a KV head's query heads at 16
// positions per wave on the int8 matrix cores (attention.rs:66-67), shared by
// the decode-batch rows (rows_dec.h) and the batch-1 decode step.
#pragma once

#include "bufload.h"
#include "fixed.h"
#include "gemm_mfma.h"

namespace myl {

// A block-uniform pointer kept in scalar registers: a descriptor built from a
// copy in vector registers makes every buffer load a loop over the lanes.
template <class T>
__device__ inline const T* uniform_ptr(const T* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return reinterpret_cast<const T*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}

// Sum of the eight int16 values of a 16-byte chunk.
__device__ inline int32_t sum8_i16(const uint4 x) {
    const uint32_t w[4] = {x.x, x.y, x.z, x.w};
    int32_t s = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) s += (int32_t)(int16_t)(w[i] & 0xFFFFu) + (int32_t)(int16_t)(w[i] >> 16);
    return s;
}

// Exact scores z_j = (i32)RNE(q . k_j * mult, shift) (attention.rs:66-67) of
// the G < 16 query heads sharing a KV head at the 16 positions j0 .. j0 + 15,
// by one wave on v_mfma_i32_16x16x64_i8: lane l holds position (column)
// l % 16 and query head (row) l % 16, each the 16-dimension block l / 16 of
// every 64-dimension step, split into byte planes x = 256 hi + lo' + 128
// (lo' = lo - 128), so
//   q . k = 65536 hh + 256 (hl + lh) + ll + 128 sum(q) + 128 sum(k) - 16384 HD
// with hh = sum(q_hi k_hi) and so on, every plane sum exact in i32 (at most
// 2^15 HD in magnitude).  Rows G .. 14 of the query tile are padding; row 15
// holds ones, so the hh and ll products' row 15 are sum(k_hi) and sum(k_lo')
// of each position, which give sum(k) = 256 sum(k_hi) + sum(k_lo') + 128 HD.
// kg: the KV head's K rows (block-uniform), L of them readable (loads past
// them read zero); qg: the G query vectors, contiguous; scores of head h at
// z[h * zld + j] for j < L.
template <int HD>
__device__ inline void qk_planes_wave(int L, int j0, const int16_t* kg, const int16_t* qg, int G, int64_t score_mult,
                                      uint8_t score_shift, int32_t* __restrict__ z, size_t zld) {
    constexpr int NS = HD / 64;  // 64-dimension steps
    const int lane = threadIdx.x & 63;
    const int c = lane & 15, kb = lane >> 4;
    const int j = j0 + c;
    const __amdgpu_buffer_rsrc_t rk = weight_rsrc(uniform_ptr(kg), (uint32_t)L * HD * 2u);
    // rows G and beyond read zero
    const __amdgpu_buffer_rsrc_t rq = weight_rsrc(uniform_ptr(qg), (uint32_t)G * HD * 2u);
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
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        // lane l holds rows (heads) 4 (l / 16) + rr of column (position) l % 16
        const int h = 4 * kb + rr;
        const int32_t qs = __shfl(qsum, h, 64);
        if (h < G && j < L) {
            const int64_t dot = 65536 * (int64_t)hh[rr] + 256 * (int64_t)mid[rr] + (int64_t)ll[rr] +
                                128 * (int64_t)qs + kterm;
            z[(size_t)h * zld + j] = (int32_t)rshift_round64(wmul64(dot, score_mult), score_shift);
        }
    }
}

}  // namespace myl
