// wave.h -- exact wave-level integer reductions on CDNA data-parallel
// primitives (DPP) instead of LDS permutes.
//
// A 16-lane row is summed with four DPP moves (quad_perm xor 1, quad_perm
// xor 2, row_half_mirror, row_mirror): after the two quad steps every lane of
// a quad holds the quad sum; the half-row mirror pairs quad 0 with quad 1,
// the row mirror pairs the two half rows, so every lane of the row ends with
// the row total.  The four row totals are then read with v_readlane (lanes 0,
// 16, 32, 48) and added in scalar registers: the result is wave-uniform.
// All additions wrap (two's complement), so a sum whose true value fits the
// type is exact whatever the order.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace myl {

namespace dpp {
constexpr int kXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141; // row_half_mirror
constexpr int kMirror = 0x140;     // row_mirror
}  // namespace dpp

template <int CTRL>
__device__ inline int32_t dpp_mov(int32_t v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, true);
}

// Every lane of each 16-lane row receives the row's wrapping sum.
__device__ inline int32_t row_sum16_i32(int32_t v) {
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kXor1>(v));
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kXor2>(v));
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kHalfMirror>(v));
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kMirror>(v));
    return v;
}

__device__ inline uint64_t dpp_add64_step_lo_hi(uint64_t v, int32_t lo, int32_t hi) {
    return v + (((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

template <int CTRL>
__device__ inline uint64_t dpp_add64(uint64_t v) {
    const int32_t lo = dpp_mov<CTRL>((int32_t)(uint32_t)v);
    const int32_t hi = dpp_mov<CTRL>((int32_t)(uint32_t)(v >> 32));
    return dpp_add64_step_lo_hi(v, lo, hi);
}

__device__ inline uint64_t row_sum16_u64(uint64_t v) {
    v = dpp_add64<dpp::kXor1>(v);
    v = dpp_add64<dpp::kXor2>(v);
    v = dpp_add64<dpp::kHalfMirror>(v);
    v = dpp_add64<dpp::kMirror>(v);
    return v;
}

__device__ inline int32_t readlane_i32(int32_t v, int lane) { return __builtin_amdgcn_readlane(v, lane); }

__device__ inline uint64_t readlane_u64(uint64_t v, int lane) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)v, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int32_t)(uint32_t)(v >> 32), lane);
    return ((uint64_t)hi << 32) | lo;
}

// Wave-uniform wrapping sum of one int32 per lane (all 64 lanes active).
__device__ inline int32_t wave_sum_i32(int32_t v) {
    v = row_sum16_i32(v);
    return (int32_t)((uint32_t)readlane_i32(v, 0) + (uint32_t)readlane_i32(v, 16) + (uint32_t)readlane_i32(v, 32) +
                     (uint32_t)readlane_i32(v, 48));
}

// Wave-uniform wrapping sum of one 64-bit value per lane (all 64 lanes active).
__device__ inline uint64_t wave_sum_u64(uint64_t v) {
    v = row_sum16_u64(v);
    return readlane_u64(v, 0) + readlane_u64(v, 16) + readlane_u64(v, 32) + readlane_u64(v, 48);
}

__device__ inline int64_t wave_sum_i64(int64_t v) { return (int64_t)wave_sum_u64((uint64_t)v); }

// Every lane of each 8-lane half row receives the half row's wrapping sum.
__device__ inline int32_t row_sum8_i32(int32_t v) {
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kXor1>(v));
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kXor2>(v));
    v = (int32_t)((uint32_t)v + (uint32_t)dpp_mov<dpp::kHalfMirror>(v));
    return v;
}

// Wave-uniform signed maximum of one int32 per lane (all lanes active).
__device__ inline int32_t wave_max_i32(int32_t v) {
    v = max(v, dpp_mov<dpp::kXor1>(v));
    v = max(v, dpp_mov<dpp::kXor2>(v));
    v = max(v, dpp_mov<dpp::kHalfMirror>(v));
    v = max(v, dpp_mov<dpp::kMirror>(v));
    return max(max(readlane_i32(v, 0), readlane_i32(v, 16)), max(readlane_i32(v, 32), readlane_i32(v, 48)));
}

// Block-wide maximum / wrapping sum for blocks of up to 16 waves; red needs
// one slot per wave.  Every thread gets the result: after the barrier each
// wave reads the slots in parallel (lane l, slot l) and reduces them again
// with DPP, instead of one LDS read and wait per slot.
__device__ inline int32_t block_max_i32_dpp(int32_t v, int32_t* red) {
    v = wave_max_i32(v);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6, l = threadIdx.x & 63;
    if (l == 0) red[w] = v;
    __syncthreads();
    return wave_max_i32(l < nw ? red[l] : INT32_MIN);
}

__device__ inline uint32_t block_sum_u32_dpp(uint32_t v, uint32_t* red) {
    v = (uint32_t)wave_sum_i32((int32_t)v);
    const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6, l = threadIdx.x & 63;
    if (l == 0) red[w] = v;
    __syncthreads();
    return (uint32_t)wave_sum_i32(l < nw ? (int32_t)red[l] : 0);
}

template <int CTRL>
__device__ inline uint64_t dpp_max64(uint64_t v) {
    const uint32_t lo = (uint32_t)dpp_mov<CTRL>((int32_t)(uint32_t)v);
    const uint32_t hi = (uint32_t)dpp_mov<CTRL>((int32_t)(uint32_t)(v >> 32));
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    return o > v ? o : v;
}

// Wave-uniform unsigned maximum of one 64-bit value per lane (all lanes active).
__device__ inline uint64_t wave_max_u64(uint64_t v) {
    v = dpp_max64<dpp::kXor1>(v);
    v = dpp_max64<dpp::kXor2>(v);
    v = dpp_max64<dpp::kHalfMirror>(v);
    v = dpp_max64<dpp::kMirror>(v);
    uint64_t m = readlane_u64(v, 0);
    for (int l = 16; l < 64; l += 16) {
        const uint64_t o = readlane_u64(v, l);
        m = o > m ? o : m;
    }
    return m;
}

}  // namespace myl
