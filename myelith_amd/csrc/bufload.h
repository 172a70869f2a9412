// bufload.h -- loads through raw buffer descriptors (gfx9-family dword 3).
//
// A load whose byte offset is at or past the descriptor's num_records
// returns zero in hardware, so an out-of-range slot needs no predicate: the
// loads stay straight-line code, and the compiler's in-order vmcnt
// accounting can wait for an early load while later ones are still in
// flight (a load under a branch makes the wait before the first use of any
// earlier load a wait for all of them).  Unlike plain loads from read-only
// kernel arguments, buffer loads keep their program order around
// __builtin_amdgcn_sched_barrier, so a kernel can issue what it needs first
// ahead of what it needs last.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace myl {

__device__ inline __amdgpu_buffer_rsrc_t weight_rsrc(const void* p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Cached loads (cache policy 0) of operands.
constexpr int kPreCpol = 0;
__device__ inline uint4 cload16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, kPreCpol);
    return make_uint4((uint32_t)v[0], (uint32_t)v[1], (uint32_t)v[2], (uint32_t)v[3]);
}
__device__ inline uint2 cload8(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, kPreCpol);
    return make_uint2((uint32_t)v[0], (uint32_t)v[1]);
}
__device__ inline uint32_t cload4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, kPreCpol);
}

}  // namespace myl
