// abi_internal.h -- the context object behind the opaque myl_ctx handle.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "../../include/myl_hip.h"
#include "internal.h"

struct myl_ctx {
    int device = 0;
    hipStream_t stream = nullptr;      // stream of every launch (own_stream or the caller's)
    hipStream_t own_stream = nullptr;
    hipDeviceProp_t prop{};
    std::string err;
    void* scratch_ptr = nullptr;
    size_t scratch_bytes = 0;
    myl::MmCtx mm{};                   // split-K accumulator of the matrix-core path

    int fail(int code, const std::string& msg);
    int hip(hipError_t e, const char* what);
    // Grow-only device scratch for host-slice staging (valid until the next call).
    void* scratch(size_t bytes);
    // The matrix-core launch context with an all-zero accumulator of at least
    // `elems` entries and an activation-plane buffer of at least plane_bytes
    // (both grown on demand within caps; nullptr only when allocation fails).
    const myl::MmCtx* mm_ctx(size_t elems, size_t plane_bytes = 0);
};

namespace myl {

inline bool fits_int(size_t v) { return v <= (size_t)INT32_MAX; }

// Looks up, with `device` current, the device address of the scratch array of
// the allocation-free product (noalloc.hip) once per device.
int noalloc_setup(int device);

}  // namespace myl
