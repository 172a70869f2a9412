// noalloc.hip -- the W8A16 product for callers that cannot allocate device
// memory (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc): myl_linear_w8a16_dev_noalloc.
//
// The product of two or more activation rows needs scratch: the activations'
// signed byte planes (2 * M * K bytes, gemm_mfma2.h) and, when K is split
// across blocks, the exact i64 partial sums (M * N entries).  Here both live
// in one file-scope device array, `scratch`, of fixed size; every GPU holds its
// own copy from module load until the process ends.  Its device address is
// looked up once per device by myl_init (noalloc_setup, with that device
// current) and kept per device; host code never passes the array's name,
// which on the host is only a stand-in, to a kernel.
//
// Every call on a GPU shares that GPU's copy: calls that overlap on one GPU
// (two streams, two threads, two contexts) race on it and must be ordered by
// the caller.  The accumulator slice a call may use is cleared by a fill
// kernel at the start of each call (no hipMemsetAsync: callers may capture
// the call into a graph).
#include "abi_internal.h"
#include "gemm_dispatch.h"

#include <algorithm>
#include <mutex>
#include <string>
#include <vector>

namespace {

// Byte planes of up to 4 MiB (e.g. 64 rows x K = 32768), then 256 Ki i64
// partial sums (products with more outputs do not split K).
constexpr size_t kPlaneBytes = (size_t)4 << 20;
constexpr size_t kAccElems = (size_t)256 << 10;
constexpr size_t kScratchBytes = kPlaneBytes + kAccElems * 8;

}  // namespace

static __device__ __align__(256) int8_t scratch[kScratchBytes];

namespace {

std::mutex g_mu;
std::vector<void*> g_scratch;  // device index -> address of that device's `scratch`

void* scratch_of(int device) {
    std::lock_guard<std::mutex> lock(g_mu);
    return device >= 0 && (size_t)device < g_scratch.size() ? g_scratch[device] : nullptr;
}

__global__ __launch_bounds__(256) void clear_u64_kernel(unsigned long long* __restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace

namespace myl {

int noalloc_setup(int device) {
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if ((size_t)device < g_scratch.size() && g_scratch[device]) return MYL_OK;
    }
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return MYL_E_HIP;
    std::lock_guard<std::mutex> lock(g_mu);
    if ((size_t)device >= g_scratch.size()) g_scratch.resize((size_t)device + 1, nullptr);
    g_scratch[device] = p;
    return MYL_OK;
}

}  // namespace myl

extern "C" {

size_t myl_noalloc_scratch_bytes(void) { return kScratchBytes; }

int myl_linear_w8a16_dev_noalloc(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N,
                                 size_t K, const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac,
                                 const uint8_t* out_frac_pc, int16_t* out, size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    const char* what = "linear_w8a16_dev_noalloc";
    if (K == 0) return ctx->fail(MYL_E_INVALID, std::string(what) + ": K must be > 0");
    if (ldx < K || ldo < N) return ctx->fail(MYL_E_INVALID, std::string(what) + ": leading dimension too small");
    if (!myl::fits_int(M) || !myl::fits_int(N) || !myl::fits_int(K) || !myl::fits_int(ldx) || !myl::fits_int(ldo))
        return ctx->fail(MYL_E_INVALID, std::string(what) + ": shape too large");
    if (M == 0 || N == 0) return MYL_OK;
    if (M >= 2 && 2 * M * K > kPlaneBytes)
        return ctx->fail(MYL_E_INVALID, std::string(what) + ": 2 * M * K = " + std::to_string(2 * M * K) +
                                            " bytes of activation planes exceed the " +
                                            std::to_string(kPlaneBytes) + "-byte scratch");
    char* base = static_cast<char*>(scratch_of(ctx->device));
    if (!base) return ctx->fail(MYL_E_HIP, std::string(what) + ": the device scratch was not set up by myl_init");
    myl::MmCtx mm;
    mm.cus = ctx->prop.multiProcessorCount > 0 ? ctx->prop.multiProcessorCount : 1;
    mm.planes = reinterpret_cast<int8_t*>(base);
    mm.planes_bytes = kPlaneBytes;
    mm.acc = reinterpret_cast<unsigned long long*>(base + kPlaneBytes);
    mm.acc_elems = kAccElems;
    if (M >= 2) {
        // the split products read this slice as zeros (their finish kernels
        // clear it again, but a call that failed part way may not have)
        const size_t n = std::min(M * N, kAccElems);
        clear_u64_kernel<<<(unsigned)std::min<size_t>((n + 255) / 256, 1024), 256, 0, ctx->stream>>>(mm.acc, n);
        const int rc = ctx->hip(hipGetLastError(), what);
        if (rc) return rc;
    }
    return ctx->hip(myl::linear_w8a16(x, (int)M, (int)ldx, W, (int)N, (int)K, w_shifts, act_frac, out_frac,
                                      out_frac_pc, out, (int)ldo, ctx->stream, &mm),
                    what);
}

}  // extern "C"
