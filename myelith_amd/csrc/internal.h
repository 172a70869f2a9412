// internal.h -- launchers shared between the kernel TUs and the C-ABI layer.
// All pointers are device pointers; lengths are validated by the caller.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace myl {

// Matrix-core (M > 1) launch context: the device's CU count and an i64
// split-K accumulator of acc_elems entries that is all zeros between calls
// (the split-K epilogue clears what it reads).  acc may be null: the
// products then run without K splitting.
struct MmCtx {
    unsigned long long* acc = nullptr;
    size_t acc_elems = 0;
    int cus = 256;
    // byte planes of the activations for the large-M product (gemm_mfma2.h);
    // null or too small: that product is not used
    int8_t* planes = nullptr;
    size_t planes_bytes = 0;
};

// y[m][r] = clamp_i16(rescale_i64(W[r].x[m], w_shifts[r] + act_frac, out_frac_pc ? out_frac_pc[r] : out_frac))
hipError_t linear_w8a16(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const uint8_t* w_shifts,
                        uint8_t act_frac, uint8_t out_frac, const uint8_t* out_frac_pc, int16_t* out, int ldo,
                        hipStream_t st,
                        const MmCtx* mm = nullptr);
hipError_t read_probe(const void* p, size_t bytes, uint32_t* out, int cus, hipStream_t st);
hipError_t linear_w8a16_mult(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const int32_t* mult,
                             const uint8_t* shift, int16_t* out, int ldo, hipStream_t st,
                        const MmCtx* mm = nullptr);
hipError_t logits_w8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, const uint8_t* row_shifts,
                     uint8_t norm_frac, uint8_t logit_frac, int32_t* out, int ldo, hipStream_t st,
                        const MmCtx* mm = nullptr);
hipError_t logits_w16(const int16_t* x, int M, int ldx, const int16_t* W, int N, int K, const uint8_t* row_shifts,
                      uint8_t norm_frac, uint8_t logit_frac, int32_t* out, int ldo, hipStream_t st,
                        const MmCtx* mm = nullptr);
hipError_t dot_raw_w8(const int16_t* x, int M, int ldx, const int8_t* W, int N, int K, int64_t* out, int ldo,
                      hipStream_t st,
                        const MmCtx* mm = nullptr);
hipError_t rmsnorm(const int16_t* x, int M, int ldx, const uint8_t* xs, const int8_t* g, const uint8_t* gs, int n,
                   const int16_t* lut, int lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                   int64_t inv_n_q20, uint8_t out_frac, int16_t* out, int ldo, hipStream_t st);
hipError_t softmax(const int32_t* z, int M, int n, int ldz, const int16_t* lut, int lut_len, uint8_t lut_shift,
                   uint8_t frac_bits, int32_t* out, int ldo, hipStream_t st);
// scratch: 2 * q_len * kv_len int32
hipError_t attention_generic(const int16_t* q, const int16_t* k, const int16_t* v, const uint8_t* mask, int q_len,
                             int kv_len, int hd, int64_t score_mult, uint8_t score_shift, const int16_t* lut,
                             int lut_len, uint8_t lut_shift, uint8_t prob_frac, int32_t* scratch, int16_t* out,
                             hipStream_t st);
// rows[i] = positions[i] % n_pos (computed by the caller)
hipError_t rope(int16_t* q, int16_t* k, int n, int hd, const int16_t* cos_lut, const int16_t* sin_lut,
                const int32_t* rows, uint8_t frac_bits, hipStream_t st);
hipError_t add_bias(int16_t* out, const int16_t* b, const uint8_t* bs, int n, uint8_t out_frac, hipStream_t st);
hipError_t silu_gate(const int16_t* gate, const int16_t* up, int n, const int16_t* silu, int silu_len,
                     uint8_t gate_frac, uint8_t up_frac, uint8_t down_in_frac, uint8_t silu_in_frac, int16_t silu_off,
                     uint8_t silu_out_frac, int16_t* h, hipStream_t st);
hipError_t argmax(const int32_t* v, int M, int n, int ldv, int64_t* out, hipStream_t st);
hipError_t sample_cdf(const int32_t* z, int M, int n, int ldz, const uint64_t* states, int64_t* tokens,
                      uint64_t* new_states, hipStream_t st);
// RMSNorm rows written as byte planes [2M x n] (hi row 2m, lo' row 2m + 1) for
// the int8 products; rows of up to rmsnorm_planes_ok(n) elements.
bool rmsnorm_planes_ok(int n);
hipError_t rmsnorm_planes(const int16_t* x, int M, int ldx, const uint8_t* xs, const int8_t* g, const uint8_t* gs,
                          int n, const int16_t* lut, int lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac,
                          int64_t inv_n_q20, uint8_t out_frac, int8_t* planes, hipStream_t st);
// The same over long rows with more blocks: per-chunk maxima into part
// [M][ceil(n / kArgChunk)], then one reduction per row.
constexpr int kArgChunk = 8192;
hipError_t argmax_rows(const int32_t* v, int M, int n, int ldv, int64_t* out, uint64_t* part, hipStream_t st);
// build-defined integer log-softmax at a target per row (Q16)
hipError_t logsoftmax(const int32_t* z, int M, int n, int ldz, const int16_t* lut, int lut_len, const int64_t* targets,
                      int64_t* out, hipStream_t st);

}  // namespace myl
