// abi.cpp -- the C ABI of libmyl_hip.so (include/myl_hip.h): context, error
// reporting, device memory, the Backend-trait mirror and the device-pointer
// forms.  Argument checks reproduce the reference's assert!/panic cases as
// MYL_E_INVALID; the arithmetic itself lives in the kernels.
#include "abi_internal.h"

#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

using namespace myl;

// ---------------------------------------------------------------------------
// context and errors
// ---------------------------------------------------------------------------

int myl_ctx::fail(int code, const std::string& msg) {
    err = msg;
    return code;
}

int myl_ctx::hip(hipError_t e, const char* what) {
    if (e == hipSuccess) return MYL_OK;
    err = std::string(what) + ": " + hipGetErrorString(e);
    return MYL_E_HIP;
}

void* myl_ctx::scratch(size_t bytes) {
    bytes = (bytes + 255) & ~(size_t)255;
    if (bytes > scratch_bytes) {
        if (scratch_ptr) {
            (void)hipStreamSynchronize(stream);
            (void)hipFree(scratch_ptr);
        }
        scratch_ptr = nullptr;
        scratch_bytes = 0;
        if (hipMalloc(&scratch_ptr, bytes) != hipSuccess) return nullptr;
        scratch_bytes = bytes;
    }
    return scratch_ptr;
}

// Products with more outputs than this never split K (their tiles alone fill
// the chip), so the accumulator stays at most 32 MiB; a request beyond the
// cap still gets a capped accumulator, which the byte-plane products of
// smaller outputs need.
static constexpr size_t kMmAccCap = (size_t)4 << 20;

// Activation planes beyond this stay with the tiled kernel (1 GiB: 4096
// rows of the widest product, K = 18944, need 155 MiB).
static constexpr size_t kMmPlaneCap = (size_t)1 << 30;

const myl::MmCtx* myl_ctx::mm_ctx(size_t elems, size_t plane_bytes) {
    mm.cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1;
    elems = std::min(elems, kMmAccCap);
    if (elems > mm.acc_elems) {
        (void)hipStreamSynchronize(stream);
        if (mm.acc) (void)hipFree(mm.acc);
        mm.acc = nullptr;
        mm.acc_elems = 0;
        void* p = nullptr;
        if (hipMalloc(&p, elems * 8) != hipSuccess) return nullptr;
        if (hipMemset(p, 0, elems * 8) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
            (void)hipFree(p);
            return nullptr;
        }
        mm.acc = (unsigned long long*)p;
        mm.acc_elems = elems;
    }
    if (plane_bytes > mm.planes_bytes && plane_bytes <= kMmPlaneCap) {
        (void)hipStreamSynchronize(stream);
        if (mm.planes) (void)hipFree(mm.planes);
        mm.planes = nullptr;
        mm.planes_bytes = 0;
        void* p = nullptr;
        if (hipMalloc(&p, plane_bytes) == hipSuccess) {
            mm.planes = (int8_t*)p;
            mm.planes_bytes = plane_bytes;
        }
    }
    return &mm;
}

extern "C" {

const char* myl_backend_name(void) { return "rocm"; }
const char* myl_hardware_family(void) { return "amd-gpu"; }
const char* myl_feature_tag(void) { return "rocm"; }

int myl_init(int device_id, myl_ctx** out) {
    if (!out) return MYL_E_INVALID;
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || device_id < 0 || device_id >= n) return MYL_E_INVALID;
    if (hipSetDevice(device_id) != hipSuccess) return MYL_E_HIP;
    myl_ctx* c = new (std::nothrow) myl_ctx();
    if (!c) return MYL_E_NOMEM;
    c->device = device_id;
    if (hipGetDeviceProperties(&c->prop, device_id) != hipSuccess || hipStreamCreate(&c->own_stream) != hipSuccess) {
        delete c;
        return MYL_E_HIP;
    }
    c->stream = c->own_stream;
    // the allocation-free product's scratch address on this device (current)
    if (noalloc_setup(device_id) != MYL_OK) {
        (void)hipStreamDestroy(c->own_stream);
        delete c;
        return MYL_E_HIP;
    }
    *out = c;
    return MYL_OK;
}

void myl_destroy(myl_ctx* ctx) {
    if (!ctx) return;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    if (ctx->scratch_ptr) (void)hipFree(ctx->scratch_ptr);
    if (ctx->mm.acc) (void)hipFree(ctx->mm.acc);
    if (ctx->mm.planes) (void)hipFree(ctx->mm.planes);
    (void)hipStreamSynchronize(ctx->own_stream);
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
}

const char* myl_last_error(const myl_ctx* ctx) { return ctx ? ctx->err.c_str() : "null context"; }

int myl_device_info(const myl_ctx* ctx, char* gcn_arch, size_t cap, int* cu_count, uint64_t* hbm_bytes) {
    if (!ctx) return MYL_E_INVALID;
    if (gcn_arch && cap) {
        std::strncpy(gcn_arch, ctx->prop.gcnArchName, cap - 1);
        gcn_arch[cap - 1] = 0;
    }
    if (cu_count) *cu_count = ctx->prop.multiProcessorCount;
    if (hbm_bytes) *hbm_bytes = (uint64_t)ctx->prop.totalGlobalMem;
    return MYL_OK;
}

int myl_synchronize(myl_ctx* ctx) {
    if (!ctx) return MYL_E_INVALID;
    return ctx->hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

void* myl_stream(myl_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int myl_set_stream(myl_ctx* ctx, void* stream) {
    if (!ctx) return MYL_E_INVALID;
    (void)hipStreamSynchronize(ctx->stream);
    ctx->stream = stream ? (hipStream_t)stream : ctx->own_stream;
    return MYL_OK;
}

int myl_read_probe(myl_ctx* ctx, const void* p, size_t bytes, uint32_t* out) {
    if (!ctx || !p || !out) return MYL_E_INVALID;
    if (bytes % 16 || ((uintptr_t)p & 15)) return ctx->fail(MYL_E_INVALID, "read_probe: 16-byte aligned, whole 16-byte words");
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ctx->device) != hipSuccess || cus < 1) cus = 256;
    return ctx->hip(read_probe(p, bytes, out, cus, ctx->stream), "read_probe");
}

int myl_malloc(myl_ctx* ctx, size_t bytes, void** dptr) {
    if (!ctx || !dptr) return MYL_E_INVALID;
    (void)hipSetDevice(ctx->device);
    hipError_t e = hipMalloc(dptr, bytes ? bytes : 1);
    if (e == hipErrorOutOfMemory) return ctx->fail(MYL_E_NOMEM, "hipMalloc: out of device memory");
    return ctx->hip(e, "hipMalloc");
}

int myl_free(myl_ctx* ctx, void* dptr) {
    if (!ctx) return MYL_E_INVALID;
    (void)hipStreamSynchronize(ctx->stream);
    return ctx->hip(hipFree(dptr), "hipFree");
}

int myl_memcpy_htod(myl_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx) return MYL_E_INVALID;
    int rc = ctx->hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream), "hipMemcpyAsync H2D");
    if (rc) return rc;
    return ctx->hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

int myl_memcpy_dtoh(myl_ctx* ctx, void* dst, const void* src, size_t bytes) {
    if (!ctx) return MYL_E_INVALID;
    int rc = ctx->hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream), "hipMemcpyAsync D2H");
    if (rc) return rc;
    return ctx->hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Host-slice staging: one scratch allocation carved into aligned pieces.
// ---------------------------------------------------------------------------

namespace {

struct Stage {
    myl_ctx* ctx;
    size_t used = 0;
    struct Piece { const void* host; size_t off, bytes; bool in, out; void* host_out; };
    std::vector<Piece> pieces;
    char* base = nullptr;

    size_t add(size_t bytes) {
        size_t off = used;
        used += (bytes + 255) & ~(size_t)255;
        return off;
    }
    // in: host -> device before the launch
    size_t in(const void* host, size_t bytes) {
        size_t off = add(bytes);
        pieces.push_back({host, off, bytes, true, false, nullptr});
        return off;
    }
    // out: device -> host after the launch (inout when host_in != null)
    size_t out(void* host, size_t bytes, bool also_in = false) {
        size_t off = add(bytes);
        pieces.push_back({host, off, bytes, also_in, true, host});
        return off;
    }
    int upload() {
        base = (char*)ctx->scratch(used ? used : 256);
        if (!base) return ctx->fail(MYL_E_NOMEM, "device scratch allocation failed");
        for (auto& p : pieces)
            if (p.in && p.bytes) {
                int rc = ctx->hip(hipMemcpyAsync(base + p.off, p.host, p.bytes, hipMemcpyHostToDevice, ctx->stream),
                                  "hipMemcpyAsync H2D");
                if (rc) return rc;
            }
        return MYL_OK;
    }
    template <class T> T* at(size_t off) { return reinterpret_cast<T*>(base + off); }
    int download() {
        for (auto& p : pieces)
            if (p.out && p.bytes) {
                int rc = ctx->hip(hipMemcpyAsync(p.host_out, base + p.off, p.bytes, hipMemcpyDeviceToHost, ctx->stream),
                                  "hipMemcpyAsync D2H");
                if (rc) return rc;
            }
        return ctx->hip(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
    }
};

}  // namespace

extern "C" {

// ---------------------------------------------------------------------------
// 1. Backend-trait mirror
// ---------------------------------------------------------------------------

int myl_linear_w8a16(myl_ctx* ctx, const int16_t* x, const int8_t* W, int16_t* out, size_t in_features,
                     size_t out_features, const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac) {
    if (!ctx) return MYL_E_INVALID;
    if (in_features == 0) return ctx->fail(MYL_E_INVALID, "linear_w8a16: in_features must be > 0 (linear.rs:61)");
    if (out_features == 0) return MYL_OK;
    if (!fits_int(in_features) || !fits_int(out_features)) return ctx->fail(MYL_E_INVALID, "linear_w8a16: shape too large");
    Stage s{ctx};
    size_t ox = s.in(x, in_features * 2), ow = s.in(W, in_features * out_features), os = s.in(w_shifts, out_features);
    size_t oo = s.out(out, out_features * 2);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(linear_w8a16(s.at<int16_t>(ox), 1, (int)in_features, s.at<int8_t>(ow), (int)out_features,
                               (int)in_features, s.at<uint8_t>(os), act_frac, out_frac, nullptr, s.at<int16_t>(oo),
                               (int)out_features, ctx->stream), "linear_w8a16");
    return rc ? rc : s.download();
}

int myl_linear_w8a16_pc(myl_ctx* ctx, const int16_t* x, const int8_t* W, int16_t* out, size_t in_features,
                        size_t out_features, const uint8_t* w_shifts, uint8_t act_frac, const uint8_t* out_frac) {
    if (!ctx) return MYL_E_INVALID;
    if (in_features == 0) return ctx->fail(MYL_E_INVALID, "linear_w8a16_pc: in_features must be > 0 (linear.rs:110)");
    if (out_features == 0) return MYL_OK;
    if (!fits_int(in_features) || !fits_int(out_features)) return ctx->fail(MYL_E_INVALID, "linear_w8a16_pc: shape too large");
    Stage s{ctx};
    size_t ox = s.in(x, in_features * 2), ow = s.in(W, in_features * out_features), os = s.in(w_shifts, out_features);
    size_t of = s.in(out_frac, out_features);
    size_t oo = s.out(out, out_features * 2);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(linear_w8a16(s.at<int16_t>(ox), 1, (int)in_features, s.at<int8_t>(ow), (int)out_features,
                               (int)in_features, s.at<uint8_t>(os), act_frac, 0, s.at<uint8_t>(of), s.at<int16_t>(oo),
                               (int)out_features, ctx->stream), "linear_w8a16_pc");
    return rc ? rc : s.download();
}

int myl_add_bias_i16(myl_ctx* ctx, int16_t* out, const int16_t* bias, const uint8_t* bias_shifts, size_t n,
                     uint8_t out_frac) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return MYL_OK;
    if (!fits_int(n)) return ctx->fail(MYL_E_INVALID, "add_bias_i16: too long");
    Stage s{ctx};
    size_t oo = s.out(out, n * 2, true), ob = s.in(bias, n * 2), os = s.in(bias_shifts, n);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(add_bias(s.at<int16_t>(oo), s.at<int16_t>(ob), s.at<uint8_t>(os), (int)n, out_frac, ctx->stream),
                  "add_bias_i16");
    return rc ? rc : s.download();
}

int myl_rmsnorm(myl_ctx* ctx, const int16_t* x, const uint8_t* x_shifts, const int8_t* gamma,
                const uint8_t* gamma_shifts, size_t n, const int16_t* rsqrt_lut, size_t lut_len,
                uint8_t lut_input_shift, uint8_t lut_output_frac, int64_t inv_n_q20, int16_t* out, uint8_t out_frac) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "rmsnorm: x_shifts must not be empty (rmsnorm.rs:96)");
    if (lut_input_shift % 2) return ctx->fail(MYL_E_INVALID, "rmsnorm: lut_input_shift must be even (rmsnorm.rs:76)");
    if (lut_len < 2 || !fits_int(lut_len) || !fits_int(n)) return ctx->fail(MYL_E_INVALID, "rmsnorm: bad LUT or length");
    Stage s{ctx};
    size_t ox = s.in(x, n * 2), oxs = s.in(x_shifts, n), og = s.in(gamma, n), ogs = s.in(gamma_shifts, n);
    size_t ol = s.in(rsqrt_lut, lut_len * 2), oo = s.out(out, n * 2);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(rmsnorm(s.at<int16_t>(ox), 1, (int)n, s.at<uint8_t>(oxs), s.at<int8_t>(og), s.at<uint8_t>(ogs),
                          (int)n, s.at<int16_t>(ol), (int)lut_len, lut_input_shift, lut_output_frac, inv_n_q20,
                          out_frac, s.at<int16_t>(oo), (int)n, ctx->stream), "rmsnorm");
    return rc ? rc : s.download();
}

int myl_softmax(myl_ctx* ctx, const int32_t* logits, int32_t* out, size_t n, const int16_t* exp_lut,
                size_t lut_len, uint8_t lut_shift, uint8_t frac_bits) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "softmax: empty logits divide by zero (softmax.rs:43)");
    if (!fits_int(n) || !fits_int(lut_len)) return ctx->fail(MYL_E_INVALID, "softmax: too long");
    Stage s{ctx};
    size_t oz = s.in(logits, n * 4), ol = s.in(exp_lut, lut_len * 2), oo = s.out(out, n * 4);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(softmax(s.at<int32_t>(oz), 1, (int)n, (int)n, s.at<int16_t>(ol), (int)lut_len, lut_shift, frac_bits,
                          s.at<int32_t>(oo), (int)n, ctx->stream), "softmax");
    return rc ? rc : s.download();
}

int myl_attention(myl_ctx* ctx, const int16_t* q, const int16_t* k, const int16_t* v, int16_t* out,
                  size_t q_len, size_t kv_len, size_t head_dim, const uint8_t* mask, int64_t score_mult,
                  uint8_t score_shift, const int16_t* exp_lut, size_t lut_len, uint8_t lut_shift, uint8_t prob_frac) {
    if (!ctx) return MYL_E_INVALID;
    if (kv_len == 0) return ctx->fail(MYL_E_INVALID, "attention: k/v must not be empty (attention.rs:56)");
    if (q_len == 0) return MYL_OK;
    if (!fits_int(q_len * kv_len) || !fits_int(head_dim)) return ctx->fail(MYL_E_INVALID, "attention: too large");
    Stage s{ctx};
    size_t oq = s.in(q, q_len * head_dim * 2), ok = s.in(k, kv_len * head_dim * 2), ov = s.in(v, kv_len * head_dim * 2);
    size_t om = mask ? s.in(mask, q_len * kv_len) : 0;
    size_t ol = s.in(exp_lut, lut_len * 2);
    size_t osc = s.add(q_len * kv_len * 8);
    size_t oo = s.out(out, q_len * head_dim * 2);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(attention_generic(s.at<int16_t>(oq), s.at<int16_t>(ok), s.at<int16_t>(ov),
                                    mask ? s.at<uint8_t>(om) : nullptr, (int)q_len, (int)kv_len, (int)head_dim,
                                    score_mult, score_shift, s.at<int16_t>(ol), (int)lut_len, lut_shift, prob_frac,
                                    s.at<int32_t>(osc), s.at<int16_t>(oo), ctx->stream), "attention");
    return rc ? rc : s.download();
}

int myl_rope(myl_ctx* ctx, int16_t* q, int16_t* k, size_t n, size_t head_dim, const int16_t* cos_lut,
             const int16_t* sin_lut, size_t lut_len, const uint64_t* positions, uint8_t frac_bits) {
    if (!ctx) return MYL_E_INVALID;
    const size_t half = head_dim / 2;
    if (half == 0 || lut_len / half == 0) return ctx->fail(MYL_E_INVALID, "rope: empty LUT rows (rope.rs:46,52)");
    if (n == 0) return MYL_OK;
    const size_t n_pos = lut_len / half;
    std::vector<int32_t> rows(n);
    for (size_t i = 0; i < n; ++i) rows[i] = (int32_t)(positions[i] % n_pos);
    Stage s{ctx};
    size_t oq = s.out(q, n * head_dim * 2, true), ok = s.out(k, n * head_dim * 2, true);
    size_t oc = s.in(cos_lut, lut_len * 2), os = s.in(sin_lut, lut_len * 2), orow = s.in(rows.data(), n * 4);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(rope(s.at<int16_t>(oq), s.at<int16_t>(ok), (int)n, (int)head_dim, s.at<int16_t>(oc),
                       s.at<int16_t>(os), s.at<int32_t>(orow), frac_bits, ctx->stream), "rope");
    return rc ? rc : s.download();
}

int myl_mlp(myl_ctx* ctx, const int16_t* x, const int8_t* W_gate, const int8_t* W_up, const int8_t* W_down,
            int16_t* out, size_t hidden, size_t inter, const uint8_t* gate_w_shifts, const uint8_t* up_w_shifts,
            const uint8_t* down_w_shifts, const int16_t* silu_lut, size_t silu_len, uint8_t in_frac,
            uint8_t gate_out_frac, uint8_t up_out_frac, uint8_t down_in_frac, uint8_t silu_in_frac,
            int16_t silu_lut_offset, uint8_t silu_out_frac, const uint8_t* out_frac) {
    if (!ctx) return MYL_E_INVALID;
    if (hidden == 0 || inter == 0) return ctx->fail(MYL_E_INVALID, "mlp: hidden and intermediate must be > 0");
    if (silu_len == 0) return ctx->fail(MYL_E_INVALID, "mlp: empty SiLU LUT");
    Stage s{ctx};
    size_t ox = s.in(x, hidden * 2), og = s.in(W_gate, hidden * inter), ou = s.in(W_up, hidden * inter);
    size_t od = s.in(W_down, hidden * inter), ogs = s.in(gate_w_shifts, inter), ous = s.in(up_w_shifts, inter);
    size_t ods = s.in(down_w_shifts, hidden), ol = s.in(silu_lut, silu_len * 2), of = s.in(out_frac, hidden);
    size_t tg = s.add(inter * 2), tu = s.add(inter * 2), th = s.add(inter * 2);
    size_t oo = s.out(out, hidden * 2);
    int rc = s.upload();
    if (rc) return rc;
    hipStream_t st = ctx->stream;
    hipError_t e = linear_w8a16(s.at<int16_t>(ox), 1, (int)hidden, s.at<int8_t>(og), (int)inter, (int)hidden,
                                s.at<uint8_t>(ogs), in_frac, gate_out_frac, nullptr, s.at<int16_t>(tg), (int)inter, st);
    if (e == hipSuccess)
        e = linear_w8a16(s.at<int16_t>(ox), 1, (int)hidden, s.at<int8_t>(ou), (int)inter, (int)hidden,
                         s.at<uint8_t>(ous), in_frac, up_out_frac, nullptr, s.at<int16_t>(tu), (int)inter, st);
    if (e == hipSuccess)
        e = silu_gate(s.at<int16_t>(tg), s.at<int16_t>(tu), (int)inter, s.at<int16_t>(ol), (int)silu_len, gate_out_frac,
                      up_out_frac, down_in_frac, silu_in_frac, silu_lut_offset, silu_out_frac, s.at<int16_t>(th), st);
    if (e == hipSuccess)
        e = linear_w8a16(s.at<int16_t>(th), 1, (int)inter, s.at<int8_t>(od), (int)hidden, (int)inter,
                         s.at<uint8_t>(ods), down_in_frac, 0, s.at<uint8_t>(of), s.at<int16_t>(oo), (int)hidden, st);
    rc = ctx->hip(e, "mlp");
    return rc ? rc : s.download();
}

int myl_argmax_int(myl_ctx* ctx, const int32_t* values, size_t n, int64_t* out_index) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "argmax_int: empty logits (sampling.rs:10)");
    if (!fits_int(n)) return ctx->fail(MYL_E_INVALID, "argmax_int: too long");
    Stage s{ctx};
    size_t ov = s.in(values, n * 4), oo = s.out(out_index, 8);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(argmax(s.at<int32_t>(ov), 1, (int)n, (int)n, s.at<int64_t>(oo), ctx->stream), "argmax");
    return rc ? rc : s.download();
}

int myl_sample_integer_cdf(myl_ctx* ctx, const int32_t* logits, size_t n, uint64_t state, int64_t* token,
                           uint64_t* new_state) {
    if (!ctx || !token || !new_state) return MYL_E_INVALID;
    if (n == 0) {  // logits_to_weights of nothing: total 0 (sampling.rs:31-33)
        *token = 0;
        *new_state = state;
        return MYL_OK;
    }
    if (!fits_int(n)) return ctx->fail(MYL_E_INVALID, "sample_integer_cdf: too long");
    Stage s{ctx};
    size_t ov = s.in(logits, n * 4), os = s.in(&state, 8), ot = s.out(token, 8), on = s.out(new_state, 8);
    int rc = s.upload();
    if (rc) return rc;
    rc = ctx->hip(sample_cdf(s.at<int32_t>(ov), 1, (int)n, (int)n, s.at<uint64_t>(os), s.at<int64_t>(ot),
                             s.at<uint64_t>(on), ctx->stream),
                  "sample_integer_cdf");
    return rc ? rc : s.download();
}

// ---------------------------------------------------------------------------
// 2. Device-pointer forms
// ---------------------------------------------------------------------------

static int check_gemv(myl_ctx* ctx, size_t M, size_t ldx, size_t N, size_t K, size_t ldo, const char* what) {
    if (K == 0) return ctx->fail(MYL_E_INVALID, std::string(what) + ": K must be > 0");
    if (ldx < K || ldo < N) return ctx->fail(MYL_E_INVALID, std::string(what) + ": leading dimension too small");
    if (!fits_int(M) || !fits_int(N) || !fits_int(K) || !fits_int(ldx) || !fits_int(ldo))
        return ctx->fail(MYL_E_INVALID, std::string(what) + ": shape too large");
    return MYL_OK;
}

int myl_linear_w8a16_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N,
                         size_t K, const uint8_t* w_shifts, uint8_t act_frac, uint8_t out_frac,
                         const uint8_t* out_frac_pc, int16_t* out, size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    int rc = check_gemv(ctx, M, ldx, N, K, ldo, "linear_w8a16_dev");
    if (rc || M == 0 || N == 0) return rc;
    const MmCtx* mm = ctx->mm_ctx(M > 1 ? M * N : 0, M >= 2 ? 2 * M * K : 0);
    return ctx->hip(linear_w8a16(x, (int)M, (int)ldx, W, (int)N, (int)K, w_shifts, act_frac, out_frac, out_frac_pc,
                                 out, (int)ldo, ctx->stream, mm), "linear_w8a16_dev");
}

int myl_linear_w8a16_mult_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N,
                              size_t K, const int32_t* mult, const uint8_t* shift, int16_t* out, size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    int rc = check_gemv(ctx, M, ldx, N, K, ldo, "linear_w8a16_mult_dev");
    if (rc || M == 0 || N == 0) return rc;
    const MmCtx* mm = ctx->mm_ctx(M > 1 ? M * N : 0, M >= 2 ? 2 * M * K : 0);
    return ctx->hip(linear_w8a16_mult(x, (int)M, (int)ldx, W, (int)N, (int)K, mult, shift, out, (int)ldo, ctx->stream,
                                      mm), "linear_w8a16_mult_dev");
}

int myl_logits_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const void* W, int w_bits, size_t N,
                   size_t K, const uint8_t* row_shifts, uint8_t norm_frac, uint8_t logit_frac, int32_t* out,
                   size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    int rc = check_gemv(ctx, M, ldx, N, K, ldo, "logits_dev");
    if (rc || M == 0 || N == 0) return rc;
    const MmCtx* mm = ctx->mm_ctx(M > 1 ? M * N : 0, M >= 2 ? 2 * M * K : 0);
    if (w_bits == 8)
        return ctx->hip(logits_w8(x, (int)M, (int)ldx, (const int8_t*)W, (int)N, (int)K, row_shifts, norm_frac,
                                  logit_frac, out, (int)ldo, ctx->stream, mm), "logits_dev");
    if (w_bits == 16)
        return ctx->hip(logits_w16(x, (int)M, (int)ldx, (const int16_t*)W, (int)N, (int)K, row_shifts, norm_frac,
                                   logit_frac, out, (int)ldo, ctx->stream, mm), "logits_dev");
    return ctx->fail(MYL_E_INVALID, "logits_dev: w_bits must be 8 or 16");
}

int myl_dot_i8_i16_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const int8_t* W, size_t N, size_t K,
                       int64_t* out, size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    int rc = check_gemv(ctx, M, ldx, N, K, ldo, "dot_i8_i16_dev");
    if (rc || M == 0 || N == 0) return rc;
    const MmCtx* mm = ctx->mm_ctx(M > 1 ? M * N : 0, M >= 2 ? 2 * M * K : 0);
    return ctx->hip(dot_raw_w8(x, (int)M, (int)ldx, W, (int)N, (int)K, out, (int)ldo, ctx->stream, mm),
                    "dot_i8_i16_dev");
}

int myl_rmsnorm_dev(myl_ctx* ctx, const int16_t* x, size_t M, size_t ldx, const uint8_t* x_shifts,
                    const int8_t* gamma, const uint8_t* gamma_shifts, size_t n, const int16_t* rsqrt_lut,
                    size_t lut_len, uint8_t lut_input_shift, uint8_t lut_output_frac, int64_t inv_n_q20,
                    uint8_t out_frac, int16_t* out, size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "rmsnorm_dev: n must be > 0 (rmsnorm.rs:96)");
    if (lut_input_shift % 2) return ctx->fail(MYL_E_INVALID, "rmsnorm_dev: lut_input_shift must be even");
    if (lut_len < 2 || ldx < n || ldo < n || !fits_int(M) || !fits_int(ldx) || !fits_int(ldo))
        return ctx->fail(MYL_E_INVALID, "rmsnorm_dev: bad shape");
    if (M == 0) return MYL_OK;
    return ctx->hip(rmsnorm(x, (int)M, (int)ldx, x_shifts, gamma, gamma_shifts, (int)n, rsqrt_lut, (int)lut_len,
                            lut_input_shift, lut_output_frac, inv_n_q20, out_frac, out, (int)ldo, ctx->stream),
                    "rmsnorm_dev");
}

int myl_softmax_dev(myl_ctx* ctx, const int32_t* logits, size_t M, size_t n, size_t ldz, const int16_t* exp_lut,
                    size_t lut_len, uint8_t lut_shift, uint8_t frac_bits, int32_t* out, size_t ldo) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "softmax_dev: empty rows (softmax.rs:43)");
    if (ldz < n || ldo < n || !fits_int(M) || !fits_int(ldz) || !fits_int(ldo) || !fits_int(lut_len))
        return ctx->fail(MYL_E_INVALID, "softmax_dev: bad shape");
    if (M == 0) return MYL_OK;
    return ctx->hip(softmax(logits, (int)M, (int)n, (int)ldz, exp_lut, (int)lut_len, lut_shift, frac_bits, out,
                            (int)ldo, ctx->stream), "softmax_dev");
}

int myl_argmax_dev(myl_ctx* ctx, const int32_t* values, size_t M, size_t n, size_t ldv, int64_t* out_index) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "argmax_dev: empty rows (sampling.rs:10)");
    if (ldv < n || !fits_int(M) || !fits_int(ldv)) return ctx->fail(MYL_E_INVALID, "argmax_dev: bad shape");
    if (M == 0) return MYL_OK;
    return ctx->hip(argmax(values, (int)M, (int)n, (int)ldv, out_index, ctx->stream), "argmax_dev");
}

int myl_sample_dev(myl_ctx* ctx, const int32_t* logits, size_t M, size_t n, size_t ldz, const uint64_t* states,
                   int64_t* tokens, uint64_t* new_states) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "sample_dev: empty rows");
    if (ldz < n || !fits_int(M) || !fits_int(n) || !fits_int(ldz)) return ctx->fail(MYL_E_INVALID, "sample_dev: bad shape");
    if (M == 0) return MYL_OK;
    return ctx->hip(sample_cdf(logits, (int)M, (int)n, (int)ldz, states, tokens, new_states, ctx->stream), "sample_dev");
}

int myl_logsoftmax_dev(myl_ctx* ctx, const int32_t* logits, size_t M, size_t n, size_t ldz, const int16_t* exp_lut,
                       size_t lut_len, const int64_t* targets, int64_t* out) {
    if (!ctx) return MYL_E_INVALID;
    if (n == 0) return ctx->fail(MYL_E_INVALID, "logsoftmax_dev: empty rows");
    if (ldz < n || !fits_int(M) || !fits_int(n) || !fits_int(ldz) || !fits_int(lut_len))
        return ctx->fail(MYL_E_INVALID, "logsoftmax_dev: bad shape");
    if (M == 0) return MYL_OK;
    return ctx->hip(logsoftmax(logits, (int)M, (int)n, (int)ldz, exp_lut, (int)lut_len, targets, out, ctx->stream),
                    "logsoftmax_dev");
}

}  // extern "C"
