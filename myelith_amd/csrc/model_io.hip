// model_io.hip -- filling a device model with tensors in the reference layout
// (the IntegerModel fields that runtime/src/loader.rs:712-849 builds) and
// reading them back, plus myl_model_load_artifact: an artifact directory
// streamed from its files to HBM.
//
// The device keeps two row orders of its own: q/k/v rows pair-ordered per head
// (row j and j + hd/2 adjacent, for the fused RoPE) and gate/up rows
// interleaved (gate r, up r adjacent, for the fused SiLU product).  A logical
// tensor is copied to a staging buffer and scattered to its stored rows by a
// row-map kernel; downloads gather the other way.
#include "artifact.h"
#include "model_internal.h"
#include "sha256.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <string>
#include <vector>

namespace {

using myl::kLayerSlots;
using myl::kModelSlots;

// One block per row: stored row map[r] <- staged row r (scatter), or staged
// row r <- stored row map[r] (gather).  Rows are whole 16-byte vectors.
__global__ void __launch_bounds__(256) rows_permute_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst,
                                                           const int32_t* __restrict__ map, size_t vecs, int gather) {
    const size_t r = blockIdx.x;
    const size_t m = (size_t)map[r];
    const uint4* s = src + (gather ? m : r) * vecs;
    uint4* d = dst + (gather ? r : m) * vecs;
    for (size_t i = threadIdx.x; i < vecs; i += blockDim.x) d[i] = s[i];
}

// Element form for per-row shift tables and biases.
template <class T>
__global__ void __launch_bounds__(256) elems_permute_kernel(const T* __restrict__ src, T* __restrict__ dst,
                                                            const int32_t* __restrict__ map, int n, int gather) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    if (gather) dst[i] = src[map[i]];
    else dst[map[i]] = src[i];
}

// Where one tensor of the reference layout lives in the device model.
struct Target {
    void* dst = nullptr;        // stored tensor
    uint64_t rows = 0, cols = 0;  // logical shape (cols = 0: 1-D of `rows` elements)
    int bits = 8;
    const int32_t* map_dev = nullptr;  // logical row -> stored row; nullptr = identity
    uint8_t* shifts = nullptr;         // stored per-row shifts (same map)
    bool store = true;                 // false: accepted and not kept
    size_t slot = 0;
};

int resolve(myl_model* m, const std::string& name, int bits, Target* t) {
    myl_ctx* c = m->ctx;
    const myl_synth_spec& s = m->spec;
    const uint64_t H = m->H, I = m->I, V = m->V, nq = m->nq, nkv = m->nkv;
    if (bits != 8 && bits != 16) return c->fail(MYL_E_INVALID, "tensor " + name + ": bits must be 8 or 16");
    if (name == "model.embed_tokens.weight") {
        *t = Target{m->emb, V, H, 8, nullptr, m->emb_shifts, true, myl::SLOT_EMB};
    } else if (name == "model.norm.weight") {
        *t = Target{m->final_gamma, H, 0, 8, nullptr, m->final_gamma_s, true, myl::SLOT_FINAL_GAMMA};
    } else if (name == "lm_head.weight" && bits == 16) {
        if (!s.lm_head_int16) return c->fail(MYL_E_INVALID, "lm_head.weight: the model has no int16 LM head");
        *t = Target{m->lm16, V, H, 16, nullptr, m->lm16_shifts, true, myl::SLOT_LM16};
    } else if (name == "lm_head.weight") {
        // Kept only when it is the head the forward pass reads (model.rs:285-307).
        const bool keep = !m->tied && !s.lm_head_int16;
        *t = Target{keep ? m->lm8 : nullptr, V, H, 8, nullptr, keep ? m->lm8_shifts : nullptr, keep, myl::SLOT_LM8};
    } else {
        static const char* prefix = "model.layers.";
        const size_t pl = std::strlen(prefix);
        if (name.compare(0, pl, prefix) != 0) return c->fail(MYL_E_INVALID, "unknown tensor " + name);
        size_t i = pl;
        uint64_t l = 0;
        while (i < name.size() && name[i] >= '0' && name[i] <= '9' && l < (1u << 20)) l = l * 10 + (uint64_t)(name[i++] - '0');
        if (i == pl || i >= name.size() || name[i] != '.' || l >= s.layers)
            return c->fail(MYL_E_INVALID, "unknown tensor " + name);
        const std::string sfx = name.substr(i + 1);
        LayerDev& L = m->layers[l];
        const int32_t* qm = m->qkv_map_dev;
        const int32_t* gm = m->gu_map_dev;
        const size_t base = kModelSlots + (size_t)l * kLayerSlots;
        if (sfx == "input_layernorm.weight") *t = Target{L.in_gamma, H, 0, 8, nullptr, L.in_gamma_s, true, myl::SLOT_IN_GAMMA};
        else if (sfx == "post_attention_layernorm.weight")
            *t = Target{L.post_gamma, H, 0, 8, nullptr, L.post_gamma_s, true, myl::SLOT_POST_GAMMA};
        else if (sfx == "self_attn.q_proj.weight") *t = Target{L.wqkv, nq, H, 8, qm, L.sqkv, true, myl::SLOT_Q};
        else if (sfx == "self_attn.k_proj.weight") *t = Target{L.wqkv, nkv, H, 8, qm + nq, L.sqkv, true, myl::SLOT_K};
        else if (sfx == "self_attn.v_proj.weight") *t = Target{L.wqkv, nkv, H, 8, qm + nq + nkv, L.sqkv, true, myl::SLOT_V};
        else if (sfx == "self_attn.o_proj.weight") *t = Target{L.wo, H, nq, 8, nullptr, L.so, true, myl::SLOT_O};
        else if (sfx == "mlp.gate_proj.weight") *t = Target{L.wgu, I, H, 8, gm, L.sgu, true, myl::SLOT_GATE};
        else if (sfx == "mlp.up_proj.weight") *t = Target{L.wgu, I, H, 8, gm + I, L.sgu, true, myl::SLOT_UP};
        else if (sfx == "mlp.down_proj.weight") *t = Target{L.wd, H, I, 8, nullptr, L.sd, true, myl::SLOT_DOWN};
        else if (sfx == "self_attn.q_proj.bias" || sfx == "self_attn.k_proj.bias" || sfx == "self_attn.v_proj.bias") {
            if (!s.attention_bias) return c->fail(MYL_E_INVALID, name + ": the model has no attention biases");
            const int which = sfx[10] == 'q' ? 0 : sfx[10] == 'k' ? 1 : 2;
            const uint64_t off = which == 0 ? 0 : which == 1 ? nq : nq + nkv;
            *t = Target{L.bqkv, which == 0 ? nq : nkv, 0, 16, qm + off, L.bsqkv, true, (size_t)myl::SLOT_BQ + which};
        } else {
            return c->fail(MYL_E_INVALID, "unknown tensor " + name);
        }
        if (t->bits != bits)
            return c->fail(MYL_E_INVALID, name + ": expected " + std::to_string(t->bits) + "-bit data");
        t->slot += base;
        return MYL_OK;
    }
    if (t->bits != bits) return c->fail(MYL_E_INVALID, name + ": expected " + std::to_string(t->bits) + "-bit data");
    return MYL_OK;
}

// Pinned host and device staging, two of each so that filling one overlaps
// the copy of the other.
struct Staging {
    static constexpr size_t kBytes = 32u << 20;
    myl_model* m;
    uint8_t* host[2] = {nullptr, nullptr};
    uint8_t* dev[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    bool used[2] = {false, false};
    int k = 0;

    explicit Staging(myl_model* mm) : m(mm) {}
    int init() {
        for (int i = 0; i < 2; ++i) {
            if (hipHostMalloc((void**)&host[i], kBytes, hipHostMallocDefault) != hipSuccess ||
                hipMalloc((void**)&dev[i], kBytes) != hipSuccess || hipEventCreate(&ev[i]) != hipSuccess)
                return m->ctx->fail(MYL_E_NOMEM, "tensor staging buffers");
        }
        return MYL_OK;
    }
    ~Staging() {
        if (m->ctx) (void)hipStreamSynchronize(m->ctx->stream);
        for (int i = 0; i < 2; ++i) {
            if (ev[i]) (void)hipEventDestroy(ev[i]);
            if (dev[i]) (void)hipFree(dev[i]);
            if (host[i]) (void)hipHostFree(host[i]);
        }
    }
    // The next buffer pair, once its previous copies have finished.
    int acquire() {
        k ^= 1;
        if (used[k]) return m->ctx->hip(hipEventSynchronize(ev[k]), "staging");
        return MYL_OK;
    }
    int release() {
        used[k] = true;
        return m->ctx->hip(hipEventRecord(ev[k], m->ctx->stream), "staging");
    }
};

// Source of a tensor's bytes: host memory, or a file hashed as it is read.
struct Reader {
    const uint8_t* mem = nullptr;
    std::FILE* file = nullptr;
    myl::Sha256* hash = nullptr;
    bool read(uint8_t* dst, size_t n) {
        if (mem) {
            std::memcpy(dst, mem, n);
            mem += n;
        } else if (std::fread(dst, 1, n, file) != n) {
            return false;
        }
        if (hash) hash->update(dst, n);
        return true;
    }
};

// Stored rows of a logical tensor <- the reader's bytes.
int put_tensor(myl_model* m, Staging& st, const Target& t, Reader& rd, const uint8_t* shifts) {
    myl_ctx* c = m->ctx;
    hipStream_t s = c->stream;
    const size_t esz = (size_t)t.bits / 8;
    if (t.cols == 0) {  // 1-D: gamma vectors and biases
        const size_t bytes = t.rows * esz;
        if (int rc = st.acquire()) return rc;
        if (!rd.read(st.host[st.k], bytes)) return c->fail(MYL_E_INVALID, "short read");
        if (t.store) {
            hipError_t e;
            if (t.map_dev) {
                e = hipMemcpyAsync(st.dev[st.k], st.host[st.k], bytes, hipMemcpyHostToDevice, s);
                const int n = (int)t.rows;
                if (e == hipSuccess && esz == 2)
                    elems_permute_kernel<int16_t><<<(n + 255) / 256, 256, 0, s>>>(
                        (const int16_t*)st.dev[st.k], (int16_t*)t.dst, t.map_dev, n, 0);
                else if (e == hipSuccess)
                    elems_permute_kernel<int8_t><<<(n + 255) / 256, 256, 0, s>>>((const int8_t*)st.dev[st.k],
                                                                                 (int8_t*)t.dst, t.map_dev, n, 0);
                if (e == hipSuccess) e = hipGetLastError();
            } else {
                e = hipMemcpyAsync(t.dst, st.host[st.k], bytes, hipMemcpyHostToDevice, s);
            }
            if (int rc = c->hip(e, "tensor upload")) return rc;
        }
        if (int rc = st.release()) return rc;
    } else {
        const size_t row_bytes = t.cols * esz;
        if (row_bytes % 16) return c->fail(MYL_E_UNSUPPORTED, "tensor rows must be multiples of 16 bytes");
        const size_t chunk = std::max<size_t>(1, Staging::kBytes / row_bytes);
        if (row_bytes > Staging::kBytes) return c->fail(MYL_E_UNSUPPORTED, "tensor rows larger than the staging buffer");
        for (size_t r0 = 0; r0 < t.rows; r0 += chunk) {
            const size_t nr = std::min(chunk, (size_t)t.rows - r0);
            if (int rc = st.acquire()) return rc;
            if (!rd.read(st.host[st.k], nr * row_bytes)) return c->fail(MYL_E_INVALID, "short read");
            if (t.store) {
                hipError_t e;
                if (t.map_dev) {
                    e = hipMemcpyAsync(st.dev[st.k], st.host[st.k], nr * row_bytes, hipMemcpyHostToDevice, s);
                    if (e == hipSuccess)
                        rows_permute_kernel<<<(unsigned)nr, 256, 0, s>>>((const uint4*)st.dev[st.k], (uint4*)t.dst,
                                                                         t.map_dev + r0, row_bytes / 16, 0);
                    if (e == hipSuccess) e = hipGetLastError();
                } else {
                    e = hipMemcpyAsync((uint8_t*)t.dst + r0 * row_bytes, st.host[st.k], nr * row_bytes,
                                       hipMemcpyHostToDevice, s);
                }
                if (int rc = c->hip(e, "tensor upload")) return rc;
            }
            if (int rc = st.release()) return rc;
        }
    }
    if (t.store && shifts) {
        if (int rc = st.acquire()) return rc;
        std::memcpy(st.host[st.k], shifts, t.rows);
        hipError_t e;
        if (t.map_dev) {
            e = hipMemcpyAsync(st.dev[st.k], st.host[st.k], t.rows, hipMemcpyHostToDevice, s);
            const int n = (int)t.rows;
            if (e == hipSuccess)
                elems_permute_kernel<uint8_t><<<(n + 255) / 256, 256, 0, s>>>(st.dev[st.k], t.shifts, t.map_dev, n, 0);
            if (e == hipSuccess) e = hipGetLastError();
        } else {
            e = hipMemcpyAsync(t.shifts, st.host[st.k], t.rows, hipMemcpyHostToDevice, s);
        }
        if (int rc = c->hip(e, "shift upload")) return rc;
        if (int rc = st.release()) return rc;
    }
    m->have[t.slot] = 1;
    if (t.slot == myl::SLOT_LM16) m->lm16_planes_ok = false;
    if (t.slot >= (size_t)myl::kModelSlots) {
        const int ls = (int)((t.slot - myl::kModelSlots) % myl::kLayerSlots);
        const bool frag_src = ls == myl::SLOT_Q || ls == myl::SLOT_K || ls == myl::SLOT_V || ls == myl::SLOT_GATE ||
                              ls == myl::SLOT_UP || ls == myl::SLOT_DOWN;
        if (frag_src && m->frag_state > 0) m->frag_state = 0;
    }
    return MYL_OK;
}

bool shape_ok(const Target& t, const uint64_t* shape, uint32_t ndim) {
    if (t.cols == 0) return ndim == 1 && shape[0] == t.rows;
    return ndim == 2 && shape[0] == t.rows && shape[1] == t.cols;
}

// The model's upload staging, created on first use and released by
// myl_model_finalize (or with the model).
void staging_free(void* p) { delete static_cast<Staging*>(p); }

Staging* staging_of(myl_model* m) {
    if (!m->io) {
        Staging* st = new (std::nothrow) Staging(m);
        if (!st) return nullptr;
        if (st->init()) {
            delete st;
            return nullptr;
        }
        m->io = st;
        m->io_free = staging_free;
    }
    return static_cast<Staging*>(m->io);
}

int create_from_dims(myl_ctx* ctx, const myl_model_dims& d, uint32_t max_pos, const myl_luts* luts, myl_model** out) {
    myl_synth_spec s{};
    s.seed = 0;
    s.vocab = d.vocab;
    s.hidden = d.hidden;
    s.layers = d.layers;
    s.heads = d.heads;
    s.kv_heads = d.kv_heads;
    s.head_dim = d.head_dim;
    s.inter = d.inter;
    s.max_pos = max_pos ? max_pos : d.max_context;
    s.lm_head_int16 = d.lm_head_int16 ? 1 : 0;
    s.attention_bias = d.attention_bias ? 1 : 0;
    return myl::model_setup(ctx, s, d.tie_word_embeddings != 0, luts, out);
}

}  // namespace

extern "C" {

int myl_model_create(myl_ctx* ctx, const myl_model_dims* dims, uint32_t max_pos, const myl_luts* luts,
                     myl_model** out) {
    if (!ctx || !dims || !luts || !out) return MYL_E_INVALID;
    *out = nullptr;
    return create_from_dims(ctx, *dims, max_pos, luts, out);
}

int myl_model_upload_tensor(myl_model* m, const char* name, const void* data, int bits, const uint64_t* shape,
                            uint32_t ndim, const uint8_t* shifts, size_t n_shifts) {
    if (!m || !name || !data || !shape || !shifts) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    Target t;
    if (int rc = resolve(m, name, bits, &t)) return rc;
    if (!shape_ok(t, shape, ndim)) return c->fail(MYL_E_INVALID, std::string(name) + ": shape does not match the model");
    if (n_shifts != t.rows) return c->fail(MYL_E_INVALID, std::string(name) + ": one shift per row expected");
    Staging* st = staging_of(m);
    if (!st) return c->fail(MYL_E_NOMEM, "tensor staging buffers");
    Reader rd;
    rd.mem = (const uint8_t*)data;
    if (int rc = put_tensor(m, *st, t, rd, shifts)) return rc;
    return c->hip(hipStreamSynchronize(c->stream), "tensor upload");
}

int myl_model_download_tensor(myl_model* m, const char* name, int bits, void* data, size_t bytes, uint8_t* shifts,
                              size_t n_shifts) {
    if (!m || !name || !data) return MYL_E_INVALID;
    myl_ctx* c = m->ctx;
    hipStream_t s = c->stream;
    Target t;
    if (int rc = resolve(m, name, bits, &t)) return rc;
    if (!t.store) return c->fail(MYL_E_INVALID, std::string(name) + ": not kept by this model");
    const size_t esz = (size_t)bits / 8;
    const size_t total = t.rows * (t.cols ? t.cols : 1) * esz;
    if (bytes != total) return c->fail(MYL_E_INVALID, std::string(name) + ": byte count mismatch");
    if (shifts && n_shifts != t.rows) return c->fail(MYL_E_INVALID, std::string(name) + ": one shift per row expected");
    Staging* stp = staging_of(m);
    if (!stp) return c->fail(MYL_E_NOMEM, "tensor staging buffers");
    Staging& st = *stp;
    if (int rc = c->hip(hipStreamSynchronize(s), "tensor download")) return rc;
    auto gather = [&](const void* src, void* dst_host, size_t n, size_t elem) -> int {
        // n elements of `elem` bytes (elem 1 or 2) through the map
        hipError_t e = hipSuccess;
        if (elem == 2)
            elems_permute_kernel<int16_t><<<((int)n + 255) / 256, 256, 0, s>>>((const int16_t*)src, (int16_t*)st.dev[0],
                                                                               t.map_dev, (int)n, 1);
        else
            elems_permute_kernel<uint8_t><<<((int)n + 255) / 256, 256, 0, s>>>((const uint8_t*)src, st.dev[0], t.map_dev,
                                                                               (int)n, 1);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipMemcpyAsync(dst_host, st.dev[0], n * elem, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        return c->hip(e, "tensor download");
    };
    if (t.cols == 0) {
        if (t.map_dev) {
            if (int rc = gather(t.dst, data, t.rows, esz)) return rc;
        } else {
            hipError_t e = hipMemcpyAsync(data, t.dst, total, hipMemcpyDeviceToHost, s);
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (int rc = c->hip(e, "tensor download")) return rc;
        }
    } else {
        const size_t row_bytes = t.cols * esz;
        const size_t chunk = std::max<size_t>(1, Staging::kBytes / row_bytes);
        for (size_t r0 = 0; r0 < t.rows; r0 += chunk) {
            const size_t nr = std::min(chunk, (size_t)t.rows - r0);
            uint8_t* out = (uint8_t*)data + r0 * row_bytes;
            hipError_t e;
            if (t.map_dev) {
                rows_permute_kernel<<<(unsigned)nr, 256, 0, s>>>((const uint4*)t.dst, (uint4*)st.dev[0], t.map_dev + r0,
                                                                 row_bytes / 16, 1);
                e = hipGetLastError();
                if (e == hipSuccess) e = hipMemcpyAsync(st.host[0], st.dev[0], nr * row_bytes, hipMemcpyDeviceToHost, s);
            } else {
                e = hipMemcpyAsync(st.host[0], (const uint8_t*)t.dst + r0 * row_bytes, nr * row_bytes,
                                   hipMemcpyDeviceToHost, s);
            }
            if (e == hipSuccess) e = hipStreamSynchronize(s);
            if (int rc = c->hip(e, "tensor download")) return rc;
            std::memcpy(out, st.host[0], nr * row_bytes);
        }
    }
    if (shifts) {
        if (t.map_dev) return gather(t.shifts, shifts, t.rows, 1);
        hipError_t e = hipMemcpyAsync(shifts, t.shifts, t.rows, hipMemcpyDeviceToHost, s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);
        return c->hip(e, "shift download");
    }
    return MYL_OK;
}

int myl_model_set_layer_scales(myl_model* m, uint32_t layer, const myl_layer_fracs* fracs, const uint8_t* res_in,
                               const uint8_t* res_mid) {
    if (!m || !fracs || !res_in || !res_mid) return MYL_E_INVALID;
    if (layer >= m->spec.layers) return m->ctx->fail(MYL_E_INVALID, "set_layer_scales: layer out of range");
    m->layers[layer].f = *fracs;
    m->h_res_in[layer].assign(res_in, res_in + m->H);
    m->h_res_mid[layer].assign(res_mid, res_mid + m->H);
    m->scales_have[layer] = 1;
    m->ready = false;
    return MYL_OK;
}

int myl_model_set_final_scales(myl_model* m, uint8_t final_norm_frac, const uint8_t* final_res) {
    if (!m || !final_res) return MYL_E_INVALID;
    m->final_norm_frac = final_norm_frac;
    m->h_final_res.assign(final_res, final_res + m->H);
    m->final_have = true;
    m->ready = false;
    return MYL_OK;
}

int myl_model_get_layer_scales(myl_model* m, uint32_t layer, myl_layer_fracs* fracs, uint8_t* res_in,
                               uint8_t* res_mid) {
    if (!m) return MYL_E_INVALID;
    if (layer >= m->spec.layers) return m->ctx->fail(MYL_E_INVALID, "get_layer_scales: layer out of range");
    if (fracs) *fracs = m->layers[layer].f;
    if (res_in) std::memcpy(res_in, m->h_res_in[layer].data(), m->H);
    if (res_mid) std::memcpy(res_mid, m->h_res_mid[layer].data(), m->H);
    return MYL_OK;
}

int myl_model_get_final_scales(myl_model* m, uint8_t* final_norm_frac, uint8_t* final_res) {
    if (!m) return MYL_E_INVALID;
    if (final_norm_frac) *final_norm_frac = m->final_norm_frac;
    if (final_res) std::memcpy(final_res, m->h_final_res.data(), m->H);
    return MYL_OK;
}

int myl_model_finalize(myl_model* m) {
    if (!m) return MYL_E_INVALID;
    const int rc = myl::model_finalize(m);
    if (!rc && m->io) {
        m->io_free(m->io);
        m->io = nullptr;
    }
    return rc;
}

int myl_model_load_artifact(myl_ctx* ctx, const myl_artifact* a, uint32_t max_pos, myl_model** out) {
    if (!ctx || !a || !out) return MYL_E_INVALID;
    *out = nullptr;
    const myl_model_dims& d = a->dims;
    auto lut = [&](const char* n) -> const std::vector<int16_t>& { return a->luts.at(n).values; };
    const std::vector<int16_t>&rs = lut("rsqrt"), &si = lut("silu"), &ex = lut("exp"), &co = lut("cos"), &sn = lut("sin");
    if (co.size() != sn.size()) return ctx->fail(MYL_E_INVALID, "artifact: cos and sin tables differ in length");
    myl_luts luts{rs.data(), rs.size(), si.data(), si.size(), ex.data(), ex.size(), co.data(), sn.data(), co.size()};
    if (!max_pos && !d.max_context) return ctx->fail(MYL_E_INVALID, "artifact: max_context is 0 and no max_pos given");
    myl_model* m = nullptr;
    if (int rc = create_from_dims(ctx, d, max_pos, &luts, &m)) return rc;
    std::unique_ptr<myl_model> guard(m);
    int rc = MYL_OK;
    {
        Staging st(m);
        rc = st.init();
        std::vector<uint8_t> shifts;
        for (size_t i = 0; !rc && i < a->required.size(); ++i) {
            const myl::ArtRequired& q = a->required[i];
            const myl::ArtWeight& w = a->weights.at(q.key);
            Target t;
            if ((rc = resolve(m, q.name, q.bits, &t))) break;
            if (!q.upload) t.store = false;
            if ((rc = myl::art_row_shifts(a, w, &shifts))) {
                rc = ctx->fail(rc, a->error);
                break;
            }
            std::FILE* f = std::fopen(a->path(w.file).c_str(), "rb");
            if (!f) {
                rc = ctx->fail(MYL_E_INVALID, "cannot read " + w.file);
                break;
            }
            myl::Sha256 h;
            Reader rd;
            rd.file = f;
            rd.hash = &h;
            rc = put_tensor(m, st, t, rd, t.store ? shifts.data() : nullptr);
            std::fclose(f);
            if (rc) break;
            const std::string digest = h.hex();
            if (digest != w.hash)
                rc = ctx->fail(MYL_E_INVALID, w.key + ": SHA-256 " + digest + " does not match the manifest hash " + w.hash);
        }
        // Manifest entries the model does not read are hashed all the same
        // (load_weights checks every entry, loader.rs:326-485).
        for (const auto& kv : a->weights) {
            if (rc) break;
            bool seen = false;
            for (const myl::ArtRequired& q : a->required) seen = seen || q.key == kv.first;
            if (seen) continue;
            std::string digest;
            if (!myl::art_hash_file(a->path(kv.second.file), &digest))
                rc = ctx->fail(MYL_E_INVALID, "cannot read " + kv.second.file);
            else if (digest != kv.second.hash)
                rc = ctx->fail(MYL_E_INVALID, kv.first + ": SHA-256 " + digest + " does not match the manifest hash " +
                                                  kv.second.hash);
            else if (myl::art_row_shifts(a, kv.second, &shifts))
                rc = ctx->fail(MYL_E_INVALID, a->error);
        }
    }
    for (uint32_t l = 0; !rc && l < d.layers; ++l)
        rc = myl_model_set_layer_scales(m, l, &a->layer_fracs[l], a->res_in[l].data(), a->res_mid[l].data());
    if (!rc) rc = myl_model_set_final_scales(m, a->final_norm_frac, a->final_res.data());
    if (!rc) rc = myl::model_finalize(m);
    if (rc) return rc;
    *out = guard.release();
    return MYL_OK;
}

}  // extern "C"
