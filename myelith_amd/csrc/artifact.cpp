// artifact.cpp -- reader of the reference's artifact directory
// (runtime/src/loader.rs:33-849): manifests, scales, LUTs and the checks of
// load_model / build_model.  Host code only; the device upload is in
// model_io.hip.
#include "artifact.h"
#include "json.h"
#include "sha256.h"

#include <sys/stat.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <memory>
#include <new>
#include <sstream>

namespace myl {

std::string manifest_key(const std::string& hf_name) {
    std::string k = hf_name;
    for (char& c : k)
        if (c == '.') c = '_';
    return k;
}

bool art_read_file(const std::string& path, std::string* out) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return false;
    std::ostringstream ss;
    ss << f.rdbuf();
    if (f.bad()) return false;
    *out = ss.str();
    return true;
}

bool art_file_size(const std::string& path, uint64_t* n) {
    struct stat st;
    if (stat(path.c_str(), &st) != 0 || !S_ISREG(st.st_mode)) return false;
    *n = (uint64_t)st.st_size;
    return true;
}

// SHA-256 of a whole file, read in 8 MiB pieces.
bool art_hash_file(const std::string& path, std::string* hex) {
    std::FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) return false;
    Sha256 h;
    std::unique_ptr<char[]> buf(new (std::nothrow) char[8 << 20]);
    if (!buf) {
        std::fclose(f);
        return false;
    }
    size_t n;
    while ((n = std::fread(buf.get(), 1, 8 << 20, f)) > 0) h.update(buf.get(), n);
    const bool ok = !std::ferror(f);
    std::fclose(f);
    if (ok) *hex = h.hex();
    return ok;
}

// The per-row shifts of a manifest entry: its shifts file (size checked at
// open, hash checked here when the manifest gives one), or the uniform
// entry.shift replicated per row (loader.rs:452-485).
int art_row_shifts(const myl_artifact* a, const ArtWeight& w, std::vector<uint8_t>* out) {
    const uint64_t rows = w.shape.empty() ? 0 : w.shape[0];
    if (!w.has_shifts_file) {
        out->assign(rows, (uint8_t)w.shift);
        return MYL_OK;
    }
    std::string bytes;
    if (!art_read_file(a->path(w.shifts_file), &bytes))
        return a->fail(MYL_E_INVALID, "cannot read " + w.shifts_file);
    if (bytes.size() != rows)
        return a->fail(MYL_E_INVALID, w.key + ": " + std::to_string(bytes.size()) + " shifts in '" + w.shifts_file +
                                          "', expected " + std::to_string(rows) + " rows");
    if (w.has_shifts_hash) {
        const std::string d = Sha256::hex_of(bytes.data(), bytes.size());
        if (d != w.shifts_hash)
            return a->fail(MYL_E_INVALID, w.key + ": SHA-256 " + d + " of the shifts file does not match the manifest hash " +
                                              w.shifts_hash);
    }
    out->assign(bytes.begin(), bytes.end());
    return MYL_OK;
}

}  // namespace myl

namespace {

using myl::ArtLut;
using myl::ArtRequired;
using myl::ArtScale;
using myl::ArtWeight;
using myl::Json;

int load_json(myl_artifact* a, const char* file, std::string* text, Json* j) {
    if (!myl::art_read_file(a->path(file), text)) return a->fail(MYL_E_INVALID, std::string("cannot read ") + file);
    std::string err;
    if (!myl::JsonParser::parse(*text, j, &err))
        return a->fail(MYL_E_INVALID, std::string("invalid ") + file + ": " + err);
    return MYL_OK;
}

bool get_str(const Json& o, const char* k, std::string* out) {
    const Json* v = o.get(k);
    if (!v || !v->is_string()) return false;
    *out = v->s;
    return true;
}

bool get_u64(const Json& o, const char* k, uint64_t* out) {
    const Json* v = o.get(k);
    int64_t x;
    if (!v || !v->as_i64(&x) || x < 0) return false;
    *out = (uint64_t)x;
    return true;
}

bool get_i64(const Json& o, const char* k, int64_t* out) {
    const Json* v = o.get(k);
    return v && v->as_i64(out);
}

bool get_f64(const Json& o, const char* k, double* out) {
    const Json* v = o.get(k);
    return v && v->as_f64(out);
}

// theta_v.json (loader.rs:41-53): absent fields read as "unknown" / "".
int read_theta_v(myl_artifact* a) {
    std::string text;
    Json j;
    if (int rc = load_json(a, "theta_v.json", &text, &j)) return rc;
    if (!j.is_object()) return a->fail(MYL_E_INVALID, "invalid theta_v.json: not an object");
    if (!get_str(j, "version", &a->version)) a->version = "unknown";
    get_str(j, "weights_hash", &a->weights_hash);
    get_str(j, "scales_hash", &a->scales_hash);
    get_str(j, "luts_hash", &a->luts_hash);
    // verify_version_against_spec (loader.rs:56-72)
    if (a->version != MYL_TV_VERSION)
        return a->fail(MYL_E_INVALID, "theta_v version of the artifact (" + a->version +
                                          ") does not match the execution spec of this library (" MYL_TV_VERSION ")");
    return MYL_OK;
}

// model_config.json (loader.rs:240-304, ModelDims / load_model_dims).
int read_dims(myl_artifact* a) {
    std::string text;
    Json j;
    if (int rc = load_json(a, "model_config.json", &text, &j)) return rc;
    if (!j.is_object()) return a->fail(MYL_E_INVALID, "invalid model_config.json: not an object");
    if (!get_str(j, "family", &a->family)) return a->fail(MYL_E_INVALID, "invalid model_config.json: missing field family");
    if (!get_str(j, "variant", &a->variant))
        return a->fail(MYL_E_INVALID, "invalid model_config.json: missing field variant");
    static const char* names[] = {"num_layers", "hidden_size", "intermediate_size", "num_heads",
                                  "num_kv_heads", "head_dim", "vocab_size", "max_context"};
    uint64_t v[8];
    for (int i = 0; i < 8; ++i) {
        if (!get_u64(j, names[i], &v[i]))
            return a->fail(MYL_E_INVALID, std::string("invalid model_config.json: missing field ") + names[i]);
        if (v[i] > 0xFFFFFFFFull)
            return a->fail(MYL_E_UNSUPPORTED, std::string("model_config.json: ") + names[i] + " exceeds 32 bits");
    }
    const Json* tie = j.get("tie_word_embeddings");
    const Json* bias = j.get("attention_bias");
    if (!tie || !tie->is_bool())
        return a->fail(MYL_E_INVALID, "invalid model_config.json: missing field tie_word_embeddings");
    if (!bias || !bias->is_bool())
        return a->fail(MYL_E_INVALID, "invalid model_config.json: missing field attention_bias");
    myl_model_dims& d = a->dims;
    d.layers = (uint32_t)v[0];
    d.hidden = (uint32_t)v[1];
    d.inter = (uint32_t)v[2];
    d.heads = (uint32_t)v[3];
    d.kv_heads = (uint32_t)v[4];
    d.head_dim = (uint32_t)v[5];
    d.vocab = (uint32_t)v[6];
    d.max_context = (uint32_t)v[7];
    d.tie_word_embeddings = tie->b ? 1 : 0;
    d.attention_bias = bias->b ? 1 : 0;
    if (!d.layers || !d.hidden || !d.heads || !d.kv_heads || !d.head_dim || !d.vocab)
        return a->fail(MYL_E_INVALID, "model_config.json: every model dimension must be > 0");
    if ((uint64_t)d.hidden != (uint64_t)d.heads * d.head_dim)
        return a->fail(MYL_E_INVALID, "model_config.json: hidden_size (" + std::to_string(d.hidden) + ") != num_heads (" +
                                          std::to_string(d.heads) + ") * head_dim (" + std::to_string(d.head_dim) + ")");
    if (d.heads % d.kv_heads)
        return a->fail(MYL_E_INVALID, "model_config.json: num_heads (" + std::to_string(d.heads) +
                                          ") is not a multiple of num_kv_heads (" + std::to_string(d.kv_heads) + ")");
    return MYL_OK;
}

// weights_manifest.json (loader.rs:311-486, load_weights) without the content
// hashes: dtype rules, shapes, file sizes, shift ranges.
int read_weights(myl_artifact* a) {
    std::string text;
    Json j;
    if (int rc = load_json(a, "weights_manifest.json", &text, &j)) return rc;
    if (!j.is_object()) return a->fail(MYL_E_INVALID, "invalid weights_manifest.json: not an object");
    for (const auto& kv : j.members) {
        const std::string& name = kv.first;
        const Json& e = kv.second;
        ArtWeight w;
        w.key = name;
        if (!e.is_object() || !get_str(e, "original_name", &w.original_name) || !get_str(e, "file", &w.file) ||
            !get_str(e, "dtype", &w.dtype) || !get_str(e, "hash", &w.hash) || !get_f64(e, "scale", &w.scale) ||
            !get_i64(e, "shift", &w.shift))
            return a->fail(MYL_E_INVALID, "invalid weights_manifest.json: incomplete entry " + name);
        const Json* shape = e.get("shape");
        if (!shape || !shape->is_array()) return a->fail(MYL_E_INVALID, "invalid weights_manifest.json: shape of " + name);
        for (const Json& d : shape->items) {
            int64_t x;
            if (!d.as_i64(&x) || x < 0) return a->fail(MYL_E_INVALID, "invalid weights_manifest.json: shape of " + name);
            w.shape.push_back((uint64_t)x);
        }
        const Json* sf = e.get("shifts_file");
        if (sf && sf->is_string()) {
            w.has_shifts_file = true;
            w.shifts_file = sf->s;
        } else if (sf && sf->kind != Json::Null) {
            return a->fail(MYL_E_INVALID, "invalid weights_manifest.json: shifts_file of " + name);
        }
        const Json* sh = e.get("shifts_hash");
        if (sh && sh->is_string()) {
            w.has_shifts_hash = true;
            w.shifts_hash = sh->s;
        } else if (sh && sh->kind != Json::Null) {
            return a->fail(MYL_E_INVALID, "invalid weights_manifest.json: shifts_hash of " + name);
        }

        uint64_t elem_bytes;
        if (w.dtype == "int16") {
            const bool is_bias = name.size() >= 5 && name.compare(name.size() - 5, 5, "_bias") == 0;
            if (name != "lm_head" && !is_bias)
                return a->fail(MYL_E_INVALID, name + ": int16 is allowed only for the LM head and attention biases");
            if (!w.has_shifts_file) return a->fail(MYL_E_INVALID, name + ": int16 entry without shifts_file");
            if (!is_bias && w.shape.size() != 2)
                return a->fail(MYL_E_INVALID, name + ": the LM head expects shape [vocab, hidden]");
            if (is_bias && w.shape.size() != 1) return a->fail(MYL_E_INVALID, name + ": a bias expects a 1-D shape");
            elem_bytes = 2;
        } else if (w.dtype == "int8") {
            if (w.shape.empty()) return a->fail(MYL_E_INVALID, name + ": empty shape in the manifest");
            elem_bytes = 1;
        } else {
            return a->fail(MYL_E_INVALID, name + ": unsupported dtype '" + w.dtype + "' (expected 'int8')");
        }
        uint64_t size;
        if (!myl::art_file_size(a->path(w.file), &size)) return a->fail(MYL_E_INVALID, "cannot read " + w.file);
        const uint64_t expect = w.elems() * elem_bytes;
        if (size != expect)
            return a->fail(MYL_E_INVALID, name + ": " + std::to_string(size) + " bytes in '" + w.file + "', but the shape needs " +
                                              std::to_string(expect) + " bytes");
        if (w.has_shifts_file) {
            uint64_t ss;
            if (!myl::art_file_size(a->path(w.shifts_file), &ss))
                return a->fail(MYL_E_INVALID, "cannot read " + w.shifts_file);
            if (ss != w.shape[0])
                return a->fail(MYL_E_INVALID, name + ": " + std::to_string(ss) + " shifts in '" + w.shifts_file +
                                                  "', expected " + std::to_string(w.shape[0]) + " rows");
        } else if (w.shift < 0 || w.shift > 255) {
            return a->fail(MYL_E_INVALID, name + ": shift " + std::to_string(w.shift) +
                                              " is outside 0..=255 (and no shifts_file is given)");
        }
        a->weights[name] = std::move(w);
    }
    return MYL_OK;
}

// scales.json (loader.rs:552-579, load_scales).
int read_scales(myl_artifact* a) {
    std::string text;
    Json j;
    if (int rc = load_json(a, "scales.json", &text, &j)) return rc;
    if (!j.is_object()) return a->fail(MYL_E_INVALID, "invalid scales.json: not an object");
    for (const auto& kv : j.members) {
        const Json& e = kv.second;
        ArtScale s;
        double absmax;
        if (!e.is_object() || !get_i64(e, "shift", &s.shift) || !get_f64(e, "scale", &s.scale) ||
            !get_f64(e, "absmax_observed", &absmax))
            return a->fail(MYL_E_INVALID, "invalid scales.json: incomplete entry " + kv.first);
        const Json* arr = e.get("shifts");
        if (arr && arr->is_array()) {
            s.has_shifts = true;
            for (const Json& x : arr->items) {
                int64_t v;
                if (!x.as_i64(&v)) return a->fail(MYL_E_INVALID, "invalid scales.json: shifts of " + kv.first);
                s.shifts.push_back(v);
            }
        } else if (arr && arr->kind != Json::Null) {
            return a->fail(MYL_E_INVALID, "invalid scales.json: shifts of " + kv.first);
        }
        if (s.shift < 0 || s.shift > 255)
            return a->fail(MYL_E_INVALID, kv.first + ": shift " + std::to_string(s.shift) + " is outside 0..=255");
        const double expect = std::ldexp(1.0, -(int)s.shift);
        if (std::fabs(s.scale - expect) > expect * 1e-9)
            return a->fail(MYL_E_INVALID, kv.first + ": scale is not the power of two of shift " + std::to_string(s.shift));
        a->scales[kv.first] = std::move(s);
    }
    return MYL_OK;
}

// luts.json (loader.rs:496-545, load_luts): tables read and hashed here.
int read_luts(myl_artifact* a) {
    std::string text;
    Json j;
    if (int rc = load_json(a, "luts.json", &text, &j)) return rc;
    if (!j.is_object()) return a->fail(MYL_E_INVALID, "invalid luts.json: not an object");
    for (const auto& kv : j.members) {
        const Json& e = kv.second;
        ArtLut t;
        if (!e.is_object() || !get_str(e, "file", &t.file) || !get_str(e, "hash", &t.hash) ||
            !get_u64(e, "length", &t.length) || !get_str(e, "dtype", &t.dtype))
            return a->fail(MYL_E_INVALID, "invalid luts.json: incomplete entry " + kv.first);
        if (t.dtype != "int16")
            return a->fail(MYL_E_INVALID, kv.first + ": unsupported dtype '" + t.dtype + "' (expected 'int16')");
        std::string bytes;
        if (!myl::art_read_file(a->path(t.file), &bytes)) return a->fail(MYL_E_INVALID, "cannot read " + t.file);
        if (bytes.size() != t.length * 2)
            return a->fail(MYL_E_INVALID, kv.first + ": " + std::to_string(bytes.size()) + " bytes in '" + t.file +
                                              "', but length " + std::to_string(t.length) + " needs " +
                                              std::to_string(t.length * 2) + " bytes");
        const std::string d = myl::Sha256::hex_of(bytes.data(), bytes.size());
        if (d != t.hash)
            return a->fail(MYL_E_INVALID, kv.first + ": SHA-256 " + d + " does not match the manifest hash " + t.hash);
        t.values.resize(t.length);
        for (uint64_t i = 0; i < t.length; ++i)
            t.values[i] = (int16_t)(uint16_t)((uint8_t)bytes[2 * i] | (uint16_t)(uint8_t)bytes[2 * i + 1] << 8);
        a->luts[kv.first] = std::move(t);
    }
    return MYL_OK;
}

// ThetaV::verify (loader.rs:76-87) on the bytes of the three manifests.
int verify_manifest_hashes(myl_artifact* a) {
    static const char* files[3] = {"weights_manifest.json", "scales.json", "luts.json"};
    static const char* what[3] = {"weights hash mismatch", "scales hash mismatch", "luts hash mismatch"};
    const std::string* want[3] = {&a->weights_hash, &a->scales_hash, &a->luts_hash};
    for (int i = 0; i < 3; ++i) {
        std::string bytes;
        if (!myl::art_read_file(a->path(files[i]), &bytes)) return a->fail(MYL_E_INVALID, std::string("cannot read ") + files[i]);
        if (myl::Sha256::hex_of(bytes.data(), bytes.size()) != *want[i]) return a->fail(MYL_E_INVALID, what[i]);
    }
    return MYL_OK;
}

int require_scale(myl_artifact* a, const std::string& name, uint8_t* out) {
    auto it = a->scales.find(name);
    if (it == a->scales.end()) return a->fail(MYL_E_INVALID, "missing calibrated activation scale in scales.json: " + name);
    *out = (uint8_t)it->second.shift;
    return MYL_OK;
}

// LoadedScales::shifts_per_channel (loader.rs:216-236): the per-channel
// array, or the scalar shift broadcast to every channel.
int require_scale_pc(myl_artifact* a, const std::string& name, uint32_t n, std::vector<uint8_t>* out) {
    auto it = a->scales.find(name);
    if (it == a->scales.end()) return a->fail(MYL_E_INVALID, "missing calibrated activation scale in scales.json: " + name);
    const ArtScale& s = it->second;
    if (!s.has_shifts) {
        out->assign(n, (uint8_t)s.shift);
        return MYL_OK;
    }
    if (s.shifts.size() != n)
        return a->fail(MYL_E_INVALID, name + ": " + std::to_string(s.shifts.size()) + " per-channel shifts, expected " +
                                          std::to_string(n));
    out->resize(n);
    for (uint32_t i = 0; i < n; ++i) {
        if (s.shifts[i] < 0 || s.shifts[i] > 255)
            return a->fail(MYL_E_INVALID, name + ": shift " + std::to_string(s.shifts[i]) + " is outside 0..=255");
        (*out)[i] = (uint8_t)s.shifts[i];
    }
    return MYL_OK;
}

// require_tensor (loader.rs:690-695) plus the shape the forward pass reads.
int require_tensor(myl_artifact* a, const std::string& hf_name, uint64_t rows, uint64_t cols, bool upload) {
    const std::string key = myl::manifest_key(hf_name);
    auto it = a->weights.find(key);
    if (it == a->weights.end() || it->second.dtype != "int8")
        return a->fail(MYL_E_INVALID, "missing weight in the artifact: " + hf_name);
    const ArtWeight& w = it->second;
    const bool ok = cols ? (w.shape.size() == 2 && w.shape[0] == rows && w.shape[1] == cols)
                         : (w.shape.size() == 1 && w.shape[0] == rows);
    if (!ok) {
        std::string sh;
        for (uint64_t d : w.shape) sh += (sh.empty() ? "" : ", ") + std::to_string(d);
        return a->fail(MYL_E_INVALID, hf_name + ": shape [" + sh + "] does not match the model dimensions");
    }
    a->required.push_back(ArtRequired{key, hf_name, rows, cols, 8, upload});
    return MYL_OK;
}

// build_model (loader.rs:712-849): every tensor, scale and table the model
// consumes must be present with the shapes the dimensions imply.
int resolve_model(myl_artifact* a) {
    myl_model_dims& d = a->dims;
    const uint64_t H = d.hidden, I = d.inter, V = d.vocab, nq = (uint64_t)d.heads * d.head_dim,
                   nkv = (uint64_t)d.kv_heads * d.head_dim;
    auto lm16 = a->weights.find("lm_head");
    d.lm_head_int16 = lm16 != a->weights.end() ? 1 : 0;
    if (d.lm_head_int16) {
        const ArtWeight& w = lm16->second;
        if (w.shape.size() != 2 || w.shape[0] != V || w.shape[1] != H)
            return a->fail(MYL_E_INVALID, "LM head shape does not match vocab_size " + std::to_string(V) + " / hidden_size " +
                                              std::to_string(H));
        a->required.push_back(ArtRequired{"lm_head", "lm_head.weight", V, H, 16, true});
    }
    if (int rc = require_tensor(a, "model.embed_tokens.weight", V, H, true)) return rc;
    if (!d.tie_word_embeddings)
        if (int rc = require_tensor(a, "lm_head.weight", V, H, !d.lm_head_int16)) return rc;
    if (int rc = require_tensor(a, "model.norm.weight", H, 0, true)) return rc;
    if (int rc = require_scale(a, "model.norm", &a->final_norm_frac)) return rc;
    if (int rc = require_scale_pc(a, "model.norm.input", d.hidden, &a->final_res)) return rc;

    a->layer_fracs.resize(d.layers);
    a->res_in.resize(d.layers);
    a->res_mid.resize(d.layers);
    for (uint32_t l = 0; l < d.layers; ++l) {
        const std::string p = "model.layers." + std::to_string(l);
        if (d.attention_bias) {
            const char* sfx[3] = {"q_proj", "k_proj", "v_proj"};
            const uint64_t len[3] = {nq, nkv, nkv};
            for (int i = 0; i < 3; ++i) {
                const std::string hf = p + ".self_attn." + sfx[i] + ".bias";
                const std::string key = myl::manifest_key(hf);
                auto it = a->weights.find(key);
                if (it == a->weights.end() || it->second.dtype != "int16")
                    return a->fail(MYL_E_INVALID, "missing int16 bias '" + key +
                                                      "' in the artifact (artifacts before theta_v 0.13.0 carry int8 "
                                                      "biases and must be recalibrated)");
                if (it->second.shape[0] != len[i])
                    return a->fail(MYL_E_INVALID, "bias length of " + hf + " (" + std::to_string(it->second.shape[0]) +
                                                      ") does not match " + std::to_string(len[i]));
                a->required.push_back(ArtRequired{key, hf, len[i], 0, 16, true});
            }
        }
        myl_layer_fracs& f = a->layer_fracs[l];
        int rc = 0;
        if (!rc) rc = require_scale(a, p + ".input_layernorm", &f.norm_attn_frac);
        if (!rc) rc = require_scale(a, p + ".self_attn.q_proj", &f.q_frac);
        if (!rc) rc = require_scale(a, p + ".self_attn.k_proj", &f.k_frac);
        if (!rc) rc = require_scale(a, p + ".self_attn.v_proj", &f.v_frac);
        if (!rc) rc = require_scale(a, p + ".self_attn", &f.attn_out_frac);
        if (!rc) rc = require_scale(a, p + ".post_attention_layernorm", &f.norm_mlp_frac);
        if (!rc) rc = require_scale(a, p + ".mlp.gate_proj", &f.gate_frac);
        if (!rc) rc = require_scale(a, p + ".mlp.up_proj", &f.up_frac);
        if (!rc) rc = require_scale(a, p + ".mlp.down_proj.input", &f.down_in_frac);
        if (!rc) rc = require_scale_pc(a, p + ".input_layernorm.input", d.hidden, &a->res_in[l]);
        if (!rc) rc = require_scale_pc(a, p + ".post_attention_layernorm.input", d.hidden, &a->res_mid[l]);
        if (!rc) rc = require_tensor(a, p + ".input_layernorm.weight", H, 0, true);
        if (!rc) rc = require_tensor(a, p + ".post_attention_layernorm.weight", H, 0, true);
        if (!rc) rc = require_tensor(a, p + ".self_attn.q_proj.weight", nq, H, true);
        if (!rc) rc = require_tensor(a, p + ".self_attn.k_proj.weight", nkv, H, true);
        if (!rc) rc = require_tensor(a, p + ".self_attn.v_proj.weight", nkv, H, true);
        if (!rc) rc = require_tensor(a, p + ".self_attn.o_proj.weight", H, nq, true);
        if (!rc) rc = require_tensor(a, p + ".mlp.gate_proj.weight", I, H, true);
        if (!rc) rc = require_tensor(a, p + ".mlp.up_proj.weight", I, H, true);
        if (!rc) rc = require_tensor(a, p + ".mlp.down_proj.weight", H, I, true);
        if (rc) return rc;
    }
    for (const char* t : {"cos", "sin", "exp", "silu", "rsqrt"})
        if (!a->luts.count(t)) return a->fail(MYL_E_INVALID, std::string("missing lookup table in the artifact: ") + t);
    return MYL_OK;
}

void put_err(char* err, size_t cap, const std::string& msg) {
    if (!err || !cap) return;
    const size_t n = msg.size() < cap - 1 ? msg.size() : cap - 1;
    std::memcpy(err, msg.data(), n);
    err[n] = 0;
}

}  // namespace

extern "C" {

int myl_sha256_hex(const void* data, size_t n, char out[65]) {
    if ((!data && n) || !out) return MYL_E_INVALID;
    const std::string h = myl::Sha256::hex_of(data, n);
    std::memcpy(out, h.c_str(), 65);
    return MYL_OK;
}

int myl_artifact_open(const char* dir, myl_artifact** out, char* err, size_t err_cap) {
    if (!dir || !out) return MYL_E_INVALID;
    *out = nullptr;
    std::unique_ptr<myl_artifact> a(new (std::nothrow) myl_artifact());
    if (!a) return MYL_E_NOMEM;
    a->dir = dir;
    // load_model order (loader.rs:611-636), then build_model.
    int rc = read_theta_v(a.get());
    if (!rc) rc = read_dims(a.get());
    if (!rc) rc = read_weights(a.get());
    if (!rc) rc = read_scales(a.get());
    if (!rc) rc = read_luts(a.get());
    if (!rc) rc = verify_manifest_hashes(a.get());
    if (!rc) rc = resolve_model(a.get());
    if (rc) {
        put_err(err, err_cap, a->error);
        return rc;
    }
    put_err(err, err_cap, "");
    *out = a.release();
    return MYL_OK;
}

void myl_artifact_close(myl_artifact* a) { delete a; }

const char* myl_artifact_last_error(const myl_artifact* a) { return a ? a->error.c_str() : "no artifact"; }

int myl_artifact_dims(const myl_artifact* a, myl_model_dims* out) {
    if (!a || !out) return MYL_E_INVALID;
    *out = a->dims;
    return MYL_OK;
}

int myl_artifact_verify(myl_artifact* a) {
    if (!a) return MYL_E_INVALID;
    for (const auto& kv : a->weights) {
        const ArtWeight& w = kv.second;
        std::string d;
        if (!myl::art_hash_file(a->path(w.file), &d)) return a->fail(MYL_E_INVALID, "cannot read " + w.file);
        if (d != w.hash)
            return a->fail(MYL_E_INVALID, w.key + ": SHA-256 " + d + " does not match the manifest hash " + w.hash);
        std::vector<uint8_t> sh;
        if (int rc = myl::art_row_shifts(a, w, &sh)) return rc;
    }
    return MYL_OK;
}

int myl_artifact_lut(const myl_artifact* a, const char* name, int16_t* out, size_t cap, size_t* len) {
    if (!a || !name) return MYL_E_INVALID;
    auto it = a->luts.find(name);
    if (it == a->luts.end()) return MYL_E_INVALID;
    const std::vector<int16_t>& v = it->second.values;
    if (len) *len = v.size();
    if (out) {
        if (cap < v.size()) return MYL_E_INVALID;
        std::memcpy(out, v.data(), v.size() * 2);
    }
    return MYL_OK;
}

int myl_artifact_layer_scales(const myl_artifact* a, uint32_t layer, myl_layer_fracs* fracs, uint8_t* res_in,
                              uint8_t* res_mid) {
    if (!a || layer >= a->dims.layers) return MYL_E_INVALID;
    if (fracs) *fracs = a->layer_fracs[layer];
    if (res_in) std::memcpy(res_in, a->res_in[layer].data(), a->dims.hidden);
    if (res_mid) std::memcpy(res_mid, a->res_mid[layer].data(), a->dims.hidden);
    return MYL_OK;
}

int myl_artifact_final_scales(const myl_artifact* a, uint8_t* final_norm_frac, uint8_t* final_res) {
    if (!a) return MYL_E_INVALID;
    if (final_norm_frac) *final_norm_frac = a->final_norm_frac;
    if (final_res) std::memcpy(final_res, a->final_res.data(), a->dims.hidden);
    return MYL_OK;
}

}  // extern "C"
