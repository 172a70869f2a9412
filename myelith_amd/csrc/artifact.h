// artifact.h -- the parsed artifact directory (runtime/src/loader.rs:33-600),
// shared by the reader (artifact.cpp) and the device uploader (model_io.hip).
#pragma once

#include "../../include/myl_hip.h"

#include <cstdint>
#include <map>
#include <string>
#include <vector>

namespace myl {

// One weights_manifest.json entry (loader.rs:89-107, WeightManifestEntry).
struct ArtWeight {
    std::string key, original_name, file, dtype, hash;
    std::vector<uint64_t> shape;
    double scale = 0.0;
    int64_t shift = 0;
    bool has_shifts_file = false, has_shifts_hash = false;
    std::string shifts_file, shifts_hash;
    uint64_t elems() const {
        uint64_t n = 1;
        for (uint64_t d : shape) n *= d;
        return n;
    }
    int bits() const { return dtype == "int16" ? 16 : 8; }
};

// One scales.json entry (loader.rs:196-210, ScaleEntry).
struct ArtScale {
    int64_t shift = 0;
    double scale = 0.0;
    bool has_shifts = false;
    std::vector<int64_t> shifts;
};

// One luts.json entry (loader.rs:172-178) with its table.
struct ArtLut {
    std::string file, hash, dtype;
    uint64_t length = 0;
    std::vector<int16_t> values;
};

// A tensor the model consumes: the manifest key and the reference name the
// uploader takes (model.rs field <- HF original name, loader.rs:728-812).
struct ArtRequired {
    std::string key, name;
    uint64_t rows = 0, cols = 0;  // cols = 0 for 1-D tensors
    int bits = 8;
    bool upload = true;           // false: validated and hashed, not consumed
};

std::string manifest_key(const std::string& hf_name);

}  // namespace myl

struct myl_artifact;

namespace myl {
bool art_read_file(const std::string& path, std::string* out);
bool art_file_size(const std::string& path, uint64_t* n);
bool art_hash_file(const std::string& path, std::string* hex);
int art_row_shifts(const myl_artifact* a, const ArtWeight& w, std::vector<uint8_t>* out);
}  // namespace myl

struct myl_artifact {
    std::string dir;
    std::string version, weights_hash, scales_hash, luts_hash;  // theta_v.json
    std::string family, variant;
    myl_model_dims dims{};
    std::map<std::string, myl::ArtWeight> weights;  // by manifest key
    std::map<std::string, myl::ArtScale> scales;    // by module name
    std::map<std::string, myl::ArtLut> luts;        // by table name
    // resolved by the build_model checks (loader.rs:712-849)
    std::vector<myl::ArtRequired> required;
    std::vector<myl_layer_fracs> layer_fracs;
    std::vector<std::vector<uint8_t>> res_in, res_mid;
    std::vector<uint8_t> final_res;
    uint8_t final_norm_frac = 0;
    mutable std::string error;

    int fail(int code, const std::string& msg) const {
        error = msg;
        return code;
    }
    std::string path(const std::string& file) const { return dir + "/" + file; }
};
