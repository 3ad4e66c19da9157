// Shared host-side helpers: error state, the safetensors reader and the
// config loader.
#pragma once

#include <cstddef>
#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../../include/tmg.h"

namespace tmg {

// Sets the thread-local error text and returns `code`.
int set_error(int code, const std::string &msg);
void clear_error();
// The first n draws of the reference's StdRng::seed_from_u64(seed) +
// StandardUniform f32 (stdrng.cpp).
void stdrng_uniform(uint64_t seed, size_t n, float *out);

// ---- safetensors (reference src/safetensors_loader.rs:103-147) ----------

enum class DType { BF16, F16, F32, Other };

struct TensorEntry {
    std::string name;
    std::string dtype_name;
    DType dtype = DType::Other;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;  // byte offsets relative to the data section
    uint64_t numel() const {
        uint64_t n = 1;
        for (auto d : shape) n *= d;
        return n;
    }
};

// A read-only memory map of one .safetensors file with its parsed header.
class SafeTensorsFile {
  public:
    SafeTensorsFile() = default;
    ~SafeTensorsFile();
    SafeTensorsFile(const SafeTensorsFile &) = delete;
    SafeTensorsFile &operator=(const SafeTensorsFile &) = delete;

    // Returns TMG_OK or an error code (message via set_error).
    int open(const std::string &path);
    // A TMB1 file (reference src/tmb.rs) seen through the same interface:
    // every index entry becomes a 1-D tensor, BF16 for the weight matrices
    // and F32 for the embedding and norms, as the writer stores them.  The
    // embedded config is parsed into *cfg.
    int open_tmb(const std::string &path, tmg_config *cfg);
    const TensorEntry *find(const std::string &name) const;
    const uint8_t *data(const TensorEntry &e) const { return base_ + data_off_ + e.begin; }
    const std::vector<TensorEntry> &entries() const { return entries_; }

  private:
    int map_file(const std::string &path);
    std::string path_;
    uint8_t *base_ = nullptr;
    size_t size_ = 0;
    uint64_t data_off_ = 0;
    std::vector<TensorEntry> entries_;
    std::unordered_map<std::string, size_t> index_;
};

// Converts one element-wise tensor (BF16/F16/F32) to f32, as the reference
// does for norm weights and the embedding (src/model.rs:78-88, :192-199).
int tensor_to_f32(const SafeTensorsFile &f, const TensorEntry &e, std::vector<float> *out);

// f16 -> f32 (reference src/safetensors_loader.rs:149-173).
float f16_to_f32(uint16_t h);

// ---- config (reference src/config.rs:112-184) ----------------------------

int config_load(const std::string &path, tmg_config *out);
struct JsonValue;
int config_from_json(const JsonValue &cfg, tmg_config *out);

// ---- TMB1 (reference src/tmb.rs) --------------------------------------------

// True when the file starts with the TMB1 magic (reference is_tmb,
// src/model.rs:98-103).
bool is_tmb(const std::string &path);
// write_tmb (src/tmb.rs:137-262): repack a safetensors model (config.json
// next to it) into a TMB1 file.
int tmb_write(const std::string &src, const std::string &dst);
// config_path_for_model: <dir of model>/config.json if it exists.
bool config_path_for_model(const std::string &model_path, std::string *out);

}  // namespace tmg
