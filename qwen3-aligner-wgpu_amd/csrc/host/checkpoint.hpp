// checkpoint.hpp -- the real-checkpoint loader: safetensors shards mapped
// read-only, the `-hf` tensor names mapped onto the original ones, tensors
// narrowed to the run's 16-bit format, config.json read into the model's
// dimensions, and the aligner built from them (src/weights.rs:207-290,
// src/config.rs:186-235, src/decoder.rs:570-633,816-871,
// src/audio_encoder_gpu.rs:235-335,737-782, src/align_inference.rs:356-450).
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

#include "qa_host.h"

namespace qah {

// safetensors dtypes this loader converts from (others are rejected on use).
enum StDtype : int { ST_F16 = 0, ST_BF16 = 1, ST_F32 = 2, ST_OTHER = 3 };

struct StTensor {
  int dtype = ST_OTHER;
  std::string dtype_name;
  std::vector<int64_t> shape;
  const uint8_t* data = nullptr;  // inside a mapped shard
  size_t bytes = 0;
  int64_t numel() const {
    int64_t n = 1;
    for (int64_t d : shape) n *= d;
    return n;
  }
};

class Checkpoint {
 public:
  Checkpoint() = default;
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;
  ~Checkpoint();

  // `dir` holds model.safetensors, or model.safetensors.index.json and the
  // shards it names, and normally config.json.
  static std::unique_ptr<Checkpoint> open(const std::string& dir, std::string* err);

  const StTensor* find(const std::string& name) const;
  size_t count() const { return tensors_.size(); }
  // Element-wise conversion to QA_F16 / QA_BF16 (round to nearest even) or
  // to f32; elems must equal the tensor's element count.
  bool read_h16(const std::string& name, int dtype, uint16_t* dst, int64_t elems,
                std::string* err) const;
  bool read_f32(const std::string& name, float* dst, int64_t elems, std::string* err) const;
  bool config(qah_ckpt_config* out, std::string* err) const;

 private:
  bool map_shard(const std::string& path, std::string* err);
  std::vector<std::pair<void*, size_t>> maps_;
  std::unordered_map<std::string, StTensor> tensors_;
  std::string config_text_;
};

// The audio tower's geometry for config.json's fields: frames per chunk,
// attention window in tokens, mel rows after the stem, chunks for
// max_seconds of audio.  Refuses a geometry the tower or the decoder cannot
// run (QA_EINVAL / QA_EUNSUPPORTED with a message in *err).
struct Geometry {
  int64_t cs, wlen, fdim, max_chunks;
};
int tower_geometry(const qah_ckpt_config& c, double max_seconds, Geometry* g, std::string* err);

// The aligner (tower, decoder, head and embedding) built from a checkpoint:
// shapes checked against config.json, weights narrowed to `dtype`.
int load_aligner(const Checkpoint& ck, qa_ctx* ctx, int dtype, double max_seconds, int max_rows,
                 qah_aenc** enc, qah_tdec** dec, qah_aligner** al, std::string* err);

}  // namespace qah
