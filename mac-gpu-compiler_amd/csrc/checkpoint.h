// Safetensors checkpoint + config.json reader, and the seeded random-init writer.
//
// Reader: the file contract of Model::load_model / Model::weight
// (metal_infrence_engine/src/cpu_inference.rs:58-96): u64 little-endian header length, a JSON
// object {name: {dtype, shape, data_offsets}} (plus an ignored "__metadata__"), then the data
// section, which must be 2-byte aligned; config.json sits next to the weights file.
#pragma once

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/qe.h"

namespace qe {

struct TensorInfo {
  std::string name;
  std::string dtype;
  std::vector<int64_t> shape;
  int64_t off0 = 0, off1 = 0;  // byte offsets into the data section
};

class Checkpoint {
 public:
  Checkpoint() = default;
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;
  ~Checkpoint();

  // Returns QE_OK or a QE_ERR_* code with a message in err.
  int open(const std::string& path, std::string& err);

  const qe_config& config() const { return cfg_; }
  const std::vector<TensorInfo>& tensors() const { return tensors_; }

  // BF16 view of a tensor with exactly `numel` elements (Model::weight's checks,
  // cpu_inference.rs:87-96). Returns nullptr and sets err on a missing name, a non-BF16
  // dtype, or a size mismatch.
  const uint16_t* bf16(const std::string& name, uint64_t numel, std::string& err) const;

  // bench.rs:106-116: all tensor bytes except model.embed_tokens.weight, plus one row of it
  uint64_t weight_bytes_per_token() const;

 private:
  void* map_ = nullptr;
  size_t len_ = 0;
  const uint8_t* data_ = nullptr;
  size_t data_len_ = 0;
  std::vector<TensorInfo> tensors_;
  std::unordered_map<std::string, size_t> index_;
  qe_config cfg_{};
};

// Canonical Qwen3 tensor names for layer l (HF layout).
std::string layer_tensor(uint64_t l, const char* suffix);

// Writes a seeded random-init checkpoint (see qe_write_random_checkpoint in qe.h).
int write_random_checkpoint(const std::string& dir, uint64_t seed, const qe_config& cfg,
                            std::string& err);

void random_prompt(uint64_t seed, uint64_t n, uint32_t vocab, uint32_t* out);

}  // namespace qe
