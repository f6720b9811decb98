// Safetensors checkpoints, memory-mapped (crates/orion-models/src/loader.rs):
// every `*.safetensors` file of a model directory, in sorted path order, is
// mapped and its header parsed; a tensor name resolves to the first file
// holding it (loader.rs:119-156).  Tensors stay in the file's dtype: the
// device upload converts (bf16 is copied as is), where the reference widens
// every tensor to f32 at this boundary (loader.rs:74-98).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

namespace orion {

struct CheckpointTensor {
  std::string name;
  std::string dtype_name;  // as written in the header ("BF16", "F32", ...)
  int dtype = -1;          // ORION_DTYPE_F32 / F16 / BF16, or -1 (unsupported)
  std::vector<int64_t> shape;
  const void* data = nullptr;  // inside the file mapping
  size_t bytes = 0;
};

class Checkpoint {
 public:
  // Error kinds, as the reference's ModelError names them.
  enum class Error { kNone, kPathNotFound, kMissingFile, kIo, kMalformed };

  static std::unique_ptr<Checkpoint> open(const std::string& dir, Error* kind, std::string* err);
  ~Checkpoint();
  Checkpoint(const Checkpoint&) = delete;
  Checkpoint& operator=(const Checkpoint&) = delete;

  size_t num_shards() const { return maps_.size(); }
  const std::vector<std::string>& names() const { return names_; }  // sorted
  const CheckpointTensor* find(const std::string& name) const;

 private:
  Checkpoint() = default;
  struct Map {
    std::string path;
    void* base = nullptr;
    size_t size = 0;
  };
  std::vector<Map> maps_;
  std::map<std::string, CheckpointTensor> index_;
  std::vector<std::string> names_;
};

}  // namespace orion
