// Checkpoint import for the device runtime: the safetensors repository of
// io/safetensors.rs:87-410 (single file or sharded index, header validation), the Qwen2 HF
// config and tensor plan of io/hf.rs:306-500, and a loader that moves each tensor's raw
// bytes to HBM and widens / transposes it there (fi_convert_to_f32) straight into the device
// model's weight buffers.
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <vector>

#include "fr_runtime.h"

namespace fr {

// io/safetensors.rs:11-45
enum class StDType : int32_t { F32 = 0, F16 = 1, BF16 = 2 };

struct StEntry {
  std::string path;
  StDType dtype = StDType::F32;
  std::vector<uint64_t> shape;
  uint64_t data_start = 0;  // 8 + header length
  uint64_t begin = 0, end = 0;  // data_offsets, relative to data_start
  uint64_t byte_len() const { return end - begin; }
  uint64_t absolute_offset() const { return data_start + begin; }
};

class SafeTensorsRepository {
 public:
  // model.safetensors.index.json when present, else model.safetensors (safetensors.rs:93-120).
  static SafeTensorsRepository open(const std::string& model_dir);
  size_t tensor_count() const { return tensors_.size(); }
  size_t shard_count() const { return shard_count_; }
  uint64_t total_data_bytes() const;
  const StEntry* get(const std::string& name) const;
  const std::map<std::string, StEntry>& tensors() const { return tensors_; }

 private:
  std::map<std::string, StEntry> tensors_;
  size_t shard_count_ = 0;
};

// One checkpoint tensor mapped to a device-model weight (hf.rs:47-53).
struct TensorPlan {
  std::string external_name, internal_name;
  std::vector<uint64_t> expected_source_shape;
  bool transpose = false;
  bool required = true;
};

// config.json of a Qwen2 checkpoint -> ModelConfig (hf.rs:306-369, 502-533).  The device
// decoder implements the SwiGLU (silu-gated) MLP only: other activations are Unsupported.
ModelConfig read_hf_config(const std::string& model_dir);
std::vector<TensorPlan> qwen2_tensor_plans(const ModelConfig& config);  // hf.rs:380-500

// hf.rs:66-118
struct HfInspection {
  size_t shard_count = 0, tensor_count = 0;
  uint64_t total_data_bytes = 0;
  size_t mapped_required = 0, mapped_optional = 0;
  std::vector<std::string> missing_required, missing_optional, shape_mismatches;
  bool compatible() const { return missing_required.empty() && shape_mismatches.empty(); }
};
HfInspection inspect_hf(const std::string& model_dir);

// Every planned tensor of the checkpoint into `model` (hf.rs:208-304 with the conversion of
// safetensors.rs:198-222 done on the device); returns the number of tensors loaded.
size_t load_hf_weights(DeviceModel* model, const std::string& model_dir);

}  // namespace fr
