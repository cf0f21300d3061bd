// Safetensors repository, Qwen2 HF config / tensor plan and the device-side weight loader.
#include "fr_checkpoint.h"

#include <sys/stat.h>

#include <cmath>
#include <cstdio>
#include <memory>
#include <set>

#include "fr_json.h"

namespace fr {

namespace {

struct FileCloser {
  void operator()(std::FILE* f) const {
    if (f != nullptr) std::fclose(f);
  }
};
using File = std::unique_ptr<std::FILE, FileCloser>;

std::string join_path(const std::string& dir, const std::string& name) {
  if (dir.empty() || dir.back() == '/') return dir + name;
  return dir + "/" + name;
}

bool is_file(const std::string& path) {
  struct stat st {};
  return ::stat(path.c_str(), &st) == 0 && S_ISREG(st.st_mode);
}

File open_file(const std::string& path) {
  File f(std::fopen(path.c_str(), "rb"));
  if (!f) fail(ErrorKind::Io, "failed to open " + path);
  return f;
}

uint64_t file_length(std::FILE* f, const std::string& path) {
  if (::fseeko(f, 0, SEEK_END) != 0) fail(ErrorKind::Io, "failed to seek " + path);
  const off_t len = ::ftello(f);
  if (len < 0) fail(ErrorKind::Io, "failed to size " + path);
  return static_cast<uint64_t>(len);
}

void read_at(std::FILE* f, const std::string& path, uint64_t offset, void* dst, size_t bytes) {
  if (::fseeko(f, static_cast<off_t>(offset), SEEK_SET) != 0) fail(ErrorKind::Io, "failed to seek " + path);
  if (bytes > 0 && std::fread(dst, 1, bytes, f) != bytes) fail(ErrorKind::Io, "failed to read " + path);
}

std::string read_text(const std::string& path) {
  File f = open_file(path);
  const uint64_t len = file_length(f.get(), path);
  std::string text(static_cast<size_t>(len), '\0');
  read_at(f.get(), path, 0, text.data(), text.size());
  return text;
}

// Strict UTF-8 (no overlong forms, no surrogates, at most U+10FFFF), the rule of
// String::from_utf8 that safetensors.rs:260-267 applies to the header.
bool valid_utf8(const std::string& s) {
  size_t i = 0;
  const size_t n = s.size();
  while (i < n) {
    const unsigned char c = static_cast<unsigned char>(s[i]);
    if (c < 0x80) {
      ++i;
      continue;
    }
    int len;
    uint32_t cp, min;
    if ((c & 0xe0) == 0xc0) {
      len = 2, cp = c & 0x1f, min = 0x80;
    } else if ((c & 0xf0) == 0xe0) {
      len = 3, cp = c & 0x0f, min = 0x800;
    } else if ((c & 0xf8) == 0xf0) {
      len = 4, cp = c & 0x07, min = 0x10000;
    } else {
      return false;
    }
    if (i + len > n) return false;
    for (int k = 1; k < len; ++k) {
      const unsigned char d = static_cast<unsigned char>(s[i + k]);
      if ((d & 0xc0) != 0x80) return false;
      cp = (cp << 6) | (d & 0x3f);
    }
    if (cp < min || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
    i += len;
  }
  return true;
}

uint64_t dtype_size(StDType d) { return d == StDType::F32 ? 4 : 2; }

StDType parse_dtype(const std::string& s) {
  if (s == "F32") return StDType::F32;
  if (s == "F16") return StDType::F16;
  if (s == "BF16") return StDType::BF16;
  fail(ErrorKind::Unsupported, "safetensors dtype '" + s + "' is not supported yet");
}

// dtype size x element count with overflow checks (safetensors.rs:424-447); a rank-0 tensor
// holds one element.
uint64_t checked_byte_len(StDType dtype, const std::vector<uint64_t>& shape) {
  uint64_t count = 1;
  for (uint64_t d : shape) {
    if (d != 0 && count > UINT64_MAX / d) fail(ErrorKind::Runtime, "tensor element count overflow");
    count *= d;
  }
  const uint64_t size = dtype_size(dtype);
  if (count > UINT64_MAX / size) fail(ErrorKind::Runtime, "tensor byte length overflow");
  return count * size;
}

std::string shape_text(const std::vector<uint64_t>& shape) {
  std::string s = "[";
  for (size_t i = 0; i < shape.size(); ++i) s += (i ? ", " : "") + std::to_string(shape[i]);
  return s + "]";
}

// safetensors.rs:301-397
StEntry parse_entry(const std::string& path, uint64_t data_start, uint64_t file_len, const JsonValue& value) {
  value.as_object();
  StEntry e;
  e.path = path;
  e.data_start = data_start;
  const JsonValue* dtype = value.find("dtype");
  if (dtype == nullptr) fail(ErrorKind::Parse, "safetensors tensor entry is missing dtype");
  e.dtype = parse_dtype(dtype->as_str());
  const JsonValue* shape = value.find("shape");
  if (shape == nullptr) fail(ErrorKind::Parse, "safetensors tensor entry is missing shape");
  for (const JsonValue& d : shape->as_array()) e.shape.push_back(d.as_u64());
  const JsonValue* offsets = value.find("data_offsets");
  if (offsets == nullptr) fail(ErrorKind::Parse, "safetensors tensor entry is missing data_offsets");
  const auto& off = offsets->as_array();
  if (off.size() != 2) fail(ErrorKind::Parse, "safetensors tensor data_offsets must contain exactly two integers");
  e.begin = off[0].as_u64();
  e.end = off[1].as_u64();
  if (e.end < e.begin) fail(ErrorKind::Parse, "safetensors tensor data_offsets end must be >= start");
  const uint64_t expected = checked_byte_len(e.dtype, e.shape);
  if (e.byte_len() != expected) {
    fail(ErrorKind::InvalidType, "safetensors tensor byte length mismatch, expected " + std::to_string(expected) +
                                     " bytes but got " + std::to_string(e.byte_len()));
  }
  if (e.end > UINT64_MAX - data_start) fail(ErrorKind::Runtime, "safetensors tensor end offset overflow");
  if (data_start + e.end > file_len) fail(ErrorKind::Parse, "tensor data in '" + path + "' extends beyond file length");
  return e;
}

// safetensors.rs:225-299
std::map<std::string, StEntry> load_entries(const std::string& path) {
  File f = open_file(path);
  const uint64_t file_len = file_length(f.get(), path);
  if (file_len < 8) fail(ErrorKind::Io, "failed to read the header length of " + path);
  unsigned char len_bytes[8];
  read_at(f.get(), path, 0, len_bytes, 8);
  uint64_t header_len = 0;
  for (int i = 7; i >= 0; --i) header_len = (header_len << 8) | len_bytes[i];  // little endian
  if (header_len > UINT64_MAX - 8) fail(ErrorKind::Runtime, "safetensors header offset overflow");
  const uint64_t data_start = 8 + header_len;
  if (data_start > file_len) fail(ErrorKind::Parse, "safetensors file '" + path + "' is truncated");
  std::string header(static_cast<size_t>(header_len), '\0');
  read_at(f.get(), path, 8, header.data(), header.size());
  if (!valid_utf8(header)) fail(ErrorKind::Parse, "safetensors header in '" + path + "' is not valid UTF-8");
  const JsonValue root = JsonValue::parse(header);
  std::map<std::string, StEntry> entries;
  for (const auto& kv : root.as_object()) {
    if (kv.first == "__metadata__") continue;
    entries[kv.first] = parse_entry(path, data_start, file_len, kv.second);
  }
  return entries;
}

// hf.rs:604-690: required / optional config keys (null counts as absent).
const JsonValue* optional_key(const JsonValue& root, const std::string& key) {
  const JsonValue* v = root.find(key);
  return (v == nullptr || v->is_null()) ? nullptr : v;
}

uint64_t required_usize(const JsonValue& root, const std::string& key) { return root.get(key).as_u64(); }

float to_finite_f32(const JsonValue& v, const std::string& key) {
  const double d = v.as_f64();
  if (!std::isfinite(d)) fail(ErrorKind::Parse, "config key '" + key + "' must be finite");
  return static_cast<float>(d);
}

int32_t to_i32(uint64_t v, const std::string& key) {
  if (v > static_cast<uint64_t>(INT32_MAX)) fail(ErrorKind::InvalidConfig, "config key '" + key + "' is too large");
  return static_cast<int32_t>(v);
}

}  // namespace

// ----------------------------------------------------------------------------- repository
SafeTensorsRepository SafeTensorsRepository::open(const std::string& model_dir) {
  SafeTensorsRepository repo;
  const std::string index_path = join_path(model_dir, "model.safetensors.index.json");
  if (is_file(index_path)) {
    // safetensors.rs:122-162: every shard the weight map names, and only the mapped tensors
    const JsonValue index = JsonValue::parse(read_text(index_path));
    const auto& weight_map = index.get("weight_map").as_object();
    std::set<std::string> shard_names;
    for (const auto& kv : weight_map) shard_names.insert(kv.second.as_str());
    std::map<std::string, std::map<std::string, StEntry>> shards;
    for (const std::string& s : shard_names) shards[s] = load_entries(join_path(model_dir, s));
    for (const auto& kv : weight_map) {
      const std::string& shard = kv.second.as_str();
      const auto sit = shards.find(shard);
      if (sit == shards.end()) fail(ErrorKind::MissingWeight, "missing shard '" + shard + "' referenced by index");
      const auto eit = sit->second.find(kv.first);
      if (eit == sit->second.end()) {
        fail(ErrorKind::MissingWeight,
             "tensor '" + kv.first + "' referenced by index is absent from shard '" + shard + "'");
      }
      repo.tensors_[kv.first] = eit->second;
    }
    repo.shard_count_ = shards.size();
    return repo;
  }
  const std::string single = join_path(model_dir, "model.safetensors");
  if (is_file(single)) {
    repo.tensors_ = load_entries(single);
    repo.shard_count_ = 1;
    return repo;
  }
  fail(ErrorKind::Io, "no model.safetensors or model.safetensors.index.json found under " + model_dir);
}

uint64_t SafeTensorsRepository::total_data_bytes() const {
  uint64_t total = 0;
  for (const auto& kv : tensors_) total += kv.second.byte_len();
  return total;
}

const StEntry* SafeTensorsRepository::get(const std::string& name) const {
  const auto it = tensors_.find(name);
  return it == tensors_.end() ? nullptr : &it->second;
}

// ----------------------------------------------------------------------------- HF config
ModelConfig read_hf_config(const std::string& model_dir) {
  const JsonValue root = JsonValue::parse(read_text(join_path(model_dir, "config.json")));
  const std::string& model_type = root.get("model_type").as_str();
  if (model_type != "qwen2") fail(ErrorKind::Unsupported, "model_type '" + model_type + "' is not supported yet");
  const uint64_t hidden = required_usize(root, "hidden_size");
  const uint64_t intermediate = required_usize(root, "intermediate_size");
  const uint64_t heads = required_usize(root, "num_attention_heads");
  if (heads == 0 || hidden % heads != 0) {
    fail(ErrorKind::InvalidConfig, "hidden_size must be divisible by num_attention_heads");
  }
  const uint64_t head_dim = hidden / heads;
  const JsonValue* prf = optional_key(root, "partial_rotary_factor");
  const float factor = prf ? to_finite_f32(*prf, "partial_rotary_factor") : 1.0f;
  // ((head_dim as f32) * factor).round() as usize: f32 product, half away from zero, negative
  // values saturate to zero
  const float rot = std::round(static_cast<float>(head_dim) * factor);

  ModelConfig c;
  c.hidden_size = to_i32(hidden, "hidden_size");
  c.intermediate_size = to_i32(intermediate, "intermediate_size");
  c.num_layers = to_i32(required_usize(root, "num_hidden_layers"), "num_hidden_layers");
  c.num_attention_heads = to_i32(heads, "num_attention_heads");
  const JsonValue* kvh = optional_key(root, "num_key_value_heads");
  c.num_key_value_heads = kvh ? to_i32(kvh->as_u64(), "num_key_value_heads") : c.num_attention_heads;
  c.vocab_size = to_i32(required_usize(root, "vocab_size"), "vocab_size");
  c.max_position_embeddings = to_i32(required_usize(root, "max_position_embeddings"), "max_position_embeddings");
  c.rms_norm_eps = to_finite_f32(root.get("rms_norm_eps"), "rms_norm_eps");
  const JsonValue* theta = optional_key(root, "rope_theta");
  c.rope_theta = theta ? to_finite_f32(*theta, "rope_theta") : 10000.0f;
  c.rotary_dims = rot > 0.0f ? to_i32(static_cast<uint64_t>(std::min(rot, 2147483647.0f)), "rotary_dims") : 0;
  const JsonValue* tie = optional_key(root, "tie_word_embeddings");
  c.tie_word_embeddings = tie ? tie->as_bool() : false;
  // hf.rs:523-532 accepts silu / swish / gelu / relu; the device decoder is SwiGLU
  const std::string& act = root.get("hidden_act").as_str();
  if (act == "gelu" || act == "relu") {
    fail(ErrorKind::Unsupported, "activation '" + act + "' is not supported by the device decoder (silu-gated MLP only)");
  }
  if (act != "silu" && act != "swish") fail(ErrorKind::Unsupported, "activation '" + act + "' is not supported yet");
  return c;
}

std::vector<TensorPlan> qwen2_tensor_plans(const ModelConfig& c) {
  const uint64_t h = static_cast<uint64_t>(c.hidden_size), f = static_cast<uint64_t>(c.intermediate_size);
  const uint64_t v = static_cast<uint64_t>(c.vocab_size);
  const uint64_t kvw = static_cast<uint64_t>(c.num_key_value_heads) * static_cast<uint64_t>(c.head_dim());
  std::vector<TensorPlan> plans;
  auto add = [&](std::string ext, std::string internal, std::vector<uint64_t> shape, bool transpose, bool required) {
    plans.push_back(TensorPlan{std::move(ext), std::move(internal), std::move(shape), transpose, required});
  };
  add("model.embed_tokens.weight", "tok_embeddings.weight", {v, h}, false, true);
  for (int l = 0; l < c.num_layers; ++l) {
    const std::string src = "model.layers." + std::to_string(l) + ".";
    const std::string dst = "layers." + std::to_string(l) + ".";
    add(src + "input_layernorm.weight", dst + "attention_norm.weight", {h}, false, true);
    add(src + "self_attn.q_proj.weight", dst + "attention.wq.weight", {h, h}, true, true);
    add(src + "self_attn.k_proj.weight", dst + "attention.wk.weight", {kvw, h}, true, true);
    add(src + "self_attn.v_proj.weight", dst + "attention.wv.weight", {kvw, h}, true, true);
    add(src + "self_attn.o_proj.weight", dst + "attention.wo.weight", {h, h}, true, true);
    add(src + "post_attention_layernorm.weight", dst + "ffn_norm.weight", {h}, false, true);
    add(src + "mlp.up_proj.weight", dst + "feed_forward.w1.weight", {f, h}, true, true);
    add(src + "mlp.down_proj.weight", dst + "feed_forward.w2.weight", {h, f}, true, true);
    add(src + "mlp.gate_proj.weight", dst + "feed_forward.w3.weight", {f, h}, true, true);
    add(src + "self_attn.q_proj.bias", dst + "attention.wq.bias", {h}, false, false);
    add(src + "self_attn.k_proj.bias", dst + "attention.wk.bias", {kvw}, false, false);
    add(src + "self_attn.v_proj.bias", dst + "attention.wv.bias", {kvw}, false, false);
  }
  add("model.norm.weight", "norm.weight", {h}, false, true);
  if (!c.tie_word_embeddings) add("lm_head.weight", "output.weight", {v, h}, false, true);
  return plans;
}

HfInspection inspect_hf(const std::string& model_dir) {
  const ModelConfig config = read_hf_config(model_dir);
  const SafeTensorsRepository repo = SafeTensorsRepository::open(model_dir);
  HfInspection r;
  r.shard_count = repo.shard_count();
  r.tensor_count = repo.tensor_count();
  r.total_data_bytes = repo.total_data_bytes();
  for (const TensorPlan& p : qwen2_tensor_plans(config)) {
    const StEntry* e = repo.get(p.external_name);
    if (e == nullptr) {
      (p.required ? r.missing_required : r.missing_optional).push_back(p.external_name);
      continue;
    }
    if (e->shape != p.expected_source_shape) {
      r.shape_mismatches.push_back(p.external_name + " expected " + shape_text(p.expected_source_shape) +
                                   " but found " + shape_text(e->shape));
    }
    ++(p.required ? r.mapped_required : r.mapped_optional);
  }
  return r;
}

// ----------------------------------------------------------------------------- loader
size_t load_hf_weights(DeviceModel* model, const std::string& model_dir) {
  const SafeTensorsRepository repo = SafeTensorsRepository::open(model_dir);
  fi_context* ctx = model->ctx();
  std::map<std::string, File> files;  // one open handle per shard
  std::vector<unsigned char> host;
  DeviceBuffer staging;
  size_t loaded = 0;
  for (const TensorPlan& p : qwen2_tensor_plans(model->config())) {
    const StEntry* e = repo.get(p.external_name);
    if (e == nullptr) {
      if (p.required) fail(ErrorKind::MissingWeight, "missing required tensor '" + p.external_name + "'");
      continue;
    }
    if (e->shape != p.expected_source_shape) {
      fail(ErrorKind::InvalidShape, "tensor '" + p.external_name + "' expected shape " +
                                        shape_text(p.expected_source_shape) + " but found " + shape_text(e->shape));
    }
    if (p.transpose && e->shape.size() != 2) {
      fail(ErrorKind::InvalidShape, "only rank-2 tensors can be transposed during safetensors loading");
    }
    uint64_t count = 1;
    for (uint64_t d : e->shape) count *= d;  // bounded by the checked byte length
    const bool rank2 = e->shape.size() == 2;
    const int64_t rows = rank2 ? static_cast<int64_t>(e->shape[0]) : 1;
    const int64_t cols = rank2 ? static_cast<int64_t>(e->shape[1]) : static_cast<int64_t>(count);
    DeviceBuffer* slot = model->weight_slot(p.internal_name, static_cast<size_t>(count));
    const size_t bytes = static_cast<size_t>(e->byte_len());
    if (bytes > 0) {
      auto it = files.find(e->path);
      if (it == files.end()) it = files.emplace(e->path, open_file(e->path)).first;
      host.resize(bytes);
      read_at(it->second.get(), e->path, e->absolute_offset(), host.data(), bytes);
      staging.reserve(ctx, bytes);
      check(fi_buf_upload(ctx, staging.get(), bytes, host.data(), bytes));
      const int32_t dt = e->dtype == StDType::F32 ? FI_DTYPE_F32 : (e->dtype == StDType::BF16 ? FI_DTYPE_BF16 : FI_DTYPE_F16);
      check(fi_convert_to_f32(ctx, staging.get(), dt, rows, cols, p.transpose ? 1 : 0, slot->f32()));
      check(fi_ctx_sync(ctx));  // the host and device staging buffers are reused by the next tensor
    }
    ++loaded;
  }
  return loaded;
}

}  // namespace fr
