// Device-resident model, KV block pool and the batched decoder forward of the host runtime.
// Every device operation goes through the C ABI of include/ferrisinfer_kernel.h.
#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>

#include "fr_runtime.h"

namespace fr {

void fail(ErrorKind kind, const std::string& message) { throw Error{kind, message}; }

void check(int32_t status) {
  if (status != FI_OK) {
    const char* msg = fi_last_error();
    throw Error{static_cast<ErrorKind>(status - 1), msg ? msg : "backend error"};
  }
}

// ----------------------------------------------------------------------------- DeviceBuffer
DeviceBuffer::DeviceBuffer(fi_context* ctx, size_t bytes) { reserve(ctx, bytes); }

DeviceBuffer::~DeviceBuffer() {
  if (ptr_ != nullptr) (void)fi_buf_free(ctx_, ptr_);
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept : ctx_(o.ctx_), ptr_(o.ptr_), bytes_(o.bytes_) {
  o.ptr_ = nullptr;
  o.bytes_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept {
  if (this != &o) {
    if (ptr_ != nullptr) (void)fi_buf_free(ctx_, ptr_);
    ctx_ = o.ctx_;
    ptr_ = o.ptr_;
    bytes_ = o.bytes_;
    o.ptr_ = nullptr;
    o.bytes_ = 0;
  }
  return *this;
}

void DeviceBuffer::reserve(fi_context* ctx, size_t bytes) {
  if (bytes <= bytes_ && ptr_ != nullptr) return;
  if (ptr_ != nullptr) {
    check(fi_buf_free(ctx_, ptr_));
    ptr_ = nullptr;
    bytes_ = 0;
  }
  ctx_ = ctx;
  check(fi_buf_alloc(ctx, bytes == 0 ? 4 : bytes, &ptr_));
  bytes_ = bytes == 0 ? 4 : bytes;
}

// ----------------------------------------------------------------------------- model
void ModelConfig::validate() const {
  // model/config.rs:27-70
  if (hidden_size <= 0 || intermediate_size <= 0 || num_layers <= 0 || num_attention_heads <= 0 ||
      num_key_value_heads <= 0 || vocab_size <= 0 || max_position_embeddings <= 0) {
    fail(ErrorKind::InvalidConfig, "model dimensions must be greater than zero");
  }
  if (hidden_size % num_attention_heads != 0) fail(ErrorKind::InvalidConfig, "hidden_size must be divisible by num_attention_heads");
  if (num_attention_heads % num_key_value_heads != 0) {
    fail(ErrorKind::InvalidConfig, "num_attention_heads must be divisible by num_key_value_heads");
  }
  if (rotary_dims > head_dim()) fail(ErrorKind::InvalidConfig, "rope.rotary_dims cannot exceed attention head dimension");
}

DeviceModel::DeviceModel(fi_context* ctx, const ModelConfig& config, int32_t rope_positions, int32_t weight_dtype)
    : ctx_(ctx), config_(config), layers_(config.num_layers), rope_positions_(rope_positions),
      weight_dtype_(weight_dtype) {
  config.validate();
  if (weight_dtype != FI_DTYPE_F32 && weight_dtype != FI_DTYPE_BF16) {
    fail(ErrorKind::InvalidType, "projection weight dtype must be f32 or bf16");
  }
  const int pairs = config.rotary_dims / 2;
  if (pairs > 0) {
    rope_cos_.reserve(ctx, static_cast<size_t>(rope_positions) * pairs * sizeof(float));
    rope_sin_.reserve(ctx, static_cast<size_t>(rope_positions) * pairs * sizeof(float));
    check(fi_rope_table(ctx, rope_positions, config.head_dim(), config.rotary_dims, config.rope_theta,
                        rope_cos_.f32(), rope_sin_.f32()));
  }
}

void DeviceModel::set_weight(const std::string& name, const float* host, size_t count) {
  DeviceBuffer* dst = weight_slot(name, count);
  check(fi_buf_upload(ctx_, dst->get(), count * sizeof(float), host, count * sizeof(float)));
}

void DeviceModel::set_weight_device(const std::string& name, const void* device, int32_t src_dtype, size_t count) {
  DeviceBuffer* dst = weight_slot(name, count);
  check(fi_convert_to_f32(ctx_, device, src_dtype, 1, static_cast<int64_t>(count), 0, static_cast<float*>(dst->get())));
  check(fi_ctx_sync(ctx_));  // the caller may release the source once this returns
}

DeviceBuffer* DeviceModel::weight_slot(const std::string& name, size_t count) {
  if (finalized_) fail(ErrorKind::Runtime, "weights are packed; tensor " + name + " can no longer be set");
  const ModelConfig& c = config_;
  const size_t h = c.hidden_size, f = c.intermediate_size, kvw = static_cast<size_t>(c.num_key_value_heads) * c.head_dim();
  auto put = [&](DeviceBuffer* dst, size_t expected) {
    if (count != expected) {
      fail(ErrorKind::InvalidShape, "tensor " + name + " has " + std::to_string(count) + " elements, expected " +
                                        std::to_string(expected));
    }
    dst->reserve(ctx_, count * sizeof(float));
    return dst;
  };
  if (name == "tok_embeddings.weight") return put(&tok_embeddings_, static_cast<size_t>(c.vocab_size) * h);
  if (name == "norm.weight") return put(&norm_, h);
  if (name == "output.weight") return put(&output_, static_cast<size_t>(c.vocab_size) * h);
  const std::string prefix = "layers.";
  if (name.compare(0, prefix.size(), prefix) == 0) {
    const size_t dot = name.find('.', prefix.size());
    const std::string index = name.substr(prefix.size(), dot == std::string::npos ? std::string::npos : dot - prefix.size());
    if (dot == std::string::npos || index.empty() || index.size() > 9 ||
        index.find_first_not_of("0123456789") != std::string::npos) {
      fail(ErrorKind::MissingWeight, "unknown tensor name: " + name);
    }
    const int layer = std::stoi(index);
    if (layer >= c.num_layers) fail(ErrorKind::InvalidShape, "layer index out of range in " + name);
    const std::string rest = name.substr(dot + 1);
    Layer& w = layers_[layer];
    if (rest == "attention_norm.weight") return put(&w.attention_norm, h);
    if (rest == "attention.wq.weight") return put(&w.wq, h * h);
    if (rest == "attention.wq.bias") return put(&w.wq_bias, h);
    if (rest == "attention.wk.weight") return put(&w.wk, h * kvw);
    if (rest == "attention.wk.bias") return put(&w.wk_bias, kvw);
    if (rest == "attention.wv.weight") return put(&w.wv, h * kvw);
    if (rest == "attention.wv.bias") return put(&w.wv_bias, kvw);
    if (rest == "attention.wo.weight") return put(&w.wo, h * h);
    if (rest == "attention.wo.bias") return put(&w.wo_bias, h);
    if (rest == "ffn_norm.weight") return put(&w.ffn_norm, h);
    if (rest == "feed_forward.w1.weight") return put(&w.w1, h * f);
    if (rest == "feed_forward.w1.bias") return put(&w.w1_bias, f);
    if (rest == "feed_forward.w2.weight") return put(&w.w2, f * h);
    if (rest == "feed_forward.w2.bias") return put(&w.w2_bias, h);
    if (rest == "feed_forward.w3.weight") return put(&w.w3, h * f);
    if (rest == "feed_forward.w3.bias") return put(&w.w3_bias, f);
  }
  fail(ErrorKind::MissingWeight, "unknown tensor name: " + name);
}

void DeviceModel::validate() const {
  if (finalized_) return;  // checked before packing; the unpacked projections are gone
  // model/decoder.rs:30-52 required_weight_keys
  auto need = [](const DeviceBuffer& b, const std::string& name) {
    if (b.get() == nullptr) fail(ErrorKind::MissingWeight, "missing required tensor: " + name);
  };
  need(tok_embeddings_, "tok_embeddings.weight");
  for (int l = 0; l < config_.num_layers; ++l) {
    const Layer& w = layers_[l];
    const std::string p = "layers." + std::to_string(l) + ".";
    need(w.attention_norm, p + "attention_norm.weight");
    need(w.wq, p + "attention.wq.weight");
    need(w.wk, p + "attention.wk.weight");
    need(w.wv, p + "attention.wv.weight");
    need(w.wo, p + "attention.wo.weight");
    need(w.ffn_norm, p + "ffn_norm.weight");
    need(w.w1, p + "feed_forward.w1.weight");
    need(w.w2, p + "feed_forward.w2.weight");
    need(w.w3, p + "feed_forward.w3.weight");
  }
  need(norm_, "norm.weight");
  if (!config_.tie_word_embeddings) need(output_, "output.weight");
}

void DeviceModel::finalize() {
  if (finalized_) return;
  validate();
  const ModelConfig& c = config_;
  const int32_t h = c.hidden_size, f = c.intermediate_size, kvw = c.num_key_value_heads * c.head_dim();
  if (h % 4 != 0 || f % 4 != 0) {
    fail(ErrorKind::Unsupported, "hidden and intermediate sizes must be multiples of 4 for the packed projections");
  }
  auto floats = [](int32_t k, int32_t n, int32_t pw) {
    size_t out = 0;
    check(fi_weight_packed_floats(k, n, pw, &out));
    return out;
  };
  auto bf16_bytes = [](int32_t k, int32_t n, int32_t pair) {
    size_t out = 0;
    check(fi_weight_packed_bf16_elems(k, n, pair, &out));
    return out * sizeof(uint16_t);
  };
  packed_.resize(c.num_layers);
  for (int32_t l = 0; l < c.num_layers; ++l) {
    Layer& w = layers_[l];
    Packed& p = packed_[l];
    const int32_t ns[3] = {h, kvw, kvw};
    if (weight_dtype_ == FI_DTYPE_BF16) {
      const void* srcs[3] = {w.wq.get(), w.wk.get(), w.wv.get()};
      p.qkv.reserve(ctx_, bf16_bytes(h, h + 2 * kvw, 0));
      check(fi_weight_pack_bf16_columns(ctx_, srcs, ns, 3, FI_DTYPE_F32, h, static_cast<uint16_t*>(p.qkv.get())));
      p.wo.reserve(ctx_, bf16_bytes(h, h, 0));
      check(fi_weight_pack_bf16(ctx_, w.wo.get(), FI_DTYPE_F32, 0, h, h, static_cast<uint16_t*>(p.wo.get())));
      p.w13.reserve(ctx_, bf16_bytes(h, f, 1));
      check(fi_weight_pack_bf16_pair(ctx_, w.w1.get(), w.w3.get(), FI_DTYPE_F32, h, f,
                                     static_cast<uint16_t*>(p.w13.get())));
      p.w2.reserve(ctx_, bf16_bytes(f, h, 0));
      check(fi_weight_pack_bf16(ctx_, w.w2.get(), FI_DTYPE_F32, 0, f, h, static_cast<uint16_t*>(p.w2.get())));
    } else {
      const float* srcs[3] = {w.wq.f32(), w.wk.f32(), w.wv.f32()};
      p.qkv.reserve(ctx_, floats(h, h + 2 * kvw, kQkvPack) * sizeof(float));
      check(fi_weight_pack_columns(ctx_, srcs, ns, 3, h, kQkvPack, p.qkv.f32()));
      p.wo.reserve(ctx_, floats(h, h, kWoPack) * sizeof(float));
      check(fi_weight_pack(ctx_, w.wo.f32(), 0, h, h, kWoPack, p.wo.f32()));
      p.w13.reserve(ctx_, floats(h, 2 * f, 2) * sizeof(float));
      check(fi_weight_pack_pair(ctx_, w.w1.f32(), w.w3.f32(), h, f, p.w13.f32()));
      p.w2.reserve(ctx_, floats(f, h, kW2Pack) * sizeof(float));
      check(fi_weight_pack(ctx_, w.w2.f32(), 0, f, h, kW2Pack, p.w2.f32()));
    }
  }
  if (weight_dtype_ == FI_DTYPE_BF16) {
    lm_packed_.reserve(ctx_, bf16_bytes(h, c.vocab_size, 0));
    check(fi_weight_pack_bf16(ctx_, output_weight(), FI_DTYPE_F32, 1, h, c.vocab_size,
                              static_cast<uint16_t*>(lm_packed_.get())));
  } else {
    lm_packed_.reserve(ctx_, floats(h, c.vocab_size, kLmPack) * sizeof(float));
    check(fi_weight_pack(ctx_, output_weight(), 1, h, c.vocab_size, kLmPack, lm_packed_.f32()));
  }
  check(fi_ctx_sync(ctx_));
  for (Layer& w : layers_) {
    w.wq = DeviceBuffer();
    w.wk = DeviceBuffer();
    w.wv = DeviceBuffer();
    w.wo = DeviceBuffer();
    w.w1 = DeviceBuffer();
    w.w2 = DeviceBuffer();
    w.w3 = DeviceBuffer();
  }
  output_ = DeviceBuffer();
  finalized_ = true;
}

// ----------------------------------------------------------------------------- block pool
BlockPool::BlockPool(fi_context* ctx, int32_t layers, int32_t num_blocks, int32_t block_size, int32_t kv_heads,
                     int32_t head_dim, int32_t kv_dtype)
    : num_blocks_(num_blocks), block_size_(block_size), kv_dtype_(kv_dtype) {
  if (layers <= 0 || num_blocks <= 0 || block_size <= 0 || kv_heads <= 0 || head_dim <= 0) {
    fail(ErrorKind::InvalidConfig, "KV cache dimensions must be greater than zero");
  }
  if (kv_dtype != FI_DTYPE_F32 && kv_dtype != FI_DTYPE_BF16) fail(ErrorKind::InvalidType, "KV dtype must be f32 or bf16");
  free_.reserve(num_blocks);
  for (int32_t b = num_blocks - 1; b >= 0; --b) free_.push_back(b);
  refs_.assign(num_blocks, 0);
  const size_t elem = kv_dtype == FI_DTYPE_F32 ? 4 : 2;
  const size_t bytes = static_cast<size_t>(num_blocks) * kv_heads * block_size * head_dim * elem;
  for (int32_t l = 0; l < layers; ++l) {
    k_.emplace_back(ctx, bytes);
    v_.emplace_back(ctx, bytes);
  }
}

int32_t BlockPool::allocate() {
  if (free_.empty()) fail(ErrorKind::Runtime, "KV block pool ran out of free blocks");
  const int32_t b = free_.back();
  free_.pop_back();
  refs_[b] = 1;
  return b;
}

void BlockPool::incref(int32_t block) { refs_.at(block) += 1; }

void BlockPool::decref(int32_t block) {
  int32_t& r = refs_.at(block);
  if (r <= 0) fail(ErrorKind::Runtime, "KV block " + std::to_string(block) + " released twice");
  if (--r == 0) free_.push_back(block);
}

// ----------------------------------------------------------------------------- forward
ForwardExecutor::ForwardExecutor(const DeviceModel* model, BlockPool* pool, bool graph_decode)
    : model_(model), pool_(pool), ctx_(model->ctx()), graph_decode_(graph_decode) {}

ForwardExecutor::~ForwardExecutor() {
  // ticks still in flight read the buffers freed below
  if (!inflight_.empty()) (void)fi_ctx_sync(ctx_);
  drop_graphs();
  for (int i = 0; i < 2; ++i) {
    (void)fi_host_free(ctx_, h_meta_[i]);
    (void)fi_host_free(ctx_, h_out_[i]);
    (void)fi_event_destroy(events_[i]);
  }
}

void ForwardExecutor::host_reserve(int slot, size_t meta_bytes, size_t out_bytes) {
  auto fit = [&](void*& p, size_t& cap, size_t bytes) {
    if (bytes <= cap) return;
    const size_t want = (std::max(bytes, 2 * cap) + 4095) & ~static_cast<size_t>(4095);
    if (p != nullptr) {
      check(fi_host_free(ctx_, p));  // waits for the copies that may still use it
      p = nullptr;
      cap = 0;
    }
    check(fi_host_alloc(ctx_, want, &p));
    cap = want;
  };
  fit(h_meta_[slot], h_meta_bytes_[slot], meta_bytes);
  fit(h_out_[slot], h_out_bytes_[slot], out_bytes);
  if (events_[slot] == nullptr) check(fi_event_create(ctx_, &events_[slot]));
}

void ForwardExecutor::drop_graphs() {
  if (!graphs_.empty()) graph_drops_ += graphs_.size();
  for (auto& kv : graphs_) (void)fi_graph_destroy(kv.second);
  graphs_.clear();
  seen_.clear();
}

void ForwardExecutor::grow(DeviceBuffer& b, size_t bytes) {
  const void* before = b.get();
  b.reserve(ctx_, bytes);
  if (b.get() != before) buffers_moved_ += 1;
}

void ForwardExecutor::copy_only(const PackedBatch& b) {
  // A tick whose sequences only shared a prefix still owes the copy-on-write of a partially
  // filled shared block.
  const int32_t n = static_cast<int32_t>(b.copy_src.size());
  if (n == 0) return;
  std::vector<int32_t> host(b.copy_src);
  host.insert(host.end(), b.copy_dst.begin(), b.copy_dst.end());
  host.insert(host.end(), b.copy_count.begin(), b.copy_count.end());
  grow(meta_, host.size() * 4);
  check(fi_buf_upload(ctx_, meta_.get(), host.size() * 4, host.data(), host.size() * 4));
  const int32_t* d = static_cast<const int32_t*>(meta_.get());
  const ModelConfig& c = model_->config();
  for (int32_t l = 0; l < c.num_layers; ++l) {
    check(fi_kv_copy_blocks(ctx_, pool_->k(l), pool_->v(l), pool_->kv_dtype(), d, d + n, d + 2 * n, n,
                            pool_->num_blocks(), pool_->block_size(), c.num_key_value_heads, c.head_dim()));
  }
  check(fi_ctx_sync(ctx_));
  check(fi_ctx_check_faults(ctx_));
}

void ForwardExecutor::reserve(size_t tokens, size_t seqs) {
  if (tokens <= cap_tokens_ && seqs <= cap_seqs_) return;
  cap_tokens_ = std::max(tokens, cap_tokens_);
  cap_seqs_ = std::max(seqs, cap_seqs_);
  const ModelConfig& c = model_->config();
  const size_t t = cap_tokens_, h = c.hidden_size, f = c.intermediate_size;
  grow(hidden_, t * h * 4);
  grow(normed_, t * h * 4);
  grow(q_, t * h * 4);
  grow(attn_, t * h * 4);
  grow(h1_, t * h * 4);
  grow(act_, t * f * 4);
  grow(last_norm_, cap_seqs_ * h * 4);
  grow(out_, cap_seqs_ * 8);
}

void ForwardExecutor::splits(int32_t m, int32_t k, int32_t n, int32_t pack_width, int32_t* out) const {
  if (model_->weight_dtype() == FI_DTYPE_BF16) {
    check(fi_gemm_bf16_splits(ctx_, m, k, n, out));
  } else {
    check(fi_gemm_packed_splits(ctx_, m, k, n, pack_width, out));
  }
}

void ForwardExecutor::projection(const float* a, int32_t lda, const DeviceBuffer& w, int32_t k, int32_t n,
                                 int32_t pack_width, int32_t m, int32_t splits, float* out) const {
  if (model_->weight_dtype() == FI_DTYPE_BF16) {
    check(fi_gemm_bf16(ctx_, a, FI_DTYPE_F32, lda, static_cast<const uint16_t*>(w.get()), k, n, m, splits, out));
  } else {
    check(fi_gemm_packed(ctx_, a, lda, w.f32(), k, n, pack_width, m, splits, out));
  }
}

uint64_t sampler_state_new(uint64_t seed) { return seed == 0 ? 0x9e3779b97f4a7c15ULL : seed; }

uint64_t sampler_state_next(uint64_t x) {
  x ^= x >> 12;
  x ^= x << 25;
  x ^= x >> 27;
  return x;
}

// The launch sequence of one tick (runtime/reference.rs:372-423 / 664-710: embed, L blocks,
// final norm, head).  Block order as reference.rs:163-370: rmsnorm -> q,k,v (+bias) -> rope ->
// attention (the chunk's own K/V appended first, so they are read from the pool) -> wo (+bias)
// -> +x -> rmsnorm -> w1, w3 (+bias) -> silu(w3) * w1 -> w2 (+bias) -> +h1.  Each rmsnorm runs
// fused with the residual add before it; the last one applies the model's final norm.  Nothing
// here allocates, copies to or from the host or waits, so the sequence can be captured.
void ForwardExecutor::enqueue(const Plan& p) {
  const ModelConfig& c = model_->config();
  const int32_t T = p.T, B = p.B;
  const int32_t H = c.hidden_size, F = c.intermediate_size, hq = c.num_attention_heads;
  const int32_t hkv = c.num_key_value_heads, D = c.head_dim(), W = H + 2 * hkv * D;
  const float scale = 1.0f / std::sqrt(static_cast<float>(D));  // attention.rs:659
  const bool bf16 = model_->weight_dtype() == FI_DTYPE_BF16;
  // the fused decode path needs four-column RoPE items (rotary_dims / 2 and the pass-through
  // width multiples of 4)
  const bool fused_qkv_decode = (c.rotary_dims / 2) % 4 == 0 && (D - c.rotary_dims) % 4 == 0;
  float* hidden = hidden_.f32();
  float* normed = normed_.f32();
  float* q = q_.f32();
  float* attn = attn_.f32();
  float* h1 = h1_.f32();
  float* act = act_.f32();
  float* part = parts_.f32();

  check(fi_embedding(ctx_, model_->tok_embeddings(), c.vocab_size, H, p.ids, T, hidden));
  check(fi_rms_norm(ctx_, hidden, model_->layer(0).attention_norm.f32(), normed, T, H, c.rms_norm_eps));
  for (int32_t l = 0; l < c.num_layers; ++l) {
    const DeviceModel::Layer& w = model_->layer(l);
    const DeviceModel::Packed& pk = model_->packed(l);
    projection(normed, H, pk.qkv, H, W, DeviceModel::kQkvPack, T, p.s_qkv, part);
    if (p.kind == BatchKind::Decode && fused_qkv_decode) {
      // one launch: every attention workgroup forms its query rows from the partials and the
      // last partition of each sequence appends the new token's K/V before reading the keys.
      // The copy-on-write copies only committed rows, never the new token's slot, so it may
      // run first.
      if (p.n_copy > 0) {
        check(fi_kv_copy_blocks(ctx_, pool_->k(l), pool_->v(l), pool_->kv_dtype(), p.cs, p.cd, p.cc, p.n_copy,
                                pool_->num_blocks(), pool_->block_size(), hkv, D));
      }
      check(fi_attn_decode_paged_qkv(ctx_, part, p.s_qkv, w.wq_bias.f32(), w.wk_bias.f32(), w.wv_bias.f32(), p.pos,
                                     model_->rope_cos(), model_->rope_sin(), c.rotary_dims, model_->rope_positions(),
                                     p.slot, pool_->k(l), pool_->v(l), pool_->kv_dtype(), p.bt, p.max_blocks, p.ctx, B,
                                     p.max_context_len, hq, hkv, D, pool_->block_size(), pool_->num_blocks(), scale,
                                     q, attn));
    } else {
      check(fi_qkv_rope_append(ctx_, part, p.s_qkv, w.wq_bias.f32(), w.wk_bias.f32(), w.wv_bias.f32(), p.pos,
                               model_->rope_cos(), model_->rope_sin(), c.rotary_dims, model_->rope_positions(),
                               p.slot, pool_->k(l), pool_->v(l), pool_->kv_dtype(), pool_->num_blocks(),
                               pool_->block_size(), T, hq, hkv, D, q));
      if (p.n_copy > 0) {
        check(fi_kv_copy_blocks(ctx_, pool_->k(l), pool_->v(l), pool_->kv_dtype(), p.cs, p.cd, p.cc, p.n_copy,
                                pool_->num_blocks(), pool_->block_size(), hkv, D));
      }
      if (p.kind == BatchKind::Decode) {
        check(fi_attn_decode_paged(ctx_, q, pool_->k(l), pool_->v(l), pool_->kv_dtype(), p.bt, p.max_blocks, p.ctx,
                                   B, p.max_context_len, hq, hkv, D, pool_->block_size(), pool_->num_blocks(), scale,
                                   attn));
      } else {
        check(fi_attn_prefill_paged(ctx_, q, pool_->k(l), pool_->v(l), pool_->kv_dtype(), p.bt, p.max_blocks, p.cu,
                                    p.ctx, B, p.max_query_len, hq, hkv, D, pool_->block_size(),
                                    pool_->num_blocks(), scale, attn));
      }
    }
    projection(attn, H, pk.wo, H, H, DeviceModel::kWoPack, T, p.s_o, part);
    check(fi_splitk_residual_rms_norm(ctx_, part, p.s_o, w.wo_bias.f32(), hidden, h1, w.ffn_norm.f32(), normed, T, H,
                                      c.rms_norm_eps));
    if (bf16) {
      check(fi_gemm_bf16_swiglu(ctx_, normed, FI_DTYPE_F32, H, static_cast<const uint16_t*>(pk.w13.get()), H, F, T,
                                w.w1_bias.f32(), w.w3_bias.f32(), act, FI_DTYPE_F32));
    } else {
      check(fi_gemm_packed_swiglu(ctx_, normed, H, pk.w13.f32(), H, F, T, w.w1_bias.f32(), w.w3_bias.f32(), act));
    }
    projection(act, F, pk.w2, F, H, DeviceModel::kW2Pack, T, p.s_w2, part);
    const float* next_norm = l + 1 < c.num_layers ? model_->layer(l + 1).attention_norm.f32() : model_->norm();
    check(fi_splitk_residual_rms_norm(ctx_, part, p.s_w2, w.w2_bias.f32(), h1, hidden, next_norm, normed, T, H,
                                      c.rms_norm_eps));
  }
  // the final norm ran over every row; each sequence's last row feeds the head.  A decode tick
  // has one row per sequence, in sequence order, so the head reads the normed rows in place.
  const float* head_in = normed;
  if (!(p.kind == BatchKind::Decode && T == B)) {
    check(fi_embedding(ctx_, normed, T, H, p.last, B, last_norm_.f32()));
    head_in = last_norm_.f32();
  }
  const void* lm = model_->lm_head_packed();
  int32_t* tok = static_cast<int32_t*>(out_.get());
  float* prob = out_.f32() + B;
  if (p.greedy) {
    // fused greedy head (matmul_rhs_transposed_argmax_f32, matmul.rs:190-274), as the
    // reference session's greedy path (session.rs:349-356, 393-398)
    if (bf16) {
      check(fi_lm_head_argmax_bf16(ctx_, head_in, FI_DTYPE_F32, H, static_cast<const uint16_t*>(lm), B, H,
                                   c.vocab_size, tok, prob));
    } else {
      check(fi_lm_head_argmax_packed(ctx_, head_in, H, static_cast<const float*>(lm), B, H, c.vocab_size,
                                     tok, prob));
    }
  } else {
    // last-row logits (matmul_rhs_transposed, one K split) and sample_last_token per row
    // (session.rs:357-373, 399-406) with each sequence's sampler state; the states and the
    // per-row configuration were uploaded to samp_ before this sequence
    float* logits = logits_[p.ss].f32();
    if (bf16) {
      check(fi_gemm_bf16(ctx_, head_in, FI_DTYPE_F32, H, static_cast<const uint16_t*>(lm), H, c.vocab_size,
                         B, 1, logits));
    } else {
      check(fi_gemm_packed(ctx_, head_in, H, static_cast<const float*>(lm), H, c.vocab_size,
                           DeviceModel::kLmPack, B, 1, logits));
    }
    uint8_t* d = static_cast<uint8_t*>(samp_[p.ss].get());
    check(fi_sample_tokens(ctx_, logits, c.vocab_size, B, c.vocab_size, reinterpret_cast<const float*>(d + B * 8),
                           reinterpret_cast<const int32_t*>(d + B * 12), reinterpret_cast<const float*>(d + B * 16),
                           reinterpret_cast<uint64_t*>(d), tok, prob));
  }
}

void ForwardExecutor::last_logits(float* host, size_t capacity, int64_t* rows) const {
  const int32_t lrows = samp_last_ >= 0 ? logits_rows_[samp_last_] : 0;
  const size_t n = static_cast<size_t>(lrows) * model_->config().vocab_size;
  if (n > capacity) fail(ErrorKind::InvalidShape, "last logits need " + std::to_string(n) + " floats");
  // the slot of the last returned tick: a tick enqueued behind it writes the other one
  if (n) check(fi_buf_download(ctx_, host, n * sizeof(float), logits_[samp_last_].get(), n * sizeof(float)));
  *rows = lrows;
}

std::vector<TokenSample> ForwardExecutor::run(const PackedBatch& b, const SamplerConfig& sampler,
                                              std::vector<uint64_t>* states) {
  launch(b, sampler, states);
  return collect(states);
}

bool ForwardExecutor::can_feed(const PackedBatch& b) const {
  // out_ holds the previous launch's samples; reserve() reallocates it only past cap_seqs_ rows
  return inflight_.size() == 1 && inflight_.front().B > 0 && b.kind == BatchKind::Decode &&
         b.copy_src.empty() && !b.context_lens.empty() && b.context_lens.size() <= cap_seqs_;
}

void ForwardExecutor::launch(const PackedBatch& b, const SamplerConfig& sampler, const std::vector<uint64_t>* states,
                             const std::vector<int32_t>* feed) {
  const auto t_start = std::chrono::steady_clock::now();
  enqueue_s_ = 0.0;
  if (inflight_.size() >= 2) fail(ErrorKind::Runtime, "two ticks are already in flight");
  const ModelConfig& c = model_->config();
  const int32_t T = static_cast<int32_t>(b.token_ids.size());
  const int32_t B = static_cast<int32_t>(b.context_lens.size());
  if (feed != nullptr && (feed->size() != static_cast<size_t>(B) || T != B || !can_feed(b))) {
    fail(ErrorKind::Runtime, "a tick fed from the previous tick's samples must be a decode tick behind it");
  }
  if (T == 0 || B == 0) {
    copy_only(b);  // waits for the stream
    inflight_.push_back(Pending{-1, 0, true, 0});
    return;
  }
  if (!model_->finalized()) fail(ErrorKind::Runtime, "model weights are not packed (DeviceModel::finalize)");
  reserve(T, B);
  const int32_t H = c.hidden_size, F = c.intermediate_size, W = H + 2 * c.num_key_value_heads * c.head_dim();
  const bool greedy = sampler.is_greedy();
  // A graph records the copy-on-write launch and its pair count; the shape key does not carry
  // them, so a decode tick with copies runs eagerly (today only prefill ticks carry copies).
  const bool use_graph = graph_decode_ && b.kind == BatchKind::Decode && b.copy_src.empty();

  Plan p{};
  p.kind = b.kind;
  p.T = T;
  p.B = B;
  p.max_query_len = b.max_query_len;
  p.n_copy = static_cast<int32_t>(b.copy_src.size());
  p.greedy = greedy;
  p.max_blocks = b.max_blocks;
  p.max_context_len = b.max_context_len;
  // split-K counts of the three partial-output projections; one partials buffer serves all
  splits(T, H, W, DeviceModel::kQkvPack, &p.s_qkv);
  splits(T, H, H, DeviceModel::kWoPack, &p.s_o);
  splits(T, F, H, DeviceModel::kW2Pack, &p.s_w2);
  const size_t parts = std::max({static_cast<size_t>(p.s_qkv) * T * W, static_cast<size_t>(p.s_o) * T * H,
                                 static_cast<size_t>(p.s_w2) * T * H});
  if (parts > cap_parts_) {
    grow(parts_, parts * 4);
    cap_parts_ = parts;
  }

  // The block table as uploaded: the packer's [B, max_blocks], or, for a replayable decode tick,
  // padded to the width of max_context_len rounded up to kGraphContextBucket tokens.
  const int32_t bs = pool_->block_size();
  std::vector<int32_t> padded;
  const std::vector<int32_t>* tables = &b.block_tables;
  if (use_graph) {
    const int64_t bucket = ((static_cast<int64_t>(b.max_context_len) + kGraphContextBucket - 1) / kGraphContextBucket) *
                           kGraphContextBucket;
    p.max_context_len = static_cast<int32_t>(std::max<int64_t>(bucket, kGraphContextBucket));
    p.max_blocks = (p.max_context_len + bs - 1) / bs;
    if (p.max_blocks < b.max_blocks) fail(ErrorKind::Runtime, "graph block-table width below the packed width");
    padded.assign(static_cast<size_t>(B) * p.max_blocks, 0);
    for (int32_t i = 0; i < B; ++i) {
      std::copy(b.block_tables.begin() + static_cast<size_t>(i) * b.max_blocks,
                b.block_tables.begin() + static_cast<size_t>(i + 1) * b.max_blocks,
                padded.begin() + static_cast<size_t>(i) * p.max_blocks);
    }
    tables = &padded;
  }

  // One upload of all integer metadata (8-byte aligned sections).
  std::vector<uint8_t> host;
  auto section = [&](const void* data, size_t bytes) {
    size_t off = (host.size() + 7) & ~static_cast<size_t>(7);
    host.resize(off + bytes);
    if (bytes) std::memcpy(host.data() + off, data, bytes);
    return off;
  };
  const size_t o_ids = section(b.token_ids.data(), b.token_ids.size() * 4);
  const size_t o_pos = section(b.positions.data(), b.positions.size() * 4);
  const size_t o_slot = section(b.slot_mapping.data(), b.slot_mapping.size() * 8);
  const size_t o_cu = section(b.cu_seqlens.data(), b.cu_seqlens.size() * 4);
  const size_t o_ctx = section(b.context_lens.data(), b.context_lens.size() * 4);
  const size_t o_bt = section(tables->data(), tables->size() * 4);
  const size_t o_last = section(b.last_rows.data(), b.last_rows.size() * 4);
  const size_t o_cs = section(b.copy_src.data(), b.copy_src.size() * 4);
  const size_t o_cd = section(b.copy_dst.data(), b.copy_dst.size() * 4);
  const size_t o_cc = section(b.copy_count.data(), b.copy_count.size() * 4);
  // last, so the sections above keep the offsets the graphs recorded; present in every launch
  // (all -1 when nothing is fed), so the buffer's size does not depend on feeding
  std::vector<int32_t> no_feed;
  if (feed == nullptr) no_feed.assign(static_cast<size_t>(B), -1);
  const size_t o_feed = section(feed ? feed->data() : no_feed.data(), static_cast<size_t>(B) * 4);
  // the same rows for the 8-byte sampler states, as pairs of 4-byte words
  std::vector<int32_t> feed2(static_cast<size_t>(B) * 2, -1);
  if (feed != nullptr) {
    for (int32_t i = 0; i < B; ++i) {
      const int32_t r = (*feed)[static_cast<size_t>(i)];
      if (r >= 0) {
        feed2[2 * static_cast<size_t>(i)] = 2 * r;
        feed2[2 * static_cast<size_t>(i) + 1] = 2 * r + 1;
      }
    }
  }
  const size_t o_feed2 = section(feed2.data(), feed2.size() * 4);
  // a sampled tick's sampler buffer: states [B] u64, temperature [B] f32, top_k [B] i32,
  // top_p [B] f32, in the tick's sampling slot
  const int32_t ss = greedy ? 0 : samp_next_;
  std::vector<uint8_t> cfg;
  if (!greedy) {
    if (states == nullptr || states->size() != static_cast<size_t>(B)) {
      fail(ErrorKind::InvalidShape, "sampled batch requires one sampler state per sequence");
    }
    cfg.resize(static_cast<size_t>(B) * 20);
    std::memcpy(cfg.data(), states->data(), static_cast<size_t>(B) * 8);
    const int32_t k32 = static_cast<int32_t>(std::min<int64_t>(std::max<int64_t>(sampler.top_k, 0), INT32_MAX));
    for (int32_t i = 0; i < B; ++i) {
      std::memcpy(cfg.data() + B * 8 + i * 4, &sampler.temperature, 4);
      std::memcpy(cfg.data() + B * 12 + i * 4, &k32, 4);
      std::memcpy(cfg.data() + B * 16 + i * 4, &sampler.top_p, 4);
    }
  }
  // through the launch's pinned slot: the copies are ordered on the stream behind a tick still
  // in flight, which reads the previous contents
  const int32_t slot = next_slot_;
  const size_t cfg_off = (host.size() + 7) & ~static_cast<size_t>(7);
  host_reserve(slot, cfg_off + cfg.size(), static_cast<size_t>(B) * 16 + 16);
  std::memcpy(h_meta_[slot], host.data(), host.size());
  if (!cfg.empty()) std::memcpy(static_cast<uint8_t*>(h_meta_[slot]) + cfg_off, cfg.data(), cfg.size());
  grow(meta_, host.size());
  check(fi_buf_upload_async(ctx_, meta_.get(), host.size(), h_meta_[slot], host.size()));
  auto at = [&](size_t off) { return static_cast<uint8_t*>(meta_.get()) + off; };
  p.ids = reinterpret_cast<const int32_t*>(at(o_ids));
  p.pos = reinterpret_cast<const int32_t*>(at(o_pos));
  p.slot = reinterpret_cast<const int64_t*>(at(o_slot));
  p.cu = reinterpret_cast<const int32_t*>(at(o_cu));
  p.ctx = reinterpret_cast<const int32_t*>(at(o_ctx));
  p.bt = reinterpret_cast<const int32_t*>(at(o_bt));
  p.last = reinterpret_cast<const int32_t*>(at(o_last));
  p.cs = reinterpret_cast<const int32_t*>(at(o_cs));
  p.cd = reinterpret_cast<const int32_t*>(at(o_cd));
  p.cc = reinterpret_cast<const int32_t*>(at(o_cc));
  if (feed != nullptr) {
    check(fi_token_feed(ctx_, static_cast<const int32_t*>(out_.get()), out_rows_,
                        reinterpret_cast<const int32_t*>(at(o_feed)), B, reinterpret_cast<int32_t*>(at(o_ids))));
  }

  if (!greedy) {
    p.ss = ss;
    grow(logits_[ss], static_cast<size_t>(B) * c.vocab_size * 4);
    grow(samp_[ss], cfg.size());
    check(fi_buf_upload_async(ctx_, samp_[ss].get(), cfg.size(), static_cast<uint8_t*>(h_meta_[slot]) + cfg_off,
                              cfg.size()));
    if (feed != nullptr) {
      // fed rows continue from the states the previous tick advanced, in the other slot
      check(fi_token_feed(ctx_, static_cast<const int32_t*>(samp_[ss ^ 1].get()), 2 * out_rows_,
                          reinterpret_cast<const int32_t*>(at(o_feed2)), 2 * B,
                          static_cast<int32_t*>(samp_[ss].get())));
    }
    // top_k above 1024 (after clamping to the vocabulary) samples from a reserved area; a
    // reallocation bumps the workspace generation, which drops the captured graphs below
    if (std::min<int64_t>(std::max<int64_t>(sampler.top_k, 1), c.vocab_size) > 1024) {
      check(fi_sample_reserve(ctx_, B, c.vocab_size));
    }
    logits_rows_[ss] = B;
    samp_next_ = ss ^ 1;
  }

  if (use_graph) {
    uint64_t ws = 0;
    check(fi_ctx_workspace_generation(ctx_, &ws));
    if (ws != graphs_workspace_ || buffers_moved_ != graphs_buffers_) {
      drop_graphs();
      graphs_workspace_ = ws;
      graphs_buffers_ = buffers_moved_;
    }
    const std::array<int32_t, 4> key{B, p.max_blocks, p.max_context_len, greedy ? 1 : 2 + ss};
    auto it = graphs_.find(key);
    if (it != graphs_.end()) {
      check(fi_graph_launch(ctx_, it->second));
      graph_replays_ += 1;
    } else if (seen_[key]++ == 0) {
      enqueue(p);  // first occurrence: eager, sizing the context workspace for this shape
    } else {
      check(fi_graph_begin(ctx_));
      fi_graph* g = nullptr;
      try {
        enqueue(p);
      } catch (...) {
        (void)fi_graph_end(ctx_, nullptr);
        throw;
      }
      check(fi_graph_end(ctx_, &g));
      graphs_[key] = g;
      graph_captures_ += 1;
      check(fi_graph_launch(ctx_, g));
      graph_replays_ += 1;
    }
  } else {
    enqueue(p);
  }

  // the samples (B ids, then B probabilities), the fault words and a sampled tick's advanced
  // states into the pinned slot
  out_rows_ = B;
  uint8_t* h = static_cast<uint8_t*>(h_out_[slot]);
  check(fi_buf_download_async(ctx_, h, static_cast<size_t>(B) * 8, out_.get(), static_cast<size_t>(B) * 8));
  check(fi_ctx_faults_async(ctx_, reinterpret_cast<uint32_t*>(h + static_cast<size_t>(B) * 8)));
  if (!greedy) {
    check(fi_buf_download_async(ctx_, h + static_cast<size_t>(B) * 8 + 16, static_cast<size_t>(B) * 8,
                                samp_[ss].get(), static_cast<size_t>(B) * 8));
  }
  check(fi_event_record(ctx_, events_[slot]));
  inflight_.push_back(Pending{slot, B, greedy, ss});
  next_slot_ ^= 1;
  enqueue_s_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_start).count();
}

std::vector<TokenSample> ForwardExecutor::collect(std::vector<uint64_t>* states) {
  const auto t_start = std::chrono::steady_clock::now();
  wait_s_ = 0.0;
  if (inflight_.empty()) fail(ErrorKind::Runtime, "no tick in flight");
  const Pending p = inflight_.front();
  inflight_.pop_front();
  if (p.B == 0) return {};
  check(fi_event_wait(events_[p.slot]));
  const uint8_t* h = static_cast<const uint8_t*>(h_out_[p.slot]);
  uint32_t words[4];
  std::memcpy(words, h + static_cast<size_t>(p.B) * 8, sizeof(words));
  // a fault bit: the check waits for the stream, reports and clears it
  if ((words[0] | words[1] | words[2] | words[3]) != 0) check(fi_ctx_check_faults(ctx_));
  if (!p.greedy) {
    if (states == nullptr || states->size() != static_cast<size_t>(p.B)) {
      fail(ErrorKind::InvalidShape, "sampled batch requires one sampler state per sequence");
    }
    std::memcpy(states->data(), h + static_cast<size_t>(p.B) * 8 + 16, static_cast<size_t>(p.B) * 8);
  }
  samp_last_ = p.greedy ? -1 : p.ss;
  std::vector<TokenSample> out(p.B);
  for (int32_t i = 0; i < p.B; ++i) {
    int32_t id;
    float prob;
    std::memcpy(&id, h + static_cast<size_t>(i) * 4, 4);
    std::memcpy(&prob, h + static_cast<size_t>(p.B + i) * 4, 4);
    out[i] = TokenSample{static_cast<uint32_t>(id), prob};
  }
  wait_s_ = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_start).count();
  return out;
}

void ForwardExecutor::discard() {
  if (inflight_.empty()) return;
  const Pending p = inflight_.front();
  inflight_.pop_front();
  if (p.B == 0) return;
  check(fi_event_wait(events_[p.slot]));
  uint32_t words[4];
  std::memcpy(words, static_cast<const uint8_t*>(h_out_[p.slot]) + static_cast<size_t>(p.B) * 8, sizeof(words));
  if ((words[0] | words[1] | words[2] | words[3]) != 0) check(fi_ctx_check_faults(ctx_));
}

}  // namespace fr
