// Oracle restatement of crates/ferrisinfer-runtime/src/{paged_kv,kv_cache,reference,session,
// sequence,prefix_index,block_manager,scheduler}.rs — TEST INFRASTRUCTURE ONLY (see oracle.h).
#include "oracle_runtime.h"

#include <algorithm>
#include <cstring>

namespace orc {

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

static void validate_kv_config(const KvCacheConfig& c) {
  // kv_cache.rs:599-617 / paged_kv.rs:798-816 (dtype is always f32 here)
  if (c.num_layers == 0 || c.num_kv_heads == 0 || c.head_dim == 0 || c.max_sequence_length == 0) {
    fail(ErrorKind::InvalidConfig, "KV cache dimensions must be greater than zero");
  }
}

static void validate_prefix_length(const KvCacheConfig& c, size_t length) {
  // paged_kv.rs:865-882
  if (length == 0) fail(ErrorKind::InvalidShape, "KV cache prefix length must be greater than zero");
  if (length > c.max_sequence_length) {
    fail(ErrorKind::InvalidShape, "KV cache prefix length " + std::to_string(length) +
                                      " exceeds capacity " + std::to_string(c.max_sequence_length));
  }
}

// ===========================================================================
// PagedKvCacheStorage (paged_kv.rs:164-792)
// ===========================================================================
PagedKvCacheStorage::PagedKvCacheStorage(const KvCacheConfig& config, size_t page_size)
    : config_(config), page_size_(page_size) {
  validate_kv_config(config);
  if (page_size == 0) fail(ErrorKind::InvalidConfig, "paged KV cache page size must be greater than zero");
  size_t page_count = div_ceil(config.max_sequence_length, page_size);
  size_t slot = slot_width();
  view_key_.assign(config.num_layers, std::vector<float>(config.max_sequence_length * slot, 0.0f));
  view_value_ = view_key_;
  pages_.resize(config.num_layers);
  block_tables_.assign(config.num_layers, std::vector<std::optional<size_t>>(page_count));
  free_ids_.resize(config.num_layers);
  for (size_t l = 0; l < config.num_layers; ++l) {
    for (size_t p = 0; p < page_count; ++p) {
      Page page;
      page.id = p;
      page.key.assign(page_size * slot, 0.0f);
      page.value.assign(page_size * slot, 0.0f);
      pages_[l].push_back(std::move(page));
    }
    // initial_free_page_ids: (0..n).rev(), so pop() hands out page 0 first (paged_kv.rs:794-796)
    for (size_t p = page_count; p-- > 0;) free_ids_[l].push_back(p);
  }
}

void PagedKvCacheStorage::check_layer(size_t layer) const {
  if (layer >= config_.num_layers) {
    fail(ErrorKind::InvalidShape, "KV cache layer index out of bounds: " + std::to_string(layer));
  }
}

const PagedKvCacheStorage::Page& PagedKvCacheStorage::page(size_t layer, size_t id) const {
  check_layer(layer);
  if (id >= pages_[layer].size()) {
    fail(ErrorKind::InvalidShape, "KV cache page id out of bounds for layer " +
                                      std::to_string(layer) + ": " + std::to_string(id));
  }
  return pages_[layer][id];
}

size_t PagedKvCacheStorage::allocated_page_count(size_t layer) const {
  check_layer(layer);
  size_t n = 0;
  for (const auto& s : block_tables_[layer]) n += s.has_value() ? 1 : 0;
  return n;
}

size_t PagedKvCacheStorage::free_page_count(size_t layer) const {
  check_layer(layer);
  return free_ids_[layer].size();
}

std::vector<KvCachePageInfo> PagedKvCacheStorage::page_infos(size_t layer) const {
  check_layer(layer);
  std::vector<KvCachePageInfo> out;
  for (const auto& p : pages_[layer]) {
    out.push_back({p.id, p.assigned_logical_block.value_or(0) * page_size_, p.committed_tokens});
  }
  return out;
}

std::vector<KvBlockTableEntry> PagedKvCacheStorage::block_table(size_t layer,
                                                                size_t token_count) const {
  // paged_kv.rs:260-314
  validate_prefix_length(config_, token_count);
  check_layer(layer);
  size_t remaining = token_count;
  size_t blocks = div_ceil(token_count, page_size_);
  std::vector<KvBlockTableEntry> table;
  for (size_t lb = 0; lb < blocks; ++lb) {
    if (lb >= block_tables_[layer].size() || !block_tables_[layer][lb].has_value()) {
      fail(ErrorKind::Runtime, "KV cache block table missing physical page for logical block " +
                                   std::to_string(lb));
    }
    size_t id = *block_tables_[layer][lb];
    const Page& p = page(layer, id);
    size_t from_page = std::min(remaining, page_size_);
    if (p.committed_tokens < from_page) {
      fail(ErrorKind::Runtime,
           "KV cache block table touched uncommitted tokens in page " + std::to_string(p.id));
    }
    table.push_back({lb, id, lb * page_size_, from_page});
    remaining -= from_page;
  }
  if (remaining != 0) fail(ErrorKind::Runtime, "KV cache block table ran out of committed pages");
  return table;
}

PrefixHandle PagedKvCacheStorage::capture_prefix_handle(size_t token_count) const {
  PrefixHandle h;
  h.token_count = token_count;
  h.page_size = page_size_;
  for (size_t l = 0; l < config_.num_layers; ++l) h.layer_block_tables.push_back(block_table(l, token_count));
  return h;
}

size_t PagedKvCacheStorage::allocate_page_for_logical_block(size_t layer, size_t lb) {
  // paged_kv.rs:469-527
  check_layer(layer);
  if (lb < block_tables_[layer].size() && block_tables_[layer][lb].has_value()) return *block_tables_[layer][lb];
  if (free_ids_[layer].empty()) {
    fail(ErrorKind::Runtime, "KV cache layer " + std::to_string(layer) + " ran out of free pages");
  }
  size_t id = free_ids_[layer].back();
  free_ids_[layer].pop_back();
  if (lb >= block_tables_[layer].size()) {
    fail(ErrorKind::InvalidShape, "KV cache logical block index out of bounds for layer " +
                                      std::to_string(layer) + ": " + std::to_string(lb));
  }
  block_tables_[layer][lb] = id;
  Page& p = pages_[layer][id];
  p.assigned_logical_block = lb;
  p.committed_tokens = 0;
  return id;
}

void PagedKvCacheStorage::reset() {
  // paged_kv.rs:529-549
  size_t n = page_count_per_layer();
  for (auto& layer : pages_) {
    for (auto& p : layer) {
      p.assigned_logical_block.reset();
      p.committed_tokens = 0;
    }
  }
  for (auto& t : block_tables_) std::fill(t.begin(), t.end(), std::nullopt);
  for (auto& f : free_ids_) {
    f.clear();
    for (size_t p = n; p-- > 0;) f.push_back(p);
  }
}

void PagedKvCacheStorage::import_prefix_from(const PagedKvCacheStorage& source,
                                             const PrefixHandle& handle) {
  // paged_kv.rs:329-389, 551-581
  if (page_size_ != source.page_size_ || page_size_ != handle.page_size) {
    fail(ErrorKind::InvalidConfig, "paged KV prefix import requires matching page sizes");
  }
  if (config_.num_layers != source.config_.num_layers ||
      config_.num_layers != handle.layer_block_tables.size() ||
      config_.num_kv_heads != source.config_.num_kv_heads ||
      config_.head_dim != source.config_.head_dim ||
      config_.max_sequence_length != source.config_.max_sequence_length) {
    fail(ErrorKind::InvalidConfig, "paged KV prefix import requires matching cache configurations");
  }
  if (handle.token_count > config_.max_sequence_length) {
    fail(ErrorKind::InvalidShape, "paged KV prefix handle length exceeds capacity");
  }
  reset();
  size_t slot = slot_width();
  for (size_t l = 0; l < handle.layer_block_tables.size(); ++l) {
    for (const auto& e : handle.layer_block_tables[l]) {
      const Page& src = source.page(l, e.block_id);
      if (src.committed_tokens < e.token_count) {
        fail(ErrorKind::Runtime, "KV cache prefix import touched uncommitted tokens in source block " +
                                     std::to_string(e.block_id));
      }
      size_t elems = e.token_count * slot;
      size_t off = e.start_position * slot;
      size_t dst_id = allocate_page_for_logical_block(l, e.logical_block_index);
      std::memcpy(view_key_[l].data() + off, src.key.data(), elems * sizeof(float));
      std::memcpy(view_value_[l].data() + off, src.value.data(), elems * sizeof(float));
      Page& dst = pages_[l][dst_id];
      std::memcpy(dst.key.data(), src.key.data(), elems * sizeof(float));
      std::memcpy(dst.value.data(), src.value.data(), elems * sizeof(float));
      dst.committed_tokens = e.token_count;
    }
  }
}

void PagedKvCacheStorage::write_slot(size_t layer, size_t position, const float* key,
                                     const float* value) {
  // paged_kv.rs:583-631
  if (position >= config_.max_sequence_length) fail(ErrorKind::Runtime, "KV cache capacity exceeded");
  size_t slot = slot_width();
  size_t lb = position / page_size_;
  size_t off = position % page_size_;
  size_t id = allocate_page_for_logical_block(layer, lb);
  std::memcpy(view_key_[layer].data() + position * slot, key, slot * sizeof(float));
  std::memcpy(view_value_[layer].data() + position * slot, value, slot * sizeof(float));
  Page& p = pages_[layer][id];
  std::memcpy(p.key.data() + off * slot, key, slot * sizeof(float));
  std::memcpy(p.value.data() + off * slot, value, slot * sizeof(float));
  p.committed_tokens = std::max(p.committed_tokens, off + 1);
}

void PagedKvCacheStorage::write_sequence(size_t layer, size_t start, size_t seq_len,
                                         const float* key, const float* value) {
  // paged_kv.rs:679-767
  if (start + seq_len > config_.max_sequence_length) fail(ErrorKind::Runtime, "KV cache capacity exceeded");
  size_t slot = slot_width();
  size_t t = 0;
  while (t < seq_len) {
    size_t position = start + t;
    size_t lb = position / page_size_;
    size_t off = position % page_size_;
    size_t in_page = std::min(page_size_ - off, seq_len - t);
    size_t id = allocate_page_for_logical_block(layer, lb);
    std::memcpy(view_key_[layer].data() + position * slot, key + t * slot, in_page * slot * sizeof(float));
    std::memcpy(view_value_[layer].data() + position * slot, value + t * slot, in_page * slot * sizeof(float));
    Page& p = pages_[layer][id];
    std::memcpy(p.key.data() + off * slot, key + t * slot, in_page * slot * sizeof(float));
    std::memcpy(p.value.data() + off * slot, value + t * slot, in_page * slot * sizeof(float));
    p.committed_tokens = std::max(p.committed_tokens, off + in_page);
    t += in_page;
  }
}

void PagedKvCacheStorage::read_prefix(size_t layer, size_t length, std::vector<float>* key,
                                      std::vector<float>* value) const {
  // paged_kv.rs:769-791: concatenate pages in block-table order
  validate_prefix_length(config_, length);
  size_t slot = slot_width();
  key->clear();
  value->clear();
  key->reserve(length * slot);
  value->reserve(length * slot);
  for (const auto& e : block_table(layer, length)) {
    const Page& p = page(layer, e.block_id);
    size_t n = e.token_count * slot;
    key->insert(key->end(), p.key.begin(), p.key.begin() + n);
    value->insert(value->end(), p.value.begin(), p.value.begin() + n);
  }
}

// ===========================================================================
// ContiguousKvCacheStorage (kv_cache.rs:66-270)
// ===========================================================================
ContiguousKvCacheStorage::ContiguousKvCacheStorage(const KvCacheConfig& config) : config_(config) {
  validate_kv_config(config);
  size_t n = config.max_sequence_length * config.num_kv_heads * config.head_dim;
  key_.assign(config.num_layers, std::vector<float>(n, 0.0f));
  value_ = key_;
}

void ContiguousKvCacheStorage::write_slot(size_t layer, size_t position, const float* key,
                                          const float* value) {
  if (layer >= config_.num_layers) fail(ErrorKind::InvalidShape, "KV cache layer index out of bounds: " + std::to_string(layer));
  size_t slot = config_.num_kv_heads * config_.head_dim;
  if ((position + 1) * slot > key_[layer].size()) fail(ErrorKind::InvalidShape, "tensor element range out of bounds");
  std::memcpy(key_[layer].data() + position * slot, key, slot * sizeof(float));
  std::memcpy(value_[layer].data() + position * slot, value, slot * sizeof(float));
}

void ContiguousKvCacheStorage::write_sequence(size_t layer, size_t start, size_t seq_len,
                                              const float* key, const float* value) {
  if (start + seq_len > config_.max_sequence_length) fail(ErrorKind::Runtime, "KV cache capacity exceeded");
  if (layer >= config_.num_layers) fail(ErrorKind::InvalidShape, "KV cache layer index out of bounds: " + std::to_string(layer));
  size_t slot = config_.num_kv_heads * config_.head_dim;
  std::memcpy(key_[layer].data() + start * slot, key, seq_len * slot * sizeof(float));
  std::memcpy(value_[layer].data() + start * slot, value, seq_len * slot * sizeof(float));
}

void ContiguousKvCacheStorage::read_prefix(size_t layer, size_t length, std::vector<float>* key,
                                           std::vector<float>* value) const {
  validate_prefix_length(config_, length);
  if (layer >= config_.num_layers) fail(ErrorKind::InvalidShape, "KV cache layer index out of bounds: " + std::to_string(layer));
  size_t n = length * config_.num_kv_heads * config_.head_dim;
  key->assign(key_[layer].begin(), key_[layer].begin() + n);
  value->assign(value_[layer].begin(), value_[layer].begin() + n);
}

// ===========================================================================
// KvCache (kv_cache.rs:359-597)
// ===========================================================================
KvCache KvCache::contiguous(const KvCacheConfig& config) {
  KvCache kv;
  kv.contiguous_ = std::make_shared<ContiguousKvCacheStorage>(config);
  return kv;
}

KvCache KvCache::paged(const KvCacheConfig& config, size_t page_size) {
  KvCache kv;
  kv.paged_ = std::make_shared<PagedKvCacheStorage>(config, page_size);
  return kv;
}

const KvCacheConfig& KvCache::config() const {
  return paged_ ? paged_->config() : contiguous_->config();
}

size_t KvCache::remaining_tokens() const {
  size_t max = config().max_sequence_length;
  return used_tokens_ >= max ? 0 : max - used_tokens_;
}

void KvCache::reset() {
  if (paged_) paged_->reset();
  used_tokens_ = 0;
}

void KvCache::advance(size_t tokens) {
  size_t next = used_tokens_ + tokens;
  if (next > config().max_sequence_length) fail(ErrorKind::Runtime, "KV cache capacity exceeded");
  used_tokens_ = next;
}

size_t KvCache::reserve_slot() {
  size_t position = used_tokens_;
  advance(1);
  return position;
}

void KvCache::write(size_t layer, size_t position, const float* key, const float* value) {
  if (position >= used_tokens_) {
    fail(ErrorKind::InvalidShape, "KV cache position " + std::to_string(position) +
                                      " has not been reserved yet; committed tokens " + std::to_string(used_tokens_));
  }
  if (paged_) {
    paged_->write_slot(layer, position, key, value);
  } else {
    contiguous_->write_slot(layer, position, key, value);
  }
}

void KvCache::write_uncommitted(size_t layer, size_t position, const float* key,
                                const float* value) {
  if (position > used_tokens_) {
    fail(ErrorKind::InvalidShape, "KV cache position " + std::to_string(position) +
                                      " is beyond the next writable slot " + std::to_string(used_tokens_));
  }
  if (paged_) {
    paged_->write_slot(layer, position, key, value);
  } else {
    contiguous_->write_slot(layer, position, key, value);
  }
}

void KvCache::write_sequence_uncommitted(size_t layer, size_t start, size_t seq_len,
                                         const float* key, const float* value) {
  if (start > used_tokens_) {
    fail(ErrorKind::InvalidShape, "KV cache sequence start " + std::to_string(start) +
                                      " is beyond committed tokens " + std::to_string(used_tokens_));
  }
  if (paged_) {
    paged_->write_sequence(layer, start, seq_len, key, value);
  } else {
    contiguous_->write_sequence(layer, start, seq_len, key, value);
  }
}

void KvCache::read_prefix(size_t layer, size_t length, std::vector<float>* key,
                          std::vector<float>* value) const {
  if (length > used_tokens_) {
    fail(ErrorKind::InvalidShape, "KV cache prefix length " + std::to_string(length) +
                                      " exceeds committed tokens " + std::to_string(used_tokens_));
  }
  if (paged_) {
    paged_->read_prefix(layer, length, key, value);
  } else {
    contiguous_->read_prefix(layer, length, key, value);
  }
}

std::optional<PrefixHandle> KvCache::prefix_handle(size_t token_count) const {
  if (token_count == 0) return std::nullopt;
  if (token_count > used_tokens_) {
    fail(ErrorKind::InvalidShape, "KV cache prefix handle length " + std::to_string(token_count) +
                                      " exceeds committed tokens " + std::to_string(used_tokens_));
  }
  if (paged_) return paged_->capture_prefix_handle(token_count);
  return std::nullopt;
}

void KvCache::copy_prefix_from(const KvCache& source, size_t token_count) {
  // kv_cache.rs:532-564
  const KvCacheConfig& d = config();
  const KvCacheConfig& s = source.config();
  if (d.num_layers != s.num_layers || d.num_kv_heads != s.num_kv_heads || d.head_dim != s.head_dim ||
      d.max_sequence_length != s.max_sequence_length) {
    fail(ErrorKind::InvalidConfig, "KV cache prefix copy requires matching cache configurations");
  }
  if (token_count > source.used_tokens_) {
    fail(ErrorKind::InvalidShape, "KV cache prefix length exceeds source committed tokens");
  }
  reset();
  if (token_count == 0) return;
  if (paged_ && source.paged_) {
    PrefixHandle h = source.paged_->capture_prefix_handle(token_count);
    paged_->import_prefix_from(*source.paged_, h);
  } else {
    std::vector<float> k, v;
    for (size_t l = 0; l < d.num_layers; ++l) {
      source.read_prefix(l, token_count, &k, &v);
      if (paged_) {
        paged_->write_sequence(l, 0, token_count, k.data(), v.data());
      } else {
        contiguous_->write_sequence(l, 0, token_count, k.data(), v.data());
      }
    }
  }
  advance(token_count);
}

// ===========================================================================
// Model (model/config.rs, model/decoder.rs)
// ===========================================================================
void Model::validate() const {
  const ModelConfig& c = config;
  if (c.hidden_size == 0 || c.intermediate_size == 0 || c.num_layers == 0 ||
      c.num_attention_heads == 0 || c.num_key_value_heads == 0 || c.vocab_size == 0 ||
      c.max_position_embeddings == 0) {
    fail(ErrorKind::InvalidConfig, "model dimensions must be greater than zero");
  }
  if (c.hidden_size % c.num_attention_heads != 0) fail(ErrorKind::InvalidConfig, "hidden_size must be divisible by num_attention_heads");
  if (c.num_attention_heads % c.num_key_value_heads != 0) fail(ErrorKind::InvalidConfig, "num_attention_heads must be divisible by num_key_value_heads");
  if (c.rotary_dims > c.head_dim()) fail(ErrorKind::InvalidConfig, "rope.rotary_dims cannot exceed attention head dimension");
}

void Model::set_weight(const std::string& name, const float* data, size_t count) {
  const ModelConfig& c = config;
  size_t h = c.hidden_size, f = c.intermediate_size, kvh = c.num_key_value_heads * c.head_dim();
  auto assign = [&](std::vector<float>* dst, size_t expected) {
    if (count != expected) {
      fail(ErrorKind::InvalidShape, "tensor " + name + " has " + std::to_string(count) +
                                        " elements, expected " + std::to_string(expected));
    }
    dst->assign(data, data + count);
  };
  if (layers.size() != c.num_layers) layers.resize(c.num_layers);
  if (name == "tok_embeddings.weight") return assign(&tok_embeddings, c.vocab_size * h);
  if (name == "norm.weight") return assign(&norm, h);
  if (name == "output.weight") return assign(&output, c.vocab_size * h);
  const std::string prefix = "layers.";
  if (name.compare(0, prefix.size(), prefix) == 0) {
    size_t dot = name.find('.', prefix.size());
    size_t layer = std::stoul(name.substr(prefix.size(), dot - prefix.size()));
    if (layer >= c.num_layers) fail(ErrorKind::InvalidShape, "layer index out of range in " + name);
    std::string rest = name.substr(dot + 1);
    LayerWeights& w = layers[layer];
    if (rest == "attention_norm.weight") return assign(&w.attention_norm, h);
    if (rest == "attention.wq.weight") return assign(&w.wq, h * h);
    if (rest == "attention.wq.bias") return assign(&w.wq_bias, h);
    if (rest == "attention.wk.weight") return assign(&w.wk, h * kvh);
    if (rest == "attention.wk.bias") return assign(&w.wk_bias, kvh);
    if (rest == "attention.wv.weight") return assign(&w.wv, h * kvh);
    if (rest == "attention.wv.bias") return assign(&w.wv_bias, kvh);
    if (rest == "attention.wo.weight") return assign(&w.wo, h * h);
    if (rest == "attention.wo.bias") return assign(&w.wo_bias, h);
    if (rest == "ffn_norm.weight") return assign(&w.ffn_norm, h);
    if (rest == "feed_forward.w1.weight") return assign(&w.w1, h * f);
    if (rest == "feed_forward.w1.bias") return assign(&w.w1_bias, f);
    if (rest == "feed_forward.w2.weight") return assign(&w.w2, f * h);
    if (rest == "feed_forward.w2.bias") return assign(&w.w2_bias, h);
    if (rest == "feed_forward.w3.weight") return assign(&w.w3, h * f);
    if (rest == "feed_forward.w3.bias") return assign(&w.w3_bias, f);
  }
  fail(ErrorKind::MissingWeight, "unknown tensor name: " + name);
}

static const float* opt(const std::vector<float>& v) { return v.empty() ? nullptr : v.data(); }

static void require(const std::vector<float>& v, const std::string& name) {
  if (v.empty()) fail(ErrorKind::MissingWeight, "missing required tensor: " + name);
}

static void require_layer(const Model& m, size_t l) {
  const LayerWeights& w = m.layers.at(l);
  std::string p = "layers." + std::to_string(l) + ".";
  require(w.attention_norm, p + "attention_norm.weight");
  require(w.wq, p + "attention.wq.weight");
  require(w.wk, p + "attention.wk.weight");
  require(w.wv, p + "attention.wv.weight");
  require(w.wo, p + "attention.wo.weight");
  require(w.ffn_norm, p + "ffn_norm.weight");
  require(w.w1, p + "feed_forward.w1.weight");
  require(w.w2, p + "feed_forward.w2.weight");
  require(w.w3, p + "feed_forward.w3.weight");
}

// reference.rs:163-370 decoder_block_forward_buffered_f32, and its decode twin
// reference.rs:712-871 (same op order; attention choice made by `attend`).
template <typename Attend>
static void block_forward(const Model& m, size_t layer, const std::vector<float>& input,
                          size_t seq_len, size_t position_offset, std::vector<float>* output,
                          Attend&& attend) {
  const ModelConfig& c = m.config;
  const LayerWeights& w = m.layers[layer];
  size_t h = c.hidden_size, hq = c.num_attention_heads, hkv = c.num_key_value_heads;
  size_t d = c.head_dim(), kvw = hkv * d, f = c.intermediate_size;
  if (hq % hkv != 0) fail(ErrorKind::InvalidConfig, "decoder block requires num_heads to be divisible by num_kv_heads");
  std::vector<float> normed(seq_len * h), query(seq_len * h), key(seq_len * kvw), value(seq_len * kvw);
  std::vector<float> attention(seq_len * h), gated(seq_len * f), gate(seq_len * f);
  rms_norm_f32(input.data(), w.attention_norm.data(), seq_len, h, c.rms_norm_eps, normed.data());
  linear_f32_with_bias(normed.data(), w.wq.data(), opt(w.wq_bias), seq_len, h, h, query.data());
  linear_f32_with_bias(normed.data(), w.wk.data(), opt(w.wk_bias), seq_len, h, kvw, key.data());
  linear_f32_with_bias(normed.data(), w.wv.data(), opt(w.wv_bias), seq_len, h, kvw, value.data());
  rope_f32(query.data(), key.data(), seq_len, hq, hkv, d, position_offset, c.rotary_dims, c.rope_theta);
  attend(query, key, value, &attention);
  linear_f32_with_bias(attention.data(), w.wo.data(), opt(w.wo_bias), seq_len, h, h, normed.data());
  add_f32_in_place(normed.data(), input.data(), seq_len * h);
  rms_norm_f32(normed.data(), w.ffn_norm.data(), seq_len, h, c.rms_norm_eps, attention.data());
  linear_f32_with_bias(attention.data(), w.w1.data(), opt(w.w1_bias), seq_len, h, f, gated.data());
  linear_f32_with_bias(attention.data(), w.w3.data(), opt(w.w3_bias), seq_len, h, f, gate.data());
  silu_f32_in_place(gate.data(), seq_len * f);
  mul_f32_in_place(gated.data(), gate.data(), seq_len * f);
  output->assign(seq_len * h, 0.0f);
  linear_f32_with_bias(gated.data(), w.w2.data(), opt(w.w2_bias), seq_len, f, h, output->data());
  add_f32_in_place(output->data(), normed.data(), seq_len * h);
}

static std::vector<float> final_norm(const Model& m, const std::vector<float>& hidden, size_t rows) {
  require(m.norm, "norm.weight");
  std::vector<float> out(rows * m.config.hidden_size);
  rms_norm_f32(hidden.data(), m.norm.data(), rows, m.config.hidden_size, m.config.rms_norm_eps, out.data());
  return out;
}

static std::vector<float> embed(const Model& m, const std::vector<uint32_t>& ids) {
  require(m.tok_embeddings, "tok_embeddings.weight");
  std::vector<float> hidden(ids.size() * m.config.hidden_size);
  embedding_gather_f32(m.tok_embeddings.data(), m.config.vocab_size, m.config.hidden_size, ids.data(),
                       ids.size(), hidden.data());
  return hidden;
}

std::vector<float> decoder_model_forward(const Model& m, const std::vector<uint32_t>& ids) {
  // reference.rs:517-524, 624-662
  if (ids.empty()) fail(ErrorKind::InvalidShape, "decoder_model_hidden_f32 requires at least one token");
  const ModelConfig& c = m.config;
  std::vector<float> hidden = embed(m, ids), next;
  size_t t = ids.size();
  for (size_t l = 0; l < c.num_layers; ++l) {
    require_layer(m, l);
    block_forward(m, l, hidden, t, 0, &next,
                  [&](const std::vector<float>& q, const std::vector<float>& k,
                      const std::vector<float>& v, std::vector<float>* out) {
                    prefixed_causal_attention_f32(q.data(), k.data(), v.data(), t, 0, c.num_attention_heads,
                                                  c.num_key_value_heads, c.head_dim(), out->data());
                  });
    hidden.swap(next);
  }
  std::vector<float> normed = final_norm(m, hidden, t);
  const std::vector<float>& ow = m.output_weight();
  require(ow, "output.weight");
  std::vector<float> logits(t * c.vocab_size);
  matmul_rhs_transposed_f32(normed.data(), ow.data(), t, c.hidden_size, c.vocab_size, logits.data());
  return logits;
}

std::vector<float> prefill_hidden_with_kv_capture(const Model& m, const std::vector<uint32_t>& ids,
                                                  KvCache* kv) {
  // reference.rs:372-465
  if (ids.empty()) fail(ErrorKind::InvalidShape, "prefill reference path requires at least one token");
  if (ids.size() > kv->remaining_tokens()) fail(ErrorKind::Runtime, "batch prefill exceeds KV cache capacity");
  const ModelConfig& c = m.config;
  size_t t = ids.size(), start = kv->used_tokens();
  size_t hq = c.num_attention_heads, hkv = c.num_key_value_heads, d = c.head_dim();
  std::vector<float> hidden = embed(m, ids), next;
  for (size_t l = 0; l < c.num_layers; ++l) {
    require_layer(m, l);
    block_forward(m, l, hidden, t, start, &next,
                  [&](const std::vector<float>& q, const std::vector<float>& k,
                      const std::vector<float>& v, std::vector<float>* out) {
                    if (start == 0) {
                      prefixed_causal_attention_f32(q.data(), k.data(), v.data(), t, 0, hq, hkv, d, out->data());
                    } else if (!kv->is_paged()) {
                      const ContiguousKvCacheStorage* s = kv->contiguous_storage();
                      cached_prefixed_causal_attention_f32(q.data(), s->layer_key(l), s->layer_value(l), start,
                                                           k.data(), v.data(), t, hq, hkv, d, out->data());
                    } else {
                      std::vector<float> ck, cv;
                      kv->read_prefix(l, start, &ck, &cv);
                      cached_prefixed_causal_attention_f32(q.data(), ck.data(), cv.data(), start, k.data(),
                                                           v.data(), t, hq, hkv, d, out->data());
                    }
                    kv->write_sequence_uncommitted(l, start, t, k.data(), v.data());
                  });
    hidden.swap(next);
  }
  return final_norm(m, hidden, t);
}

std::vector<float> token_hidden_with_kv_cache(const Model& m, uint32_t token, KvCache* kv,
                                              size_t position) {
  // reference.rs:664-871 + decode_causal_attention_with_kv_cache_f32 (467-515)
  const ModelConfig& c = m.config;
  size_t hq = c.num_attention_heads, hkv = c.num_key_value_heads, d = c.head_dim();
  std::vector<float> hidden = embed(m, {token}), next;
  for (size_t l = 0; l < c.num_layers; ++l) {
    require_layer(m, l);
    block_forward(m, l, hidden, 1, position, &next,
                  [&](const std::vector<float>& q, const std::vector<float>& k,
                      const std::vector<float>& v, std::vector<float>* out) {
                    if (position == 0) {
                      prefixed_causal_attention_f32(q.data(), k.data(), v.data(), 1, 0, hq, hkv, d, out->data());
                    } else if (!kv->is_paged()) {
                      const ContiguousKvCacheStorage* s = kv->contiguous_storage();
                      decode_causal_attention_f32(q.data(), s->layer_key(l), s->layer_value(l), position,
                                                  k.data(), v.data(), hq, hkv, d, out->data());
                    } else {
                      std::vector<float> ck, cv;
                      kv->read_prefix(l, position, &ck, &cv);
                      cached_prefixed_causal_attention_f32(q.data(), ck.data(), cv.data(), position, k.data(),
                                                           v.data(), 1, hq, hkv, d, out->data());
                    }
                    kv->write_uncommitted(l, position, k.data(), v.data());
                  });
    hidden.swap(next);
  }
  return final_norm(m, hidden, 1);
}

TokenSample sample_from_hidden_row(const Model& m, const float* hidden_row) {
  const std::vector<float>& ow = m.output_weight();
  require(ow, "output.weight");
  TokenSample s{};
  matmul_rhs_transposed_argmax_f32(hidden_row, ow.data(), m.config.hidden_size, m.config.vocab_size,
                                   &s.token_id, &s.probability);
  return s;
}

std::vector<float> logits_from_hidden_row(const Model& m, const float* hidden_row) {
  const std::vector<float>& ow = m.output_weight();
  require(ow, "output.weight");
  std::vector<float> logits(m.config.vocab_size);
  matmul_rhs_transposed_f32(hidden_row, ow.data(), 1, m.config.hidden_size, m.config.vocab_size, logits.data());
  return logits;
}

// ===========================================================================
// Session (session.rs:92-413), greedy sampler
// ===========================================================================
static KvCache make_session_kv(const Model& m, const SessionConfig& sc) {
  KvCacheConfig kc;
  kc.num_layers = m.config.num_layers;
  kc.num_kv_heads = m.config.num_key_value_heads;
  kc.head_dim = m.config.head_dim();
  kc.max_sequence_length = sc.max_sequence_length;
  return sc.page_size == 0 ? KvCache::contiguous(kc) : KvCache::paged(kc, sc.page_size);
}

bool SamplerConfig::is_greedy() const { return sampler_is_greedy(temperature, top_k, top_p); }

bool SamplerConfig::operator==(const SamplerConfig& o) const {
  return temperature == o.temperature && top_k == o.top_k && top_p == o.top_p &&
         repetition_penalty == o.repetition_penalty && seed == o.seed;
}

// session.rs:104-139: the sampler state starts from the configuration's seed
Session::Session(std::shared_ptr<const Model> model, const SessionConfig& config)
    : model_(std::move(model)), config_(config), kv_(make_session_kv(*model_, config)),
      sampler_state_(sampler_state_new(config.sampler.seed)) {}

void Session::set_sampler(const SamplerConfig& sampler) {
  config_.sampler = sampler;
  sampler_state_ = sampler_state_new(sampler.seed);
}

// session.rs:349-373, 393-406: a greedy configuration takes the fused argmax head
// (matmul_rhs_transposed_argmax); otherwise the last row's logits go through
// sample_last_token with the session's sampler state.
TokenSample Session::sample_hidden_row(const float* hidden_row) {
  if (config_.sampler.is_greedy()) return sample_from_hidden_row(*model_, hidden_row);
  const std::vector<float> logits = logits_from_hidden_row(*model_, hidden_row);
  const SamplerConfig& c = config_.sampler;
  TokenSample t{};
  sample_last_token(logits.data(), 1, logits.size(), c.temperature, c.top_k, c.top_p, &sampler_state_, &t.token_id,
                    &t.probability);
  return t;
}

std::optional<PrefixHandle> Session::prefix_handle(size_t token_count) const {
  if (token_count > position_) {
    fail(ErrorKind::InvalidShape, "session prefix handle length " + std::to_string(token_count) +
                                      " exceeds committed tokens " + std::to_string(position_));
  }
  return kv_.prefix_handle(token_count);
}

void Session::copy_prefix_from_session(const Session& source, size_t token_count) {
  if (token_count > source.history_.size()) {
    fail(ErrorKind::InvalidShape, "session prefix length exceeds source token history");
  }
  reset();
  kv_.copy_prefix_from(source.kv_, token_count);
  position_ = token_count;
  history_.assign(source.history_.begin(), source.history_.begin() + token_count);
  if (token_count == source.position_ && model_ == source.model_ && config_.sampler == source.config_.sampler) {
    last_sample_ = source.last_sample_;
    last_hidden_ = source.last_hidden_;
    sampler_state_ = source.sampler_state_;  // session.rs:195-201
  }
}

void Session::reset() {
  kv_.reset();
  position_ = 0;
  history_.clear();
  last_sample_.reset();
  last_hidden_.clear();
  sampler_state_ = sampler_state_new(config_.sampler.seed);  // session.rs:206-212
}

void Session::prefill_tokens(const std::vector<uint32_t>& ids) {
  if (ids.empty()) fail(ErrorKind::InvalidShape, "prefill_tokens requires at least one token");
  if (position_ != kv_.used_tokens()) fail(ErrorKind::Runtime, "session position and KV cache usage diverged");
  if (ids.size() > 1) {
    process_prefill(ids);
    return;
  }
  process_token(ids[0]);
}

TokenSample Session::step_reference() {
  if (history_.empty()) fail(ErrorKind::Runtime, "step_reference requires at least one prefetched token");
  if (!last_sample_) fail(ErrorKind::Runtime, "step_reference requires a sampled token from a prefetched token");
  TokenSample s = *last_sample_;
  process_token(s.token_id);
  return s;
}

std::vector<TokenSample> Session::generate_from_tokens(const std::vector<uint32_t>& prompt, size_t max_new_tokens,
                                                       std::optional<uint32_t> stop_token, FinishReason* finish) {
  reset();
  prefill_tokens(prompt);
  const size_t budget = std::min(max_new_tokens, config_.max_generated_tokens);
  FinishReason reason = budget < max_new_tokens ? FinishReason::SessionLimit : FinishReason::MaxNewTokens;
  std::vector<TokenSample> out;
  for (size_t i = 0; i < budget; ++i) {
    if (position_ >= config_.max_sequence_length) {
      reason = FinishReason::SequenceLength;
      break;
    }
    TokenSample s = step_reference();
    out.push_back(s);
    if (stop_token && *stop_token == s.token_id) {
      reason = FinishReason::StopToken;
      break;
    }
  }
  *finish = reason;
  return out;
}

void Session::process_token(uint32_t token) {
  if (position_ >= config_.max_sequence_length) fail(ErrorKind::Runtime, "cannot process tokens beyond max sequence length");
  if (position_ != kv_.used_tokens()) fail(ErrorKind::Runtime, "session position and KV cache usage diverged");
  std::vector<float> hidden = token_hidden_with_kv_cache(*model_, token, &kv_, position_);
  TokenSample s = sample_hidden_row(hidden.data());
  kv_.advance(1);
  position_ += 1;
  history_.push_back(token);
  last_sample_ = s;
  last_hidden_ = hidden;
}

void Session::process_prefill(const std::vector<uint32_t>& ids) {
  if (position_ + ids.size() > config_.max_sequence_length) {
    fail(ErrorKind::Runtime, "cannot process tokens beyond max sequence length");
  }
  std::vector<float> hidden = prefill_hidden_with_kv_capture(*model_, ids, &kv_);
  size_t h = model_->config.hidden_size;
  const float* last = hidden.data() + (ids.size() - 1) * h;
  TokenSample s = sample_hidden_row(last);
  kv_.advance(ids.size());
  position_ += ids.size();
  history_.insert(history_.end(), ids.begin(), ids.end());
  last_sample_ = s;
  last_hidden_.assign(last, last + h);
}

// ===========================================================================
// SequenceState (sequence.rs:181-203)
// ===========================================================================
void SequenceState::record_prefill(size_t appended) {
  cached_tokens += appended;
  if (phase != SequencePhase::Finished) {
    phase = pending_prompt_tokens() == 0 ? SequencePhase::Decode : SequencePhase::Prefill;
  }
}

void SequenceState::record_generated_token(uint32_t token) {
  generated.push_back(token);
  cached_tokens += 1;
  if (phase != SequencePhase::Finished) phase = SequencePhase::Decode;
}

// ===========================================================================
// PrefixIndex (prefix_index.rs:24-113)
// ===========================================================================
void PrefixIndex::upsert(const PrefixIndexEntry& e) {
  if (min_share_ == 0 || e.prompt_tokens.size() < min_share_ || e.cached_prompt_tokens < min_share_) return;
  std::vector<uint32_t> key(e.prompt_tokens.begin(), e.prompt_tokens.begin() + min_share_);
  buckets_[key].push_back(e);
}

std::optional<std::pair<uint64_t, size_t>> PrefixIndex::best_match(
    uint64_t target, const std::vector<uint32_t>& prompt) const {
  if (min_share_ == 0 || prompt.size() < min_share_) return std::nullopt;
  std::vector<uint32_t> key(prompt.begin(), prompt.begin() + min_share_);
  auto it = buckets_.find(key);
  if (it == buckets_.end()) return std::nullopt;
  std::optional<std::pair<uint64_t, size_t>> best;
  for (const auto& cand : it->second) {
    if (cand.sequence_id == target) continue;
    size_t common = 0;
    while (common < prompt.size() && common < cand.prompt_tokens.size() &&
           prompt[common] == cand.prompt_tokens[common]) {
      ++common;
    }
    size_t shared = std::min(common, cand.cached_prompt_tokens);
    // normalize_shared_prefix_len (prefix_index.rs:98-109)
    if (shared == prompt.size() && cand.session_position > shared) shared = shared == 0 ? 0 : shared - 1;
    if (shared < min_share_) continue;
    // Iterator::max_by_key returns the last maximum.
    if (!best || shared >= best->second) best = std::make_pair(cand.sequence_id, shared);
  }
  return best;
}

// ===========================================================================
// PrefixBlockManager (block_manager.rs:58-172)
// ===========================================================================
std::vector<ManagedBlockId> PrefixBlockManager::apply(uint64_t owner, const PrefixHandle& h,
                                                      bool increment) {
  std::vector<ManagedBlockId> released;
  for (size_t l = 0; l < h.layer_block_tables.size(); ++l) {
    for (const auto& e : h.layer_block_tables[l]) {
      ManagedBlockId id{owner, l, e.block_id};
      if (increment) {
        ref_counts_[id] += 1;
      } else {
        auto it = ref_counts_.find(id);
        if (it != ref_counts_.end()) {
          if (it->second > 0) it->second -= 1;
          if (it->second == 0) {
            ref_counts_.erase(it);
            released.push_back(id);
          }
        }
      }
    }
  }
  return released;
}

std::vector<ManagedBlockId> PrefixBlockManager::update_owned_prefix(uint64_t seq,
                                                                    std::optional<PrefixHandle> h) {
  std::vector<ManagedBlockId> released;
  auto it = owned_.find(seq);
  if (it != owned_.end()) {
    PrefixHandle prev = std::move(it->second);
    owned_.erase(it);
    auto r = apply(seq, prev, false);
    released.insert(released.end(), r.begin(), r.end());
  }
  if (h) {
    apply(seq, *h, true);
    owned_[seq] = std::move(*h);
  }
  return released;
}

std::vector<ManagedBlockId> PrefixBlockManager::update_shared_prefix(
    uint64_t seq, std::optional<SharedPrefixAssignment> a) {
  std::vector<ManagedBlockId> released;
  auto it = shared_.find(seq);
  if (it != shared_.end()) {
    SharedPrefixAssignment prev = std::move(it->second);
    shared_.erase(it);
    auto r = apply(prev.source_sequence_id, prev.handle, false);
    released.insert(released.end(), r.begin(), r.end());
  }
  if (a) {
    apply(a->source_sequence_id, a->handle, true);
    shared_[seq] = std::move(*a);
  }
  return released;
}

std::vector<ManagedBlockId> PrefixBlockManager::remove_sequence(uint64_t seq) {
  auto released = update_shared_prefix(seq, std::nullopt);
  auto r = update_owned_prefix(seq, std::nullopt);
  released.insert(released.end(), r.begin(), r.end());
  return released;
}

size_t PrefixBlockManager::block_ref_count(const ManagedBlockId& id) const {
  auto it = ref_counts_.find(id);
  return it == ref_counts_.end() ? 0 : it->second;
}

const PrefixHandle* PrefixBlockManager::owned_prefix(uint64_t seq) const {
  auto it = owned_.find(seq);
  return it == owned_.end() ? nullptr : &it->second;
}

const SharedPrefixAssignment* PrefixBlockManager::shared_prefix(uint64_t seq) const {
  auto it = shared_.find(seq);
  return it == shared_.end() ? nullptr : &it->second;
}

// ===========================================================================
// ReferenceScheduler (scheduler.rs:109-648)
// ===========================================================================
ReferenceScheduler::ReferenceScheduler(std::shared_ptr<const Model> model,
                                       const SessionConfig& session_config,
                                       const SchedulerConfig& config)
    : model_(std::move(model)), session_config_(session_config), config_(config),
      prefix_index_(config.min_prefix_share_tokens) {
  if (config.max_batch_size == 0) fail(ErrorKind::InvalidConfig, "scheduler max_batch_size must be greater than zero");
  if (config.max_prefill_chunk_tokens == 0) fail(ErrorKind::InvalidConfig, "scheduler max_prefill_chunk_tokens must be greater than zero");
  if (config.max_prefill_batch_tokens == 0) fail(ErrorKind::InvalidConfig, "scheduler max_prefill_batch_tokens must be greater than zero");
  if (config.max_consecutive_prefill_ticks == 0) fail(ErrorKind::InvalidConfig, "scheduler max_consecutive_prefill_ticks must be greater than zero");
}

size_t ReferenceScheduler::index_of(uint64_t seq) const {
  for (size_t i = 0; i < sequences_.size(); ++i) {
    if (sequences_[i].state.sequence_id == seq) return i;
  }
  fail(ErrorKind::Runtime, "scheduler sequence " + std::to_string(seq) + " is missing");
}

const SequenceState* ReferenceScheduler::sequence_state(uint64_t seq) const {
  for (const auto& e : sequences_) {
    if (e.state.sequence_id == seq) return &e.state;
  }
  return nullptr;
}

const Session* ReferenceScheduler::session(uint64_t seq) const {
  for (const auto& e : sequences_) {
    if (e.state.sequence_id == seq) return e.session.get();
  }
  return nullptr;
}

size_t ReferenceScheduler::resident_session_count() const {
  size_t n = 0;
  for (const auto& e : sequences_) n += e.session ? 1 : 0;
  return n;
}

bool ReferenceScheduler::has_pending() const {
  for (const auto& e : sequences_) {
    if (e.state.phase != SequencePhase::Finished) return true;
  }
  return false;
}

uint64_t ReferenceScheduler::submit(const std::vector<uint32_t>& prompt, size_t max_new_tokens,
                                    std::optional<uint32_t> stop_token) {
  if (prompt.empty()) fail(ErrorKind::InvalidShape, "scheduler requests require at least one prompt token");
  if (prompt.size() > session_config_.max_sequence_length) {
    fail(ErrorKind::InvalidShape, "scheduler request prompt exceeds session max sequence length");
  }
  Entry e;
  e.state.request_id = next_request_id_++;
  e.state.sequence_id = next_sequence_id_++;
  e.state.prompt = prompt;
  e.state.requested_max_new_tokens = max_new_tokens;
  e.state.max_new_tokens = std::min(max_new_tokens, session_config_.max_generated_tokens);
  e.state.stop_token = stop_token;
  e.session = std::make_unique<Session>(model_, session_config_);
  uint64_t seq = e.state.sequence_id;
  sequences_.push_back(std::move(e));
  block_manager_.update_shared_prefix(seq, std::nullopt);
  refresh_sequence_prefix_metadata(seq);
  rebuild_prefix_index();
  return seq;
}

std::vector<uint64_t> ReferenceScheduler::collect_prefill_ids() const {
  std::vector<uint64_t> ids;
  size_t total = 0;
  for (const auto& e : sequences_) {
    if (e.state.phase != SequencePhase::Prefill) continue;
    size_t chunk = e.state.next_prefill_chunk_len(config_.max_prefill_chunk_tokens);
    if (chunk == 0) continue;
    if (!ids.empty() && total + chunk > config_.max_prefill_batch_tokens) break;
    total += chunk;
    ids.push_back(e.state.sequence_id);
    if (ids.size() >= config_.max_batch_size || total >= config_.max_prefill_batch_tokens) break;
  }
  return ids;
}

std::vector<uint64_t> ReferenceScheduler::collect_decode_ids() const {
  std::vector<uint64_t> ids;
  for (const auto& e : sequences_) {
    if (e.state.phase != SequencePhase::Decode) continue;
    if (ids.size() >= config_.max_batch_size) break;
    ids.push_back(e.state.sequence_id);
  }
  return ids;
}

bool ReferenceScheduler::should_schedule_decode(size_t prefill, size_t decode) const {
  if (decode == 0) return false;
  if (prefill == 0) return true;
  if (consecutive_prefill_ticks_ >= config_.max_consecutive_prefill_ticks) return true;
  return consecutive_prefill_ticks_ > 0 && decode == config_.max_batch_size && prefill < config_.max_batch_size;
}

std::optional<SchedulerTick> ReferenceScheduler::plan_next_tick() const {
  auto prefill = collect_prefill_ids();
  auto decode = collect_decode_ids();
  if (prefill.empty()) {
    if (decode.empty()) return std::nullopt;
    return SchedulerTick{BatchKind::Decode, decode};
  }
  if (decode.empty()) return SchedulerTick{BatchKind::Prefill, prefill};
  if (should_schedule_decode(prefill.size(), decode.size())) return SchedulerTick{BatchKind::Decode, decode};
  return SchedulerTick{BatchKind::Prefill, prefill};
}

void ReferenceScheduler::rebuild_prefix_index() {
  prefix_index_.clear();
  for (const auto& e : sequences_) {
    if (e.state.phase == SequencePhase::Finished) continue;
    prefix_index_.upsert({e.state.sequence_id, e.state.prompt, e.state.cached_prompt_tokens(), e.state.cached_tokens});
  }
}

void ReferenceScheduler::refresh_sequence_prefix_metadata(uint64_t seq) {
  const Entry& e = sequences_[index_of(seq)];
  std::optional<PrefixHandle> h;
  if (e.state.phase != SequencePhase::Finished) {
    if (!e.session) fail(ErrorKind::Runtime, "scheduler sequence no longer retains an active session");
    h = e.session->prefix_handle(e.state.cached_prompt_tokens());
  }
  block_manager_.update_owned_prefix(seq, std::move(h));
}

size_t ReferenceScheduler::maybe_share_prefix(uint64_t seq, int64_t* source_out) {
  rebuild_prefix_index();
  if (config_.min_prefix_share_tokens == 0) return 0;
  size_t ti = index_of(seq);
  const Entry& target = sequences_[ti];
  if (target.state.cached_prompt_tokens() != 0 || target.state.phase != SequencePhase::Prefill) return 0;
  auto cand = prefix_index_.best_match(seq, target.state.prompt);
  if (!cand) return 0;
  size_t si = index_of(cand->first);
  size_t shared = cand->second;
  if (shared == 0) return 0;
  *source_out = static_cast<int64_t>(cand->first);
  Entry& source = sequences_[si];
  if (!source.session) fail(ErrorKind::Runtime, "scheduler sequence no longer retains an active session");
  std::optional<SharedPrefixAssignment> assignment;
  if (auto h = source.session->prefix_handle(shared)) {
    assignment = SharedPrefixAssignment{source.state.sequence_id, std::move(*h)};
  }
  Entry& tgt = sequences_[ti];
  tgt.session->copy_prefix_from_session(*source.session, shared);
  tgt.state.record_prefill(shared);
  block_manager_.update_shared_prefix(seq, std::move(assignment));
  refresh_sequence_prefix_metadata(seq);
  rebuild_prefix_index();
  return shared;
}

std::vector<ManagedBlockId> ReferenceScheduler::release_sequence_resources(uint64_t seq) {
  sequences_[index_of(seq)].session.reset();
  return block_manager_.remove_sequence(seq);
}

SequenceExecutionUpdate ReferenceScheduler::execute_prefill(uint64_t seq) {
  size_t max_chunk = config_.max_prefill_chunk_tokens;
  int64_t source = -1;
  size_t reused = maybe_share_prefix(seq, &source);
  Entry& e = sequences_[index_of(seq)];
  size_t appended = e.state.next_prefill_chunk_len(max_chunk);
  if (appended > 0) {
    size_t start = e.state.cached_prompt_tokens();
    std::vector<uint32_t> chunk(e.state.prompt.begin() + start, e.state.prompt.begin() + start + appended);
    e.session->prefill_tokens(chunk);
    e.state.record_prefill(appended);
  }
  FinishReason reason = FinishReason::None;
  if (e.state.generation_budget_reached()) {
    reason = e.state.generation_budget_finish_reason();
  } else if (e.session->position() >= e.session->config().max_sequence_length) {
    reason = FinishReason::SequenceLength;
  }
  if (reason != FinishReason::None) e.state.finish(reason);
  SequenceExecutionUpdate u{};
  u.request_id = e.state.request_id;
  u.sequence_id = seq;
  u.batch_kind = BatchKind::Prefill;
  u.reused_prompt_tokens = reused;
  u.appended_prompt_tokens = appended;
  u.shared_from = reused > 0 ? source : -1;
  u.has_token = false;
  u.phase = e.state.phase;
  u.finish_reason = reason;
  if (reason != FinishReason::None) u.released_prefix_blocks = release_sequence_resources(seq);
  return u;
}

SequenceExecutionUpdate ReferenceScheduler::execute_decode(uint64_t seq) {
  Entry& e = sequences_[index_of(seq)];
  SequenceExecutionUpdate u{};
  u.request_id = e.state.request_id;
  u.sequence_id = seq;
  u.batch_kind = BatchKind::Decode;
  u.shared_from = -1;
  FinishReason reason = FinishReason::None;
  if (e.session->position() >= e.session->config().max_sequence_length) {
    reason = FinishReason::SequenceLength;
    e.state.finish(reason);
    u.has_token = false;
  } else {
    TokenSample s = e.session->step_reference();
    e.state.record_generated_token(s.token_id);
    if (e.state.stop_token && *e.state.stop_token == s.token_id) {
      reason = FinishReason::StopToken;
    } else if (e.state.generation_budget_reached()) {
      reason = e.state.generation_budget_finish_reason();
    } else if (e.session->position() >= e.session->config().max_sequence_length) {
      reason = FinishReason::SequenceLength;
    }
    if (reason != FinishReason::None) e.state.finish(reason);
    u.has_token = true;
    u.generated = s;
  }
  u.phase = e.state.phase;
  u.finish_reason = reason;
  if (reason != FinishReason::None) u.released_prefix_blocks = release_sequence_resources(seq);
  return u;
}

std::optional<SchedulerReport> ReferenceScheduler::execute_next_tick() {
  auto tick = plan_next_tick();
  if (!tick) return std::nullopt;
  SchedulerReport report;
  report.tick = *tick;
  for (uint64_t seq : tick->sequence_ids) {
    SequenceExecutionUpdate u =
        tick->kind == BatchKind::Prefill ? execute_prefill(seq) : execute_decode(seq);
    refresh_sequence_prefix_metadata(seq);
    rebuild_prefix_index();
    report.updates.push_back(std::move(u));
  }
  consecutive_prefill_ticks_ = tick->kind == BatchKind::Prefill ? consecutive_prefill_ticks_ + 1 : 0;
  return report;
}

// ===========================================================================
// GlobalPagePacker
// ===========================================================================
GlobalPagePacker::GlobalPagePacker(size_t num_pages, size_t page_size) : page_size_(page_size) {
  if (num_pages == 0 || page_size == 0) fail(ErrorKind::InvalidConfig, "page pool dimensions must be greater than zero");
  for (size_t p = num_pages; p-- > 0;) free_.push_back(static_cast<int32_t>(p));
  refs_.assign(num_pages, 0);
}

int32_t GlobalPagePacker::allocate() {
  if (free_.empty()) fail(ErrorKind::Runtime, "page pool ran out of free pages");
  int32_t p = free_.back();
  free_.pop_back();
  refs_[p] = 1;
  return p;
}

void GlobalPagePacker::decref(int32_t page) {
  if (--refs_.at(page) == 0) free_.push_back(page);
}

PackedTick GlobalPagePacker::pack(const SchedulerReport& report) {
  PackedTick t;
  t.kind = static_cast<int32_t>(report.tick.kind);
  t.cu_seqlens.push_back(0);
  std::vector<uint64_t> finished;
  for (const auto& u : report.updates) {
    Seq& s = seqs_[u.sequence_id];
    size_t n = 0;
    if (u.batch_kind == BatchKind::Prefill) {
      if (u.reused_prompt_tokens > 0) {
        // the target's pages become the source's: full pages by id, the partial one copied
        Seq& src = seqs_.at(static_cast<uint64_t>(u.shared_from));
        for (int32_t p : s.pages) decref(p);
        s.pages.clear();
        size_t full = u.reused_prompt_tokens / page_size_;
        for (size_t i = 0; i < full; ++i) {
          refs_.at(src.pages[i]) += 1;
          s.pages.push_back(src.pages[i]);
        }
        size_t rem = u.reused_prompt_tokens % page_size_;
        if (rem) {
          int32_t p = allocate();
          s.pages.push_back(p);
          t.copy_src.push_back(src.pages[full]);
          t.copy_dst.push_back(p);
          t.copy_count.push_back(static_cast<int32_t>(rem));
        }
        s.position = u.reused_prompt_tokens;
      }
      n = u.appended_prompt_tokens;
    } else {
      n = u.has_token ? 1 : 0;
    }
    if (n > 0) {
      size_t end = s.position + n;
      while (s.pages.size() * page_size_ < end) s.pages.push_back(allocate());
      for (size_t p = s.position; p < end; ++p) {
        size_t logical = p / page_size_, offset = p % page_size_;
        t.positions.push_back(static_cast<int32_t>(p));
        t.slot_mapping.push_back(static_cast<int64_t>(s.pages[logical]) * static_cast<int64_t>(page_size_) +
                                 static_cast<int64_t>(offset));
      }
      t.sequence_ids.push_back(u.sequence_id);
      t.cu_seqlens.push_back(static_cast<int32_t>(t.positions.size()));
      t.context_lens.push_back(static_cast<int32_t>(end));
      t.block_tables.emplace_back(s.pages.begin(), s.pages.begin() + (end + page_size_ - 1) / page_size_);
      s.position = end;
    }
    if (u.finish_reason != FinishReason::None) finished.push_back(u.sequence_id);
  }
  for (uint64_t id : finished) {
    Seq& s = seqs_[id];
    for (int32_t p : s.pages) decref(p);
    s.pages.clear();
  }
  return t;
}

}  // namespace orc
