// Oracle restatement of crates/ferrisinfer-runtime (paged KV, KV cache, reference forward,
// session, sequence state, prefix index, prefix block manager, scheduler) — TEST
// INFRASTRUCTURE ONLY (see oracle.h).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <optional>
#include <string>
#include <vector>

#include "oracle.h"

namespace orc {

// ---- runtime/kv_cache.rs:5-12 ----
struct KvCacheConfig {
  size_t num_layers = 0;
  size_t num_kv_heads = 0;
  size_t head_dim = 0;
  size_t max_sequence_length = 0;
};

// ---- runtime/paged_kv.rs:19-128 ----
struct KvCachePageInfo {
  size_t page_id;
  size_t start_position;
  size_t token_count;
};

struct KvBlockTableEntry {
  size_t logical_block_index;
  size_t block_id;
  size_t start_position;
  size_t token_count;
  bool operator==(const KvBlockTableEntry& o) const {
    return logical_block_index == o.logical_block_index && block_id == o.block_id &&
           start_position == o.start_position && token_count == o.token_count;
  }
};

struct PrefixHandle {
  size_t token_count = 0;
  size_t page_size = 0;
  std::vector<std::vector<KvBlockTableEntry>> layer_block_tables;
};

// ---- runtime/paged_kv.rs:130-792 PagedKvCacheStorage ----
class PagedKvCacheStorage {
 public:
  PagedKvCacheStorage(const KvCacheConfig& config, size_t page_size);

  size_t page_size() const { return page_size_; }
  size_t page_count_per_layer() const { return pages_.empty() ? 0 : pages_[0].size(); }
  size_t layer_count() const { return config_.num_layers; }
  const KvCacheConfig& config() const { return config_; }
  size_t allocated_page_count(size_t layer) const;
  size_t free_page_count(size_t layer) const;
  std::vector<KvCachePageInfo> page_infos(size_t layer) const;
  std::vector<KvBlockTableEntry> block_table(size_t layer, size_t token_count) const;
  PrefixHandle capture_prefix_handle(size_t token_count) const;
  void import_prefix_from(const PagedKvCacheStorage& source, const PrefixHandle& handle);
  void reset();
  void write_slot(size_t layer, size_t position, const float* key, const float* value);
  void write_sequence(size_t layer, size_t start, size_t seq_len, const float* key,
                      const float* value);
  // Gather of the committed prefix by block table (paged_kv.rs:769-791).
  void read_prefix(size_t layer, size_t length, std::vector<float>* key,
                   std::vector<float>* value) const;

 private:
  struct Page {
    size_t id;
    std::optional<size_t> assigned_logical_block;
    size_t committed_tokens = 0;
    std::vector<float> key;
    std::vector<float> value;
  };
  size_t slot_width() const { return config_.num_kv_heads * config_.head_dim; }
  size_t allocate_page_for_logical_block(size_t layer, size_t logical_block);
  const Page& page(size_t layer, size_t id) const;
  void check_layer(size_t layer) const;

  KvCacheConfig config_;
  size_t page_size_;
  std::vector<std::vector<float>> view_key_, view_value_;  // layer_views mirror
  std::vector<std::vector<Page>> pages_;
  std::vector<std::vector<std::optional<size_t>>> block_tables_;
  std::vector<std::vector<size_t>> free_ids_;
};

// ---- runtime/kv_cache.rs:66-200 ContiguousKvCacheStorage ----
class ContiguousKvCacheStorage {
 public:
  explicit ContiguousKvCacheStorage(const KvCacheConfig& config);
  void write_slot(size_t layer, size_t position, const float* key, const float* value);
  void write_sequence(size_t layer, size_t start, size_t seq_len, const float* key,
                      const float* value);
  void read_prefix(size_t layer, size_t length, std::vector<float>* key,
                   std::vector<float>* value) const;
  const float* layer_key(size_t layer) const { return key_.at(layer).data(); }
  const float* layer_value(size_t layer) const { return value_.at(layer).data(); }
  void reset() {}
  const KvCacheConfig& config() const { return config_; }

 private:
  KvCacheConfig config_;
  std::vector<std::vector<float>> key_, value_;
};

// ---- runtime/kv_cache.rs:359-597 KvCache ----
class KvCache {
 public:
  static KvCache contiguous(const KvCacheConfig& config);
  static KvCache paged(const KvCacheConfig& config, size_t page_size);

  bool is_paged() const { return paged_ != nullptr; }
  const KvCacheConfig& config() const;
  size_t used_tokens() const { return used_tokens_; }
  size_t remaining_tokens() const;
  void reset();
  void advance(size_t tokens);
  // kv_cache.rs:419-423: the next position, committed at once.
  size_t reserve_slot();
  // kv_cache.rs:441-451: a write at a committed position only (ensure_position_committed).
  void write(size_t layer, size_t position, const float* key, const float* value);
  void write_uncommitted(size_t layer, size_t position, const float* key, const float* value);
  void write_sequence_uncommitted(size_t layer, size_t start, size_t seq_len, const float* key,
                                  const float* value);
  void read_prefix(size_t layer, size_t length, std::vector<float>* key,
                   std::vector<float>* value) const;
  std::optional<PrefixHandle> prefix_handle(size_t token_count) const;
  void copy_prefix_from(const KvCache& source, size_t token_count);
  const ContiguousKvCacheStorage* contiguous_storage() const { return contiguous_.get(); }
  const PagedKvCacheStorage* paged_storage() const { return paged_.get(); }

 private:
  std::shared_ptr<ContiguousKvCacheStorage> contiguous_;
  std::shared_ptr<PagedKvCacheStorage> paged_;
  size_t used_tokens_ = 0;
};

// ---- model/config.rs:5-72 + model/decoder.rs:30-114 (weights as [in, out]) ----
struct ModelConfig {
  size_t hidden_size = 0;
  size_t intermediate_size = 0;
  size_t num_layers = 0;
  size_t num_attention_heads = 0;
  size_t num_key_value_heads = 0;
  size_t vocab_size = 0;
  size_t max_position_embeddings = 0;
  float rms_norm_eps = 1e-6f;
  float rope_theta = 10000.0f;
  size_t rotary_dims = 0;
  bool tie_word_embeddings = false;
  size_t head_dim() const { return hidden_size / num_attention_heads; }
};

struct LayerWeights {
  std::vector<float> attention_norm, wq, wq_bias, wk, wk_bias, wv, wv_bias, wo, wo_bias;
  std::vector<float> ffn_norm, w1, w1_bias, w2, w2_bias, w3, w3_bias;
};

struct Model {
  ModelConfig config;
  std::vector<float> tok_embeddings;  // [V, H]
  std::vector<LayerWeights> layers;
  std::vector<float> norm;    // [H]
  std::vector<float> output;  // [V, H] when not tied
  void validate() const;
  const std::vector<float>& output_weight() const {
    return config.tie_word_embeddings ? tok_embeddings : output;
  }
  // Sets a named tensor using the reference names (model/decoder.rs:30-52).
  void set_weight(const std::string& name, const float* data, size_t count);
};

struct TokenSample {
  uint32_t token_id;
  float probability;
};

enum class FinishReason : int32_t;

// ---- runtime/reference.rs model drivers ----
// Full-sequence logits [T, V] (reference.rs:517-524).
std::vector<float> decoder_model_forward(const Model& m, const std::vector<uint32_t>& ids);
// Prefill with KV capture; returns final-normed hidden [T, H] (reference.rs:372-423).
std::vector<float> prefill_hidden_with_kv_capture(const Model& m, const std::vector<uint32_t>& ids,
                                                  KvCache* kv);
// Decode one token at `position`; returns final-normed hidden [1, H] (reference.rs:664-710).
std::vector<float> token_hidden_with_kv_cache(const Model& m, uint32_t token, KvCache* kv,
                                              size_t position);
TokenSample sample_from_hidden_row(const Model& m, const float* hidden_row);
std::vector<float> logits_from_hidden_row(const Model& m, const float* hidden_row);

// ---- runtime/sampler.rs:3-43 SamplerConfig (greedy by default) ----
struct SamplerConfig {
  float temperature = 0.0f;
  size_t top_k = 1;
  float top_p = 1.0f;
  float repetition_penalty = 1.0f;
  uint64_t seed = 0;
  bool is_greedy() const;
  bool operator==(const SamplerConfig& o) const;  // sampler_configs_match (session.rs:415-421)
};

// ---- runtime/session.rs:92-413 Session ----
struct SessionConfig {
  size_t max_sequence_length = 4096;
  size_t max_generated_tokens = 512;
  size_t page_size = 0;  // 0 = contiguous KV, else paged with this page size
  SamplerConfig sampler;
};

class Session {
 public:
  Session(std::shared_ptr<const Model> model, const SessionConfig& config);
  size_t position() const { return position_; }
  const SessionConfig& config() const { return config_; }
  const KvCache& kv_cache() const { return kv_; }
  const std::vector<uint32_t>& token_history() const { return history_; }
  std::optional<TokenSample> last_sample() const { return last_sample_; }
  uint64_t sampler_state() const { return sampler_state_; }
  // Replaces the session's sampler configuration and restarts its state (a test hook; the
  // reference fixes it at construction).
  void set_sampler(const SamplerConfig& sampler);
  std::optional<PrefixHandle> prefix_handle(size_t token_count) const;
  void copy_prefix_from_session(const Session& source, size_t token_count);
  void reset();
  void prefill_tokens(const std::vector<uint32_t>& ids);
  TokenSample step_reference();
  // session.rs:262-331 generate_reference_from_tokens: reset, prefill the prompt, then step up
  // to min(max_new_tokens, max_generated_tokens) times, stopping at the stop token or at the
  // sequence length.  Returns the generated samples and the finish reason.
  std::vector<TokenSample> generate_from_tokens(const std::vector<uint32_t>& prompt, size_t max_new_tokens,
                                                std::optional<uint32_t> stop_token, FinishReason* finish);
  // Logits of the last processed position, recomputed by the logits path (parity aid).
  std::vector<float> last_hidden() const { return last_hidden_; }

 private:
  void process_token(uint32_t token);
  void process_prefill(const std::vector<uint32_t>& ids);
  TokenSample sample_hidden_row(const float* hidden_row);
  std::shared_ptr<const Model> model_;
  SessionConfig config_;
  KvCache kv_;
  size_t position_ = 0;
  std::vector<uint32_t> history_;
  std::optional<TokenSample> last_sample_;
  uint64_t sampler_state_;
  std::vector<float> last_hidden_;
};

// ---- runtime/sequence.rs:43-237 ----
enum class SequencePhase : int32_t { Prefill = 0, Decode = 1, Finished = 2 };
enum class FinishReason : int32_t {
  None = -1,
  StopToken = 0,
  MaxNewTokens = 1,
  SessionLimit = 2,
  SequenceLength = 3,
  Cancelled = 4,
};
enum class BatchKind : int32_t { Prefill = 0, Decode = 1 };

struct SequenceState {
  uint64_t request_id = 0;
  uint64_t sequence_id = 0;
  std::vector<uint32_t> prompt;
  std::vector<uint32_t> generated;
  size_t cached_tokens = 0;
  size_t requested_max_new_tokens = 0;
  size_t max_new_tokens = 0;
  std::optional<uint32_t> stop_token;
  SequencePhase phase = SequencePhase::Prefill;
  FinishReason finish_reason = FinishReason::None;

  size_t cached_prompt_tokens() const { return std::min(cached_tokens, prompt.size()); }
  size_t pending_prompt_tokens() const { return prompt.size() - cached_prompt_tokens(); }
  size_t next_prefill_chunk_len(size_t max_chunk) const {
    return std::min(pending_prompt_tokens(), max_chunk);
  }
  // sequence.rs:135-139
  std::vector<uint32_t> next_prefill_chunk(size_t max_chunk) const {
    size_t start = cached_prompt_tokens();
    return std::vector<uint32_t>(prompt.begin() + start, prompt.begin() + start + next_prefill_chunk_len(max_chunk));
  }
  bool is_finished() const { return phase == SequencePhase::Finished; }
  size_t total_tokens() const { return prompt.size() + generated.size(); }
  bool generation_budget_reached() const { return generated.size() >= max_new_tokens; }
  FinishReason generation_budget_finish_reason() const {
    return requested_max_new_tokens > max_new_tokens ? FinishReason::SessionLimit
                                                     : FinishReason::MaxNewTokens;
  }
  void record_prefill(size_t appended);
  void record_generated_token(uint32_t token);
  void finish(FinishReason reason) {
    phase = SequencePhase::Finished;
    finish_reason = reason;
  }
};

// ---- runtime/prefix_index.rs:1-113 ----
struct PrefixIndexEntry {
  uint64_t sequence_id;
  std::vector<uint32_t> prompt_tokens;
  size_t cached_prompt_tokens;
  size_t session_position;
};

class PrefixIndex {
 public:
  explicit PrefixIndex(size_t min_share) : min_share_(min_share) {}
  void clear() { buckets_.clear(); }
  void upsert(const PrefixIndexEntry& entry);
  // Returns (sequence_id, shared_prefix_tokens) of the best candidate.
  std::optional<std::pair<uint64_t, size_t>> best_match(uint64_t target,
                                                        const std::vector<uint32_t>& prompt) const;

 private:
  size_t min_share_;
  std::map<std::vector<uint32_t>, std::vector<PrefixIndexEntry>> buckets_;
};

// ---- runtime/block_manager.rs:58-172 ----
struct ManagedBlockId {
  uint64_t owner_sequence_id;
  size_t layer_index;
  size_t block_id;
  bool operator<(const ManagedBlockId& o) const {
    if (owner_sequence_id != o.owner_sequence_id) return owner_sequence_id < o.owner_sequence_id;
    if (layer_index != o.layer_index) return layer_index < o.layer_index;
    return block_id < o.block_id;
  }
  bool operator==(const ManagedBlockId& o) const {
    return owner_sequence_id == o.owner_sequence_id && layer_index == o.layer_index &&
           block_id == o.block_id;
  }
};

struct SharedPrefixAssignment {
  uint64_t source_sequence_id;
  PrefixHandle handle;
};

class PrefixBlockManager {
 public:
  std::vector<ManagedBlockId> update_owned_prefix(uint64_t seq, std::optional<PrefixHandle> h);
  std::vector<ManagedBlockId> update_shared_prefix(uint64_t seq,
                                                   std::optional<SharedPrefixAssignment> a);
  std::vector<ManagedBlockId> remove_sequence(uint64_t seq);
  size_t block_ref_count(const ManagedBlockId& id) const;
  size_t tracked_block_count() const { return ref_counts_.size(); }
  const PrefixHandle* owned_prefix(uint64_t seq) const;
  const SharedPrefixAssignment* shared_prefix(uint64_t seq) const;

 private:
  std::vector<ManagedBlockId> apply(uint64_t owner, const PrefixHandle& h, bool increment);
  std::map<uint64_t, PrefixHandle> owned_;
  std::map<uint64_t, SharedPrefixAssignment> shared_;
  std::map<ManagedBlockId, size_t> ref_counts_;
};

// ---- runtime/scheduler.rs:16-648 ----
struct SchedulerConfig {
  size_t max_batch_size = 16;
  size_t max_prefill_chunk_tokens = 256;
  size_t max_prefill_batch_tokens = 1024;
  size_t max_consecutive_prefill_ticks = 2;
  size_t min_prefix_share_tokens = 64;
};

struct SequenceExecutionUpdate {
  uint64_t request_id;
  uint64_t sequence_id;
  BatchKind batch_kind;
  size_t reused_prompt_tokens;
  size_t appended_prompt_tokens;
  int64_t shared_from;  // sequence the prefix was copied from, -1 if none (test aid)
  bool has_token;
  TokenSample generated;
  SequencePhase phase;
  FinishReason finish_reason;
  std::vector<ManagedBlockId> released_prefix_blocks;
};

struct SchedulerTick {
  BatchKind kind;
  std::vector<uint64_t> sequence_ids;
};

struct SchedulerReport {
  SchedulerTick tick;
  std::vector<SequenceExecutionUpdate> updates;
};

class ReferenceScheduler {
 public:
  ReferenceScheduler(std::shared_ptr<const Model> model, const SessionConfig& session_config,
                     const SchedulerConfig& config);
  uint64_t submit(const std::vector<uint32_t>& prompt, size_t max_new_tokens,
                  std::optional<uint32_t> stop_token);
  std::optional<SchedulerTick> plan_next_tick() const;
  std::optional<SchedulerReport> execute_next_tick();
  bool has_pending() const;
  // scheduler.rs:184-189: sequences still holding a session.
  size_t resident_session_count() const;
  const SequenceState* sequence_state(uint64_t seq) const;
  const Session* session(uint64_t seq) const;
  const PrefixBlockManager& block_manager() const { return block_manager_; }
  // The sampler configuration of the sessions submitted from now on (SessionConfig::sampler).
  void set_sampler(const SamplerConfig& sampler) { session_config_.sampler = sampler; }

 private:
  struct Entry {
    SequenceState state;
    std::unique_ptr<Session> session;
  };
  std::vector<uint64_t> collect_prefill_ids() const;
  std::vector<uint64_t> collect_decode_ids() const;
  bool should_schedule_decode(size_t prefill, size_t decode) const;
  size_t maybe_share_prefix(uint64_t seq, int64_t* source);
  SequenceExecutionUpdate execute_prefill(uint64_t seq);
  SequenceExecutionUpdate execute_decode(uint64_t seq);
  void rebuild_prefix_index();
  void refresh_sequence_prefix_metadata(uint64_t seq);
  std::vector<ManagedBlockId> release_sequence_resources(uint64_t seq);
  size_t index_of(uint64_t seq) const;

  std::shared_ptr<const Model> model_;
  SessionConfig session_config_;
  SchedulerConfig config_;
  uint64_t next_request_id_ = 0;
  uint64_t next_sequence_id_ = 0;
  size_t consecutive_prefill_ticks_ = 0;
  PrefixIndex prefix_index_;
  PrefixBlockManager block_manager_;
  std::vector<Entry> sequences_;
};

// ---- Batch packer restated over a global page pool (test oracle for the GPU runtime's
// packing).  It applies the reference's logical-block math (paged_kv.rs:605-606, 717-720:
// position p -> logical block p / page_size, offset p % page_size, slot = block * page_size +
// offset), first-touch allocation from a LIFO free list initialised [n-1 .. 0]
// (paged_kv.rs:469-527, 794-796) shared by all sequences, prefix sharing by page id with a
// copy of a partially filled last page, and release of a finished sequence's pages (in
// block-table order, after its tick) when their reference count drops to zero.
struct PackedTick {
  int32_t kind = 0;
  std::vector<uint64_t> sequence_ids;
  std::vector<int32_t> positions;
  std::vector<int64_t> slot_mapping;
  std::vector<int32_t> cu_seqlens;
  std::vector<int32_t> context_lens;
  std::vector<std::vector<int32_t>> block_tables;  // per sequence, ceil(ctx / page) entries
  std::vector<int32_t> copy_src, copy_dst, copy_count;
};

class GlobalPagePacker {
 public:
  GlobalPagePacker(size_t num_pages, size_t page_size);
  PackedTick pack(const SchedulerReport& report);
  size_t free_pages() const { return free_.size(); }
  const std::vector<int32_t>& pages_of(uint64_t seq) { return seqs_[seq].pages; }

 private:
  struct Seq {
    std::vector<int32_t> pages;
    size_t position = 0;
  };
  int32_t allocate();
  void decref(int32_t page);
  size_t page_size_;
  std::vector<int32_t> free_;
  std::vector<int32_t> refs_;
  std::map<uint64_t, Seq> seqs_;
};

}  // namespace orc
