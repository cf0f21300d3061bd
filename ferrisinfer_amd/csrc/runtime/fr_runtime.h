// Host runtime of the MI355X path (C++17): the reference's ReferenceScheduler / Session /
// KvCache API (crates/ferrisinfer-runtime/src/{scheduler,session,kv_cache,paged_kv,
// block_manager,prefix_index,sequence}.rs) driving the HIP backend only through the C ABI of
// include/ferrisinfer_kernel.h.
//
// The scheduler decides ticks exactly as the reference does, but executes each tick as ONE
// ragged batch: every sequence of the tick is packed (cu_seqlens, positions, slot_mapping,
// block tables, context lengths) and the decoder runs once over the batch.  KV lives in one
// global block pool; a shared prefix is referenced by block id (refcounted) and only a
// partially filled last block is copied.
#pragma once

#include <array>
#include <cstdint>
#include <deque>
#include <map>
#include <optional>
#include <string>
#include <vector>

#include "../../../include/ferrisinfer_kernel.h"

namespace fr {

// Mirrors core/error.rs:5-16; status codes are kind + 1 at the C boundary.
enum class ErrorKind : int32_t {
  Io = 0, Parse, InvalidShape, InvalidLayout, InvalidType, InvalidConfig, MissingWeight, Unsupported, Runtime,
};

struct Error {
  ErrorKind kind;
  std::string message;
};

[[noreturn]] void fail(ErrorKind kind, const std::string& message);
// Throws the backend's error (status + fi_last_error) when status != 0.
void check(int32_t status);

// ---------------------------------------------------------------------------------------
// Device memory owned by the runtime.
class DeviceBuffer {
 public:
  DeviceBuffer() = default;
  DeviceBuffer(fi_context* ctx, size_t bytes);
  ~DeviceBuffer();
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept;
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
  void* get() const { return ptr_; }
  float* f32() const { return static_cast<float*>(ptr_); }
  size_t bytes() const { return bytes_; }
  // Grows (reallocating, contents lost) to at least `bytes`.
  void reserve(fi_context* ctx, size_t bytes);

 private:
  fi_context* ctx_ = nullptr;
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

// ---------------------------------------------------------------------------------------
// model/config.rs:5-72
struct ModelConfig {
  int32_t hidden_size = 0;
  int32_t intermediate_size = 0;
  int32_t num_layers = 0;
  int32_t num_attention_heads = 0;
  int32_t num_key_value_heads = 0;
  int32_t vocab_size = 0;
  int32_t max_position_embeddings = 0;
  float rms_norm_eps = 1e-6f;
  float rope_theta = 10000.0f;
  int32_t rotary_dims = 0;
  bool tie_word_embeddings = false;
  int32_t head_dim() const { return hidden_size / num_attention_heads; }
  void validate() const;
};

// Weights resident in HBM, named and shaped as model/decoder.rs:30-114 ([in, out] layout).
class DeviceModel {
 public:
  struct Layer {
    DeviceBuffer attention_norm, wq, wq_bias, wk, wk_bias, wv, wv_bias, wo, wo_bias;
    DeviceBuffer ffn_norm, w1, w1_bias, w2, w2_bias, w3, w3_bias;
  };
  // Projections re-laid out once for the projection GEMMs (include/ferrisinfer_kernel.h): q|k|v
  // as one column-concatenated matrix, wo, w1/w3 as a SwiGLU pair, w2.  f32 weights are packed
  // for fi_gemm_packed (pack widths below); bf16 weights (rounded to nearest even from the f32
  // tensors, exact for bf16 checkpoints) for fi_gemm_bf16.
  struct Packed {
    DeviceBuffer qkv, wo, w13, w2;
  };
  // q|k|v, wo and w2 on the 32-column layout (three-piece bf16 products); the SwiGLU pair and
  // the greedy head keep their two-column packs
  static constexpr int32_t kQkvPack = 32, kWoPack = 32, kW2Pack = 32, kLmPack = 2;

  // weight_dtype: FI_DTYPE_F32 or FI_DTYPE_BF16, the storage of the packed projections and head.
  DeviceModel(fi_context* ctx, const ModelConfig& config, int32_t rope_positions, int32_t weight_dtype = FI_DTYPE_F32);
  void set_weight(const std::string& name, const float* host, size_t count);
  // The same from device memory: `count` elements of src_dtype (FI_DTYPE_F32 / _BF16 / _F16)
  // widened into the weight's f32 slot on the device.
  void set_weight_device(const std::string& name, const void* device, int32_t src_dtype, size_t count);
  // The device buffer of weight `name` sized for `count` floats (contents undefined until
  // written); InvalidShape when count is not the tensor's size, MissingWeight for an unknown
  // name.  set_weight uploads into it; the checkpoint loader converts into it on the device.
  DeviceBuffer* weight_slot(const std::string& name, size_t count);
  void validate() const;  // every required tensor present (MissingWeight otherwise)
  // Packs every projection once the weights are complete and releases the unpacked copies
  // (the tied embedding stays: the gather reads it).  Idempotent.
  void finalize();
  bool finalized() const { return finalized_; }
  const Packed& packed(int i) const { return packed_.at(i); }
  const void* lm_head_packed() const { return lm_packed_.get(); }
  int32_t weight_dtype() const { return weight_dtype_; }
  const ModelConfig& config() const { return config_; }
  const Layer& layer(int i) const { return layers_.at(i); }
  const float* tok_embeddings() const { return tok_embeddings_.f32(); }
  const float* norm() const { return norm_.f32(); }
  const float* output_weight() const {
    return config_.tie_word_embeddings ? tok_embeddings_.f32() : output_.f32();
  }
  const float* rope_cos() const { return rope_cos_.f32(); }
  const float* rope_sin() const { return rope_sin_.f32(); }
  int32_t rope_positions() const { return rope_positions_; }
  fi_context* ctx() const { return ctx_; }

 private:
  fi_context* ctx_;
  ModelConfig config_;
  std::vector<Layer> layers_;
  std::vector<Packed> packed_;
  DeviceBuffer tok_embeddings_, norm_, output_, rope_cos_, rope_sin_, lm_packed_;
  int32_t rope_positions_;
  int32_t weight_dtype_;
  bool finalized_ = false;
};

// ---------------------------------------------------------------------------------------
// Global KV block pool: per layer K and V [num_blocks, Hkv, block_size, D].  The free list
// generalises the reference's per-session LIFO page list (runtime/paged_kv.rs:469-527,
// 794-796): it starts as [n-1, ..., 0] and pops from the back, so block 0 goes first; a block
// returns to the back of the list when its refcount drops to zero.
class BlockPool {
 public:
  BlockPool(fi_context* ctx, int32_t layers, int32_t num_blocks, int32_t block_size, int32_t kv_heads,
            int32_t head_dim, int32_t kv_dtype);
  int32_t allocate();
  // The block the k-th next allocate() would return with no frees in between, or -1.
  int32_t peek(size_t k) const {
    return k < free_.size() ? free_[free_.size() - 1 - k] : -1;
  }
  void incref(int32_t block);
  void decref(int32_t block);
  int32_t refcount(int32_t block) const { return refs_.at(block); }
  size_t free_count() const { return free_.size(); }
  int32_t num_blocks() const { return num_blocks_; }
  int32_t block_size() const { return block_size_; }
  int32_t kv_dtype() const { return kv_dtype_; }
  void* k(int32_t layer) const { return k_.at(layer).get(); }
  void* v(int32_t layer) const { return v_.at(layer).get(); }

 private:
  int32_t num_blocks_, block_size_, kv_dtype_;
  std::vector<int32_t> free_;
  std::vector<int32_t> refs_;
  std::vector<DeviceBuffer> k_, v_;
};

// ---------------------------------------------------------------------------------------
// runtime/sequence.rs:43-237
enum class Phase : int32_t { Prefill = 0, Decode = 1, Finished = 2 };
enum class FinishReason : int32_t {
  None = -1, StopToken = 0, MaxNewTokens = 1, SessionLimit = 2, SequenceLength = 3, Cancelled = 4,
};
enum class BatchKind : int32_t { Prefill = 0, Decode = 1 };

struct TokenSample {
  uint32_t token_id = 0;
  float probability = 0.0f;
};

// One request: the reference's SequenceState plus the state its Session keeps (position,
// token history, last sample) and its KV block table in the global pool.
struct Sequence {
  uint64_t request_id = 0;
  uint64_t sequence_id = 0;
  std::vector<uint32_t> prompt;
  std::vector<uint32_t> generated;
  size_t cached_tokens = 0;
  size_t requested_max_new_tokens = 0;
  size_t max_new_tokens = 0;
  std::optional<uint32_t> stop_token;
  Phase phase = Phase::Prefill;
  FinishReason finish_reason = FinishReason::None;
  // session state (runtime/session.rs:92-102)
  bool resident = true;
  size_t position = 0;
  std::vector<uint32_t> history;
  std::optional<TokenSample> last_sample;
  uint64_t sampler_state = 0;  // SamplerState of the session (session.rs:100, 138)
  // KV: logical block i -> pool block blocks[i]
  std::vector<int32_t> blocks;

  size_t cached_prompt_tokens() const { return cached_tokens < prompt.size() ? cached_tokens : prompt.size(); }
  size_t pending_prompt_tokens() const { return prompt.size() - cached_prompt_tokens(); }
  size_t next_prefill_chunk_len(size_t max_chunk) const {
    return pending_prompt_tokens() < max_chunk ? pending_prompt_tokens() : max_chunk;
  }
  bool generation_budget_reached() const { return generated.size() >= max_new_tokens; }
  FinishReason generation_budget_finish_reason() const {
    return requested_max_new_tokens > max_new_tokens ? FinishReason::SessionLimit : FinishReason::MaxNewTokens;
  }
  void record_prefill(size_t appended);
  void record_generated_token(uint32_t token);
  void finish(FinishReason reason) {
    phase = Phase::Finished;
    finish_reason = reason;
  }
};

// runtime/block_manager.rs:5-56 (ManagedBlockId) — the reference's prefix metadata; layer
// tables of one sequence are identical here since all layers share the block table.
struct ManagedBlockId {
  uint64_t owner_sequence_id;
  int32_t layer_index;
  int32_t block_id;
  bool operator<(const ManagedBlockId& o) const {
    if (owner_sequence_id != o.owner_sequence_id) return owner_sequence_id < o.owner_sequence_id;
    if (layer_index != o.layer_index) return layer_index < o.layer_index;
    return block_id < o.block_id;
  }
};

struct PrefixHandle {
  size_t token_count = 0;
  int32_t layers = 0;
  std::vector<int32_t> blocks;  // ceil(token_count / block_size) entries, same on every layer
};

class PrefixBlockManager {
 public:
  std::vector<ManagedBlockId> update_owned_prefix(uint64_t seq, std::optional<PrefixHandle> h);
  // update_owned_prefix for callers that drop the release list (scheduler.rs:575-588)
  void refresh_owned_prefix(uint64_t seq, std::optional<PrefixHandle> h);
  std::vector<ManagedBlockId> update_shared_prefix(uint64_t seq, std::optional<std::pair<uint64_t, PrefixHandle>> a);
  std::vector<ManagedBlockId> remove_sequence(uint64_t seq);
  size_t ref_count(const ManagedBlockId& id) const;

 private:
  std::vector<ManagedBlockId> apply(uint64_t owner, const PrefixHandle& h, bool increment);
  std::map<uint64_t, PrefixHandle> owned_;
  std::map<uint64_t, std::pair<uint64_t, PrefixHandle>> shared_;
  std::map<ManagedBlockId, size_t> refs_;
};

// runtime/prefix_index.rs:24-113
class PrefixIndex {
 public:
  struct Entry {
    uint64_t sequence_id;
    const std::vector<uint32_t>* prompt;
    size_t cached_prompt_tokens;
    size_t session_position;
  };
  explicit PrefixIndex(size_t min_share) : min_share_(min_share) {}
  void rebuild(const std::vector<Sequence>& seqs);
  std::optional<std::pair<uint64_t, size_t>> best_match(uint64_t target, const std::vector<uint32_t>& prompt) const;

 private:
  size_t min_share_;
  std::map<std::vector<uint32_t>, std::vector<Entry>> buckets_;
};

// runtime/scheduler.rs:16-35, session.rs:29-46
struct SchedulerConfig {
  size_t max_batch_size = 16;
  size_t max_prefill_chunk_tokens = 256;
  size_t max_prefill_batch_tokens = 1024;
  size_t max_consecutive_prefill_ticks = 2;
  size_t min_prefix_share_tokens = 64;
};

// runtime/sampler.rs:3-43: SamplerConfig (greedy by default) and SamplerState (xorshift64*).
struct SamplerConfig {
  float temperature = 0.0f;
  int64_t top_k = 1;
  float top_p = 1.0f;
  float repetition_penalty = 1.0f;
  uint64_t seed = 0;
  bool is_greedy() const { return temperature <= 0.0f || top_k == 1 || top_p <= 0.0f; }  // sampler.rs:40-42
};
uint64_t sampler_state_new(uint64_t seed);   // SamplerState::new (sampler.rs:55-63)
uint64_t sampler_state_next(uint64_t state);  // the state after one draw (sampler.rs:65-70)

struct SessionConfig {
  size_t max_sequence_length = 4096;
  size_t max_generated_tokens = 512;
  SamplerConfig sampler;  // every session's sampler (session.rs:29-46)
};

// runtime/scheduler.rs:54-71
struct SequenceUpdate {
  uint64_t request_id;
  uint64_t sequence_id;
  BatchKind batch_kind;
  size_t reused_prompt_tokens;
  size_t appended_prompt_tokens;
  bool has_token;
  TokenSample generated;
  Phase phase;
  FinishReason finish_reason;
  std::vector<ManagedBlockId> released_prefix_blocks;
};

struct TickReport {
  BatchKind kind;
  std::vector<uint64_t> sequence_ids;
  std::vector<SequenceUpdate> updates;
};

// Metadata of one packed ragged batch, as uploaded to the device (host copy for tests).
struct PackedBatch {
  BatchKind kind = BatchKind::Prefill;
  std::vector<uint64_t> sequence_ids;      // sequences with tokens in the batch, in tick order
  std::vector<int32_t> token_ids;          // [T]
  std::vector<int32_t> positions;          // [T]
  std::vector<int64_t> slot_mapping;       // [T]
  std::vector<int32_t> cu_seqlens;         // [B+1]
  std::vector<int32_t> context_lens;       // [B]
  std::vector<int32_t> block_tables;       // [B, max_blocks]
  int32_t max_blocks = 0;
  std::vector<int32_t> last_rows;          // [B] index of each sequence's last token
  std::vector<int32_t> copy_src, copy_dst, copy_count;  // copy-on-write of partial blocks
  int32_t max_query_len = 0;
  int32_t max_context_len = 0;
};

// Runs the decoder over packed batches (one launch sequence per tick).
//
// Decode ticks can be replayed from HIP graphs (BackendCapabilities.graph_capture,
// kernel/backend.rs:3-10; docs/performance-roadmap.md:321-326).  A decode tick's launch sequence
// is fixed by (batch size, block-table stride, max_context_len, sampler kind) once every device
// buffer it touches stays put; the batch metadata is re-uploaded into the same buffer before each
// replay.  With graphs on, a decode tick rounds max_context_len up to a multiple of
// kGraphContextBucket tokens and pads the block table to that width: the extra partitions of the
// decode kernel find no keys and exit, and each sequence's reduction order depends only on its own
// context length, so replays give the eager path's bits.  A shape is captured the second time it
// occurs (the first, eager run sizes the context workspace); graphs are dropped whenever a buffer
// they recorded moves (an executor buffer grows, or the context workspace's generation changes).
class ForwardExecutor {
 public:
  static constexpr int32_t kGraphContextBucket = 1024;
  ForwardExecutor(const DeviceModel* model, BlockPool* pool, bool graph_decode = false);
  ~ForwardExecutor();
  ForwardExecutor(const ForwardExecutor&) = delete;
  ForwardExecutor& operator=(const ForwardExecutor&) = delete;
  // Returns one sample per batch sequence from its last row: the fused argmax head for a
  // greedy sampler, else the row's logits through the device sampler with states[i]
  // (advanced in place by one draw per sequence).  run = launch + collect.
  std::vector<TokenSample> run(const PackedBatch& batch, const SamplerConfig& sampler, std::vector<uint64_t>* states);
  // Enqueues one tick (uploads, forward, the copy of its samples and fault words into pinned
  // host memory) and returns without waiting.  feed_rows (a decode tick enqueued behind the
  // previous launch): row i's input token, and for a sampled tick its sampler state, are the
  // previous launch's sample and advanced state of row feed_rows[i] when that is >= 0, read on
  // the device; other rows keep the batch's token id and states[i].
  void launch(const PackedBatch& batch, const SamplerConfig& sampler, const std::vector<uint64_t>* states,
              const std::vector<int32_t>* feed_rows = nullptr);
  // Waits for the oldest launched tick and returns its samples (states: the sampled path's
  // advanced states, downloaded).
  std::vector<TokenSample> collect(std::vector<uint64_t>* states);
  // Waits for the oldest launched tick and drops its samples.
  void discard();
  size_t in_flight() const { return inflight_.size(); }
  // Whether launch(batch, ..., feed_rows) can run behind the single tick in flight: a decode
  // tick that keeps the previous tick's samples in place (no reallocation of them).
  bool can_feed(const PackedBatch& batch) const;
  // Host seconds of the last launch (enqueueing every launch) and the last collect (waiting for
  // the samples).
  double last_enqueue_seconds() const { return enqueue_s_; }
  double last_wait_seconds() const { return wait_s_; }
  // Decode ticks replayed from a graph, graphs captured, graphs dropped (since creation).
  std::array<uint64_t, 3> graph_counters() const { return {graph_replays_, graph_captures_, graph_drops_}; }
  // The logits rows the last run sampled from ([rows, vocab] f32, batch order) into host
  // memory of `capacity` floats; rows is 0 after a greedy run (its head is fused with the
  // argmax and writes no logits).
  void last_logits(float* host, size_t capacity, int64_t* rows) const;

 private:
  // Every scalar and device pointer of one tick's launch sequence.
  struct Plan {
    BatchKind kind;
    int32_t T, B, max_blocks, max_context_len, max_query_len, n_copy;
    int32_t s_qkv, s_o, s_w2;
    const int32_t *ids, *pos, *cu, *ctx, *bt, *last, *cs, *cd, *cc;
    const int64_t* slot;
    bool greedy;
    int32_t ss;  // sampling slot: the logits and sampler buffers of a sampled tick
  };
  void reserve(size_t tokens, size_t seqs);
  void grow(DeviceBuffer& b, size_t bytes);  // reserve, noting a moved buffer
  void copy_only(const PackedBatch& batch);
  void splits(int32_t m, int32_t k, int32_t n, int32_t pack_width, int32_t* out) const;
  void projection(const float* a, int32_t lda, const DeviceBuffer& w, int32_t k, int32_t n, int32_t pack_width,
                  int32_t m, int32_t splits, float* out) const;
  void enqueue(const Plan& p);
  void drop_graphs();
  void host_reserve(int slot, size_t meta_bytes, size_t out_bytes);
  // One launched tick: its pinned slot and batch size (B = 0: a copy-only tick, no samples).
  struct Pending {
    int32_t slot;
    int32_t B;
    bool greedy;
    int32_t ss;
  };
  const DeviceModel* model_;
  BlockPool* pool_;
  fi_context* ctx_;
  DeviceBuffer meta_, hidden_, normed_, q_, attn_, h1_, act_, parts_, last_norm_;
  // Sampled ticks alternate between two sampling slots, each a logits buffer [B, vocab] and a
  // sampler buffer (states [B] u64, temperature [B], top_k [B], top_p [B]): a tick enqueued
  // behind a sampled tick reads that tick's advanced states from the other slot.
  DeviceBuffer logits_[2], samp_[2];
  // one tick's samples: B token ids, then B probabilities (one download)
  DeviceBuffer out_;
  size_t cap_tokens_ = 0, cap_seqs_ = 0, cap_parts_ = 0;
  double enqueue_s_ = 0.0, wait_s_ = 0.0;
  bool graph_decode_;
  uint64_t buffers_moved_ = 0;             // bumped whenever an executor buffer is reallocated
  uint64_t graphs_buffers_ = 0, graphs_workspace_ = 0;  // generations the cached graphs recorded
  // (B, stride, max_context_len, 1 greedy / 2 + sampling slot)
  std::map<std::array<int32_t, 4>, fi_graph*> graphs_;
  std::map<std::array<int32_t, 4>, int32_t> seen_;       // eager runs per shape since the last drop
  uint64_t graph_replays_ = 0, graph_captures_ = 0, graph_drops_ = 0;
  int32_t logits_rows_[2] = {0, 0};  // rows each sampling slot's logits hold
  int32_t samp_next_ = 0;            // the slot of the next sampled launch
  int32_t samp_last_ = -1;           // the slot of the last collected tick (-1: greedy or none)
  // Consecutive launches alternate between two pinned slots (metadata staging, then a sampled
  // tick's sampler configuration; samples, the four fault words, then the advanced sampler
  // states) and two events; at most two ticks are in flight.
  std::deque<Pending> inflight_;
  void* h_meta_[2] = {nullptr, nullptr};
  void* h_out_[2] = {nullptr, nullptr};
  size_t h_meta_bytes_[2] = {0, 0}, h_out_bytes_[2] = {0, 0};
  fi_event* events_[2] = {nullptr, nullptr};
  int32_t next_slot_ = 0;
  int32_t out_rows_ = 0;  // samples the last launch leaves in out_
};

// runtime/scheduler.rs:109-648 over the batched executor.
class Scheduler {
 public:
  Scheduler(DeviceModel* model, BlockPool* pool, const SessionConfig& session, const SchedulerConfig& config,
            bool graph_decode = false);
  uint64_t submit(const std::vector<uint32_t>& prompt, size_t max_new_tokens, std::optional<uint32_t> stop_token);
  std::optional<std::pair<BatchKind, std::vector<uint64_t>>> plan_next_tick() const;
  // run_ahead: once this tick is enqueued, also enqueue the next tick when it will be a decode
  // tick (stream overlap, docs/performance-roadmap.md:321-326).  Its batch follows from the
  // state this tick leaves except the token ids (and a sampled session's sampler states), which
  // are this tick's samples, fed on the device.  The next call keeps it when its own planning packs the same batch and drops it
  // otherwise (after a submit, for instance): the ticks and their results are those of calls
  // without run_ahead.
  std::optional<TickReport> execute_next_tick(bool run_ahead = false);
  // [ticks enqueued ahead, kept, dropped, 1 if the last tick was one enqueued ahead]
  std::array<uint64_t, 4> run_ahead_counters() const {
    return {ahead_launched_, ahead_kept_, ahead_dropped_, last_tick_ahead_ ? 1u : 0u};
  }
  bool has_pending() const;
  const Sequence* sequence(uint64_t id) const;
  const PackedBatch& last_batch() const { return last_batch_; }
  // Host seconds of the last tick: [scheduling and packing, enqueueing the forward, waiting
  // for its samples, the whole tick].
  std::array<double, 4> last_tick_profile() const { return tick_profile_; }
  const PrefixBlockManager& block_manager() const { return block_manager_; }
  const BlockPool& pool() const { return *pool_; }
  const ForwardExecutor& executor() const { return executor_; }

 private:
  size_t index_of(uint64_t id) const;
  std::vector<uint64_t> collect_prefill_ids() const;
  std::vector<uint64_t> collect_decode_ids() const;
  bool should_schedule_decode(size_t prefill, size_t decode) const;
  std::optional<PrefixHandle> prefix_handle(const Sequence& s, size_t tokens) const;
  void refresh_prefix_metadata(uint64_t id);
  size_t maybe_share_prefix(uint64_t id, PackedBatch* batch, uint64_t* source_id);
  void share_blocks(Sequence& target, const Sequence& source, size_t tokens, PackedBatch* batch);
  void append_to_batch(Sequence& s, const std::vector<uint32_t>& tokens, PackedBatch* batch);
  std::vector<ManagedBlockId> release(uint64_t id);
  void finalize_batch(PackedBatch* batch) const;
  bool launch_ahead(const PackedBatch& current);
  bool ahead_matches(const PackedBatch& batch) const;
  void drop_ahead();

  DeviceModel* model_;
  BlockPool* pool_;
  ForwardExecutor executor_;
  SessionConfig session_;
  SchedulerConfig config_;
  uint64_t next_request_id_ = 0;
  uint64_t next_sequence_id_ = 0;
  size_t consecutive_prefill_ticks_ = 0;
  PrefixIndex prefix_index_;
  PrefixBlockManager block_manager_;
  std::vector<Sequence> sequences_;
  PackedBatch last_batch_;
  std::array<double, 4> tick_profile_{};
  // The tick enqueued ahead: its batch (token ids of fed rows unset), the row of the previous
  // tick each of its rows is fed from (-1: the batch's own id), and that tick's samples.
  struct Ahead {
    bool active = false;
    uint64_t state = 0;
    PackedBatch batch;
    std::vector<int32_t> feed_rows;
    std::vector<TokenSample> fed;
  };
  Ahead ahead_;
  uint64_t state_ = 0;  // bumped by every submit: an ahead tick planned before one is dropped
  uint64_t ahead_launched_ = 0, ahead_kept_ = 0, ahead_dropped_ = 0;
  bool last_tick_ahead_ = false;
};

}  // namespace fr
