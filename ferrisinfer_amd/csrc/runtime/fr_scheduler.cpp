// Scheduler of the host runtime: the reference's tick planning, prefix sharing and finish
// rules (crates/ferrisinfer-runtime/src/scheduler.rs:16-648, sequence.rs, prefix_index.rs,
// block_manager.rs, session.rs) with each tick executed as one packed batch.
//
// The reference executes a tick's sequences one after another (scheduler.rs:399-407).  Here
// the per-sequence bookkeeping runs in that same order on the host — prefix matching,
// block-table growth, positions, finish checks — and only the arithmetic is batched.  That
// is equivalent because (a) every decision in the loop depends on token counts, never on the
// sampled values of the same tick, and (b) per layer, the KV append of all sequences
// precedes the attention of all sequences, so a sequence that shares a prefix computed
// earlier in the same tick reads it in the same layer pass.  Samples produced by the forward
// are written back afterwards (including the last_sample a target copies from a source
// whose whole history it shared, session.rs:193-201), and blocks of sequences that finish in
// the tick return to the pool only after the forward.
#include <algorithm>
#include <chrono>
#include <map>

#include "fr_runtime.h"

namespace fr {

// ----------------------------------------------------------------------------- Sequence
void Sequence::record_prefill(size_t appended) {
  cached_tokens += appended;
  if (phase != Phase::Finished) phase = pending_prompt_tokens() == 0 ? Phase::Decode : Phase::Prefill;
}

void Sequence::record_generated_token(uint32_t token) {
  generated.push_back(token);
  cached_tokens += 1;
  if (phase != Phase::Finished) phase = Phase::Decode;
}

// ----------------------------------------------------------------------------- block manager
std::vector<ManagedBlockId> PrefixBlockManager::apply(uint64_t owner, const PrefixHandle& h, bool increment) {
  std::vector<ManagedBlockId> released;
  for (int32_t l = 0; l < h.layers; ++l) {
    for (int32_t blk : h.blocks) {
      ManagedBlockId id{owner, l, blk};
      if (increment) {
        refs_[id] += 1;
      } else {
        auto it = refs_.find(id);
        if (it != refs_.end()) {
          if (it->second > 0) it->second -= 1;
          if (it->second == 0) {
            refs_.erase(it);
            released.push_back(id);
          }
        }
      }
    }
  }
  return released;
}

std::vector<ManagedBlockId> PrefixBlockManager::update_owned_prefix(uint64_t seq, std::optional<PrefixHandle> h) {
  std::vector<ManagedBlockId> released;
  auto it = owned_.find(seq);
  if (it != owned_.end()) {
    PrefixHandle prev = std::move(it->second);
    owned_.erase(it);
    released = apply(seq, prev, false);
  }
  if (h) {
    apply(seq, *h, true);
    owned_[seq] = std::move(*h);
  }
  return released;
}

void PrefixBlockManager::refresh_owned_prefix(uint64_t seq, std::optional<PrefixHandle> h) {
  // Replacing a handle by an identical one decrements and re-increments the same counts: the
  // reference discards the release list of this call (scheduler.rs:575-588), so skipping
  // the round trip leaves every observable count unchanged.
  auto it = owned_.find(seq);
  if (h && it != owned_.end() && it->second.token_count == h->token_count && it->second.layers == h->layers &&
      it->second.blocks == h->blocks) {
    return;
  }
  (void)update_owned_prefix(seq, std::move(h));
}

std::vector<ManagedBlockId> PrefixBlockManager::update_shared_prefix(
    uint64_t seq, std::optional<std::pair<uint64_t, PrefixHandle>> a) {
  std::vector<ManagedBlockId> released;
  auto it = shared_.find(seq);
  if (it != shared_.end()) {
    auto prev = std::move(it->second);
    shared_.erase(it);
    released = apply(prev.first, prev.second, false);
  }
  if (a) {
    apply(a->first, a->second, true);
    shared_[seq] = std::move(*a);
  }
  return released;
}

std::vector<ManagedBlockId> PrefixBlockManager::remove_sequence(uint64_t seq) {
  auto released = update_shared_prefix(seq, std::nullopt);
  auto more = update_owned_prefix(seq, std::nullopt);
  released.insert(released.end(), more.begin(), more.end());
  return released;
}

size_t PrefixBlockManager::ref_count(const ManagedBlockId& id) const {
  auto it = refs_.find(id);
  return it == refs_.end() ? 0 : it->second;
}

// ----------------------------------------------------------------------------- prefix index
void PrefixIndex::rebuild(const std::vector<Sequence>& seqs) {
  buckets_.clear();
  if (min_share_ == 0) return;
  for (const Sequence& s : seqs) {
    if (s.phase == Phase::Finished) continue;
    if (s.prompt.size() < min_share_ || s.cached_prompt_tokens() < min_share_) continue;
    std::vector<uint32_t> key(s.prompt.begin(), s.prompt.begin() + min_share_);
    buckets_[key].push_back(Entry{s.sequence_id, &s.prompt, s.cached_prompt_tokens(), s.cached_tokens});
  }
}

std::optional<std::pair<uint64_t, size_t>> PrefixIndex::best_match(uint64_t target,
                                                                   const std::vector<uint32_t>& prompt) const {
  if (min_share_ == 0 || prompt.size() < min_share_) return std::nullopt;
  std::vector<uint32_t> key(prompt.begin(), prompt.begin() + min_share_);
  auto it = buckets_.find(key);
  if (it == buckets_.end()) return std::nullopt;
  std::optional<std::pair<uint64_t, size_t>> best;
  for (const Entry& e : it->second) {
    if (e.sequence_id == target) continue;
    const std::vector<uint32_t>& other = *e.prompt;
    size_t common = 0;
    while (common < prompt.size() && common < other.size() && prompt[common] == other[common]) ++common;
    size_t shared = std::min(common, e.cached_prompt_tokens);
    // keep one token to compute when the whole target prompt would be shared
    // (prefix_index.rs:98-109)
    if (shared == prompt.size() && e.session_position > shared) shared = shared == 0 ? 0 : shared - 1;
    if (shared < min_share_) continue;
    if (!best || shared >= best->second) best = std::make_pair(e.sequence_id, shared);  // last max wins
  }
  return best;
}

// ----------------------------------------------------------------------------- scheduler
Scheduler::Scheduler(DeviceModel* model, BlockPool* pool, const SessionConfig& session, const SchedulerConfig& config,
                     bool graph_decode)
    : model_(model), pool_(pool), executor_(model, pool, graph_decode), session_(session), config_(config),
      prefix_index_(config.min_prefix_share_tokens) {
  if (config.max_batch_size == 0) fail(ErrorKind::InvalidConfig, "scheduler max_batch_size must be greater than zero");
  if (config.max_prefill_chunk_tokens == 0) {
    fail(ErrorKind::InvalidConfig, "scheduler max_prefill_chunk_tokens must be greater than zero");
  }
  if (config.max_prefill_batch_tokens == 0) {
    fail(ErrorKind::InvalidConfig, "scheduler max_prefill_batch_tokens must be greater than zero");
  }
  if (config.max_consecutive_prefill_ticks == 0) {
    fail(ErrorKind::InvalidConfig, "scheduler max_consecutive_prefill_ticks must be greater than zero");
  }
  model->validate();
  model->finalize();
  if (static_cast<size_t>(model->rope_positions()) < session.max_sequence_length &&
      model->config().rotary_dims > 0) {
    fail(ErrorKind::InvalidConfig, "RoPE table shorter than the session max sequence length");
  }
}

size_t Scheduler::index_of(uint64_t id) const {
  for (size_t i = 0; i < sequences_.size(); ++i) {
    if (sequences_[i].sequence_id == id) return i;
  }
  fail(ErrorKind::Runtime, "scheduler sequence " + std::to_string(id) + " is missing");
}

const Sequence* Scheduler::sequence(uint64_t id) const {
  for (const Sequence& s : sequences_) {
    if (s.sequence_id == id) return &s;
  }
  return nullptr;
}

bool Scheduler::has_pending() const {
  for (const Sequence& s : sequences_) {
    if (s.phase != Phase::Finished) return true;
  }
  return false;
}

uint64_t Scheduler::submit(const std::vector<uint32_t>& prompt, size_t max_new_tokens,
                           std::optional<uint32_t> stop_token) {
  // scheduler.rs:204-250
  if (prompt.empty()) fail(ErrorKind::InvalidShape, "scheduler requests require at least one prompt token");
  if (prompt.size() > session_.max_sequence_length) {
    fail(ErrorKind::InvalidShape, "scheduler request prompt exceeds session max sequence length");
  }
  for (uint32_t t : prompt) {
    if (t >= static_cast<uint32_t>(model_->config().vocab_size)) {
      fail(ErrorKind::InvalidShape, "token id " + std::to_string(t) + " is out of vocabulary range " +
                                        std::to_string(model_->config().vocab_size));
    }
  }
  Sequence s;
  s.request_id = next_request_id_++;
  s.sequence_id = next_sequence_id_++;
  s.prompt = prompt;
  s.requested_max_new_tokens = max_new_tokens;
  s.max_new_tokens = std::min(max_new_tokens, session_.max_generated_tokens);
  s.stop_token = stop_token;
  s.sampler_state = sampler_state_new(session_.sampler.seed);  // Session::new (session.rs:110, 138)
  const uint64_t id = s.sequence_id;
  sequences_.push_back(std::move(s));
  state_ += 1;  // the next tick's plan may change
  block_manager_.update_shared_prefix(id, std::nullopt);
  refresh_prefix_metadata(id);
  return id;
}

std::vector<uint64_t> Scheduler::collect_prefill_ids() const {
  // scheduler.rs:271-303
  std::vector<uint64_t> ids;
  size_t total = 0;
  for (const Sequence& s : sequences_) {
    if (s.phase != Phase::Prefill) continue;
    const size_t chunk = s.next_prefill_chunk_len(config_.max_prefill_chunk_tokens);
    if (chunk == 0) continue;
    if (!ids.empty() && total + chunk > config_.max_prefill_batch_tokens) break;
    total += chunk;
    ids.push_back(s.sequence_id);
    if (ids.size() >= config_.max_batch_size || total >= config_.max_prefill_batch_tokens) break;
  }
  return ids;
}

std::vector<uint64_t> Scheduler::collect_decode_ids() const {
  // scheduler.rs:305-312
  std::vector<uint64_t> ids;
  for (const Sequence& s : sequences_) {
    if (s.phase != Phase::Decode) continue;
    if (ids.size() >= config_.max_batch_size) break;
    ids.push_back(s.sequence_id);
  }
  return ids;
}

bool Scheduler::should_schedule_decode(size_t prefill, size_t decode) const {
  // scheduler.rs:314-328
  if (decode == 0) return false;
  if (prefill == 0) return true;
  if (consecutive_prefill_ticks_ >= config_.max_consecutive_prefill_ticks) return true;
  return consecutive_prefill_ticks_ > 0 && decode == config_.max_batch_size && prefill < config_.max_batch_size;
}

std::optional<std::pair<BatchKind, std::vector<uint64_t>>> Scheduler::plan_next_tick() const {
  // scheduler.rs:253-269
  auto prefill = collect_prefill_ids();
  auto decode = collect_decode_ids();
  if (prefill.empty()) {
    if (decode.empty()) return std::nullopt;
    return std::make_pair(BatchKind::Decode, decode);
  }
  if (decode.empty()) return std::make_pair(BatchKind::Prefill, prefill);
  if (should_schedule_decode(prefill.size(), decode.size())) return std::make_pair(BatchKind::Decode, decode);
  return std::make_pair(BatchKind::Prefill, prefill);
}

std::optional<PrefixHandle> Scheduler::prefix_handle(const Sequence& s, size_t tokens) const {
  // session.rs:163-175 + kv_cache.rs:510-530: None for 0 tokens, error past the position
  if (tokens > s.position) {
    fail(ErrorKind::InvalidShape, "session prefix handle length " + std::to_string(tokens) +
                                      " exceeds committed tokens " + std::to_string(s.position));
  }
  if (tokens == 0) return std::nullopt;
  const size_t bs = static_cast<size_t>(pool_->block_size());
  PrefixHandle h;
  h.token_count = tokens;
  h.layers = model_->config().num_layers;
  h.blocks.assign(s.blocks.begin(), s.blocks.begin() + (tokens + bs - 1) / bs);
  return h;
}

void Scheduler::refresh_prefix_metadata(uint64_t id) {
  // scheduler.rs:575-588
  const Sequence& s = sequences_[index_of(id)];
  std::optional<PrefixHandle> h;
  if (s.phase != Phase::Finished) h = prefix_handle(s, s.cached_prompt_tokens());
  block_manager_.refresh_owned_prefix(id, std::move(h));
}

void Scheduler::share_blocks(Sequence& target, const Sequence& source, size_t tokens, PackedBatch* batch) {
  // The device counterpart of copy_prefix_from_session (session.rs:177-204): full blocks are
  // referenced by id; a last partially filled block is copied (copy-on-write) after the
  // source's rows of this layer are appended.
  const size_t bs = static_cast<size_t>(pool_->block_size());
  for (int32_t blk : target.blocks) pool_->decref(blk);
  target.blocks.clear();
  const size_t full = tokens / bs;
  for (size_t i = 0; i < full; ++i) {
    pool_->incref(source.blocks[i]);
    target.blocks.push_back(source.blocks[i]);
  }
  const size_t rem = tokens % bs;
  if (rem != 0) {
    const int32_t dst = pool_->allocate();
    target.blocks.push_back(dst);
    batch->copy_src.push_back(source.blocks[full]);
    batch->copy_dst.push_back(dst);
    batch->copy_count.push_back(static_cast<int32_t>(rem));
  }
}

size_t Scheduler::maybe_share_prefix(uint64_t id, PackedBatch* batch, uint64_t* source_id) {
  // scheduler.rs:353-391.  The reference rebuilds its prefix index after every sequence
  // update and again here; only this lookup reads it, so building it here, from the current
  // sequence states, gives the same matches.
  if (config_.min_prefix_share_tokens == 0) return 0;
  const size_t ti = index_of(id);
  if (sequences_[ti].cached_prompt_tokens() != 0 || sequences_[ti].phase != Phase::Prefill) return 0;
  prefix_index_.rebuild(sequences_);
  auto cand = prefix_index_.best_match(id, sequences_[ti].prompt);
  if (!cand || cand->second == 0) return 0;
  const size_t si = index_of(cand->first);
  const size_t shared = cand->second;
  *source_id = cand->first;
  Sequence& target = sequences_[ti];
  const Sequence& source = sequences_[si];
  if (!source.resident) fail(ErrorKind::Runtime, "scheduler sequence no longer retains an active session");
  if (shared > source.history.size()) fail(ErrorKind::InvalidShape, "session prefix length exceeds source token history");
  std::optional<std::pair<uint64_t, PrefixHandle>> assignment;
  if (auto h = prefix_handle(source, shared)) assignment = std::make_pair(source.sequence_id, std::move(*h));
  share_blocks(target, source, shared, batch);
  target.position = shared;
  target.history.assign(source.history.begin(), source.history.begin() + shared);
  // import_prefix_from (session.rs:188-211): reset, then the source's last sample and sampler
  // state when the whole source history is imported (every session has the same sampler);
  // either may still be produced by this tick's forward (see execute_next_tick)
  target.last_sample.reset();
  target.sampler_state = sampler_state_new(session_.sampler.seed);
  if (shared == source.position) {
    target.last_sample = source.last_sample;
    target.sampler_state = source.sampler_state;
  }
  target.record_prefill(shared);
  block_manager_.update_shared_prefix(id, std::move(assignment));
  refresh_prefix_metadata(id);
  return shared;
}

void Scheduler::append_to_batch(Sequence& s, const std::vector<uint32_t>& tokens, PackedBatch* batch) {
  // Grows the block table for positions [position, position + n) (first touch allocates, as
  // allocate_page_for_logical_block, paged_kv.rs:469-527) and packs the rows.
  const size_t bs = static_cast<size_t>(pool_->block_size());
  const size_t start = s.position;
  const size_t end = start + tokens.size();
  while (s.blocks.size() * bs < end) s.blocks.push_back(pool_->allocate());
  for (size_t i = 0; i < tokens.size(); ++i) {
    const size_t pos = start + i;
    batch->token_ids.push_back(static_cast<int32_t>(tokens[i]));
    batch->positions.push_back(static_cast<int32_t>(pos));
    batch->slot_mapping.push_back(static_cast<int64_t>(s.blocks[pos / bs]) * static_cast<int64_t>(bs) +
                                  static_cast<int64_t>(pos % bs));
  }
  batch->sequence_ids.push_back(s.sequence_id);
  batch->context_lens.push_back(static_cast<int32_t>(end));
  batch->cu_seqlens.push_back(static_cast<int32_t>(batch->token_ids.size()));
  batch->last_rows.push_back(static_cast<int32_t>(batch->token_ids.size()) - 1);
  batch->max_query_len = std::max<int32_t>(batch->max_query_len, static_cast<int32_t>(tokens.size()));
  batch->max_context_len = std::max<int32_t>(batch->max_context_len, static_cast<int32_t>(end));
}

void Scheduler::finalize_batch(PackedBatch* batch) const {
  const size_t bs = static_cast<size_t>(pool_->block_size());
  const size_t B = batch->sequence_ids.size();
  int32_t max_blocks = 1;
  for (size_t i = 0; i < B; ++i) {
    max_blocks = std::max<int32_t>(max_blocks, static_cast<int32_t>((batch->context_lens[i] + bs - 1) / bs));
  }
  batch->max_blocks = max_blocks;
  batch->block_tables.assign(B * max_blocks, 0);
  for (size_t i = 0; i < B; ++i) {
    const Sequence& s = sequences_[index_of(batch->sequence_ids[i])];
    const size_t n = (batch->context_lens[i] + bs - 1) / bs;
    for (size_t j = 0; j < n; ++j) batch->block_tables[i * max_blocks + j] = s.blocks[j];
  }
}

bool Scheduler::launch_ahead(const PackedBatch& current) {
  // The next tick as its own call would pack it (execute_next_tick's decode branch with
  // append_to_batch and finalize_batch), from the state this tick leaves: positions, phases and
  // finished sequences are settled before its forward, and blocks are taken from the top of the
  // pool's free list in row order.  Only the token ids, and a sampled session's sampler states,
  // wait for this tick's samples.
  if (executor_.in_flight() != 1) return false;
  const auto plan = plan_next_tick();
  if (!plan || plan->first != BatchKind::Decode) return false;
  const size_t bs = static_cast<size_t>(pool_->block_size());
  std::map<uint64_t, int32_t> row_of;
  for (size_t i = 0; i < current.sequence_ids.size(); ++i) row_of[current.sequence_ids[i]] = static_cast<int32_t>(i);
  PackedBatch nb;
  nb.kind = BatchKind::Decode;
  nb.cu_seqlens.push_back(0);
  std::vector<int32_t> feed;
  std::vector<std::vector<int32_t>> tables;
  size_t taken = 0;
  for (uint64_t id : plan->second) {
    const Sequence& s = sequences_[index_of(id)];
    if (s.position >= session_.max_sequence_length) continue;  // finishes with no row
    if (s.history.empty()) return false;                       // that call fails on its own
    const auto it = row_of.find(id);
    const int32_t row = it == row_of.end() ? -1 : it->second;
    if (row < 0 && !s.last_sample) return false;
    std::vector<int32_t> blocks = s.blocks;
    const size_t pos = s.position, end = pos + 1;
    while (blocks.size() * bs < end) {
      const int32_t blk = pool_->peek(taken++);
      if (blk < 0) return false;  // the pool runs out: that call reports it
      blocks.push_back(blk);
    }
    nb.token_ids.push_back(row < 0 ? static_cast<int32_t>(s.last_sample->token_id) : 0);
    nb.positions.push_back(static_cast<int32_t>(pos));
    nb.slot_mapping.push_back(static_cast<int64_t>(blocks[pos / bs]) * static_cast<int64_t>(bs) +
                              static_cast<int64_t>(pos % bs));
    nb.sequence_ids.push_back(id);
    nb.context_lens.push_back(static_cast<int32_t>(end));
    nb.cu_seqlens.push_back(static_cast<int32_t>(nb.token_ids.size()));
    nb.last_rows.push_back(static_cast<int32_t>(nb.token_ids.size()) - 1);
    nb.max_query_len = std::max<int32_t>(nb.max_query_len, 1);
    nb.max_context_len = std::max<int32_t>(nb.max_context_len, static_cast<int32_t>(end));
    tables.push_back(std::move(blocks));
    feed.push_back(row);
  }
  if (nb.sequence_ids.empty() || !executor_.can_feed(nb)) return false;
  int32_t max_blocks = 1;
  for (int32_t len : nb.context_lens) max_blocks = std::max<int32_t>(max_blocks, static_cast<int32_t>((len + bs - 1) / bs));
  nb.max_blocks = max_blocks;
  nb.block_tables.assign(nb.sequence_ids.size() * max_blocks, 0);
  for (size_t i = 0; i < tables.size(); ++i) {
    const size_t n = (static_cast<size_t>(nb.context_lens[i]) + bs - 1) / bs;
    for (size_t j = 0; j < n; ++j) nb.block_tables[i * max_blocks + j] = tables[i][j];
  }
  // states of rows fed from this tick are gathered on the device; the others are the host's
  std::vector<uint64_t> states(nb.sequence_ids.size(), 0);
  for (size_t i = 0; i < states.size(); ++i) {
    if (feed[i] < 0) states[i] = sequences_[index_of(nb.sequence_ids[i])].sampler_state;
  }
  executor_.launch(nb, session_.sampler, &states, &feed);
  ahead_.active = true;
  ahead_.state = state_;
  ahead_.batch = std::move(nb);
  ahead_.feed_rows = std::move(feed);
  ahead_.fed.clear();
  ahead_launched_ += 1;
  return true;
}

bool Scheduler::ahead_matches(const PackedBatch& b) const {
  const PackedBatch& a = ahead_.batch;
  if (a.kind != b.kind || a.sequence_ids != b.sequence_ids || a.positions != b.positions ||
      a.slot_mapping != b.slot_mapping || a.cu_seqlens != b.cu_seqlens || a.context_lens != b.context_lens ||
      a.block_tables != b.block_tables || a.max_blocks != b.max_blocks || a.last_rows != b.last_rows ||
      a.max_query_len != b.max_query_len || a.max_context_len != b.max_context_len || !b.copy_src.empty() ||
      a.token_ids.size() != b.token_ids.size() || ahead_.feed_rows.size() != b.token_ids.size()) {
    return false;
  }
  // the device fed row i with the previous tick's sample feed_rows[i]
  for (size_t i = 0; i < b.token_ids.size(); ++i) {
    const int32_t r = ahead_.feed_rows[i];
    const int32_t fed = r >= 0 ? (static_cast<size_t>(r) < ahead_.fed.size()
                                      ? static_cast<int32_t>(ahead_.fed[r].token_id) : -1)
                               : a.token_ids[i];
    if (fed != b.token_ids[i]) return false;
  }
  return true;
}

void Scheduler::drop_ahead() {
  ahead_.active = false;
  ahead_dropped_ += 1;
  executor_.discard();  // waits for it; its K/V rows sit in slots the kept ticks write again
}

std::vector<ManagedBlockId> Scheduler::release(uint64_t id) {
  // scheduler.rs:590-599: the session goes; its pool blocks are returned after the forward
  sequences_[index_of(id)].resident = false;
  return block_manager_.remove_sequence(id);
}

std::optional<TickReport> Scheduler::execute_next_tick(bool run_ahead) {
  // scheduler.rs:393-538
  const auto t0 = std::chrono::steady_clock::now();
  last_tick_ahead_ = false;
  // a call that failed may have left launched ticks behind
  if (!ahead_.active) {
    while (executor_.in_flight() > 0) executor_.discard();
  }
  // a tick enqueued ahead was planned from the state the last tick left; a submit since may
  // change this tick's plan
  if (ahead_.active && ahead_.state != state_) drop_ahead();
  auto plan = plan_next_tick();
  if (!plan) {
    if (ahead_.active) drop_ahead();
    return std::nullopt;
  }
  TickReport report;
  report.kind = plan->first;
  report.sequence_ids = plan->second;
  PackedBatch batch;
  batch.kind = plan->first;
  batch.cu_seqlens.push_back(0);
  std::vector<uint64_t> to_release;
  // sequences whose last_sample must be copied from a source after the forward
  std::vector<std::pair<uint64_t, uint64_t>> copy_sample;
  std::vector<uint64_t> computed;  // sequences of this tick already given rows, in order

  for (uint64_t id : plan->second) {
    SequenceUpdate u{};
    u.sequence_id = id;
    u.batch_kind = plan->first;
    FinishReason reason = FinishReason::None;
    if (plan->first == BatchKind::Prefill) {
      uint64_t source_id = 0;
      const size_t reused = maybe_share_prefix(id, &batch, &source_id);
      Sequence& s = sequences_[index_of(id)];
      const size_t appended = s.next_prefill_chunk_len(config_.max_prefill_chunk_tokens);
      if (reused > 0 && reused == sequences_[index_of(source_id)].position &&
          std::find(computed.begin(), computed.end(), source_id) != computed.end()) {
        // The whole history was shared from a source that ran earlier in this tick: in
        // sequential order the source had already drawn its new sample, so the copied
        // sampler state is the one after that draw; its last sample is taken after the forward
        // (when this sequence adds no rows of its own).
        if (!session_.sampler.is_greedy()) {
          Sequence& t = sequences_[index_of(id)];
          t.sampler_state = sampler_state_next(t.sampler_state);
        }
        if (appended == 0) copy_sample.emplace_back(id, source_id);
      }
      if (appended > 0) {
        // session.rs:220-244 / 381-412
        if (s.position + appended > session_.max_sequence_length) {
          fail(ErrorKind::Runtime, "cannot process tokens beyond max sequence length");
        }
        const size_t start = s.cached_prompt_tokens();
        std::vector<uint32_t> chunk(s.prompt.begin() + start, s.prompt.begin() + start + appended);
        append_to_batch(s, chunk, &batch);
        computed.push_back(id);
        s.position += appended;
        s.history.insert(s.history.end(), chunk.begin(), chunk.end());
        s.record_prefill(appended);
      }
      if (s.generation_budget_reached()) {
        reason = s.generation_budget_finish_reason();
      } else if (s.position >= session_.max_sequence_length) {
        reason = FinishReason::SequenceLength;
      }
      if (reason != FinishReason::None) s.finish(reason);
      u.request_id = s.request_id;
      u.reused_prompt_tokens = reused;
      u.appended_prompt_tokens = appended;
      u.has_token = false;
      u.phase = s.phase;
    } else {
      Sequence& s = sequences_[index_of(id)];
      if (s.position >= session_.max_sequence_length) {
        reason = FinishReason::SequenceLength;
        s.finish(reason);
        u.has_token = false;
      } else {
        // step_reference (session.rs:246-262): feed the last sample, keep it as the result
        if (s.history.empty()) fail(ErrorKind::Runtime, "step_reference requires at least one prefetched token");
        if (!s.last_sample) fail(ErrorKind::Runtime, "step_reference requires a sampled token from a prefetched token");
        const TokenSample fed = *s.last_sample;
        append_to_batch(s, {fed.token_id}, &batch);
        s.position += 1;
        s.history.push_back(fed.token_id);
        s.record_generated_token(fed.token_id);
        if (s.stop_token && *s.stop_token == fed.token_id) {
          reason = FinishReason::StopToken;
        } else if (s.generation_budget_reached()) {
          reason = s.generation_budget_finish_reason();
        } else if (s.position >= session_.max_sequence_length) {
          reason = FinishReason::SequenceLength;
        }
        if (reason != FinishReason::None) s.finish(reason);
        u.has_token = true;
        u.generated = fed;
      }
      u.request_id = s.request_id;
      u.reused_prompt_tokens = 0;
      u.appended_prompt_tokens = 0;
      u.phase = s.phase;
    }
    u.finish_reason = reason;
    if (reason != FinishReason::None) {
      u.released_prefix_blocks = release(id);
      to_release.push_back(id);
    }
    refresh_prefix_metadata(id);
    report.updates.push_back(std::move(u));
  }
  consecutive_prefill_ticks_ = plan->first == BatchKind::Prefill ? consecutive_prefill_ticks_ + 1 : 0;

  finalize_batch(&batch);
  const double sched_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
  double enqueue_s = 0.0, wait_s = 0.0;
  bool in_flight = false;  // this tick is the one enqueued ahead by the last call
  if (ahead_.active) {
    if (ahead_matches(batch)) {
      in_flight = true;
      ahead_.active = false;
      ahead_kept_ += 1;
      last_tick_ahead_ = true;
    } else {
      drop_ahead();
    }
  }
  const bool work = !batch.sequence_ids.empty() || !batch.copy_src.empty();
  std::vector<uint64_t> states(batch.sequence_ids.size());
  for (size_t i = 0; i < states.size(); ++i) states[i] = sequences_[index_of(batch.sequence_ids[i])].sampler_state;
  const auto t_enqueue = std::chrono::steady_clock::now();
  if (work && !in_flight) executor_.launch(batch, session_.sampler, &states);
  // The blocks of finished sequences go back to the pool now (the reference returns them after
  // the forward): every later use of them is enqueued behind this tick.
  for (uint64_t id : to_release) {
    Sequence& s = sequences_[index_of(id)];
    for (int32_t blk : s.blocks) pool_->decref(blk);
    s.blocks.clear();
  }
  if (run_ahead && work && copy_sample.empty()) launch_ahead(batch);
  enqueue_s = std::chrono::duration<double>(std::chrono::steady_clock::now() - t_enqueue).count();
  if (work) {
    std::vector<TokenSample> samples = executor_.collect(&states);
    wait_s = executor_.last_wait_seconds();
    for (size_t i = 0; i < batch.sequence_ids.size(); ++i) {
      Sequence& s = sequences_[index_of(batch.sequence_ids[i])];
      s.last_sample = samples[i];
      s.sampler_state = states[i];
    }
    if (ahead_.active) ahead_.fed = std::move(samples);
  }
  for (auto& [target, source] : copy_sample) {
    Sequence& t = sequences_[index_of(target)];
    const Sequence& src = sequences_[index_of(source)];
    t.last_sample = src.last_sample;
    t.sampler_state = src.sampler_state;
  }
  last_batch_ = std::move(batch);
  tick_profile_ = {sched_s, enqueue_s, wait_s,
                   std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count()};
  return report;
}

}  // namespace fr
