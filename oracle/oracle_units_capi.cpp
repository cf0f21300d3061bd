// C entry points that expose the oracle's runtime units one at a time — prefix index, prefix
// block manager, sequence state, KV cache, session generation and scheduler planning — so the
// reference's own unit tests (runtime/{prefix_index,block_manager,sequence,kv_cache,session,
// scheduler}.rs #[cfg(test)] modules) can be run against them.  TEST INFRASTRUCTURE ONLY (see
// oracle.h).
//
// Prefix handles cross this boundary flattened: header {token_count, page_size, layers},
// counts[layers] entries per layer, then entries[sum(counts)][4] = {logical_block_index,
// block_id, start_position, token_count} (runtime/paged_kv.rs:19-128).  Released block lists are
// rows {owner_sequence_id, layer_index, block_id} (block_manager.rs:7-33).
#include <cstring>
#include <memory>
#include <string>

#include "oracle_handles.h"

using namespace orc;

extern "C" const char* orc_runtime_last_error(void);

namespace {
thread_local std::string g_err;
template <typename F>
int32_t guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const OracleError& e) {
    g_err = e.message;
    return static_cast<int32_t>(e.kind) + 1;
  } catch (const std::exception& e) {
    g_err = e.what();
    return static_cast<int32_t>(ErrorKind::Runtime) + 1;
  }
}

PrefixHandle decode_handle(int64_t token_count, int64_t page_size, int64_t layers, const int64_t* counts,
                           const int64_t* entries) {
  PrefixHandle h;
  h.token_count = static_cast<size_t>(token_count);
  h.page_size = static_cast<size_t>(page_size);
  h.layer_block_tables.resize(static_cast<size_t>(layers));
  size_t k = 0;
  for (int64_t l = 0; l < layers; ++l) {
    for (int64_t i = 0; i < counts[l]; ++i, ++k) {
      const int64_t* e = entries + 4 * k;
      h.layer_block_tables[l].push_back(KvBlockTableEntry{static_cast<size_t>(e[0]), static_cast<size_t>(e[1]),
                                                          static_cast<size_t>(e[2]), static_cast<size_t>(e[3])});
    }
  }
  return h;
}

// Writes a handle in the flattened form; `cap` bounds the entries written.
void encode_handle(const PrefixHandle& h, int64_t* header, int64_t* counts, int64_t layers_cap, int64_t* entries,
                   int64_t cap) {
  header[0] = static_cast<int64_t>(h.token_count);
  header[1] = static_cast<int64_t>(h.page_size);
  header[2] = static_cast<int64_t>(h.layer_block_tables.size());
  if (static_cast<int64_t>(h.layer_block_tables.size()) > layers_cap) fail(ErrorKind::InvalidShape, "layer capacity");
  int64_t k = 0;
  for (size_t l = 0; l < h.layer_block_tables.size(); ++l) {
    counts[l] = static_cast<int64_t>(h.layer_block_tables[l].size());
    for (const auto& e : h.layer_block_tables[l]) {
      if (k >= cap) fail(ErrorKind::InvalidShape, "entry capacity");
      int64_t* o = entries + 4 * k++;
      o[0] = static_cast<int64_t>(e.logical_block_index);
      o[1] = static_cast<int64_t>(e.block_id);
      o[2] = static_cast<int64_t>(e.start_position);
      o[3] = static_cast<int64_t>(e.token_count);
    }
  }
}

void encode_released(const std::vector<ManagedBlockId>& r, int64_t* out, int64_t cap, int64_t* n_out) {
  if (static_cast<int64_t>(r.size()) > cap) fail(ErrorKind::InvalidShape, "released capacity");
  for (size_t i = 0; i < r.size(); ++i) {
    out[3 * i] = static_cast<int64_t>(r[i].owner_sequence_id);
    out[3 * i + 1] = static_cast<int64_t>(r[i].layer_index);
    out[3 * i + 2] = static_cast<int64_t>(r[i].block_id);
  }
  *n_out = static_cast<int64_t>(r.size());
}
}  // namespace

extern "C" {

const char* orc_units_last_error(void) { return g_err.c_str(); }

// ---------------------------------------------------------------- prefix index (prefix_index.rs:24-113)
void* orc_prefix_index_create(int64_t min_share) { return new PrefixIndex(static_cast<size_t>(min_share)); }
void orc_prefix_index_destroy(void* p) { delete static_cast<PrefixIndex*>(p); }
int32_t orc_prefix_index_upsert(void* p, uint64_t seq, const uint32_t* toks, int64_t n, int64_t cached,
                                int64_t position) {
  return guard([&] {
    static_cast<PrefixIndex*>(p)->upsert(PrefixIndexEntry{seq, std::vector<uint32_t>(toks, toks + n),
                                                          static_cast<size_t>(cached), static_cast<size_t>(position)});
  });
}
int32_t orc_prefix_index_best_match(void* p, uint64_t target, const uint32_t* toks, int64_t n, int32_t* found,
                                    uint64_t* seq, int64_t* shared) {
  return guard([&] {
    auto m = static_cast<PrefixIndex*>(p)->best_match(target, std::vector<uint32_t>(toks, toks + n));
    *found = m ? 1 : 0;
    if (m) {
      *seq = m->first;
      *shared = static_cast<int64_t>(m->second);
    }
  });
}

// ---------------------------------------------------------------- block manager (block_manager.rs:58-172)
void* orc_block_manager_create(void) { return new PrefixBlockManager(); }
void orc_block_manager_destroy(void* p) { delete static_cast<PrefixBlockManager*>(p); }
int32_t orc_block_manager_update_owned(void* p, uint64_t seq, int32_t has, int64_t token_count, int64_t page_size,
                                       int64_t layers, const int64_t* counts, const int64_t* entries, int64_t* released,
                                       int64_t cap, int64_t* n_out) {
  return guard([&] {
    std::optional<PrefixHandle> h;
    if (has) h = decode_handle(token_count, page_size, layers, counts, entries);
    encode_released(static_cast<PrefixBlockManager*>(p)->update_owned_prefix(seq, std::move(h)), released, cap,
                    n_out);
  });
}
int32_t orc_block_manager_update_shared(void* p, uint64_t seq, int32_t has, uint64_t source, int64_t token_count,
                                        int64_t page_size, int64_t layers, const int64_t* counts,
                                        const int64_t* entries, int64_t* released, int64_t cap, int64_t* n_out) {
  return guard([&] {
    std::optional<SharedPrefixAssignment> a;
    if (has) a = SharedPrefixAssignment{source, decode_handle(token_count, page_size, layers, counts, entries)};
    encode_released(static_cast<PrefixBlockManager*>(p)->update_shared_prefix(seq, std::move(a)), released, cap,
                    n_out);
  });
}
int32_t orc_block_manager_remove(void* p, uint64_t seq, int64_t* released, int64_t cap, int64_t* n_out) {
  return guard([&] { encode_released(static_cast<PrefixBlockManager*>(p)->remove_sequence(seq), released, cap, n_out); });
}
int64_t orc_block_manager_ref_count(void* p, uint64_t owner, int64_t layer, int64_t block) {
  return static_cast<int64_t>(static_cast<PrefixBlockManager*>(p)->block_ref_count(
      ManagedBlockId{owner, static_cast<size_t>(layer), static_cast<size_t>(block)}));
}
int64_t orc_block_manager_tracked(void* p) {
  return static_cast<int64_t>(static_cast<PrefixBlockManager*>(p)->tracked_block_count());
}
// flags: bit 0 = has an owned prefix, bit 1 = has a shared prefix; *source = the shared prefix's source
int32_t orc_block_manager_prefixes(void* p, uint64_t seq, int32_t* flags, uint64_t* source) {
  return guard([&] {
    const auto* m = static_cast<PrefixBlockManager*>(p);
    const SharedPrefixAssignment* sh = m->shared_prefix(seq);
    *flags = (m->owned_prefix(seq) ? 1 : 0) | (sh ? 2 : 0);
    *source = sh ? sh->source_sequence_id : 0;
  });
}

// ---------------------------------------------------------------- sequence state (sequence.rs:43-237)
void* orc_sequence_create(uint64_t request, uint64_t seq, const uint32_t* prompt, int64_t n, int64_t requested,
                          int64_t budget, int64_t stop) {
  auto* s = new SequenceState();
  s->request_id = request;
  s->sequence_id = seq;
  s->prompt.assign(prompt, prompt + n);
  s->requested_max_new_tokens = static_cast<size_t>(requested);
  s->max_new_tokens = static_cast<size_t>(budget);
  if (stop >= 0) s->stop_token = static_cast<uint32_t>(stop);
  return s;
}
void orc_sequence_destroy(void* p) { delete static_cast<SequenceState*>(p); }
void orc_sequence_record_prefill(void* p, int64_t appended) {
  static_cast<SequenceState*>(p)->record_prefill(static_cast<size_t>(appended));
}
void orc_sequence_record_generated(void* p, uint32_t token) { static_cast<SequenceState*>(p)->record_generated_token(token); }
void orc_sequence_finish(void* p, int32_t reason) {
  static_cast<SequenceState*>(p)->finish(static_cast<FinishReason>(reason));
}
// fields: request, sequence, prompt_len, generated_len, cached, cached_prompt, pending, requested_max,
// max_new, stop (-1 = none), phase, finish (-1 = none), finished, budget_reached,
// budget_finish_reason, total_tokens
void orc_sequence_query(void* p, int64_t* f) {
  const auto* s = static_cast<SequenceState*>(p);
  f[0] = static_cast<int64_t>(s->request_id);
  f[1] = static_cast<int64_t>(s->sequence_id);
  f[2] = static_cast<int64_t>(s->prompt.size());
  f[3] = static_cast<int64_t>(s->generated.size());
  f[4] = static_cast<int64_t>(s->cached_tokens);
  f[5] = static_cast<int64_t>(s->cached_prompt_tokens());
  f[6] = static_cast<int64_t>(s->pending_prompt_tokens());
  f[7] = static_cast<int64_t>(s->requested_max_new_tokens);
  f[8] = static_cast<int64_t>(s->max_new_tokens);
  f[9] = s->stop_token ? static_cast<int64_t>(*s->stop_token) : -1;
  f[10] = static_cast<int64_t>(s->phase);
  f[11] = static_cast<int64_t>(s->finish_reason);
  f[12] = s->is_finished() ? 1 : 0;
  f[13] = s->generation_budget_reached() ? 1 : 0;
  f[14] = static_cast<int64_t>(s->generation_budget_finish_reason());
  f[15] = static_cast<int64_t>(s->total_tokens());
}
int64_t orc_sequence_generated(void* p, uint32_t* out, int64_t cap) {
  const auto* s = static_cast<SequenceState*>(p);
  int64_t n = std::min<int64_t>(cap, static_cast<int64_t>(s->generated.size()));
  std::memcpy(out, s->generated.data(), static_cast<size_t>(n) * sizeof(uint32_t));
  return static_cast<int64_t>(s->generated.size());
}
int64_t orc_sequence_next_chunk(void* p, int64_t max_chunk, uint32_t* out, int64_t cap) {
  auto c = static_cast<SequenceState*>(p)->next_prefill_chunk(static_cast<size_t>(max_chunk));
  int64_t n = std::min<int64_t>(cap, static_cast<int64_t>(c.size()));
  std::memcpy(out, c.data(), static_cast<size_t>(n) * sizeof(uint32_t));
  return static_cast<int64_t>(c.size());
}

// ---------------------------------------------------------------- KV cache (kv_cache.rs:359-597)
void* orc_kvcache_create(int64_t layers, int64_t hkv, int64_t d, int64_t max_seq, int64_t page_size) {
  KvCache* kv = nullptr;
  guard([&] {
    KvCacheConfig c;
    c.num_layers = static_cast<size_t>(layers);
    c.num_kv_heads = static_cast<size_t>(hkv);
    c.head_dim = static_cast<size_t>(d);
    c.max_sequence_length = static_cast<size_t>(max_seq);
    kv = new KvCache(page_size == 0 ? KvCache::contiguous(c) : KvCache::paged(c, static_cast<size_t>(page_size)));
  });
  return kv;
}
void orc_kvcache_destroy(void* p) { delete static_cast<KvCache*>(p); }
int32_t orc_kvcache_reserve_slot(void* p, int64_t* pos) {
  return guard([&] { *pos = static_cast<int64_t>(static_cast<KvCache*>(p)->reserve_slot()); });
}
int32_t orc_kvcache_advance(void* p, int64_t n) {
  return guard([&] { static_cast<KvCache*>(p)->advance(static_cast<size_t>(n)); });
}
int32_t orc_kvcache_write(void* p, int64_t layer, int64_t pos, const float* k, const float* v) {
  return guard([&] { static_cast<KvCache*>(p)->write(static_cast<size_t>(layer), static_cast<size_t>(pos), k, v); });
}
int32_t orc_kvcache_write_uncommitted(void* p, int64_t layer, int64_t pos, const float* k, const float* v) {
  return guard([&] {
    static_cast<KvCache*>(p)->write_uncommitted(static_cast<size_t>(layer), static_cast<size_t>(pos), k, v);
  });
}
int32_t orc_kvcache_write_sequence_uncommitted(void* p, int64_t layer, int64_t start, int64_t n, const float* k,
                                               const float* v) {
  return guard([&] {
    static_cast<KvCache*>(p)->write_sequence_uncommitted(static_cast<size_t>(layer), static_cast<size_t>(start),
                                                         static_cast<size_t>(n), k, v);
  });
}
int32_t orc_kvcache_read_prefix(void* p, int64_t layer, int64_t len, float* k, float* v) {
  return guard([&] {
    std::vector<float> kk, vv;
    static_cast<KvCache*>(p)->read_prefix(static_cast<size_t>(layer), static_cast<size_t>(len), &kk, &vv);
    std::memcpy(k, kk.data(), kk.size() * sizeof(float));
    std::memcpy(v, vv.data(), vv.size() * sizeof(float));
  });
}
// out: used, remaining, paged, layers, elements of one layer's key tensor
void orc_kvcache_counts(void* p, int64_t* out) {
  const auto* kv = static_cast<KvCache*>(p);
  const KvCacheConfig& c = kv->config();
  out[0] = static_cast<int64_t>(kv->used_tokens());
  out[1] = static_cast<int64_t>(kv->remaining_tokens());
  out[2] = kv->is_paged() ? 1 : 0;
  out[3] = static_cast<int64_t>(c.num_layers);
  out[4] = static_cast<int64_t>(c.max_sequence_length * c.num_kv_heads * c.head_dim);
}
void orc_kvcache_reset(void* p) { static_cast<KvCache*>(p)->reset(); }
int32_t orc_kvcache_prefix_handle(void* p, int64_t tokens, int32_t* has, int64_t* header, int64_t* counts,
                                  int64_t layers_cap, int64_t* entries, int64_t cap) {
  return guard([&] {
    auto h = static_cast<KvCache*>(p)->prefix_handle(static_cast<size_t>(tokens));
    *has = h ? 1 : 0;
    if (h) encode_handle(*h, header, counts, layers_cap, entries, cap);
  });
}
int32_t orc_kvcache_copy_prefix_from(void* dst, void* src, int64_t tokens) {
  return guard([&] { static_cast<KvCache*>(dst)->copy_prefix_from(*static_cast<KvCache*>(src), static_cast<size_t>(tokens)); });
}

// ---------------------------------------------------------------- session (session.rs:92-413)
int32_t orc_session_history(void* p, uint32_t* out, int64_t cap, int64_t* n_out) {
  return guard([&] {
    const auto& h = static_cast<OrcSession*>(p)->session->token_history();
    if (static_cast<int64_t>(h.size()) > cap) fail(ErrorKind::InvalidShape, "history capacity");
    std::memcpy(out, h.data(), h.size() * sizeof(uint32_t));
    *n_out = static_cast<int64_t>(h.size());
  });
}
// out: used tokens, paged
void orc_session_kv_counts(void* p, int64_t* out) {
  const KvCache& kv = static_cast<OrcSession*>(p)->session->kv_cache();
  out[0] = static_cast<int64_t>(kv.used_tokens());
  out[1] = kv.is_paged() ? 1 : 0;
}
int32_t orc_session_prefix_handle(void* p, int64_t tokens, int32_t* has, int64_t* header, int64_t* counts,
                                  int64_t layers_cap, int64_t* entries, int64_t cap) {
  return guard([&] {
    auto h = static_cast<OrcSession*>(p)->session->prefix_handle(static_cast<size_t>(tokens));
    *has = h ? 1 : 0;
    if (h) encode_handle(*h, header, counts, layers_cap, entries, cap);
  });
}
int32_t orc_session_generate(void* p, const uint32_t* prompt, int64_t n, int64_t max_new, int64_t stop,
                             uint32_t* tokens, float* probs, int64_t cap, int64_t* n_out, int32_t* finish) {
  return guard([&] {
    std::optional<uint32_t> st;
    if (stop >= 0) st = static_cast<uint32_t>(stop);
    FinishReason reason = FinishReason::None;
    auto out = static_cast<OrcSession*>(p)->session->generate_from_tokens(std::vector<uint32_t>(prompt, prompt + n),
                                                                          static_cast<size_t>(max_new), st, &reason);
    if (static_cast<int64_t>(out.size()) > cap) fail(ErrorKind::InvalidShape, "generation capacity");
    for (size_t i = 0; i < out.size(); ++i) {
      tokens[i] = out[i].token_id;
      probs[i] = out[i].probability;
    }
    *n_out = static_cast<int64_t>(out.size());
    *finish = static_cast<int32_t>(reason);
  });
}

// ---------------------------------------------------------------- scheduler (scheduler.rs:109-648)
int32_t orc_scheduler_plan(void* p, int32_t* has, int32_t* kind, uint64_t* ids, int64_t cap, int64_t* n_out) {
  return guard([&] {
    auto t = static_cast<OrcScheduler*>(p)->sched->plan_next_tick();
    *has = t ? 1 : 0;
    *n_out = 0;
    if (!t) return;
    if (static_cast<int64_t>(t->sequence_ids.size()) > cap) fail(ErrorKind::InvalidShape, "tick capacity");
    *kind = static_cast<int32_t>(t->kind);
    for (size_t i = 0; i < t->sequence_ids.size(); ++i) ids[i] = t->sequence_ids[i];
    *n_out = static_cast<int64_t>(t->sequence_ids.size());
  });
}
// out: phase, finish reason (-1 = none), cached tokens, generated count, has session
int32_t orc_scheduler_sequence(void* p, uint64_t seq, int64_t* out) {
  return guard([&] {
    const auto* sched = static_cast<OrcScheduler*>(p)->sched.get();
    const SequenceState* s = sched->sequence_state(seq);
    if (!s) fail(ErrorKind::Runtime, "scheduler sequence " + std::to_string(seq) + " is missing");
    out[0] = static_cast<int64_t>(s->phase);
    out[1] = static_cast<int64_t>(s->finish_reason);
    out[2] = static_cast<int64_t>(s->cached_tokens);
    out[3] = static_cast<int64_t>(s->generated.size());
    out[4] = sched->session(seq) ? 1 : 0;
  });
}
int64_t orc_scheduler_resident_sessions(void* p) {
  return static_cast<int64_t>(static_cast<OrcScheduler*>(p)->sched->resident_session_count());
}
int32_t orc_scheduler_shared_prefix(void* p, uint64_t seq, int32_t* has, uint64_t* source) {
  return guard([&] {
    const SharedPrefixAssignment* a = static_cast<OrcScheduler*>(p)->sched->block_manager().shared_prefix(seq);
    *has = a ? 1 : 0;
    *source = a ? a->source_sequence_id : 0;
  });
}

}  // extern "C"
