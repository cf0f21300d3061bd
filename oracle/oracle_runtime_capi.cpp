// C entry points for the oracle's runtime restatement (paged KV, model forward, session,
// scheduler) and the paged-decode CPU baseline — TEST INFRASTRUCTURE ONLY (see oracle.h).
#include <algorithm>
#include <cstring>
#include <memory>
#include <string>

#include "oracle_handles.h"

using namespace orc;

extern "C" const char* orc_last_error(void);
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
}  // namespace

extern "C" {

const char* orc_runtime_last_error(void) { return g_err.c_str(); }

// ---------------------------------------------------------------- paged KV storage
void* orc_paged_kv_create(int64_t layers, int64_t hkv, int64_t d, int64_t max_seq, int64_t page) {
  void* out = nullptr;
  guard([&] {
    KvCacheConfig c{static_cast<size_t>(layers), static_cast<size_t>(hkv), static_cast<size_t>(d),
                    static_cast<size_t>(max_seq)};
    out = new PagedKvCacheStorage(c, static_cast<size_t>(page));
  });
  return out;
}
void orc_paged_kv_destroy(void* s) { delete static_cast<PagedKvCacheStorage*>(s); }
int32_t orc_paged_kv_write_sequence(void* s, int64_t layer, int64_t start, int64_t n,
                                    const float* k, const float* v) {
  return guard([&] { static_cast<PagedKvCacheStorage*>(s)->write_sequence(layer, start, n, k, v); });
}
int32_t orc_paged_kv_write_slot(void* s, int64_t layer, int64_t pos, const float* k, const float* v) {
  return guard([&] { static_cast<PagedKvCacheStorage*>(s)->write_slot(layer, pos, k, v); });
}
int32_t orc_paged_kv_read_prefix(void* s, int64_t layer, int64_t len, float* k, float* v) {
  return guard([&] {
    std::vector<float> kk, vv;
    static_cast<PagedKvCacheStorage*>(s)->read_prefix(layer, len, &kk, &vv);
    std::memcpy(k, kk.data(), kk.size() * sizeof(float));
    std::memcpy(v, vv.data(), vv.size() * sizeof(float));
  });
}
// entries: int64[n_out * 4] = (logical_block_index, block_id, start_position, token_count)
int32_t orc_paged_kv_block_table(void* s, int64_t layer, int64_t tokens, int64_t* entries,
                                 int64_t capacity, int64_t* n_out) {
  return guard([&] {
    auto t = static_cast<PagedKvCacheStorage*>(s)->block_table(layer, tokens);
    if (static_cast<int64_t>(t.size()) > capacity) fail(ErrorKind::InvalidShape, "block table capacity too small");
    for (size_t i = 0; i < t.size(); ++i) {
      entries[4 * i + 0] = t[i].logical_block_index;
      entries[4 * i + 1] = t[i].block_id;
      entries[4 * i + 2] = t[i].start_position;
      entries[4 * i + 3] = t[i].token_count;
    }
    *n_out = static_cast<int64_t>(t.size());
  });
}
// infos: int64[pages * 3] = (page_id, start_position, token_count)
int32_t orc_paged_kv_page_infos(void* s, int64_t layer, int64_t* infos, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    auto t = static_cast<PagedKvCacheStorage*>(s)->page_infos(layer);
    if (static_cast<int64_t>(t.size()) > capacity) fail(ErrorKind::InvalidShape, "page info capacity too small");
    for (size_t i = 0; i < t.size(); ++i) {
      infos[3 * i + 0] = t[i].page_id;
      infos[3 * i + 1] = t[i].start_position;
      infos[3 * i + 2] = t[i].token_count;
    }
    *n_out = static_cast<int64_t>(t.size());
  });
}
int64_t orc_paged_kv_allocated_pages(void* s, int64_t layer) {
  int64_t n = -1;
  guard([&] { n = static_cast<PagedKvCacheStorage*>(s)->allocated_page_count(layer); });
  return n;
}
int64_t orc_paged_kv_free_pages(void* s, int64_t layer) {
  int64_t n = -1;
  guard([&] { n = static_cast<PagedKvCacheStorage*>(s)->free_page_count(layer); });
  return n;
}
void orc_paged_kv_reset(void* s) { static_cast<PagedKvCacheStorage*>(s)->reset(); }
int32_t orc_paged_kv_import_prefix(void* dst, const void* src, int64_t tokens) {
  return guard([&] {
    const auto* source = static_cast<const PagedKvCacheStorage*>(src);
    PrefixHandle h = source->capture_prefix_handle(tokens);
    static_cast<PagedKvCacheStorage*>(dst)->import_prefix_from(*source, h);
  });
}

// ---------------------------------------------------------------- model

void* orc_model_create(int64_t hidden, int64_t intermediate, int64_t layers, int64_t heads,
                       int64_t kv_heads, int64_t vocab, int64_t max_pos, float eps, float theta,
                       int64_t rotary_dims, int32_t tie) {
  OrcModel* m = nullptr;
  guard([&] {
    auto model = std::make_shared<Model>();
    ModelConfig& c = model->config;
    c.hidden_size = hidden;
    c.intermediate_size = intermediate;
    c.num_layers = layers;
    c.num_attention_heads = heads;
    c.num_key_value_heads = kv_heads;
    c.vocab_size = vocab;
    c.max_position_embeddings = max_pos;
    c.rms_norm_eps = eps;
    c.rope_theta = theta;
    c.rotary_dims = rotary_dims;
    c.tie_word_embeddings = tie != 0;
    model->validate();
    model->layers.resize(layers);
    m = new OrcModel{model};
  });
  return m;
}
void orc_model_destroy(void* m) { delete static_cast<OrcModel*>(m); }
int32_t orc_model_set_weight(void* m, const char* name, const float* data, int64_t count) {
  return guard([&] { static_cast<OrcModel*>(m)->model->set_weight(name, data, count); });
}
int32_t orc_model_forward_logits(void* m, const uint32_t* ids, int64_t n, float* logits) {
  return guard([&] {
    std::vector<uint32_t> v(ids, ids + n);
    auto out = decoder_model_forward(*static_cast<OrcModel*>(m)->model, v);
    std::memcpy(logits, out.data(), out.size() * sizeof(float));
  });
}

// ---------------------------------------------------------------- session
void* orc_session_create(void* m, int64_t max_seq, int64_t max_gen, int64_t page_size) {
  OrcSession* s = nullptr;
  guard([&] {
    SessionConfig sc;
    sc.max_sequence_length = max_seq;
    sc.max_generated_tokens = max_gen;
    sc.page_size = page_size;
    s = new OrcSession{std::make_unique<Session>(static_cast<OrcModel*>(m)->model, sc)};
  });
  return s;
}
void orc_session_destroy(void* s) { delete static_cast<OrcSession*>(s); }
int32_t orc_session_set_sampler(void* s, float temperature, int64_t top_k, float top_p, uint64_t seed) {
  return guard([&] {
    SamplerConfig c;
    c.temperature = temperature;
    c.top_k = static_cast<size_t>(top_k);
    c.top_p = top_p;
    c.seed = seed;
    static_cast<OrcSession*>(s)->session->set_sampler(c);
  });
}
int32_t orc_session_sampler_state(void* s, uint64_t* out) {
  return guard([&] { *out = static_cast<OrcSession*>(s)->session->sampler_state(); });
}
int32_t orc_session_prefill(void* s, const uint32_t* ids, int64_t n) {
  return guard([&] { static_cast<OrcSession*>(s)->session->prefill_tokens(std::vector<uint32_t>(ids, ids + n)); });
}
int32_t orc_session_step(void* s, uint32_t* token, float* prob) {
  return guard([&] {
    TokenSample t = static_cast<OrcSession*>(s)->session->step_reference();
    *token = t.token_id;
    *prob = t.probability;
  });
}
int32_t orc_session_last_sample(void* s, uint32_t* token, float* prob) {
  return guard([&] {
    auto t = static_cast<OrcSession*>(s)->session->last_sample();
    if (!t) fail(ErrorKind::Runtime, "session has no sample yet");
    *token = t->token_id;
    *prob = t->probability;
  });
}
int32_t orc_session_last_hidden(void* s, float* out) {
  return guard([&] {
    auto h = static_cast<OrcSession*>(s)->session->last_hidden();
    std::memcpy(out, h.data(), h.size() * sizeof(float));
  });
}
int64_t orc_session_position(void* s) { return static_cast<OrcSession*>(s)->session->position(); }
int32_t orc_session_copy_prefix(void* dst, void* src, int64_t tokens) {
  return guard([&] {
    static_cast<OrcSession*>(dst)->session->copy_prefix_from_session(*static_cast<OrcSession*>(src)->session, tokens);
  });
}
int32_t orc_session_read_prefix(void* s, int64_t layer, int64_t len, float* k, float* v) {
  return guard([&] {
    std::vector<float> kk, vv;
    static_cast<OrcSession*>(s)->session->kv_cache().read_prefix(layer, len, &kk, &vv);
    std::memcpy(k, kk.data(), kk.size() * sizeof(float));
    std::memcpy(v, vv.data(), vv.size() * sizeof(float));
  });
}

// ---------------------------------------------------------------- scheduler
void* orc_scheduler_create(void* m, int64_t max_seq, int64_t max_gen, int64_t page_size,
                           int64_t max_batch, int64_t max_chunk, int64_t max_batch_tokens,
                           int64_t max_consecutive_prefill, int64_t min_share) {
  OrcScheduler* s = nullptr;
  guard([&] {
    SessionConfig sc;
    sc.max_sequence_length = max_seq;
    sc.max_generated_tokens = max_gen;
    sc.page_size = page_size;
    SchedulerConfig c;
    c.max_batch_size = max_batch;
    c.max_prefill_chunk_tokens = max_chunk;
    c.max_prefill_batch_tokens = max_batch_tokens;
    c.max_consecutive_prefill_ticks = max_consecutive_prefill;
    c.min_prefix_share_tokens = min_share;
    auto o = std::make_unique<OrcScheduler>();
    o->sched = std::make_unique<ReferenceScheduler>(static_cast<OrcModel*>(m)->model, sc, c);
    s = o.release();
  });
  return s;
}
void orc_scheduler_destroy(void* s) { delete static_cast<OrcScheduler*>(s); }
int32_t orc_scheduler_set_sampler(void* s, float temperature, int64_t top_k, float top_p, uint64_t seed) {
  return guard([&] {
    SamplerConfig c;
    c.temperature = temperature;
    c.top_k = static_cast<size_t>(top_k);
    c.top_p = top_p;
    c.seed = seed;
    static_cast<OrcScheduler*>(s)->sched->set_sampler(c);
  });
}
int32_t orc_scheduler_submit(void* s, const uint32_t* ids, int64_t n, int64_t max_new, int64_t stop,
                             uint64_t* seq_out) {
  return guard([&] {
    std::optional<uint32_t> st;
    if (stop >= 0) st = static_cast<uint32_t>(stop);
    *seq_out = static_cast<OrcScheduler*>(s)->sched->submit(std::vector<uint32_t>(ids, ids + n), max_new, st);
  });
}
// Returns 1 in *executed when a tick ran, 0 when nothing was pending.
int32_t orc_scheduler_execute_next_tick(void* s, int32_t* executed) {
  return guard([&] {
    auto* o = static_cast<OrcScheduler*>(s);
    o->last = o->sched->execute_next_tick();
    *executed = o->last ? 1 : 0;
    if (o->last && o->packer) o->packed = o->packer->pack(*o->last);
  });
}
// Attaches a global page packer (pool of num_pages pages of page_size) that packs every
// following tick.
int32_t orc_scheduler_attach_packer(void* s, int64_t num_pages, int64_t page_size) {
  return guard([&] {
    static_cast<OrcScheduler*>(s)->packer = std::make_unique<GlobalPagePacker>(num_pages, page_size);
  });
}
// sizes: [T, B, max_blocks, copies, kind]
int32_t orc_scheduler_packed_sizes(void* s, int64_t* sizes) {
  return guard([&] {
    const PackedTick& t = static_cast<OrcScheduler*>(s)->packed;
    size_t mb = 1;
    for (const auto& r : t.block_tables) mb = std::max(mb, r.size());
    sizes[0] = static_cast<int64_t>(t.positions.size());
    sizes[1] = static_cast<int64_t>(t.sequence_ids.size());
    sizes[2] = static_cast<int64_t>(mb);
    sizes[3] = static_cast<int64_t>(t.copy_src.size());
    sizes[4] = t.kind;
  });
}
// block_tables is [B, max_blocks], zero padded.
int32_t orc_scheduler_packed(void* s, int32_t* positions, int64_t* slots, int32_t* cu, int32_t* ctx_lens,
                             int32_t* block_tables, int64_t max_blocks, int32_t* copy_src, int32_t* copy_dst,
                             int32_t* copy_count, uint64_t* seq_ids) {
  return guard([&] {
    const PackedTick& t = static_cast<OrcScheduler*>(s)->packed;
    std::copy(t.positions.begin(), t.positions.end(), positions);
    std::copy(t.slot_mapping.begin(), t.slot_mapping.end(), slots);
    std::copy(t.cu_seqlens.begin(), t.cu_seqlens.end(), cu);
    std::copy(t.context_lens.begin(), t.context_lens.end(), ctx_lens);
    for (size_t b = 0; b < t.block_tables.size(); ++b) {
      for (int64_t j = 0; j < max_blocks; ++j) {
        block_tables[b * max_blocks + j] = j < static_cast<int64_t>(t.block_tables[b].size()) ? t.block_tables[b][j] : 0;
      }
    }
    std::copy(t.copy_src.begin(), t.copy_src.end(), copy_src);
    std::copy(t.copy_dst.begin(), t.copy_dst.end(), copy_dst);
    std::copy(t.copy_count.begin(), t.copy_count.end(), copy_count);
    std::copy(t.sequence_ids.begin(), t.sequence_ids.end(), seq_ids);
  });
}
int32_t orc_scheduler_packer_pages(void* s, uint64_t seq, int32_t* out, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    const auto& pages = static_cast<OrcScheduler*>(s)->packer->pages_of(seq);
    if (static_cast<int64_t>(pages.size()) > capacity) fail(ErrorKind::InvalidShape, "page capacity too small");
    std::copy(pages.begin(), pages.end(), out);
    *n_out = static_cast<int64_t>(pages.size());
  });
}
int32_t orc_scheduler_packer_free(void* s, int64_t* out) {
  return guard([&] { *out = static_cast<int64_t>(static_cast<OrcScheduler*>(s)->packer->free_pages()); });
}

// Block ids of a live sequence's paged session storage for `tokens` tokens of `layer`
// (PagedKvCacheStorage::block_table); n_out = 0 when the sequence holds no session.
int32_t orc_scheduler_session_blocks(void* s, uint64_t seq, int64_t layer, int64_t tokens, int64_t* out,
                                     int64_t capacity, int64_t* n_out) {
  return guard([&] {
    *n_out = 0;
    const Session* sess = static_cast<OrcScheduler*>(s)->sched->session(seq);
    if (!sess || !sess->kv_cache().paged_storage()) return;
    auto t = sess->kv_cache().paged_storage()->block_table(layer, tokens);
    if (static_cast<int64_t>(t.size()) > capacity) fail(ErrorKind::InvalidShape, "block capacity too small");
    for (size_t i = 0; i < t.size(); ++i) out[i] = static_cast<int64_t>(t[i].block_id);
    *n_out = static_cast<int64_t>(t.size());
  });
}

int32_t orc_scheduler_has_pending(void* s) { return static_cast<OrcScheduler*>(s)->sched->has_pending() ? 1 : 0; }
// Per-update rows: int64[9] = (sequence_id, batch_kind, reused, appended, has_token, token_id,
// phase, finish_reason, released_block_count); probability in probs[i].
int32_t orc_scheduler_last_report(void* s, int32_t* kind, int64_t* rows, float* probs, int64_t capacity,
                                  int64_t* n_out) {
  return guard([&] {
    auto* o = static_cast<OrcScheduler*>(s);
    if (!o->last) fail(ErrorKind::Runtime, "no tick report");
    const auto& r = *o->last;
    if (static_cast<int64_t>(r.updates.size()) > capacity) fail(ErrorKind::InvalidShape, "report capacity too small");
    *kind = static_cast<int32_t>(r.tick.kind);
    for (size_t i = 0; i < r.updates.size(); ++i) {
      const auto& u = r.updates[i];
      int64_t* row = rows + 9 * i;
      row[0] = u.sequence_id;
      row[1] = static_cast<int64_t>(u.batch_kind);
      row[2] = u.reused_prompt_tokens;
      row[3] = u.appended_prompt_tokens;
      row[4] = u.has_token ? 1 : 0;
      row[5] = u.has_token ? u.generated.token_id : -1;
      row[6] = static_cast<int64_t>(u.phase);
      row[7] = static_cast<int64_t>(u.finish_reason);
      row[8] = static_cast<int64_t>(u.released_prefix_blocks.size());
      probs[i] = u.has_token ? u.generated.probability : 0.0f;
    }
    *n_out = static_cast<int64_t>(r.updates.size());
  });
}
// Released blocks of update i: int64[n*3] = (owner, layer, block_id).
int32_t orc_scheduler_last_released(void* s, int64_t update, int64_t* out, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    auto* o = static_cast<OrcScheduler*>(s);
    if (!o->last) fail(ErrorKind::Runtime, "no tick report");
    const auto& rel = o->last->updates.at(update).released_prefix_blocks;
    if (static_cast<int64_t>(rel.size()) > capacity) fail(ErrorKind::InvalidShape, "released capacity too small");
    for (size_t i = 0; i < rel.size(); ++i) {
      out[3 * i] = rel[i].owner_sequence_id;
      out[3 * i + 1] = rel[i].layer_index;
      out[3 * i + 2] = rel[i].block_id;
    }
    *n_out = static_cast<int64_t>(rel.size());
  });
}
// Generated tokens of a sequence so far.
int32_t orc_scheduler_generated(void* s, uint64_t seq, uint32_t* out, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    const SequenceState* st = static_cast<OrcScheduler*>(s)->sched->sequence_state(seq);
    if (!st) fail(ErrorKind::Runtime, "unknown sequence");
    if (static_cast<int64_t>(st->generated.size()) > capacity) fail(ErrorKind::InvalidShape, "capacity too small");
    std::memcpy(out, st->generated.data(), st->generated.size() * sizeof(uint32_t));
    *n_out = static_cast<int64_t>(st->generated.size());
  });
}
int32_t orc_scheduler_block_ref_count(void* s, uint64_t owner, int64_t layer, int64_t block, int64_t* out) {
  return guard([&] {
    *out = static_cast<OrcScheduler*>(s)->sched->block_manager().block_ref_count({owner, static_cast<size_t>(layer),
                                                                                  static_cast<size_t>(block)});
  });
}

// ---------------------------------------------------------------- paged decode CPU baseline
// The reference's paged decode step for one layer (runtime/reference.rs:497-508): for each
// sequence, gather the committed prefix of L-1 tokens from its pages by block table
// (paged_kv.rs:769-791), then cached_prefixed_causal_attention_f32 with the current token
// (position L-1) as the one-row suffix.  Pages use the reference layout
// [num_blocks, page_size, Hkv, D]; block_tables is [B, max_blocks] int32.
int32_t orc_paged_decode_gather_attention(const float* q, const float* k_pages, const float* v_pages,
                                          const int32_t* block_tables, int64_t max_blocks,
                                          const int32_t* context_lens, int64_t num_seqs, int64_t hq,
                                          int64_t hkv, int64_t d, int64_t page_size, float* out) {
  return guard([&] {
    size_t slot = static_cast<size_t>(hkv * d);
    std::vector<float> ck, cv;
    for (int64_t b = 0; b < num_seqs; ++b) {
      int64_t len = context_lens[b];
      if (len <= 0) fail(ErrorKind::InvalidShape, "context length must be positive");
      if ((len + page_size - 1) / page_size > max_blocks) fail(ErrorKind::InvalidShape, "block table too short");
      int64_t prefix = len - 1;
      ck.clear();
      cv.clear();
      for (int64_t start = 0; start < prefix; start += page_size) {
        int64_t blk = block_tables[b * max_blocks + start / page_size];
        int64_t n = std::min<int64_t>(page_size, prefix - start);
        const float* kp = k_pages + static_cast<size_t>(blk) * page_size * slot;
        const float* vp = v_pages + static_cast<size_t>(blk) * page_size * slot;
        ck.insert(ck.end(), kp, kp + n * slot);
        cv.insert(cv.end(), vp, vp + n * slot);
      }
      int64_t last_blk = block_tables[b * max_blocks + prefix / page_size];
      const float* ks = k_pages + (static_cast<size_t>(last_blk) * page_size + prefix % page_size) * slot;
      const float* vs = v_pages + (static_cast<size_t>(last_blk) * page_size + prefix % page_size) * slot;
      cached_prefixed_causal_attention_f32(q + b * hq * d, ck.data(), cv.data(), prefix, ks, vs, 1, hq, hkv,
                                           d, out + b * hq * d);
    }
  });
}

}  // extern "C"
