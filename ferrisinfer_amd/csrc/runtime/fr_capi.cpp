// C entry points of libferrisinfer_runtime.so (include/ferrisinfer_runtime.h).
#include <array>
#include <cstring>
#include <memory>
#include <string>

#include "../../../include/ferrisinfer_runtime.h"
#include "fr_checkpoint.h"
#include "fr_runtime.h"

namespace {
thread_local std::string g_err;

struct Runtime {
  fi_context* ctx = nullptr;
  std::unique_ptr<fr::DeviceModel> model;
  std::unique_ptr<fr::BlockPool> pool;
  std::unique_ptr<fr::Scheduler> scheduler;
  fr::SessionConfig session;
  fr::SchedulerConfig sched;
  bool graph_decode = false;
  std::optional<fr::TickReport> last;
  ~Runtime() {
    scheduler.reset();
    pool.reset();
    model.reset();
    if (ctx) fi_ctx_destroy(ctx);
  }
  fr::Scheduler& scheduler_ready() {
    if (!scheduler) scheduler = std::make_unique<fr::Scheduler>(model.get(), pool.get(), session, sched, graph_decode);
    return *scheduler;
  }
};

template <typename F>
int32_t guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const fr::Error& e) {
    g_err = e.message;
    return static_cast<int32_t>(e.kind) + 1;
  } catch (const std::exception& e) {
    g_err = e.what();
    return FI_ERR_RUNTIME;
  }
}
Runtime* rt(void* h) { return static_cast<Runtime*>(h); }
// the last tick's batch, or an empty one before the first tick (observers create nothing)
const fr::PackedBatch& last_batch_of(void* h) {
  static const fr::PackedBatch empty;
  return rt(h)->scheduler ? rt(h)->scheduler->last_batch() : empty;
}
}  // namespace

extern "C" {

const char* fr_last_error(void) { return g_err.c_str(); }

int32_t fr_create(int32_t ordinal, const fr_model_config* mc, const fr_runtime_config* rc, void** out) {
  return guard([&] {
    if (!mc || !rc || !out) fr::fail(fr::ErrorKind::InvalidConfig, "fr_create: null argument");
    auto r = std::make_unique<Runtime>();
    fr::check(fi_ctx_create(ordinal, &r->ctx));
    fr::ModelConfig c;
    c.hidden_size = mc->hidden_size;
    c.intermediate_size = mc->intermediate_size;
    c.num_layers = mc->num_layers;
    c.num_attention_heads = mc->num_attention_heads;
    c.num_key_value_heads = mc->num_key_value_heads;
    c.vocab_size = mc->vocab_size;
    c.max_position_embeddings = mc->max_position_embeddings;
    c.rms_norm_eps = mc->rms_norm_eps;
    c.rope_theta = mc->rope_theta;
    c.rotary_dims = mc->rotary_dims;
    c.tie_word_embeddings = mc->tie_word_embeddings != 0;
    r->session.max_sequence_length = rc->max_sequence_length;
    r->session.max_generated_tokens = rc->max_generated_tokens;
    if (rc->top_k < 0) fr::fail(fr::ErrorKind::InvalidConfig, "sampler top_k must not be negative");
    r->session.sampler.temperature = rc->temperature;
    r->session.sampler.top_k = rc->top_k;
    r->session.sampler.top_p = rc->top_p;
    r->session.sampler.repetition_penalty = rc->repetition_penalty;
    r->session.sampler.seed = rc->seed;
    if (!r->session.sampler.is_greedy() && std::min<int64_t>(std::max<int64_t>(rc->top_k, 1), mc->vocab_size) > 1024 &&
        mc->vocab_size > (1 << 20)) {
      fr::fail(fr::ErrorKind::Unsupported,
               "sampler top_k above 1024 is served for vocabularies of at most 1048576 logits");
    }
    r->sched.max_batch_size = rc->max_batch_size;
    r->sched.max_prefill_chunk_tokens = rc->max_prefill_chunk_tokens;
    r->sched.max_prefill_batch_tokens = rc->max_prefill_batch_tokens;
    r->sched.max_consecutive_prefill_ticks = rc->max_consecutive_prefill_ticks;
    r->sched.min_prefix_share_tokens = rc->min_prefix_share_tokens;
    if (rc->weight_dtype != FI_DTYPE_F32 && rc->weight_dtype != FI_DTYPE_BF16) {
      fr::fail(fr::ErrorKind::InvalidType, "projection weight dtype must be f32 or bf16");
    }
    r->graph_decode = rc->graph_decode != 0;
    r->model = std::make_unique<fr::DeviceModel>(r->ctx, c, static_cast<int32_t>(rc->max_sequence_length),
                                                 rc->weight_dtype);
    r->pool = std::make_unique<fr::BlockPool>(r->ctx, c.num_layers, rc->num_blocks, rc->block_size,
                                              c.num_key_value_heads, c.head_dim(), rc->kv_dtype);
    *out = r.release();
  });
}

int32_t fr_destroy(void* h) {
  return guard([&] { delete rt(h); });
}

int32_t fr_set_weight(void* h, const char* name, const float* data, int64_t count) {
  return guard([&] {
    if (rt(h)->scheduler) fr::fail(fr::ErrorKind::Runtime, "weights are frozen once requests were submitted");
    rt(h)->model->set_weight(name, data, static_cast<size_t>(count));
  });
}

int32_t fr_set_weight_device(void* h, const char* name, const void* d_data, int32_t src_dtype, int64_t count) {
  return guard([&] {
    if (rt(h)->scheduler) fr::fail(fr::ErrorKind::Runtime, "weights are frozen once requests were submitted");
    if (!d_data || count < 0) fr::fail(fr::ErrorKind::InvalidConfig, "fr_set_weight_device: null data or negative count");
    rt(h)->model->set_weight_device(name, d_data, src_dtype, static_cast<size_t>(count));
  });
}

int32_t fr_hf_read_config(const char* model_dir, fr_model_config* out) {
  return guard([&] {
    if (!model_dir || !out) fr::fail(fr::ErrorKind::InvalidConfig, "fr_hf_read_config: null argument");
    const fr::ModelConfig c = fr::read_hf_config(model_dir);
    out->hidden_size = c.hidden_size;
    out->intermediate_size = c.intermediate_size;
    out->num_layers = c.num_layers;
    out->num_attention_heads = c.num_attention_heads;
    out->num_key_value_heads = c.num_key_value_heads;
    out->vocab_size = c.vocab_size;
    out->max_position_embeddings = c.max_position_embeddings;
    out->rms_norm_eps = c.rms_norm_eps;
    out->rope_theta = c.rope_theta;
    out->rotary_dims = c.rotary_dims;
    out->tie_word_embeddings = c.tie_word_embeddings ? 1 : 0;
  });
}

int32_t fr_hf_inspect(const char* model_dir, int64_t* counts) {
  return guard([&] {
    if (!model_dir || !counts) fr::fail(fr::ErrorKind::InvalidConfig, "fr_hf_inspect: null argument");
    const fr::HfInspection r = fr::inspect_hf(model_dir);
    counts[0] = static_cast<int64_t>(r.shard_count);
    counts[1] = static_cast<int64_t>(r.tensor_count);
    counts[2] = static_cast<int64_t>(r.total_data_bytes);
    counts[3] = static_cast<int64_t>(r.mapped_required);
    counts[4] = static_cast<int64_t>(r.mapped_optional);
    counts[5] = static_cast<int64_t>(r.missing_required.size());
    counts[6] = static_cast<int64_t>(r.missing_optional.size());
    counts[7] = static_cast<int64_t>(r.shape_mismatches.size());
  });
}

int32_t fr_safetensors_info(const char* model_dir, int64_t* tensors, int64_t* shards, int64_t* total_bytes) {
  return guard([&] {
    if (!model_dir || !tensors || !shards || !total_bytes) fr::fail(fr::ErrorKind::InvalidConfig, "fr_safetensors_info: null argument");
    const fr::SafeTensorsRepository repo = fr::SafeTensorsRepository::open(model_dir);
    *tensors = static_cast<int64_t>(repo.tensor_count());
    *shards = static_cast<int64_t>(repo.shard_count());
    *total_bytes = static_cast<int64_t>(repo.total_data_bytes());
  });
}

int32_t fr_safetensors_entry(const char* model_dir, const char* name, int32_t* dtype, int64_t* shape, int32_t capacity,
                             int32_t* rank, char* path, int64_t path_capacity, int64_t* offset, int64_t* byte_len) {
  return guard([&] {
    if (!model_dir || !name || !dtype || !shape || !rank || !path || !offset || !byte_len) {
      fr::fail(fr::ErrorKind::InvalidConfig, "fr_safetensors_entry: null argument");
    }
    const fr::SafeTensorsRepository repo = fr::SafeTensorsRepository::open(model_dir);
    const fr::StEntry* e = repo.get(name);
    if (e == nullptr) {
      fr::fail(fr::ErrorKind::MissingWeight, std::string("tensor '") + name + "' was not found in safetensors repository");
    }
    if (static_cast<int64_t>(e->shape.size()) > capacity) fr::fail(fr::ErrorKind::InvalidShape, "shape capacity too small");
    if (static_cast<int64_t>(e->path.size()) + 1 > path_capacity) fr::fail(fr::ErrorKind::InvalidShape, "path capacity too small");
    *dtype = e->dtype == fr::StDType::F32 ? FI_DTYPE_F32 : (e->dtype == fr::StDType::BF16 ? FI_DTYPE_BF16 : FI_DTYPE_F16);
    *rank = static_cast<int32_t>(e->shape.size());
    for (size_t i = 0; i < e->shape.size(); ++i) shape[i] = static_cast<int64_t>(e->shape[i]);
    std::memcpy(path, e->path.c_str(), e->path.size() + 1);
    *offset = static_cast<int64_t>(e->absolute_offset());
    *byte_len = static_cast<int64_t>(e->byte_len());
  });
}

int32_t fr_load_hf_weights(void* h, const char* model_dir, int64_t* loaded) {
  return guard([&] {
    if (!model_dir) fr::fail(fr::ErrorKind::InvalidConfig, "fr_load_hf_weights: null directory");
    if (rt(h)->scheduler) fr::fail(fr::ErrorKind::Runtime, "weights are frozen once requests were submitted");
    const size_t n = fr::load_hf_weights(rt(h)->model.get(), model_dir);
    if (loaded) *loaded = static_cast<int64_t>(n);
  });
}

int32_t fr_submit(void* h, const uint32_t* ids, int64_t n, int64_t max_new, int64_t stop, uint64_t* seq_out) {
  return guard([&] {
    std::optional<uint32_t> st;
    if (stop >= 0) st = static_cast<uint32_t>(stop);
    *seq_out = rt(h)->scheduler_ready().submit(std::vector<uint32_t>(ids, ids + n), static_cast<size_t>(max_new), st);
  });
}

int32_t fr_execute_next_tick(void* h, int32_t* executed) {
  return guard([&] {
    rt(h)->last = rt(h)->scheduler_ready().execute_next_tick();
    *executed = rt(h)->last ? 1 : 0;
  });
}

int32_t fr_execute_next_tick_ex(void* h, int32_t flags, int32_t* executed) {
  return guard([&] {
    if ((flags & ~FR_TICK_RUN_AHEAD) != 0) fr::fail(fr::ErrorKind::InvalidConfig, "unknown tick flags");
    rt(h)->last = rt(h)->scheduler_ready().execute_next_tick((flags & FR_TICK_RUN_AHEAD) != 0);
    *executed = rt(h)->last ? 1 : 0;
  });
}

int32_t fr_run_ahead_counters(void* h, uint64_t* out) {
  return guard([&] {
    std::array<uint64_t, 4> c{};
    if (rt(h)->scheduler) c = rt(h)->scheduler->run_ahead_counters();
    for (size_t i = 0; i < c.size(); ++i) out[i] = c[i];
  });
}

int32_t fr_has_pending(void* h) { return rt(h)->scheduler && rt(h)->scheduler->has_pending() ? 1 : 0; }

int32_t fr_last_report(void* h, int32_t* kind, int64_t* rows, float* probs, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    const auto& last = rt(h)->last;
    if (!last) fr::fail(fr::ErrorKind::Runtime, "no tick report");
    if (static_cast<int64_t>(last->updates.size()) > capacity) fr::fail(fr::ErrorKind::InvalidShape, "report capacity too small");
    *kind = static_cast<int32_t>(last->kind);
    for (size_t i = 0; i < last->updates.size(); ++i) {
      const fr::SequenceUpdate& u = last->updates[i];
      int64_t* row = rows + 9 * i;
      row[0] = static_cast<int64_t>(u.sequence_id);
      row[1] = static_cast<int64_t>(u.batch_kind);
      row[2] = static_cast<int64_t>(u.reused_prompt_tokens);
      row[3] = static_cast<int64_t>(u.appended_prompt_tokens);
      row[4] = u.has_token ? 1 : 0;
      row[5] = u.has_token ? static_cast<int64_t>(u.generated.token_id) : -1;
      row[6] = static_cast<int64_t>(u.phase);
      row[7] = static_cast<int64_t>(u.finish_reason);
      row[8] = static_cast<int64_t>(u.released_prefix_blocks.size());
      probs[i] = u.has_token ? u.generated.probability : 0.0f;
    }
    *n_out = static_cast<int64_t>(last->updates.size());
  });
}

int32_t fr_last_released(void* h, int64_t update, int64_t* out, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    const auto& last = rt(h)->last;
    if (!last) fr::fail(fr::ErrorKind::Runtime, "no tick report");
    const auto& rel = last->updates.at(static_cast<size_t>(update)).released_prefix_blocks;
    if (static_cast<int64_t>(rel.size()) > capacity) fr::fail(fr::ErrorKind::InvalidShape, "released capacity too small");
    for (size_t i = 0; i < rel.size(); ++i) {
      out[3 * i] = static_cast<int64_t>(rel[i].owner_sequence_id);
      out[3 * i + 1] = rel[i].layer_index;
      out[3 * i + 2] = rel[i].block_id;
    }
    *n_out = static_cast<int64_t>(rel.size());
  });
}

int32_t fr_generated(void* h, uint64_t seq, uint32_t* out, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    const fr::Sequence* s = rt(h)->scheduler ? rt(h)->scheduler->sequence(seq) : nullptr;
    if (!s) fr::fail(fr::ErrorKind::Runtime, "unknown sequence");
    if (static_cast<int64_t>(s->generated.size()) > capacity) fr::fail(fr::ErrorKind::InvalidShape, "capacity too small");
    std::memcpy(out, s->generated.data(), s->generated.size() * sizeof(uint32_t));
    *n_out = static_cast<int64_t>(s->generated.size());
  });
}

int32_t fr_sequence_blocks(void* h, uint64_t seq, int32_t* out, int64_t capacity, int64_t* n_out) {
  return guard([&] {
    const fr::Sequence* s = rt(h)->scheduler ? rt(h)->scheduler->sequence(seq) : nullptr;
    if (!s) fr::fail(fr::ErrorKind::Runtime, "unknown sequence");
    if (static_cast<int64_t>(s->blocks.size()) > capacity) fr::fail(fr::ErrorKind::InvalidShape, "capacity too small");
    std::memcpy(out, s->blocks.data(), s->blocks.size() * sizeof(int32_t));
    *n_out = static_cast<int64_t>(s->blocks.size());
  });
}

int32_t fr_pool_free_count(void* h, int64_t* out) {
  return guard([&] { *out = static_cast<int64_t>(rt(h)->pool->free_count()); });
}

int32_t fr_graph_counters(void* h, uint64_t* out) {
  return guard([&] {
    // observers report an empty state before the first submit (creating the scheduler here
    // would freeze the weights)
    std::array<uint64_t, 3> c{};
    if (rt(h)->scheduler) c = rt(h)->scheduler->executor().graph_counters();
    for (size_t i = 0; i < c.size(); ++i) out[i] = c[i];
  });
}

int32_t fr_last_tick_profile(void* h, double* out) {
  return guard([&] {
    std::array<double, 4> p{};
    if (rt(h)->scheduler) p = rt(h)->scheduler->last_tick_profile();
    for (size_t i = 0; i < p.size(); ++i) out[i] = p[i];
  });
}

int32_t fr_last_logits(void* h, float* out, int64_t capacity, int64_t* rows) {
  return guard([&] {
    if (!rows || capacity < 0 || (capacity > 0 && !out)) fr::fail(fr::ErrorKind::InvalidConfig, "fr_last_logits: bad buffer");
    *rows = 0;
    if (rt(h)->scheduler) rt(h)->scheduler->executor().last_logits(out, static_cast<size_t>(capacity), rows);
  });
}

int32_t fr_last_batch_sizes(void* h, int64_t* sizes) {
  return guard([&] {
    const fr::PackedBatch& b = last_batch_of(h);
    sizes[0] = static_cast<int64_t>(b.token_ids.size());
    sizes[1] = static_cast<int64_t>(b.sequence_ids.size());
    sizes[2] = b.max_blocks;
    sizes[3] = static_cast<int64_t>(b.copy_src.size());
    sizes[4] = static_cast<int64_t>(b.kind);
    sizes[5] = b.max_query_len;
    sizes[6] = b.max_context_len;
  });
}

int32_t fr_last_batch(void* h, int32_t* token_ids, int32_t* positions, int64_t* slots, int32_t* cu_seqlens,
                      int32_t* context_lens, int32_t* block_tables, int32_t* copy_src, int32_t* copy_dst,
                      int32_t* copy_count, uint64_t* sequence_ids) {
  return guard([&] {
    const fr::PackedBatch& b = last_batch_of(h);
    auto cp = [](void* dst, const void* src, size_t bytes) {
      if (bytes) std::memcpy(dst, src, bytes);
    };
    cp(token_ids, b.token_ids.data(), b.token_ids.size() * 4);
    cp(positions, b.positions.data(), b.positions.size() * 4);
    cp(slots, b.slot_mapping.data(), b.slot_mapping.size() * 8);
    cp(cu_seqlens, b.cu_seqlens.data(), b.cu_seqlens.size() * 4);
    cp(context_lens, b.context_lens.data(), b.context_lens.size() * 4);
    cp(block_tables, b.block_tables.data(), b.block_tables.size() * 4);
    cp(copy_src, b.copy_src.data(), b.copy_src.size() * 4);
    cp(copy_dst, b.copy_dst.data(), b.copy_dst.size() * 4);
    cp(copy_count, b.copy_count.data(), b.copy_count.size() * 4);
    cp(sequence_ids, b.sequence_ids.data(), b.sequence_ids.size() * 8);
  });
}

}  // extern "C"
