/*
 * ferrisinfer_runtime.h — C ABI of the host runtime above the HIP backend
 * (libferrisinfer_runtime.so).  It keeps the reference's scheduler / session API
 * (crates/ferrisinfer-runtime/src/scheduler.rs:109-648, session.rs:92-413): requests are
 * submitted, ticks are planned exactly as ReferenceScheduler::plan_next_tick and executed as
 * one packed ragged batch on the GPU, and each tick returns the reference's per-sequence
 * execution report (scheduler.rs:54-71).  Status codes and fr_last_error() follow
 * include/ferrisinfer_kernel.h.  A Rust host would keep its own scheduler and call the kernel
 * ABI directly; this library is the C++ stand-in for that host.
 */
#ifndef FERRISINFER_RUNTIME_H
#define FERRISINFER_RUNTIME_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ModelConfig (model/config.rs:5-20) with the Qwen2/Llama rope and norm parameters. */
typedef struct fr_model_config {
  int32_t hidden_size;
  int32_t intermediate_size;
  int32_t num_layers;
  int32_t num_attention_heads;
  int32_t num_key_value_heads;
  int32_t vocab_size;
  int32_t max_position_embeddings;
  float rms_norm_eps;
  float rope_theta;
  int32_t rotary_dims;
  int32_t tie_word_embeddings;
} fr_model_config;

/* SessionConfig (session.rs:29-46), SchedulerConfig (scheduler.rs:16-35) and the block pool. */
typedef struct fr_runtime_config {
  int64_t max_sequence_length;
  int64_t max_generated_tokens;
  int64_t max_batch_size;
  int64_t max_prefill_chunk_tokens;
  int64_t max_prefill_batch_tokens;
  int64_t max_consecutive_prefill_ticks;
  int64_t min_prefix_share_tokens;
  int32_t num_blocks;
  int32_t block_size;
  int32_t kv_dtype; /* FI_DTYPE_F32 or FI_DTYPE_BF16 */
  /* SamplerConfig of every session (sampler.rs:3-43, session.rs:29-46).  Greedy when
   * temperature <= 0, top_k == 1 or top_p <= 0 (a zero-filled struct is greedy): the fused
   * argmax head.  Otherwise sample_last_token on the device (fi_sample_tokens) with one
   * SamplerState per sequence started from `seed`; top_k, clamped to the vocabulary, must not
   * exceed 1024 (Unsupported at fr_create). */
  float temperature;
  int64_t top_k;
  float top_p;
  float repetition_penalty; /* carried, unused by the sampler (as in the reference) */
  uint64_t seed;
  /* Storage of the packed projection weights and head: FI_DTYPE_F32 (fi_gemm_packed) or
   * FI_DTYPE_BF16 (fi_gemm_bf16: weights rounded to nearest even at packing, exact for bf16
   * checkpoints, which the reference widens at load, io/safetensors.rs:540-542). */
  int32_t weight_dtype;
  /* Non-zero: decode ticks replay HIP graphs of their launch sequence (fi_graph_*), captured
   * per (batch size, context bucket, sampler kind); results are the eager path's. */
  int32_t graph_decode;
} fr_runtime_config;

const char* fr_last_error(void);

/* Creates a runtime on device `ordinal`: device model (weights uploaded by fr_set_weight
 * with the reference's names and [in, out] layout, model/decoder.rs:30-114), KV block pool
 * and scheduler. */
int32_t fr_create(int32_t ordinal, const fr_model_config* model, const fr_runtime_config* config,
                  void** out);
int32_t fr_destroy(void* runtime);
int32_t fr_set_weight(void* runtime, const char* name, const float* data, int64_t count);
/* fr_set_weight from device memory on the runtime's GPU: `count` elements of src_dtype
 * (FI_DTYPE_F32, _BF16 or _F16), widened to f32 as the checkpoint loader widens them
 * (fi_convert_to_f32; io/safetensors.rs:437-471, 538-568).  For weights generated or staged in
 * HBM, which then never cross PCIe. */
int32_t fr_set_weight_device(void* runtime, const char* name, const void* d_data, int32_t src_dtype, int64_t count);

/* ReferenceScheduler::submit (scheduler.rs:204-250); stop < 0 means no stop token. */
/* ---------------------------------------------------------------- checkpoint import
 * HF Qwen2 checkpoints (config.json + model.safetensors or a sharded
 * model.safetensors.index.json) with F32 / BF16 / F16 tensors.
 *
 * fr_hf_read_config: config.json -> model config (io/hf.rs:306-369 parse_qwen2_config;
 * model_type must be "qwen2"; hidden_act silu / swish, other activations Unsupported: the
 * device decoder is silu-gated).  rotary_dims = round(head_dim * partial_rotary_factor). */
int32_t fr_hf_read_config(const char* model_dir, fr_model_config* out);
/* io/hf.rs:66-118 HfSource::inspect: counts[8] = shard count, tensor count, total data bytes,
 * mapped required, mapped optional, missing required, missing optional, shape mismatches. */
int32_t fr_hf_inspect(const char* model_dir, int64_t* counts);
/* io/safetensors.rs:87-187 SafeTensorsRepository::open / tensor_count / shard_count /
 * total_data_bytes, with the header validation of :225-397 (Io, Parse, InvalidType,
 * Unsupported and Runtime errors as the reference raises them). */
int32_t fr_safetensors_info(const char* model_dir, int64_t* tensors, int64_t* shards, int64_t* total_bytes);
/* One tensor's entry: dtype (FI_DTYPE_F32 / _BF16 / _F16), shape (rank <= capacity), the
 * shard file path (NUL-terminated) and the absolute byte offset and length of its data
 * (safetensors.rs:47-83 SafeTensorEntry). */
int32_t fr_safetensors_entry(const char* model_dir, const char* name, int32_t* dtype, int64_t* shape, int32_t capacity,
                             int32_t* rank, char* path, int64_t path_capacity, int64_t* offset, int64_t* byte_len);
/* Loads every planned tensor (io/hf.rs:208-304, 380-500: names, expected shapes, [out, in] ->
 * [in, out] transposes, optional q/k/v biases, lm_head unless tied) into the runtime's model:
 * each tensor's raw bytes go to HBM and are widened / transposed there (fi_convert_to_f32).
 * The runtime's model config must be the checkpoint's (fr_hf_read_config); shape mismatches
 * are InvalidShape, absent required tensors MissingWeight.  loaded (may be NULL) = tensors
 * loaded. */
int32_t fr_load_hf_weights(void* runtime, const char* model_dir, int64_t* loaded);

int32_t fr_submit(void* runtime, const uint32_t* prompt, int64_t n, int64_t max_new_tokens,
                  int64_t stop, uint64_t* sequence_id);
/* ReferenceScheduler::execute_next_tick (scheduler.rs:393-415); *executed = 0 when idle. */
int32_t fr_execute_next_tick(void* runtime, int32_t* executed);
/* fr_execute_next_tick with flags.  FR_TICK_RUN_AHEAD: once this tick is enqueued, also enqueue
 * the next tick when it will be a decode tick, so the device runs it while the host returns
 * this tick's report and plans the next call (the roadmap's stream overlap,
 * docs/performance-roadmap.md:321-326; the reference runs its ticks one after the other).  The
 * next tick's batch follows from the state this tick leaves, except its token ids and, for a
 * sampled session, its sampler states, which are this tick's samples and advanced states and
 * are fed on the device.  The next call (with or without the flag) keeps
 * the enqueued tick when its own planning packs the same batch, and otherwise waits for it and
 * drops it: a submit in between drops it.  Reports, tokens, probabilities, block ids and
 * released blocks are those of calls without the flag.  A caller that expects no submit before
 * its next call sets the flag; a wrong expectation costs the dropped tick's device time. */
#define FR_TICK_RUN_AHEAD 1
int32_t fr_execute_next_tick_ex(void* runtime, int32_t flags, int32_t* executed);
/* [ticks enqueued ahead, kept, dropped, 1 if the last executed tick was one enqueued ahead].
 * Before the first submit it reports zeros (observers create no scheduler). */
int32_t fr_run_ahead_counters(void* runtime, uint64_t* out4);
int32_t fr_has_pending(void* runtime);
/* Report of the last tick: rows of 9 int64 (sequence_id, batch_kind, reused, appended,
 * has_token, token_id, phase, finish_reason, released_block_count) + probabilities. */
int32_t fr_last_report(void* runtime, int32_t* kind, int64_t* rows, float* probs, int64_t capacity,
                       int64_t* n_out);
/* Released prefix blocks of update `index`: (owner, layer, block) triples. */
int32_t fr_last_released(void* runtime, int64_t index, int64_t* out, int64_t capacity,
                         int64_t* n_out);
int32_t fr_generated(void* runtime, uint64_t sequence_id, uint32_t* out, int64_t capacity,
                     int64_t* n_out);
int32_t fr_sequence_blocks(void* runtime, uint64_t sequence_id, int32_t* out, int64_t capacity,
                           int64_t* n_out);
int32_t fr_pool_free_count(void* runtime, int64_t* out);
/* Decode ticks replayed from graphs, graphs captured, graphs dropped (buffers moved). */
int32_t fr_graph_counters(void* runtime, uint64_t* out3);
/* The last packed batch: sizes = [T, B, max_blocks, copies, kind, max_query_len,
 * max_context_len]; then its arrays (token ids, positions, slot mapping, cu_seqlens, context
 * lengths, block tables [B, max_blocks], copy-on-write src/dst/count, sequence ids). */
int32_t fr_last_batch_sizes(void* runtime, int64_t* sizes);
/* The logits rows the last tick sampled from, one per batch sequence in the batch's order
 * ([rows, vocab] f32 into `capacity` floats): each sequence's last-row logits, the
 * decode-workspace / prefill logits the reference's session passes to sample_last_token
 * (session.rs:357-373, 399-406).  rows = 0 after a greedy tick, whose head is fused with the
 * argmax and writes no logits. */
int32_t fr_last_logits(void* runtime, float* out, int64_t capacity, int64_t* rows);
int32_t fr_last_batch(void* runtime, int32_t* token_ids, int32_t* positions, int64_t* slots,
                      int32_t* cu_seqlens, int32_t* context_lens, int32_t* block_tables,
                      int32_t* copy_src, int32_t* copy_dst, int32_t* copy_count,
                      uint64_t* sequence_ids);
/* Host seconds of the last tick: out[4] = [scheduling + packing, enqueueing the batched
 * forward, waiting for its samples, whole tick].  The reference times whole ticks only
 * (cli/main.rs:1763-1767); the split shows where a tick's time goes. */
int32_t fr_last_tick_profile(void* runtime, double* out);

#ifdef __cplusplus
}
#endif

#endif /* FERRISINFER_RUNTIME_H */
