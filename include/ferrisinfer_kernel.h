/*
 * ferrisinfer_kernel.h — C ABI of the MI355X (gfx950) HIP backend of FerrisInfer's
 * ragged-batch attention hot path.
 *
 * The reference has no compute FFI: its hot path is Rust free functions in
 * crates/ferrisinfer-kernel/src/cpu/{attention,matmul,reduction,elementwise}.rs called from crates/ferrisinfer-runtime/src/reference.rs,
 * KV storage behind the KvCacheStorage trait (runtime/kv_cache.rs:36-64), and a device
 * layer that binds a C driver by dlsym (kernel/gpu/nvidia.rs:678-727).  This header is the
 * C surface a `ferrisinfer-kernel-sys` crate (or ctypes / cgo) binds in their place.  Each
 * declaration cites the reference interface it replaces.
 *
 * Conventions (mirroring kernel/gpu/nvidia.rs:887-932 and core/error.rs:5-16):
 *   - every function returns int32_t status: 0 = ok, otherwise ErrorKind index + 1
 *     (Io=1 Parse=2 InvalidShape=3 InvalidLayout=4 InvalidType=5 InvalidConfig=6
 *      MissingWeight=7 Unsupported=8 Runtime=9); fi_last_error() gives the message
 *     (thread-local, valid until the next failing call on that thread);
 *   - pointers named d_* are device pointers (HBM); everything else is host memory;
 *   - ops enqueue on the context's stream and return without synchronising; only
 *     fi_buf_download and fi_ctx_sync wait;
 *   - callers own every buffer; ops never allocate their outputs.  Split-KV decode keeps
 *     a grow-only workspace inside the context;
 *   - one host thread drives a context at a time (the reference scheduler is &mut self).
 *
 * Layouts:
 *   activations are row-major f32: q [T, Hq, D], k/v [T, Hkv, D], hidden [T, H];
 *   weights are [in, out] row-major f32 (model/decoder.rs:76-104);
 *   the KV pool holds, per layer, K and V arrays [num_blocks, Hkv, block_size, D] in
 *   f32 or bf16; physical slot = block_id * block_size + offset
 *   (runtime/paged_kv.rs:605-606);
 *   block_tables is int32 [num_seqs, max_blocks_per_seq]; context_lens int32 [num_seqs];
 *   cu_seqlens int32 [num_seqs + 1]; slot_mapping int64 [T] (negative = skip).
 */
#ifndef FERRISINFER_KERNEL_H
#define FERRISINFER_KERNEL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FI_OK = 0,
  FI_ERR_IO = 1,
  FI_ERR_PARSE = 2,
  FI_ERR_INVALID_SHAPE = 3,
  FI_ERR_INVALID_LAYOUT = 4,
  FI_ERR_INVALID_TYPE = 5,
  FI_ERR_INVALID_CONFIG = 6,
  FI_ERR_MISSING_WEIGHT = 7,
  FI_ERR_UNSUPPORTED = 8,
  FI_ERR_RUNTIME = 9
};

/* Element dtypes: KV storage (core/dtype.rs:1-42 F32 / BF16) and, with F16, the safetensors
 * payloads fi_convert_to_f32 imports (io/safetensors.rs:11-16). */
enum { FI_DTYPE_F32 = 0, FI_DTYPE_BF16 = 1, FI_DTYPE_F16 = 2 };

typedef struct fi_context fi_context;

/* ---------------------------------------------------------------- errors / context */

/* Message of the last failing call on this thread
 * (FerrisError::message, core/error.rs:36-38). */
const char* fi_last_error(void);

/* Opens device `ordinal` and creates a context with its own stream.
 * Replaces NvidiaCudaBackend::new / primary-context retain (kernel/gpu/nvidia.rs:214-262). */
int32_t fi_ctx_create(int32_t ordinal, fi_context** out);

/* Releases the context (RAII Drop of the reference context, kernel/gpu/nvidia.rs:409-415). */
int32_t fi_ctx_destroy(fi_context* ctx);

/* Waits for all work enqueued on the context's stream (cuCtxSynchronize, nvidia.rs:387-389). */
int32_t fi_ctx_sync(fi_context* ctx);

/* Uses `stream` (a hipStream_t of the same device) for all later ops; NULL restores the
 * context's own stream.  No reference counterpart (the reference launches nothing). */
int32_t fi_ctx_set_stream(fi_context* ctx, void* stream);

/* The hipStream_t the context currently enqueues on. */
void* fi_ctx_stream(fi_context* ctx);

/* Device name, gfx arch, HBM bytes and CU count
 * (device probe, kernel/gpu/nvidia.rs:756-804). */
int32_t fi_device_info(fi_context* ctx, char* name, size_t name_len, char* arch, size_t arch_len,
                       uint64_t* hbm_bytes, int32_t* compute_units);

/* ---------------------------------------------------------------- graph capture
 * BackendCapabilities.graph_capture (kernel/backend.rs:3-10) and the roadmap's graph capture of
 * the decode step (docs/performance-roadmap.md:321-326; the reference backend captures nothing).
 * fi_graph_begin starts capturing the context's stream (which must not be the null stream);
 * every op enqueued on the context until fi_graph_end is recorded instead of run.  fi_graph_end
 * instantiates the recording (out = NULL discards it); fi_graph_launch replays it on the
 * context's stream with the device pointers and scalar arguments it was recorded with (device
 * memory contents, e.g. re-uploaded batch metadata, may change between replays).  While a capture
 * is open, calls that allocate, copy to or from the host or wait (fi_buf_*, fi_ctx_sync,
 * fi_ctx_check_faults) return Runtime, and an op that would grow the context workspace returns
 * Runtime instead; run such a launch once outside capture first. */
typedef struct fi_graph fi_graph;
int32_t fi_graph_begin(fi_context* ctx);
int32_t fi_graph_end(fi_context* ctx, fi_graph** out);
int32_t fi_graph_launch(fi_context* ctx, fi_graph* graph);
int32_t fi_graph_destroy(fi_graph* graph);

/* Counts reallocations of the context workspace (ops that split K or the decode partials of
 * fi_attn_decode_paged live there).  A graph recorded at generation g reads the workspace of
 * generation g: replay it only while the generation is unchanged. */
int32_t fi_ctx_workspace_generation(fi_context* ctx, uint64_t* generation);

/* ---------------------------------------------------------------- memory */

/* Device allocation; rejects 0 bytes like validate_buffer_len (kernel/gpu/nvidia.rs:910-919). */
int32_t fi_buf_alloc(fi_context* ctx, size_t bytes, void** d_out);
int32_t fi_buf_free(fi_context* ctx, void* d_ptr);
/* Host->device / device->host copies with the exact-length rule of validate_copy_len
 * (kernel/gpu/nvidia.rs:921-932; cuMemcpyHtoD/DtoH at nvidia.rs:340-470). */
int32_t fi_buf_upload(fi_context* ctx, void* d_dst, size_t dst_bytes, const void* src,
                      size_t src_bytes);
int32_t fi_buf_download(fi_context* ctx, void* dst, size_t dst_bytes, const void* d_src,
                        size_t src_bytes);
/* Backend::fill_zero (kernel/backend.rs:40); the reference's NVIDIA backend returns
 * Unsupported (nvidia.rs:319-323). */
int32_t fi_buf_zero(fi_context* ctx, void* d_ptr, size_t bytes);

/* ---------------------------------------------------------------- stream overlap
 * No counterpart in the reference's kernel layer, whose copies all wait (cuMemcpyHtoD/DtoH,
 * kernel/gpu/nvidia.rs:340-470).  These serve the roadmap's stream overlap
 * (docs/performance-roadmap.md:321-326): a host runtime enqueues the next decode step while the
 * device still runs the current one, and waits only for the samples it needs.
 *   - fi_host_alloc / fi_host_free: pinned host memory (fi_host_free waits for the stream).
 *   - fi_buf_upload_async / fi_buf_download_async: the copies of fi_buf_upload / download,
 *     enqueued on the context's stream without waiting (same exact-length rule).  The host
 *     memory should be pinned so the copy overlaps the host; it must stay valid and unchanged
 *     until the copy has run, which an event recorded after it reports.
 *   - fi_ctx_faults_async: enqueues a copy of the context's four device fault words into
 *     h_words[4]; a non-zero word means fi_ctx_check_faults will report (and clear) a fault.
 *   - fi_event_record marks the context's stream; fi_event_wait returns once everything
 *     enqueued before the mark has run. */
int32_t fi_host_alloc(fi_context* ctx, size_t bytes, void** h_out);
int32_t fi_host_free(fi_context* ctx, void* h_ptr);
int32_t fi_buf_upload_async(fi_context* ctx, void* d_dst, size_t dst_bytes, const void* h_src,
                            size_t src_bytes);
int32_t fi_buf_download_async(fi_context* ctx, void* h_dst, size_t dst_bytes, const void* d_src,
                              size_t src_bytes);
int32_t fi_ctx_faults_async(fi_context* ctx, uint32_t* h_words);
typedef struct fi_event fi_event;
int32_t fi_event_create(fi_context* ctx, fi_event** out);
int32_t fi_event_record(fi_context* ctx, fi_event* ev);
int32_t fi_event_wait(fi_event* ev);
int32_t fi_event_destroy(fi_event* ev);

/* Feeds one step's sampled token ids into the next step's input ids on the device:
 * ids[i] = prev_tokens[rows[i]] where rows[i] >= 0; other entries keep their value.  A row at or
 * beyond prev_count leaves its entry unchanged and is reported as Runtime by the next
 * fi_ctx_check_faults.  The device side of the reference's step_reference feeding the previous
 * sample (runtime/session.rs:246-262), for a host that enqueues the step before it has read the
 * sample back. */
int32_t fi_token_feed(fi_context* ctx, const int32_t* d_prev_tokens, int32_t prev_count,
                      const int32_t* d_rows, int32_t n, int32_t* d_ids);

/* ---------------------------------------------------------------- KV pool ops */

/* Scatters this step's K/V rows into the paged pool by slot_mapping, converting f32 to the
 * pool dtype (bf16: round-to-nearest-even).  Replaces KvCacheStorage::write_uncommitted_f32
 * and write_sequence_uncommitted_f32 (runtime/kv_cache.rs:48-62; paged write path
 * runtime/paged_kv.rs:583-631, 679-767).  Rows whose slot is negative are skipped; a slot
 * beyond num_blocks * block_size is skipped and reported as Runtime by the next
 * fi_ctx_check_faults(). */
int32_t fi_kv_append(fi_context* ctx, const float* d_key, const float* d_value,
                     const int64_t* d_slot_mapping, int32_t num_tokens, void* d_k_cache,
                     void* d_v_cache, int32_t kv_dtype, int32_t num_blocks, int32_t block_size,
                     int32_t num_kv_heads, int32_t head_dim);

/* Copies `num_tokens` leading token rows of block src_blocks[i] into dst_blocks[i] for
 * every pair (copy-on-write of a partially shared prefix block).  Replaces the page copy of
 * PagedKvCacheStorage::import_prefix_from (runtime/paged_kv.rs:329-389) for a block that
 * cannot be shared by id. */
int32_t fi_kv_copy_blocks(fi_context* ctx, void* d_k_cache, void* d_v_cache, int32_t kv_dtype,
                          const int32_t* d_src_blocks, const int32_t* d_dst_blocks,
                          const int32_t* d_token_counts, int32_t num_pairs, int32_t num_blocks,
                          int32_t block_size, int32_t num_kv_heads, int32_t head_dim);

/* Gathers the first `length` token rows of one sequence's K and V from the paged pool of one
 * layer into contiguous f32 [length, Hkv, D] tensors (bf16 pools widen exactly, bits << 16).
 * Replaces KvCacheStorage::read_prefix_f32 (runtime/kv_cache.rs:63) over paged storage:
 * PagedKvCacheStorage::read_prefix_f32 concatenating pages by block table
 * (runtime/paged_kv.rs:769-791, block_table at :260-314).  block_table holds the sequence's
 * num_table_blocks block ids in logical order; a length beyond num_table_blocks * block_size
 * is Runtime (the reference's "ran out of committed pages"), a negative one InvalidShape.
 * A block id outside the pool writes zero rows and is reported as Runtime by the next
 * fi_ctx_check_faults().  head_dim must be a multiple of 4 and the pools and outputs 16-byte
 * aligned. */
int32_t fi_kv_gather(fi_context* ctx, const void* d_k_cache, const void* d_v_cache, int32_t kv_dtype,
                     const int32_t* d_block_table, int32_t num_table_blocks, int32_t length,
                     int32_t num_blocks, int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                     float* d_k_out, float* d_v_out);

/* Reads and clears the context's device fault flags (out-of-range slots / token ids seen by
 * kernels since the last check); returns Runtime with a message when any was set.  Waits
 * for the stream. */
int32_t fi_ctx_check_faults(fi_context* ctx);

/* ---------------------------------------------------------------- attention */

/* Paged decode attention, one query token per sequence, all keys [0, context_len) read
 * through the block table (the current token's K/V must already be appended).
 * Split-KV over fixed partitions (512 tokens when Hkv * D >= 512, else 256) with a
 * log-sum-exp merge, so the summation order depends only on context_len and the model shape.  Replaces, per sequence, read_prefix_f32 +
 * cached_prefixed_causal_attention_f32 (runtime/reference.rs:497-508,
 * runtime/paged_kv.rs:769-791, kernel/cpu/attention.rs:332-518) and
 * decode_causal_attention_f32 (kernel/cpu/attention.rs:520-686).
 * q/out: f32 [num_seqs, Hq, D]; scale is 1/sqrt(D) in the reference (attention.rs:659).
 * max_context_len must bound every context_lens entry (it sizes the grid); an entry beyond
 * the partitions it sizes is clamped to them on device and reported as Runtime by
 * fi_ctx_check_faults. */
int32_t fi_attn_decode_paged(fi_context* ctx, const float* d_q, const void* d_k_cache,
                             const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                             int32_t max_blocks_per_seq, const int32_t* d_context_lens,
                             int32_t num_seqs, int32_t max_context_len, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t num_blocks, float scale, float* d_out);

/* A decode step's attention with the q|k|v consumer folded in: fi_qkv_rope_append followed by
 * fi_attn_decode_paged in one launch, for batches of one new token per sequence (sequence b's
 * token is row b of the projection).  Replaces the bias adds, rope_f32, the
 * KvCacheStorage::write_*_f32 append and the paged decode attention of the block
 * (runtime/reference.rs:163-300, 497-508; kernel/cpu/attention.rs:165-220, 332-686;
 * runtime/kv_cache.rs:48-62).  The arguments are those two calls' (the pools are written:
 * sequence b's new K/V row lands at slot_mapping[b], which must lie inside context_lens[b]
 * through the block table).  Every workgroup of the attention forms its query rows from
 * qkv_parts [splits, num_seqs, (Hq + 2 Hkv) * D] (+ biases, each may be NULL, + RoPE at
 * positions[b]); the workgroup holding a sequence's last partition appends the K/V row of its
 * kv head before reading the keys.  Launches of more than six workgroups a CU (large batches
 * of long contexts) run the two calls instead, with q_out [num_seqs, Hq, D] as the query
 * buffer between them; q_out is left unwritten otherwise.  Outputs and the pool contents
 * equal those of the two calls bit for bit either way.  rotary_dims / 2 and head_dim - rotary_dims must be multiples of 4
 * (Unsupported otherwise); the partials, biases and RoPE tables 16-byte aligned.  A slot or a
 * position out of range is reported as by fi_qkv_rope_append. */
int32_t fi_attn_decode_paged_qkv(fi_context* ctx, const float* d_qkv_parts, int32_t splits, const float* d_bias_q,
                                 const float* d_bias_k, const float* d_bias_v, const int32_t* d_positions,
                                 const float* d_cos, const float* d_sin, int32_t rotary_dims, int32_t max_positions,
                                 const int64_t* d_slot_mapping, void* d_k_cache, void* d_v_cache, int32_t kv_dtype,
                                 const int32_t* d_block_tables, int32_t max_blocks_per_seq,
                                 const int32_t* d_context_lens, int32_t num_seqs, int32_t max_context_len,
                                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 int32_t num_blocks, float scale, float* d_q_out, float* d_out);

/* fi_attn_decode_paged without any allocation: the same kernels, same arguments and bit-identical
 * outputs, with the split-KV partials in a fixed device array of this library (96 MiB per GPU,
 * part of the library's code object: every process that loads the library onto a GPU holds it
 * there, whether or not it calls this entry point, until the process exits)
 * instead of the grow-only context workspace.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  A launch whose partials (num_seqs * Hq * ceil(max_context_len /
 * partition) * (D + 2) * 4 bytes, when it has more than one partition) exceed the array is rejected
 * as Runtime.  Every call on one GPU shares the array, so calls that overlap on one GPU (several
 * streams or contexts) race; calls on one stream are ordered. */
int32_t fi_attn_decode_paged_noalloc(fi_context* ctx, const float* d_q, const void* d_k_cache,
                                     const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                                     int32_t max_blocks_per_seq, const int32_t* d_context_lens,
                                     int32_t num_seqs, int32_t max_context_len, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                     int32_t num_blocks, float scale, float* d_out);

/* Varlen causal prefill attention over the paged pool (MFMA).  Sequence b contributes
 * qlen_b = cu_seqlens[b+1] - cu_seqlens[b] query rows of q/out [T, Hq, D] at positions
 * [context_lens[b] - qlen_b, context_lens[b]); each attends keys [0, position] read through
 * block_tables (the chunk's own K/V rows must already be appended).  Replaces
 * causal_self_attention_f32 / cached_prefixed_causal_attention_f32 with the paged prefix
 * gather (kernel/cpu/attention.rs:222-518, runtime/reference.rs:425-465,
 * runtime/paged_kv.rs:769-791).  max_query_len must bound every qlen_b (it sizes the grid); a
 * longer qlen_b is reported as Runtime by fi_ctx_check_faults and its rows past the tiles that
 * max_query_len sized are left unwritten.  q, out and the pools must be 16-byte aligned
 * (InvalidLayout otherwise). */
int32_t fi_attn_prefill_paged(fi_context* ctx, const float* d_q, const void* d_k_cache,
                              const void* d_v_cache, int32_t kv_dtype,
                              const int32_t* d_block_tables, int32_t max_blocks_per_seq,
                              const int32_t* d_cu_seqlens, const int32_t* d_context_lens,
                              int32_t num_seqs, int32_t max_query_len, int32_t num_q_heads,
                              int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                              int32_t num_blocks, float scale, float* d_out);

/* fi_attn_prefill_paged over a bf16 pool on bf16 MFMA (v_mfma_f32_16x16x32_bf16): the queries
 * and the softmax probabilities are rounded to bf16 (nearest even) for the two products;
 * scores, softmax and accumulation stay f32.  The bf16-storage counterpart of the same
 * reference attention (within the bf16 tolerance of the f32-math path above), for callers
 * that store K/V in bf16 and want the bf16 MFMA rate. */
int32_t fi_attn_prefill_paged_bf16(fi_context* ctx, const float* d_q, const void* d_k_cache,
                                   const void* d_v_cache, const int32_t* d_block_tables,
                                   int32_t max_blocks_per_seq, const int32_t* d_cu_seqlens,
                                   const int32_t* d_context_lens, int32_t num_seqs, int32_t max_query_len,
                                   int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t block_size, int32_t num_blocks, float scale, float* d_out);

/* ---------------------------------------------------------------- decoder-block ops */

/* out[r, :] = table[ids[r], :].  Replaces embedding_gather_f32
 * (kernel/cpu/attention.rs:3-99).  An id >= vocab writes a zero row and is reported as
 * Runtime by fi_ctx_check_faults (the reference returns InvalidShape, attention.rs:35-40;
 * the host runtime validates ids before upload and raises that). */
int32_t fi_embedding(fi_context* ctx, const float* d_table, int32_t vocab, int32_t hidden,
                     const int32_t* d_ids, int32_t num_tokens, float* d_out);

/* RMSNorm over rows: ms = sum(x^2)/H, out = (x / sqrt(ms + eps)) * w.
 * Replaces rms_norm_f32 (kernel/cpu/reduction.rs:3-73). */
int32_t fi_rms_norm(fi_context* ctx, const float* d_x, const float* d_weight, float* d_out,
                    int32_t rows, int32_t hidden, float eps);

/* sum = a + residual (stored), out = rms_norm(sum) * w: the residual add_f32_in_place
 * followed by rms_norm_f32 of the decoder block (runtime/reference.rs:337-343, 827-833). */
int32_t fi_add_rms_norm(fi_context* ctx, const float* d_a, const float* d_residual, float* d_sum,
                        const float* d_weight, float* d_out, int32_t rows, int32_t hidden,
                        float eps);

/* Builds the RoPE cos/sin tables [max_positions, rotary_dims/2] on the host with the
 * reference's loop (iterated f32 inverse frequency with exponent -2/head_dim, glibc sin/cos,
 * kernel/cpu/attention.rs:1253-1277) and uploads them.  Validation as rope_f32
 * (attention.rs:190-209). */
int32_t fi_rope_table(fi_context* ctx, int32_t max_positions, int32_t head_dim,
                      int32_t rotary_dims, float theta, float* d_cos, float* d_sin);

/* Rotates q [T, Hq, D] and k [T, Hkv, D] in place at per-token positions (NeoX half
 * split, products rounded before the add).  Replaces rope_f32 with position_offset
 * (kernel/cpu/attention.rs:165-220) for a ragged batch; bit-identical to the reference.  A
 * position outside [0, max_positions) leaves its token unrotated and is reported as Runtime by
 * fi_ctx_check_faults (as in fi_qkv_rope_append). */
int32_t fi_rope(fi_context* ctx, float* d_q, float* d_k, const int32_t* d_positions,
                const float* d_cos, const float* d_sin, int32_t num_tokens, int32_t num_q_heads,
                int32_t num_kv_heads, int32_t head_dim, int32_t rotary_dims,
                int32_t max_positions);

/* SwiGLU: out = up * (gate * (1 / (1 + exp(-gate)))); out may alias up or gate.  Replaces silu_f32_in_place +
 * mul_f32_in_place (kernel/cpu/elementwise.rs:118-207; use at runtime/reference.rs:346-360). */
int32_t fi_silu_mul(fi_context* ctx, const float* d_up, const float* d_gate, float* d_out,
                    int64_t n);

/* out = a + b.  Replaces add_f32_in_place (kernel/cpu/elementwise.rs:48-76). */
int32_t fi_add(fi_context* ctx, const float* d_a, const float* d_b, float* d_out, int64_t n);

/* ---------------------------------------------------------------- projections */

/* C[M,N] = A[M,K] * B (+ bias[N]) on MFMA (f32 in, f32 accumulate).  b_layout 0: B is
 * [K, N] = the reference's [in, out] weight (matmul_f32 + bias add of linear_f32_with_bias,
 * kernel/cpu/matmul.rs:46-118, runtime/reference.rs:1135-1191); b_layout 1: B is [N, K]
 * (matmul_rhs_transposed_f32, kernel/cpu/matmul.rs:120-188: the lm_head logits against the
 * [vocab, hidden] output or tied embedding weight).  Skinny shapes split K across
 * workgroups and sum the splits in a fixed order (deterministic); the split partials use
 * the context workspace. */
int32_t fi_gemm(fi_context* ctx, const float* d_a, const float* d_b, const float* d_bias,
                float* d_c, int32_t m, int32_t k, int32_t n, int32_t b_layout);

/* Fused greedy head: for each of m rows, logits = hidden_row * W^T with W [vocab, hidden],
 * returns the FIRST index of the maximum logit and 1 / sum(exp(logit - max)).  Replaces
 * matmul_rhs_transposed_argmax_f32 (kernel/cpu/matmul.rs:190-274, 532-589): strict > within a
 * tile, ties between tiles keep the left one.  Logits are never materialised.  The
 * probability's rounding depends on the tiling, as the reference's depends on its thread
 * chunks (matmul.rs:232-270). */
int32_t fi_lm_head_argmax(fi_context* ctx, const float* d_hidden, const float* d_weight,
                          int32_t m, int32_t hidden, int32_t vocab, int32_t* d_token,
                          float* d_prob);

/* ---------------------------------------------------------------- packed-weight path
 *
 * The decoder block's projections (matmul_f32 / linear_f32_with_bias over [in, out]
 * weights, kernel/cpu/matmul.rs:46-118, runtime/reference.rs:1103-1191) on weights re-laid
 * out once at upload, which the architecture assigns to the GPU backend
 * (docs/architecture.md:53, 97).  Packed layout: slabs of 16*pack_width output columns, each
 * holding its K rows (zero-padded to a multiple of 16) in MFMA fragment order, so a wave
 * streams a slab with contiguous 16-byte loads.  Pack width 32 selects a 32-column layout
 * whose lanes hold eight consecutive k of one column per 16-k step (32 contiguous bytes);
 * fi_gemm_packed then multiplies in f32 accuracy on bf16 MFMA, both operands split exactly
 * into three bf16 pieces and the six cross products above 2^-24 relative accumulated in f32.
 * fi_gemm_packed writes split-K partials [splits, M, N]; the consumers below sum them in split
 * order (deterministic) and fuse the elementwise ops the reference runs after each
 * projection. */

/* Floats of the packed form of a [K, N] weight. */
int32_t fi_weight_packed_floats(int32_t k, int32_t n, int32_t pack_width, size_t* floats);

/* Packs a device weight: src_layout 0 = [K, N] ([in, out], model/decoder.rs:76-104),
 * 1 = [N, K] (the [vocab, hidden] output / tied embedding weight of matmul_rhs_transposed,
 * kernel/cpu/matmul.rs:120-188).  pack_width 1, 2, 4 or 32. */
int32_t fi_weight_pack(fi_context* ctx, const float* d_src, int32_t src_layout, int32_t k, int32_t n,
                       int32_t pack_width, float* d_dst);

/* Packs the column concatenation of up to three [K, ns[i]] weights (the q, k, v projections
 * of one layer as a single [H, (Hq + 2 Hkv) * D] matrix).  d_srcs is a host array of device
 * pointers. */
int32_t fi_weight_pack_columns(fi_context* ctx, const float* const* d_srcs, const int32_t* ns, int32_t count,
                               int32_t k, int32_t pack_width, float* d_dst);

/* SwiGLU pair pack (pack width 2) of the up (w1) and gate (w3) weights, both [K, N]: each
 * lane vector holds (up, gate) of one output column. */
int32_t fi_weight_pack_pair(fi_context* ctx, const float* d_first, const float* d_second, int32_t k, int32_t n,
                            float* d_dst);

/* The split count fi_gemm_packed should use for an M x K x N product (enough workgroups to
 * fill the device, every split non-empty). */
int32_t fi_gemm_packed_splits(fi_context* ctx, int32_t m, int32_t k, int32_t n, int32_t pack_width,
                              int32_t* splits);

/* d_out[z] = A * B restricted to split z's K range, z < splits; A [M, K] row-major with row
 * stride lda (a multiple of 4, 16-byte aligned rows).  Sum the splits in order (the consumers
 * do) for matmul_f32 (kernel/cpu/matmul.rs:46-118). */
int32_t fi_gemm_packed(fi_context* ctx, const float* d_a, int32_t lda, const float* d_bp, int32_t k, int32_t n,
                       int32_t pack_width, int32_t m, int32_t splits, float* d_out);

/* out[M, N] = (A W1 + b1) * silu(A W3 + b3) with the pair-packed weight: the up / gate
 * projections, silu_f32_in_place and mul_f32_in_place of the decoder block
 * (runtime/reference.rs:346-360, kernel/cpu/elementwise.rs:118-207) in one launch. */
int32_t fi_gemm_packed_swiglu(fi_context* ctx, const float* d_a, int32_t lda, const float* d_bp_pair, int32_t k,
                              int32_t n, int32_t m, const float* d_bias_up, const float* d_bias_gate, float* d_out);

/* fi_lm_head_argmax over a weight packed from its [vocab, hidden] layout with pack width 2
 * (matmul_rhs_transposed_argmax_f32, kernel/cpu/matmul.rs:190-274): first maximal index
 * and 1 / sum(exp(logit - max)) per row.  Uses the context workspace. */
int32_t fi_lm_head_argmax_packed(fi_context* ctx, const float* d_hidden, int32_t lda, const float* d_bp, int32_t m,
                                 int32_t hidden, int32_t vocab, int32_t* d_token, float* d_prob);

/* sum = (sum_z parts[z] + bias) + residual (stored), out = rms_norm(sum) * weight: the
 * projection's bias add, the residual add_f32_in_place and the next rms_norm_f32 of the
 * decoder block (runtime/reference.rs:330-343, 362-368; kernel/cpu/reduction.rs:3-73).
 * parts is [splits, rows, hidden]; bias may be NULL. */
int32_t fi_splitk_residual_rms_norm(fi_context* ctx, const float* d_parts, int32_t splits, const float* d_bias,
                                    const float* d_residual, float* d_sum, const float* d_weight, float* d_out,
                                    int32_t rows, int32_t hidden, float eps);

/* The fused QKV projection's split partials [splits, T, (Hq + 2 Hkv) * D] (+ q/k/v biases,
 * each may be NULL) -> RoPE of q and k at positions (bit-identical to fi_rope) -> q to
 * d_q_out [T, Hq, D], k and v appended to the pool by slot_mapping (as fi_kv_append).
 * Replaces the bias adds, rope_f32 and KvCacheStorage::write_*_f32 of the block
 * (runtime/reference.rs:163-300, kernel/cpu/attention.rs:165-220, runtime/kv_cache.rs:48-62). */
int32_t fi_qkv_rope_append(fi_context* ctx, const float* d_parts, int32_t splits, const float* d_bias_q,
                           const float* d_bias_k, const float* d_bias_v, const int32_t* d_positions,
                           const float* d_cos, const float* d_sin, int32_t rotary_dims, int32_t max_positions,
                           const int64_t* d_slot_mapping, void* d_k_cache, void* d_v_cache, int32_t kv_dtype,
                           int32_t num_blocks, int32_t block_size, int32_t num_tokens, int32_t num_q_heads,
                           int32_t num_kv_heads, int32_t head_dim, float* d_q_out);

/* ---- Projections over bf16-stored weights (bf16 configurations) ----
 * The reference loads bf16 weights by exact widening (io/safetensors.rs:540-542) and runs the
 * f32 kernels; this path keeps the weights bf16 in HBM, packed for v_mfma_f32_16x16x32_bf16,
 * rounds the f32 activations to bf16 (nearest even) and accumulates in f32.  The outputs use
 * the formats of the f32 packed path above, so the same consumers sum the split partials.
 * Activations (a_dtype) may also be given as bf16 bits already rounded to nearest even (by
 * fi_convert_f32_to_bf16, fi_splitk_residual_rms_norm_bf16 or a bf16 SwiGLU output): the
 * products are then bit-identical to the f32 call, and the kernels read half the activation
 * bytes. */

/* bf16 elements of the packed form of a [K, N] weight (pair != 0: the up/gate pair of two
 * [K, N] weights). */
int32_t fi_weight_packed_bf16_elems(int32_t k, int32_t n, int32_t pair, size_t* elems);

/* Packs a device weight given as f32 (rounded to nearest even) or bf16 bits (src_dtype):
 * src_layout 0 = [K, N] ([in, out], model/decoder.rs:76-104), 1 = [N, K] (the tied
 * [vocab, hidden] weight of matmul_rhs_transposed, kernel/cpu/matmul.rs:120-188). */
int32_t fi_weight_pack_bf16(fi_context* ctx, const void* d_src, int32_t src_dtype, int32_t src_layout, int32_t k,
                            int32_t n, uint16_t* d_dst);

/* Column concatenation of up to three [K, ns[i]] weights (the fused q|k|v projection).  d_srcs
 * is a host array of device pointers. */
int32_t fi_weight_pack_bf16_columns(fi_context* ctx, const void* const* d_srcs, const int32_t* ns, int32_t count,
                                    int32_t src_dtype, int32_t k, uint16_t* d_dst);

/* SwiGLU pair pack of the up (w1) and gate (w3) weights, both [K, N]. */
int32_t fi_weight_pack_bf16_pair(fi_context* ctx, const void* d_up, const void* d_gate, int32_t src_dtype, int32_t k,
                                 int32_t n, uint16_t* d_dst);

/* The split count fi_gemm_bf16 should use for an M x K x N product. */
int32_t fi_gemm_bf16_splits(fi_context* ctx, int32_t m, int32_t k, int32_t n, int32_t* splits);

/* d_out[z] = A * W over split z's K range (as fi_gemm_packed): matmul_f32 / linear_f32_with_bias
 * (kernel/cpu/matmul.rs:46-118, 424-499) with bf16 operands and f32 accumulation.  A [M, K] of
 * a_dtype (FI_DTYPE_F32 or FI_DTYPE_BF16) with row stride lda in elements (f32: a multiple of 4,
 * at least K rounded up to 4; bf16: a multiple of 8, at least K rounded up to 8; 16-byte
 * aligned rows). */
int32_t fi_gemm_bf16(fi_context* ctx, const void* d_a, int32_t a_dtype, int32_t lda, const uint16_t* d_bp, int32_t k,
                     int32_t n, int32_t m, int32_t splits, float* d_out);

/* out[M, N] = (A W1 + b1) * silu(A W3 + b3) over the pair-packed bf16 weight (the decoder
 * block's up/gate projections and SwiGLU, runtime/reference.rs:346-360,
 * kernel/cpu/elementwise.rs:118-207).  A as for fi_gemm_bf16; out_dtype FI_DTYPE_F32 or
 * FI_DTYPE_BF16 (the f32 result rounded to nearest even, the input of a bf16-activation
 * fi_gemm_bf16).  Uses the context workspace when K is split. */
int32_t fi_gemm_bf16_swiglu(fi_context* ctx, const void* d_a, int32_t a_dtype, int32_t lda, const uint16_t* d_bp_pair,
                            int32_t k, int32_t n, int32_t m, const float* d_bias_up, const float* d_bias_gate,
                            void* d_out, int32_t out_dtype);

/* Greedy head over a bf16 weight packed from its [vocab, hidden] layout
 * (matmul_rhs_transposed_argmax_f32, kernel/cpu/matmul.rs:190-274): first maximal index and
 * 1 / sum(exp(logit - max)) per row.  Uses the context workspace. */
int32_t fi_lm_head_argmax_bf16(fi_context* ctx, const void* d_hidden, int32_t a_dtype, int32_t lda,
                               const uint16_t* d_bp, int32_t m, int32_t hidden, int32_t vocab, int32_t* d_token,
                               float* d_prob);

/* fi_splitk_residual_rms_norm with the normalised output stored as bf16 bits, each value the
 * f32 result rounded to nearest even (the sum stays f32): the producer of bf16 activations for
 * fi_gemm_bf16 / fi_gemm_bf16_swiglu.  d_out 8-byte aligned when hidden is a multiple of 4. */
int32_t fi_splitk_residual_rms_norm_bf16(fi_context* ctx, const float* d_parts, int32_t splits, const float* d_bias,
                                         const float* d_residual, float* d_sum, const float* d_weight,
                                         uint16_t* d_out, int32_t rows, int32_t hidden, float eps);

/* d_dst[i] = bf16 bits of d_src[i] rounded to nearest even (NaN stays NaN), n elements; the
 * narrowing of f32 activations for the bf16 projections.  Source and destination must not
 * overlap. */
int32_t fi_convert_f32_to_bf16(fi_context* ctx, const float* d_src, int64_t n, uint16_t* d_dst);

/* ---------------------------------------------------------------- sampling */

/* Samples one token per logits row on the device: sample_last_token
 * (runtime/sampler.rs:121-241) for row r's configuration (d_temperature[r], d_top_k[r],
 * d_top_p[r]), or argmax_last_token (sampler.rs:77-119) when that configuration is greedy
 * (SamplerConfig::is_greedy, sampler.rs:40-42: temperature <= 0, top_k == 1 or top_p <= 0).
 * d_logits [rows, ld] f32 holds each sequence's last-token logits (the row the reference takes
 * from [seq_len, vocab]); d_rng_state[r] is row r's SamplerState (sampler.rs:51-75; seed 0 maps
 * to 0x9e3779b97f4a7c15 when the state is created), advanced by one draw for a sampled row and
 * left as it is for a greedy row.  Writes the token id and its probability (weight / retained
 * total, or 1 / sum exp(l - max) when greedy).  top_k below 1 counts as 1 (usize::max(1)).  A
 * top_k above 1024 after clamping to the vocabulary is served, up to the whole vocabulary, when
 * fi_sample_reserve has set aside room for at least this call's rows and vocab; otherwise such
 * a row, like a distribution whose total weight is not finite and positive
 * (sampler.rs:195-200, Runtime), writes token -1 and is reported as Runtime by the next
 * fi_ctx_check_faults().  Probabilities may differ from the host's in the last bits (device
 * expf); tokens are the reference's. */
int32_t fi_sample_tokens(fi_context* ctx, const float* d_logits, int32_t ld, int32_t rows, int32_t vocab,
                         const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                         uint64_t* d_rng_state, int32_t* d_token, float* d_prob);

/* Sets aside device memory (about 16 bytes per logit per row; grow-only, freed with the
 * context) so that fi_sample_tokens serves rows whose clamped top_k exceeds 1024 in calls of
 * up to `rows` rows of `vocab` logits (vocab at most 1048576, else Unsupported).  The same
 * top_k field of SamplerConfig (runtime/sampler.rs:3-10, 152-172) is taken up to the
 * vocabulary by the reference; device-side configurations need the room reserved on the host
 * beforehand.  Not during graph capture; a reallocation bumps fi_ctx_workspace_generation. */
int32_t fi_sample_reserve(fi_context* ctx, int32_t rows, int32_t vocab);

/* ---------------------------------------------------------------- checkpoint import
 * d_dst = the f32 widening of d_src, a [rows, cols] row-major tensor of src_dtype (FI_DTYPE_F32,
 * _BF16 or _F16; rank-1 tensors as rows = 1); transpose != 0 writes the [cols, rows] transpose
 * (dst[c * rows + r] = src[r * cols + c]).  BF16 widens as bits << 16; F16 by the IEEE rule
 * (subnormals normalised, infinities and NaN payloads kept).  Replaces the host conversion of
 * io/safetensors.rs:437-471 (convert_to_f32_vec, transpose_2d) and :538-568 (bf16_to_f32,
 * f16_to_f32).  d_src and d_dst must not overlap. */
int32_t fi_convert_to_f32(fi_context* ctx, const void* d_src, int32_t src_dtype, int64_t rows, int64_t cols,
                          int32_t transpose, float* d_dst);

#ifdef __cplusplus
}
#endif

#endif /* FERRISINFER_KERNEL_H */
