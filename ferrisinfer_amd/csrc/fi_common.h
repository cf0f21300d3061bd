// Internal definitions shared by the HIP translation units of libferrisinfer_kernel.so.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "../../include/ferrisinfer_kernel.h"

// Device-side fault bits (kernels OR them into fi_context::d_faults).
enum : uint32_t {
  FI_FAULT_SLOT_RANGE = 1u << 0,   // kv append: slot beyond the pool
  FI_FAULT_TOKEN_RANGE = 1u << 1,  // embedding: token id beyond the vocabulary
  FI_FAULT_BLOCK_RANGE = 1u << 2,  // attention: block id beyond the pool
  FI_FAULT_SAMPLE_TOPK = 1u << 3,       // sampling: top_k (after clamping to the vocabulary) above 1024
  FI_FAULT_SAMPLE_NONFINITE = 1u << 4,  // sampling: the candidate weights do not sum to a finite, positive total
  FI_FAULT_CONTEXT_RANGE = 1u << 5,     // decode attention: a context length beyond the partitions max_context_len sized
  FI_FAULT_QUERY_RANGE = 1u << 6,       // prefill attention: a query length beyond the tiles max_query_len sized
  FI_FAULT_POSITION_RANGE = 1u << 7,    // RoPE: a position outside the cos/sin table
};

// Arrival counters a context holds for decode attention's in-kernel merge: launches with more
// (sequence, kv head) groups than this merge in a separate launch.
#define FI_MERGE_COUNTERS 65536

struct fi_context {
  int device = 0;
  hipStream_t own_stream = nullptr;
  hipStream_t stream = nullptr;
  uint32_t* d_faults = nullptr;  // [4] fault words, zeroed at create and by check_faults
  void* workspace = nullptr;     // grow-only scratch for split-KV partials
  size_t workspace_bytes = 0;
  int compute_units = 0;
  void* noalloc_scratch = nullptr;  // this device's address of the library's fixed decode scratch array
  uint64_t workspace_generation = 0;  // bumped whenever the workspace or the sampling area is reallocated
  bool capturing = false;             // the stream is being captured into a graph
  void* sample_area = nullptr;        // fi_sample_reserve: per-row sort and replay arrays for top-k above 1024
  size_t sample_bytes = 0;
  // decode attention: arrival counters of the split-KV merge, one per (sequence, kv head),
  // FI_MERGE_COUNTERS of them, zeroed at create; each launch leaves them zero
  unsigned* d_merge_counters = nullptr;
};

// A captured and instantiated launch sequence of one context's stream.
struct fi_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  int device = 0;
};

struct fi_event {
  hipEvent_t event = nullptr;
  int device = 0;
};

namespace fi {

// Records `message` as the thread's last error and returns `code`.
int32_t set_error(int32_t code, const std::string& message);

// Maps a HIP error to Runtime with "<call> returned HIP error N (name)", the shape of
// cuda_check (kernel/gpu/nvidia.rs:887-904).
int32_t hip_error(hipError_t err, const char* call);

// Makes ctx's device current; returns a status.
int32_t enter(fi_context* ctx);

// Ensures ctx->workspace holds at least `bytes` (grow-only; never shrinks).
int32_t ensure_workspace(fi_context* ctx, size_t bytes);

// Looks up (once per device, with ctx's device current) the device address of the fixed
// split-KV scratch array used by fi_attn_decode_paged_noalloc and stores it in ctx.
int32_t decode_noalloc_attach(fi_context* ctx);

// Split-KV decode partials for the given launch shape.
int32_t decode_scratch(fi_context* ctx, int32_t num_seqs, int32_t hq, int32_t parts, int32_t head_dim,
                       float** part_acc, float** part_ml);

// Reduces per-tile greedy-head states [m, n_tiles, 3] (max, index bits, scaled sum) to the
// first maximal index and 1 / sum per row.
int32_t argmax_merge(fi_context* ctx, const float* amax, int32_t n_tiles, int32_t m, int32_t* token, float* prob);

// out[M, N] = (sum_z up + bias_up) * silu(sum_z gate + bias_gate) over split partials
// [splits, M, 2N] holding (up c, gate c) at columns (2c, 2c + 1).
int32_t splitk_swiglu(fi_context* ctx, const float* parts, int32_t splits, const float* bias_up,
                      const float* bias_gate, int32_t m, int32_t n, void* out, bool out_bf16);

}  // namespace fi

#define FI_TRY_HIP(call)                                 \
  do {                                                   \
    hipError_t fi_err_ = (call);                         \
    if (fi_err_ != hipSuccess) return fi::hip_error(fi_err_, #call); \
  } while (0)

#define FI_TRY(expr)                \
  do {                              \
    int32_t fi_st_ = (expr);        \
    if (fi_st_ != FI_OK) return fi_st_; \
  } while (0)

#define FI_REQUIRE(cond, code, msg) \
  do {                              \
    if (!(cond)) return fi::set_error((code), (msg)); \
  } while (0)

// Launch-error check after a kernel launch.
#define FI_CHECK_LAUNCH(name)                                 \
  do {                                                        \
    hipError_t fi_err_ = hipGetLastError();                   \
    if (fi_err_ != hipSuccess) return fi::hip_error(fi_err_, name); \
  } while (0)
