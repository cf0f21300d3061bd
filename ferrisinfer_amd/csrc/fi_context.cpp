// Context, errors and device memory of libferrisinfer_kernel.so (host code only).
// Mirrors the lifecycle and error shape of the reference's NVIDIA driver layer
// (crates/ferrisinfer-kernel/src/gpu/nvidia.rs) on the HIP runtime.
#include <cstring>
#include <string>

#include "fi_common.h"

namespace {
thread_local std::string g_last_error;
}

namespace fi {

int32_t set_error(int32_t code, const std::string& message) {
  g_last_error = message;
  return code;
}

int32_t hip_error(hipError_t err, const char* call) {
  return set_error(FI_ERR_RUNTIME, std::string(call) + " returned HIP error " +
                                       std::to_string(static_cast<int>(err)) + " (" +
                                       hipGetErrorName(err) + ")");
}

int32_t enter(fi_context* ctx) {
  FI_REQUIRE(ctx != nullptr, FI_ERR_INVALID_CONFIG, "null fi_context");
  FI_TRY_HIP(hipSetDevice(ctx->device));
  return FI_OK;
}

int32_t ensure_workspace(fi_context* ctx, size_t bytes) {
  if (bytes <= ctx->workspace_bytes) return FI_OK;
  // A graph being captured would keep the old address; growing is refused instead (the caller
  // runs the launch once outside capture first, which sizes the workspace).
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME,
             "the context workspace would grow during graph capture (needs " + std::to_string(bytes) +
                 " bytes, holds " + std::to_string(ctx->workspace_bytes) + ")");
  if (ctx->workspace != nullptr) {
    // The old workspace may still be read by queued kernels.
    FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
    FI_TRY_HIP(hipFree(ctx->workspace));
    ctx->workspace = nullptr;
    ctx->workspace_bytes = 0;
  }
  size_t rounded = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
  FI_TRY_HIP(hipMalloc(&ctx->workspace, rounded));
  ctx->workspace_bytes = rounded;
  ctx->workspace_generation += 1;
  return FI_OK;
}

}  // namespace fi

extern "C" {

const char* fi_last_error(void) { return g_last_error.c_str(); }

int32_t fi_ctx_create(int32_t ordinal, fi_context** out) {
  FI_REQUIRE(out != nullptr, FI_ERR_INVALID_CONFIG, "fi_ctx_create: null output pointer");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count == 0) {
    return fi::set_error(FI_ERR_UNSUPPORTED, "no HIP device is available");
  }
  FI_REQUIRE(ordinal >= 0 && ordinal < count, FI_ERR_INVALID_CONFIG,
             "device ordinal " + std::to_string(ordinal) + " out of range (" +
                 std::to_string(count) + " devices)");
  FI_TRY_HIP(hipSetDevice(ordinal));
  hipDeviceProp_t prop;
  FI_TRY_HIP(hipGetDeviceProperties(&prop, ordinal));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return fi::set_error(FI_ERR_UNSUPPORTED, std::string("libferrisinfer_kernel is built for gfx950, device is ") +
                                                 prop.gcnArchName);
  }
  auto* ctx = new fi_context();
  ctx->device = ordinal;
  ctx->compute_units = prop.multiProcessorCount;
  hipError_t err = hipStreamCreate(&ctx->own_stream);
  if (err != hipSuccess) {
    delete ctx;
    return fi::hip_error(err, "hipStreamCreate");
  }
  ctx->stream = ctx->own_stream;
  err = hipMalloc(&ctx->d_faults, 4 * sizeof(uint32_t));
  if (err == hipSuccess) err = hipMemset(ctx->d_faults, 0, 4 * sizeof(uint32_t));
  if (err != hipSuccess) {
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return fi::hip_error(err, "hipMalloc(fault flags)");
  }
  err = hipMalloc(&ctx->d_merge_counters, FI_MERGE_COUNTERS * sizeof(unsigned));
  if (err == hipSuccess) err = hipMemset(ctx->d_merge_counters, 0, FI_MERGE_COUNTERS * sizeof(unsigned));
  if (err != hipSuccess) {
    if (ctx->d_merge_counters) (void)hipFree(ctx->d_merge_counters);
    (void)hipFree(ctx->d_faults);
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return fi::hip_error(err, "hipMalloc(merge counters)");
  }
  int32_t st = fi::decode_noalloc_attach(ctx);
  if (st != FI_OK) {
    (void)hipFree(ctx->d_merge_counters);
    (void)hipFree(ctx->d_faults);
    (void)hipStreamDestroy(ctx->own_stream);
    delete ctx;
    return st;
  }
  *out = ctx;
  return FI_OK;
}

int32_t fi_ctx_destroy(fi_context* ctx) {
  if (ctx == nullptr) return FI_OK;
  FI_TRY(fi::enter(ctx));
  if (ctx->capturing) {  // a capture left open: end and discard it
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(ctx->stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
    ctx->capturing = false;
  }
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->workspace) (void)hipFree(ctx->workspace);
  if (ctx->sample_area) (void)hipFree(ctx->sample_area);
  if (ctx->d_faults) (void)hipFree(ctx->d_faults);
  if (ctx->d_merge_counters) (void)hipFree(ctx->d_merge_counters);
  if (ctx->own_stream) (void)hipStreamDestroy(ctx->own_stream);
  delete ctx;
  return FI_OK;
}

int32_t fi_ctx_sync(fi_context* ctx) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_ctx_sync: the stream is being captured into a graph");
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  return FI_OK;
}

int32_t fi_ctx_set_stream(fi_context* ctx, void* stream) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_ctx_set_stream: the stream is being captured");
  ctx->stream = stream ? static_cast<hipStream_t>(stream) : ctx->own_stream;
  return FI_OK;
}

void* fi_ctx_stream(fi_context* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int32_t fi_device_info(fi_context* ctx, char* name, size_t name_len, char* arch, size_t arch_len,
                       uint64_t* hbm_bytes, int32_t* compute_units) {
  FI_TRY(fi::enter(ctx));
  hipDeviceProp_t prop;
  FI_TRY_HIP(hipGetDeviceProperties(&prop, ctx->device));
  if (name && name_len) {
    std::strncpy(name, prop.name, name_len - 1);
    name[name_len - 1] = '\0';
  }
  if (arch && arch_len) {
    std::strncpy(arch, prop.gcnArchName, arch_len - 1);
    arch[arch_len - 1] = '\0';
  }
  if (hbm_bytes) *hbm_bytes = prop.totalGlobalMem;
  if (compute_units) *compute_units = prop.multiProcessorCount;
  return FI_OK;
}

int32_t fi_buf_alloc(fi_context* ctx, size_t bytes, void** d_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_buf_alloc: the stream is being captured into a graph");
  FI_REQUIRE(d_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_buf_alloc: null output pointer");
  FI_REQUIRE(bytes > 0, FI_ERR_INVALID_SHAPE, "device buffers must be larger than zero bytes");
  FI_TRY_HIP(hipMalloc(d_out, bytes));
  return FI_OK;
}

int32_t fi_buf_free(fi_context* ctx, void* d_ptr) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_buf_free: the stream is being captured into a graph");
  if (d_ptr == nullptr) return FI_OK;
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  FI_TRY_HIP(hipFree(d_ptr));
  return FI_OK;
}

int32_t fi_buf_upload(fi_context* ctx, void* d_dst, size_t dst_bytes, const void* src,
                      size_t src_bytes) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_buf_upload: the stream is being captured into a graph");
  FI_REQUIRE(dst_bytes == src_bytes, FI_ERR_INVALID_SHAPE,
             "upload requires matching lengths; buffer has " + std::to_string(dst_bytes) +
                 " bytes but host slice has " + std::to_string(src_bytes) + " bytes");
  if (src_bytes == 0) return FI_OK;
  FI_TRY_HIP(hipMemcpyAsync(d_dst, src, src_bytes, hipMemcpyHostToDevice, ctx->stream));
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  return FI_OK;
}

int32_t fi_buf_download(fi_context* ctx, void* dst, size_t dst_bytes, const void* d_src,
                        size_t src_bytes) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_buf_download: the stream is being captured into a graph");
  FI_REQUIRE(dst_bytes == src_bytes, FI_ERR_INVALID_SHAPE,
             "download requires matching lengths; host slice has " + std::to_string(dst_bytes) +
                 " bytes but buffer has " + std::to_string(src_bytes) + " bytes");
  if (src_bytes == 0) return FI_OK;
  FI_TRY_HIP(hipMemcpyAsync(dst, d_src, src_bytes, hipMemcpyDeviceToHost, ctx->stream));
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  return FI_OK;
}

// ---------------------------------------------------------------- stream overlap
// Pinned host memory, copies that return once enqueued, and events: what a host runtime needs
// to enqueue the next step while the device still runs the current one.

int32_t fi_host_alloc(fi_context* ctx, size_t bytes, void** h_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_host_alloc: the stream is being captured into a graph");
  FI_REQUIRE(h_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_host_alloc: null output pointer");
  FI_REQUIRE(bytes > 0, FI_ERR_INVALID_SHAPE, "host buffers must be larger than zero bytes");
  FI_TRY_HIP(hipHostMalloc(h_out, bytes, hipHostMallocDefault));
  return FI_OK;
}

int32_t fi_host_free(fi_context* ctx, void* h_ptr) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_host_free: the stream is being captured into a graph");
  if (h_ptr == nullptr) return FI_OK;
  // queued copies may still read or write it
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  FI_TRY_HIP(hipHostFree(h_ptr));
  return FI_OK;
}

int32_t fi_buf_upload_async(fi_context* ctx, void* d_dst, size_t dst_bytes, const void* h_src,
                            size_t src_bytes) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_buf_upload_async: the stream is being captured into a graph");
  FI_REQUIRE(dst_bytes == src_bytes, FI_ERR_INVALID_SHAPE,
             "upload requires matching lengths; buffer has " + std::to_string(dst_bytes) +
                 " bytes but host slice has " + std::to_string(src_bytes) + " bytes");
  if (src_bytes == 0) return FI_OK;
  FI_REQUIRE(d_dst && h_src, FI_ERR_INVALID_CONFIG, "fi_buf_upload_async: null pointer");
  FI_TRY_HIP(hipMemcpyAsync(d_dst, h_src, src_bytes, hipMemcpyHostToDevice, ctx->stream));
  return FI_OK;
}

int32_t fi_buf_download_async(fi_context* ctx, void* h_dst, size_t dst_bytes, const void* d_src,
                              size_t src_bytes) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_buf_download_async: the stream is being captured into a graph");
  FI_REQUIRE(dst_bytes == src_bytes, FI_ERR_INVALID_SHAPE,
             "download requires matching lengths; host slice has " + std::to_string(dst_bytes) +
                 " bytes but buffer has " + std::to_string(src_bytes) + " bytes");
  if (src_bytes == 0) return FI_OK;
  FI_REQUIRE(h_dst && d_src, FI_ERR_INVALID_CONFIG, "fi_buf_download_async: null pointer");
  FI_TRY_HIP(hipMemcpyAsync(h_dst, d_src, src_bytes, hipMemcpyDeviceToHost, ctx->stream));
  return FI_OK;
}

int32_t fi_ctx_faults_async(fi_context* ctx, uint32_t* h_words) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_ctx_faults_async: the stream is being captured into a graph");
  FI_REQUIRE(h_words != nullptr, FI_ERR_INVALID_CONFIG, "fi_ctx_faults_async: null pointer");
  FI_TRY_HIP(hipMemcpyAsync(h_words, ctx->d_faults, 4 * sizeof(uint32_t), hipMemcpyDeviceToHost, ctx->stream));
  return FI_OK;
}

int32_t fi_event_create(fi_context* ctx, fi_event** out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(out != nullptr, FI_ERR_INVALID_CONFIG, "fi_event_create: null output pointer");
  hipEvent_t e = nullptr;
  FI_TRY_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  auto* ev = new fi_event();
  ev->event = e;
  ev->device = ctx->device;
  *out = ev;
  return FI_OK;
}

int32_t fi_event_record(fi_context* ctx, fi_event* ev) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(ev != nullptr && ev->device == ctx->device, FI_ERR_INVALID_CONFIG,
             "fi_event_record: event of another device or null");
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_event_record: the stream is being captured into a graph");
  FI_TRY_HIP(hipEventRecord(ev->event, ctx->stream));
  return FI_OK;
}

int32_t fi_event_wait(fi_event* ev) {
  FI_REQUIRE(ev != nullptr, FI_ERR_INVALID_CONFIG, "fi_event_wait: null event");
  FI_TRY_HIP(hipSetDevice(ev->device));
  FI_TRY_HIP(hipEventSynchronize(ev->event));
  return FI_OK;
}

int32_t fi_event_destroy(fi_event* ev) {
  if (ev == nullptr) return FI_OK;
  FI_TRY_HIP(hipSetDevice(ev->device));
  hipError_t err = hipEventDestroy(ev->event);
  delete ev;
  if (err != hipSuccess) return fi::hip_error(err, "hipEventDestroy");
  return FI_OK;
}

int32_t fi_ctx_workspace_generation(fi_context* ctx, uint64_t* generation) {
  FI_REQUIRE(ctx != nullptr && generation != nullptr, FI_ERR_INVALID_CONFIG,
             "fi_ctx_workspace_generation: null argument");
  *generation = ctx->workspace_generation;
  return FI_OK;
}

int32_t fi_graph_begin(fi_context* ctx) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_graph_begin: a capture is already open");
  FI_REQUIRE(ctx->stream != nullptr, FI_ERR_UNSUPPORTED, "fi_graph_begin: the null stream cannot be captured");
  FI_TRY_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal));
  ctx->capturing = true;
  return FI_OK;
}

int32_t fi_graph_end(fi_context* ctx, fi_graph** out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(ctx->capturing, FI_ERR_RUNTIME, "fi_graph_end: no capture is open");
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  hipError_t err = hipStreamEndCapture(ctx->stream, &g);
  if (err != hipSuccess) {
    if (g) (void)hipGraphDestroy(g);
    return fi::hip_error(err, "hipStreamEndCapture");
  }
  if (out == nullptr) {  // discard
    (void)hipGraphDestroy(g);
    return FI_OK;
  }
  hipGraphExec_t exec = nullptr;
  err = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (err != hipSuccess) {
    (void)hipGraphDestroy(g);
    return fi::hip_error(err, "hipGraphInstantiate");
  }
  auto* graph = new fi_graph();
  graph->graph = g;
  graph->exec = exec;
  graph->device = ctx->device;
  *out = graph;
  return FI_OK;
}

int32_t fi_graph_launch(fi_context* ctx, fi_graph* graph) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(graph != nullptr && graph->device == ctx->device, FI_ERR_INVALID_CONFIG,
             "fi_graph_launch: graph of another device or null");
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_graph_launch: the stream is being captured");
  FI_TRY_HIP(hipGraphLaunch(graph->exec, ctx->stream));
  return FI_OK;
}

int32_t fi_graph_destroy(fi_graph* graph) {
  if (graph == nullptr) return FI_OK;
  FI_TRY_HIP(hipSetDevice(graph->device));
  hipError_t e1 = hipGraphExecDestroy(graph->exec);
  hipError_t e2 = hipGraphDestroy(graph->graph);
  delete graph;
  if (e1 != hipSuccess) return fi::hip_error(e1, "hipGraphExecDestroy");
  if (e2 != hipSuccess) return fi::hip_error(e2, "hipGraphDestroy");
  return FI_OK;
}

int32_t fi_ctx_check_faults(fi_context* ctx) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_ctx_check_faults: the stream is being captured into a graph");
  uint32_t words[4] = {0, 0, 0, 0};
  FI_TRY_HIP(hipMemcpyAsync(words, ctx->d_faults, sizeof(words), hipMemcpyDeviceToHost, ctx->stream));
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  uint32_t bits = words[0] | words[1] | words[2] | words[3];
  if (bits == 0) return FI_OK;
  uint32_t zero[4] = {0, 0, 0, 0};
  FI_TRY_HIP(hipMemcpyAsync(ctx->d_faults, zero, sizeof(zero), hipMemcpyHostToDevice, ctx->stream));
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  std::string msg = "device kernels reported:";
  if (bits & FI_FAULT_SLOT_RANGE) msg += " KV slot beyond the block pool;";
  if (bits & FI_FAULT_TOKEN_RANGE) msg += " token id out of vocabulary range;";
  if (bits & FI_FAULT_BLOCK_RANGE) msg += " block id beyond the block pool;";
  if (bits & FI_FAULT_SAMPLE_TOPK) msg += " sampling top_k above the device limit of 1024;";
  if (bits & FI_FAULT_SAMPLE_NONFINITE) msg += " failed to build a finite sampling distribution;";
  if (bits & FI_FAULT_CONTEXT_RANGE) msg += " context length beyond max_context_len;";
  if (bits & FI_FAULT_QUERY_RANGE) msg += " query length beyond max_query_len (its rows past the tiles were not computed);";
  if (bits & FI_FAULT_POSITION_RANGE) msg += " position outside the RoPE table;";
  return fi::set_error(FI_ERR_RUNTIME, msg);
}

}  // extern "C"
