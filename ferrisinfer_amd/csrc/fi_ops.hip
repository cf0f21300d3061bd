// Decoder-block ops that feed attention: embedding gather, RMSNorm (plain and fused with the
// residual add), RoPE over per-token positions, SwiGLU and residual add.  All are HBM-bound
// row/elementwise kernels: one workgroup per row, 16-byte accesses where the width allows.
#include <cmath>
#include <vector>

#include "fi_common.h"
#include "fi_device.h"

namespace {

constexpr int kRowThreads = 256;

// Block-wide sum of one float per thread (256 threads = 4 waves).
__device__ float block_sum(float v, float* s_scratch) {
  v = fi::wave_sum(v);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) s_scratch[w] = v;
  __syncthreads();
  float total = (s_scratch[0] + s_scratch[1]) + (s_scratch[2] + s_scratch[3]);
  __syncthreads();
  return total;
}

// ids[i] = prev[rows[i]] where rows[i] >= 0: the previous step's sampled tokens fed as this
// step's inputs (runtime/session.rs:246-262 feeds the last sample).  A row outside prev leaves
// the entry unchanged and raises the TOKEN_RANGE fault bit.
__global__ __launch_bounds__(kRowThreads) void token_feed_kernel(const int32_t* __restrict__ prev, int prev_count,
                                                                 const int32_t* __restrict__ rows, int n,
                                                                 int32_t* __restrict__ ids,
                                                                 uint32_t* __restrict__ faults) {
  const int i = blockIdx.x * kRowThreads + threadIdx.x;
  if (i >= n) return;
  const int r = rows[i];
  if (r < 0) return;
  if (r >= prev_count) {
    atomicOr(faults, FI_FAULT_TOKEN_RANGE);
    return;
  }
  ids[i] = prev[r];
}

// out[r, :] = table[ids[r], :]  (kernel/cpu/attention.rs:3-99).  An id outside the vocabulary
// writes a zero row and raises the TOKEN_RANGE fault bit.
__global__ __launch_bounds__(kRowThreads) void embedding_kernel(const float* __restrict__ table, int vocab,
                                                                int hidden, const int32_t* __restrict__ ids,
                                                                float* __restrict__ out,
                                                                uint32_t* __restrict__ faults) {
  const int r = blockIdx.x;
  const int id = ids[r];
  float* dst = out + (size_t)r * hidden;
  if (id < 0 || id >= vocab) {
    if (threadIdx.x == 0) atomicOr(faults, FI_FAULT_TOKEN_RANGE);
    for (int c = threadIdx.x; c < hidden; c += kRowThreads) dst[c] = 0.0f;
    return;
  }
  const float* src = table + (size_t)id * hidden;
  if ((hidden & 3) == 0) {
    const float4* s4 = reinterpret_cast<const float4*>(src);
    float4* d4 = reinterpret_cast<float4*>(dst);
    for (int c = threadIdx.x; c < hidden / 4; c += kRowThreads) d4[c] = s4[c];
  } else {
    for (int c = threadIdx.x; c < hidden; c += kRowThreads) dst[c] = src[c];
  }
}

// RMSNorm (kernel/cpu/reduction.rs:3-73): ms = sum(x^2)/H; inv = 1/sqrt(ms + eps);
// out = (x * inv) * w.  With `residual`, first x = a + residual is formed and stored to
// `sum_out` (the reference's add_f32_in_place before the ffn/final norm,
// runtime/reference.rs:337-343).
__global__ __launch_bounds__(kRowThreads) void rms_norm_kernel(const float* __restrict__ a,
                                                               const float* __restrict__ residual,
                                                               float* __restrict__ sum_out,
                                                               const float* __restrict__ w,
                                                               float* __restrict__ out, int hidden,
                                                               float eps) {
  __shared__ float s_scratch[4];
  const int r = blockIdx.x;
  const float* x = a + (size_t)r * hidden;
  float ss = 0.0f;
  for (int c = threadIdx.x; c < hidden; c += kRowThreads) {
    float v = x[c];
    if (residual) {
      v = v + residual[(size_t)r * hidden + c];
      sum_out[(size_t)r * hidden + c] = v;
    }
    ss += v * v;
  }
  const float total = block_sum(ss, s_scratch);
  const float inv = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
  const float* xs = residual ? sum_out + (size_t)r * hidden : x;
  for (int c = threadIdx.x; c < hidden; c += kRowThreads) {
    out[(size_t)r * hidden + c] = (xs[c] * inv) * w[c];
  }
}

// NeoX half-split rotation with per-token positions (kernel/cpu/attention.rs:1242-1292):
// (lo, hi) <- (lo*c - hi*s, hi*c + lo*s) for pairs (j, j + rot/2).  cos/sin come from the
// host table built with the reference's loop, and FMA contraction is switched off so each
// product is rounded before the add, as Rust computes it: the result is bit-identical.
__global__ __launch_bounds__(kRowThreads) void rope_kernel(float* __restrict__ q, float* __restrict__ k,
                                                           const int32_t* __restrict__ positions,
                                                           const float* __restrict__ cos_t,
                                                           const float* __restrict__ sin_t, int hq,
                                                           int hkv, int d, int pairs, int max_positions,
                                                           uint32_t* __restrict__ faults) {
  const int t = blockIdx.x;
  const int pos = positions[t];
  if (pos < 0 || pos >= max_positions) {
    if (threadIdx.x == 0) atomicOr(faults, FI_FAULT_POSITION_RANGE);
    return;
  }
  const float* ct = cos_t + (size_t)pos * pairs;
  const float* st = sin_t + (size_t)pos * pairs;
  const int per_token = (hq + hkv) * pairs;
  for (int i = threadIdx.x; i < per_token; i += kRowThreads) {
    const int h = i / pairs, j = i % pairs;
    float* base = h < hq ? q + ((size_t)t * hq + h) * d : k + ((size_t)t * hkv + (h - hq)) * d;
    {
#pragma clang fp contract(off)
      const float lo = base[j], hi = base[j + pairs];
      const float c = ct[j], s = st[j];
      base[j] = lo * c - hi * s;
      base[j + pairs] = hi * c + lo * s;
    }
  }
}

// SwiGLU (runtime/reference.rs:346-360): gate <- gate * (1 / (1 + exp(-gate))); out = up * gate.
// `out` may alias `up` or `gate` (each element is read before it is written).
__global__ void silu_mul_kernel(const float* up, const float* gate, float* out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) {
    const float g = gate[i];
    const float sig = 1.0f / (1.0f + expf(-g));
    out[i] = up[i] * (g * sig);
  }
}

__global__ void add_kernel(const float* __restrict__ a, const float* __restrict__ b,
                           float* __restrict__ out, int64_t n) {
  int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) out[i] = a[i] + b[i];
}

unsigned elementwise_grid(int64_t n) {
  int64_t blocks = (n + 255) / 256;
  return static_cast<unsigned>(blocks < 8192 ? (blocks < 1 ? 1 : blocks) : 8192);
}

}  // namespace

extern "C" {

int32_t fi_embedding(fi_context* ctx, const float* d_table, int32_t vocab, int32_t hidden,
                     const int32_t* d_ids, int32_t num_tokens, float* d_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(vocab > 0 && hidden > 0 && num_tokens >= 0, FI_ERR_INVALID_SHAPE,
             "fi_embedding: vocab and hidden must be positive");
  if (num_tokens == 0) return FI_OK;
  FI_REQUIRE(d_table && d_ids && d_out, FI_ERR_INVALID_CONFIG, "fi_embedding: null pointer");
  hipLaunchKernelGGL(embedding_kernel, dim3(num_tokens), dim3(kRowThreads), 0, ctx->stream, d_table, vocab,
                     hidden, d_ids, d_out, ctx->d_faults);
  FI_CHECK_LAUNCH("embedding_kernel");
  return FI_OK;
}

int32_t fi_token_feed(fi_context* ctx, const int32_t* d_prev_tokens, int32_t prev_count, const int32_t* d_rows,
                      int32_t n, int32_t* d_ids) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(n >= 0 && prev_count >= 0, FI_ERR_INVALID_SHAPE, "fi_token_feed: negative count");
  if (n == 0) return FI_OK;
  FI_REQUIRE(d_prev_tokens && d_rows && d_ids, FI_ERR_INVALID_CONFIG, "fi_token_feed: null pointer");
  hipLaunchKernelGGL(token_feed_kernel, dim3((n + kRowThreads - 1) / kRowThreads), dim3(kRowThreads), 0,
                     ctx->stream, d_prev_tokens, prev_count, d_rows, n, d_ids, ctx->d_faults);
  FI_CHECK_LAUNCH("token_feed_kernel");
  return FI_OK;
}

int32_t fi_rms_norm(fi_context* ctx, const float* d_x, const float* d_weight, float* d_out,
                    int32_t rows, int32_t hidden, float eps) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(rows >= 0 && hidden > 0, FI_ERR_INVALID_SHAPE, "fi_rms_norm: hidden must be positive");
  if (rows == 0) return FI_OK;
  FI_REQUIRE(d_x && d_weight && d_out, FI_ERR_INVALID_CONFIG, "fi_rms_norm: null pointer");
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kRowThreads), 0, ctx->stream, d_x, nullptr, nullptr,
                     d_weight, d_out, hidden, eps);
  FI_CHECK_LAUNCH("rms_norm_kernel");
  return FI_OK;
}

int32_t fi_add_rms_norm(fi_context* ctx, const float* d_a, const float* d_residual, float* d_sum,
                        const float* d_weight, float* d_out, int32_t rows, int32_t hidden, float eps) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(rows >= 0 && hidden > 0, FI_ERR_INVALID_SHAPE, "fi_add_rms_norm: hidden must be positive");
  if (rows == 0) return FI_OK;
  FI_REQUIRE(d_a && d_residual && d_sum && d_weight && d_out, FI_ERR_INVALID_CONFIG,
             "fi_add_rms_norm: null pointer");
  hipLaunchKernelGGL(rms_norm_kernel, dim3(rows), dim3(kRowThreads), 0, ctx->stream, d_a, d_residual, d_sum,
                     d_weight, d_out, hidden, eps);
  FI_CHECK_LAUNCH("rms_norm_kernel");
  return FI_OK;
}

int32_t fi_rope_table(fi_context* ctx, int32_t max_positions, int32_t head_dim, int32_t rotary_dims,
                      float theta, float* d_cos, float* d_sin) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(!ctx->capturing, FI_ERR_RUNTIME, "fi_rope_table: the stream is being captured into a graph");
  FI_REQUIRE(max_positions > 0 && head_dim > 0, FI_ERR_INVALID_SHAPE,
             "fi_rope_table: positions and head_dim must be positive");
  FI_REQUIRE(rotary_dims >= 0 && rotary_dims <= head_dim && rotary_dims % 2 == 0, FI_ERR_INVALID_SHAPE,
             "rotary_dims must be an even value no larger than head_dim");
  FI_REQUIRE(theta > 0.0f, FI_ERR_INVALID_CONFIG, "rope theta must be positive");
  const int pairs = rotary_dims / 2;
  if (pairs == 0) return FI_OK;
  FI_REQUIRE(d_cos && d_sin, FI_ERR_INVALID_CONFIG, "fi_rope_table: null pointer");
  // The reference's loop (attention.rs:1253-1277): inv_0 = 1, inv_{j+1} = inv_j * theta^(-2/D)
  // in f32, angle = pos * inv_j, then sin/cos from libm.
  std::vector<float> c(static_cast<size_t>(max_positions) * pairs), s(c.size());
  const float step_exponent = -2.0f / static_cast<float>(head_dim);
  const float step = std::pow(theta, step_exponent);
  for (int p = 0; p < max_positions; ++p) {
    const float pos = static_cast<float>(p);
    float inv = 1.0f;
    for (int j = 0; j < pairs; ++j) {
      const float angle = pos * inv;
      s[static_cast<size_t>(p) * pairs + j] = std::sin(angle);
      c[static_cast<size_t>(p) * pairs + j] = std::cos(angle);
      inv = inv * step;
    }
  }
  FI_TRY_HIP(hipMemcpyAsync(d_cos, c.data(), c.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  FI_TRY_HIP(hipMemcpyAsync(d_sin, s.data(), s.size() * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  FI_TRY_HIP(hipStreamSynchronize(ctx->stream));
  return FI_OK;
}

int32_t fi_rope(fi_context* ctx, float* d_q, float* d_k, const int32_t* d_positions, const float* d_cos,
                const float* d_sin, int32_t num_tokens, int32_t num_q_heads, int32_t num_kv_heads,
                int32_t head_dim, int32_t rotary_dims, int32_t max_positions) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_tokens >= 0 && num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0, FI_ERR_INVALID_SHAPE,
             "fi_rope: head counts and head_dim must be positive");
  FI_REQUIRE(rotary_dims >= 0 && rotary_dims <= head_dim && rotary_dims % 2 == 0, FI_ERR_INVALID_SHAPE,
             "rotary_dims must be an even value no larger than head_dim");
  if (num_tokens == 0 || rotary_dims == 0) return FI_OK;
  FI_REQUIRE(d_q && d_k && d_positions && d_cos && d_sin, FI_ERR_INVALID_CONFIG, "fi_rope: null pointer");
  hipLaunchKernelGGL(rope_kernel, dim3(num_tokens), dim3(kRowThreads), 0, ctx->stream, d_q, d_k, d_positions,
                     d_cos, d_sin, num_q_heads, num_kv_heads, head_dim, rotary_dims / 2, max_positions,
                     ctx->d_faults);
  FI_CHECK_LAUNCH("rope_kernel");
  return FI_OK;
}

int32_t fi_silu_mul(fi_context* ctx, const float* d_up, const float* d_gate, float* d_out, int64_t n) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(n >= 0, FI_ERR_INVALID_SHAPE, "fi_silu_mul: negative size");
  if (n == 0) return FI_OK;
  FI_REQUIRE(d_up && d_gate && d_out, FI_ERR_INVALID_CONFIG, "fi_silu_mul: null pointer");
  hipLaunchKernelGGL(silu_mul_kernel, dim3(elementwise_grid(n)), dim3(256), 0, ctx->stream, d_up, d_gate,
                     d_out, n);
  FI_CHECK_LAUNCH("silu_mul_kernel");
  return FI_OK;
}

int32_t fi_add(fi_context* ctx, const float* d_a, const float* d_b, float* d_out, int64_t n) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(n >= 0, FI_ERR_INVALID_SHAPE, "fi_add: negative size");
  if (n == 0) return FI_OK;
  FI_REQUIRE(d_a && d_b && d_out, FI_ERR_INVALID_CONFIG, "fi_add: null pointer");
  hipLaunchKernelGGL(add_kernel, dim3(elementwise_grid(n)), dim3(256), 0, ctx->stream, d_a, d_b, d_out, n);
  FI_CHECK_LAUNCH("add_kernel");
  return FI_OK;
}

}  // extern "C"
