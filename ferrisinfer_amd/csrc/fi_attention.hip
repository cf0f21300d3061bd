// Paged decode attention (split-KV with a log-sum-exp merge kernel), KV append and
// block copy for gfx950.  The arithmetic replaces the reference's per-sequence gather +
// online-softmax loops (crates/ferrisinfer-kernel/src/cpu/attention.rs:332-686,
// runtime/paged_kv.rs:769-791).
//
// KV pool layout (per layer): K and V are [num_blocks][Hkv][block_size][D], so one
// (block, kv_head) is a contiguous block_size*D run: a 16-token f32 block of D=128 is 8 KiB
// read with 16-byte loads.
#include "fi_common.h"
#include "fi_device.h"

namespace {

// Tunables (compile-time).  The partition size fixes the reduction order for a given context
// length, so it is a constant of the library, not of a launch.
#ifndef FI_DECODE_PART_TOKENS
#define FI_DECODE_PART_TOKENS 512
#endif
#ifndef FI_DECODE_KLANES_MAX
#define FI_DECODE_KLANES_MAX 8  // lanes sharing one K row (8 or 16)
#endif
#ifndef FI_DECODE_VUNROLL
#define FI_DECODE_VUNROLL 2  // V loads per lane per (double-buffered) step
#endif

constexpr int kPartTokens = FI_DECODE_PART_TOKENS;
constexpr int kThreads = 256;     // 4 wave64 per workgroup
constexpr int kMaxParts = 256;    // merge weights live in LDS
constexpr int kMaxContext = kPartTokens * kMaxParts;

template <typename KVT>
struct KvIO;

template <>
struct KvIO<float> {
  static constexpr int kVecElems = 4;  // one 16-byte load
  __device__ static void load_vec(const float* p, float* out) {
    float4 v = *reinterpret_cast<const float4*>(p);
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  }
  __device__ static void load_pair(const float* p, float* out) {
    float2 v = *reinterpret_cast<const float2*>(p);
    out[0] = v.x;
    out[1] = v.y;
  }
};

template <>
struct KvIO<uint16_t> {
  static constexpr int kVecElems = 8;
  __device__ static void load_vec(const uint16_t* p, float* out) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = fi::bf16_bits_to_f32(w[i] & 0xffffu);
      out[2 * i + 1] = fi::bf16_bits_to_f32(w[i] >> 16);
    }
  }
  __device__ static void load_pair(const uint16_t* p, float* out) {
    uint32_t w = *reinterpret_cast<const uint32_t*>(p);
    out[0] = fi::bf16_bits_to_f32(w & 0xffffu);
    out[1] = fi::bf16_bits_to_f32(w >> 16);
  }
};

struct DecodeArgs {
  const float* q;
  const void* k_cache;
  const void* v_cache;
  const int* block_tables;
  const int* context_lens;
  float* part_acc;  // [num_seqs * Hq * parts_per_seq, D]
  float* part_ml;   // [num_seqs * Hq * parts_per_seq, 2]
  float* out;
  uint32_t* faults;
  int num_seqs;
  int max_blocks;
  int parts_per_seq;
  int hq;
  int hkv;
  int group;
  int block_size;
  int num_blocks;
  float scale;
};

// One workgroup = one (sequence, kv_head, partition of kPartTokens tokens).  The GQA group
// of query heads sharing the kv head is processed together so each K/V byte is read once.
//   setup: the partition's token -> pool row indices go to LDS once (block-table lookups);
//   pass 1 (K): KLANES lanes share a token row with 16-byte loads; the next row-step's loads
//     are issued before the current one is reduced (two register buffers), dot products are
//     reduced across the row's lanes with DPP, scores go to LDS;
//   softmax over the partition in LDS (the first V loads are already in flight);
//   pass 2 (V): D/vec lanes cover a row with 16-byte loads, again double-buffered; per-lane
//     accumulators are folded across rows with shuffles and across waves in LDS.
// Rows past the partition end are clamped to its last row: they share addresses with valid
// lanes (no extra traffic) and are masked out of the scores and weights.
// A sequence with one partition writes its normalised output directly; otherwise each
// workgroup stores (max, sum, unnormalised acc) for decode_merge_kernel.
template <int D, typename KVT, int MAXG>
__global__ __launch_bounds__(kThreads) void decode_partition_kernel(DecodeArgs a) {
  constexpr int EPV = KvIO<KVT>::kVecElems;   // elements per 16-byte vector
  constexpr int VECS = D / EPV;               // vectors per row
  static_assert(VECS <= 64, "a row must fit one wave of 16-byte loads");
  constexpr int KLANES = VECS < FI_DECODE_KLANES_MAX ? VECS : FI_DECODE_KLANES_MAX;  // lanes per K row
  constexpr int KVPL = VECS / KLANES;          // vectors per lane (K)
  constexpr int KEPL = KVPL * EPV;             // elements per lane (K)
  constexpr int KROWS_W = 64 / KLANES;         // K rows per wave per step
  constexpr int KSTEP = 4 * KROWS_W;           // K rows per workgroup per step
  constexpr int VLANES = VECS;                 // lanes per row in the V pass
  constexpr int VROWS_W = 64 / VLANES;         // V rows per wave per load
  constexpr int VU = FI_DECODE_VUNROLL;        // V loads per lane per step
  constexpr int VSTEP = 4 * VROWS_W * VU;      // V rows per workgroup per step

  __shared__ float s_q[MAXG][D];
  __shared__ float s_p[MAXG][kPartTokens];
  __shared__ uint32_t s_row[kPartTokens];
  __shared__ float s_ml[MAXG][2];
  __shared__ float s_red[4][MAXG][D];

  const KVT* __restrict__ k_cache = static_cast<const KVT*>(a.k_cache);
  const KVT* __restrict__ v_cache = static_cast<const KVT*>(a.v_cache);
  const int parts_per_seq = a.parts_per_seq;
  const int group = a.group;
  const int wg = blockIdx.x;
  const int part = wg % parts_per_seq;
  const int rest = wg / parts_per_seq;
  const int kvh = rest % a.hkv;
  const int seq = rest / a.hkv;
  const int ctx = a.context_lens[seq];
  const int tid = threadIdx.x;
  const size_t head0 = (size_t)seq * a.hq + (size_t)kvh * group;  // first query head of the group
  if (ctx <= 0) {  // no keys: defined output of zeros
    if (part == 0) {
      for (int i = tid; i < group * D; i += kThreads) a.out[head0 * D + i] = 0.0f;
    }
    return;
  }
  const int t0 = part * kPartTokens;
  if (t0 >= ctx) return;  // whole workgroup exits together
  const int n = min(kPartTokens, ctx - t0);
  const int nparts = (ctx + kPartTokens - 1) / kPartTokens;
  const int w = tid >> 6;
  const int lane = tid & 63;

  for (int i = tid; i < MAXG * D; i += kThreads) {
    int g = i / D, d = i % D;
    s_q[g][d] = g < group ? a.q[(head0 + g) * D + d] : 0.0f;  // zero rows keep scores of g >= group at 0
  }
  for (int t = tid; t < n; t += kThreads) {
    const int bs = a.block_size;
    const int abs = t0 + t;
    const int lb = abs / bs;
    int id = lb < a.max_blocks ? a.block_tables[(size_t)seq * a.max_blocks + lb] : -1;
    if (id < 0 || id >= a.num_blocks) {
      atomicOr(a.faults, FI_FAULT_BLOCK_RANGE);
      id = 0;
    }
    s_row[t] = (static_cast<uint32_t>(id) * a.hkv + kvh) * bs + (abs - lb * bs);
  }
  __syncthreads();

  // ---- pass 1: scores ----
  {
    const int r = lane / KLANES;
    const int c = lane % KLANES;
    const int ksteps = (n + KSTEP - 1) / KSTEP;
    float qreg[MAXG][KEPL];
#pragma unroll
    for (int g = 0; g < MAXG; ++g)
#pragma unroll
      for (int j = 0; j < KVPL; ++j)
#pragma unroll
        for (int e = 0; e < EPV; ++e) qreg[g][j * EPV + e] = s_q[g][(j * KLANES + c) * EPV + e];

    auto load_k = [&](int step, float* buf) {
      const int tok = min(step * KSTEP + w * KROWS_W + r, n - 1);
      const KVT* row = k_cache + (size_t)s_row[tok] * D;
#pragma unroll
      for (int j = 0; j < KVPL; ++j) KvIO<KVT>::load_vec(row + (j * KLANES + c) * EPV, buf + j * EPV);
    };
    auto score_k = [&](int step, const float* buf) {
      const int tok = step * KSTEP + w * KROWS_W + r;
#pragma unroll
      for (int g = 0; g < MAXG; ++g) {
        float dot = 0.0f;
#pragma unroll
        for (int e = 0; e < KEPL; ++e) dot += qreg[g][e] * buf[e];
        dot = fi::group_sum<KLANES>(dot);
        if (g % KLANES == c && tok < n) s_p[g][tok] = dot * a.scale;
      }
    };
    float kb0[KEPL], kb1[KEPL];
    load_k(0, kb0);
    for (int step = 0; step < ksteps; step += 2) {
      if (step + 1 < ksteps) load_k(step + 1, kb1);
      score_k(step, kb0);
      if (step + 1 < ksteps) {
        if (step + 2 < ksteps) load_k(step + 2, kb0);
        score_k(step + 1, kb1);
      }
    }
  }

  // ---- pass 2 prologue: first V loads go out before the softmax ----
  const int vr = lane / VLANES;
  const int vc = lane % VLANES;
  const int vsteps = (n + VSTEP - 1) / VSTEP;
  auto load_v = [&](int step, float (*buf)[EPV]) {
#pragma unroll
    for (int u = 0; u < VU; ++u) {
      const int tok = min(step * VSTEP + (u * 4 + w) * VROWS_W + vr, n - 1);
      KvIO<KVT>::load_vec(v_cache + (size_t)s_row[tok] * D + vc * EPV, buf[u]);
    }
  };
  float vb0[VU][EPV], vb1[VU][EPV];
  load_v(0, vb0);
  __syncthreads();

  // ---- softmax over the partition ----
  for (int g = w; g < group; g += 4) {
    float m = -INFINITY;
    for (int t = lane; t < n; t += 64) m = fmaxf(m, s_p[g][t]);
    m = fi::wave_max(m);
    float l = 0.0f;
    for (int t = lane; t < n; t += 64) {
      float p = __expf(s_p[g][t] - m);
      s_p[g][t] = p;
      l += p;
    }
    l = fi::wave_sum(l);
    if (lane == 0) {
      s_ml[g][0] = m;
      s_ml[g][1] = l;
    }
  }
  __syncthreads();

  // ---- pass 2: weighted values ----
  {
    float acc[MAXG][EPV];
#pragma unroll
    for (int g = 0; g < MAXG; ++g)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[g][e] = 0.0f;
    auto accumulate = [&](int step, float (*buf)[EPV]) {
#pragma unroll
      for (int u = 0; u < VU; ++u) {
        const int tok = step * VSTEP + (u * 4 + w) * VROWS_W + vr;
        const bool valid = tok < n;
        const int tt = valid ? tok : 0;
#pragma unroll
        for (int g = 0; g < MAXG; ++g) {
          const float p = valid ? s_p[g][tt] : 0.0f;
#pragma unroll
          for (int e = 0; e < EPV; ++e) acc[g][e] += p * buf[u][e];
        }
      }
    };
    for (int step = 0; step < vsteps; step += 2) {
      if (step + 1 < vsteps) load_v(step + 1, vb1);
      accumulate(step, vb0);
      if (step + 1 < vsteps) {
        if (step + 2 < vsteps) load_v(step + 2, vb0);
        accumulate(step + 1, vb1);
      }
    }
    // rows of a wave share columns: fold them with lane shuffles, then waves through LDS
#pragma unroll
    for (int m = VLANES; m < 64; m <<= 1)
#pragma unroll
      for (int g = 0; g < MAXG; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] += __shfl_xor(acc[g][e], m, 64);
    if (vr == 0) {
#pragma unroll
      for (int g = 0; g < MAXG; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) s_red[w][g][vc * EPV + e] = acc[g][e];
    }
  }
  __syncthreads();

  for (int i = tid; i < group * D; i += kThreads) {
    int g = i / D, d = i % D;
    float sum = (s_red[0][g][d] + s_red[1][g][d]) + (s_red[2][g][d] + s_red[3][g][d]);
    if (nparts == 1) {
      a.out[(head0 + g) * D + d] = sum * (1.0f / s_ml[g][1]);
    } else {
      size_t slot = (head0 + g) * parts_per_seq + part;
      a.part_acc[slot * D + d] = sum;
      if (d == 0) {
        a.part_ml[slot * 2] = s_ml[g][0];
        a.part_ml[slot * 2 + 1] = s_ml[g][1];
      }
    }
  }
}

// Combines the partitions of one (sequence, kv_head) group: M = max m_p,
// L = sum l_p e^(m_p-M), out = sum acc_p e^(m_p-M) / L per query head.  Sequences with a
// single partition were finished by the partition kernel.  A separate launch orders the
// partials' stores before these loads.  The first partitions' partials are fetched before
// the weights are known so the loads overlap.
template <int D, int MAXG>
__global__ __launch_bounds__(kThreads) void decode_merge_kernel(DecodeArgs a) {
  constexpr int kPrefetch = 8;
  constexpr int kPerThread = (MAXG * D + kThreads - 1) / kThreads;
  __shared__ float s_w[MAXG][kMaxParts];
  __shared__ float s_inv[MAXG];
  const int pair = blockIdx.x;
  const int seq = pair / a.hkv;
  const int kvh = pair % a.hkv;
  const int ctx = a.context_lens[seq];
  const int nparts = (ctx + kPartTokens - 1) / kPartTokens;
  if (nparts <= 1) return;
  const int group = a.group;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const size_t head0 = (size_t)seq * a.hq + (size_t)kvh * group;
  const int P = a.parts_per_seq;

  float pre[kPerThread][kPrefetch];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int i = tid + k * kThreads;
    const int g = i / D, d = i % D;
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p)
      pre[k][p] = (g < group && p < nparts) ? a.part_acc[((head0 + g) * P + p) * D + d] : 0.0f;
  }
  for (int g = w; g < group; g += 4) {
    const float* ml = a.part_ml + (head0 + g) * P * 2;
    float m = -INFINITY;
    for (int p = lane; p < nparts; p += 64) m = fmaxf(m, ml[p * 2]);
    m = fi::wave_max(m);
    float l = 0.0f;
    for (int p = lane; p < nparts; p += 64) {
      float wgt = __expf(ml[p * 2] - m);
      s_w[g][p] = wgt;
      l += ml[p * 2 + 1] * wgt;
    }
    l = fi::wave_sum(l);
    if (lane == 0) s_inv[g] = 1.0f / l;
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int i = tid + k * kThreads;
    const int g = i / D, d = i % D;
    if (g >= group) continue;
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) acc += pre[k][p] * (p < nparts ? s_w[g][p] : 0.0f);
    for (int p = kPrefetch; p < nparts; ++p) acc += a.part_acc[((head0 + g) * P + p) * D + d] * s_w[g][p];
    a.out[(head0 + g) * D + d] = acc * s_inv[g];
  }
}

// One workgroup per token: copies the token's [Hkv, D] K and V rows into their pool slot.
template <typename KVT>
__global__ __launch_bounds__(256) void kv_append_kernel(const float* __restrict__ key,
                                                        const float* __restrict__ value,
                                                        const int64_t* __restrict__ slots,
                                                        KVT* __restrict__ k_cache,
                                                        KVT* __restrict__ v_cache, int64_t pool_slots,
                                                        int block_size, int hkv, int d,
                                                        uint32_t* __restrict__ faults) {
  const int t = blockIdx.x;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  if (slot >= pool_slots) {
    if (threadIdx.x == 0) atomicOr(faults, FI_FAULT_SLOT_RANGE);
    return;
  }
  const int64_t blk = slot / block_size;
  const int off = static_cast<int>(slot % block_size);
  const int row = hkv * d;
  for (int i = threadIdx.x; i < row; i += blockDim.x) {
    const int h = i / d, e = i % d;
    const size_t dst = (((size_t)blk * hkv + h) * block_size + off) * d + e;
    const float kf = key[(size_t)t * row + i];
    const float vf = value[(size_t)t * row + i];
    if constexpr (sizeof(KVT) == 4) {
      k_cache[dst] = kf;
      v_cache[dst] = vf;
    } else {
      k_cache[dst] = static_cast<KVT>(fi::f32_to_bf16_bits(kf));
      v_cache[dst] = static_cast<KVT>(fi::f32_to_bf16_bits(vf));
    }
  }
}

// One workgroup per (pair, kv_head): copies the first n token rows of a block.
template <typename KVT>
__global__ __launch_bounds__(256) void kv_copy_blocks_kernel(KVT* __restrict__ k_cache,
                                                             KVT* __restrict__ v_cache,
                                                             const int* __restrict__ src,
                                                             const int* __restrict__ dst,
                                                             const int* __restrict__ counts,
                                                             int num_blocks, int block_size, int hkv,
                                                             int d, uint32_t* __restrict__ faults) {
  const int pair = blockIdx.x / hkv;
  const int h = blockIdx.x % hkv;
  const int s = src[pair], t = dst[pair];
  const int n = min(max(counts[pair], 0), block_size);
  if (s < 0 || s >= num_blocks || t < 0 || t >= num_blocks) {
    if (threadIdx.x == 0) atomicOr(faults, FI_FAULT_BLOCK_RANGE);
    return;
  }
  const size_t so = ((size_t)s * hkv + h) * block_size * d;
  const size_t to = ((size_t)t * hkv + h) * block_size * d;
  for (int i = threadIdx.x; i < n * d; i += blockDim.x) {
    k_cache[to + i] = k_cache[so + i];
    v_cache[to + i] = v_cache[so + i];
  }
}

__global__ void fill_zero_kernel(uint8_t* __restrict__ p, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t stride = (size_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) p[i] = 0;
}

int32_t zero_async(fi_context* ctx, void* p, size_t bytes) {
  if (bytes == 0) return FI_OK;
  size_t blocks = (bytes + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx->stream,
                     static_cast<uint8_t*>(p), bytes);
  FI_CHECK_LAUNCH("fill_zero_kernel");
  return FI_OK;
}

template <int D, typename KVT, int MAXG>
int32_t launch_decode_group(fi_context* ctx, const DecodeArgs& args, unsigned grid) {
  hipLaunchKernelGGL((decode_partition_kernel<D, KVT, MAXG>), dim3(grid), dim3(kThreads), 0, ctx->stream, args);
  FI_CHECK_LAUNCH("decode_partition_kernel");
  if (args.parts_per_seq > 1) {
    hipLaunchKernelGGL((decode_merge_kernel<D, MAXG>), dim3(static_cast<unsigned>(args.num_seqs) * args.hkv),
                       dim3(kThreads), 0, ctx->stream, args);
    FI_CHECK_LAUNCH("decode_merge_kernel");
  }
  return FI_OK;
}

template <int D, typename KVT>
int32_t launch_decode(fi_context* ctx, const DecodeArgs& args, unsigned grid) {
  if (args.group <= 1) return launch_decode_group<D, KVT, 1>(ctx, args, grid);
  if (args.group <= 2) return launch_decode_group<D, KVT, 2>(ctx, args, grid);
  if (args.group <= 4) return launch_decode_group<D, KVT, 4>(ctx, args, grid);
  if (args.group <= 8) return launch_decode_group<D, KVT, 8>(ctx, args, grid);
  return fi::set_error(FI_ERR_UNSUPPORTED, "decode attention supports at most 8 query heads per KV head");
}

template <int D>
int32_t launch_decode_dtype(fi_context* ctx, int32_t dtype, const DecodeArgs& args, unsigned grid) {
  if (dtype == FI_DTYPE_F32) return launch_decode<D, float>(ctx, args, grid);
  return launch_decode<D, uint16_t>(ctx, args, grid);
}

}  // namespace

namespace fi {

// Split-KV decode partials live in the context workspace (grow-only).
int32_t decode_scratch(fi_context* ctx, int32_t num_seqs, int32_t hq, int32_t parts, int32_t head_dim,
                       float** part_acc, float** part_ml) {
  size_t slots = static_cast<size_t>(num_seqs) * hq * parts;
  size_t acc_bytes = slots * head_dim * sizeof(float);
  size_t ml_bytes = slots * 2 * sizeof(float);
  FI_TRY(ensure_workspace(ctx, acc_bytes + ml_bytes));
  *part_acc = static_cast<float*>(ctx->workspace);
  *part_ml = reinterpret_cast<float*>(static_cast<char*>(ctx->workspace) + acc_bytes);
  return FI_OK;
}

}  // namespace fi

extern "C" {

int32_t fi_buf_zero(fi_context* ctx, void* d_ptr, size_t bytes) {
  FI_TRY(fi::enter(ctx));
  if (bytes == 0) return FI_OK;
  FI_REQUIRE(d_ptr != nullptr, FI_ERR_INVALID_CONFIG, "fi_buf_zero: null pointer");
  return zero_async(ctx, d_ptr, bytes);
}

int32_t fi_kv_append(fi_context* ctx, const float* d_key, const float* d_value,
                     const int64_t* d_slot_mapping, int32_t num_tokens, void* d_k_cache,
                     void* d_v_cache, int32_t kv_dtype, int32_t num_blocks, int32_t block_size,
                     int32_t num_kv_heads, int32_t head_dim) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_tokens >= 0, FI_ERR_INVALID_SHAPE, "fi_kv_append: negative token count");
  FI_REQUIRE(num_blocks > 0 && block_size > 0 && num_kv_heads > 0 && head_dim > 0,
             FI_ERR_INVALID_CONFIG, "fi_kv_append: pool dimensions must be greater than zero");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_kv_append: KV dtype must be f32 or bf16");
  if (num_tokens == 0) return FI_OK;
  FI_REQUIRE(d_key && d_value && d_slot_mapping && d_k_cache && d_v_cache, FI_ERR_INVALID_CONFIG,
             "fi_kv_append: null pointer");
  const int64_t pool_slots = static_cast<int64_t>(num_blocks) * block_size;
  if (kv_dtype == FI_DTYPE_F32) {
    hipLaunchKernelGGL(kv_append_kernel<float>, dim3(num_tokens), dim3(256), 0, ctx->stream, d_key, d_value,
                       d_slot_mapping, static_cast<float*>(d_k_cache), static_cast<float*>(d_v_cache),
                       pool_slots, block_size, num_kv_heads, head_dim, ctx->d_faults);
  } else {
    hipLaunchKernelGGL(kv_append_kernel<uint16_t>, dim3(num_tokens), dim3(256), 0, ctx->stream, d_key,
                       d_value, d_slot_mapping, static_cast<uint16_t*>(d_k_cache),
                       static_cast<uint16_t*>(d_v_cache), pool_slots, block_size, num_kv_heads, head_dim,
                       ctx->d_faults);
  }
  FI_CHECK_LAUNCH("kv_append_kernel");
  return FI_OK;
}

int32_t fi_kv_copy_blocks(fi_context* ctx, void* d_k_cache, void* d_v_cache, int32_t kv_dtype,
                          const int32_t* d_src_blocks, const int32_t* d_dst_blocks,
                          const int32_t* d_token_counts, int32_t num_pairs, int32_t num_blocks,
                          int32_t block_size, int32_t num_kv_heads, int32_t head_dim) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_pairs >= 0, FI_ERR_INVALID_SHAPE, "fi_kv_copy_blocks: negative pair count");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_kv_copy_blocks: KV dtype must be f32 or bf16");
  FI_REQUIRE(num_blocks > 0 && block_size > 0 && num_kv_heads > 0 && head_dim > 0,
             FI_ERR_INVALID_CONFIG, "fi_kv_copy_blocks: pool dimensions must be greater than zero");
  if (num_pairs == 0) return FI_OK;
  dim3 grid(static_cast<unsigned>(num_pairs) * num_kv_heads);
  if (kv_dtype == FI_DTYPE_F32) {
    hipLaunchKernelGGL(kv_copy_blocks_kernel<float>, grid, dim3(256), 0, ctx->stream,
                       static_cast<float*>(d_k_cache), static_cast<float*>(d_v_cache), d_src_blocks,
                       d_dst_blocks, d_token_counts, num_blocks, block_size, num_kv_heads, head_dim,
                       ctx->d_faults);
  } else {
    hipLaunchKernelGGL(kv_copy_blocks_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream,
                       static_cast<uint16_t*>(d_k_cache), static_cast<uint16_t*>(d_v_cache), d_src_blocks,
                       d_dst_blocks, d_token_counts, num_blocks, block_size, num_kv_heads, head_dim,
                       ctx->d_faults);
  }
  FI_CHECK_LAUNCH("kv_copy_blocks_kernel");
  return FI_OK;
}

int32_t fi_attn_decode_paged(fi_context* ctx, const float* d_q, const void* d_k_cache,
                             const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                             int32_t max_blocks_per_seq, const int32_t* d_context_lens,
                             int32_t num_seqs, int32_t max_context_len, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t num_blocks, float scale, float* d_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_seqs >= 0 && max_context_len >= 0, FI_ERR_INVALID_SHAPE,
             "fi_attn_decode_paged: negative sizes");
  FI_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
             FI_ERR_INVALID_SHAPE, "number of query heads must be divisible by number of KV heads");
  FI_REQUIRE(block_size > 0 && num_blocks > 0 && max_blocks_per_seq > 0, FI_ERR_INVALID_CONFIG,
             "fi_attn_decode_paged: pool dimensions must be greater than zero");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_attn_decode_paged: KV dtype must be f32 or bf16");
  FI_REQUIRE(max_context_len <= kMaxContext, FI_ERR_UNSUPPORTED,
             "fi_attn_decode_paged: context longer than " + std::to_string(kMaxContext) + " tokens");
  FI_REQUIRE(static_cast<int64_t>(max_context_len) <= static_cast<int64_t>(max_blocks_per_seq) * block_size,
             FI_ERR_INVALID_SHAPE, "fi_attn_decode_paged: max_context_len exceeds the block-table width");
  FI_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, FI_ERR_UNSUPPORTED,
             "fi_attn_decode_paged: head_dim must be 32, 64 or 128");
  if (num_seqs == 0) return FI_OK;
  FI_REQUIRE(d_q && d_k_cache && d_v_cache && d_block_tables && d_context_lens && d_out,
             FI_ERR_INVALID_CONFIG, "fi_attn_decode_paged: null pointer");
  const int32_t parts = max_context_len == 0 ? 1 : (max_context_len + kPartTokens - 1) / kPartTokens;
  DecodeArgs args{};
  args.q = d_q;
  args.k_cache = d_k_cache;
  args.v_cache = d_v_cache;
  args.block_tables = d_block_tables;
  args.context_lens = d_context_lens;
  args.out = d_out;
  args.faults = ctx->d_faults;
  args.num_seqs = num_seqs;
  args.max_blocks = max_blocks_per_seq;
  args.parts_per_seq = parts;
  args.hq = num_q_heads;
  args.hkv = num_kv_heads;
  args.group = num_q_heads / num_kv_heads;
  args.block_size = block_size;
  args.num_blocks = num_blocks;
  args.scale = scale;
  if (parts > 1) {
    FI_TRY(fi::decode_scratch(ctx, num_seqs, num_q_heads, parts, head_dim, &args.part_acc, &args.part_ml));
  }
  const unsigned grid = static_cast<unsigned>(num_seqs) * num_kv_heads * parts;
  switch (head_dim) {
    case 32:
      return launch_decode_dtype<32>(ctx, kv_dtype, args, grid);
    case 64:
      return launch_decode_dtype<64>(ctx, kv_dtype, args, grid);
    default:
      return launch_decode_dtype<128>(ctx, kv_dtype, args, grid);
  }
}

}  // extern "C"
