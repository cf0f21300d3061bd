// Varlen causal prefill attention over the paged KV pool, on MFMA (v_mfma_f32_16x16x4_f32).
// Replaces causal_self_attention_f32 / prefixed_causal_attention_f32 /
// cached_prefixed_causal_attention_f32 (crates/ferrisinfer-kernel/src/cpu/attention.rs:222-518,
// 688-962) plus the paged prefix gather that feeds them (runtime/paged_kv.rs:769-791,
// runtime/reference.rs:425-465) for a ragged batch packed by cu_seqlens.
//
// Sequence b has qlen_b = cu_seqlens[b+1] - cu_seqlens[b] new query tokens at positions
// [ctx_b - qlen_b, ctx_b); query position p attends keys [0, p] read through the block table
// (its own K/V rows must already be appended).  One workgroup = (sequence, query head,
// 64-token query tile): 4 waves x 16 query rows.  Per 32-key tile: K and V are staged in LDS
// (bf16 widened), S = Q K^T on MFMA with Q held in registers, causal mask + online softmax
// with row reductions by DPP across the 16 lanes holding a row, P is moved through LDS from
// the accumulator layout to the A-operand layout, and O += P V on MFMA.
#include "fi_common.h"
#include "fi_device.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kQTile = 64;    // query tokens per workgroup
constexpr int kKTile = 32;    // keys per LDS tile
constexpr int kThreads = 256;

struct PrefillArgs {
  const float* q;            // [T, Hq, D]
  const void* k_cache;       // [blocks, Hkv, bs, D]
  const void* v_cache;
  const int* cu_seqlens;     // [B+1]
  const int* context_lens;   // [B]
  const int* block_tables;   // [B, max_blocks]
  float* out;                // [T, Hq, D]
  uint32_t* faults;
  int max_blocks;
  int hq, hkv, group;
  int block_size, num_blocks;
  float scale;
};

template <int kLanes>
__device__ __forceinline__ float group_max(float v) {
  v = fmaxf(v, fi::dpp_mov<0xB1>(v));
  v = fmaxf(v, fi::dpp_mov<0x4E>(v));
  v = fmaxf(v, fi::dpp_mov<0x141>(v));
  v = fmaxf(v, fi::dpp_mov<0x140>(v));
  return v;
}

__device__ __forceinline__ float load_kv(const float* p) { return *p; }
__device__ __forceinline__ float load_kv(const uint16_t* p) { return fi::bf16_bits_to_f32(*p); }

template <int D, typename KVT>
__global__ __launch_bounds__(kThreads) void prefill_kernel(PrefillArgs a) {
  constexpr int KSTEPS = D / 4;      // MFMA k-steps over the head dimension
  constexpr int DT = D / 16;         // 16-wide output column tiles
  __shared__ float Ks[kKTile][D + 1];
  __shared__ float Vs[kKTile][D + 4];
  __shared__ float Ps[4][16][kKTile + 1];
  __shared__ int s_row[kKTile];

  const KVT* __restrict__ k_cache = static_cast<const KVT*>(a.k_cache);
  const KVT* __restrict__ v_cache = static_cast<const KVT*>(a.v_cache);
  const int qt = blockIdx.x, seq = blockIdx.y, h = blockIdx.z;
  const int qs = a.cu_seqlens[seq];
  const int qlen = a.cu_seqlens[seq + 1] - qs;
  const int q0 = qt * kQTile;
  if (q0 >= qlen) return;
  const int ctx = a.context_lens[seq];
  const int start = ctx - qlen;  // position of the first query token
  const int kvh = h / a.group;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lk = lane >> 4;
  const int r0 = q0 + w * 16;  // first query row (within the sequence) of this wave

  // Q fragment: A[i][k] = Q[r0 + li][4*step + lk]
  float qreg[KSTEPS];
  {
    const int row = r0 + li;
    const float* qp = a.q + ((size_t)(qs + min(row, qlen - 1)) * a.hq + h) * D;
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) qreg[s] = qp[4 * s + lk];
  }

  v4f o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  float m_row[4], l_row[4];
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    m_row[v] = -INFINITY;
    l_row[v] = 0.0f;
  }

  const int kend = start + min(qlen, q0 + kQTile);  // keys needed by the last row of the tile
  for (int k0 = 0; k0 < kend; k0 += kKTile) {
    // ---- stage K and V rows [k0, k0 + 32) ----
    if (tid < kKTile) {
      const int kp = k0 + tid;
      int row = -1;
      if (kp < ctx) {
        const int lb = kp / a.block_size;
        int id = lb < a.max_blocks ? a.block_tables[(size_t)seq * a.max_blocks + lb] : -1;
        if (id < 0 || id >= a.num_blocks) {
          atomicOr(a.faults, FI_FAULT_BLOCK_RANGE);
          id = 0;
        }
        row = (id * a.hkv + kvh) * a.block_size + (kp - lb * a.block_size);
      }
      s_row[tid] = row;
    }
    __syncthreads();
    for (int i = tid; i < kKTile * D; i += kThreads) {
      const int j = i / D, d = i % D;
      const int row = s_row[j];
      float kv = 0.0f, vv = 0.0f;
      if (row >= 0) {
        kv = load_kv(k_cache + (size_t)row * D + d);
        vv = load_kv(v_cache + (size_t)row * D + d);
      }
      Ks[j][d] = kv;
      Vs[j][d] = vv;
    }
    __syncthreads();

    // ---- S = Q K^T for this wave's 16 rows x 32 keys ----
    v4f s_acc[2] = {v4f{0.0f, 0.0f, 0.0f, 0.0f}, v4f{0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
    for (int s = 0; s < KSTEPS; ++s) {
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const float b = Ks[jt * 16 + li][4 * s + lk];
        s_acc[jt] = __builtin_amdgcn_mfma_f32_16x16x4f32(qreg[s], b, s_acc[jt], 0, 0, 0);
      }
    }
    // element (jt, v): row r0 + 4*lk + v, key k0 + 16*jt + li
    float p[2][4];
    float alpha[4];
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int qpos = start + r0 + 4 * lk + v;
      float mx = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        const int kp = k0 + 16 * jt + li;
        const float sv = s_acc[jt][v] * a.scale;
        p[jt][v] = (kp <= qpos && kp < ctx) ? sv : -INFINITY;
        mx = fmaxf(mx, p[jt][v]);
      }
      mx = group_max<16>(mx);
      const float m_new = fmaxf(m_row[v], mx);
      alpha[v] = m_new == -INFINITY ? 1.0f : __expf(m_row[v] - m_new);
      float ls = 0.0f;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt) {
        p[jt][v] = p[jt][v] == -INFINITY ? 0.0f : __expf(p[jt][v] - m_new);
        ls += p[jt][v];
      }
      ls = fi::group_sum<16>(ls);
      l_row[v] = l_row[v] * alpha[v] + ls;
      m_row[v] = m_new;
    }
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) o[t][v] *= alpha[v];
    // P to LDS in accumulator layout, read back as the A operand
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int v = 0; v < 4; ++v) Ps[w][4 * lk + v][16 * jt + li] = p[jt][v];
    __syncthreads();
    // ---- O += P V ----
#pragma unroll
    for (int s = 0; s < kKTile / 4; ++s) {
      const float pa = Ps[w][li][4 * s + lk];
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const float vb = Vs[4 * s + lk][16 * t + li];
        o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(pa, vb, o[t], 0, 0, 0);
      }
    }
    __syncthreads();
  }

#pragma unroll
  for (int v = 0; v < 4; ++v) {
    const int row = r0 + 4 * lk + v;
    if (row >= qlen) continue;
    const float inv = 1.0f / l_row[v];
    float* op = a.out + ((size_t)(qs + row) * a.hq + h) * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) op[16 * t + li] = o[t][v] * inv;
  }
}

template <int D>
int32_t launch_prefill(fi_context* ctx, int32_t dtype, const PrefillArgs& args, dim3 grid) {
  if (dtype == FI_DTYPE_F32) {
    hipLaunchKernelGGL((prefill_kernel<D, float>), grid, dim3(kThreads), 0, ctx->stream, args);
  } else {
    hipLaunchKernelGGL((prefill_kernel<D, uint16_t>), grid, dim3(kThreads), 0, ctx->stream, args);
  }
  FI_CHECK_LAUNCH("prefill_kernel");
  return FI_OK;
}

}  // namespace

extern "C" {

int32_t fi_attn_prefill_paged(fi_context* ctx, const float* d_q, const void* d_k_cache,
                              const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                              int32_t max_blocks_per_seq, const int32_t* d_cu_seqlens,
                              const int32_t* d_context_lens, int32_t num_seqs, int32_t max_query_len,
                              int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                              int32_t block_size, int32_t num_blocks, float scale, float* d_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_seqs >= 0 && max_query_len >= 0, FI_ERR_INVALID_SHAPE, "fi_attn_prefill_paged: negative sizes");
  FI_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, FI_ERR_INVALID_SHAPE,
             "number of query heads must be divisible by number of KV heads");
  FI_REQUIRE(block_size > 0 && num_blocks > 0 && max_blocks_per_seq > 0, FI_ERR_INVALID_CONFIG,
             "fi_attn_prefill_paged: pool dimensions must be greater than zero");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_attn_prefill_paged: KV dtype must be f32 or bf16");
  FI_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, FI_ERR_UNSUPPORTED,
             "fi_attn_prefill_paged: head_dim must be 32, 64 or 128");
  if (num_seqs == 0 || max_query_len == 0) return FI_OK;
  FI_REQUIRE(d_q && d_k_cache && d_v_cache && d_block_tables && d_cu_seqlens && d_context_lens && d_out,
             FI_ERR_INVALID_CONFIG, "fi_attn_prefill_paged: null pointer");
  PrefillArgs args{};
  args.q = d_q;
  args.k_cache = d_k_cache;
  args.v_cache = d_v_cache;
  args.cu_seqlens = d_cu_seqlens;
  args.context_lens = d_context_lens;
  args.block_tables = d_block_tables;
  args.out = d_out;
  args.faults = ctx->d_faults;
  args.max_blocks = max_blocks_per_seq;
  args.hq = num_q_heads;
  args.hkv = num_kv_heads;
  args.group = num_q_heads / num_kv_heads;
  args.block_size = block_size;
  args.num_blocks = num_blocks;
  args.scale = scale;
  dim3 grid((max_query_len + kQTile - 1) / kQTile, num_seqs, num_q_heads);
  switch (head_dim) {
    case 32:
      return launch_prefill<32>(ctx, kv_dtype, args, grid);
    case 64:
      return launch_prefill<64>(ctx, kv_dtype, args, grid);
    default:
      return launch_prefill<128>(ctx, kv_dtype, args, grid);
  }
}

}  // extern "C"
