// Varlen causal prefill attention over the paged KV pool, on MFMA.  f32 pools run
// prefill_x3_kernel (f32 accuracy from three-piece bf16 products on v_mfma_f32_16x16x32_bf16,
// at the end of this file); bf16 pools run prefill_kernel (K/V widened exactly, f32 MFMA,
// v_mfma_f32_16x16x4_f32) or, through fi_attn_prefill_paged_bf16, prefill_bf16_kernel.
// Replaces causal_self_attention_f32 / prefixed_causal_attention_f32 /
// cached_prefixed_causal_attention_f32 (crates/ferrisinfer-kernel/src/cpu/attention.rs:222-518,
// 688-962) plus the paged prefix gather that feeds them (runtime/paged_kv.rs:769-791,
// runtime/reference.rs:425-465) for a ragged batch packed by cu_seqlens.
//
// Sequence b has qlen_b = cu_seqlens[b+1] - cu_seqlens[b] new query tokens at positions
// [ctx_b - qlen_b, ctx_b); query position p attends keys [0, p] read through the block table
// (its own K/V rows must already be appended).
//
// One workgroup = (sequence, kv head, tile of 64·RG/G query tokens) with all G query heads of
// the GQA group: RG 16-row groups per wave (RG = 1 or 2, chosen per launch from the grid
// size), so every K/V byte a workgroup stages serves G heads and, with RG = 2, every LDS
// fragment read feeds two MFMAs.  Keys are processed in chunks (32 keys f32, 64 bf16): the
// chunk's K and V rows are staged in LDS (16-byte loads; bf16 widened for the f32 kernel),
// the next chunk's rows are fetched into registers while the current one is multiplied, two
// barriers per chunk.  The products are taken transposed: S^T = K Q^T leaves each lane the
// scores of one row, so the online softmax needs two cross-lane steps for the row maximum
// and none for the sum until the end, and O^T = V^T P^T takes the probabilities as its B
// operand straight from registers (the key order of its k index is matched in the V reads).
// The causal mask is applied only on chunks that reach past a tile's first query.
//
// Tiles run largest first: a one-workgroup planning kernel sorts the (sequence, tile) pairs by
// the number of key chunks they attend, so the long tiles of long sequences do not start last
// and leave the device idle behind them.
#include "fi_common.h"
#include "fi_device.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kRows = 64;     // (head, token) rows per workgroup
constexpr int kKeys = 32;     // keys per staged chunk

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
  int num_seqs;
  int max_query_len;
  const int* order;          // (sequence, query tile) pairs, largest first
  // prefill_x3_kernel with key splits: each (tile, kv head) runs as kv_splits workgroups over
  // consecutive ranges of its key chunks, writing partials (unnormalised O, reference point and
  // row sum per row) that prefill_split_merge_kernel combines in split order
  int kv_splits;
  float* part;
};

// One workgroup sorts the (sequence, query tile) pairs by the number of kb-key chunks they
// attend, largest first (counting sort over 1024 buckets; order within a bucket arbitrary,
// which no result depends on; tiles past a sequence's end sort last).
__global__ __launch_bounds__(1024) void prefill_plan_kernel(const int* __restrict__ cu, const int* __restrict__ ctxl,
                                                            int num_seqs, int ntiles, int qt_rows, int kb, int fold,
                                                            int* __restrict__ order, uint32_t* __restrict__ faults) {
  __shared__ int hist[1024];
  __shared__ int part[1024];
  __shared__ int s_live;
  const int tid = threadIdx.x;
  const int total = num_seqs * ntiles;
  hist[tid] = 0;
  // a query length beyond the tiles that max_query_len sized: its tail rows get no workgroup
  for (int s = tid; s < num_seqs; s += 1024) {
    if (cu[s + 1] - cu[s] > ntiles * qt_rows) atomicOr(faults, FI_FAULT_QUERY_RANGE);
  }
  __syncthreads();
  auto bucket = [&](int t) {  // 0 = past the sequence's end, else chunks + 1 (capped)
    const int seq = t / ntiles, qt = t - (t / ntiles) * ntiles;
    const int qs = cu[seq], qlen = cu[seq + 1] - qs;
    const int q0 = qt * qt_rows;
    if (q0 >= qlen) return 0;
    const int kend = ctxl[seq] - qlen + min(qlen, q0 + qt_rows);
    return min(max((kend + kb - 1) / kb, 0) + 1, 1023);
  };
  for (int t = tid; t < total; t += 1024) atomicAdd(&hist[1023 - bucket(t)], 1);
  __syncthreads();
  if (tid == 0) s_live = total - hist[1023];  // tiles with rows (bucket 0 sorts last)
  const int v = hist[tid];  // exclusive scan of the bucket counts (Hillis-Steele)
  part[tid] = v;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int x = tid >= off ? part[tid - off] : 0;
    __syncthreads();
    part[tid] += x;
    __syncthreads();
  }
  hist[tid] = part[tid] - v;
  __syncthreads();
  // fold (a launch that fits the device in one round, two workgroups per CU): sorted position
  // p of the n live tiles goes to rank p in the first half and to rank half + (n - 1 - p) in
  // the second, so ranks r and r + half, which the dispatcher places on the same CU, pair a
  // long tile with a short one
  const int n = s_live, half = (n + 1) / 2;
  for (int t = tid; t < total; t += 1024) {
    const int p = atomicAdd(&hist[1023 - bucket(t)], 1);
    order[fold && p < n && p >= half ? half + (n - 1 - p) : p] = t;
  }
}

// Four consecutive K/V elements of one row as raw registers, widened when staged.
template <typename KVT>
struct Quad;
template <>
struct Quad<float> {
  using Raw = float4;
  __device__ static Raw load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ static float4 widen(const Raw& r) { return r; }
  __device__ static Raw zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }
};
template <>
struct Quad<uint16_t> {
  using Raw = uint2;
  __device__ static Raw load(const uint16_t* p) { return *reinterpret_cast<const uint2*>(p); }
  __device__ static float4 widen(const Raw& r) {
    return make_float4(fi::bf16_bits_to_f32(r.x & 0xffffu), fi::bf16_bits_to_f32(r.x >> 16),
                       fi::bf16_bits_to_f32(r.y & 0xffffu), fi::bf16_bits_to_f32(r.y >> 16));
  }
  __device__ static Raw zero() { return make_uint2(0u, 0u); }
};

__device__ __forceinline__ float pick(const float4& v, int e) {
  return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

template <int D, typename KVT, int G, int RG>
__global__ __launch_bounds__(kThreads, 2) void prefill_kernel(PrefillArgs a) {
  using QD = Quad<KVT>;
  constexpr int QT = kRows * RG / G;      // query tokens per workgroup (RG 16-row groups a wave)
  constexpr int DV = D / 4;               // 4-element quads per row
  constexpr int DS = D / 16;              // 16-wide d steps of the Q K^T contraction
  constexpr int DH = D / 64 > 0 ? D / 64 : 1;  // 64-wide halves of the output (D = 32: one, masked)
  constexpr int QUADS = kKeys * DV;       // quads per staged K (or V) chunk
  constexpr int PER_T = (QUADS + kThreads - 1) / kThreads;
  static_assert(QUADS % kThreads == 0, "chunk must split evenly over the workgroup");
  __shared__ float4 Ks[kKeys][DV + 1];
  __shared__ float4 Vs[kKeys][DV + 1];

  const KVT* __restrict__ k_cache = static_cast<const KVT*>(a.k_cache);
  const KVT* __restrict__ v_cache = static_cast<const KVT*>(a.v_cache);
  // Workgroup L takes the (L / Hkv)-th largest (sequence, tile) pair for kv head L % Hkv:
  // the heaviest tiles start first, and hardware workgroup L runs on XCD L % 8, so each XCD
  // keeps to one kv head's K/V (Hkv = 8) or a fixed subset of heads.
  const int ntiles = (a.max_query_len + QT - 1) / QT;
  const int rank = blockIdx.x / a.hkv, kvh = blockIdx.x % a.hkv;
  const int tile = a.order[rank];
  const int qt = tile % ntiles, seq = tile / ntiles;
  const int qs = a.cu_seqlens[seq];
  const int qlen = a.cu_seqlens[seq + 1] - qs;
  const int q0 = qt * QT;
  if (q0 >= qlen) return;
  const int ctx = a.context_lens[seq];
  const int start = ctx - qlen;  // position of the first query token
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lk = lane >> 4;

  // Transposed products on v_mfma_f32_16x16x4_f32.  S^T = K Q^T: MFMA step (t, e) contracts
  // d = 16 t + 4 lk + e, so both operands are float4 LDS / register reads; the accumulator
  // gives lane (li, lk) the scores of row li (of each row group) at keys 16 jt + 4 lk + v.
  // O^T = V^T P^T: MFMA step (jt, v) contracts key 16 jt + 4 lk + v, exactly the key whose
  // probability the lane holds, so P is the B operand straight from registers; output tile
  // (h, p) has d rows 64 h + 4 li + p, so one float4 V read feeds four MFMAs.
  int row_r[RG], qpos[RG];
  float4 qf[RG][DS];  // row li of group g, d = 16 t + 4 lk .. + 3
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    row_r[g] = 16 * (w + 4 * g) + li;
    qpos[g] = start + q0 + row_r[g] % QT;
    const int ah = row_r[g] / QT, at = row_r[g] % QT;
    const bool a_ok = ah < a.group && q0 + at < qlen;
    const float* qp = a.q + ((size_t)(qs + q0 + (a_ok ? at : 0)) * a.hq + kvh * a.group + (a_ok ? ah : 0)) * D;
#pragma unroll
    for (int t = 0; t < DS; ++t)
      qf[g][t] = a_ok ? *reinterpret_cast<const float4*>(qp + 16 * t + 4 * lk) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  v4f o[RG][DH][4];  // O^T tile (h, p) of group g: d = 64 h + 4 (4 lk + v) + p, row li
  float m_row[RG], l_part[RG];  // running max (log2 units); this lane's share of the row sum
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int h = 0; h < DH; ++h)
#pragma unroll
      for (int p = 0; p < 4; ++p) o[g][h][p] = v4f{0.f, 0.f, 0.f, 0.f};
    m_row[g] = -INFINITY;
    l_part[g] = 0.0f;
  }
  const float c2 = a.scale * 1.4426950408889634f;  // scores -> log2 units

  const int kend = start + min(qlen, q0 + QT);  // keys needed by the tile's last token
  const int nchunks = max((kend + kKeys - 1) / kKeys, 1);

  // Chunk staging: quad i = tid + r * kThreads -> key i / DV, quad column i % DV.  The block
  // ids of chunk c + 2 are loaded while chunk c is multiplied and the K/V rows of chunk c + 1
  // are in flight, so no load waits on another.  Every load is unconditional (chunk index and
  // key clamped, padding keys zeroed by a select): a divergent branch around a load makes the
  // compiler drain all outstanding loads where the paths merge.
  typename QD::Raw kr[PER_T], vr[PER_T];
  int ids[PER_T], offs[PER_T];
  bool bad_block = false;
  auto lookup = [&](int c) {  // block ids and in-block rows of chunk c's keys
    c = min(c, nchunks - 1);
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int key = (tid + r * kThreads) / DV;
      const int kpc = max(min(c * kKeys + key, kend - 1), 0);  // kend <= 0 only when ctx < qlen
      const int lb = kpc / a.block_size;
      const bool in_table = lb < a.max_blocks;
      ids[r] = a.block_tables[(size_t)seq * a.max_blocks + (in_table ? lb : 0)];
      ids[r] = in_table ? ids[r] : -1;
      offs[r] = kpc - lb * a.block_size;
    }
  };
  auto fetch = [&](int c) {  // K/V quads of chunk c from the ids of the last lookup
    c = min(c, nchunks - 1);
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int i = tid + r * kThreads;
      const int key = i / DV, col = i % DV;
      const bool valid = c * kKeys + key < kend;
      const bool bad = ids[r] < 0 || ids[r] >= a.num_blocks;
      bad_block |= bad;
      const size_t row = ((size_t)(bad ? 0 : ids[r]) * a.hkv + kvh) * a.block_size + offs[r];
      const typename QD::Raw kx = QD::load(k_cache + row * D + 4 * col);
      const typename QD::Raw vx = QD::load(v_cache + row * D + 4 * col);
      kr[r] = valid ? kx : QD::zero();
      vr[r] = valid ? vx : QD::zero();
    }
  };
  auto stage = [&]() {
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int i = tid + r * kThreads;
      Ks[i / DV][i % DV] = QD::widen(kr[r]);
      Vs[i / DV][i % DV] = QD::widen(vr[r]);
    }
  };

  lookup(0);
  fetch(0);
  lookup(1);
  stage();
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int k0 = c * kKeys;
    fetch(c + 1);   // the last chunk re-reads itself: the loads stay unconditional
    lookup(c + 2);
    __builtin_amdgcn_sched_barrier(0);

    // ---- S^T = K Q^T: 32 keys (2 key tiles) x 16 rows per group ----
    v4f s_acc[RG][2];
#pragma unroll
    for (int g = 0; g < RG; ++g) s_acc[g][0] = s_acc[g][1] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < DS; ++t) {
      const float4 kb0 = Ks[li][4 * t + lk];
      const float4 kb1 = Ks[16 + li][4 * t + lk];
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int g = 0; g < RG; ++g) {
          const float bv = pick(qf[g][t], e);
          s_acc[g][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(pick(kb0, e), bv, s_acc[g][0], 0, 0, 0);
          s_acc[g][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(pick(kb1, e), bv, s_acc[g][1], 0, 0, 0);
        }
    }
    // causal / context mask only where the chunk reaches past the tile's first query position
    // (workgroup-uniform; tested once, outside the unrolled score loops; -inf stays -inf when
    // scaled below)
    if (k0 + kKeys - 1 > start + q0) {
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int jt = 0; jt < 2; ++jt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int kp = k0 + 16 * jt + 4 * lk + v;
            s_acc[g][jt][v] = (kp <= qpos[g] && kp < ctx) ? s_acc[g][jt][v] : -INFINITY;
          }
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      float mx = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float x = s_acc[g][jt][v] * c2;
          s_acc[g][jt][v] = x;
          mx = fmaxf(mx, x);
        }
      mx = fmaxf(mx, fi::lane_xor16(mx, lane));
      mx = fmaxf(mx, fi::lane_xor32(mx, lane));
      const float m_new = fmaxf(m_row[g], mx);  // finite: key 0 of chunk 0 is visible to every row
      const float alpha = __builtin_amdgcn_exp2f(m_row[g] - m_new);
      m_row[g] = m_new;
      float ls = 0.0f;
#pragma unroll
      for (int jt = 0; jt < 2; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float pexp = __builtin_amdgcn_exp2f(s_acc[g][jt][v] - m_new);
          s_acc[g][jt][v] = pexp;
          ls += pexp;
        }
      l_part[g] = l_part[g] * alpha + ls;
#pragma unroll
      for (int h = 0; h < DH; ++h)
#pragma unroll
        for (int p = 0; p < 4; ++p) o[g][h][p] *= alpha;
    }

    // ---- O^T += V^T P^T: MFMA step (jt, v) is key 16 jt + 4 lk + v ----
#pragma unroll
    for (int jt = 0; jt < 2; ++jt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int key = 16 * jt + 4 * lk + v;
#pragma unroll
        for (int h = 0; h < DH; ++h) {
          const float4 va = (D >= 64 || h == 0) && (64 * h + 4 * li < D) ? Vs[key][16 * h + li]
                                                                         : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
          for (int p = 0; p < 4; ++p)
#pragma unroll
            for (int g = 0; g < RG; ++g)
              o[g][h][p] = __builtin_amdgcn_mfma_f32_16x16x4f32(pick(va, p), s_acc[g][jt][v], o[g][h][p], 0, 0, 0);
        }
      }
    __syncthreads();  // every wave is done with this chunk's K/V
    if (c + 1 < nchunks) {
      stage();
      __syncthreads();
    }
  }

  if (bad_block) atomicOr(a.faults, FI_FAULT_BLOCK_RANGE);

  // ---- normalise and store: lane holds row li of each group, d = 64 h + 16 lk + 4 v + p ----
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    float l_row = l_part[g] + fi::lane_xor16(l_part[g], lane);
    l_row += fi::lane_xor32(l_row, lane);
    const int hd = row_r[g] / QT, t = row_r[g] % QT;
    if (hd < a.group && q0 + t < qlen) {
      const float inv = 1.0f / l_row;
      float* op = a.out + ((size_t)(qs + q0 + t) * a.hq + kvh * a.group + hd) * D;
#pragma unroll
      for (int h = 0; h < DH; ++h)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int d0 = 64 * h + 16 * lk + 4 * v;
          if (d0 < D) {
            *reinterpret_cast<float4*>(op + d0) = make_float4(o[g][h][0][v] * inv, o[g][h][1][v] * inv,
                                                              o[g][h][2][v] * inv, o[g][h][3][v] * inv);
          }
        }
    }
  }
}

// Sorts the tiles largest first into the context workspace (one small launch before the
// attention kernel) and sizes the grid: one workgroup per (tile, kv head).
#ifndef FI_PREFILL_FOLD
#define FI_PREFILL_FOLD 1
#endif

int32_t plan_tiles(fi_context* ctx, PrefillArgs& args, int qt, int kb, const char* name, dim3* grid, int splits = 1,
                   size_t part_floats = 0) {
  const int ntiles = (args.max_query_len + qt - 1) / qt;
  const long pairs = (long)ntiles * args.num_seqs;
  FI_REQUIRE(pairs * args.hkv * splits <= 0x7fffffffL, FI_ERR_INVALID_SHAPE, std::string(name) + ": grid too large");
  // the tile order, then (split launches) each workgroup's partials
  const size_t order_bytes = ((size_t)pairs * sizeof(int) + 255) & ~static_cast<size_t>(255);
  const size_t part_bytes = splits > 1 ? (size_t)pairs * args.hkv * splits * part_floats * sizeof(float) : 0;
  FI_TRY(fi::ensure_workspace(ctx, order_bytes + part_bytes));
  int* order = static_cast<int*>(ctx->workspace);
  args.kv_splits = splits;
  args.part = splits > 1 ? reinterpret_cast<float*>(static_cast<char*>(ctx->workspace) + order_bytes) : nullptr;
  // one round of workgroups (two per CU): pair long and short tiles on each CU
  const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  const int fold = FI_PREFILL_FOLD && splits == 1 && pairs * args.hkv <= 2 * cus;
  hipLaunchKernelGGL(prefill_plan_kernel, dim3(1), dim3(1024), 0, ctx->stream, args.cu_seqlens, args.context_lens,
                     args.num_seqs, ntiles, qt, kb, fold, order, ctx->d_faults);
  FI_CHECK_LAUNCH("prefill_plan_kernel");
  args.order = order;
  *grid = dim3(static_cast<unsigned>(pairs * args.hkv * splits));
  return FI_OK;
}

// Row groups per wave: two when the grid still gives every CU two workgroups (every K/V
// fragment read from LDS then feeds two MFMAs), one for launches with few (sequence, tile,
// kv head) triples, such as a prefill chunk over two kv heads.
int row_groups(fi_context* ctx, const PrefillArgs& args, int g) {
  const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  const int qt2 = kRows * 2 / g;
  const long tiles2 = (long)((args.max_query_len + qt2 - 1) / qt2) * args.num_seqs * args.hkv;
  return tiles2 >= 2 * cus ? 2 : 1;
}

template <int D, typename KVT, int RG>
int32_t launch_prefill_rg(fi_context* ctx, PrefillArgs& args, int g) {
  const int qt = kRows * RG / g;
  dim3 grid;
  FI_TRY(plan_tiles(ctx, args, qt, kKeys, "fi_attn_prefill_paged", &grid));
  switch (g) {
    case 1:
      hipLaunchKernelGGL((prefill_kernel<D, KVT, 1, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
    case 2:
      hipLaunchKernelGGL((prefill_kernel<D, KVT, 2, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
    case 4:
      hipLaunchKernelGGL((prefill_kernel<D, KVT, 4, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
    default:
      hipLaunchKernelGGL((prefill_kernel<D, KVT, 8, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
  }
  FI_CHECK_LAUNCH("prefill_kernel");
  return FI_OK;
}

template <int D, typename KVT>
int32_t launch_prefill(fi_context* ctx, const PrefillArgs& args_in) {
  PrefillArgs args = args_in;
  const int g = args.group <= 1 ? 1 : (args.group <= 2 ? 2 : (args.group <= 4 ? 4 : 8));
  return row_groups(ctx, args, g) == 2 ? launch_prefill_rg<D, KVT, 2>(ctx, args, g)
                                       : launch_prefill_rg<D, KVT, 1>(ctx, args, g);
}

// ---- bf16-MFMA variant for a bf16 pool (fi_attn_prefill_paged_bf16) ----
// Same workgroup shape, tile order and chunk pipeline as prefill_kernel, on
// v_mfma_f32_16x16x32_bf16: K and V stay bf16 in LDS, row-major (V^T fragments come from
// ds_read_b64_tr_b16), Q and the softmax probabilities are rounded to bf16 (nearest even);
// scores, softmax and accumulation stay f32.  64-key chunks.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4s lds_v4s;

// ds_read_b64_tr_b16 at an LDS address (8-byte aligned)
__device__ __forceinline__ v4s lds_read_tr16(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(p));
}
#ifndef FI_PREFILL_BF16_WAVES
#define FI_PREFILL_BF16_WAVES 2  // waves per SIMD the register budget must allow
#endif

template <int D, int G, int RG>
__global__ __launch_bounds__(kThreads, FI_PREFILL_BF16_WAVES) void prefill_bf16_kernel(PrefillArgs a) {
  constexpr int QT = kRows * RG / G;    // query tokens per workgroup (RG 16-row groups a wave)
  constexpr int KB = 64;                 // keys per chunk
  constexpr int DS = D / 32;             // 32-wide d steps of Q K^T
  constexpr int DT = D / 16;             // 16-wide output d tiles of P V
  constexpr int JT = KB / 16;            // 16-key score tiles per chunk
  constexpr int KS = KB / 32;            // 32-key steps of P V
  constexpr int RV = D / 8;              // 16-byte vectors per K/V row
  constexpr int PER_T = KB * RV / kThreads;
  static_assert(KB * RV % kThreads == 0 && kThreads % KB == 0, "chunk must split over the workgroup");
  constexpr int KP = D + 8;              // padded LDS rows of V (transposing reads)
  // K rows of D = 128 at 288 bytes: the score fragments' 16-byte reads (16 rows, 4 column
  // groups) run at ~190 B/clk per CU against ~113 B/clk at 272 bytes (measured on gfx950;
  // the transposing V reads run at ~110 B/clk at either pitch)
  constexpr int KPK = D == 128 ? D + 16 : D + 8;
  // double-buffered: chunk c + 1 is staged into the other buffer while chunk c is consumed,
  // so one barrier per chunk orders both the reuse and the new contents
  __shared__ __align__(16) uint16_t Ks[2][KB][KPK];
  __shared__ __align__(16) uint16_t Vs[2][KB][KP];  // row-major like K; read through transpose loads

  const uint16_t* __restrict__ k_cache = static_cast<const uint16_t*>(a.k_cache);
  const uint16_t* __restrict__ v_cache = static_cast<const uint16_t*>(a.v_cache);
  const int ntiles = (a.max_query_len + QT - 1) / QT;
  const int rank = blockIdx.x / a.hkv, kvh = blockIdx.x % a.hkv;
  const int tile = a.order[rank];
  const int qt = tile % ntiles, seq = tile / ntiles;
  const int qs = a.cu_seqlens[seq];
  const int qlen = a.cu_seqlens[seq + 1] - qs;
  const int q0 = qt * QT;
  if (q0 >= qlen) return;
  const int ctx = a.context_lens[seq];
  const int start = ctx - qlen;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int li = lane & 15, lk = lane >> 4;

  // Transposed products: S^T = K Q^T leaves each lane the scores of one row (row li of each
  // of the wave's row groups, keys 16 jt + 4 lk + v of score tile jt), so the row statistics
  // need only the four lanes li + 16 lk, and O^T = V^T P^T takes those scores as its B operand
  // straight from registers: MFMA k index 8 lk + e of 32-key step u stands for key
  // 32 u + 4 lk + e (e < 4) or 32 u + 16 + 4 lk + (e - 4), and V^T is read at the same keys.
  // Every K and V fragment read from LDS serves the wave's RG row groups.
  int row_r[RG], qpos[RG];
  bf16x8 qf[RG][DS];  // B operand: row li of group g, d = 32 t + 8 lk + e
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    row_r[g] = 16 * (w + 4 * g) + li;
    qpos[g] = start + q0 + row_r[g] % QT;
    const int ah = row_r[g] / QT, at = row_r[g] % QT;
    const bool a_ok = ah < a.group && q0 + at < qlen;
    const float* qp = a.q + ((size_t)(qs + q0 + (a_ok ? at : 0)) * a.hq + kvh * a.group + (a_ok ? ah : 0)) * D;
#pragma unroll
    for (int t = 0; t < DS; ++t) {
      const float4 lo = *reinterpret_cast<const float4*>(qp + 32 * t + 8 * lk);
      const float4 hi = *reinterpret_cast<const float4*>(qp + 32 * t + 8 * lk + 4);
      const f32x8 v = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      const f32x8 z = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      qf[g][t] = __builtin_convertvector(a_ok ? v : z, bf16x8);
    }
  }
  v4f o[RG][DT];  // O^T tile dt of group g: d = 16 dt + 4 lk + v, row li
  float m_row[RG], l_part[RG];  // running max (log2 units); this lane's share of the row sum
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[g][dt] = v4f{0.f, 0.f, 0.f, 0.f};
    m_row[g] = -INFINITY;
    l_part[g] = 0.0f;
  }
  const float c2 = a.scale * 1.4426950408889634f;  // scores -> log2 units
  constexpr float kLazy = 8.0f;  // headroom of the exponents' reference point (log2 units)

  const int kend = start + min(qlen, q0 + QT);
  const int nchunks = max((kend + KB - 1) / KB, 1);

  // staging: thread owns key `lane` of the chunk and row vectors w + 4 r; one block lookup per
  // chunk, looked up a chunk ahead, loads unconditional (clamped key, padding keys zeroed)
  uint4 kr[PER_T], vr[PER_T];
  int id_next = 0, off_next = 0;
  bool bad_block = false;
  bool part_next = false, valid_next = true;  // the fetched chunk: partial (uniform), this lane's key valid
  // blocks that divide the chunk (the common case): the lane's block within the chunk and its
  // offset are constants, so the lookup needs no division
  const bool aligned = KB % a.block_size == 0;  // workgroup-uniform
  const int lane_blk = aligned ? lane / a.block_size : 0;
  const int lane_off = aligned ? lane - lane_blk * a.block_size : 0;
  const int chunk_blks = aligned ? KB / a.block_size : 0;
  auto lookup = [&](int c) {
    c = min(c, nchunks - 1);
    const int kpc = max(min(c * KB + lane, kend - 1), 0);
    const bool exact = aligned && c * KB + lane < kend;  // the unclamped key: lb, off are constants
    const int lb = exact ? c * chunk_blks + lane_blk : kpc / a.block_size;
    const bool in_table = lb < a.max_blocks;
    const int id = a.block_tables[(size_t)seq * a.max_blocks + (in_table ? lb : 0)];
    id_next = in_table ? id : -1;
    off_next = exact ? lane_off : kpc - lb * a.block_size;
  };
  auto fetch = [&](int c) {
    c = min(c, nchunks - 1);
    part_next = (c + 1) * KB > kend;  // workgroup-uniform: the chunk has padding keys
    valid_next = c * KB + lane < kend;
    const bool bad = id_next < 0 || id_next >= a.num_blocks;
    bad_block |= bad;
    const size_t row = ((size_t)(bad ? 0 : id_next) * a.hkv + kvh) * a.block_size + off_next;
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int dv = w + 4 * r;
      kr[r] = *reinterpret_cast<const uint4*>(k_cache + row * D + 8 * dv);
      vr[r] = *reinterpret_cast<const uint4*>(v_cache + row * D + 8 * dv);
    }
  };
  // padding keys of a partial chunk are stored as zero (their clamped loads hold a valid row)
  auto stage = [&](int buf) {
    if (part_next && !valid_next) {
#pragma unroll
      for (int r = 0; r < PER_T; ++r) {
        kr[r] = make_uint4(0u, 0u, 0u, 0u);
        vr[r] = make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int dv = w + 4 * r;
      *reinterpret_cast<uint4*>(&Ks[buf][lane][8 * dv]) = kr[r];
      *reinterpret_cast<uint4*>(&Vs[buf][lane][8 * dv]) = vr[r];
    }
  };

  lookup(0);
  fetch(0);
  lookup(1);
  stage(0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const int k0 = c * KB;
    const int buf = c & 1;
    fetch(c + 1);
    lookup(c + 2);
    __builtin_amdgcn_sched_barrier(0);

    // ---- S^T = K Q^T: 64 keys x 16 rows per group ----
    // every K fragment of the chunk is read before the first MFMA (the fence keeps the
    // compiler from sinking the reads back next to their uses)
    bf16x8 kfr[JT][DS];
#pragma unroll
    for (int jt = 0; jt < JT; ++jt)
#pragma unroll
      for (int t = 0; t < DS; ++t) kfr[jt][t] = *reinterpret_cast<const bf16x8*>(&Ks[buf][16 * jt + li][32 * t + 8 * lk]);
    __builtin_amdgcn_sched_barrier(0);
    v4f s_acc[RG][JT];
#pragma unroll
    for (int jt = 0; jt < JT; ++jt) {
#pragma unroll
      for (int g = 0; g < RG; ++g) s_acc[g][jt] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < DS; ++t) {
#pragma unroll
        for (int g = 0; g < RG; ++g)
          s_acc[g][jt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kfr[jt][t], qf[g][t], s_acc[g][jt], 0, 0, 0);
      }
    }
    // causal / context mask only where the chunk reaches past the tile's first query position
    // (workgroup-uniform; tested once, outside the unrolled score loops, so that unmasked chunks
    // run straight-line code)
    if (k0 + KB - 1 > start + q0) {
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int jt = 0; jt < JT; ++jt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int kp = k0 + 16 * jt + 4 * lk + v;
            s_acc[g][jt][v] = (kp <= qpos[g] && kp < ctx) ? s_acc[g][jt][v] : -INFINITY;
          }
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      // raw scores: the maximum is taken before scaling (c2 > 0 and rounding are monotone, so
      // max(s) * c2 is the maximum of the scaled scores) and each exponent is one fma
      float mx = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) mx = fmaxf(mx, s_acc[g][jt][v]);
      mx = fmaxf(mx, fi::lane_xor16(mx, lane));
      mx = fmaxf(mx, fi::lane_xor32(mx, lane));
      // the reference point of the exponents moves only when the chunk's maximum passes it by
      // more than kLazy (log2 units): probabilities stay below 2^kLazy, which f32 sums and the
      // bf16 operand of P V hold with their usual relative precision, and the normalisation by
      // the row sum (taken against the same point) cancels it.  Chunk 0 always sets it (finite:
      // key 0 is visible to every row).
      const float m_chunk = mx * c2;
      const float m_new = m_chunk > m_row[g] + kLazy ? m_chunk : m_row[g];
      const float alpha = __builtin_amdgcn_exp2f(m_row[g] - m_new);
      m_row[g] = m_new;
      float ls = 0.0f;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float pexp = __builtin_amdgcn_exp2f(fmaf(s_acc[g][jt][v], c2, -m_new));
          s_acc[g][jt][v] = pexp;
          ls += pexp;
        }
      l_part[g] = l_part[g] * alpha + ls;
      // alpha is exactly 1 where the reference point did not move: skip the rescale when that
      // holds for every lane of the wave (after the first chunks, nearly always)
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[g][dt] *= alpha;
      }
    }

    // ---- O^T += V^T P^T over the chunk's 32-key steps ----
#pragma unroll
    for (int u = 0; u < KS; ++u) {
      bf16x8 pb[RG];
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        const f32x8 pf = {s_acc[g][2 * u][0], s_acc[g][2 * u][1], s_acc[g][2 * u][2], s_acc[g][2 * u][3],
                          s_acc[g][2 * u + 1][0], s_acc[g][2 * u + 1][1], s_acc[g][2 * u + 1][2],
                          s_acc[g][2 * u + 1][3]};
        pb[g] = __builtin_convertvector(pf, bf16x8);  // nearest even
      }
      // ds_read_b64_tr_b16: within each 16-lane group, lane i receives element i % 4 of the
      // 8-byte reads of lanes 4 e + i / 4 (e = 0..3).  Lane (li, lk) points at key
      // 32 u + 4 lk + li / 4 (+ 16 for the upper half), d 16 dt + 4 (li % 4) .. + 3, so it
      // receives V at d = 16 dt + li for keys 32 u + 4 lk + e (+ 16): the keys its P holds.
      const int vrow = 32 * u + 4 * lk + (li >> 2), vcol = 4 * (li & 3);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        const v4s lo = lds_read_tr16(&Vs[buf][vrow][16 * dt + vcol]);
        const v4s hi = lds_read_tr16(&Vs[buf][vrow + 16][16 * dt + vcol]);
        const bf16x8 va = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
#pragma unroll
        for (int g = 0; g < RG; ++g) o[g][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pb[g], o[g][dt], 0, 0, 0);
      }
    }
    // the other buffer was last read in chunk c - 1, which every wave finished before the
    // previous barrier; this barrier publishes chunk c + 1 and retires chunk c's buffer
    if (c + 1 < nchunks) stage(buf ^ 1);  // workgroup-uniform
    __syncthreads();
  }

  if (bad_block) atomicOr(a.faults, FI_FAULT_BLOCK_RANGE);

  // ---- normalise and store: lane holds row li of each group, d = 16 dt + 4 lk + v ----
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    float l_row = l_part[g] + fi::lane_xor16(l_part[g], lane);
    l_row += fi::lane_xor32(l_row, lane);
    const int h = row_r[g] / QT, t = row_r[g] % QT;
    if (h < a.group && q0 + t < qlen) {
      const float inv = 1.0f / l_row;
      float* op = a.out + ((size_t)(qs + q0 + t) * a.hq + kvh * a.group + h) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        *reinterpret_cast<float4*>(op + 16 * dt + 4 * lk) =
            make_float4(o[g][dt][0] * inv, o[g][dt][1] * inv, o[g][dt][2] * inv, o[g][dt][3] * inv);
      }
    }
  }
}

template <int D, int RG>
int32_t launch_prefill_bf16_rg(fi_context* ctx, PrefillArgs& args, int g) {
  const int qt = kRows * RG / g;
  dim3 grid;
  FI_TRY(plan_tiles(ctx, args, qt, 64, "fi_attn_prefill_paged_bf16", &grid));
  switch (g) {
    case 1:
      hipLaunchKernelGGL((prefill_bf16_kernel<D, 1, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
    case 2:
      hipLaunchKernelGGL((prefill_bf16_kernel<D, 2, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
    case 4:
      hipLaunchKernelGGL((prefill_bf16_kernel<D, 4, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
    default:
      hipLaunchKernelGGL((prefill_bf16_kernel<D, 8, RG>), grid, dim3(kThreads), 0, ctx->stream, args);
      break;
  }
  FI_CHECK_LAUNCH("prefill_bf16_kernel");
  return FI_OK;
}

template <int D>
int32_t launch_prefill_bf16(fi_context* ctx, const PrefillArgs& args_in) {
  PrefillArgs args = args_in;
  const int g = args.group <= 1 ? 1 : (args.group <= 2 ? 2 : (args.group <= 4 ? 4 : 8));
  return row_groups(ctx, args, g) == 2 ? launch_prefill_bf16_rg<D, 2>(ctx, args, g)
                                       : launch_prefill_bf16_rg<D, 1>(ctx, args, g);
}

// ---- f32 pools in f32 accuracy on bf16 MFMA (fi_attn_prefill_paged over an f32 pool) ----
// The workgroup shape, tile order, transposed products, masking and softmax of
// prefill_bf16_kernel, with every operand carried in f32 accuracy: K and V are split exactly
// into three bf16 planes (x = hi + mid + lo: hi = RNE(x), mid = RNE(x - hi), lo the rest) when
// a 32-key chunk is staged, Q and the probabilities are split on use, and each product is the
// sum of the six cross products above 2^-24 relative (the three dropped ones are below one f32
// rounding together), accumulated in f32 on v_mfma_f32_16x16x32_bf16: the f32 result at 2.7x
// the f32 MFMA rate.  One LDS buffer (52 KB at D = 128, two workgroups per CU); the next chunk
// is in registers while the current one is multiplied, two barriers per chunk.
__device__ __forceinline__ void split3(const f32x8& x, bf16x8 (&p)[3]) {
  uint4 h, m, l;
  fi::split3_pk(x[0], x[1], h.x, m.x, l.x);
  fi::split3_pk(x[2], x[3], h.y, m.y, l.y);
  fi::split3_pk(x[4], x[5], h.z, m.z, l.z);
  fi::split3_pk(x[6], x[7], h.w, m.w, l.w);
  p[0] = __builtin_bit_cast(bf16x8, h);
  p[1] = __builtin_bit_cast(bf16x8, m);
  p[2] = __builtin_bit_cast(bf16x8, l);
}

// four f32 values -> their three bf16 pieces, each as 8 bytes
__device__ __forceinline__ void split3_quad(const float4& v, uint2 (&p)[3]) {
  fi::split3_pk(v.x, v.y, p[0].x, p[1].x, p[2].x);
  fi::split3_pk(v.z, v.w, p[0].y, p[1].y, p[2].y);
}

// acc += A B over three-piece operands: the six cross products above 2^-24, smallest first
__device__ __forceinline__ v4f mma6(const bf16x8 (&a)[3], const bf16x8 (&b)[3], v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[1], acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[0], b[0], acc, 0, 0, 0);
}

template <int D, int G, int RG, bool SPLIT>
__global__ __launch_bounds__(kThreads, 2) void prefill_x3_kernel(PrefillArgs a) {
  constexpr int QT = kRows * RG / G;    // query tokens per workgroup (RG 16-row groups a wave)
  constexpr int KB = 32;                 // keys per chunk: one 32-key step of P V
  constexpr int DS = D / 32;             // 32-wide d steps of Q K^T
  constexpr int DT = D / 16;             // 16-wide output d tiles of P V
  constexpr int JT = KB / 16;            // 16-key score tiles per chunk
  constexpr int DQ = D / 4;              // float4 quads per K/V row
  constexpr int KR = kThreads / KB;      // quad columns staged per pass (thread: key tid % KB)
  constexpr int PER_T = DQ / KR;         // quads per thread per K (and V) chunk
  static_assert(DQ % KR == 0 && PER_T >= 1, "chunk must split over the workgroup");
  constexpr int KP = D + 8;              // padded LDS rows
  __shared__ __align__(16) uint16_t Ks[3][KB][KP];  // the three pieces of K, row-major
  __shared__ __align__(16) uint16_t Vs[3][KB][KP];  // of V, read through transpose loads

  const float* __restrict__ k_cache = static_cast<const float*>(a.k_cache);
  const float* __restrict__ v_cache = static_cast<const float*>(a.v_cache);
  const int ntiles = (a.max_query_len + QT - 1) / QT;
  const int wg = blockIdx.x / a.hkv, kvh = blockIdx.x % a.hkv;
  const int rank = SPLIT ? wg / a.kv_splits : wg;
  const int split = SPLIT ? wg - rank * a.kv_splits : 0;
  const int tile = a.order[rank];
  const int qt = tile % ntiles, seq = tile / ntiles;
  const int qs = a.cu_seqlens[seq];
  const int qlen = a.cu_seqlens[seq + 1] - qs;
  const int q0 = qt * QT;
  if (q0 >= qlen) return;
  const int ctx = a.context_lens[seq];
  const int start = ctx - qlen;
  // the wave index is wave-uniform: held in a scalar register through the chunk loop
  const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int li = lane & 15, lk = lane >> 4;

  // Q stays f32 (B operand row li of group g, d = 32 t + 8 lk .. +7) and is split on use
  int row_r[RG], qpos[RG];
  f32x8 qf[RG][DS];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    row_r[g] = 16 * (w + 4 * g) + li;
    qpos[g] = start + q0 + row_r[g] % QT;
    const int ah = row_r[g] / QT, at = row_r[g] % QT;
    const bool a_ok = ah < a.group && q0 + at < qlen;
    const float* qp = a.q + ((size_t)(qs + q0 + (a_ok ? at : 0)) * a.hq + kvh * a.group + (a_ok ? ah : 0)) * D;
#pragma unroll
    for (int t = 0; t < DS; ++t) {
      const float4 lo = *reinterpret_cast<const float4*>(qp + 32 * t + 8 * lk);
      const float4 hi = *reinterpret_cast<const float4*>(qp + 32 * t + 8 * lk + 4);
      const f32x8 v = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
      const f32x8 z = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      qf[g][t] = a_ok ? v : z;
    }
  }
  v4f o[RG][DT];  // O^T tile dt of group g: d = 16 dt + 4 lk + v, row li
  float m_row[RG], l_part[RG];
#pragma unroll
  for (int g = 0; g < RG; ++g) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[g][dt] = v4f{0.f, 0.f, 0.f, 0.f};
    m_row[g] = -INFINITY;
    l_part[g] = 0.0f;
  }
  const float c2 = a.scale * 1.4426950408889634f;  // scores -> log2 units
  constexpr float kLazy = 8.0f;  // headroom of the exponents' reference point (log2 units)

  const int kend = start + min(qlen, q0 + QT);
  const int nchunks = max((kend + KB - 1) / KB, 1);
  // the chunks this workgroup multiplies: all, or its split's consecutive share
  const int c_lo = SPLIT ? split * nchunks / a.kv_splits : 0;
  const int c_hi = SPLIT ? (split + 1) * nchunks / a.kv_splits : nchunks;

  // staging: thread owns key tid % KB of the chunk and quad columns tid / KB + KR r; one block
  // lookup per chunk, looked up a chunk ahead; loads unconditional (clamped key)
  const int skey = tid % KB, sq0 = tid / KB;
  float4 kr[PER_T], vr[PER_T];
  int id_next = 0, off_next = 0;
  bool bad_block = false;
  bool part_next = false, valid_next = true;
  const bool aligned = KB % a.block_size == 0;  // workgroup-uniform
  const int key_blk = aligned ? skey / a.block_size : 0;
  const int key_off = aligned ? skey - key_blk * a.block_size : 0;
  const int chunk_blks = aligned ? KB / a.block_size : 0;
  auto lookup = [&](int c) {
    c = min(c, nchunks - 1);
    const int kpc = max(min(c * KB + skey, kend - 1), 0);
    const bool exact = aligned && c * KB + skey < kend;
    const int lb = exact ? c * chunk_blks + key_blk : kpc / a.block_size;
    const bool in_table = lb < a.max_blocks;
    const int id = a.block_tables[(size_t)seq * a.max_blocks + (in_table ? lb : 0)];
    id_next = in_table ? id : -1;
    off_next = exact ? key_off : kpc - lb * a.block_size;
  };
  // K rows of the next chunk are fetched after the score products, V rows after P V: the V
  // registers are then not live through P V, which with the K registers and f32 Q would
  // exceed the 256 VGPRs of two waves a SIMD
  size_t row_next = 0;
  auto fetch = [&](int c) {
    c = min(c, nchunks - 1);
    part_next = (c + 1) * KB > kend;  // workgroup-uniform: the chunk has padding keys
    valid_next = c * KB + skey < kend;
    const bool bad = id_next < 0 || id_next >= a.num_blocks;
    bad_block |= bad;
    row_next = ((size_t)(bad ? 0 : id_next) * a.hkv + kvh) * a.block_size + off_next;
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int dq = sq0 + KR * r;
      kr[r] = *reinterpret_cast<const float4*>(k_cache + row_next * D + 4 * dq);
    }
  };
  auto fetch_v = [&]() {
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int dq = sq0 + KR * r;
      vr[r] = *reinterpret_cast<const float4*>(v_cache + row_next * D + 4 * dq);
    }
  };
  // padding keys of a partial chunk are stored as zero (their clamped loads hold a valid row)
  auto stage = [&]() {
    if (part_next && !valid_next) {
#pragma unroll
      for (int r = 0; r < PER_T; ++r) kr[r] = vr[r] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int r = 0; r < PER_T; ++r) {
      const int dq = sq0 + KR * r;
      uint2 pk[3], pv[3];
      split3_quad(kr[r], pk);
      split3_quad(vr[r], pv);
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        *reinterpret_cast<uint2*>(&Ks[p][skey][4 * dq]) = pk[p];
        *reinterpret_cast<uint2*>(&Vs[p][skey][4 * dq]) = pv[p];
      }
      __builtin_amdgcn_sched_barrier(0);  // one quad's pieces live at a time
    }
  };

  lookup(c_lo);
  fetch(c_lo);
  fetch_v();
  lookup(c_lo + 1);
  stage();
  __syncthreads();
  for (int c = c_lo; c < c_hi; ++c) {
    const int k0 = c * KB;

    // ---- S^T = K Q^T: 32 keys x 16 rows per group ----
    v4f s_acc[RG][JT];
#pragma unroll
    for (int g = 0; g < RG; ++g)
#pragma unroll
      for (int jt = 0; jt < JT; ++jt) s_acc[g][jt] = v4f{0.f, 0.f, 0.f, 0.f};
    // K fragments one d step ahead of their MFMAs, in two register slots (each step fenced, so
    // the lookahead and the registers it holds stay bounded)
    bf16x8 kf[2][JT][3];
    auto read_k = [&](int t, int slot) {
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int p = 0; p < 3; ++p)
          kf[slot][jt][p] = *reinterpret_cast<const bf16x8*>(&Ks[p][16 * jt + li][32 * t + 8 * lk]);
    };
    read_k(0, 0);
#pragma unroll
    for (int t = 0; t < DS; ++t) {
      if (t + 1 < DS) read_k(t + 1, (t + 1) & 1);
#pragma unroll
      for (int g = 0; g < RG; ++g) {
        bf16x8 qp[3];
        split3(qf[g][t], qp);
#pragma unroll
        for (int jt = 0; jt < JT; ++jt) s_acc[g][jt] = mma6(kf[t & 1][jt], qp, s_acc[g][jt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // the next chunk's K rows are fetched here, after the score products (whose K fragments
    // and Q pieces are the register peak), and land during the softmax and P V
    __builtin_amdgcn_sched_barrier(0);
    fetch(c + 1);  // the last chunk re-reads itself: the loads stay unconditional
    lookup(c + 2);
    __builtin_amdgcn_sched_barrier(0);
    // causal / context mask only where the chunk reaches past the tile's first query position
    // (workgroup-uniform, tested once outside the unrolled score loops)
    if (k0 + KB - 1 > start + q0) {
#pragma unroll
      for (int g = 0; g < RG; ++g)
#pragma unroll
        for (int jt = 0; jt < JT; ++jt)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int kp = k0 + 16 * jt + 4 * lk + v;
            s_acc[g][jt][v] = (kp <= qpos[g] && kp < ctx) ? s_acc[g][jt][v] : -INFINITY;
          }
    }
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      // the softmax of prefill_bf16_kernel: maximum of the raw scores, a lazily moved reference
      // point, one fma per exponent, the rescale skipped where no row's point moved
      float mx = -INFINITY;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) mx = fmaxf(mx, s_acc[g][jt][v]);
      mx = fmaxf(mx, fi::lane_xor16(mx, lane));
      mx = fmaxf(mx, fi::lane_xor32(mx, lane));
      const float m_chunk = mx * c2;
      const float m_new = m_chunk > m_row[g] + kLazy ? m_chunk : m_row[g];
      // a split's first chunks may hold no key a row sees (it starts past the row's
      // position): its reference point stays -inf and its probabilities 0 until one does
      const bool none = SPLIT && m_new == -INFINITY;
      const float alpha = none ? 1.0f : __builtin_amdgcn_exp2f(m_row[g] - m_new);
      m_row[g] = m_new;
      float ls = 0.0f;
#pragma unroll
      for (int jt = 0; jt < JT; ++jt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float pexp = none ? 0.0f : __builtin_amdgcn_exp2f(fmaf(s_acc[g][jt][v], c2, -m_new));
          s_acc[g][jt][v] = pexp;
          ls += pexp;
        }
      l_part[g] = l_part[g] * alpha + ls;
      if (__builtin_amdgcn_ballot_w64(alpha != 1.0f) != 0) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) o[g][dt] *= alpha;
      }
    }

    // ---- O^T += V^T P^T over the chunk's 32 keys (MFMA k index 8 lk + e: key 4 lk + e for
    // e < 4, 16 + 4 lk + e - 4 above, the keys this lane's probabilities belong to) ----
    bf16x8 pp[RG][3];
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      const f32x8 pf = {s_acc[g][0][0], s_acc[g][0][1], s_acc[g][0][2], s_acc[g][0][3],
                        s_acc[g][1][0], s_acc[g][1][1], s_acc[g][1][2], s_acc[g][1][3]};
      split3(pf, pp[g]);
    }
    // ds_read_b64_tr_b16 as in prefill_bf16_kernel: lane (li, lk) points at key 4 lk + li / 4
    // (+ 16 for the upper half), d 16 dt + 4 (li % 4) .. + 3, and receives V at d = 16 dt + li
    // for keys 4 lk + e (+ 16)
    const int vrow = 4 * lk + (li >> 2), vcol = 4 * (li & 3);
    // one d tile's V^T fragments at a time: the staging registers of the next chunk are live
    // here, and a second slot (reads one tile ahead) measured slower for the spills it adds
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      bf16x8 vf[3];
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const v4s lo = lds_read_tr16(&Vs[p][vrow][16 * dt + vcol]);
        const v4s hi = lds_read_tr16(&Vs[p][vrow + 16][16 * dt + vcol]);
        vf[p] = __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
#pragma unroll
      for (int g = 0; g < RG; ++g) o[g][dt] = mma6(vf, pp[g], o[g][dt]);
      __builtin_amdgcn_sched_barrier(0);
    }
    fetch_v();  // its V rows: the loads are in flight while the waves meet at the barrier
    __syncthreads();  // every wave is done with this chunk's K/V
    if (c + 1 < c_hi) {  // workgroup-uniform
      stage();
      __syncthreads();
    }
  }

  if (bad_block) atomicOr(a.faults, FI_FAULT_BLOCK_RANGE);

  // ---- normalise and store: lane holds row li of each group, d = 16 dt + 4 lk + v ----
  // the lane's row and column are formed again here (lane id from mbcnt, the sequence's rows
  // reloaded) rather than kept live through the chunk loop, where registers are at the limit
  const int lane_e = __builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u));
  const int li_e = lane_e & 15, lk_e = lane_e >> 4;
  if constexpr (SPLIT) {
    // this split's partials: O [rows][D] unnormalised, then (reference point, row sum) [rows],
    // for every row of the tile (the merge skips the padding ones)
    constexpr int ROWS = kRows * RG;
    const size_t unit = ((size_t)tile * a.kv_splits + split) * a.hkv + kvh;
    float* po = a.part + unit * ROWS * D;
    float* pml = a.part + (size_t)gridDim.x * ROWS * D + unit * ROWS * 2;
#pragma unroll
    for (int g = 0; g < RG; ++g) {
      float l_row = l_part[g] + fi::lane_xor16(l_part[g], lane);
      l_row += fi::lane_xor32(l_row, lane);
      const int rr = 16 * (w + 4 * g) + li_e;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        *reinterpret_cast<float4*>(po + (size_t)rr * D + 16 * dt + 4 * lk_e) =
            make_float4(o[g][dt][0], o[g][dt][1], o[g][dt][2], o[g][dt][3]);
      if (lk_e == 0) *reinterpret_cast<float2*>(pml + (size_t)rr * 2) = make_float2(m_row[g], l_row);
    }
    return;
  }
  const int qs_e = a.cu_seqlens[seq], qlen_e = a.cu_seqlens[seq + 1] - qs_e;
#pragma unroll
  for (int g = 0; g < RG; ++g) {
    float l_row = l_part[g] + fi::lane_xor16(l_part[g], lane);
    l_row += fi::lane_xor32(l_row, lane);
    const int rr = 16 * (w + 4 * g) + li_e;
    const int h = rr / QT, t = rr % QT;
    if (h < a.group && q0 + t < qlen_e) {
      const float inv = 1.0f / l_row;
      float* op = a.out + ((size_t)(qs_e + q0 + t) * a.hq + kvh * a.group + h) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        *reinterpret_cast<float4*>(op + 16 * dt + 4 * lk_e) =
            make_float4(o[g][dt][0] * inv, o[g][dt][1] * inv, o[g][dt][2] * inv, o[g][dt][3] * inv);
      }
    }
  }
}

#ifndef FI_PREFILL_MAX_SPLITS
#define FI_PREFILL_MAX_SPLITS 4  // key splits of a small f32-pool prefill launch, at most
#endif

// One workgroup per (tile, kv head) of a split launch: each row's output is the splits'
// partials combined in split order, each rescaled from its own reference point to the largest
// (a split with no key the row sees carries -inf and adds nothing; the split holding key 0
// always sees one), then normalised by the combined row sum.
template <int D, int RG>
__global__ __launch_bounds__(kThreads) void prefill_split_merge_kernel(PrefillArgs a, int qt_tokens, int ntiles) {
  constexpr int ROWS = kRows * RG, DQ = D / 4;
  constexpr int ITER = ROWS * DQ / kThreads;  // (row, column quad) items a thread
  constexpr int BATCH = ITER < 4 ? ITER : 4;  // items whose loads are issued together
  constexpr int MAXS = FI_PREFILL_MAX_SPLITS;
  static_assert(ROWS * DQ % kThreads == 0 && ITER % BATCH == 0, "items must split over the workgroup");
  const int tile = blockIdx.x / a.hkv, kvh = blockIdx.x % a.hkv;
  const int seq = tile / ntiles, q0 = (tile % ntiles) * qt_tokens;
  const int qs = a.cu_seqlens[seq], qlen = a.cu_seqlens[seq + 1] - qs;
  if (q0 >= qlen) return;
  const int S = a.kv_splits;
  const float* pml = a.part + (size_t)gridDim.x * S * ROWS * D;
  const size_t unit0 = (size_t)tile * S * a.hkv + kvh;  // split sp: unit0 + sp * hkv
  for (int it0 = 0; it0 < ITER; it0 += BATCH) {
    // every split's (point, sum) and O quad of BATCH items are loaded before any is combined
    // (splits past S read split 0 and are dropped)
    float2 ml[BATCH][MAXS];
    float4 ov[BATCH][MAXS];
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const int idx = threadIdx.x + (it0 + b) * kThreads;
      const int r = idx / DQ, dq = idx - (idx / DQ) * DQ;
#pragma unroll
      for (int sp = 0; sp < MAXS; ++sp) {
        const size_t unit = unit0 + (size_t)(sp < S ? sp : 0) * a.hkv;
        ml[b][sp] = *reinterpret_cast<const float2*>(pml + (unit * ROWS + r) * 2);
        ov[b][sp] = *reinterpret_cast<const float4*>(a.part + (unit * ROWS + r) * D + 4 * dq);
      }
    }
#pragma unroll
    for (int b = 0; b < BATCH; ++b) {
      const int idx = threadIdx.x + (it0 + b) * kThreads;
      const int r = idx / DQ, dq = idx - (idx / DQ) * DQ;
      const int h = r / qt_tokens, t = r - (r / qt_tokens) * qt_tokens;
      if (h >= a.group || q0 + t >= qlen) continue;
      float mx = -INFINITY;
#pragma unroll
      for (int sp = 0; sp < MAXS; ++sp)
        if (sp < S) mx = fmaxf(mx, ml[b][sp].x);
      float l = 0.0f;
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
      for (int sp = 0; sp < MAXS; ++sp) {
        if (sp >= S || ml[b][sp].x == -INFINITY) continue;
        const float wgt = __builtin_amdgcn_exp2f(ml[b][sp].x - mx);
        const float4 o = ov[b][sp];
        l = l + wgt * ml[b][sp].y;
        acc = make_float4(acc.x + wgt * o.x, acc.y + wgt * o.y, acc.z + wgt * o.z, acc.w + wgt * o.w);
      }
      const float inv = 1.0f / l;
      *reinterpret_cast<float4*>(a.out + ((size_t)(qs + q0 + t) * a.hq + kvh * a.group + h) * D + 4 * dq) =
          make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
  }
}

template <int D, int G, int RG, bool SPLIT>
void launch_x3(fi_context* ctx, const PrefillArgs& args, dim3 grid) {
  hipLaunchKernelGGL((prefill_x3_kernel<D, G, RG, SPLIT>), grid, dim3(kThreads), 0, ctx->stream, args);
}

template <int D, int RG, bool SPLIT>
void launch_x3_g(fi_context* ctx, const PrefillArgs& args, dim3 grid, int g) {
  switch (g) {
    case 1:
      launch_x3<D, 1, RG, SPLIT>(ctx, args, grid);
      break;
    case 2:
      launch_x3<D, 2, RG, SPLIT>(ctx, args, grid);
      break;
    case 4:
      launch_x3<D, 4, RG, SPLIT>(ctx, args, grid);
      break;
    default:
      launch_x3<D, 8, RG, SPLIT>(ctx, args, grid);
      break;
  }
}

template <int D, int RG>
int32_t launch_prefill_x3_rg(fi_context* ctx, PrefillArgs& args, int g) {
  const int qt = kRows * RG / g;
  // Key splits for launches that leave most workgroup slots empty (one row group; a launch with
  // two per CU runs two row groups a wave instead): up to four workgroups a CU, each with at
  // least two 32-key chunks (a tile's keys are at least max_query_len).
  int splits = 1;
  if (RG == 1) {
    const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
    const long wgs = (long)((args.max_query_len + qt - 1) / qt) * args.num_seqs * args.hkv;
    splits = static_cast<int>(std::min<long>(FI_PREFILL_MAX_SPLITS, (4 * cus) / std::max<long>(wgs, 1)));
    splits = std::max(1, std::min(splits, args.max_query_len / 64));
  }
  dim3 grid;
  FI_TRY(plan_tiles(ctx, args, qt, 32, "fi_attn_prefill_paged", &grid, splits, kRows * RG * (D + 2)));
  if constexpr (RG == 1) {
    if (splits > 1) {
      launch_x3_g<D, RG, true>(ctx, args, grid, g);
      FI_CHECK_LAUNCH("prefill_x3_kernel");
      const int ntiles = (args.max_query_len + qt - 1) / qt;
      hipLaunchKernelGGL((prefill_split_merge_kernel<D, RG>), dim3(grid.x / splits), dim3(kThreads), 0, ctx->stream,
                         args, qt, ntiles);
      FI_CHECK_LAUNCH("prefill_split_merge_kernel");
      return FI_OK;
    }
  }
  launch_x3_g<D, RG, false>(ctx, args, grid, g);
  FI_CHECK_LAUNCH("prefill_x3_kernel");
  return FI_OK;
}

template <int D>
int32_t launch_prefill_x3(fi_context* ctx, const PrefillArgs& args_in) {
  PrefillArgs args = args_in;
  const int g = args.group <= 1 ? 1 : (args.group <= 2 ? 2 : (args.group <= 4 ? 4 : 8));
  return row_groups(ctx, args, g) == 2 ? launch_prefill_x3_rg<D, 2>(ctx, args, g)
                                       : launch_prefill_x3_rg<D, 1>(ctx, args, g);
}

// f32 pools: the three-piece bf16 kernel; bf16 pools: K/V widened exactly to f32 on f32 MFMA
template <int D>
int32_t launch_prefill_dtype(fi_context* ctx, int32_t dtype, const PrefillArgs& args) {
  if (dtype == FI_DTYPE_F32) return launch_prefill_x3<D>(ctx, args);
  return launch_prefill<D, uint16_t>(ctx, args);
}

// Checks the arguments of a prefill entry point and fills the kernel arguments; *empty when
// there is nothing to compute.
int32_t prefill_args(fi_context* ctx, const char* name, const float* d_q, const void* d_k_cache,
                     const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                     int32_t max_blocks_per_seq, const int32_t* d_cu_seqlens, const int32_t* d_context_lens,
                     int32_t num_seqs, int32_t max_query_len, int32_t num_q_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t block_size, int32_t num_blocks, float scale, float* d_out,
                     PrefillArgs* args, bool* empty) {
  const std::string n(name);
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_seqs >= 0 && max_query_len >= 0, FI_ERR_INVALID_SHAPE, n + ": negative sizes");
  FI_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0, FI_ERR_INVALID_SHAPE,
             "number of query heads must be divisible by number of KV heads");
  FI_REQUIRE(block_size > 0 && num_blocks > 0 && max_blocks_per_seq > 0, FI_ERR_INVALID_CONFIG,
             n + ": pool dimensions must be greater than zero");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             n + ": KV dtype must be f32 or bf16");
  FI_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, FI_ERR_UNSUPPORTED,
             n + ": head_dim must be 32, 64 or 128");
  FI_REQUIRE(num_q_heads / num_kv_heads <= 8, FI_ERR_UNSUPPORTED, n + " supports at most 8 query heads per KV head");
  *empty = num_seqs == 0 || max_query_len == 0;
  if (*empty) return FI_OK;
  FI_REQUIRE(d_q && d_k_cache && d_v_cache && d_block_tables && d_cu_seqlens && d_context_lens && d_out,
             FI_ERR_INVALID_CONFIG, n + ": null pointer");
  FI_REQUIRE((reinterpret_cast<uintptr_t>(d_q) & 15) == 0 && (reinterpret_cast<uintptr_t>(d_out) & 15) == 0 &&
                 (reinterpret_cast<uintptr_t>(d_k_cache) & 15) == 0 && (reinterpret_cast<uintptr_t>(d_v_cache) & 15) == 0,
             FI_ERR_INVALID_LAYOUT, n + ": q, out and the K/V pools must be 16-byte aligned (vector accesses)");
  PrefillArgs& g = *args;
  g = PrefillArgs{};
  g.q = d_q;
  g.k_cache = d_k_cache;
  g.v_cache = d_v_cache;
  g.cu_seqlens = d_cu_seqlens;
  g.context_lens = d_context_lens;
  g.block_tables = d_block_tables;
  g.out = d_out;
  g.faults = ctx->d_faults;
  g.max_blocks = max_blocks_per_seq;
  g.hq = num_q_heads;
  g.hkv = num_kv_heads;
  g.group = num_q_heads / num_kv_heads;
  g.block_size = block_size;
  g.num_blocks = num_blocks;
  g.scale = scale;
  g.num_seqs = num_seqs;
  g.max_query_len = max_query_len;
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
  PrefillArgs args{};
  bool empty = false;
  FI_TRY(prefill_args(ctx, "fi_attn_prefill_paged", d_q, d_k_cache, d_v_cache, kv_dtype, d_block_tables,
                      max_blocks_per_seq, d_cu_seqlens, d_context_lens, num_seqs, max_query_len, num_q_heads,
                      num_kv_heads, head_dim, block_size, num_blocks, scale, d_out, &args, &empty));
  if (empty) return FI_OK;
  switch (head_dim) {
    case 32:
      return launch_prefill_dtype<32>(ctx, kv_dtype, args);
    case 64:
      return launch_prefill_dtype<64>(ctx, kv_dtype, args);
    default:
      return launch_prefill_dtype<128>(ctx, kv_dtype, args);
  }
}

int32_t fi_attn_prefill_paged_bf16(fi_context* ctx, const float* d_q, const void* d_k_cache,
                                   const void* d_v_cache, const int32_t* d_block_tables,
                                   int32_t max_blocks_per_seq, const int32_t* d_cu_seqlens,
                                   const int32_t* d_context_lens, int32_t num_seqs, int32_t max_query_len,
                                   int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim,
                                   int32_t block_size, int32_t num_blocks, float scale, float* d_out) {
  PrefillArgs args{};
  bool empty = false;
  FI_TRY(prefill_args(ctx, "fi_attn_prefill_paged_bf16", d_q, d_k_cache, d_v_cache, FI_DTYPE_BF16,
                      d_block_tables, max_blocks_per_seq, d_cu_seqlens, d_context_lens, num_seqs, max_query_len,
                      num_q_heads, num_kv_heads, head_dim, block_size, num_blocks, scale, d_out, &args, &empty));
  if (empty) return FI_OK;
  switch (head_dim) {
    case 32:
      return launch_prefill_bf16<32>(ctx, args);
    case 64:
      return launch_prefill_bf16<64>(ctx, args);
    default:
      return launch_prefill_bf16<128>(ctx, args);
  }
}

}  // extern "C"
