// Paged decode attention (split-KV with a log-sum-exp merge), KV append and
// block copy for gfx950.  The arithmetic replaces the reference's per-sequence gather +
// online-softmax loops (crates/ferrisinfer-kernel/src/cpu/attention.rs:332-686,
// runtime/paged_kv.rs:769-791).
//
// KV pool layout (per layer): K and V are [num_blocks][Hkv][block_size][D], so one
// (block, kv_head) is a contiguous block_size*D run: a 16-token f32 block of D=128 is 8 KiB
// read with 16-byte loads.
#include <mutex>

#include "fi_common.h"
#include "fi_device.h"

// Split-KV partials of fi_attn_decode_paged_noalloc: a fixed array of this library, one copy
// per device (each GPU holds it from the load of this code object until the process ends).
// In host code `scratch` names a host-side stand-in, never the device memory: host code uses
// only the per-device address that decode_noalloc_attach obtains from hipGetSymbolAddress.
// Calls that overlap on one GPU share this memory and race.
#define FI_DECODE_NOALLOC_SCRATCH_BYTES (96u << 20)
static __device__ __align__(256) unsigned char scratch[FI_DECODE_NOALLOC_SCRATCH_BYTES];

namespace {

// Tunables (compile-time).  The wave chunk fixes the reduction order for a given context
// length and model shape, so it is a constant of the library, not of a launch.
#ifndef FI_DECODE_WIDE_WAVE_TOKENS
#define FI_DECODE_WIDE_WAVE_TOKENS 128  // context tokens per wave when Hkv * D >= 512
#endif
#ifndef FI_DECODE_NARROW_WAVE_TOKENS
#define FI_DECODE_NARROW_WAVE_TOKENS 64  // narrow KV rows (few, small heads): more workgroups
#endif
#ifndef FI_DECODE_INFLIGHT_BYTES
#define FI_DECODE_INFLIGHT_BYTES 16384  // f32 K or V bytes each wave keeps in flight (bf16: half)
#endif

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxParts = 256;  // merge weights live in LDS

// Tokens per wave for a model shape (never a batch property: outputs stay batch-invariant).
constexpr int wave_tokens_for(int hkv, int d) {
  return hkv * d >= 512 ? FI_DECODE_WIDE_WAVE_TOKENS : FI_DECODE_NARROW_WAVE_TOKENS;
}

constexpr int clamp_int(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

// 16-byte K/V vectors: the raw register form stays in flight, widening happens at use.
template <typename KVT>
struct KvIO;

template <>
struct KvIO<float> {
  using Raw = float4;
  static constexpr int kVecElems = 4;
  __device__ static Raw load(const float* p) { return *reinterpret_cast<const float4*>(p); }
  __device__ static void widen(const Raw& v, float* out) {
    out[0] = v.x;
    out[1] = v.y;
    out[2] = v.z;
    out[3] = v.w;
  }
};

template <>
struct KvIO<uint16_t> {
  using Raw = uint4;
  static constexpr int kVecElems = 8;
  __device__ static Raw load(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }
  __device__ static void widen(const Raw& v, float* out) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = fi::bf16_bits_to_f32(w[i] & 0xffffu);
      out[2 * i + 1] = fi::bf16_bits_to_f32(w[i] >> 16);
    }
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
  // Merge in the partition kernel: one arrival counter per (sequence, kv head), zero between
  // launches (the last arriver resets it).  Null: decode_merge_kernel merges.
  unsigned* counters;
  // Fused q|k|v consumer (decode ticks, one new token per sequence), when qkv_parts is set:
  // every workgroup forms its group's query rows from the q|k|v projection's split-K partials
  // (+ bias, RoPE) instead of reading q, and the last partition's workgroup of each
  // (sequence, kv head) first writes the new token's K/V row into the pool at slots[seq].
  const float* qkv_parts;  // [qkv_splits][num_seqs][Hq D + 2 Hkv D]
  int qkv_splits;
  const float* bias_q;
  const float* bias_k;
  const float* bias_v;
  const int* positions;  // [num_seqs] RoPE positions
  const float* cos_t;    // [max_positions][rotary_dims / 2]
  const float* sin_t;
  int rotary_dims;
  int max_positions;
  const int64_t* slots;  // [num_seqs] pool slots of the new tokens
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

// Orders this wave's LDS stores before its later LDS loads by other lanes (a compiler
// barrier only: a wave's LDS operations execute in order).
__device__ __forceinline__ void wave_lds_sync() { __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); }

// Keeps the instruction scheduler from moving code across this point, so loads issued
// before it stay ahead of the arithmetic after it (the ring's depth is what stays in flight).
__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

// A partial of another workgroup: a plain load after a kernel boundary, a device-coherent
// load (past the XCDs' private L2s) inside the partition kernel.
template <bool COHERENT>
__device__ __forceinline__ float load_partial(float* p) {
  if constexpr (COHERENT) return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return *p;
}

// Combines the partitions of one (sequence, kv_head) group: M = max m_p,
// L = sum l_p e^(m_p-M), out = sum acc_p e^(m_p-M) / L per query head.  The first
// partitions' partials are fetched before the weights are known so the loads overlap.  The
// same arithmetic, in the same order, runs in decode_merge_kernel and in the partition
// kernel's last-arriving workgroup, so both give identical outputs.
template <int D, int MAXG, bool COHERENT>
__device__ __forceinline__ void merge_unit(const DecodeArgs& a, size_t head0, int nparts, float (*s_w)[kMaxParts],
                                           float* s_inv) {
  constexpr int kPrefetch = 8;
  constexpr int kPerThread = (MAXG * D + kThreads - 1) / kThreads;
  const int group = a.group;
  const int tid = threadIdx.x;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int P = a.parts_per_seq;

  float pre[kPerThread][kPrefetch];
#pragma unroll
  for (int k = 0; k < kPerThread; ++k) {
    const int i = tid + k * kThreads;
    const int g = i / D, d = i % D;
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p)
      pre[k][p] = (g < group && p < nparts) ? load_partial<COHERENT>(&a.part_acc[((head0 + g) * P + p) * D + d]) : 0.0f;
  }
  for (int g = w; g < group; g += 4) {
    // each lane's (max, sum) pairs are read once and kept for the weights
    constexpr int kPartsPerLane = kMaxParts / 64;
    float* ml = a.part_ml + (head0 + g) * P * 2;
    float2 mlv[kPartsPerLane];
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kPartsPerLane; ++j) {
      const int p = lane + 64 * j;
      if constexpr (COHERENT)
        mlv[j] = p < nparts ? make_float2(load_partial<true>(&ml[2 * p]), load_partial<true>(&ml[2 * p + 1]))
                            : make_float2(-INFINITY, 0.0f);
      else
        mlv[j] = p < nparts ? reinterpret_cast<const float2*>(ml)[p] : make_float2(-INFINITY, 0.0f);
      m = fmaxf(m, mlv[j].x);
    }
    m = fi::wave_max(m);
    float l = 0.0f;
#pragma unroll
    for (int j = 0; j < kPartsPerLane; ++j) {
      const int p = lane + 64 * j;
      if (p < nparts) {
        const float wgt = __expf(mlv[j].x - m);
        s_w[g][p] = wgt;
        l += mlv[j].y * wgt;
      }
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
    for (int p = kPrefetch; p < nparts; ++p)
      acc += load_partial<COHERENT>(&a.part_acc[((head0 + g) * P + p) * D + d]) * s_w[g][p];
    a.out[(head0 + g) * D + d] = acc * s_inv[g];
  }
}

// The fused q|k|v consumer's share of one workgroup: the group's query rows into s_q and,
// with `append`, the new token's K and V rows of kv head kvh into the pool.  The arithmetic
// is qkv_rope_append4_kernel's (fi::qkv_value4, fi::rope4, fi::put_kv4), so the rows equal
// that kernel's bit for bit.
template <int D, typename KVT, int G>
__device__ __forceinline__ void qkv_prologue(const DecodeArgs& a, int seq, int kvh, bool append, float (*s_q)[D],
                                             int tid, int ctx_raw) {
  const int half = a.rotary_dims / 2;
  const int pass = D - 2 * half;
  const int qph = (half + pass) / 4;  // four-column items per head row
  const int group = a.group;
  const int qw = a.hq * D, kw = a.hkv * D;
  const int width = qw + 2 * kw;
  const size_t plane = (size_t)a.num_seqs * width;
  const float* p0 = a.qkv_parts + (size_t)seq * width;
  const int64_t pool_slots = (int64_t)a.num_blocks * a.block_size;
  const int64_t slot = a.slots[seq];
  const bool write_kv = append && slot >= 0 && slot < pool_slots;
  if (append && tid == 0 && slot >= pool_slots) atomicOr(a.faults, FI_FAULT_SLOT_RANGE);
  const int64_t blk = write_kv ? slot / a.block_size : 0;
  const int off = write_kv ? static_cast<int>(slot % a.block_size) : 0;
  const size_t row = (((size_t)blk * a.hkv + kvh) * a.block_size + off) * D;
  KVT* k_pool = static_cast<KVT*>(const_cast<void*>(a.k_cache));
  KVT* v_pool = static_cast<KVT*>(const_cast<void*>(a.v_cache));
  const int rot_items = (group + (write_kv ? 1 : 0)) * qph;
  const int items = rot_items + (write_kv ? D / 4 : 0);
  for (int idx = tid; idx < items; idx += kThreads) {
    if (idx < rot_items) {
      const int g = idx / qph, r = 4 * (idx - g * qph);
      const bool is_q = g < group;
      const int col0 = is_q ? (kvh * group + g) * D : qw + kvh * D;
      const int bcol0 = is_q ? (kvh * group + g) * D : kvh * D;
      const float* bias = is_q ? a.bias_q : a.bias_k;
      if (r < half) {
        // a decode token's position is its sequence's last key, context_lens - 1: the table
        // rows at that position are loaded with the partials (no dependent round trip on the
        // position), and again at the given position where it differs
        const int guess = min(max(ctx_raw - 1, 0), a.max_positions - 1);
        float4 c = *reinterpret_cast<const float4*>(a.cos_t + (size_t)guess * half + r);
        float4 sn = *reinterpret_cast<const float4*>(a.sin_t + (size_t)guess * half + r);
        int pos = a.positions[seq];
        if (pos < 0 || pos >= a.max_positions) {
          atomicOr(a.faults, FI_FAULT_POSITION_RANGE);
          pos = 0;
        }
        const float4 lo = fi::qkv_value4(p0, plane, a.qkv_splits, bias, bcol0 + r, col0 + r);
        const float4 hi = fi::qkv_value4(p0, plane, a.qkv_splits, bias, bcol0 + r + half, col0 + r + half);
        if (pos != guess) {
          c = *reinterpret_cast<const float4*>(a.cos_t + (size_t)pos * half + r);
          sn = *reinterpret_cast<const float4*>(a.sin_t + (size_t)pos * half + r);
        }
        float4 y0, y1;
        fi::rope4(lo, hi, c, sn, y0, y1);
        if (is_q) {
          *reinterpret_cast<float4*>(&s_q[g][r]) = y0;
          *reinterpret_cast<float4*>(&s_q[g][r + half]) = y1;
        } else {
          fi::put_kv4(k_pool, row + r, y0);
          fi::put_kv4(k_pool, row + r + half, y1);
        }
      } else {
        const int i = 2 * half + (r - half);
        const float4 y = fi::qkv_value4(p0, plane, a.qkv_splits, bias, bcol0 + i, col0 + i);
        if (is_q) {
          *reinterpret_cast<float4*>(&s_q[g][i]) = y;
        } else {
          fi::put_kv4(k_pool, row + i, y);
        }
      }
    } else {
      const int i = 4 * (idx - rot_items);
      const float4 x = fi::qkv_value4(p0, plane, a.qkv_splits, a.bias_v, kvh * D + i, qw + kw + kvh * D + i);
      fi::put_kv4(v_pool, row + i, x);
    }
  }
}

// One workgroup = one (sequence, kv_head, partition of 4*WT tokens); partitions are
// numbered fastest across (sequence, kv_head) so the first-dispatched workgroups hold the
// full leading partitions and the ragged tails come last.  The GQA group of query heads
// sharing the kv head is processed together so every K/V byte is read once.
//   setup: the partition's token -> pool row indices go to LDS (block-table lookups) while
//     each lane loads its slice of the group's query rows into registers;
//   each wave then owns WT consecutive tokens and runs on its own (no workgroup
//   barrier until the combine):
//     K: KL lanes share a token row with 16-byte loads, a compile-time ring keeps
//        ~FI_DECODE_INFLIGHT_BYTES of K in flight, dot products are reduced across the
//        row's lanes with DPP; each lane keeps the scores of its own query head;
//     softmax over the wave's tokens in registers (the first V loads are already issued);
//        probabilities go to the wave's LDS slice;
//     V: VL lanes cover a row, again through a ring of in-flight loads; accumulators are
//        folded across the wave's rows with lane shuffles;
//   combine: the waves' (max, sum, acc) are merged through LDS in wave order.
// Rows past the end are clamped to the last valid row (same addresses, no extra traffic)
// and carry probability 0.  A sequence with one partition writes its normalised output;
// otherwise each workgroup stores (max, sum, unnormalised acc), and the last workgroup of the
// (sequence, kv_head) group to finish merges them (counters given), or decode_merge_kernel
// does in a launch of its own.
template <int D, typename KVT, int G, int WT>
__global__ __launch_bounds__(kThreads) void decode_partition_kernel(DecodeArgs a) {
  constexpr int kWaveTokens = WT;
  constexpr int kPartTokens = kWaves * WT;
  using IO = KvIO<KVT>;
  using Raw = typename IO::Raw;
  constexpr int EPV = IO::kVecElems;          // elements per 16-byte vector
  constexpr int VECS = D / EPV;               // vectors per row
  static_assert(VECS >= 1 && VECS <= 64 && (VECS & (VECS - 1)) == 0, "row of 16-byte vectors");
  constexpr int KL = VECS < 8 ? VECS : 8;     // lanes per K row
  constexpr int KV = VECS / KL;               // vectors per lane per K row
  constexpr int KE = KV * EPV;                // elements per lane per K row
  constexpr int KR = 64 / KL;                 // K rows per wave step
  constexpr int KSTEPS = kWaveTokens / KR;
  constexpr int HPL = (G + KL - 1) / KL;      // query heads whose scores a lane keeps
  constexpr int VL = VECS;                    // lanes per V row (one vector each)
  constexpr int VR = 64 / VL;                 // V rows per wave step
  constexpr int VSTEPS = kWaveTokens / VR;
  constexpr int ROWB = D * static_cast<int>(sizeof(KVT));
  // bf16 rows carry twice the arithmetic per byte: half the bytes in flight keeps the
  // register ring (and occupancy) the same as for f32.
  constexpr int INFLIGHT = FI_DECODE_INFLIGHT_BYTES * static_cast<int>(sizeof(KVT)) / 4;
  constexpr int KDEPTH = clamp_int(INFLIGHT / (KR * ROWB), 1, KSTEPS);
  constexpr int VDEPTH = clamp_int(INFLIGHT / (VR * ROWB), 1, VSTEPS);
  static_assert(kWaveTokens % KR == 0 && kWaveTokens % VR == 0, "wave chunk must tile the rows");

  __shared__ uint32_t s_row[kPartTokens];
  __shared__ float s_q[G][D];  // fused q|k|v: the group's query rows
  __shared__ float s_p[kWaves][kWaveTokens][G];
  __shared__ float s_ml[kWaves][G][2];
  __shared__ float s_acc[kWaves][G][D];

  const KVT* __restrict__ k_cache = static_cast<const KVT*>(a.k_cache);
  const KVT* __restrict__ v_cache = static_cast<const KVT*>(a.v_cache);
  const int group = a.group;
  const int units = a.num_seqs * a.hkv;
  const int part = blockIdx.x / units;
  const int unit = blockIdx.x - part * units;
  const int seq = unit / a.hkv;
  const int kvh = unit - seq * a.hkv;
  const int tid = threadIdx.x;
  int ctx = a.context_lens[seq];
  const int ctx_raw = ctx;
  if (ctx > a.parts_per_seq * kPartTokens) {  // beyond the grid: clamp and report
    if (part == 0 && tid == 0) atomicOr(a.faults, FI_FAULT_CONTEXT_RANGE);
    ctx = a.parts_per_seq * kPartTokens;
  }
  const size_t head0 = (size_t)seq * a.hq + (size_t)kvh * group;  // first query head of the group
  const bool fused = a.qkv_parts != nullptr;  // uniform
  if (ctx <= 0) {  // no keys: defined output of zeros (the new token's K/V still appended)
    if (part == 0) {
      for (int i = tid; i < group * D; i += kThreads) a.out[head0 * D + i] = 0.0f;
      if (fused) qkv_prologue<D, KVT, G>(a, seq, kvh, true, s_q, tid, ctx_raw);
    }
    return;
  }
  const int t0 = part * kPartTokens;
  if (t0 >= ctx) return;  // whole workgroup exits together
  const int n_part = min(kPartTokens, ctx - t0);
  const int nparts = (ctx + kPartTokens - 1) / kPartTokens;
  const int w = tid >> 6;
  const int lane = tid & 63;
  const int wt0 = w * kWaveTokens;              // the wave's first token within the partition
  const int n = min(kWaveTokens, n_part - wt0);  // the wave's tokens (<= 0: idle wave)

  // K-pass lane roles: row r of each step, vector column c
  const int r = lane / KL;
  const int c = lane % KL;
  // this lane's slice of the group's query rows: from q (issued before the block lookups, so
  // the loads overlap them), or from the fused consumer's rows in LDS after the barrier below
  float qreg[G][KE];
  auto load_q = [&](const float* src, size_t stride) {
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int j = 0; j < KV; ++j) {
        float4 lo = make_float4(0.f, 0.f, 0.f, 0.f), hi = lo;
        if (g < group) {
          const float* qp = src + g * stride + (j * KL + c) * EPV;
          lo = *reinterpret_cast<const float4*>(qp);
          if constexpr (EPV == 8) hi = *reinterpret_cast<const float4*>(qp + 4);
        }
        float* dst = &qreg[g][j * EPV];
        dst[0] = lo.x;
        dst[1] = lo.y;
        dst[2] = lo.z;
        dst[3] = lo.w;
        if constexpr (EPV == 8) {
          dst[4] = hi.x;
          dst[5] = hi.y;
          dst[6] = hi.z;
          dst[7] = hi.w;
        }
      }
  };
  // the partition's block-table entries are loaded first, so that their round trip overlaps
  // the query rows' (or the fused consumer's partials')
  constexpr int kRowsPerThread = (kPartTokens + kThreads - 1) / kThreads;
  const int bs = a.block_size;
  int ids[kRowsPerThread];
#pragma unroll
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int pos = t0 + min(tid + i * kThreads, n_part - 1);  // clamped: a valid entry
    const int lb = pos / bs;
    ids[i] = lb < a.max_blocks ? a.block_tables[(size_t)seq * a.max_blocks + lb] : -1;
  }
  if (fused) {
    // the last partition holds the new token: its K/V row is written before the keys are read
    qkv_prologue<D, KVT, G>(a, seq, kvh, part == nparts - 1, s_q, tid, ctx_raw);
  } else {
    load_q(a.q + head0 * D, D);
  }
#pragma unroll
  for (int i = 0; i < kRowsPerThread; ++i) {
    const int t = tid + i * kThreads;
    if (t < n_part) {
      const int pos = t0 + t;
      const int lb = pos / bs;
      int id = ids[i];
      if (id < 0 || id >= a.num_blocks) {
        atomicOr(a.faults, FI_FAULT_BLOCK_RANGE);
        id = 0;
      }
      s_row[t] = (static_cast<uint32_t>(id) * a.hkv + kvh) * bs + (pos - lb * bs);
    }
  }
  // orders the fused consumer's query rows (LDS) and the new token's K/V row (global memory,
  // written by this workgroup) before their reads
  __syncthreads();
  if (fused) load_q(&s_q[0][0], D);

  if (n > 0) {  // wave-uniform
    const uint32_t* rows = s_row + wt0;
    // ---- K: scores of this lane's rows for its query heads (h * KL + c) ----
    float sc[KSTEPS][HPL];
    {
      Raw kb[KDEPTH][KV];
      auto issue_k = [&](int s, Raw (&buf)[KV]) {
        const KVT* p = k_cache + (size_t)rows[min(s * KR + r, n - 1)] * D + c * EPV;
#pragma unroll
        for (int j = 0; j < KV; ++j) buf[j] = IO::load(p + j * KL * EPV);
      };
#pragma unroll
      for (int s = 0; s < KDEPTH; ++s) issue_k(s, kb[s]);
      sched_fence();
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        float kf[KE];
#pragma unroll
        for (int j = 0; j < KV; ++j) IO::widen(kb[s % KDEPTH][j], kf + j * EPV);
        if (s + KDEPTH < KSTEPS) issue_k(s + KDEPTH, kb[s % KDEPTH]);
        sched_fence();
        float dot[G];
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float acc = 0.0f;
#pragma unroll
          for (int e = 0; e < KE; ++e) acc += qreg[g][e] * kf[e];
          dot[g] = fi::group_sum<KL>(acc);
        }
        const bool valid = s * KR + r < n;
#pragma unroll
        for (int h = 0; h < HPL; ++h) {
          float v = dot[h * KL];
#pragma unroll
          for (int cc = 1; cc < KL; ++cc)
            if (h * KL + cc < G) v = c == cc ? dot[h * KL + cc] : v;
          sc[s][h] = valid ? v * a.scale : -INFINITY;
        }
      }
    }

    // ---- first V loads go out before the softmax ----
    const int vr = lane / VL;
    const int vc = lane % VL;
    Raw vb[VDEPTH];
    auto issue_v = [&](int s) {
      vb[s % VDEPTH] = IO::load(v_cache + (size_t)rows[min(s * VR + vr, n - 1)] * D + vc * EPV);
    };
#pragma unroll
    for (int s = 0; s < VDEPTH; ++s) issue_v(s);
    sched_fence();

    // ---- softmax over the wave's tokens (lanes sharing c hold one head's scores) ----
#pragma unroll
    for (int h = 0; h < HPL; ++h) {
      float m = -INFINITY;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) m = fmaxf(m, sc[s][h]);
#pragma unroll
      for (int x = KL; x < 64; x <<= 1) m = fmaxf(m, __shfl_xor(m, x, 64));
      float l = 0.0f;
#pragma unroll
      for (int s = 0; s < KSTEPS; ++s) {
        const float p = sc[s][h] == -INFINITY ? 0.0f : __expf(sc[s][h] - m);
        sc[s][h] = p;
        l += p;
      }
#pragma unroll
      for (int x = KL; x < 64; x <<= 1) l += __shfl_xor(l, x, 64);
      const int g = h * KL + c;
      if (g < G) {
#pragma unroll
        for (int s = 0; s < KSTEPS; ++s) s_p[w][s * KR + r][g] = sc[s][h];
        if (r == 0) {
          s_ml[w][g][0] = m;
          s_ml[w][g][1] = l;
        }
      }
    }
    wave_lds_sync();

    // ---- V: acc[g][e] = sum_t p[t][g] * V[t][vc * EPV + e] ----
    float acc[G][EPV];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
      for (int e = 0; e < EPV; ++e) acc[g][e] = 0.0f;
#pragma unroll
    for (int s = 0; s < VSTEPS; ++s) {
      float vf[EPV];
      IO::widen(vb[s % VDEPTH], vf);
      if (s + VDEPTH < VSTEPS) issue_v(s + VDEPTH);
      sched_fence();
      const float* pp = s_p[w][s * VR + vr];
      float p[G];
#pragma unroll
      for (int g = 0; g < G; ++g) p[g] = pp[g];
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] += p[g] * vf[e];
    }
#pragma unroll
    for (int x = VL; x < 64; x <<= 1)
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) acc[g][e] += __shfl_xor(acc[g][e], x, 64);
    if (vr == 0) {
#pragma unroll
      for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < EPV; ++e) s_acc[w][g][vc * EPV + e] = acc[g][e];
    }
  }
  __syncthreads();

  // ---- combine the waves (in wave order) ----
  const int nw = (n_part + kWaveTokens - 1) / kWaveTokens;
  for (int i = tid; i < group * D; i += kThreads) {
    const int g = i / D, d = i - (i / D) * D;
    float mx = s_ml[0][g][0];
    for (int v = 1; v < nw; ++v) mx = fmaxf(mx, s_ml[v][g][0]);
    float l = 0.0f, sum = 0.0f;
    for (int v = 0; v < nw; ++v) {
      const float wgt = __expf(s_ml[v][g][0] - mx);
      l += s_ml[v][g][1] * wgt;
      sum += s_acc[v][g][d] * wgt;
    }
    if (nparts == 1) {
      a.out[(head0 + g) * D + d] = sum * (1.0f / l);
    } else if (a.counters) {  // read by another workgroup of this launch: device-coherent stores
      const size_t slot = (head0 + g) * a.parts_per_seq + part;
      __hip_atomic_store(&a.part_acc[slot * D + d], sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (d == 0) {
        __hip_atomic_store(&a.part_ml[slot * 2], mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&a.part_ml[slot * 2 + 1], l, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    } else {
      const size_t slot = (head0 + g) * a.parts_per_seq + part;
      a.part_acc[slot * D + d] = sum;
      if (d == 0) {
        a.part_ml[slot * 2] = mx;
        a.part_ml[slot * 2 + 1] = l;
      }
    }
  }
  if (nparts <= 1 || a.counters == nullptr) return;  // workgroup-uniform

  // ---- the last of the group's partitions to finish merges them ----
  // Each thread waits until its coherent stores have completed, so when the counter shows
  // every partition arrived, every partial is readable at the coherence point.  No cache-wide
  // fence is used (a device-scope fence writes back the whole L2 of the XCD).  The last
  // arriver resets the counter for the next launch or graph replay.
  __shared__ float s_w[G][kMaxParts];
  __shared__ float s_inv[G];
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const unsigned arrived =
        __hip_atomic_fetch_add(&a.counters[unit], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    s_last = arrived == static_cast<unsigned>(nparts);
    if (s_last) __hip_atomic_store(&a.counters[unit], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!s_last) return;
  merge_unit<D, G, true>(a, head0, nparts, s_w, s_inv);
}

// The separate merge launch (used where the partition kernel does not merge): one workgroup
// per (sequence, kv_head) group; sequences with a single partition were finished by the
// partition kernel, and the launch boundary orders the partials' stores before these loads.
template <int D, int MAXG, int WT>
__global__ __launch_bounds__(kThreads) void decode_merge_kernel(DecodeArgs a) {
  constexpr int kPartTokens = kWaves * WT;
  __shared__ float s_w[MAXG][kMaxParts];
  __shared__ float s_inv[MAXG];
  const int pair = blockIdx.x;
  const int seq = pair / a.hkv;
  const int kvh = pair % a.hkv;
  const int ctx = min(a.context_lens[seq], a.parts_per_seq * kPartTokens);  // clamped as in the partitions
  const int nparts = (ctx + kPartTokens - 1) / kPartTokens;
  if (nparts <= 1) return;
  const size_t head0 = (size_t)seq * a.hq + (size_t)kvh * a.group;
  merge_unit<D, MAXG, false>(a, head0, nparts, s_w, s_inv);
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

// Four consecutive elements of one head row per thread over the flat (token, element) range, with
// 16-byte loads and 16-byte (f32) or 8-byte (bf16) stores: the rows' bytes move in full-width
// accesses (head dims that are multiples of 4 and 16-byte aligned sources).  Same values as
// kv_append_kernel.
template <typename KVT>
__global__ __launch_bounds__(256) void kv_append4_kernel(const float* __restrict__ key,
                                                         const float* __restrict__ value,
                                                         const int64_t* __restrict__ slots,
                                                         KVT* __restrict__ k_cache,
                                                         KVT* __restrict__ v_cache, int64_t pool_slots,
                                                         int block_size, int hkv, int d, int64_t total4,
                                                         uint32_t* __restrict__ faults) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total4) return;
  const int row4 = hkv * d / 4;
  const int64_t t = idx / row4;
  const int i = static_cast<int>(idx - t * row4) * 4;
  const int64_t slot = slots[t];
  if (slot < 0) return;
  if (slot >= pool_slots) {
    if (i == 0) atomicOr(faults, FI_FAULT_SLOT_RANGE);
    return;
  }
  const int64_t blk = slot / block_size;
  const int off = static_cast<int>(slot - blk * block_size);
  const int h = i / d, e = i - (i / d) * d;
  const size_t dst = (((size_t)blk * hkv + h) * block_size + off) * d + e;
  const float4 kf = *reinterpret_cast<const float4*>(key + t * 4 * row4 + i);
  const float4 vf = *reinterpret_cast<const float4*>(value + t * 4 * row4 + i);
  if constexpr (sizeof(KVT) == 4) {
    *reinterpret_cast<float4*>(k_cache + dst) = kf;
    *reinterpret_cast<float4*>(v_cache + dst) = vf;
  } else {
    auto pack = [](float4 x) {
      return make_uint2(fi::f32_to_bf16_bits(x.x) | (fi::f32_to_bf16_bits(x.y) << 16),
                        fi::f32_to_bf16_bits(x.z) | (fi::f32_to_bf16_bits(x.w) << 16));
    };
    *reinterpret_cast<uint2*>(k_cache + dst) = pack(kf);
    *reinterpret_cast<uint2*>(v_cache + dst) = pack(vf);
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

// One thread per 4 consecutive elements of an output row [t][h][d .. d + 3]: the pool's
// (block, head) runs [bs][D] are read row by row into token-major [length][Hkv][D].
template <typename KVT>
__global__ __launch_bounds__(256) void kv_gather_kernel(const KVT* __restrict__ k_cache,
                                                        const KVT* __restrict__ v_cache,
                                                        const int* __restrict__ table, int64_t quads,
                                                        int num_blocks, int block_size, int hkv, int d,
                                                        float* __restrict__ k_out, float* __restrict__ v_out,
                                                        uint32_t* __restrict__ faults) {
  const int dq = d / 4;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < quads; i += stride) {
    const int dd = static_cast<int>(i % dq) * 4;
    const int64_t row = i / dq;
    const int h = static_cast<int>(row % hkv);
    const int t = static_cast<int>(row / hkv);
    const int b = table[t / block_size];
    float4 kq = make_float4(0.f, 0.f, 0.f, 0.f), vq = kq;
    if (b < 0 || b >= num_blocks) {
      atomicOr(faults, FI_FAULT_BLOCK_RANGE);
    } else {
      const size_t src = (((size_t)b * hkv + h) * block_size + t % block_size) * d + dd;
      if constexpr (sizeof(KVT) == 4) {
        kq = *reinterpret_cast<const float4*>(k_cache + src);
        vq = *reinterpret_cast<const float4*>(v_cache + src);
      } else {
        const uint2 kb = *reinterpret_cast<const uint2*>(k_cache + src);
        const uint2 vb = *reinterpret_cast<const uint2*>(v_cache + src);
        kq = make_float4(fi::bf16_bits_to_f32(kb.x & 0xffffu), fi::bf16_bits_to_f32(kb.x >> 16),
                         fi::bf16_bits_to_f32(kb.y & 0xffffu), fi::bf16_bits_to_f32(kb.y >> 16));
        vq = make_float4(fi::bf16_bits_to_f32(vb.x & 0xffffu), fi::bf16_bits_to_f32(vb.x >> 16),
                         fi::bf16_bits_to_f32(vb.y & 0xffffu), fi::bf16_bits_to_f32(vb.y >> 16));
      }
    }
    *reinterpret_cast<float4*>(k_out + i * 4) = kq;
    *reinterpret_cast<float4*>(v_out + i * 4) = vq;
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

template <int D, typename KVT, int G>
int32_t launch_decode_group(fi_context* ctx, const DecodeArgs& args, unsigned grid, int wt) {
  if (wt == FI_DECODE_WIDE_WAVE_TOKENS) {
    hipLaunchKernelGGL((decode_partition_kernel<D, KVT, G, FI_DECODE_WIDE_WAVE_TOKENS>), dim3(grid), dim3(kThreads), 0,
                       ctx->stream, args);
  } else {
    hipLaunchKernelGGL((decode_partition_kernel<D, KVT, G, FI_DECODE_NARROW_WAVE_TOKENS>), dim3(grid), dim3(kThreads),
                       0, ctx->stream, args);
  }
  FI_CHECK_LAUNCH("decode_partition_kernel");
  if (args.parts_per_seq > 1 && args.counters == nullptr) {
    const dim3 grid2(static_cast<unsigned>(args.num_seqs) * args.hkv);
    if (wt == FI_DECODE_WIDE_WAVE_TOKENS) {
      hipLaunchKernelGGL((decode_merge_kernel<D, G, FI_DECODE_WIDE_WAVE_TOKENS>), grid2, dim3(kThreads), 0, ctx->stream,
                         args);
    } else {
      hipLaunchKernelGGL((decode_merge_kernel<D, G, FI_DECODE_NARROW_WAVE_TOKENS>), grid2, dim3(kThreads), 0,
                         ctx->stream, args);
    }
    FI_CHECK_LAUNCH("decode_merge_kernel");
  }
  return FI_OK;
}

template <int D, typename KVT>
int32_t launch_decode(fi_context* ctx, const DecodeArgs& args, unsigned grid, int wt) {
  if (args.group <= 1) return launch_decode_group<D, KVT, 1>(ctx, args, grid, wt);
  if (args.group <= 2) return launch_decode_group<D, KVT, 2>(ctx, args, grid, wt);
  if (args.group <= 4) return launch_decode_group<D, KVT, 4>(ctx, args, grid, wt);
  if (args.group <= 8) return launch_decode_group<D, KVT, 8>(ctx, args, grid, wt);
  return fi::set_error(FI_ERR_UNSUPPORTED, "decode attention supports at most 8 query heads per KV head");
}

template <int D>
int32_t launch_decode_dtype(fi_context* ctx, int32_t dtype, const DecodeArgs& args, unsigned grid, int wt) {
  if (dtype == FI_DTYPE_F32) return launch_decode<D, float>(ctx, args, grid, wt);
  return launch_decode<D, uint16_t>(ctx, args, grid, wt);
}

}  // namespace

namespace fi {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_noalloc_mu;
void* g_noalloc_ptr[kMaxDevices] = {};
}  // namespace

int32_t decode_noalloc_attach(fi_context* ctx) {
  FI_REQUIRE(ctx->device >= 0 && ctx->device < kMaxDevices, FI_ERR_UNSUPPORTED,
             "device ordinal " + std::to_string(ctx->device) + " beyond the library's device table");
  std::lock_guard<std::mutex> lock(g_noalloc_mu);
  if (g_noalloc_ptr[ctx->device] == nullptr) {
    void* p = nullptr;
    FI_TRY_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    FI_REQUIRE(p != nullptr, FI_ERR_RUNTIME, "hipGetSymbolAddress(scratch) returned a null address");
    g_noalloc_ptr[ctx->device] = p;
  }
  ctx->noalloc_scratch = g_noalloc_ptr[ctx->device];
  return FI_OK;
}

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
  const bool vec = head_dim % 4 == 0 && reinterpret_cast<uintptr_t>(d_key) % 16 == 0 &&
                   reinterpret_cast<uintptr_t>(d_value) % 16 == 0;
  if (vec) {
    const int64_t total4 = static_cast<int64_t>(num_tokens) * num_kv_heads * head_dim / 4;
    const dim3 grid(static_cast<unsigned>((total4 + 255) / 256));
    if (kv_dtype == FI_DTYPE_F32)
      hipLaunchKernelGGL(kv_append4_kernel<float>, grid, dim3(256), 0, ctx->stream, d_key, d_value, d_slot_mapping,
                         static_cast<float*>(d_k_cache), static_cast<float*>(d_v_cache), pool_slots, block_size,
                         num_kv_heads, head_dim, total4, ctx->d_faults);
    else
      hipLaunchKernelGGL(kv_append4_kernel<uint16_t>, grid, dim3(256), 0, ctx->stream, d_key, d_value,
                         d_slot_mapping, static_cast<uint16_t*>(d_k_cache), static_cast<uint16_t*>(d_v_cache),
                         pool_slots, block_size, num_kv_heads, head_dim, total4, ctx->d_faults);
    FI_CHECK_LAUNCH("kv_append4_kernel");
    return FI_OK;
  }
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

int32_t fi_kv_gather(fi_context* ctx, const void* d_k_cache, const void* d_v_cache, int32_t kv_dtype,
                     const int32_t* d_block_table, int32_t num_table_blocks, int32_t length,
                     int32_t num_blocks, int32_t block_size, int32_t num_kv_heads, int32_t head_dim,
                     float* d_k_out, float* d_v_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(length >= 0 && num_table_blocks >= 0, FI_ERR_INVALID_SHAPE, "fi_kv_gather: negative sizes");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_kv_gather: KV dtype must be f32 or bf16");
  FI_REQUIRE(num_blocks > 0 && block_size > 0 && num_kv_heads > 0 && head_dim > 0, FI_ERR_INVALID_CONFIG,
             "fi_kv_gather: pool dimensions must be greater than zero");
  FI_REQUIRE(head_dim % 4 == 0, FI_ERR_UNSUPPORTED, "fi_kv_gather: head_dim must be a multiple of 4");
  // paged_kv.rs:303-308: a prefix longer than the sequence's pages
  FI_REQUIRE(static_cast<int64_t>(length) <= static_cast<int64_t>(num_table_blocks) * block_size, FI_ERR_RUNTIME,
             "fi_kv_gather: KV cache block table ran out of committed pages");
  if (length == 0) return FI_OK;
  FI_REQUIRE(d_k_cache && d_v_cache && d_block_table && d_k_out && d_v_out, FI_ERR_INVALID_CONFIG,
             "fi_kv_gather: null pointer");
  FI_REQUIRE(((reinterpret_cast<uintptr_t>(d_k_cache) | reinterpret_cast<uintptr_t>(d_v_cache) |
               reinterpret_cast<uintptr_t>(d_k_out) | reinterpret_cast<uintptr_t>(d_v_out)) & 15) == 0,
             FI_ERR_INVALID_LAYOUT, "fi_kv_gather: pools and outputs must be 16-byte aligned (vector accesses)");
  const int64_t quads = static_cast<int64_t>(length) * num_kv_heads * (head_dim / 4);
  const unsigned grid = static_cast<unsigned>(std::min<int64_t>((quads + 255) / 256, 4096));
  if (kv_dtype == FI_DTYPE_F32) {
    hipLaunchKernelGGL(kv_gather_kernel<float>, dim3(grid), dim3(256), 0, ctx->stream,
                       static_cast<const float*>(d_k_cache), static_cast<const float*>(d_v_cache), d_block_table,
                       quads, num_blocks, block_size, num_kv_heads, head_dim, d_k_out, d_v_out, ctx->d_faults);
  } else {
    hipLaunchKernelGGL(kv_gather_kernel<uint16_t>, dim3(grid), dim3(256), 0, ctx->stream,
                       static_cast<const uint16_t*>(d_k_cache), static_cast<const uint16_t*>(d_v_cache),
                       d_block_table, quads, num_blocks, block_size, num_kv_heads, head_dim, d_k_out, d_v_out,
                       ctx->d_faults);
  }
  FI_CHECK_LAUNCH("kv_gather_kernel");
  return FI_OK;
}

}  // extern "C"

namespace {

// Shared by both decode entry points: validation, launch shape and launches.  With
// `noalloc` the partials go to the library's fixed scratch array instead of the context
// workspace (nothing is allocated).
// The fused q|k|v consumer's inputs (fi_attn_decode_paged_qkv).
struct QkvIn {
  const float* parts;
  int32_t splits;
  const float* bias_q;
  const float* bias_k;
  const float* bias_v;
  const int32_t* positions;
  const float* cos_t;
  const float* sin_t;
  int32_t rotary_dims;
  int32_t max_positions;
  const int64_t* slots;
};

int32_t decode_paged(fi_context* ctx, const float* d_q, const void* d_k_cache, const void* d_v_cache,
                     int32_t kv_dtype, const int32_t* d_block_tables, int32_t max_blocks_per_seq,
                     const int32_t* d_context_lens, int32_t num_seqs, int32_t max_context_len,
                     int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                     int32_t num_blocks, float scale, float* d_out, bool noalloc, const QkvIn* qkv = nullptr) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_seqs >= 0 && max_context_len >= 0, FI_ERR_INVALID_SHAPE,
             "fi_attn_decode_paged: negative sizes");
  FI_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && num_q_heads % num_kv_heads == 0,
             FI_ERR_INVALID_SHAPE, "number of query heads must be divisible by number of KV heads");
  FI_REQUIRE(block_size > 0 && num_blocks > 0 && max_blocks_per_seq > 0, FI_ERR_INVALID_CONFIG,
             "fi_attn_decode_paged: pool dimensions must be greater than zero");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_attn_decode_paged: KV dtype must be f32 or bf16");
  FI_REQUIRE(static_cast<int64_t>(max_context_len) <= static_cast<int64_t>(max_blocks_per_seq) * block_size,
             FI_ERR_INVALID_SHAPE, "fi_attn_decode_paged: max_context_len exceeds the block-table width");
  FI_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, FI_ERR_UNSUPPORTED,
             "fi_attn_decode_paged: head_dim must be 32, 64 or 128");
  const int wt = wave_tokens_for(num_kv_heads, head_dim);
  const int part_tokens = kWaves * wt;
  FI_REQUIRE(max_context_len <= part_tokens * kMaxParts, FI_ERR_UNSUPPORTED,
             "fi_attn_decode_paged: context longer than " + std::to_string(part_tokens * kMaxParts) + " tokens");
  if (qkv) {
    FI_REQUIRE(qkv->splits >= 1, FI_ERR_INVALID_SHAPE, "fi_attn_decode_paged_qkv: splits must be at least 1");
    FI_REQUIRE(qkv->rotary_dims >= 0 && qkv->rotary_dims <= head_dim && qkv->rotary_dims % 2 == 0,
               FI_ERR_INVALID_CONFIG, "rope.rotary_dims must be even and at most the head dimension");
    const int32_t half = qkv->rotary_dims / 2, pass = head_dim - 2 * half;
    FI_REQUIRE(half % 4 == 0 && pass % 4 == 0, FI_ERR_UNSUPPORTED,
               "fi_attn_decode_paged_qkv: rotary_dims / 2 and the pass-through width must be multiples of 4");
  }
  if (num_seqs == 0) return FI_OK;
  FI_REQUIRE((d_q || qkv) && d_k_cache && d_v_cache && d_block_tables && d_context_lens && d_out,
             FI_ERR_INVALID_CONFIG, "fi_attn_decode_paged: null pointer");
  if (qkv) {
    auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
    FI_REQUIRE(qkv->parts && qkv->positions && qkv->slots, FI_ERR_INVALID_CONFIG,
               "fi_attn_decode_paged_qkv: null pointer");
    FI_REQUIRE(qkv->rotary_dims == 0 || (qkv->cos_t && qkv->sin_t && qkv->max_positions > 0), FI_ERR_INVALID_CONFIG,
               "fi_attn_decode_paged_qkv: rope tables required");
    FI_REQUIRE(aligned16(qkv->parts) && (!qkv->bias_q || aligned16(qkv->bias_q)) &&
                   (!qkv->bias_k || aligned16(qkv->bias_k)) && (!qkv->bias_v || aligned16(qkv->bias_v)) &&
                   (qkv->rotary_dims == 0 || (aligned16(qkv->cos_t) && aligned16(qkv->sin_t))),
               FI_ERR_INVALID_CONFIG, "fi_attn_decode_paged_qkv: partials, biases and rope tables must be 16-byte aligned");
  }
  const int32_t parts = max_context_len == 0 ? 1 : (max_context_len + part_tokens - 1) / part_tokens;
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
  if (qkv) {
    args.q = nullptr;
    args.qkv_parts = qkv->parts;
    args.qkv_splits = qkv->splits;
    args.bias_q = qkv->bias_q;
    args.bias_k = qkv->bias_k;
    args.bias_v = qkv->bias_v;
    args.positions = qkv->positions;
    args.cos_t = qkv->cos_t;
    args.sin_t = qkv->sin_t;
    args.rotary_dims = qkv->rotary_dims;
    args.max_positions = qkv->max_positions;
    args.slots = qkv->slots;
  }
  if (parts > 1) {
    if (noalloc) {
      const size_t slots = static_cast<size_t>(num_seqs) * num_q_heads * parts;
      const size_t acc_bytes = (slots * head_dim * sizeof(float) + 255) & ~static_cast<size_t>(255);
      const size_t need = acc_bytes + slots * 2 * sizeof(float);
      FI_REQUIRE(need <= FI_DECODE_NOALLOC_SCRATCH_BYTES, FI_ERR_RUNTIME,
                 "fi_attn_decode_paged_noalloc: this launch needs " + std::to_string(need) +
                     " bytes of split-KV scratch; the fixed scratch holds " +
                     std::to_string(FI_DECODE_NOALLOC_SCRATCH_BYTES) + " bytes");
      FI_REQUIRE(ctx->noalloc_scratch != nullptr, FI_ERR_RUNTIME,
                 "fi_attn_decode_paged_noalloc: the context has no scratch address");
      args.part_acc = static_cast<float*>(ctx->noalloc_scratch);
      args.part_ml = reinterpret_cast<float*>(static_cast<char*>(ctx->noalloc_scratch) + acc_bytes);
    } else {
      FI_TRY(fi::decode_scratch(ctx, num_seqs, num_q_heads, parts, head_dim, &args.part_acc, &args.part_ml));
    }
  }
  const unsigned grid = static_cast<unsigned>(num_seqs) * num_kv_heads * parts;
  // Small launches (at most six workgroups a CU, e.g. a decode tick of a small model) merge
  // in the last-arriving partition workgroup: the separate merge launch's fixed cost is a large
  // share there (C4 tick at batch 64: 2.375 against 2.403-2.410 ms).  Large launches keep the
  // separate merge, where the merging workgroups' tail costs more than the launch (C2, 2048
  // workgroups: 113.2 against 111.4 us).
  const int64_t cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  if (parts > 1 && !noalloc && ctx->d_merge_counters != nullptr &&
      static_cast<int64_t>(num_seqs) * num_kv_heads <= FI_MERGE_COUNTERS && static_cast<int64_t>(grid) <= 6 * cus)
    args.counters = ctx->d_merge_counters;
  switch (head_dim) {
    case 32:
      return launch_decode_dtype<32>(ctx, kv_dtype, args, grid, wt);
    case 64:
      return launch_decode_dtype<64>(ctx, kv_dtype, args, grid, wt);
    default:
      return launch_decode_dtype<128>(ctx, kv_dtype, args, grid, wt);
  }
}

}  // namespace

extern "C" {

int32_t fi_attn_decode_paged(fi_context* ctx, const float* d_q, const void* d_k_cache,
                             const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                             int32_t max_blocks_per_seq, const int32_t* d_context_lens,
                             int32_t num_seqs, int32_t max_context_len, int32_t num_q_heads,
                             int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                             int32_t num_blocks, float scale, float* d_out) {
  return decode_paged(ctx, d_q, d_k_cache, d_v_cache, kv_dtype, d_block_tables, max_blocks_per_seq,
                      d_context_lens, num_seqs, max_context_len, num_q_heads, num_kv_heads, head_dim,
                      block_size, num_blocks, scale, d_out, false);
}

int32_t fi_attn_decode_paged_qkv(fi_context* ctx, const float* d_qkv_parts, int32_t splits, const float* d_bias_q,
                                 const float* d_bias_k, const float* d_bias_v, const int32_t* d_positions,
                                 const float* d_cos, const float* d_sin, int32_t rotary_dims, int32_t max_positions,
                                 const int64_t* d_slot_mapping, void* d_k_cache, void* d_v_cache, int32_t kv_dtype,
                                 const int32_t* d_block_tables, int32_t max_blocks_per_seq,
                                 const int32_t* d_context_lens, int32_t num_seqs, int32_t max_context_len,
                                 int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                 int32_t num_blocks, float scale, float* d_q_out, float* d_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_kv_heads > 0 && head_dim > 0 && block_size > 0 && max_context_len >= 0 && num_seqs >= 0,
             FI_ERR_INVALID_SHAPE, "fi_attn_decode_paged_qkv: bad shape");
  // Large launches (more than six workgroups a CU) run the consumer and the attention as two
  // launches: every workgroup of the fused kernel forms its query rows again (one more
  // dependent load round each), which costs more there than the consumer launch (C5's
  // 256-sequence decode, 32768 workgroups: 27.4 against 24.7 ms a tick).
  const int part_tokens = kWaves * wave_tokens_for(num_kv_heads, head_dim);
  const int64_t parts = max_context_len == 0 ? 1 : (max_context_len + part_tokens - 1) / part_tokens;
  const int64_t cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  if (static_cast<int64_t>(num_seqs) * num_kv_heads * parts > 6 * cus) {
    FI_REQUIRE(d_q_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_attn_decode_paged_qkv: null q_out");
    FI_TRY(fi_qkv_rope_append(ctx, d_qkv_parts, splits, d_bias_q, d_bias_k, d_bias_v, d_positions, d_cos, d_sin,
                              rotary_dims, max_positions, d_slot_mapping, d_k_cache, d_v_cache, kv_dtype, num_blocks,
                              block_size, num_seqs, num_q_heads, num_kv_heads, head_dim, d_q_out));
    return decode_paged(ctx, d_q_out, d_k_cache, d_v_cache, kv_dtype, d_block_tables, max_blocks_per_seq,
                        d_context_lens, num_seqs, max_context_len, num_q_heads, num_kv_heads, head_dim,
                        block_size, num_blocks, scale, d_out, false);
  }
  const QkvIn qkv{d_qkv_parts, splits, d_bias_q, d_bias_k, d_bias_v, d_positions, d_cos, d_sin,
                  rotary_dims, max_positions, d_slot_mapping};
  return decode_paged(ctx, nullptr, d_k_cache, d_v_cache, kv_dtype, d_block_tables, max_blocks_per_seq,
                      d_context_lens, num_seqs, max_context_len, num_q_heads, num_kv_heads, head_dim,
                      block_size, num_blocks, scale, d_out, false, &qkv);
}

int32_t fi_attn_decode_paged_noalloc(fi_context* ctx, const float* d_q, const void* d_k_cache,
                                     const void* d_v_cache, int32_t kv_dtype, const int32_t* d_block_tables,
                                     int32_t max_blocks_per_seq, const int32_t* d_context_lens,
                                     int32_t num_seqs, int32_t max_context_len, int32_t num_q_heads,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t block_size,
                                     int32_t num_blocks, float scale, float* d_out) {
  return decode_paged(ctx, d_q, d_k_cache, d_v_cache, kv_dtype, d_block_tables, max_blocks_per_seq,
                      d_context_lens, num_seqs, max_context_len, num_q_heads, num_kv_heads, head_dim,
                      block_size, num_blocks, scale, d_out, true);
}

}  // extern "C"
