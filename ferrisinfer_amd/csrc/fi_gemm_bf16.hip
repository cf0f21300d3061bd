// Projection GEMMs over bf16-stored weights on MFMA v_mfma_f32_16x16x32_bf16 (f32 accumulate):
// the bf16 configurations' linear_f32_with_bias / matmul_f32 (kernel/cpu/matmul.rs:46-118,
// 424-499), the fused SwiGLU of the decoder block (runtime/reference.rs:346-360,
// kernel/cpu/elementwise.rs:118-207) and the greedy head (matmul_rhs_transposed_argmax_f32,
// kernel/cpu/matmul.rs:190-274).  The reference widens bf16 weights to f32 at load
// (io/safetensors.rs:540-542) and multiplies in f32; here the weights stay bf16 in HBM and the
// f32 activations are rounded to bf16 (nearest even) as they are staged, so the products differ
// from the reference by the activation rounding (bf16-storage tolerance).
//
// Packed weight (bf16): 16-column slabs grouped 16 to a 256-column group, K in 32-row steps:
//   packed[(((grp * Q + q) * 16 + s) * 64 + lane) * 8 + e]
//     = W[32 q + 8 (lane / 16) + e][16 (16 grp + s) + lane % 16]      (zero past K or N)
// which is the B operand of one 16x16x32 MFMA per (slab, step) for lane `lane`: every wave
// load is 16 contiguous bytes per lane and one group's K step is 16 KiB contiguous.
//
// Kernel: a workgroup of 4 waves computes a (16 MT) x (64 NT) tile over one split's K range
// (MT = 8, 6 or 4 row tiles above 64 rows, chosen per shape so the busiest CU gets the least
// work).  The activation block (16 MT rows x 32 k, or 64 k for bf16 activations) is staged per
// step through double-buffered LDS: f32 activations are rounded to bf16 (nearest even) on the
// way in, bf16 activations (rounded the same way by their producer) are copied, so both give
// the same products; bf16 halves the bytes the vector memory path carries per step, which at
// these tile sizes is as busy as the MFMAs.  Each wave owns NT slabs and streams their
// fragments from HBM through a register ring kDepth steps deep, and reads the A fragments of
// its MT row tiles from LDS.  Two workgroups share a CU, so one's barrier wait overlaps the
// other's MFMAs.  Workgroups are ordered so each XCD takes a contiguous range of (row block
// fastest, then column group, then split): the row blocks that share a column group's weights
// run together on one L2.
#include <algorithm>

#include "fi_common.h"
#include "fi_device.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kStepK = 32;        // K per MFMA step
constexpr int kGroupSlabs = 16;   // slabs per packed column group
constexpr int kDepth = 2;         // B ring depth (K steps in flight per wave)
constexpr int kOccupancy = 2;     // workgroups per CU the register budget allows
// bf16 per staged A row: a stage of S K steps plus 8 (80 or 144 bytes: conflict-free fragment reads)
constexpr int lds_row(int steps) { return steps * kStepK + 8; }

enum { kEpiPartial = 0, kEpiPairPartial = 1, kEpiSwiglu = 2, kEpiArgmax = 3 };

struct BGemmArgs {
  const void* a;             // [M, K] f32 or bf16 bits, row stride lda (elements)
  const uint16_t* bp;        // packed bf16 weight
  float* out;
  const float* bias0;        // SwiGLU: up bias
  const float* bias1;        // SwiGLU: gate bias
  int m, k, n;               // n: output columns of the store (pair modes: per projection)
  int lda;
  int q_total, q_per_split;  // 32-k steps
  int slabs;                 // 16-column slabs holding data
  int groups;                // column groups of 64 NT columns
  int mblocks;
  int splits;
  int total;                 // groups * mblocks * splits
  int tiles;                 // greedy head: 64 NT / 4-column wave tiles holding data
  int out_bf16;              // SwiGLU: store bf16 bits (nearest even) instead of f32
};

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

template <int MT, int NT, int EPI>
__device__ __forceinline__ void store_tile(const BGemmArgs& g, v4f (&acc)[MT][NT], int m0, int slab0, int z,
                                           int lane) {
  const int li = lane & 15, lk = lane >> 4;
  if constexpr (EPI == kEpiPartial || EPI == kEpiPairPartial) {
    const int ncols = EPI == kEpiPairPartial ? 2 * g.n : g.n;
    float* out = g.out + (size_t)z * g.m * ncols;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int s = slab0 + nt;
      // pair pack: slab 2j holds the up columns 16j.., slab 2j + 1 the gate columns; the partial
      // interleaves them as (up c, gate c) at columns (2c, 2c + 1)
      const int col = EPI == kEpiPairPartial ? 2 * (16 * (s >> 1) + li) + (s & 1) : 16 * s + li;
      const bool col_ok = EPI == kEpiPairPartial ? 16 * (s >> 1) + li < g.n : col < g.n;
      if (!col_ok) continue;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + 16 * mt + 4 * lk + v;
          if (row < g.m) out[(size_t)row * ncols + col] = acc[mt][nt][v];
        }
    }
  } else if constexpr (EPI == kEpiSwiglu) {
    static_assert(NT % 2 == 0, "SwiGLU needs (up, gate) slab pairs in one wave");
#pragma unroll
    for (int nt = 0; nt < NT; nt += 2) {
      const int c = 16 * ((slab0 + nt) >> 1) + li;
      if (c >= g.n) continue;
      const float b0 = g.bias0 ? g.bias0[c] : 0.0f;
      const float b1 = g.bias1 ? g.bias1[c] : 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + 16 * mt + 4 * lk + v;
          if (row >= g.m) continue;
          const float up = g.bias0 ? acc[mt][nt][v] + b0 : acc[mt][nt][v];
          float gate = g.bias1 ? acc[mt][nt + 1][v] + b1 : acc[mt][nt + 1][v];
          gate = gate * (1.0f / (1.0f + __expf(-gate)));
          if (g.out_bf16)
            reinterpret_cast<uint16_t*>(g.out)[(size_t)row * g.n + c] =
                static_cast<uint16_t>(fi::f32_to_bf16_bits(up * gate));
          else
            g.out[(size_t)row * g.n + c] = up * gate;
        }
    }
  } else {
    // Greedy head: per row, the wave tile's (max, first index of the max, sum of exp(x - max))
    // over its 64 NT / 4 columns (strict > keeps the first maximum, matmul.rs:532-589): each
    // lane folds its NT columns, then the 16 lanes of the row are combined; ties between
    // equal maxima keep the smaller index whatever the combine order.
    const int tile = slab0 / NT;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + 16 * mt + 4 * lk + v;
        float mx = -INFINITY, sum = 0.0f;
        int best = -1;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const int col = 16 * (slab0 + nt) + li;
          const float x = acc[mt][nt][v];
          const bool ok = col < g.n;
          const bool first = ok && best < 0;
          const bool larger = ok && best >= 0 && x > mx;
          const float nsum = first ? 1.0f : (larger ? sum * __expf(mx - x) + 1.0f : (ok ? sum + __expf(x - mx) : sum));
          mx = (first || larger) ? x : mx;
          best = (first || larger) ? col : best;
          sum = nsum;
        }
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const float omx = __shfl_xor(mx, off, 64);
          const float osum = __shfl_xor(sum, off, 64);
          const int obest = __shfl_xor(best, off, 64);
          const bool take = obest >= 0 && (best < 0 || omx > mx || (omx == mx && obest < best));
          const bool merge = obest >= 0 && best >= 0;
          const float nsum = !merge ? (take ? osum : sum)
                                    : (take ? osum + sum * __expf(mx - omx) : sum + osum * __expf(omx - mx));
          mx = take ? omx : mx;
          best = take ? obest : best;
          sum = nsum;
        }
        if (li == 0 && row < g.m && tile < g.tiles) {
          float* dst = g.out + ((size_t)row * g.tiles + tile) * 3;
          dst[0] = mx;
          reinterpret_cast<int*>(dst)[1] = best;
          dst[2] = sum;
        }
      }
  }
}

template <int MT, int NT, int EPI, bool KTAIL, bool A16>
__global__ __launch_bounds__(kThreads, kOccupancy) void gemm_bf16_kernel(BGemmArgs g) {
  constexpr int ROWS = 16 * MT;
  // A stage: f32 activations one K step (32 k = 128 bytes of a row), bf16 activations two K
  // steps (64 k = again 128 contiguous bytes of a row per stage, and half the barriers)
  constexpr int KS = A16 ? 2 : 1;
  constexpr int A_VEC = A16 ? 8 : 4;                     // elements per 16-byte A load
  constexpr int A_ROWQ = KS * kStepK / A_VEC;            // loads per row and stage
  constexpr int A_QUADS = ROWS * A_ROWQ;                 // 16-byte loads per stage
  constexpr int A_PER = (A_QUADS + kThreads - 1) / kThreads;
  constexpr int LDS_ROW = lds_row(KS);
  static_assert(A_QUADS % kThreads == 0 || A_QUADS < kThreads, "A stage must split over the threads");
  static_assert(!A16 || kDepth == 2, "bf16 stages hold the ring's two K steps");
  __shared__ __align__(16) uint16_t As[2][ROWS][LDS_ROW];

  // tile of this workgroup: the grid is padded to a multiple of 8; hardware workgroup L runs on
  // XCD L % 8 and takes logical tile (L % 8) * (grid / 8) + L / 8
  const int logical = (blockIdx.x % 8) * (gridDim.x / 8) + blockIdx.x / 8;
  if (logical >= g.total) return;
  const int mb = logical % g.mblocks;
  const int rest = logical / g.mblocks;
  const int grp = rest % g.groups;
  const int z = rest / g.groups;
  const int q0 = z * g.q_per_split;
  const int nq = min(g.q_per_split, g.q_total - q0);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int m0 = mb * ROWS;
  const int slab0 = grp * (kWaves * NT) + w * NT;  // the wave's first slab

  // ---- B: slab s of the wave at step q -> 16 bytes per lane ----
  const int pgroup = slab0 / kGroupSlabs, pslab = slab0 % kGroupSlabs;
  const uint4* bbase = reinterpret_cast<const uint4*>(g.bp) +
                       ((size_t)pgroup * g.q_total * kGroupSlabs + pslab) * 64 + lane;
  auto b_ptr = [&](int q, int nt) { return bbase + ((size_t)q * kGroupSlabs + nt) * 64; };
  uint4 ring[kDepth][NT];
  auto issue_b = [&](int step, uint4 (&slot)[NT]) {
    const int q = q0 + min(step, nq - 1);  // past the range: re-read the last step (unused)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) slot[nt] = *b_ptr(q, nt);
  };

  // ---- A staging: load i = tid + r * kThreads -> row i / A_ROWQ, k group i % A_ROWQ ----
  const int nst = (nq + KS - 1) / KS;  // stages of the split
  uint4 areg[A_PER];  // f32: one float4; bf16: eight bf16
  auto load_a = [&](int stage) {
    const int kq = (q0 + KS * min(stage, nst - 1)) * kStepK;
#pragma unroll
    for (int r = 0; r < A_PER; ++r) {
      const int i = tid + r * kThreads;
      const int row = min(m0 + i / A_ROWQ, g.m - 1);
      const int kk = kq + A_VEC * (i % A_ROWQ);
      if constexpr (A16) {
        const uint16_t* a16 = static_cast<const uint16_t*>(g.a) + (size_t)row * g.lda;
        // the stage's second K step may lie past K (an odd last step): its groups are masked
        // like a K tail; rows hold at least K rounded up to 8 (lda)
        if (!KTAIL && kk + A_VEC <= g.k) {
          areg[r] = *reinterpret_cast<const uint4*>(a16 + kk);
        } else {
          // elements past K read as zero
          const int kc = min(kk, ((g.k + 7) & ~7) - 8);
          const uint4 x = *reinterpret_cast<const uint4*>(a16 + kc);
          const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
          uint32_t yw[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {  // kc < kk: the whole group lies past K
            const uint32_t lo = kc == kk && kk + 2 * e < g.k ? (xw[e] & 0xffffu) : 0u;
            const uint32_t hi = kc == kk && kk + 2 * e + 1 < g.k ? (xw[e] & 0xffff0000u) : 0u;
            yw[e] = lo | hi;
          }
          areg[r] = make_uint4(yw[0], yw[1], yw[2], yw[3]);
        }
      } else {
        const float* a32 = static_cast<const float*>(g.a) + (size_t)row * g.lda;
        float4 v;
        if constexpr (KTAIL) {
          // rows hold at least K rounded up to 4 floats (lda); elements past K read as zero
          const int kc = min(kk, ((g.k + 3) & ~3) - 4);
          const float4 x = *reinterpret_cast<const float4*>(a32 + kc);
          v = make_float4(kk < g.k ? x.x : 0.f, kk + 1 < g.k ? x.y : 0.f, kk + 2 < g.k ? x.z : 0.f,
                          kk + 3 < g.k ? x.w : 0.f);
        } else {
          v = *reinterpret_cast<const float4*>(a32 + kk);
        }
        areg[r] = __builtin_bit_cast(uint4, v);
      }
    }
  };
  auto store_a = [&](int buf) {
#pragma unroll
    for (int r = 0; r < A_PER; ++r) {
      const int i = tid + r * kThreads;
      if (A_QUADS >= kThreads || i < A_QUADS) {
        if constexpr (A16) {
          *reinterpret_cast<uint4*>(&As[buf][i / A_ROWQ][A_VEC * (i % A_ROWQ)]) = areg[r];
        } else {
          const float4 x = __builtin_bit_cast(float4, areg[r]);
          const f32x4 v = {x.x, x.y, x.z, x.w};
          const bf16x4 h = __builtin_convertvector(v, bf16x4);
          *reinterpret_cast<bf16x4*>(&As[buf][i / A_ROWQ][A_VEC * (i % A_ROWQ)]) = h;
        }
      }
    }
  };

  v4f acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[mt][nt] = v4f{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int d = 0; d < kDepth; ++d) issue_b(d, ring[d]);
  load_a(0);
  store_a(0);
  load_a(1);
  __syncthreads();
  sched_fence();

  const int li = lane & 15, lk = lane >> 4;
  auto mfmas = [&](int buf, int col, const uint4 (&slot)[NT]) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const bf16x8 af = *reinterpret_cast<const bf16x8*>(&As[buf][16 * mt + li][col + 8 * lk]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
        acc[mt][nt] =
            __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, __builtin_bit_cast(bf16x8, slot[nt]), acc[mt][nt], 0, 0, 0);
    }
  };
  if constexpr (A16) {
    // stage st = K steps 2st (ring slot 0) and 2st + 1 (slot 1; absent past the split's end):
    // MFMAs from LDS buffer st & 1, stage st + 1's activations, prefetch st + 2's, then the
    // two slots' weight steps two steps ahead (after the activation loads, as below)
    for (int st = 0; st < nst; ++st) {
      const int buf = st & 1;
      mfmas(buf, 0, ring[0]);
      if (2 * st + 1 < nq) mfmas(buf, kStepK, ring[1]);  // workgroup-uniform
      store_a(buf ^ 1);
      load_a(st + 2);
      issue_b(2 * st + 2, ring[0]);
      issue_b(2 * st + 3, ring[1]);
      __syncthreads();
      sched_fence();
    }
    store_tile<MT, NT, EPI>(g, acc, m0, slab0, z, lane);
    return;
  }
  // one K step with ring slot u (compile-time): MFMAs from LDS buffer step & 1 and the slot,
  // stage step + 1's activations, prefetch step + 2's, then refill the slot kDepth steps ahead.
  // Loads complete in issue order, so the weight loads go out after the activation loads: the
  // wait for step + 2's activations (next step's LDS store) leaves them in flight, and a weight
  // step is waited for only by the MFMAs that use it, kDepth steps after its issue.
  auto k_step = [&](int step, uint4 (&slot)[NT]) {
    const int buf = step & 1;
    mfmas(buf, 0, slot);
    store_a(buf ^ 1);
    load_a(step + 2);
    issue_b(step + kDepth, slot);
    __syncthreads();
    sched_fence();
  };
  const int full = nq / kDepth * kDepth;
  for (int s0 = 0; s0 < full; s0 += kDepth) {
#pragma unroll
    for (int u = 0; u < kDepth; ++u) k_step(s0 + u, ring[u]);
  }
  // remainder (workgroup-uniform): slot u of the ring holds step full + u
  const int rem = nq - full;
#pragma unroll
  for (int u = 0; u + 1 < kDepth; ++u)
    if (u < rem) k_step(full + u, ring[u]);
  store_tile<MT, NT, EPI>(g, acc, m0, slab0, z, lane);
}

int32_t q_steps(int32_t k) { return (k + kStepK - 1) / kStepK; }

constexpr int kNt = 4;  // slabs per wave: a workgroup covers 256 columns

#ifndef FI_BGEMM_FORCE_MT
#define FI_BGEMM_FORCE_MT 0  // a fixed row tile count above 64 rows (0: chosen per shape)
#endif

// Row tiles per wave for M rows.  Up to 64 rows: the smallest power of two holding them.
// Above, 8, 6 or 4 (128-, 96- or 64-row blocks; the accumulators of two workgroups per CU fit
// the register file at 8), whichever leaves the busiest CU the fewest row tiles of the unsplit
// grid, ceil(blocks * groups / CUs) * MT, ties going to the larger tile (more MFMAs per weight
// fragment).  wo at M 2304 (16 column groups): 288 blocks of 128 rows give some CUs two, 384
// blocks of 96 rows give them two smaller ones.
int mt_for(fi_context* ctx, int m, int slabs) {
  if (m <= 64) return m > 32 ? 4 : (m > 16 ? 2 : 1);
  if (FI_BGEMM_FORCE_MT > 0) return FI_BGEMM_FORCE_MT;
  const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  const long groups = (slabs + kWaves * kNt - 1) / (kWaves * kNt);
  int best = 8;
  long best_cost = -1;
  for (int mt : {8, 6, 4}) {
    const long blocks = (m + 16L * mt - 1) / (16L * mt);
    const long cost = (blocks * groups + cus - 1) / cus * mt;
    if (best_cost < 0 || cost < best_cost) {
      best = mt;
      best_cost = cost;
    }
  }
  return best;
}

// Split count: three workgroups per CU where the tile grid is smaller, every split at least 8 K
// steps.  Where that asks for partials (splits x M x N f32) beyond the weight's bytes (large M),
// the split count between the two is the one with the least modelled time: the busiest CU's
// row-tile K steps, ceil(tiles s / CUs) MT Q / s, at ~67 ns each (16 x 256 x 32 products at the
// kernel's ~40 % of the bf16 peak per CU), plus each extra partial written and read back at
// ~6 TB/s (wo at M 2304: 2 splits, 100 -> 83 us with the consumer 23 -> 31 us).
int split_count(fi_context* ctx, int m, int k, int slabs) {
  const int mt = mt_for(ctx, m, slabs);
  const int mblocks = (m + 16 * mt - 1) / (16 * mt);
  const int groups = (slabs + kWaves * kNt - 1) / (kWaves * kNt);
  const int q = q_steps(k);
  const long tiles = (long)mblocks * groups;
  const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  // three workgroups per CU: a CU's two resident tiles are followed by a third, so the last
  // round is a third of a round (w2 at M 2304: 2 -> 3 splits, 345 -> 314 us with its consumer)
  const long target = (long)(kOccupancy + 1) * cus;
  long s = std::max(1L, (target + tiles - 1) / tiles);
  s = std::min(s, std::max(1L, static_cast<long>(q / 8)));
  s = std::min(s, 32L);
  const long lo = std::min(s, std::max(1L, static_cast<long>(k) / (2L * std::max(m, 16))));
  if (lo < s) {
    const double partial_bytes = 8.0 * m * 16.0 * slabs;  // one more partial, written and read
    double best_ns = 0.0;
    long best = lo;
    for (long c = lo; c <= s; ++c) {
      const long per = (q + c - 1) / c;
      const double busy = static_cast<double>((tiles * c + cus - 1) / cus) * mt * per;
      const double ns = 67.0 * busy + static_cast<double>(c - 1) * partial_bytes / 6000.0;  // 6000 B/ns
      if (c == lo || ns < best_ns) {
        best = c;
        best_ns = ns;
      }
    }
    s = best;
  }
  const int per = (q + static_cast<int>(s) - 1) / static_cast<int>(s);
  return (q + per - 1) / per;  // every split non-empty
}

template <int MT, int EPI, bool A16>
void launch_mt(fi_context* ctx, const BGemmArgs& g) {
  const dim3 grid(static_cast<unsigned>((g.total + 7) / 8 * 8));
  if (g.k % kStepK == 0) {
    hipLaunchKernelGGL((gemm_bf16_kernel<MT, kNt, EPI, false, A16>), grid, dim3(kThreads), 0, ctx->stream, g);
  } else {
    hipLaunchKernelGGL((gemm_bf16_kernel<MT, kNt, EPI, true, A16>), grid, dim3(kThreads), 0, ctx->stream, g);
  }
}

template <int MT, int EPI>
void launch_mt(fi_context* ctx, const BGemmArgs& g, bool a16) {
  if (a16)
    launch_mt<MT, EPI, true>(ctx, g);
  else
    launch_mt<MT, EPI, false>(ctx, g);
}

template <int EPI>
int32_t launch_bgemm(fi_context* ctx, BGemmArgs g, int splits, bool a16) {
  const int mt = mt_for(ctx, g.m, g.slabs);
  g.mblocks = (g.m + 16 * mt - 1) / (16 * mt);
  g.groups = (g.slabs + kWaves * kNt - 1) / (kWaves * kNt);
  g.splits = splits;
  g.total = g.groups * g.mblocks * splits;
  switch (mt) {
    case 8:
      launch_mt<8, EPI>(ctx, g, a16);
      break;
    case 6:
      launch_mt<6, EPI>(ctx, g, a16);
      break;
    case 4:
      launch_mt<4, EPI>(ctx, g, a16);
      break;
    case 2:
      launch_mt<2, EPI>(ctx, g, a16);
      break;
    default:
      launch_mt<1, EPI>(ctx, g, a16);
      break;
  }
  FI_CHECK_LAUNCH("gemm_bf16_kernel");
  return FI_OK;
}

// Data slabs of an N-column weight (pair: the up and gate slabs of each 16 columns), and the
// packed slabs: whole 16-slab groups so every workgroup's loads stay inside the allocation.
int32_t data_slabs(int32_t n, bool pair) { return pair ? 2 * ((n + 15) / 16) : (n + 15) / 16; }
int32_t packed_slabs(int32_t n, bool pair) {
  return (data_slabs(n, pair) + kGroupSlabs - 1) / kGroupSlabs * kGroupSlabs;
}

struct PackSourcesBf16 {
  const void* src[3];
  int n[3];
  int count;
};

template <typename T>
__device__ __forceinline__ uint16_t as_bf16(const T* p, size_t i) {
  if constexpr (sizeof(T) == 4) {
    return static_cast<uint16_t>(fi::f32_to_bf16_bits(p[i]));
  } else {
    return p[i];
  }
}

// One thread per packed bf16.  Column mode: the packed matrix is the column concatenation of
// the sources ([K, n_i], or one [n, K] source with src_layout 1).  Pair mode: slab 2j holds
// columns 16j.. of source 0 (up), slab 2j + 1 the same columns of source 1 (gate).
template <typename T>
__global__ void weight_pack_bf16_kernel(PackSourcesBf16 s, int pair, int src_layout, int k, int q_total,
                                        size_t total, uint16_t* __restrict__ dst) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int e = static_cast<int>(i % 8);
    size_t r = i / 8;
    const int lane = static_cast<int>(r % 64);
    r /= 64;
    const int sl = static_cast<int>(r % kGroupSlabs);
    r /= kGroupSlabs;
    const int q = static_cast<int>(r % q_total);
    const int grp = static_cast<int>(r / q_total);
    const int slab = grp * kGroupSlabs + sl;
    const int kk = kStepK * q + 8 * (lane / 16) + e;
    int col, j = 0;
    if (pair) {
      col = 16 * (slab >> 1) + lane % 16;
      j = slab & 1;
    } else {
      col = 16 * slab + lane % 16;
      while (j + 1 < s.count && col >= s.n[j]) {
        col -= s.n[j];
        ++j;
      }
    }
    const int ncols = pair ? s.n[0] : s.n[j];
    const T* src = static_cast<const T*>(s.src[j]);
    uint16_t v = 0;
    if (kk < k && col < ncols) v = as_bf16(src, src_layout == 0 ? (size_t)kk * ncols + col : (size_t)col * k + kk);
    dst[i] = v;
  }
}

int32_t launch_pack(fi_context* ctx, const PackSourcesBf16& s, int32_t src_dtype, int pair, int src_layout, int k,
                    int n, uint16_t* dst) {
  size_t total = 0;
  FI_TRY(fi_weight_packed_bf16_elems(k, n, pair, &total));
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((total + 255) / 256, 65536));
  if (src_dtype == FI_DTYPE_F32) {
    hipLaunchKernelGGL(weight_pack_bf16_kernel<float>, dim3(blocks), dim3(256), 0, ctx->stream, s, pair, src_layout,
                       k, q_steps(k), total, dst);
  } else {
    hipLaunchKernelGGL(weight_pack_bf16_kernel<uint16_t>, dim3(blocks), dim3(256), 0, ctx->stream, s, pair,
                       src_layout, k, q_steps(k), total, dst);
  }
  FI_CHECK_LAUNCH("weight_pack_bf16_kernel");
  return FI_OK;
}

int32_t check_common(fi_context* ctx, const void* a, int32_t a_dtype, int32_t lda, const uint16_t* bp, int32_t m,
                     int32_t k, int32_t n) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(m >= 0 && k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "bf16 GEMM: bad shape");
  FI_REQUIRE(a_dtype == FI_DTYPE_F32 || a_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "bf16 GEMM: the activation dtype must be f32 or bf16");
  const int vec = a_dtype == FI_DTYPE_BF16 ? 8 : 4;  // elements per 16-byte load
  FI_REQUIRE(lda % vec == 0 && lda >= (k + vec - 1) / vec * vec, FI_ERR_INVALID_SHAPE,
             a_dtype == FI_DTYPE_BF16 ? "bf16 GEMM: lda must be a multiple of 8 and at least K rounded up to 8 (bf16 A)"
                                      : "bf16 GEMM: lda must be a multiple of 4 and at least K rounded up to 4");
  FI_REQUIRE(m == 0 || (a && bp), FI_ERR_INVALID_CONFIG, "bf16 GEMM: null pointer");
  FI_REQUIRE(m == 0 || (reinterpret_cast<uintptr_t>(a) % 16 == 0 && reinterpret_cast<uintptr_t>(bp) % 16 == 0),
             FI_ERR_INVALID_CONFIG, "bf16 GEMM: A and the packed weight must be 16-byte aligned");
  return FI_OK;
}

}  // namespace

extern "C" {

int32_t fi_weight_packed_bf16_elems(int32_t k, int32_t n, int32_t pair, size_t* elems) {
  FI_REQUIRE(k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_weight_packed_bf16_elems: dimensions must be positive");
  FI_REQUIRE(elems != nullptr, FI_ERR_INVALID_CONFIG, "fi_weight_packed_bf16_elems: null output");
  *elems = (size_t)packed_slabs(n, pair != 0) * q_steps(k) * 64 * 8;
  return FI_OK;
}

int32_t fi_weight_pack_bf16(fi_context* ctx, const void* d_src, int32_t src_dtype, int32_t src_layout, int32_t k,
                            int32_t n, uint16_t* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(src_layout == 0 || src_layout == 1, FI_ERR_INVALID_LAYOUT, "fi_weight_pack_bf16: src_layout must be 0 or 1");
  FI_REQUIRE(src_dtype == FI_DTYPE_F32 || src_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_weight_pack_bf16: source dtype must be f32 or bf16");
  FI_REQUIRE(k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_weight_pack_bf16: dimensions must be positive");
  FI_REQUIRE(d_src && d_dst, FI_ERR_INVALID_CONFIG, "fi_weight_pack_bf16: null pointer");
  PackSourcesBf16 s{{d_src, nullptr, nullptr}, {n, 0, 0}, 1};
  return launch_pack(ctx, s, src_dtype, 0, src_layout, k, n, d_dst);
}

int32_t fi_weight_pack_bf16_columns(fi_context* ctx, const void* const* d_srcs, const int32_t* ns, int32_t count,
                                    int32_t src_dtype, int32_t k, uint16_t* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(count >= 1 && count <= 3, FI_ERR_INVALID_CONFIG, "fi_weight_pack_bf16_columns: 1 to 3 sources");
  FI_REQUIRE(d_srcs && ns && d_dst, FI_ERR_INVALID_CONFIG, "fi_weight_pack_bf16_columns: null pointer");
  FI_REQUIRE(src_dtype == FI_DTYPE_F32 || src_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_weight_pack_bf16_columns: source dtype must be f32 or bf16");
  FI_REQUIRE(k > 0, FI_ERR_INVALID_SHAPE, "fi_weight_pack_bf16_columns: K must be positive");
  PackSourcesBf16 s{{nullptr, nullptr, nullptr}, {0, 0, 0}, count};
  int32_t n = 0;
  for (int i = 0; i < count; ++i) {
    FI_REQUIRE(d_srcs[i] && ns[i] > 0, FI_ERR_INVALID_CONFIG, "fi_weight_pack_bf16_columns: empty source");
    s.src[i] = d_srcs[i];
    s.n[i] = ns[i];
    n += ns[i];
  }
  return launch_pack(ctx, s, src_dtype, 0, 0, k, n, d_dst);
}

int32_t fi_weight_pack_bf16_pair(fi_context* ctx, const void* d_up, const void* d_gate, int32_t src_dtype, int32_t k,
                                 int32_t n, uint16_t* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(src_dtype == FI_DTYPE_F32 || src_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_weight_pack_bf16_pair: source dtype must be f32 or bf16");
  FI_REQUIRE(k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_weight_pack_bf16_pair: dimensions must be positive");
  FI_REQUIRE(d_up && d_gate && d_dst, FI_ERR_INVALID_CONFIG, "fi_weight_pack_bf16_pair: null pointer");
  PackSourcesBf16 s{{d_up, d_gate, nullptr}, {n, n, 0}, 2};
  return launch_pack(ctx, s, src_dtype, 1, 0, k, n, d_dst);
}

int32_t fi_gemm_bf16_splits(fi_context* ctx, int32_t m, int32_t k, int32_t n, int32_t* splits) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(m >= 0 && k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_gemm_bf16_splits: bad shape");
  FI_REQUIRE(splits != nullptr, FI_ERR_INVALID_CONFIG, "fi_gemm_bf16_splits: null output");
  *splits = split_count(ctx, m, k, data_slabs(n, false));
  return FI_OK;
}

int32_t fi_gemm_bf16(fi_context* ctx, const void* d_a, int32_t a_dtype, int32_t lda, const uint16_t* d_bp, int32_t k,
                     int32_t n, int32_t m, int32_t splits, float* d_out) {
  FI_TRY(check_common(ctx, d_a, a_dtype, lda, d_bp, m, k, n));
  FI_REQUIRE(splits >= 1 && splits <= q_steps(k), FI_ERR_INVALID_CONFIG, "fi_gemm_bf16: splits out of range");
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_gemm_bf16: null output");
  BGemmArgs g{};
  g.a = d_a;
  g.bp = d_bp;
  g.out = d_out;
  g.m = m;
  g.k = k;
  g.n = n;
  g.lda = lda;
  g.q_total = q_steps(k);
  g.q_per_split = (g.q_total + splits - 1) / splits;
  g.slabs = data_slabs(n, false);
  const int used = (g.q_total + g.q_per_split - 1) / g.q_per_split;
  FI_REQUIRE(used == splits, FI_ERR_INVALID_CONFIG,
             "fi_gemm_bf16: splits must divide the K steps into non-empty ranges (use fi_gemm_bf16_splits)");
  return launch_bgemm<kEpiPartial>(ctx, g, splits, a_dtype == FI_DTYPE_BF16);
}

int32_t fi_gemm_bf16_swiglu(fi_context* ctx, const void* d_a, int32_t a_dtype, int32_t lda, const uint16_t* d_bp_pair,
                            int32_t k, int32_t n, int32_t m, const float* d_bias_up, const float* d_bias_gate,
                            void* d_out, int32_t out_dtype) {
  FI_TRY(check_common(ctx, d_a, a_dtype, lda, d_bp_pair, m, k, n));
  FI_REQUIRE(out_dtype == FI_DTYPE_F32 || out_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_gemm_bf16_swiglu: the output dtype must be f32 or bf16");
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_gemm_bf16_swiglu: null output");
  const bool a16 = a_dtype == FI_DTYPE_BF16;
  BGemmArgs g{};
  g.a = d_a;
  g.bp = d_bp_pair;
  g.bias0 = d_bias_up;
  g.bias1 = d_bias_gate;
  g.m = m;
  g.k = k;
  g.n = n;
  g.lda = lda;
  g.q_total = q_steps(k);
  g.slabs = data_slabs(n, true);
  const int splits = split_count(ctx, m, k, g.slabs);
  if (splits == 1) {  // the epilogue applies SwiGLU directly
    g.out = static_cast<float*>(d_out);
    g.out_bf16 = out_dtype == FI_DTYPE_BF16;
    g.q_per_split = g.q_total;
    return launch_bgemm<kEpiSwiglu>(ctx, g, 1, a16);
  }
  // (up, gate) partial pairs per split, then the split sum + SwiGLU
  FI_TRY(fi::ensure_workspace(ctx, (size_t)splits * m * 2 * n * sizeof(float)));
  g.out = static_cast<float*>(ctx->workspace);
  g.q_per_split = (g.q_total + splits - 1) / splits;
  FI_TRY(launch_bgemm<kEpiPairPartial>(ctx, g, splits, a16));
  return fi::splitk_swiglu(ctx, g.out, splits, d_bias_up, d_bias_gate, m, n, d_out, out_dtype == FI_DTYPE_BF16);
}

int32_t fi_lm_head_argmax_bf16(fi_context* ctx, const void* d_hidden, int32_t a_dtype, int32_t lda,
                               const uint16_t* d_bp, int32_t m, int32_t hidden, int32_t vocab, int32_t* d_token,
                               float* d_prob) {
  FI_TRY(check_common(ctx, d_hidden, a_dtype, lda, d_bp, m, hidden, vocab));
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_token && d_prob, FI_ERR_INVALID_CONFIG, "fi_lm_head_argmax_bf16: null output");
  BGemmArgs g{};
  g.a = d_hidden;
  g.bp = d_bp;
  g.m = m;
  g.k = hidden;
  g.n = vocab;
  g.lda = lda;
  g.q_total = q_steps(hidden);
  g.q_per_split = g.q_total;
  g.slabs = data_slabs(vocab, false);
  g.tiles = (g.slabs + kNt - 1) / kNt;
  FI_TRY(fi::ensure_workspace(ctx, (size_t)m * g.tiles * 3 * sizeof(float)));
  g.out = static_cast<float*>(ctx->workspace);
  FI_TRY(launch_bgemm<kEpiArgmax>(ctx, g, 1, a_dtype == FI_DTYPE_BF16));
  return fi::argmax_merge(ctx, g.out, g.tiles, m, d_token, d_prob);
}

}  // extern "C"
