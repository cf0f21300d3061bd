// Weight-streaming projection GEMMs on MFMA (v_mfma_f32_16x16x4_f32) over weights re-laid
// out once at upload, plus the kernels that consume their split-K partials.  Replaces the
// decoder block's matmul_f32 / linear_f32_with_bias calls and the elementwise ops around
// them (kernel/cpu/matmul.rs:46-118, 190-274; runtime/reference.rs:163-370, 712-871,
// 1103-1191; kernel/cpu/elementwise.rs:48-207; kernel/cpu/reduction.rs:3-73).
//
// Packed weight layout.  A weight B [K, N] (the reference's [in, out]) is cut into slabs of
// 16*PW output columns; each slab stores its K rows (zero-padded to a multiple of 16) in
// MFMA-fragment order so that one wave reads each 16-row step as four 64*PW-float runs:
//   packed[((slab * Q + q) * 4 + e) * 64 * PW + lane * PW + p]
//     = B[16q + 4*(lane/16) + e][slab * 16 * PW + PW * (lane % 16) + p]
// (Q = ceil(K/16); zero outside [0,K) x [0,N)).  Lane (j, kk) = (lane % 16, lane / 16) loads
// its PW-vector for step e with one load; element p is the B operand of N-tile p, so tile p's
// column j is output column slab*16*PW + PW*j + p and a lane finally holds PW adjacent
// outputs of a row (one vector store).  The A operand is read straight from the row-major
// activations: lane (i, kk) loads A[row i][16q + 4kk .. +3] and feeds element e to step e,
// the same k order the packed B uses.
//
// Kernel shape: a workgroup of 4 waves owns one (16*MT)-row x (16*PW)-column output tile
// and a range of K steps; each wave takes a contiguous quarter of the range, keeps a ring of
// in-flight loads (no LDS, no barrier in the main loop), and the quarters are summed through
// LDS in wave order.  Workgroups along z split K further; their partials are summed by the
// consumer kernels in split order.  Every summation order is fixed by the shape, so results
// are deterministic and independent of the batch composition of other rows.
#include <algorithm>
#include <type_traits>

#include "fi_common.h"
#include "fi_device.h"

extern "C" int32_t fi_weight_packed_floats(int32_t k, int32_t n, int32_t pack_width, size_t* floats);

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kPackW32 = 32;  // pack width selecting the 32-column layout of gemm_w32_kernel

template <int PW>
struct PVec;
template <>
struct PVec<1> {
  using T = float;
  __device__ static float get(const T& v, int) { return v; }
};
template <>
struct PVec<2> {
  using T = float2;
  __device__ static float get(const T& v, int p) { return p == 0 ? v.x : v.y; }
};
template <>
struct PVec<4> {
  using T = float4;
  __device__ static float get(const T& v, int p) { return p == 0 ? v.x : (p == 1 ? v.y : (p == 2 ? v.z : v.w)); }
};

__device__ __forceinline__ void sched_fence() { __builtin_amdgcn_sched_barrier(0); }

enum Epi : int { kEpiPartial = 0, kEpiSwiglu = 1, kEpiArgmax = 2 };

struct PGemmArgs {
  const float* a;       // [M, lda]
  const float* bp;      // packed weight
  float* out;           // partial: [splits, M, N]; swiglu: [M, N]; argmax: [M, slabs, 3]
  const float* bias0;   // swiglu: bias of the first (up) weight, may be null
  const float* bias1;   // swiglu: bias of the second (gate) weight, may be null
  int m, k, n, lda;
  int q_total;          // ceil(K / 16)
  int q_per_split;      // K steps per workgroup (z)
  int slabs;
};

// A rows are clamped to M-1 (their outputs are never stored).  With K a multiple of 16 every
// step is a plain 16-byte load; otherwise (KTAIL) each element is loaded from a clamped,
// always-valid address and zeroed past the row end with a select, so there is no divergent
// branch (a branch here would force the compiler to drain the load ring).
template <bool KTAIL>
__device__ __forceinline__ float4 load_a(const float* row, int k0, int k) {
  if constexpr (!KTAIL) {
    return *reinterpret_cast<const float4*>(row + k0);
  } else {
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float x = row[min(k0 + i, k - 1)];
      v[i] = k0 + i < k ? x : 0.0f;
    }
    return make_float4(v[0], v[1], v[2], v[3]);
  }
}

// Writes one wave's (16*MT) x (16*PW) accumulator tile.  Lane (li, lk) holds
// acc[mt][p][v] = C[m0 + 16mt + 4lk + v][slab*16*PW + PW*li + p].
template <int MT, int PW, int EPI>
__device__ __forceinline__ void store_tile(const PGemmArgs& g, v4f (&acc)[MT][PW], int m0, int slab, int z,
                                           int lane) {
  const int li = lane & 15, lk = lane >> 4;
  const int col0 = slab * 16 * PW + PW * li;
  if constexpr (EPI == kEpiPartial) {
    float* out = g.out + (size_t)z * g.m * g.n;
    const bool vec = col0 + PW <= g.n && (g.n % PW) == 0;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + 16 * mt + 4 * lk + v;
        if (row >= g.m) continue;
        float* dst = out + (size_t)row * g.n + col0;
        if (vec) {
          if constexpr (PW == 4) {
            *reinterpret_cast<float4*>(dst) = make_float4(acc[mt][0][v], acc[mt][1][v], acc[mt][2][v], acc[mt][3][v]);
          } else if constexpr (PW == 2) {
            *reinterpret_cast<float2*>(dst) = make_float2(acc[mt][0][v], acc[mt][1][v]);
          } else {
            dst[0] = acc[mt][0][v];
          }
        } else {
#pragma unroll
          for (int p = 0; p < PW; ++p)
            if (col0 + p < g.n) dst[p] = acc[mt][p][v];
        }
      }
  } else if constexpr (EPI == kEpiSwiglu) {
    // pair pack: p = 0 is the up projection (w1), p = 1 the gate (w3) of output column c.
    // elementwise.rs:118-207 as used at reference.rs:346-360: gate <- gate * (1 / (1 +
    // exp(-gate))); up <- up * gate.
    static_assert(PW == 2, "SwiGLU epilogue needs the pair pack");
    const int c = slab * 16 + li;
    if (c < g.n) {
      const float b0 = g.bias0 ? g.bias0[c] : 0.0f;
      const float b1 = g.bias1 ? g.bias1[c] : 0.0f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + 16 * mt + 4 * lk + v;
          if (row >= g.m) continue;
          const float up = g.bias0 ? acc[mt][0][v] + b0 : acc[mt][0][v];
          float gate = g.bias1 ? acc[mt][1][v] + b1 : acc[mt][1][v];
          gate = gate * (1.0f / (1.0f + __expf(-gate)));
          g.out[(size_t)row * g.n + c] = up * gate;
        }
    }
  } else {
    // Greedy head: per row, the slab's (max, first index of the max, sum of exp(x - max))
    // over its columns in index order (strict > keeps the first maximum, matmul.rs:532-589);
    // lanes are combined left to right so ties keep the smaller index.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int row = m0 + 16 * mt + 4 * lk + v;
        float mx = -INFINITY, sum = 0.0f;
        int best = -1;
#pragma unroll
        for (int p = 0; p < PW; ++p) {
          const int col = col0 + p;
          if (col >= g.n) break;
          const float x = acc[mt][p][v];
          if (best < 0) {
            mx = x;
            sum = 1.0f;
            best = col;
          } else if (x > mx) {
            sum = sum * __expf(mx - x) + 1.0f;
            mx = x;
            best = col;
          } else {
            sum += __expf(x - mx);
          }
        }
        // combine the 16 lanes li = 0..15 of this row (same lk): lower lanes hold lower columns
#pragma unroll
        for (int off = 1; off < 16; off <<= 1) {
          const float omx = __shfl_xor(mx, off, 64);
          const float osum = __shfl_xor(sum, off, 64);
          const int obest = __shfl_xor(best, off, 64);
          if (obest >= 0) {
            if (best < 0) {
              mx = omx;
              sum = osum;
              best = obest;
            } else if (omx > mx || (omx == mx && obest < best)) {
              sum = osum + sum * __expf(mx - omx);
              mx = omx;
              best = obest;
            } else {
              sum = sum + osum * __expf(omx - mx);
            }
          }
        }
        if (li == 0 && row < g.m) {
          float* dst = g.out + ((size_t)row * g.slabs + slab) * 3;
          dst[0] = mx;
          reinterpret_cast<int*>(dst)[1] = best;
          dst[2] = sum;
        }
      }
  }
}

#ifndef FI_PGEMM_MIN_WAVES
#define FI_PGEMM_MIN_WAVES 2  // waves per SIMD the register budget must allow
#endif
#ifndef FI_PGEMM_RING_REGS
#define FI_PGEMM_RING_REGS 64  // VGPRs the ring of in-flight loads may hold
#endif

template <int MT, int PW, int EPI, bool KTAIL>
__global__ __launch_bounds__(kThreads, FI_PGEMM_MIN_WAVES) void gemm_packed_kernel(PGemmArgs g) {
  using BV = typename PVec<PW>::T;
  constexpr int STEP_REGS = 4 * MT + 4 * PW;  // VGPRs one K step of loads occupies
  constexpr int DEPTH = FI_PGEMM_RING_REGS / STEP_REGS < 2 ? 2 : (FI_PGEMM_RING_REGS / STEP_REGS > 8 ? 8 : FI_PGEMM_RING_REGS / STEP_REGS);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int li = lane & 15, lk = lane >> 4;
  const int slab = blockIdx.x, mblk = blockIdx.y, z = blockIdx.z;
  const int m0 = mblk * 16 * MT;

  // this wave's K steps: a contiguous quarter of the workgroup's range
  const int wq0 = z * g.q_per_split;
  const int wq1 = min(g.q_total, wq0 + g.q_per_split);
  const int per = (wq1 - wq0 + kWaves - 1) / kWaves;
  const int q_beg = min(wq1, wq0 + w * per);
  const int q_end = min(wq1, q_beg + per);

  const float* arow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) arow[mt] = g.a + (size_t)min(m0 + 16 * mt + li, g.m - 1) * g.lda + 4 * lk;
  const BV* bbase = reinterpret_cast<const BV*>(g.bp) + (size_t)slab * g.q_total * 4 * 64 + lane;

  v4f acc[MT][PW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int p = 0; p < PW; ++p) acc[mt][p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  if (q_beg < q_end) {  // wave-uniform
    // Ring of R = DEPTH + 1 slots: step s lives in slot (s - q_beg) % R.  Before step s is
    // multiplied, the loads of step s + DEPTH go into the slot step s - 1 has released, so
    // DEPTH steps stay in flight while the MFMAs of step s run.
    constexpr int R = DEPTH + 1;
    float4 ra[R][MT];
    BV rb[R][4];
    auto issue = [&](int q, int slot) {
      q = min(q, q_end - 1);  // clamped refetches hit the cache: no extra HBM traffic
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) ra[slot][mt] = load_a<KTAIL>(arow[mt], 16 * q, g.k - 4 * lk);
      const BV* bq = bbase + (size_t)q * 4 * 64;
#pragma unroll
      for (int e = 0; e < 4; ++e) rb[slot][e] = bq[e * 64];
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(q_beg + d, d);
    for (int q = q_beg; q < q_end; q += R) {
#pragma unroll
      for (int d = 0; d < R; ++d) {
        issue(q + d + DEPTH, (d + DEPTH) % R);
        sched_fence();
        if (q + d < q_end) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const float av = e == 0 ? ra[d][mt].x : (e == 1 ? ra[d][mt].y : (e == 2 ? ra[d][mt].z : ra[d][mt].w));
#pragma unroll
              for (int p = 0; p < PW; ++p)
                acc[mt][p] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, PVec<PW>::get(rb[d][e], p), acc[mt][p], 0, 0, 0);
            }
        }
        sched_fence();
      }
    }
  }

  // ---- sum the four K quarters in wave order through LDS ----
  __shared__ v4f s_part[kWaves - 1][MT * PW][64];
  if (w > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int p = 0; p < PW; ++p) s_part[w - 1][mt * PW + p][lane] = acc[mt][p];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int src = 0; src < kWaves - 1; ++src)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int p = 0; p < PW; ++p) acc[mt][p] += s_part[src][mt * PW + p][lane];

  store_tile<MT, PW, EPI>(g, acc, m0, slab, z, lane);
}

// Shared-activation variant: the 4 waves of a workgroup own 4 consecutive weight slabs and
// one (16*MT)-row block over the workgroup's K range, so the activation rows are read once
// per workgroup: 64-k chunks of A are staged through double-buffered LDS (one barrier per
// chunk) in MFMA-fragment order, while each wave streams its own slab through a register ring
// of B loads issued DEPTH steps ahead.  No cross-wave reduction: each wave stores its tile.
template <int MT, int PW, int EPI, bool KTAIL>
__global__ __launch_bounds__(kThreads, 2) void gemm_lds_kernel(PGemmArgs g) {
  using BV = typename PVec<PW>::T;
  constexpr int KC = 4;                // K steps (16 k each) per staged A chunk
  constexpr int R = KC;                // B ring slots: the slot of a step is its index in the chunk
  constexpr int DEPTH = R - 1;         // B steps in flight ahead of the MFMAs
  constexpr int A_F4 = KC * MT * 64;   // float4 per A chunk
  static_assert(A_F4 % kThreads == 0, "A chunk must split evenly over the workgroup");
  constexpr int A_PER_T = A_F4 / kThreads;
  __shared__ float4 s_a[2][A_F4];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int slab_id = blockIdx.x * kWaves + w;
  const int slab = min(slab_id, g.slabs - 1);  // a short last group still loads valid data
  const int m0 = blockIdx.y * 16 * MT, z = blockIdx.z;
  const int q0 = z * g.q_per_split;
  const int q1 = min(g.q_total, q0 + g.q_per_split);
  const int nchunks = (q1 - q0 + KC - 1) / KC;

  // A chunk slot i = (j * MT + mt) * 64 + ln holds A[m0 + 16mt + ln%16][16(q0+c*KC+j) + 4(ln/16) .. +3]
  float4 areg[A_PER_T];
  auto load_a_chunk = [&](int c) {
#pragma unroll
    for (int r = 0; r < A_PER_T; ++r) {
      const int i = tid + r * kThreads;
      const int j = i / (MT * 64), mt = (i / 64) % MT, ln = i % 64;
      const int q = min(q0 + c * KC + j, q1 - 1);
      const int row = min(m0 + 16 * mt + (ln & 15), g.m - 1);
      areg[r] = load_a<KTAIL>(g.a + (size_t)row * g.lda + 4 * (ln >> 4), 16 * q, g.k - 4 * (ln >> 4));
    }
  };
  auto store_a_chunk = [&](int buf) {
#pragma unroll
    for (int r = 0; r < A_PER_T; ++r) s_a[buf][tid + r * kThreads] = areg[r];
  };

  const BV* bbase = reinterpret_cast<const BV*>(g.bp) + (size_t)slab * g.q_total * 4 * 64 + lane;
  BV rb[R][4];
  auto issue_b = [&](int q, int slot) {
    q = min(q, q1 - 1);  // clamped refetches hit the cache: no extra HBM traffic
    const BV* bq = bbase + (size_t)q * 4 * 64;
#pragma unroll
    for (int e = 0; e < 4; ++e) rb[slot][e] = bq[e * 64];
  };

  v4f acc[MT][PW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int p = 0; p < PW; ++p) acc[mt][p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  load_a_chunk(0);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) issue_b(q0 + d, d);
  store_a_chunk(0);
  __syncthreads();
  for (int c = 0; c < nchunks; ++c) {
    const bool more = c + 1 < nchunks;  // workgroup-uniform
    if (more) load_a_chunk(c + 1);
    const float4* sa = s_a[c & 1];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int q = q0 + c * KC + j;
      issue_b(q + DEPTH, (j + DEPTH) % R);
      sched_fence();
      if (q < q1) {
        float4 af[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) af[mt] = sa[(j * MT + mt) * 64 + lane];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const float av = e == 0 ? af[mt].x : (e == 1 ? af[mt].y : (e == 2 ? af[mt].z : af[mt].w));
#pragma unroll
            for (int p = 0; p < PW; ++p)
              acc[mt][p] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, PVec<PW>::get(rb[j][e], p), acc[mt][p], 0, 0, 0);
          }
      }
      sched_fence();
    }
    if (more) store_a_chunk((c + 1) & 1);
    __syncthreads();
  }
  if (slab_id < g.slabs) store_tile<MT, PW, EPI>(g, acc, m0, slab, z, lane);
}

// ---------------------------------------------------------------------------------------
// Three-term bf16 kernel.  Each f32 operand is split exactly into three bf16 terms,
// x = hi + mid + lo (hi = x rounded to nearest even, mid the same of the exact remainder, lo the
// rest, which has at most 8 significant bits), and a product is the sum of the six terms above
// 2^-24 relative (hi*hi, hi*mid, mid*hi, hi*lo, lo*hi, mid*mid; the dropped three are below 2^-23
// together, the size of one f32 rounding) on v_mfma_f32_16x16x32_bf16 with f32 accumulation.
// Six bf16 MFMAs of 32 k take 96 cycles against 256 for the same k on
// v_mfma_f32_16x16x4_f32, so the projections keep f32 accuracy at 2.7x the f32 MFMA rate.
//
// The weights keep the packed f32 layout above: a 32-k MFMA step takes the two 16-k steps
// 2s and 2s+1, and lane (i, g) = (lane % 16, lane / 16) feeds k slots 0-3 from step 2s
// (k = 32s + 4g + e) and 4-7 from step 2s+1 (k = 32s + 16 + 4g + e) for both operands, so the
// sum runs over the same k set in a permuted slot order.  The four waves of a workgroup own
// four consecutive slabs and share the activation block: chunks of KC 32-k steps of A are
// loaded once per workgroup, split into their three bf16 terms and stored in LDS in fragment
// order (one 16-byte read per lane per term); each wave streams its slab through a register
// ring of B loads DEPTH steps ahead and splits them on use.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x8 __attribute__((ext_vector_type(8)));

// Range: the split is exact for |x| < 3.3961e38.  At or above it (and for +-inf) hi rounds to
// +-inf, the remainders become NaN and so does every product the operand enters, where the
// reference's f32 product is finite or infinite.  No model input gets there: every projection
// input leaves an RMSNorm, the attention's convex combination or SwiGLU, and the reference's own
// RMSNorm already overflows its sum of squares for |x| > 1.8e19.  Guarding it would add three
// VALU instructions per element to every weight split.
__device__ __forceinline__ void split3(const f32x8& x, bf16x8& hi, bf16x8& mid, bf16x8& lo) {
  uint4 h, m, l;
  fi::split3_pk(x[0], x[1], h.x, m.x, l.x);
  fi::split3_pk(x[2], x[3], h.y, m.y, l.y);
  fi::split3_pk(x[4], x[5], h.z, m.z, l.z);
  fi::split3_pk(x[6], x[7], h.w, m.w, l.w);
  hi = __builtin_bit_cast(bf16x8, h);
  mid = __builtin_bit_cast(bf16x8, m);
  lo = __builtin_bit_cast(bf16x8, l);
}

__device__ __forceinline__ v4f mfma_s3(const bf16x8& ah, const bf16x8& am, const bf16x8& al, const bf16x8& bh,
                                       const bf16x8& bm, const bf16x8& bl, v4f acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bm, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(am, bh, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bm, acc, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
}

template <int MT, int PW, int EPI, bool KTAIL>
__global__ __launch_bounds__(kThreads, 2) void gemm_s3_kernel(PGemmArgs g) {
  using BV = typename PVec<PW>::T;
  constexpr int KC = 2;                 // 32-k steps per staged A chunk
  constexpr int R = 2 * KC;             // B ring slots span two chunks: slot of step j of chunk c = (c % 2) KC + j
  constexpr int DEPTH = R - 1;          // B steps in flight ahead of the MFMAs
  constexpr int FRAGS = KC * MT * 64;   // A fragments (8 k of one row) per chunk
  constexpr int F_PER_T = (FRAGS + kThreads - 1) / kThreads;
  __shared__ bf16x8 s_a[2][3][FRAGS];

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int slab_id = blockIdx.x * kWaves + w;
  const int slab = min(slab_id, g.slabs - 1);  // a short last group still loads valid data
  const int m0 = blockIdx.y * 16 * MT, z = blockIdx.z;
  const int q0 = z * g.q_per_split;
  const int q1 = min(g.q_total, q0 + g.q_per_split);
  const int nsteps = (q1 - q0 + 1) / 2;  // 32-k steps; an odd last 16-k step is zero-padded
  const int nchunks = (nsteps + KC - 1) / KC;

  // fragment f = (j * MT + mt) * 64 + ln: row m0 + 16mt + ln % 16, k slots of 32-k step j of the
  // chunk for lane group ln / 16
  float4 areg[F_PER_T][2];
  auto load_a_chunk = [&](int c) {
#pragma unroll
    for (int r = 0; r < F_PER_T; ++r) {
      const int f = tid + r * kThreads;
      const int j = f / (MT * 64), mt = (f / 64) % MT, ln = f % 64;
      const int row = min(m0 + 16 * mt + (ln & 15), g.m - 1);
      const float* arow = g.a + (size_t)row * g.lda + 4 * (ln >> 4);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int q = q0 + 2 * (c * KC + j) + h;
        const float4 x = load_a<KTAIL>(arow, 16 * min(q, q1 - 1), g.k - 4 * (ln >> 4));
        const bool ok = q < q1 && f < FRAGS;
        areg[r][h] = ok ? x : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  auto store_a_chunk = [&](int buf) {
#pragma unroll
    for (int r = 0; r < F_PER_T; ++r) {
      const int f = tid + r * kThreads;
      if (FRAGS % kThreads == 0 || f < FRAGS) {
        const f32x8 x = {areg[r][0].x, areg[r][0].y, areg[r][0].z, areg[r][0].w,
                         areg[r][1].x, areg[r][1].y, areg[r][1].z, areg[r][1].w};
        bf16x8 hi, mid, lo;
        split3(x, hi, mid, lo);
        s_a[buf][0][f] = hi;
        s_a[buf][1][f] = mid;
        s_a[buf][2][f] = lo;
      }
    }
  };

  const BV* bbase = reinterpret_cast<const BV*>(g.bp) + (size_t)slab * g.q_total * 4 * 64 + lane;
  BV rb[R][2][4];
  auto issue_b = [&](int s, int slot) {  // 32-k step s of the split: 16-k steps q0 + 2s, q0 + 2s + 1
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = min(q0 + 2 * s + h, q1 - 1);  // clamped refetches hit the cache (and A is zero there)
      const BV* bq = bbase + (size_t)q * 4 * 64;
#pragma unroll
      for (int e = 0; e < 4; ++e) rb[slot][h][e] = bq[e * 64];
    }
  };

  v4f acc[MT][PW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int p = 0; p < PW; ++p) acc[mt][p] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  // one chunk: cs is the chunk's ring half (compile time)
  auto chunk = [&](int c, auto cs_tag) {
    constexpr int cs = decltype(cs_tag)::value;
    const bool more = c + 1 < nchunks;  // workgroup-uniform
    if (more) load_a_chunk(c + 1);
    const bf16x8* sa = s_a[c & 1][0];
#pragma unroll
    for (int j = 0; j < KC; ++j) {
      const int s = c * KC + j;
      issue_b(s + DEPTH, (cs * KC + j + DEPTH) % R);
      sched_fence();
      if (s < nsteps) {
#pragma unroll
        for (int p = 0; p < PW; ++p) {
          const int slot = cs * KC + j;
          const f32x8 x = {PVec<PW>::get(rb[slot][0][0], p), PVec<PW>::get(rb[slot][0][1], p),
                           PVec<PW>::get(rb[slot][0][2], p), PVec<PW>::get(rb[slot][0][3], p),
                           PVec<PW>::get(rb[slot][1][0], p), PVec<PW>::get(rb[slot][1][1], p),
                           PVec<PW>::get(rb[slot][1][2], p), PVec<PW>::get(rb[slot][1][3], p)};
          bf16x8 bh, bm, bl;
          split3(x, bh, bm, bl);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            const int f = (j * MT + mt) * 64 + lane;
            acc[mt][p] = mfma_s3(sa[f], sa[FRAGS + f], sa[2 * FRAGS + f], bh, bm, bl, acc[mt][p]);
          }
        }
      }
      sched_fence();
    }
    if (more) store_a_chunk((c + 1) & 1);
    __syncthreads();
  };

  load_a_chunk(0);
#pragma unroll
  for (int d = 0; d < DEPTH; ++d) issue_b(d, d);
  store_a_chunk(0);
  __syncthreads();
  for (int c = 0; c < nchunks; c += 2) {
    chunk(c, std::integral_constant<int, 0>{});
    if (c + 1 < nchunks) chunk(c + 1, std::integral_constant<int, 1>{});
  }
  if (slab_id < g.slabs) store_tile<MT, PW, EPI>(g, acc, m0, slab, z, lane);
}

// ---- pack width 32: the three-piece bf16 product on 32 x 32 MFMA tiles ----
//
// Packed layout (pack width 32): slabs of 32 output columns; in each 16-k step q, lane l of a
// wave holds column 32 slab + l % 32 at the eight consecutive k 16q + 8(l / 32) .. +7:
//   packed[((slab * Q + q) * 64 + l) * 8 + e] = B[16q + 8(l / 32) + e][32 slab + l % 32]
// (zero outside [0, K) x [0, N)), which is the B operand of v_mfma_f32_32x32x16_bf16 for that
// step: 32 contiguous bytes a lane.  The activations are read straight from their rows in the
// same k order (lane l: row l % 32 of a 32-row tile).  Both operands are split into their three
// bf16 pieces on use and the six cross products above 2^-24 relative accumulate in f32, as in
// gemm_s3_kernel.  A workgroup of 4 waves owns (32 MT) rows x (32 SL) columns and a range of K
// steps: each wave a contiguous quarter of it, with loads DEPTH steps ahead of the MFMAs and
// no barrier in the loop; the quarters are summed through LDS in wave order, and workgroups
// along z split K further (partials [splits, M, N], summed by the consumers in split order).
typedef float v16f __attribute__((ext_vector_type(16)));

__device__ __forceinline__ void mfma_x32(v16f& acc, const bf16x8 (&a)[3], const bf16x8 (&b)[3]) {
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[2], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[1], b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[0], b[0], acc, 0, 0, 0);
}

__device__ __forceinline__ void split3_pair(const float4& x0, const float4& x1, bf16x8 (&p)[3]) {
  const f32x8 x = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
  split3(x, p[0], p[1], p[2]);
}

template <int MT, int SL, bool KTAIL>
__global__ __launch_bounds__(kThreads, 2) void gemm_w32_kernel(PGemmArgs g) {
  constexpr int DEPTH = 2;  // steps in flight ahead of the MFMAs (3 measured slower at decode M)
  constexpr int R = DEPTH + 1;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int m0 = blockIdx.y * 32 * MT, z = blockIdx.z;
  const int q0 = z * g.q_per_split, q1 = min(g.q_total, q0 + g.q_per_split);
  const int per = (q1 - q0 + kWaves - 1) / kWaves;
  const int qb = min(q1, q0 + w * per), qe = min(q1, qb + per);
  const int kh = 8 * (lane >> 5);  // the lane's k offset within a step
  const float* arow[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int row = min(m0 + 32 * t + (lane & 31), g.m - 1);  // clamped rows are never stored
    arow[t] = g.a + (size_t)row * g.lda + kh;
  }
  const float4* wb[SL];
#pragma unroll
  for (int s = 0; s < SL; ++s) {
    const int slab = min(static_cast<int>(blockIdx.x) * SL + s, g.slabs - 1);
    wb[s] = reinterpret_cast<const float4*>(g.bp) + ((size_t)slab * g.q_total * 64 + lane) * 2;
  }
  v16f acc[MT][SL];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int s = 0; s < SL; ++s) acc[t][s] = v16f{};
  if (qb < qe) {  // wave-uniform
    float4 ra[R][MT][2], rw[R][SL][2];
    auto issue = [&](int q, int slot) {
      q = min(q, qe - 1);  // refetches past the wave's range are never multiplied
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        ra[slot][t][0] = load_a<KTAIL>(arow[t], 16 * q, g.k - kh);
        ra[slot][t][1] = load_a<KTAIL>(arow[t], 16 * q + 4, g.k - kh);
      }
#pragma unroll
      for (int s = 0; s < SL; ++s) {
        rw[slot][s][0] = wb[s][(size_t)q * 128];
        rw[slot][s][1] = wb[s][(size_t)q * 128 + 1];
      }
    };
#pragma unroll
    for (int d = 0; d < DEPTH; ++d) issue(qb + d, d);
    for (int q = qb; q < qe; q += R) {
#pragma unroll
      for (int d = 0; d < R; ++d) {
        issue(q + d + DEPTH, (d + DEPTH) % R);
        sched_fence();
        if (q + d < qe) {
          bf16x8 pa[MT][3], pw[SL][3];
#pragma unroll
          for (int t = 0; t < MT; ++t) split3_pair(ra[d][t][0], ra[d][t][1], pa[t]);
#pragma unroll
          for (int s = 0; s < SL; ++s) split3_pair(rw[d][s][0], rw[d][s][1], pw[s]);
#pragma unroll
          for (int t = 0; t < MT; ++t)
#pragma unroll
            for (int s = 0; s < SL; ++s) mfma_x32(acc[t][s], pa[t], pw[s]);
        }
        sched_fence();
      }
    }
  }
  __shared__ v16f s_part[kWaves - 1][MT * SL][64];
  if (w > 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int s = 0; s < SL; ++s) s_part[w - 1][t * SL + s][lane] = acc[t][s];
  }
  __syncthreads();
  if (w != 0) return;
#pragma unroll
  for (int src = 0; src < kWaves - 1; ++src)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int s = 0; s < SL; ++s) acc[t][s] += s_part[src][t * SL + s][lane];
  // lane l holds column l % 32 of each 32 x 32 tile, rows 8(j / 4) + 4(l / 32) + j % 4
  float* out = g.out + (size_t)z * g.m * g.n;
#pragma unroll
  for (int s = 0; s < SL; ++s) {
    const int col = (static_cast<int>(blockIdx.x) * SL + s) * 32 + (lane & 31);
    if (col >= g.n) continue;
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int row = m0 + 32 * t + 8 * (j >> 2) + 4 * (lane >> 5) + (j & 3);
        if (row < g.m) out[(size_t)row * g.n + col] = acc[t][s][j];
      }
  }
}

// Pair-pack partials [splits, M, 2N] (up, gate interleaved per column) -> out[M, N] =
// (sum up + b1) * silu(sum gate + b3), sums in split order (elementwise.rs:118-207).
// bf16 output (out_bf16): the products rounded to nearest even.
__global__ void splitk_swiglu_kernel(const float* __restrict__ parts, int splits, const float* __restrict__ b_up,
                                     const float* __restrict__ b_gate, int m, int n, void* __restrict__ out,
                                     int out_bf16) {
  const size_t total = (size_t)m * n;
  const size_t plane2 = total;  // float2 elements per split plane
  const float2* p2 = reinterpret_cast<const float2*>(parts);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    float2 x = p2[i];
    for (int z0 = 1; z0 < splits; z0 += 8) {
      float2 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p2[(size_t)(z0 + u < splits ? z0 + u : 0) * plane2 + i];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (z0 + u < splits) {
          x.x = x.x + v[u].x;
          x.y = x.y + v[u].y;
        }
    }
    const int c = static_cast<int>(i % n);
    const float up = b_up ? x.x + b_up[c] : x.x;
    float gate = b_gate ? x.y + b_gate[c] : x.y;
    gate = gate * (1.0f / (1.0f + __expf(-gate)));
    if (out_bf16)
      static_cast<uint16_t*>(out)[i] = static_cast<uint16_t>(fi::f32_to_bf16_bits(up * gate));
    else
      static_cast<float*>(out)[i] = up * gate;
  }
}

// The same for even n: two adjacent output columns a thread, their (up, gate) pairs read as
// one 16-byte vector per split.  Each value's arithmetic and order are the kernel's above.
__global__ void splitk_swiglu2_kernel(const float* __restrict__ parts, int splits, const float* __restrict__ b_up,
                                      const float* __restrict__ b_gate, int m, int n, void* __restrict__ out,
                                      int out_bf16) {
  const size_t total2 = (size_t)m * n / 2;  // column pairs = float4 elements per split plane
  const float4* p4 = reinterpret_cast<const float4*>(parts);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total2; i += (size_t)gridDim.x * blockDim.x) {
    float4 x = p4[i];
    for (int z0 = 1; z0 < splits; z0 += 8) {
      float4 v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = p4[(size_t)(z0 + u < splits ? z0 + u : 0) * total2 + i];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (z0 + u < splits) {
          x.x = x.x + v[u].x;
          x.y = x.y + v[u].y;
          x.z = x.z + v[u].z;
          x.w = x.w + v[u].w;
        }
    }
    const int c = static_cast<int>((2 * i) % n);  // even: columns c and c + 1 share the row
    const float up0 = b_up ? x.x + b_up[c] : x.x;
    const float up1 = b_up ? x.z + b_up[c + 1] : x.z;
    float g0 = b_gate ? x.y + b_gate[c] : x.y;
    float g1 = b_gate ? x.w + b_gate[c + 1] : x.w;
    g0 = g0 * (1.0f / (1.0f + __expf(-g0)));
    g1 = g1 * (1.0f / (1.0f + __expf(-g1)));
    if (out_bf16)
      static_cast<uint32_t*>(out)[i] = fi::f32_to_bf16_bits(up0 * g0) | (fi::f32_to_bf16_bits(up1 * g1) << 16);
    else
      reinterpret_cast<float2*>(out)[i] = make_float2(up0 * g0, up1 * g1);
  }
}

// Up to three source matrices; in column mode they are concatenated along N.
struct PackSources {
  const float* src[3];
  int n[3];     // columns of each source
  int count;
};

// One thread per packed float.  Column mode (pair == 0): the packed matrix is the column
// concatenation of the sources, each [K, n_i] (src_layout 0) or [n_i, K] (src_layout 1).
// Pair mode (PW = 2): source 0 supplies element p = 0 and source 1 element p = 1 of every
// lane vector, both [K, n] with n = n[0].
__global__ void weight_pack_kernel(PackSources s, int pair, int src_layout, int k, int n, int pw, int q_total,
                                   size_t total, float* __restrict__ dst) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  const int slab_cols = pair ? 16 : 16 * pw;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int p = static_cast<int>(i % pw);
    size_t r = i / pw;
    const int lane = static_cast<int>(r % 64);
    r /= 64;
    const int e = static_cast<int>(r % 4);
    r /= 4;
    const int q = static_cast<int>(r % q_total);
    const int slab = static_cast<int>(r / q_total);
    const int kk = 16 * q + 4 * (lane / 16) + e;
    const float* src = s.src[0];
    int col, ncols;
    if (pair) {
      col = slab * slab_cols + (lane % 16);
      src = s.src[p];
      ncols = s.n[0];
    } else {
      col = slab * slab_cols + pw * (lane % 16) + p;
      int j = 0;
      while (j + 1 < s.count && col >= s.n[j]) {
        col -= s.n[j];
        ++j;
      }
      src = s.src[j];
      ncols = s.n[j];
    }
    float v = 0.0f;
    if (kk < k && col < ncols) v = src_layout == 0 ? src[(size_t)kk * ncols + col] : src[(size_t)col * k + kk];
    dst[i] = v;
  }
}

// Pack width 32 (the layout of gemm_w32_kernel), one thread per packed float; in column mode
// the sources are concatenated along N as above.
__global__ void weight_pack32_kernel(PackSources s, int src_layout, int k, int q_total, size_t total,
                                     float* __restrict__ dst) {
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int e = static_cast<int>(i & 7);
    const int lane = static_cast<int>((i >> 3) & 63);
    const size_t sq = i >> 9;
    const int q = static_cast<int>(sq % q_total);
    const int slab = static_cast<int>(sq / q_total);
    const int kk = 16 * q + 8 * (lane >> 5) + e;
    int col = 32 * slab + (lane & 31);
    int j = 0;
    while (j + 1 < s.count && col >= s.n[j]) {
      col -= s.n[j];
      ++j;
    }
    const float* src = s.src[j];
    const int ncols = s.n[j];
    float v = 0.0f;
    if (kk < k && col < ncols) v = src_layout == 0 ? src[(size_t)kk * ncols + col] : src[(size_t)col * k + kk];
    dst[i] = v;
  }
}

int32_t launch_pack(fi_context* ctx, const PackSources& s, int pair, int src_layout, int k, int n, int pw,
                    float* dst) {
  size_t total = 0;
  FI_TRY(fi_weight_packed_floats(k, pair ? 2 * n : n, pw, &total));
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((total + 255) / 256, 65536));
  if (pw == kPackW32) {
    hipLaunchKernelGGL(weight_pack32_kernel, dim3(blocks), dim3(256), 0, ctx->stream, s, src_layout, k, (k + 15) / 16,
                       total, dst);
    FI_CHECK_LAUNCH("weight_pack32_kernel");
    return FI_OK;
  }
  hipLaunchKernelGGL(weight_pack_kernel, dim3(blocks), dim3(256), 0, ctx->stream, s, pair, src_layout, k, n, pw,
                     (k + 15) / 16, total, dst);
  FI_CHECK_LAUNCH("weight_pack_kernel");
  return FI_OK;
}

// ---- consumers of split-K partials ----

// sum_z parts[z * plane + i] in split order.  The loads of a batch of 8 splits are all issued
// before the first add (split counts reach 16 for skinny shapes, and a load-add chain would
// pay one memory latency per split); masked tail loads read split 0 and add exactly 0.
template <typename T>
__device__ __forceinline__ T zero_like();
template <>
__device__ __forceinline__ float zero_like<float>() { return 0.0f; }
template <>
__device__ __forceinline__ float4 zero_like<float4>() { return make_float4(0.f, 0.f, 0.f, 0.f); }
using fi::add;
using fi::put_kv4;
using fi::qkv_value4;
using fi::rope4;
using fi::sum_splits;

// One workgroup per row: h = sum_z parts[z][row] (+ bias) + residual -> sum_out; out =
// rms_norm(h) * w (reduction.rs:3-73: ms = sum(x^2)/H, inv = 1/sqrt(ms + eps), (x*inv)*w).
// Four columns per thread when hidden is a multiple of 4.
constexpr int kRowThreads = 256;
template <bool OUT16>
__global__ __launch_bounds__(kRowThreads) void splitk_residual_rms_norm_kernel(
    const float* __restrict__ parts, int splits, const float* __restrict__ bias, const float* __restrict__ residual,
    float* __restrict__ sum_out, const float* __restrict__ weight, void* __restrict__ out_v, int rows, int hidden,
    float eps) {
  __shared__ float s_red[kRowThreads / 64];
  const int row = blockIdx.x;
  const size_t plane = (size_t)rows * hidden;
  const size_t base = (size_t)row * hidden;
  float ss = 0.0f;
  const bool vec = (hidden & 3) == 0;
  // rows up to kRowQuads float4 per thread keep their sums in registers for the second pass
  // (no re-read of sum_out); wider rows loop and re-read
  constexpr int kRowQuads = 8;
  const int h4 = hidden / 4;
  const bool held = vec && h4 <= kRowQuads * kRowThreads;
  float4 xs[kRowQuads];
  float4 ws[kRowQuads];  // held rows: the norm weights, loaded with the partials (one memory round trip)
  auto sum_quad = [&](int c) {
    float4 x = sum_splits(reinterpret_cast<const float4*>(parts + base) + c, plane / 4, splits);
    if (bias) x = add(x, reinterpret_cast<const float4*>(bias)[c]);
    x = add(x, reinterpret_cast<const float4*>(residual + base)[c]);
    reinterpret_cast<float4*>(sum_out + base)[c] = x;
    ss += x.x * x.x;
    ss += x.y * x.y;
    ss += x.z * x.z;
    ss += x.w * x.w;
    return x;
  };
  if (held) {
#pragma unroll
    for (int i = 0; i < kRowQuads; ++i) {
      const int c = threadIdx.x + i * kRowThreads;
      if (c < h4) ws[i] = reinterpret_cast<const float4*>(weight)[c];
    }
#pragma unroll
    for (int i = 0; i < kRowQuads; ++i) {
      const int c = threadIdx.x + i * kRowThreads;
      if (c < h4) xs[i] = sum_quad(c);
    }
  } else if (vec) {
    for (int c = threadIdx.x; c < h4; c += kRowThreads) (void)sum_quad(c);
  } else {
    for (int c = threadIdx.x; c < hidden; c += kRowThreads) {
      float x = sum_splits(parts + base + c, plane, splits);
      if (bias) x = x + bias[c];
      x = x + residual[base + c];
      sum_out[base + c] = x;
      ss += x * x;
    }
  }
  ss = fi::wave_sum(ss);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < kRowThreads / 64; ++i) total += s_red[i];
  const float inv = 1.0f / sqrtf(total / static_cast<float>(hidden) + eps);
  // OUT16: the normalised row is stored as bf16 bits, each value rounded to nearest even
  float* out = static_cast<float*>(out_v);
  uint16_t* out16 = static_cast<uint16_t*>(out_v);
  auto norm_quad = [&](int c, const float4& x, const float4& wv) {
    const float4 y = make_float4((x.x * inv) * wv.x, (x.y * inv) * wv.y, (x.z * inv) * wv.z, (x.w * inv) * wv.w);
    if constexpr (OUT16) {
      const uint32_t b0 = fi::f32_to_bf16_bits(y.x), b1 = fi::f32_to_bf16_bits(y.y);
      const uint32_t b2 = fi::f32_to_bf16_bits(y.z), b3 = fi::f32_to_bf16_bits(y.w);
      reinterpret_cast<uint2*>(out16 + base)[c] = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
    } else {
      reinterpret_cast<float4*>(out + base)[c] = y;
    }
  };
  if (held) {
#pragma unroll
    for (int i = 0; i < kRowQuads; ++i) {
      const int c = threadIdx.x + i * kRowThreads;
      if (c < h4) norm_quad(c, xs[i], ws[i]);
    }
  } else if (vec) {
    for (int c = threadIdx.x; c < h4; c += kRowThreads)
      norm_quad(c, reinterpret_cast<const float4*>(sum_out + base)[c], reinterpret_cast<const float4*>(weight)[c]);
  } else {
    for (int c = threadIdx.x; c < hidden; c += kRowThreads) {
      const float y = (sum_out[base + c] * inv) * weight[c];
      if constexpr (OUT16)
        out16[base + c] = static_cast<uint16_t>(fi::f32_to_bf16_bits(y));
      else
        out[base + c] = y;
    }
  }
}

// The QKV projection's split partials (+ biases) -> RoPE on q and k at the token's position
// -> q to q_out, k and v appended to the pool slot (the reference order: rope before
// attention, KV written for this chunk, reference.rs:163-370).  Columns of the fused
// projection: [0, Hq*D) q, then Hkv*D of k, then Hkv*D of v.  One flat grid over (token,
// item): an item is a rotary pair (i, i + rot/2) of a q or k head, one pass-through element
// of such a head, or one value element, so every partial is read once and a decode tick of a
// few dozen tokens still spreads its loads over many workgroups.
template <typename KVT>
__device__ __forceinline__ void put_kv(KVT* cache, size_t idx, float x) {
  if constexpr (sizeof(KVT) == 4) {
    cache[idx] = x;
  } else {
    cache[idx] = static_cast<KVT>(fi::f32_to_bf16_bits(x));
  }
}


// The split-K sum of one column of the fused q|k|v partials (splits added in order) plus its
// bias, if any.
__device__ __forceinline__ float qkv_value(const float* __restrict__ p0, size_t plane, int splits,
                                           const float* __restrict__ bias, int bias_col, int col) {
  const float x = sum_splits(p0 + col, plane, splits);  // split loads batched before the adds
  return bias ? x + bias[bias_col] : x;
}

template <typename KVT>
__global__ __launch_bounds__(kRowThreads) void qkv_rope_append_kernel(
    const float* __restrict__ parts, int splits, const float* __restrict__ bias_q, const float* __restrict__ bias_k,
    const float* __restrict__ bias_v, const int* __restrict__ positions,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int rotary_dims, int max_positions,
    const int64_t* __restrict__ slots, KVT* __restrict__ k_cache, KVT* __restrict__ v_cache, int64_t pool_slots,
    int block_size, int tokens, int hq, int hkv, int d, float* __restrict__ q_out, uint32_t* __restrict__ faults) {
  const int half = rotary_dims / 2;
  const int pass = d - 2 * half;  // dimensions past the rotary ones
  const int per_head = half + pass;
  const int rot_items = (hq + hkv) * per_head;
  const int qw = hq * d, kw = hkv * d;
  const int items = rot_items + kw;
  const int gid = blockIdx.x * kRowThreads + threadIdx.x;
  const int t = gid / items;
  if (t >= tokens) return;
  const int idx = gid - t * items;
  const int width = qw + 2 * kw;
  const size_t plane = (size_t)tokens * width;
  const float* p0 = parts + (size_t)t * width;
  const int64_t slot = slots[t];
  const bool write_kv = slot >= 0 && slot < pool_slots;
  if (idx == 0 && slot >= pool_slots) atomicOr(faults, FI_FAULT_SLOT_RANGE);
  const int64_t blk = write_kv ? slot / block_size : 0;
  const int off = write_kv ? static_cast<int>(slot % block_size) : 0;
  if (idx < rot_items) {
    const int head = idx / per_head, r = idx - head * per_head;
    const bool is_q = head < hq;
    if (!is_q && !write_kv) return;
    const int col0 = is_q ? head * d : qw + (head - hq) * d;
    const float* bias = is_q ? bias_q : bias_k;
    const int bcol0 = is_q ? head * d : (head - hq) * d;
    float* qdst = q_out + (size_t)t * qw + (is_q ? head * d : 0);
    const size_t kbase = (((size_t)blk * hkv + (is_q ? 0 : head - hq)) * block_size + off) * d;
    if (r < half) {
#pragma clang fp contract(off)
      int pos = positions[t];
      if (pos < 0 || pos >= max_positions) {
        if (idx == 0) atomicOr(faults, FI_FAULT_POSITION_RANGE);
        pos = 0;
      }
      const float lo = qkv_value(p0, plane, splits, bias, bcol0 + r, col0 + r);
      const float hi = qkv_value(p0, plane, splits, bias, bcol0 + r + half, col0 + r + half);
      const float c = cos_t[(size_t)pos * half + r], sn = sin_t[(size_t)pos * half + r];
      const float y0 = lo * c - hi * sn;  // each product rounded before the add, as Rust does
      const float y1 = hi * c + lo * sn;
      if (is_q) {
        qdst[r] = y0;
        qdst[r + half] = y1;
      } else {
        put_kv(k_cache, kbase + r, y0);
        put_kv(k_cache, kbase + r + half, y1);
      }
    } else {
      const int i = 2 * half + (r - half);
      const float y = qkv_value(p0, plane, splits, bias, bcol0 + i, col0 + i);
      if (is_q) {
        qdst[i] = y;
      } else {
        put_kv(k_cache, kbase + i, y);
      }
    }
  } else if (write_kv) {
    const int v = idx - rot_items;
    const int h = v / d, i = v - h * d;
    put_kv(v_cache, (((size_t)blk * hkv + h) * block_size + off) * d + i,
           qkv_value(p0, plane, splits, bias_v, v, qw + kw + v));
  }
}

// The split-K sum of one float4 of the fused q|k|v partials (splits added in order) plus its
// bias, if any: column col of the [T, Hq*D + 2*Hkv*D] row at p0.

// Four consecutive columns per thread: the same per-element arithmetic as
// qkv_rope_append_kernel (splits summed in order, bias added, RoPE with each product rounded
// before the add) on 16-byte loads and stores.  Needs rotary_dims / 2, the pass-through width
// and D to be multiples of 4 and 16-byte aligned operands (checked by the entry point).
// Written without closures so that nothing lives in scratch memory.
template <typename KVT>
__global__ __launch_bounds__(kRowThreads) void qkv_rope_append4_kernel(
    const float* __restrict__ parts, int splits, const float* __restrict__ bias_q, const float* __restrict__ bias_k,
    const float* __restrict__ bias_v, const int* __restrict__ positions,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int rotary_dims, int max_positions,
    const int64_t* __restrict__ slots, KVT* __restrict__ k_cache, KVT* __restrict__ v_cache, int64_t pool_slots,
    int block_size, int tokens, int hq, int hkv, int d, float* __restrict__ q_out, uint32_t* __restrict__ faults) {
  const int half = rotary_dims / 2;
  const int pass = d - 2 * half;
  const int quads_per_head = (half + pass) / 4;
  const int rot_items = (hq + hkv) * quads_per_head;
  const int qw = hq * d, kw = hkv * d;
  const int items = rot_items + kw / 4;
  const int gid = blockIdx.x * kRowThreads + threadIdx.x;
  const int t = gid / items;
  if (t >= tokens) return;
  const int idx = gid - t * items;
  const int width = qw + 2 * kw;
  const size_t plane = (size_t)tokens * width;
  const float* p0 = parts + (size_t)t * width;
  const int64_t slot = slots[t];
  const bool write_kv = slot >= 0 && slot < pool_slots;
  if (idx == 0 && slot >= pool_slots) atomicOr(faults, FI_FAULT_SLOT_RANGE);
  const int64_t blk = write_kv ? slot / block_size : 0;
  const int off = write_kv ? static_cast<int>(slot % block_size) : 0;
  if (idx < rot_items) {
    const int head = idx / quads_per_head, r = 4 * (idx - head * quads_per_head);
    const bool is_q = head < hq;
    const int col0 = is_q ? head * d : qw + (head - hq) * d;
    const float* bias = is_q ? bias_q : bias_k;
    const int bcol0 = is_q ? head * d : (head - hq) * d;
    // destination of this head's row: q_out, or the K pool row of the token's slot
    float* qdst = q_out + (size_t)t * qw + (is_q ? head * d : 0);
    const size_t kbase = (((size_t)blk * hkv + (is_q ? 0 : head - hq)) * block_size + off) * d;
    if (!is_q && !write_kv) return;
    if (r < half) {
#pragma clang fp contract(off)
      int pos = positions[t];
      if (pos < 0 || pos >= max_positions) {
        if (idx == 0) atomicOr(faults, FI_FAULT_POSITION_RANGE);
        pos = 0;
      }
      const float4 lo = qkv_value4(p0, plane, splits, bias, bcol0 + r, col0 + r);
      const float4 hi = qkv_value4(p0, plane, splits, bias, bcol0 + r + half, col0 + r + half);
      const float4 c = *reinterpret_cast<const float4*>(cos_t + (size_t)pos * half + r);
      const float4 sn = *reinterpret_cast<const float4*>(sin_t + (size_t)pos * half + r);
      float4 y0, y1;
      rope4(lo, hi, c, sn, y0, y1);
      if (is_q) {
        *reinterpret_cast<float4*>(qdst + r) = y0;
        *reinterpret_cast<float4*>(qdst + r + half) = y1;
      } else {
        put_kv4(k_cache, kbase + r, y0);
        put_kv4(k_cache, kbase + r + half, y1);
      }
    } else {
      const int i = 2 * half + (r - half);
      const float4 y = qkv_value4(p0, plane, splits, bias, bcol0 + i, col0 + i);
      if (is_q) {
        *reinterpret_cast<float4*>(qdst + i) = y;
      } else {
        put_kv4(k_cache, kbase + i, y);
      }
    }
  } else if (write_kv) {
    const int v = 4 * (idx - rot_items);
    const int h = v / d, i = v - h * d;
    const float4 x = qkv_value4(p0, plane, splits, bias_v, v, qw + kw + v);
    put_kv4(v_cache, (((size_t)blk * hkv + h) * block_size + off) * d + i, x);
  }
}

int32_t q_steps(int32_t k) { return (k + 15) / 16; }

// Pack width of the greedy head's weight: width 2 runs on the shared-activation kernel (four
// slabs read one staged activation block), 12 % faster than width 4 at 64 rows, equal at one.
constexpr int kLmHeadPack = 2;

int32_t slabs_of(int32_t n, int32_t pw, bool pair) {
  const int32_t cols = pair ? 16 : (pw == kPackW32 ? 32 : 16 * pw);
  return (n + cols - 1) / cols;
}

// Row-block height for M rows: 16, 32 or 64.
int mtiles_for(int m) { return m <= 16 ? 1 : (m <= 32 ? 2 : 4); }

// Kernel choice for a launch shape.  The shared-activation kernel (4 slabs per workgroup,
// activations read once per workgroup) wins whenever there are enough slab groups to fill the
// device; narrow weights at decode M keep one slab per workgroup (4 waves splitting K), which
// has 4x the workgroups.  Pack width 4 tiles are too register-heavy for the shared variant.
struct Plan {
  bool shared;
  int mt;
  int mblocks;
  int blocks;  // workgroups per split
};

Plan plan_for(int m, int slabs, int pw) {
  Plan p{};
  p.mt = mtiles_for(m);
  p.mblocks = (m + 16 * p.mt - 1) / (16 * p.mt);
  const int groups = (slabs + kWaves - 1) / kWaves;
  p.shared = pw <= 2 && groups * p.mblocks >= 64;
  p.blocks = (p.shared ? groups : slabs) * p.mblocks;
  return p;
}

// Split count: enough workgroups to give every CU two, every split at least 8 (shared) or
// 16 (per-wave quarters) K steps, and the partials (splits x M x N floats) at most a quarter
// of the weight bytes (K x N floats) for M >= 16.
int split_count(fi_context* ctx, int m, int k, int slabs, int pw) {
  const Plan p = plan_for(m, slabs, pw);
  const int q = q_steps(k);
  const long target = 2L * (ctx->compute_units > 0 ? ctx->compute_units : 256);
  long s = std::max(1L, (target + p.blocks - 1) / p.blocks);
  s = std::min(s, std::max(1L, static_cast<long>(q / (p.shared ? 8 : 16))));
  s = std::min(s, std::max(1L, static_cast<long>(k) / (4L * std::max(m, 16))));
  s = std::min(s, 16L);
  const int per = (q + static_cast<int>(s) - 1) / static_cast<int>(s);
  return (q + per - 1) / per;  // every split non-empty
}

// Pack width 32: 32-row tiles (one for M <= 32, else two per workgroup), and two slabs per
// workgroup once that still gives half the CUs a workgroup (prefill M); at decode M one slab,
// with K split until the grid is one workgroup per CU, every split at least 8 steps.  Timed on
// the box at the C4 shapes against the f32-MFMA kernels: M = 64 q|k|v 8.3 -> 6.7 us (7
// splits), wo 8.3 -> 6.5 us (7), w2 12.2 -> 11.1 us (9); M = 1024 (one split, two slabs) q|k|v
// 41.8 -> 31.3 us, wo 24.8 -> 19.9 us, w2 83.9 -> 74.0 us.
struct W32Plan {
  int mt, sl, mblocks, blocks;
};

W32Plan w32_plan(fi_context* ctx, int m, int slabs) {
  W32Plan p{};
  p.mt = m <= 32 ? 1 : 2;
  p.mblocks = (m + 32 * p.mt - 1) / (32 * p.mt);
  const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  p.sl = static_cast<long>((slabs + 1) / 2) * p.mblocks >= cus / 2 ? 2 : 1;
  p.blocks = ((slabs + p.sl - 1) / p.sl) * p.mblocks;
  return p;
}

int w32_split_count(fi_context* ctx, int m, int k, int slabs) {
  const W32Plan p = w32_plan(ctx, m, slabs);
  const int q = q_steps(k);
  const long cus = ctx->compute_units > 0 ? ctx->compute_units : 256;
  long s = std::max(1L, std::min(cus / p.blocks, static_cast<long>(q / 8)));
  s = std::min(s, 32L);
  const int per = (q + static_cast<int>(s) - 1) / static_cast<int>(s);
  return (q + per - 1) / per;  // every split non-empty
}

template <int MT, int SL>
void launch_w32_tail(fi_context* ctx, const PGemmArgs& g, dim3 grid) {
  if (g.k % 16 != 0)
    hipLaunchKernelGGL((gemm_w32_kernel<MT, SL, true>), grid, dim3(kThreads), 0, ctx->stream, g);
  else
    hipLaunchKernelGGL((gemm_w32_kernel<MT, SL, false>), grid, dim3(kThreads), 0, ctx->stream, g);
}

int32_t launch_w32(fi_context* ctx, const PGemmArgs& g, int splits) {
  const W32Plan p = w32_plan(ctx, g.m, g.slabs);
  const dim3 grid(static_cast<unsigned>((g.slabs + p.sl - 1) / p.sl), static_cast<unsigned>(p.mblocks),
                  static_cast<unsigned>(splits));
  if (p.mt == 1)
    p.sl == 1 ? launch_w32_tail<1, 1>(ctx, g, grid) : launch_w32_tail<1, 2>(ctx, g, grid);
  else
    p.sl == 1 ? launch_w32_tail<2, 1>(ctx, g, grid) : launch_w32_tail<2, 2>(ctx, g, grid);
  FI_CHECK_LAUNCH("gemm_w32_kernel");
  return FI_OK;
}

template <int MT, int PW, int EPI, bool KTAIL>
void launch_one(fi_context* ctx, const PGemmArgs& g, const Plan& p, unsigned splits) {
  if constexpr (PW <= 2) {
    if (p.shared) {
      dim3 grid(static_cast<unsigned>((g.slabs + kWaves - 1) / kWaves), p.mblocks, splits);
      // The three-term kernel wins on two-column slabs with full 64-row tiles (w1|w3 at M 1024:
      // 180 -> 132 us; the 64-row greedy head: 209 -> 184 us); on one-column slabs and short tiles
      // its per-step splitting costs as much as it saves.
      if constexpr (PW == 2 && MT == 4)
        hipLaunchKernelGGL((gemm_s3_kernel<MT, PW, EPI, KTAIL>), grid, dim3(kThreads), 0, ctx->stream, g);
      else
        hipLaunchKernelGGL((gemm_lds_kernel<MT, PW, EPI, KTAIL>), grid, dim3(kThreads), 0, ctx->stream, g);
      return;
    }
  }
  dim3 grid(static_cast<unsigned>(g.slabs), p.mblocks, splits);
  hipLaunchKernelGGL((gemm_packed_kernel<MT, PW, EPI, KTAIL>), grid, dim3(kThreads), 0, ctx->stream, g);
}

template <int PW, int EPI>
int32_t launch_pgemm(fi_context* ctx, const PGemmArgs& g, int splits) {
  const Plan p = plan_for(g.m, g.slabs, PW);
  const unsigned sp = static_cast<unsigned>(splits);
  const bool tail = g.k % 16 != 0;
  switch (p.mt * 2 + (tail ? 1 : 0)) {
    case 2:
      launch_one<1, PW, EPI, false>(ctx, g, p, sp);
      break;
    case 3:
      launch_one<1, PW, EPI, true>(ctx, g, p, sp);
      break;
    case 4:
      launch_one<2, PW, EPI, false>(ctx, g, p, sp);
      break;
    case 5:
      launch_one<2, PW, EPI, true>(ctx, g, p, sp);
      break;
    case 8:
      launch_one<4, PW, EPI, false>(ctx, g, p, sp);
      break;
    default:
      launch_one<4, PW, EPI, true>(ctx, g, p, sp);
      break;
  }
  FI_CHECK_LAUNCH("gemm_packed_kernel");
  return FI_OK;
}

int32_t check_common(fi_context* ctx, const float* a, int32_t lda, const float* bp, int32_t m, int32_t k, int32_t n) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(m >= 0 && k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "packed gemm: k and n must be positive");
  FI_REQUIRE(lda >= k && lda % 4 == 0, FI_ERR_INVALID_LAYOUT, "packed gemm: lda must be >= k and a multiple of 4");
  FI_REQUIRE(m == 0 || (a && bp), FI_ERR_INVALID_CONFIG, "packed gemm: null pointer");
  FI_REQUIRE((reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(bp) & 15) == 0,
             FI_ERR_INVALID_LAYOUT, "packed gemm: operands must be 16-byte aligned");
  return FI_OK;
}

}  // namespace

namespace fi {

int32_t splitk_swiglu(fi_context* ctx, const float* parts, int32_t splits, const float* bias_up,
                      const float* bias_gate, int32_t m, int32_t n, void* out, bool out_bf16) {
  const size_t total = (size_t)m * n;
  const bool pairs = n % 2 == 0 && (reinterpret_cast<uintptr_t>(parts) & 15) == 0 &&
                     (reinterpret_cast<uintptr_t>(out) & (out_bf16 ? 3 : 7)) == 0;
  if (pairs) {
    const unsigned blocks = static_cast<unsigned>(std::min<size_t>((total / 2 + 255) / 256, 4096));
    hipLaunchKernelGGL(splitk_swiglu2_kernel, dim3(blocks), dim3(256), 0, ctx->stream, parts, splits, bias_up,
                       bias_gate, m, n, out, out_bf16 ? 1 : 0);
    FI_CHECK_LAUNCH("splitk_swiglu2_kernel");
    return FI_OK;
  }
  const unsigned blocks = static_cast<unsigned>(std::min<size_t>((total + 255) / 256, 4096));
  hipLaunchKernelGGL(splitk_swiglu_kernel, dim3(blocks), dim3(256), 0, ctx->stream, parts, splits, bias_up, bias_gate,
                     m, n, out, out_bf16 ? 1 : 0);
  FI_CHECK_LAUNCH("splitk_swiglu_kernel");
  return FI_OK;
}

}  // namespace fi

extern "C" {

int32_t fi_weight_packed_floats(int32_t k, int32_t n, int32_t pack_width, size_t* floats) {
  FI_REQUIRE(k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_weight_packed_floats: k and n must be positive");
  FI_REQUIRE(pack_width == 1 || pack_width == 2 || pack_width == 4 || pack_width == kPackW32, FI_ERR_INVALID_CONFIG,
             "fi_weight_packed_floats: pack width must be 1, 2, 4 or 32");
  FI_REQUIRE(floats != nullptr, FI_ERR_INVALID_CONFIG, "fi_weight_packed_floats: null output");
  const size_t per_step = pack_width == kPackW32 ? 64 * 8 : 4 * 64 * pack_width;  // floats per slab and 16-k step
  *floats = static_cast<size_t>(slabs_of(n, pack_width, false)) * q_steps(k) * per_step;
  return FI_OK;
}

int32_t fi_weight_pack(fi_context* ctx, const float* d_src, int32_t src_layout, int32_t k, int32_t n,
                       int32_t pack_width, float* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(src_layout == 0 || src_layout == 1, FI_ERR_INVALID_LAYOUT, "fi_weight_pack: src_layout must be 0 or 1");
  size_t total = 0;
  FI_TRY(fi_weight_packed_floats(k, n, pack_width, &total));
  FI_REQUIRE(d_src && d_dst, FI_ERR_INVALID_CONFIG, "fi_weight_pack: null pointer");
  PackSources s{{d_src, nullptr, nullptr}, {n, 0, 0}, 1};
  return launch_pack(ctx, s, 0, src_layout, k, n, pack_width, d_dst);
}

int32_t fi_weight_pack_columns(fi_context* ctx, const float* const* d_srcs, const int32_t* ns, int32_t count,
                               int32_t k, int32_t pack_width, float* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(count >= 1 && count <= 3, FI_ERR_INVALID_CONFIG, "fi_weight_pack_columns: 1 to 3 sources");
  FI_REQUIRE(d_srcs && ns && d_dst, FI_ERR_INVALID_CONFIG, "fi_weight_pack_columns: null pointer");
  PackSources s{{nullptr, nullptr, nullptr}, {0, 0, 0}, count};
  int32_t n = 0;
  for (int i = 0; i < count; ++i) {
    FI_REQUIRE(d_srcs[i] && ns[i] > 0, FI_ERR_INVALID_CONFIG, "fi_weight_pack_columns: empty source");
    s.src[i] = d_srcs[i];
    s.n[i] = ns[i];
    n += ns[i];
  }
  return launch_pack(ctx, s, 0, 0, k, n, pack_width, d_dst);
}

int32_t fi_weight_pack_pair(fi_context* ctx, const float* d_first, const float* d_second, int32_t k, int32_t n,
                            float* d_dst) {
  FI_TRY(fi::enter(ctx));
  size_t total = 0;
  FI_TRY(fi_weight_packed_floats(k, 2 * n, 2, &total));
  FI_REQUIRE(d_first && d_second && d_dst, FI_ERR_INVALID_CONFIG, "fi_weight_pack_pair: null pointer");
  PackSources s{{d_first, d_second, nullptr}, {n, n, 0}, 2};
  return launch_pack(ctx, s, 1, 0, k, n, 2, d_dst);
}

int32_t fi_gemm_packed_splits(fi_context* ctx, int32_t m, int32_t k, int32_t n, int32_t pack_width,
                              int32_t* splits) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(m >= 0 && k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_gemm_packed_splits: bad shape");
  FI_REQUIRE(pack_width == 1 || pack_width == 2 || pack_width == 4 || pack_width == kPackW32, FI_ERR_INVALID_CONFIG,
             "fi_gemm_packed_splits: pack width must be 1, 2, 4 or 32");
  FI_REQUIRE(splits != nullptr, FI_ERR_INVALID_CONFIG, "fi_gemm_packed_splits: null output");
  const int slabs = slabs_of(n, pack_width, false);
  *splits = pack_width == kPackW32 ? w32_split_count(ctx, m, k, slabs) : split_count(ctx, m, k, slabs, pack_width);
  return FI_OK;
}

int32_t fi_gemm_packed(fi_context* ctx, const float* d_a, int32_t lda, const float* d_bp, int32_t k, int32_t n,
                       int32_t pack_width, int32_t m, int32_t splits, float* d_out) {
  FI_TRY(check_common(ctx, d_a, lda, d_bp, m, k, n));
  FI_REQUIRE(pack_width == 1 || pack_width == 2 || pack_width == 4 || pack_width == kPackW32, FI_ERR_INVALID_CONFIG,
             "fi_gemm_packed: pack width must be 1, 2, 4 or 32");
  FI_REQUIRE(splits >= 1 && splits <= q_steps(k), FI_ERR_INVALID_CONFIG, "fi_gemm_packed: splits out of range");
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_gemm_packed: null output");
  PGemmArgs g{};
  g.a = d_a;
  g.bp = d_bp;
  g.out = d_out;
  g.m = m;
  g.k = k;
  g.n = n;
  g.lda = lda;
  g.q_total = q_steps(k);
  g.q_per_split = (g.q_total + splits - 1) / splits;
  g.slabs = slabs_of(n, pack_width, false);
  const int used = (g.q_total + g.q_per_split - 1) / g.q_per_split;
  FI_REQUIRE(used == splits, FI_ERR_INVALID_CONFIG,
             "fi_gemm_packed: splits must divide the K steps into non-empty ranges (use fi_gemm_packed_splits)");
  switch (pack_width) {
    case kPackW32:
      return launch_w32(ctx, g, splits);
    case 1:
      return launch_pgemm<1, kEpiPartial>(ctx, g, splits);
    case 2:
      return launch_pgemm<2, kEpiPartial>(ctx, g, splits);
    default:
      return launch_pgemm<4, kEpiPartial>(ctx, g, splits);
  }
}

int32_t fi_gemm_packed_swiglu(fi_context* ctx, const float* d_a, int32_t lda, const float* d_bp_pair, int32_t k,
                              int32_t n, int32_t m, const float* d_bias_up, const float* d_bias_gate, float* d_out) {
  FI_TRY(check_common(ctx, d_a, lda, d_bp_pair, m, k, n));
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_out != nullptr, FI_ERR_INVALID_CONFIG, "fi_gemm_packed_swiglu: null output");
  PGemmArgs g{};
  g.a = d_a;
  g.bp = d_bp_pair;
  g.bias0 = d_bias_up;
  g.bias1 = d_bias_gate;
  g.m = m;
  g.k = k;
  g.lda = lda;
  g.q_total = q_steps(k);
  g.slabs = slabs_of(n, 2, true);
  const int splits = split_count(ctx, m, k, g.slabs, 2);
  if (splits == 1) {  // the epilogue applies SwiGLU directly
    g.out = d_out;
    g.n = n;
    g.q_per_split = g.q_total;
    return launch_pgemm<2, kEpiSwiglu>(ctx, g, 1);
  }
  // partial (up, gate) pairs per split, then the split sum + SwiGLU
  FI_TRY(fi::ensure_workspace(ctx, (size_t)splits * m * 2 * n * sizeof(float)));
  g.out = static_cast<float*>(ctx->workspace);
  g.n = 2 * n;
  g.q_per_split = (g.q_total + splits - 1) / splits;
  FI_TRY((launch_pgemm<2, kEpiPartial>(ctx, g, splits)));
  return fi::splitk_swiglu(ctx, g.out, splits, d_bias_up, d_bias_gate, m, n, d_out, false);
}

int32_t fi_lm_head_argmax_packed(fi_context* ctx, const float* d_hidden, int32_t lda, const float* d_bp, int32_t m,
                                 int32_t hidden, int32_t vocab, int32_t* d_token, float* d_prob) {
  FI_TRY(check_common(ctx, d_hidden, lda, d_bp, m, hidden, vocab));
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_token && d_prob, FI_ERR_INVALID_CONFIG, "fi_lm_head_argmax_packed: null output");
  PGemmArgs g{};
  g.a = d_hidden;
  g.bp = d_bp;
  g.m = m;
  g.k = hidden;
  g.n = vocab;
  g.lda = lda;
  g.q_total = q_steps(hidden);
  g.q_per_split = g.q_total;
  g.slabs = slabs_of(vocab, kLmHeadPack, false);
  FI_TRY(fi::ensure_workspace(ctx, (size_t)m * g.slabs * 3 * sizeof(float)));
  g.out = static_cast<float*>(ctx->workspace);
  FI_TRY((launch_pgemm<kLmHeadPack, kEpiArgmax>(ctx, g, 1)));
  return fi::argmax_merge(ctx, g.out, g.slabs, m, d_token, d_prob);
}

int32_t fi_splitk_residual_rms_norm(fi_context* ctx, const float* d_parts, int32_t splits, const float* d_bias,
                                    const float* d_residual, float* d_sum, const float* d_weight, float* d_out,
                                    int32_t rows, int32_t hidden, float eps) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(rows >= 0 && hidden > 0 && splits >= 1, FI_ERR_INVALID_SHAPE, "fi_splitk_residual_rms_norm: bad shape");
  if (rows == 0) return FI_OK;
  FI_REQUIRE(d_parts && d_residual && d_sum && d_weight && d_out, FI_ERR_INVALID_CONFIG,
             "fi_splitk_residual_rms_norm: null pointer");
  hipLaunchKernelGGL(splitk_residual_rms_norm_kernel<false>, dim3(rows), dim3(kRowThreads), 0, ctx->stream, d_parts,
                     splits, d_bias, d_residual, d_sum, d_weight, d_out, rows, hidden, eps);
  FI_CHECK_LAUNCH("splitk_residual_rms_norm_kernel");
  return FI_OK;
}

int32_t fi_splitk_residual_rms_norm_bf16(fi_context* ctx, const float* d_parts, int32_t splits, const float* d_bias,
                                         const float* d_residual, float* d_sum, const float* d_weight,
                                         uint16_t* d_out, int32_t rows, int32_t hidden, float eps) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(rows >= 0 && hidden > 0 && splits >= 1, FI_ERR_INVALID_SHAPE,
             "fi_splitk_residual_rms_norm_bf16: bad shape");
  if (rows == 0) return FI_OK;
  FI_REQUIRE(d_parts && d_residual && d_sum && d_weight && d_out, FI_ERR_INVALID_CONFIG,
             "fi_splitk_residual_rms_norm_bf16: null pointer");
  FI_REQUIRE(hidden % 4 != 0 || reinterpret_cast<uintptr_t>(d_out) % 8 == 0, FI_ERR_INVALID_LAYOUT,
             "fi_splitk_residual_rms_norm_bf16: the output must be 8-byte aligned");
  hipLaunchKernelGGL(splitk_residual_rms_norm_kernel<true>, dim3(rows), dim3(kRowThreads), 0, ctx->stream, d_parts,
                     splits, d_bias, d_residual, d_sum, d_weight, d_out, rows, hidden, eps);
  FI_CHECK_LAUNCH("splitk_residual_rms_norm_kernel");
  return FI_OK;
}

int32_t fi_qkv_rope_append(fi_context* ctx, const float* d_parts, int32_t splits, const float* d_bias_q,
                           const float* d_bias_k, const float* d_bias_v,
                           const int32_t* d_positions, const float* d_cos, const float* d_sin, int32_t rotary_dims,
                           int32_t max_positions, const int64_t* d_slot_mapping, void* d_k_cache, void* d_v_cache,
                           int32_t kv_dtype, int32_t num_blocks, int32_t block_size, int32_t num_tokens,
                           int32_t num_q_heads, int32_t num_kv_heads, int32_t head_dim, float* d_q_out) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(num_tokens >= 0 && splits >= 1, FI_ERR_INVALID_SHAPE, "fi_qkv_rope_append: bad shape");
  FI_REQUIRE(num_q_heads > 0 && num_kv_heads > 0 && head_dim > 0 && num_q_heads % num_kv_heads == 0,
             FI_ERR_INVALID_SHAPE, "number of query heads must be divisible by number of KV heads");
  FI_REQUIRE(rotary_dims >= 0 && rotary_dims <= head_dim && rotary_dims % 2 == 0, FI_ERR_INVALID_CONFIG,
             "rope.rotary_dims must be even and at most the head dimension");
  FI_REQUIRE(num_blocks > 0 && block_size > 0, FI_ERR_INVALID_CONFIG, "fi_qkv_rope_append: pool dimensions must be positive");
  FI_REQUIRE(kv_dtype == FI_DTYPE_F32 || kv_dtype == FI_DTYPE_BF16, FI_ERR_INVALID_TYPE,
             "fi_qkv_rope_append: KV dtype must be f32 or bf16");
  if (num_tokens == 0) return FI_OK;
  FI_REQUIRE(d_parts && d_positions && d_slot_mapping && d_k_cache && d_v_cache && d_q_out, FI_ERR_INVALID_CONFIG,
             "fi_qkv_rope_append: null pointer");
  FI_REQUIRE(rotary_dims == 0 || (d_cos && d_sin && max_positions > 0), FI_ERR_INVALID_CONFIG,
             "fi_qkv_rope_append: rope tables required");
  const int64_t pool_slots = static_cast<int64_t>(num_blocks) * block_size;
  auto aligned16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int32_t half = rotary_dims / 2, pass = head_dim - 2 * half;
  const bool vec4 = half % 4 == 0 && pass % 4 == 0 && head_dim % 4 == 0 && aligned16(d_parts) && aligned16(d_q_out) &&
                    (!d_bias_q || aligned16(d_bias_q)) && (!d_bias_k || aligned16(d_bias_k)) &&
                    (!d_bias_v || aligned16(d_bias_v)) && (rotary_dims == 0 || (aligned16(d_cos) && aligned16(d_sin)));
  const int64_t items = static_cast<int64_t>(num_q_heads + num_kv_heads) * (head_dim - rotary_dims / 2) +
                        static_cast<int64_t>(num_kv_heads) * head_dim;
  const int64_t launch_items = vec4 ? items / 4 : items;
  FI_REQUIRE(launch_items * num_tokens < 0x7fffffffLL - kRowThreads, FI_ERR_INVALID_SHAPE,
             "fi_qkv_rope_append: too many tokens for one launch");
  const dim3 grid(static_cast<unsigned>((launch_items * num_tokens + kRowThreads - 1) / kRowThreads));
  if (kv_dtype == FI_DTYPE_F32) {
    if (vec4) {
      hipLaunchKernelGGL(qkv_rope_append4_kernel<float>, grid, dim3(kRowThreads), 0, ctx->stream, d_parts, splits,
                         d_bias_q, d_bias_k, d_bias_v, d_positions, d_cos, d_sin, rotary_dims, max_positions,
                         d_slot_mapping, static_cast<float*>(d_k_cache), static_cast<float*>(d_v_cache), pool_slots,
                         block_size, num_tokens, num_q_heads, num_kv_heads, head_dim, d_q_out, ctx->d_faults);
    } else {
      hipLaunchKernelGGL(qkv_rope_append_kernel<float>, grid, dim3(kRowThreads), 0, ctx->stream, d_parts, splits,
                         d_bias_q, d_bias_k, d_bias_v, d_positions, d_cos, d_sin, rotary_dims, max_positions,
                         d_slot_mapping, static_cast<float*>(d_k_cache), static_cast<float*>(d_v_cache), pool_slots,
                         block_size, num_tokens, num_q_heads, num_kv_heads, head_dim, d_q_out, ctx->d_faults);
    }
  } else if (vec4) {
    hipLaunchKernelGGL(qkv_rope_append4_kernel<uint16_t>, grid, dim3(kRowThreads), 0, ctx->stream, d_parts, splits,
                       d_bias_q, d_bias_k, d_bias_v, d_positions, d_cos, d_sin, rotary_dims, max_positions,
                       d_slot_mapping, static_cast<uint16_t*>(d_k_cache), static_cast<uint16_t*>(d_v_cache),
                       pool_slots, block_size, num_tokens, num_q_heads, num_kv_heads, head_dim, d_q_out,
                       ctx->d_faults);
  } else {
    hipLaunchKernelGGL(qkv_rope_append_kernel<uint16_t>, grid, dim3(kRowThreads), 0, ctx->stream, d_parts, splits,
                       d_bias_q, d_bias_k, d_bias_v, d_positions, d_cos, d_sin, rotary_dims, max_positions,
                       d_slot_mapping, static_cast<uint16_t*>(d_k_cache), static_cast<uint16_t*>(d_v_cache),
                       pool_slots, block_size, num_tokens, num_q_heads, num_kv_heads, head_dim, d_q_out,
                       ctx->d_faults);
  }
  FI_CHECK_LAUNCH("qkv_rope_append_kernel");
  return FI_OK;
}

}  // extern "C"
