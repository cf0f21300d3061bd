// Projection GEMMs on MFMA (v_mfma_f32_16x16x4_f32) for gfx950, plus the fused lm_head
// argmax.  Replaces matmul_f32 / linear_f32_with_bias (kernel/cpu/matmul.rs:46-118,
// runtime/reference.rs:1103-1191), matmul_rhs_transposed_f32 (matmul.rs:120-188) and
// matmul_rhs_transposed_argmax_f32 (matmul.rs:190-274, 532-589).
//
// C[M,N] = A[M,K] * B (+ bias[N]).  B is either the reference's weight layout [K,N]
// ("[in, out]", model/decoder.rs:76-104) or [N,K] (the tied embedding / output weight used
// by lm_head).  Workgroup tile 64x64x16, 4 waves each owning a 32x32 quadrant as 2x2 MFMA
// 16x16 tiles; A is staged transposed in LDS so MFMA operand reads are conflict-free; the
// next K tile is fetched into registers while the current one is multiplied.  Skinny
// decode shapes split K across workgroups; partial tiles are summed by a second kernel in a
// fixed order, so results are deterministic.
#include <algorithm>
#include <limits>

#include "fi_common.h"
#include "fi_device.h"

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BM = 64;
constexpr int BN = 64;
constexpr int BK = 16;  // K depth per LDS stage (deeper stages measured slower at every shape)
constexpr int kGemmThreads = 256;

enum Epilogue : int { kStore = 0, kPartial = 1, kArgmax = 2 };

struct GemmArgs {
  const float* a;     // [M, K]
  const float* b;     // [K, N] or [N, K]
  const float* bias;  // [N] or null
  float* c;           // [M, N] (kStore) or [splits, M, N] (kPartial)
  float* amax;        // kArgmax: per (row, n-tile) {max, index bits, sum}
  int m, k, n;
  int k_chunk;        // K range per split (multiple of the stage depth)
  int n_tiles;
};

// Each thread moves QPT = BKT / 16 float4 quads of A and of B per K stage (64 x BKT each).
// A [M, K]: quad q -> (row q / (BKT/4), k quad q % (BKT/4)), consecutive threads read
// consecutive quads of a row.
template <bool TRANS_B, int BKT>
__device__ __forceinline__ void load_tiles(const GemmArgs& g, int m0, int n0, int k0, int kend,
                                           float4 (&ra)[BKT / 16], float4 (&rb)[BKT / 16]) {
  constexpr int KQ = BKT / 4;  // quads per K row of a tile
  const bool kvec = (g.k & 3) == 0;
#pragma unroll
  for (int r = 0; r < BKT / 16; ++r) {
    const int q = threadIdx.x + r * kGemmThreads;
    const int row = m0 + q / KQ, kk = k0 + (q % KQ) * 4;
    if (row < g.m && kk + 3 < kend && kvec) {
      ra[r] = *reinterpret_cast<const float4*>(g.a + (size_t)row * g.k + kk);
    } else {
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (row < g.m && kk + i < kend) ? g.a[(size_t)row * g.k + kk + i] : 0.0f;
      ra[r] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
#pragma unroll
  for (int r = 0; r < BKT / 16; ++r) {
    const int q = threadIdx.x + r * kGemmThreads;
    if constexpr (!TRANS_B) {
      // B [K, N]: quad q -> (k row q / 16, n quad q % 16)
      const int kr = k0 + q / 16, col = n0 + (q % 16) * 4;
      if (kr < kend && col + 3 < g.n && ((g.n & 3) == 0)) {
        rb[r] = *reinterpret_cast<const float4*>(g.b + (size_t)kr * g.n + col);
      } else {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (kr < kend && col + i < g.n) ? g.b[(size_t)kr * g.n + col + i] : 0.0f;
        rb[r] = make_float4(v[0], v[1], v[2], v[3]);
      }
    } else {
      // B [N, K]: quad q -> (n row q / (BKT/4), k quad q % (BKT/4))
      const int col = n0 + q / KQ, kk = k0 + (q % KQ) * 4;
      if (col < g.n && kk + 3 < kend && kvec) {
        rb[r] = *reinterpret_cast<const float4*>(g.b + (size_t)col * g.k + kk);
      } else {
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (col < g.n && kk + i < kend) ? g.b[(size_t)col * g.k + kk + i] : 0.0f;
        rb[r] = make_float4(v[0], v[1], v[2], v[3]);
      }
    }
  }
}

template <bool TRANS_B, int BKT>
__device__ __forceinline__ void store_tiles(float (*As)[BM + 4], float (*Bs)[BN + 4], const float4 (&ra)[BKT / 16],
                                            const float4 (&rb)[BKT / 16]) {
  constexpr int KQ = BKT / 4;
#pragma unroll
  for (int r = 0; r < BKT / 16; ++r) {
    const int q = threadIdx.x + r * kGemmThreads;
    {
      const int row = q / KQ, kq = (q % KQ) * 4;
      As[kq + 0][row] = ra[r].x;
      As[kq + 1][row] = ra[r].y;
      As[kq + 2][row] = ra[r].z;
      As[kq + 3][row] = ra[r].w;
    }
    if constexpr (!TRANS_B) {
      const int kr = q / 16, col = (q % 16) * 4;
      *reinterpret_cast<float4*>(&Bs[kr][col]) = rb[r];
    } else {
      const int col = q / KQ, kq = (q % KQ) * 4;
      Bs[kq + 0][col] = rb[r].x;
      Bs[kq + 1][col] = rb[r].y;
      Bs[kq + 2][col] = rb[r].z;
      Bs[kq + 3][col] = rb[r].w;
    }
  }
}

// BKT = K depth of one LDS stage.
template <bool TRANS_B, int EPI, int BKT>
__global__ __launch_bounds__(kGemmThreads) void gemm_kernel(GemmArgs g) {
  __shared__ float As[2][BKT][BM + 4];
  __shared__ float Bs[2][BKT][BN + 4];
  const int n_tile = blockIdx.x, m_tile = blockIdx.y, split = blockIdx.z;
  const int m0 = m_tile * BM, n0 = n_tile * BN;
  const int kbeg = split * g.k_chunk;
  const int kend = min(g.k, kbeg + g.k_chunk);
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int wm = (w >> 1) * 32, wn = (w & 1) * 32;
  const int li = lane & 15, lk = lane >> 4;

  v4f acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  float4 ra[BKT / 16], rb[BKT / 16];
  int buf = 0;
  if (kbeg < kend) {
    load_tiles<TRANS_B, BKT>(g, m0, n0, kbeg, kend, ra, rb);
    store_tiles<TRANS_B, BKT>(As[0], Bs[0], ra, rb);
  }
  __syncthreads();
  for (int k0 = kbeg; k0 < kend; k0 += BKT) {
    const bool more = k0 + BKT < kend;
    if (more) load_tiles<TRANS_B, BKT>(g, m0, n0, k0 + BKT, kend, ra, rb);
#pragma unroll
    for (int kk = 0; kk < BKT; kk += 4) {
      float af[2], bf[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) af[i] = As[buf][kk + lk][wm + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 2; ++j) bf[j] = Bs[buf][kk + lk][wn + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    if (more) store_tiles<TRANS_B, BKT>(As[buf ^ 1], Bs[buf ^ 1], ra, rb);
    __syncthreads();
    buf ^= 1;
  }

  // Accumulator (i, j, v) of this lane holds C[wm + 16i + 4*lk + v][wn + 16j + li].
  if constexpr (EPI == kStore || EPI == kPartial) {
    float* out = EPI == kPartial ? g.c + (size_t)split * g.m * g.n : g.c;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const int row = m0 + wm + i * 16 + lk * 4 + v;
          const int col = n0 + wn + j * 16 + li;
          if (row < g.m && col < g.n) {
            float x = acc[i][j][v];
            if (EPI == kStore && g.bias) x = x + g.bias[col];
            out[(size_t)row * g.n + col] = x;
          }
        }
  } else {
    // lm_head argmax: stage the logits tile in LDS, then 4 threads per row scan 16 columns
    // each in index order with the reference's online update (strict > keeps the first max)
    // and combine left to right (left wins ties), matmul.rs:532-589.
    __shared__ float Ct[BM][BN + 1];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) Ct[wm + i * 16 + lk * 4 + v][wn + j * 16 + li] = acc[i][j][v];
    __syncthreads();
    const int r = tid >> 2, q = tid & 3;
    float mx = -INFINITY, sum = 0.0f;
    int best = -1;
    for (int c = q * 16; c < q * 16 + 16; ++c) {
      const int col = n0 + c;
      if (col >= g.n) break;
      const float x = Ct[r][c];
      if (x > mx) {
        sum = isfinite(mx) ? sum * __expf(mx - x) + 1.0f : 1.0f;
        mx = x;
        best = col;
      } else {
        sum += __expf(x - mx);
      }
    }
    // combine the 4 quarters of the row in order (lanes 4r..4r+3 are adjacent)
#pragma unroll
    for (int off = 1; off < 4; off <<= 1) {
      const float omx = __shfl_down(mx, off, 64);
      const float osum = __shfl_down(sum, off, 64);
      const int obest = __shfl_down(best, off, 64);
      if ((q & (2 * off - 1)) == 0 && obest >= 0) {
        if (best < 0) {
          mx = omx;
          sum = osum;
          best = obest;
        } else if (mx >= omx) {
          sum = sum + osum * __expf(omx - mx);
        } else {
          sum = osum + sum * __expf(mx - omx);
          mx = omx;
          best = obest;
        }
      }
    }
    const int row = m0 + r;
    if (q == 0 && row < g.m) {
      float* dst = g.amax + ((size_t)row * g.n_tiles + n_tile) * 3;
      dst[0] = mx;
      reinterpret_cast<int*>(dst)[1] = best;
      dst[2] = sum;
    }
  }
}

// out[m, n] = sum over splits (in split order) + bias.  Four columns per thread when `vec`
// (n a multiple of 4 and out / bias 16-byte aligned; the partials always are).
__global__ void splitk_reduce_kernel(const float* __restrict__ parts, const float* __restrict__ bias,
                                     float* __restrict__ out, int m, int n, int splits, int vec) {
  const size_t total = (size_t)m * n;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  if (vec) {
    const size_t quads = total / 4;
    const float4* __restrict__ p4 = reinterpret_cast<const float4*>(parts);
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < quads; i += stride) {
      float4 s = p4[i];
      int z = 1;
      // eight partial loads in flight per step; the sum stays in split order
      for (; z + 8 <= splits; z += 8) {
        float4 p[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) p[u] = p4[(size_t)(z + u) * quads + i];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          s.x = s.x + p[u].x;
          s.y = s.y + p[u].y;
          s.z = s.z + p[u].z;
          s.w = s.w + p[u].w;
        }
      }
      for (; z < splits; ++z) {
        const float4 p = p4[(size_t)z * quads + i];
        s.x = s.x + p.x;
        s.y = s.y + p.y;
        s.z = s.z + p.z;
        s.w = s.w + p.w;
      }
      if (bias) {
        const float4 b = reinterpret_cast<const float4*>(bias)[(i * 4 % n) / 4];
        s.x = s.x + b.x;
        s.y = s.y + b.y;
        s.z = s.z + b.z;
        s.w = s.w + b.w;
      }
      reinterpret_cast<float4*>(out)[i] = s;
    }
    return;
  }
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    float s = parts[i];
    for (int z = 1; z < splits; ++z) s += parts[(size_t)z * total + i];
    if (bias) s = s + bias[i % n];
    out[i] = s;
  }
}

// Combines two (max, index, scaled sum) states.  The larger max wins and on equal maxima the
// smaller index, so the result is the first maximal index whatever the combination order;
// the sums are rescaled to the winning max.
__device__ __forceinline__ void argmax_combine(float& mx, int& best, float& sum, float omx, int obest, float osum) {
  if (obest < 0) return;
  if (best < 0) {
    mx = omx;
    best = obest;
    sum = osum;
  } else if (omx > mx || (omx == mx && obest < best)) {
    sum = osum + sum * __expf(mx - omx);
    mx = omx;
    best = obest;
  } else {
    sum = sum + osum * __expf(omx - mx);
  }
}

// One workgroup per row merges the row's per-tile (max, index, sum) states: each thread folds
// a strided subset of tiles, then the wave and the workgroup combine.
constexpr int kMergeThreads = 256;
__global__ __launch_bounds__(kMergeThreads) void argmax_merge_kernel(const float* __restrict__ amax, int n_tiles,
                                                                      int m, int32_t* __restrict__ token,
                                                                      float* __restrict__ prob) {
  __shared__ float s_mx[kMergeThreads / 64], s_sum[kMergeThreads / 64];
  __shared__ int s_best[kMergeThreads / 64];
  const int row = blockIdx.x;
  if (row >= m) return;
  const float* p = amax + (size_t)row * n_tiles * 3;
  float mx = -INFINITY, sum = 0.0f;
  int best = -1;
  // a thread's tiles t, t + 256, ... are loaded kUnroll at a time before they are combined (in
  // the same order, so the same sums): one memory round trip per kUnroll tiles instead of one
  // per tile.  Loads past n_tiles read tile 0 and are dropped.
  constexpr int kUnroll = 8;
  for (int t0 = threadIdx.x; t0 < n_tiles; t0 += kMergeThreads * kUnroll) {
    float omx[kUnroll], osum[kUnroll];
    int obest[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int t = t0 + u * kMergeThreads;
      const int tc = t < n_tiles ? t : 0;
      omx[u] = p[tc * 3];
      obest[u] = t < n_tiles ? reinterpret_cast<const int*>(p)[tc * 3 + 1] : -1;
      osum[u] = p[tc * 3 + 2];
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) argmax_combine(mx, best, sum, omx[u], obest[u], osum[u]);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float omx = __shfl_xor(mx, off, 64);
    const float osum = __shfl_xor(sum, off, 64);
    const int obest = __shfl_xor(best, off, 64);
    argmax_combine(mx, best, sum, omx, obest, osum);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_mx[w] = mx;
    s_sum[w] = sum;
    s_best[w] = best;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < kMergeThreads / 64; ++i) argmax_combine(mx, best, sum, s_mx[i], s_best[i], s_sum[i]);
    token[row] = best;
    prob[row] = 1.0f / sum;
  }
}

}  // namespace

namespace fi {

int32_t argmax_merge(fi_context* ctx, const float* amax, int32_t n_tiles, int32_t m, int32_t* token, float* prob) {
  hipLaunchKernelGGL(argmax_merge_kernel, dim3(m), dim3(kMergeThreads), 0, ctx->stream, amax, n_tiles, m, token, prob);
  FI_CHECK_LAUNCH("argmax_merge_kernel");
  return FI_OK;
}

}  // namespace fi

namespace {

// K range per split: enough workgroups (>= 2 per CU) for skinny shapes to keep every CU
// streaming weights, in whole stages of the kernel's K depth.
int choose_k_chunk(fi_context* ctx, int m, int n, int k, int bk) {
  const int tiles = ((m + BM - 1) / BM) * ((n + BN - 1) / BN);
  const int target = 2 * (ctx->compute_units > 0 ? ctx->compute_units : 256);
  if (tiles >= target) return k;
  const int want = (target + tiles - 1) / tiles;
  int chunk = (k + want - 1) / want;
  chunk = std::max(chunk, bk == BK ? 64 : bk);
  chunk = (chunk + bk - 1) / bk * bk;
  const int max_splits = 64;
  if ((k + chunk - 1) / chunk > max_splits) chunk = ((k + max_splits - 1) / max_splits + bk - 1) / bk * bk;
  return std::min(chunk, k);
}

template <bool TRANS_B, int BKT>
int32_t launch_gemm_bk(fi_context* ctx, GemmArgs g) {
  g.k_chunk = choose_k_chunk(ctx, g.m, g.n, g.k, BKT);
  const int splits = (g.k + g.k_chunk - 1) / g.k_chunk;
  dim3 grid((g.n + BN - 1) / BN, (g.m + BM - 1) / BM, splits);
  if (splits == 1) {
    hipLaunchKernelGGL((gemm_kernel<TRANS_B, kStore, BKT>), grid, dim3(kGemmThreads), 0, ctx->stream, g);
    FI_CHECK_LAUNCH("gemm_kernel");
    return FI_OK;
  }
  const size_t part_bytes = (size_t)splits * g.m * g.n * sizeof(float);
  FI_TRY(fi::ensure_workspace(ctx, part_bytes));
  float* parts = static_cast<float*>(ctx->workspace);
  float* out = g.c;
  const float* bias = g.bias;
  g.c = parts;
  hipLaunchKernelGGL((gemm_kernel<TRANS_B, kPartial, BKT>), grid, dim3(kGemmThreads), 0, ctx->stream, g);
  FI_CHECK_LAUNCH("gemm_kernel");
  const auto aligned = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const int vec = (g.n & 3) == 0 && aligned(out) && (bias == nullptr || aligned(bias)) ? 1 : 0;
  const size_t items = vec ? (size_t)g.m * g.n / 4 : (size_t)g.m * g.n;
  unsigned blocks = static_cast<unsigned>(std::min<size_t>((items + 255) / 256, 4096));
  hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, ctx->stream, parts, bias, out, g.m, g.n,
                     splits, vec);
  FI_CHECK_LAUNCH("splitk_reduce_kernel");
  return FI_OK;
}

template <bool TRANS_B>
int32_t launch_gemm(fi_context* ctx, const GemmArgs& g) {
  return launch_gemm_bk<TRANS_B, BK>(ctx, g);
}

}  // namespace

extern "C" {

int32_t fi_gemm(fi_context* ctx, const float* d_a, const float* d_b, const float* d_bias, float* d_c,
                int32_t m, int32_t k, int32_t n, int32_t b_layout) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(m >= 0 && k > 0 && n > 0, FI_ERR_INVALID_SHAPE, "fi_gemm: k and n must be positive");
  FI_REQUIRE(b_layout == 0 || b_layout == 1, FI_ERR_INVALID_LAYOUT, "fi_gemm: b_layout must be 0 ([K,N]) or 1 ([N,K])");
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_a && d_b && d_c, FI_ERR_INVALID_CONFIG, "fi_gemm: null pointer");
  GemmArgs g{};
  g.a = d_a;
  g.b = d_b;
  g.bias = d_bias;
  g.c = d_c;
  g.m = m;
  g.k = k;
  g.n = n;
  return b_layout == 0 ? launch_gemm<false>(ctx, g) : launch_gemm<true>(ctx, g);
}

int32_t fi_lm_head_argmax(fi_context* ctx, const float* d_hidden, const float* d_weight, int32_t m,
                          int32_t hidden, int32_t vocab, int32_t* d_token, float* d_prob) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(m >= 0 && hidden > 0, FI_ERR_INVALID_SHAPE, "fi_lm_head_argmax: hidden must be positive");
  FI_REQUIRE(vocab > 0, FI_ERR_INVALID_SHAPE, "fi_lm_head_argmax requires a non-empty output width");
  if (m == 0) return FI_OK;
  FI_REQUIRE(d_hidden && d_weight && d_token && d_prob, FI_ERR_INVALID_CONFIG, "fi_lm_head_argmax: null pointer");
  GemmArgs g{};
  g.a = d_hidden;
  g.b = d_weight;
  g.m = m;
  g.k = hidden;
  g.n = vocab;
  g.k_chunk = hidden;
  g.n_tiles = (vocab + BN - 1) / BN;
  FI_TRY(fi::ensure_workspace(ctx, (size_t)m * g.n_tiles * 3 * sizeof(float)));
  g.amax = static_cast<float*>(ctx->workspace);
  dim3 grid(g.n_tiles, (m + BM - 1) / BM, 1);
  hipLaunchKernelGGL((gemm_kernel<true, kArgmax, BK>), grid, dim3(kGemmThreads), 0, ctx->stream, g);
  FI_CHECK_LAUNCH("gemm_kernel(argmax)");
  hipLaunchKernelGGL(argmax_merge_kernel, dim3(m), dim3(kMergeThreads), 0, ctx->stream, g.amax, g.n_tiles, m,
                     d_token, d_prob);
  FI_CHECK_LAUNCH("argmax_merge_kernel");
  return FI_OK;
}

}  // extern "C"
