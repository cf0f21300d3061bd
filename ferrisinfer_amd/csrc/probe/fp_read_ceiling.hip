// Read-only kernels that measure the HBM read rate the paged decode access pattern allows on
// this GPU: the same bytes the decode partition kernel must read (every context token's K and
// V row of every kv head, f32 pools laid out [num_blocks][Hkv][16][D]), with no arithmetic
// beyond a running sum.  They are measurement tools for the benchmark, not part of the kernel
// library's interface.
//   mode 0, head chunks: one workgroup per (sequence, kv head, partition of P tokens), its four
//     waves owning P/4 consecutive tokens each: the decode kernel's decomposition (random
//     16 x D row runs of one kv head, 8 KiB for f32 D=128);
//   mode 1, whole blocks: one workgroup per (sequence, partition of P tokens) covering every kv
//     head, wave w owning heads [w Hkv/4, (w+1) Hkv/4): each block's Hkv x 16 x D run (64 KiB)
//     is read contiguously;
//   mode 2, linear: the same number of rows read as one contiguous run of each pool, P rows of
//     K and of V per workgroup.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kD = 128;            // head dimension (f32 rows of 32 float4)
constexpr int kVecs = kD / 4;
constexpr int kBlock = 16;         // tokens per block
constexpr int kDepth = 16;         // float4 loads in flight per lane

struct ReadArgs {
  const float* k;
  const float* v;
  const int* tables;
  const int* lens;
  float* sink;
  int num_seqs;
  int hkv;
  int max_blocks;
  int num_blocks;
  int parts;
  int part_tokens;
  long long linear_rows;
};

// Sums rows [0, nrows) of one pool, row r at base + rowoff(r) * kD, kDepth float4 per lane in flight.
template <typename RowOf>
__device__ __forceinline__ float read_rows(const float* __restrict__ base, int nrows, const RowOf& row_of,
                                           int lane) {
  float acc = 0.0f;
  const int total = nrows * kVecs;
  for (int i0 = 0; i0 < total; i0 += 64 * kDepth) {
    float4 b[kDepth];
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      const int i = min(i0 + d * 64 + lane, total - 1);  // past the end: re-read the last vector
      b[d] = *reinterpret_cast<const float4*>(base + (size_t)row_of(i / kVecs) * kD + (i % kVecs) * 4);
    }
#pragma unroll
    for (int d = 0; d < kDepth; ++d) acc += (b[d].x + b[d].y) + (b[d].z + b[d].w);
  }
  return acc;
}

__device__ __forceinline__ int block_id(const ReadArgs& a, int seq, int lb) {
  const int id = a.tables[(size_t)seq * a.max_blocks + lb];
  return id < 0 || id >= a.num_blocks ? 0 : id;
}

struct HeadRow {  // mode 0: token rows of one kv head, indices from LDS
  const uint32_t* rows;
  __device__ uint32_t operator()(int r) const { return rows[r]; }
};

struct BlockRow {  // mode 1: rows of heads h0..h0+hpw-1 of each block, block-major then head then token
  const int* ids;  // the partition's block ids (LDS)
  int hkv, h0, hpw, n;
  __device__ uint32_t operator()(int r) const {
    const int per_block = hpw * kBlock;
    const int blk = r / per_block, rem = r - blk * per_block;
    const int h = rem / kBlock, t = rem - h * kBlock;
    const int tok = min(blk * kBlock + t, n - 1);  // past the context: re-read its last token
    return (static_cast<uint32_t>(ids[tok / kBlock]) * hkv + h0 + h) * kBlock + tok % kBlock;
  }
};

struct LinearRow {
  uint32_t first;
  __device__ uint32_t operator()(int r) const { return first + r; }
};

__global__ __launch_bounds__(kThreads) void head_chunk_kernel(ReadArgs a) {
  extern __shared__ uint32_t s_row[];
  const int units = a.num_seqs * a.hkv;
  const int part = blockIdx.x / units, unit = blockIdx.x % units;
  const int seq = unit / a.hkv, kvh = unit % a.hkv;
  const int ctx = min(min(a.lens[seq], a.parts * a.part_tokens), a.max_blocks * kBlock);
  const int t0 = part * a.part_tokens;
  if (t0 >= ctx) return;
  const int n_part = min(a.part_tokens, ctx - t0);
  for (int t = threadIdx.x; t < n_part; t += kThreads) {
    const int pos = t0 + t;
    s_row[t] = (static_cast<uint32_t>(block_id(a, seq, pos / kBlock)) * a.hkv + kvh) * kBlock + pos % kBlock;
  }
  __syncthreads();
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wt = a.part_tokens / kWaves;
  const int n = min(wt, n_part - w * wt);
  if (n <= 0) return;
  const HeadRow rows{s_row + w * wt};
  const float acc = read_rows(a.k, n, rows, lane) + read_rows(a.v, n, rows, lane);
  if (acc == 1234.5f) a.sink[blockIdx.x % 1024] = acc;  // keeps the loads
}

__global__ __launch_bounds__(kThreads) void whole_block_kernel(ReadArgs a) {
  extern __shared__ int s_ids[];
  const int seq = blockIdx.x % a.num_seqs, part = blockIdx.x / a.num_seqs;
  const int ctx = min(min(a.lens[seq], a.parts * a.part_tokens), a.max_blocks * kBlock);
  const int t0 = part * a.part_tokens;
  if (t0 >= ctx) return;
  const int n_part = min(a.part_tokens, ctx - t0);
  const int nblk = (n_part + kBlock - 1) / kBlock;
  for (int b = threadIdx.x; b < nblk; b += kThreads) s_ids[b] = block_id(a, seq, t0 / kBlock + b);
  __syncthreads();
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int hpw = a.hkv / kWaves;
  const BlockRow rows{s_ids, a.hkv, w * hpw, hpw, n_part};
  const int nrows = nblk * hpw * kBlock;
  const float acc = read_rows(a.k, nrows, rows, lane) + read_rows(a.v, nrows, rows, lane);
  if (acc == 1234.5f) a.sink[blockIdx.x % 1024] = acc;
}

__global__ __launch_bounds__(kThreads) void linear_kernel(ReadArgs a) {
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int wt = a.part_tokens / kWaves;
  const long long first = (long long)blockIdx.x * a.part_tokens + (long long)w * wt;
  const int n = static_cast<int>(min((long long)wt, a.linear_rows - first));
  if (n <= 0) return;
  const LinearRow rows{static_cast<uint32_t>(first)};
  const float acc = read_rows(a.k, n, rows, lane) + read_rows(a.v, n, rows, lane);
  if (acc == 1234.5f) a.sink[blockIdx.x % 1024] = acc;
}

}  // namespace

extern "C" {

// Reads the paged context of `num_seqs` sequences once in the chosen decomposition; see the
// mode list above.  Pools hold num_blocks x hkv x 16 x 128 f32; `sink` holds 1024 floats.
// Returns 0, or -1 for an unsupported shape (part_tokens not a positive multiple of 64, hkv not
// a multiple of 4, more linear rows than a pool holds) or launch error.
int32_t fp_paged_read(const float* k, const float* v, const int32_t* tables, const int32_t* lens,
                      int32_t num_seqs, int32_t hkv, int32_t max_blocks, int32_t num_blocks,
                      int32_t max_context_len, int64_t total_tokens, int32_t mode, int32_t part_tokens,
                      float* sink, hipStream_t stream) {
  if (part_tokens <= 0 || part_tokens % 64 != 0 || part_tokens > 2048 || hkv <= 0 || hkv % kWaves != 0 ||
      num_seqs <= 0 || max_context_len <= 0 || max_context_len > max_blocks * kBlock)
    return -1;
  ReadArgs a{k, v, tables, lens, sink, num_seqs, hkv, max_blocks, num_blocks,
             (max_context_len + part_tokens - 1) / part_tokens, part_tokens, total_tokens * hkv};
  if (mode == 0) {
    hipLaunchKernelGGL(head_chunk_kernel, dim3(a.parts * num_seqs * hkv), dim3(kThreads),
                       part_tokens * sizeof(uint32_t), stream, a);
  } else if (mode == 1) {
    hipLaunchKernelGGL(whole_block_kernel, dim3(a.parts * num_seqs), dim3(kThreads),
                       (part_tokens / kBlock) * sizeof(int), stream, a);
  } else if (mode == 2) {
    if (a.linear_rows > (long long)num_blocks * hkv * kBlock) return -1;
    const long long wgs = (a.linear_rows + part_tokens - 1) / part_tokens;
    hipLaunchKernelGGL(linear_kernel, dim3(static_cast<unsigned>(wgs)), dim3(kThreads), 0, stream, a);
  } else {
    return -1;
  }
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // extern "C"
