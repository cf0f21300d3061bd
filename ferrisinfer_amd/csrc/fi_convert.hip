// Checkpoint tensor import: widening of F32 / BF16 / F16 safetensors payloads to f32 on the
// device, with the optional rank-2 transpose the HF loader applies to projection weights
// ([out, in] -> [in, out]).  Replaces io/safetensors.rs:437-471 (convert_to_f32_vec) and
// :538-568 (bf16_to_f32, f16_to_f32): the raw bytes travel to HBM unchanged (half the PCIe
// bytes for 16-bit checkpoints) and every element is widened exactly, NaN payloads included.
#include <algorithm>

#include "fi_common.h"
#include "fi_device.h"

namespace {

constexpr int kTile = 32;      // transpose tile edge
constexpr int kTileRows = 8;   // thread rows per tile (each thread moves kTile / kTileRows elements)

// IEEE binary16 -> binary32 bit pattern.  Normal numbers re-bias the exponent (15 -> 127);
// subnormals m * 2^-24 are normalised (bit 10 of the shifted mantissa becomes the implicit
// one); infinities and NaNs keep their payload in the top mantissa bits.
__device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint32_t h) {
  const uint32_t sign = (h & 0x8000u) << 16;
  const uint32_t exp = (h >> 10) & 0x1fu, man = h & 0x3ffu;
  if (exp == 0x1fu) return sign | 0x7f800000u | (man << 13);
  if (exp != 0) return sign | ((exp + 112u) << 23) | (man << 13);
  if (man == 0) return sign;
  const uint32_t shift = static_cast<uint32_t>(__clz(man)) - 21u;  // man's top bit -> bit 10
  return sign | ((113u - shift) << 23) | (((man << shift) & 0x3ffu) << 13);
}

template <int DT>
__device__ __forceinline__ float widen(const void* src, size_t i) {
  if constexpr (DT == FI_DTYPE_F32) {
    return static_cast<const float*>(src)[i];
  } else if constexpr (DT == FI_DTYPE_BF16) {
    return __uint_as_float(static_cast<uint32_t>(static_cast<const uint16_t*>(src)[i]) << 16);
  } else {
    return __uint_as_float(f16_bits_to_f32_bits(static_cast<const uint16_t*>(src)[i]));
  }
}

template <int DT>
__global__ void widen_kernel(const void* __restrict__ src, float* __restrict__ dst, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    dst[i] = widen<DT>(src, static_cast<size_t>(i));
  }
}

// dst[c][r] = widen(src[r][c]) for src [rows, cols]: a 32 x 32 tile is read along source rows
// and written along destination rows through LDS (one padding column against bank conflicts).
template <int DT>
__global__ __launch_bounds__(kTile * kTileRows) void widen_transpose_kernel(const void* __restrict__ src,
                                                                          float* __restrict__ dst, int64_t rows,
                                                                          int64_t cols) {
  __shared__ float tile[kTile][kTile + 1];
  const int64_t r0 = static_cast<int64_t>(blockIdx.y) * kTile, c0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int tx = threadIdx.x % kTile, ty = threadIdx.x / kTile;
#pragma unroll
  for (int i = 0; i < kTile; i += kTileRows) {
    const int64_t r = r0 + ty + i, c = c0 + tx;
    if (r < rows && c < cols) tile[ty + i][tx] = widen<DT>(src, static_cast<size_t>(r * cols + c));
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile; i += kTileRows) {
    const int64_t c = c0 + ty + i, r = r0 + tx;
    if (r < rows && c < cols) dst[c * rows + r] = tile[tx][ty + i];
  }
}

template <int DT>
void launch_widen(fi_context* ctx, const void* src, int64_t rows, int64_t cols, bool transpose, float* dst) {
  if (!transpose) {
    const int64_t n = rows * cols;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(widen_kernel<DT>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx->stream, src, dst, n);
  } else {
    const dim3 grid(static_cast<unsigned>((cols + kTile - 1) / kTile), static_cast<unsigned>((rows + kTile - 1) / kTile));
    hipLaunchKernelGGL(widen_transpose_kernel<DT>, grid, dim3(kTile * kTileRows), 0, ctx->stream, src, dst, rows, cols);
  }
}

// dst[i] = bf16 bits of src[i], rounded to nearest even (NaN stays NaN): four elements per
// thread and step where both pointers allow 16- and 8-byte accesses, one otherwise.
__global__ void narrow_bf16_kernel(const float* __restrict__ src, uint16_t* __restrict__ dst, int64_t n, int vec) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (vec) {
    const int64_t n4 = n / 4;
    for (int64_t i = first; i < n4; i += stride) {
      const float4 x = reinterpret_cast<const float4*>(src)[i];
      const uint32_t b0 = fi::f32_to_bf16_bits(x.x), b1 = fi::f32_to_bf16_bits(x.y);
      const uint32_t b2 = fi::f32_to_bf16_bits(x.z), b3 = fi::f32_to_bf16_bits(x.w);
      reinterpret_cast<uint2*>(dst)[i] = make_uint2(b0 | (b1 << 16), b2 | (b3 << 16));
    }
    for (int64_t i = 4 * n4 + first; i < n; i += stride) dst[i] = static_cast<uint16_t>(fi::f32_to_bf16_bits(src[i]));
  } else {
    for (int64_t i = first; i < n; i += stride) dst[i] = static_cast<uint16_t>(fi::f32_to_bf16_bits(src[i]));
  }
}

}  // namespace

extern "C" {

int32_t fi_convert_f32_to_bf16(fi_context* ctx, const float* d_src, int64_t n, uint16_t* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(n >= 0, FI_ERR_INVALID_SHAPE, "fi_convert_f32_to_bf16: negative length");
  if (n == 0) return FI_OK;
  FI_REQUIRE(d_src != nullptr && d_dst != nullptr, FI_ERR_INVALID_CONFIG, "fi_convert_f32_to_bf16: null pointer");
  const uintptr_t s = reinterpret_cast<uintptr_t>(d_src), d = reinterpret_cast<uintptr_t>(d_dst);
  FI_REQUIRE(d + 2 * static_cast<uintptr_t>(n) <= s || s + 4 * static_cast<uintptr_t>(n) <= d, FI_ERR_INVALID_CONFIG,
             "fi_convert_f32_to_bf16: source and destination must not overlap");
  const int vec = s % 16 == 0 && d % 8 == 0;
  const int64_t blocks = std::min<int64_t>((n / (vec ? 4 : 1) + 255) / 256 + 1, 8192);
  hipLaunchKernelGGL(narrow_bf16_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, ctx->stream, d_src, d_dst,
                     n, vec);
  FI_CHECK_LAUNCH("narrow_bf16_kernel");
  return FI_OK;
}

int32_t fi_convert_to_f32(fi_context* ctx, const void* d_src, int32_t src_dtype, int64_t rows, int64_t cols,
                          int32_t transpose, float* d_dst) {
  FI_TRY(fi::enter(ctx));
  FI_REQUIRE(src_dtype == FI_DTYPE_F32 || src_dtype == FI_DTYPE_BF16 || src_dtype == FI_DTYPE_F16,
             FI_ERR_UNSUPPORTED, "fi_convert_to_f32: source dtype must be F32, BF16 or F16");
  FI_REQUIRE(rows >= 0 && cols >= 0, FI_ERR_INVALID_SHAPE, "fi_convert_to_f32: negative dimension");
  FI_REQUIRE(!transpose || (rows <= 65535L * kTile && cols <= 2147483647L), FI_ERR_INVALID_SHAPE,
             "fi_convert_to_f32: transpose grid too large");
  if (rows == 0 || cols == 0) return FI_OK;
  FI_REQUIRE(d_src != nullptr && d_dst != nullptr, FI_ERR_INVALID_CONFIG, "fi_convert_to_f32: null pointer");
  FI_REQUIRE(static_cast<const void*>(d_dst) != d_src, FI_ERR_INVALID_CONFIG,
             "fi_convert_to_f32: source and destination must not alias");
  const bool t = transpose != 0;
  switch (src_dtype) {
    case FI_DTYPE_F32:
      launch_widen<FI_DTYPE_F32>(ctx, d_src, rows, cols, t, d_dst);
      break;
    case FI_DTYPE_BF16:
      launch_widen<FI_DTYPE_BF16>(ctx, d_src, rows, cols, t, d_dst);
      break;
    default:
      launch_widen<FI_DTYPE_F16>(ctx, d_src, rows, cols, t, d_dst);
      break;
  }
  FI_CHECK_LAUNCH("widen_kernel");
  return FI_OK;
}

}  // extern "C"
