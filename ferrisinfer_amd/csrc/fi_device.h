// Device helpers shared by the gfx950 kernels (wave64 cross-lane ops, bf16 storage).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace fi {

// One DPP move inside a row of 16 lanes.  Control codes (GCN/CDNA DPP):
//   quad_perm [1,0,3,2] = 0xB1, quad_perm [2,3,0,1] = 0x4E, row_half_mirror = 0x141,
//   row_mirror = 0x140.
template <int kCtrl>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), kCtrl, 0xF, 0xF, false));
}

// Sum over aligned groups of kLanes consecutive lanes (kLanes in {1,2,4,8,16}); every lane
// of a group ends with the group total.  row_mirror = 0x140 reverses a row of 16 lanes.
template <int kLanes>
__device__ __forceinline__ float group_sum(float v) {
  static_assert(kLanes == 1 || kLanes == 2 || kLanes == 4 || kLanes == 8 || kLanes == 16, "group size");
  if constexpr (kLanes >= 2) v += dpp_mov<0xB1>(v);
  if constexpr (kLanes >= 4) v += dpp_mov<0x4E>(v);
  if constexpr (kLanes >= 8) v += dpp_mov<0x141>(v);
  if constexpr (kLanes >= 16) v += dpp_mov<0x140>(v);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// The value lane ^ 32 (lane ^ 16) holds, from v_permlane32_swap (v_permlane16_swap): a VALU
// exchange between the wave's halves (16-lane rows) with no LDS round trip.  With both
// operands x, the swap's second result holds the partner in lanes 0-31 (even rows) and its
// first result in lanes 32-63 (odd rows).
__device__ __forceinline__ float lane_xor32(float x, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(lane < 32 ? r[1] : r[0]);
}

__device__ __forceinline__ float lane_xor16(float x, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(((lane >> 4) & 1) == 0 ? r[1] : r[0]);
}

// bf16 storage: widening is exact (bits << 16); narrowing rounds to nearest even.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __builtin_bit_cast(float, bits16 << 16);
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t w = __builtin_bit_cast(uint32_t, f);
  if ((w & 0x7f800000u) == 0x7f800000u && (w & 0x007fffffu) != 0) return (w >> 16) | 0x0040u;
  w += 0x7fffu + ((w >> 16) & 1u);
  return w >> 16;
}

}  // namespace fi
