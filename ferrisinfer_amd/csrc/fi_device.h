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

// ---- three-piece bf16 split of f32 operands (the f32-accuracy products on bf16 MFMA) ----
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Two f32 values a, b as x = hi + mid + lo exactly: hi = RNE_bf16(x), mid = RNE_bf16(x - hi),
// lo = x - hi - mid (exact in bf16).  Each piece pair is rounded once (v_cvt_pk_bf16_f32, a in
// the low half) and widened back by shift and mask, so no value is converted twice.
__device__ __forceinline__ void split3_pk(float a, float b, uint32_t& h, uint32_t& m, uint32_t& l) {
  h = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{a, b}, bf16x2_t));
  const float ra = a - __builtin_bit_cast(float, h << 16);
  const float rb = b - __builtin_bit_cast(float, h & 0xffff0000u);
  m = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{ra, rb}, bf16x2_t));
  const float sa = ra - __builtin_bit_cast(float, m << 16);
  const float sb = rb - __builtin_bit_cast(float, m & 0xffff0000u);
  l = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{sa, sb}, bf16x2_t));
}

// ---- the q|k|v consumer's arithmetic (split-K sum + bias, RoPE, pool store), shared by
// qkv_rope_append4_kernel and decode attention's fused q|k|v prologue so both give identical
// values ----

__device__ __forceinline__ float add(float a, float b) { return a + b; }
__device__ __forceinline__ float4 add(float4 a, float4 b) { return make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w); }

// sum over z < splits of p[z * plane], added in split order; the split loads are issued in
// batches of eight before their adds (one memory latency per batch)
template <typename T>
__device__ __forceinline__ T sum_splits(const T* __restrict__ p, size_t plane, int splits) {
  T x = p[0];
  for (int z0 = 1; z0 < splits; z0 += 8) {
    T v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int z = z0 + u;
      v[u] = p[(size_t)(z < splits ? z : 0) * plane];
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (z0 + u < splits) x = add(x, v[u]);
    }
  }
  return x;
}

// Four consecutive columns of the q|k|v projection: the split-K partials [splits][tokens][width]
// of one token (p0 = its row in split 0) summed in split order, plus the bias, if any.
__device__ __forceinline__ float4 qkv_value4(const float* __restrict__ p0, size_t plane, int splits,
                                             const float* __restrict__ bias, int bias_col, int col) {
  float4 x = sum_splits(reinterpret_cast<const float4*>(p0 + col), plane / 4, splits);
  if (bias) x = add(x, *reinterpret_cast<const float4*>(bias + bias_col));
  return x;
}

// RoPE of four consecutive rotary pairs (lo, hi) = (x[i], x[i + half]) with their cos / sin:
// y0 = lo cos - hi sin, y1 = hi cos + lo sin, each product rounded before the add
// (kernel/cpu/attention.rs:165-220).
__device__ __forceinline__ void rope4(const float4& lo, const float4& hi, const float4& c, const float4& sn,
                                      float4& y0, float4& y1) {
#pragma clang fp contract(off)
  y0 = make_float4(lo.x * c.x - hi.x * sn.x, lo.y * c.y - hi.y * sn.y, lo.z * c.z - hi.z * sn.z,
                   lo.w * c.w - hi.w * sn.w);
  y1 = make_float4(hi.x * c.x + lo.x * sn.x, hi.y * c.y + lo.y * sn.y, hi.z * c.z + lo.z * sn.z,
                   hi.w * c.w + lo.w * sn.w);
}

// Four consecutive pool elements from one 16-byte (f32) or 8-byte (bf16, nearest even) store;
// idx is a multiple of 4 (the pool's rows are D elements, D a multiple of 4).
template <typename KVT>
__device__ __forceinline__ void put_kv4(KVT* cache, size_t idx, const float4& x) {
  if constexpr (sizeof(KVT) == 4) {
    *reinterpret_cast<float4*>(cache + idx) = x;
  } else {
    uint2 w;
    w.x = f32_to_bf16_bits(x.x) | (f32_to_bf16_bits(x.y) << 16);
    w.y = f32_to_bf16_bits(x.z) | (f32_to_bf16_bits(x.w) << 16);
    *reinterpret_cast<uint2*>(cache + idx) = w;
  }
}

}  // namespace fi
