// Feature-row dot products for gfx950: a 16-byte packet dot (dot2
// instructions for 16-bit types) and the sum over a G-lane sub-group.
#pragma once

#include "ogn_device.h"

#include <type_traits>

namespace ogn {

// Sum over aligned groups of G lanes (G a power of two up to 64): DPP inside
// each 16-lane row, cross-row swaps beyond; every lane of a group ends with
// the group's sum.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  auto dpp = [](float x, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  if constexpr (G >= 2) v += dpp(v, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  if constexpr (G >= 4) v += dpp(v, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  if constexpr (G >= 8) v += dpp(v, std::integral_constant<int, 0x141>{});  // row_half_mirror
  if constexpr (G >= 16) v += dpp(v, std::integral_constant<int, 0x140>{}); // row_mirror
  if constexpr (G >= 32) v += xor_shfl<16>(v);
  if constexpr (G >= 64) v += xor_shfl<32>(v);
  return v;
}

// Dot of two 16-byte feature packets, accumulated in fp32: fp16 and bf16
// pairs go through v_dot2c_f32_f16 / v_dot2c_f32_bf16 (products of 16-bit
// values are exact in fp32), four instructions per packet; fp32 packets take
// four FMAs.
template <int DT>
__device__ __forceinline__ float packet_dot(const uint4& a, const uint4& b, float d) {
  if constexpr (DT == OGN_F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.x), __builtin_bit_cast(h2, b.x), d, false);
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.y), __builtin_bit_cast(h2, b.y), d, false);
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.z), __builtin_bit_cast(h2, b.z), d, false);
    d = __builtin_amdgcn_fdot2(__builtin_bit_cast(h2, a.w), __builtin_bit_cast(h2, b.w), d, false);
  } else if constexpr (DT == OGN_BF16) {
    typedef short s2 __attribute__((ext_vector_type(2)));
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s2, a.x), __builtin_bit_cast(s2, b.x), d, false);
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s2, a.y), __builtin_bit_cast(s2, b.y), d, false);
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s2, a.z), __builtin_bit_cast(s2, b.z), d, false);
    d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(s2, a.w), __builtin_bit_cast(s2, b.w), d, false);
  } else {
    d = __builtin_fmaf(__uint_as_float(a.x), __uint_as_float(b.x), d);
    d = __builtin_fmaf(__uint_as_float(a.y), __uint_as_float(b.y), d);
    d = __builtin_fmaf(__uint_as_float(a.z), __uint_as_float(b.z), d);
    d = __builtin_fmaf(__uint_as_float(a.w), __uint_as_float(b.w), d);
  }
  return d;
}

}  // namespace ogn
