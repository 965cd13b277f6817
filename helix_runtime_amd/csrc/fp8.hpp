// fp8 page elements on the device: OCP FP8 E4M3 (1 sign, 4 exponent bits of
// bias 7, 3 mantissa bits, no infinities, 0x7f / 0xff NaN, largest finite
// 448) with one fp32 scale per cache for keys and one for values.
//
// A page element is the code of x / scale rounded to nearest even,
// saturating (finite values and infinities past 448 become +-448; NaN stays
// NaN).  Its value is decode(code) * scale.  Rounding runs in integer code
// (appends are bandwidth-bound); decoding uses gfx950's packed conversion
// instruction, which reads OCP E4M3 on this target.
#pragma once

#include <hip/hip_runtime.h>

namespace helix::hip {

constexpr float kFp8Max = 448.0f;

// E4M3 code of y (already divided by the scale).
__host__ __device__ __forceinline__ unsigned fp8_code(float y) {
  const unsigned u = __builtin_bit_cast(unsigned, y);
  const unsigned sign = (u >> 24) & 0x80u;
  const unsigned a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;  // NaN
  if (a < 0x3c800000u) {
    // Below 2^-6 the grid is the subnormal step 2^-9: scale by 2^9 (exact)
    // and round to an integer, ties to even; 8 is the smallest normal code.
    return sign | static_cast<unsigned>(__builtin_rintf(__builtin_bit_cast(float, a) * 512.0f));
  }
  // Normal: round the fp32 mantissa to 3 bits (ties to even) with the
  // carry running into the exponent, then rebias the exponent 127 -> 7.
  unsigned r = (a + 0x7ffffu + ((a >> 20) & 1u)) >> 20;
  r -= 120u << 3;
  return sign | (r > 0x7eu ? 0x7eu : r);
}

// Four fp32 values (already divided by the scale) as four codes, the
// first in the low byte.
__device__ __forceinline__ unsigned fp8_pack4(float a, float b, float c, float d) {
  return fp8_code(a) | (fp8_code(b) << 8) | (fp8_code(c) << 16) | (fp8_code(d) << 24);
}
__device__ __forceinline__ unsigned fp8_pack4_scaled(float4 v, float scale) {
  return fp8_pack4(v.x / scale, v.y / scale, v.z / scale, v.w / scale);
}

// Four codes (low byte first) as fp32 values times scale.
__device__ __forceinline__ float4 fp8_widen4(unsigned w, float scale) {
  const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), false);
  const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8(static_cast<int>(w), true);
  return make_float4(lo[0] * scale, lo[1] * scale, hi[0] * scale, hi[1] * scale);
}
__device__ __forceinline__ float fp8_value(unsigned code, float scale) {
  return __builtin_amdgcn_cvt_f32_fp8(static_cast<int>(code), 0) * scale;
}

// fp32 values moved onto the scaled fp8 grid (kept as fp32).
__device__ __forceinline__ float4 fp8_rounded(float4 v, float scale) {
  return fp8_widen4(fp8_pack4_scaled(v, scale), scale);
}

}  // namespace helix::hip
