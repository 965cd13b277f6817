// bf16 page elements on the device.  A bf16 page element is the fp32 value
// rounded to nearest even (NaN stays NaN, quieted; values past the largest
// bf16 become inf); widening one back to fp32 is exact.
#pragma once

#include <hip/hip_runtime.h>

namespace helix::hip {

__device__ __forceinline__ unsigned short bf16_round(float f) {
  const unsigned u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<unsigned short>((u >> 16) | 0x40u);
  return static_cast<unsigned short>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
__device__ __forceinline__ float bf16_value(unsigned bits16) {
  return __uint_as_float(bits16 << 16);
}
// Two fp32 values rounded and packed, the first in the low half.
__device__ __forceinline__ unsigned bf16_pack(float lo, float hi) {
  return static_cast<unsigned>(bf16_round(lo)) | (static_cast<unsigned>(bf16_round(hi)) << 16);
}
// Four bf16 (two per word, low half first) as fp32.
__device__ __forceinline__ float4 bf16_widen(unsigned w0, unsigned w1) {
  return make_float4(__uint_as_float(w0 << 16), __uint_as_float(w0 & 0xffff0000u),
                     __uint_as_float(w1 << 16), __uint_as_float(w1 & 0xffff0000u));
}
// fp32 values moved onto the bf16 grid (kept as fp32).
__device__ __forceinline__ float4 bf16_rounded(float4 v) {
  return make_float4(bf16_value(bf16_round(v.x)), bf16_value(bf16_round(v.y)),
                     bf16_value(bf16_round(v.z)), bf16_value(bf16_round(v.w)));
}

}  // namespace helix::hip
