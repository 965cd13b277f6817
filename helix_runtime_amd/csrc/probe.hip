// HBM streaming-read probe: every thread reads 128-bit vectors in a
// grid-stride loop (UNROLL loads in flight per thread) and writes one float,
// so the kernel moves n * 4 bytes from HBM and almost nothing back.  Used by
// bench.py to measure the attainable read bandwidth of the device.
#include "../../include/helix_paged.h"

#include <hip/hip_runtime.h>

namespace {

template <int UNROLL>
__global__ __launch_bounds__(256) void stream_read_kernel(const float4* __restrict__ data,
                                                          std::size_t n4, float* out) {
  const std::size_t stride = static_cast<std::size_t>(gridDim.x) * blockDim.x;
  std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
  float acc = 0.0f;
  for (; i + (UNROLL - 1) * stride < n4; i += UNROLL * stride) {
    float4 v[UNROLL];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) v[u] = data[i + u * stride];
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) acc += v[u].x + v[u].y + v[u].z + v[u].w;
  }
  for (; i < n4; i += stride) {
    const float4 v = data[i];
    acc += v.x + v.y + v.z + v.w;
  }
  out[blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x] = acc;
}

}  // namespace

extern "C" int helix_probe_stream_read(const float* data, size_t n_floats, float* out,
                                       unsigned blocks, helix_stream stream) {
  if (data == nullptr || out == nullptr || n_floats % 4 != 0 || blocks == 0) {
    return HELIX_INVALID_ARGUMENT;
  }
  stream_read_kernel<8><<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const float4*>(data), n_floats / 4, out);
  return hipGetLastError() == hipSuccess ? HELIX_OK : HELIX_RUNTIME;
}
