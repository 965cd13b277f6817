// HBM streaming-read probe: every thread reads 128-bit vectors in a
// grid-stride loop (UNROLL loads in flight per thread) and writes one float,
// so the kernel moves n * 4 bytes from HBM and almost nothing back.  Used by
// bench.py to measure the attainable read bandwidth of the device.  Built
// into libhelix_probe.so, which only bench.py loads; return codes are 0 (ok),
// 1 (invalid argument) and 5 (launch failed).

#include <hip/hip_runtime.h>

#include <cstdint>

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

constexpr int kProbeWord3 = 0x00020000;
typedef unsigned probe_u32x4 __attribute__((ext_vector_type(4)));

// One wavefront per work list; each step reads a K and a V chunk of 8 KiB
// with 1 KiB-per-instruction buffer loads, two steps in flight.
template <int AUX>
__global__ __launch_bounds__(64) void page_read_kernel(const float* __restrict__ pool,
                                                       const std::uint32_t* __restrict__ pairs,
                                                       int steps, float* out) {
  const int lane = threadIdx.x;
  const std::uint32_t* my = pairs + static_cast<std::size_t>(blockIdx.x) * steps * 2;
  float acc = 0.0f;
  probe_u32x4 ka[8], va[8], kb[8], vb[8];
  auto load = [&](int c, probe_u32x4 (&k)[8], probe_u32x4 (&v)[8]) {
    // Past the end: an empty buffer range, so the loads return zeros
    // without touching memory (the instruction stream stays the same).
    const int range = c < steps ? 8192 : 0;
    c = c < steps ? c : steps - 1;
    const std::uint32_t ck = __builtin_amdgcn_readfirstlane(my[2 * c]);
    const std::uint32_t cv = __builtin_amdgcn_readfirstlane(my[2 * c + 1]);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(pool + static_cast<std::size_t>(ck) * 2048), 0, range, kProbeWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(pool + static_cast<std::size_t>(cv) * 2048), 0, range, kProbeWord3);
#pragma unroll
    for (int u = 0; u < 8; ++u) k[u] = __builtin_amdgcn_raw_buffer_load_b128(rk, lane * 16, u * 1024, AUX);
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = __builtin_amdgcn_raw_buffer_load_b128(rv, lane * 16, u * 1024, AUX);
  };
  load(0, ka, va);
  load(1, kb, vb);
  for (int c = 0; c < steps; c += 2) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += __uint_as_float(ka[u][0]) + __uint_as_float(va[u][3]);
    load(c + 2, ka, va);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += __uint_as_float(kb[u][1]) + __uint_as_float(vb[u][2]);
    load(c + 3, kb, vb);
  }
  out[blockIdx.x * 64 + lane] = acc;
}

}  // namespace

extern "C" int helix_probe_page_read(const float* pool, const uint32_t* pairs, size_t steps,
                                     unsigned waves, int nontemporal, float* out,
                                     void* stream) {
  if (pool == nullptr || pairs == nullptr || out == nullptr || steps == 0 || waves == 0 ||
      steps > 0x7fffffff) {
    return 1;
  }
  const auto s = static_cast<hipStream_t>(stream);
  if (nontemporal != 0) {
    page_read_kernel<2><<<waves, 64, 0, s>>>(pool, pairs, static_cast<int>(steps), out);
  } else {
    page_read_kernel<0><<<waves, 64, 0, s>>>(pool, pairs, static_cast<int>(steps), out);
  }
  return hipGetLastError() == hipSuccess ? 0 : 5;
}

extern "C" int helix_probe_stream_read(const float* data, size_t n_floats, float* out,
                                       unsigned blocks, void* stream) {
  if (data == nullptr || out == nullptr || n_floats % 4 != 0 || blocks == 0) {
    return 1;
  }
  stream_read_kernel<8><<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(
      reinterpret_cast<const float4*>(data), n_floats / 4, out);
  return hipGetLastError() == hipSuccess ? 0 : 5;
}
