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

// One wavefront per work list; each step reads a K and a V page chunk of
// 16 rows x 128 elements of EB bytes (8 KiB for fp32, 4 KiB for bf16, 2 KiB
// for fp8) with one load of 4 elements per lane per two rows, two steps in
// flight: the decode kernel's access pattern for each page type.
template <int EB>
struct ProbeWords;
template <>
struct ProbeWords<4> {
  typedef unsigned T __attribute__((ext_vector_type(4)));
  template <int AUX>
  static __device__ T load(__amdgpu_buffer_rsrc_t r, int off, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, soff, AUX);
  }
  static __device__ float first(const T& t) { return __uint_as_float(t[0]); }
};
template <>
struct ProbeWords<2> {
  typedef unsigned T __attribute__((ext_vector_type(2)));
  template <int AUX>
  static __device__ T load(__amdgpu_buffer_rsrc_t r, int off, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, off, soff, AUX);
  }
  static __device__ float first(const T& t) { return __uint_as_float(t[0]); }
};
template <>
struct ProbeWords<1> {
  typedef unsigned T;
  template <int AUX>
  static __device__ T load(__amdgpu_buffer_rsrc_t r, int off, int soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, off, soff, AUX);
  }
  static __device__ float first(const T& t) { return __uint_as_float(t); }
};

template <int AUX, int EB>
__global__ __launch_bounds__(64) void page_read_kernel(const unsigned char* __restrict__ pool,
                                                       const std::uint32_t* __restrict__ pairs,
                                                       int steps, float* out) {
  using W = ProbeWords<EB>;
  constexpr int kChunk = 2048 * EB;  // one page of one kv head
  const int lane = threadIdx.x;
  const std::uint32_t* my = pairs + static_cast<std::size_t>(blockIdx.x) * steps * 2;
  float acc = 0.0f;
  typename W::T ka[8], va[8], kb[8], vb[8];
  auto load = [&](int c, typename W::T (&k)[8], typename W::T (&v)[8]) {
    // Past the end: an empty buffer range, so the loads return zeros
    // without touching memory (the instruction stream stays the same).
    const int range = c < steps ? kChunk : 0;
    c = c < steps ? c : steps - 1;
    const std::uint32_t ck = __builtin_amdgcn_readfirstlane(my[2 * c]);
    const std::uint32_t cv = __builtin_amdgcn_readfirstlane(my[2 * c + 1]);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(pool + static_cast<std::size_t>(ck) * kChunk), 0, range,
        kProbeWord3);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<unsigned char*>(pool + static_cast<std::size_t>(cv) * kChunk), 0, range,
        kProbeWord3);
#pragma unroll
    for (int u = 0; u < 8; ++u) k[u] = W::template load<AUX>(rk, lane * 4 * EB, u * 256 * EB);
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = W::template load<AUX>(rv, lane * 4 * EB, u * 256 * EB);
  };
  load(0, ka, va);
  load(1, kb, vb);
  for (int c = 0; c < steps; c += 2) {
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += W::first(ka[u]) + W::first(va[u]);
    load(c + 2, ka, va);
#pragma unroll
    for (int u = 0; u < 8; ++u) acc += W::first(kb[u]) + W::first(vb[u]);
    load(c + 3, kb, vb);
  }
  out[blockIdx.x * 64 + lane] = acc;
}

template <int EB>
void launch_page_read(unsigned waves, int nontemporal, const unsigned char* pool,
                      const std::uint32_t* pairs, int steps, float* out, hipStream_t s) {
  if (nontemporal) {
    page_read_kernel<2, EB><<<waves, 64, 0, s>>>(pool, pairs, steps, out);
  } else {
    page_read_kernel<0, EB><<<waves, 64, 0, s>>>(pool, pairs, steps, out);
  }
}

}  // namespace

// element_bytes: 4 (fp32 pages), 2 (bf16) or 1 (fp8); the pair indices
// count page chunks of 2048 elements.
extern "C" int helix_probe_page_read(const void* pool, const uint32_t* pairs, size_t steps,
                                     unsigned waves, int nontemporal, int element_bytes,
                                     float* out, void* stream) {
  if (pool == nullptr || pairs == nullptr || out == nullptr || steps == 0 || waves == 0 ||
      steps > 0x7fffffff || (element_bytes != 4 && element_bytes != 2 && element_bytes != 1)) {
    return 1;
  }
  const auto* p = static_cast<const unsigned char*>(pool);
  const auto s = static_cast<hipStream_t>(stream);
  const int n = static_cast<int>(steps);
  switch (element_bytes) {
    case 4: launch_page_read<4>(waves, nontemporal, p, pairs, n, out, s); break;
    case 2: launch_page_read<2>(waves, nontemporal, p, pairs, n, out, s); break;
    default: launch_page_read<1>(waves, nontemporal, p, pairs, n, out, s); break;
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
