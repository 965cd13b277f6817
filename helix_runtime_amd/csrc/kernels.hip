// Paged-KV kernels for CDNA4 (gfx950): page append / gather / copy-on-write,
// batched split-K decode attention with an uncommitted tail, the split
// combine, and a reference-shaped generic attention kernel.
//
// Data layout in HBM: one layer pool is [physical_blocks, kv_heads,
// block_tokens, head_dim] fp32, so one (block, head) page of 16 tokens x 128
// dims is one contiguous 8 KiB run.  Key and value pools of all layers live
// in one allocation (see paged_cache.cpp).
#include "kernels.hpp"

#include "bf16.hpp"
#include "fp8.hpp"
#include "prefill_body.hpp"

#include <atomic>
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <limits>
#include <type_traits>

namespace helix::hip {
namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

inline unsigned grid_for(std::size_t work, std::size_t per_block, std::size_t cap = 1u << 20) {
  std::size_t blocks = (work + per_block - 1) / per_block;
  if (blocks == 0) blocks = 1;
  return static_cast<unsigned>(blocks < cap ? blocks : cap);
}

// --------------------------------------------------------- page elements ----
// Pages hold fp32 (the reference's format), bf16 (bf16.hpp) or fp8 E4M3
// codes (fp8.hpp).  Rows passed in and gather outputs are fp32 whatever the
// type; `scale` is the fp8 scale of the pool (ignored by the other types).
// W consecutive elements between fp32 rows and pages of element type S.
template <typename S, int W>
struct Elems;
template <int W>
struct Elems<float, W> {
  static __device__ __forceinline__ void copy(float* dst, const float* src) {
    if constexpr (W == 4) {
      *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(src);
    } else {
      *dst = *src;
    }
  }
  static __device__ __forceinline__ void put(float* dst, const float* src, float) { copy(dst, src); }
  static __device__ __forceinline__ void get(float* dst, const float* src, float) { copy(dst, src); }
};
template <int W>
struct Elems<unsigned short, W> {
  static __device__ __forceinline__ void put(unsigned short* dst, const float* src, float) {
    if constexpr (W == 4) {
      const float4 v = *reinterpret_cast<const float4*>(src);
      *reinterpret_cast<uint2*>(dst) = make_uint2(bf16_pack(v.x, v.y), bf16_pack(v.z, v.w));
    } else {
      *dst = bf16_round(*src);
    }
  }
  static __device__ __forceinline__ void get(float* dst, const unsigned short* src, float) {
    if constexpr (W == 4) {
      const uint2 p = *reinterpret_cast<const uint2*>(src);
      *reinterpret_cast<float4*>(dst) = bf16_widen(p.x, p.y);
    } else {
      *dst = bf16_value(*src);
    }
  }
  static __device__ __forceinline__ void copy(unsigned short* dst, const unsigned short* src) {
    if constexpr (W == 4) {
      *reinterpret_cast<uint2*>(dst) = *reinterpret_cast<const uint2*>(src);
    } else {
      *dst = *src;
    }
  }
};

template <int W>
struct Elems<unsigned char, W> {
  static __device__ __forceinline__ void put(unsigned char* dst, const float* src, float scale) {
    if constexpr (W == 4) {
      *reinterpret_cast<unsigned*>(dst) =
          fp8_pack4_scaled(*reinterpret_cast<const float4*>(src), scale);
    } else {
      *dst = static_cast<unsigned char>(fp8_code(*src / scale));
    }
  }
  static __device__ __forceinline__ void get(float* dst, const unsigned char* src, float scale) {
    if constexpr (W == 4) {
      *reinterpret_cast<float4*>(dst) = fp8_widen4(*reinterpret_cast<const unsigned*>(src), scale);
    } else {
      *dst = fp8_value(*src, scale);
    }
  }
  static __device__ __forceinline__ void copy(unsigned char* dst, const unsigned char* src) {
    if constexpr (W == 4) {
      *reinterpret_cast<unsigned*>(dst) = *reinterpret_cast<const unsigned*>(src);
    } else {
      *dst = *src;
    }
  }
};

// ------------------------------------------------------------- append ----
// Reference: CudaPagedKvCache::append issues 2 * layers * kv_heads
// cudaMemcpyAsync D2D copies of one head vector (src/kv_cache/cuda_paged.cpp:
// 561-577).  Here one launch moves every (layer, head) vector of K and V with
// 128-bit accesses; blockIdx.y selects keys (0) or values (1).
template <typename S, int W>
__global__ void append_token_kernel(const float* __restrict__ keys,
                                    const float* __restrict__ values, S* key_base, S* value_base,
                                    std::size_t layer_stride, std::size_t layers,
                                    std::size_t heads, std::size_t block_tokens, std::size_t dim,
                                    std::uint32_t block, std::size_t offset, float2 scale) {
  const std::size_t dv = dim / W;
  const std::size_t total = layers * heads * dv;
  const float* src = blockIdx.y == 0 ? keys : values;
  S* base = blockIdx.y == 0 ? key_base : value_base;
  const float sc = blockIdx.y == 0 ? scale.x : scale.y;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t c = e % dv;
    const std::size_t lh = e / dv;
    const std::size_t h = lh % heads;
    const std::size_t l = lh / heads;
    S* dst = base + l * layer_stride +
             ((static_cast<std::size_t>(block) * heads + h) * block_tokens + offset) * dim + c * W;
    Elems<S, W>::put(dst, src + e * W, sc);
  }
}

// Reference: PagedKvCache::append_layer_major span copies
// (src/kv_cache/paged.cpp:819-843), token range [old_length, old_length+T).
struct LayerPointers {
  const float* const* keys;
  const float* const* values;
};

template <typename S, int W>
__global__ void append_bulk_kernel(LayerPointers src, S* key_base, S* value_base,
                                   std::size_t layer_stride, std::size_t layers,
                                   std::size_t heads, std::size_t block_tokens, std::size_t dim,
                                   const std::uint32_t* __restrict__ blocks,
                                   std::size_t first_block, std::size_t old_length,
                                   std::size_t tokens, float2 scale) {
  const std::size_t dv = dim / W;
  const std::size_t per_layer = heads * tokens * dv;
  const std::size_t total = layers * per_layer;
  S* base = blockIdx.y == 0 ? key_base : value_base;
  const float* const* layer_src = blockIdx.y == 0 ? src.keys : src.values;
  const float sc = blockIdx.y == 0 ? scale.x : scale.y;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t l = e / per_layer;
    const std::size_t r = e % per_layer;  // (h * tokens + t) * dv + c
    const std::size_t c = r % dv;
    const std::size_t ht = r / dv;
    const std::size_t t = ht % tokens;
    const std::size_t h = ht / tokens;
    const std::size_t pos = old_length + t;
    const std::size_t phys = blocks[pos / block_tokens - first_block];
    S* dst = base + l * layer_stride +
             ((phys * heads + h) * block_tokens + pos % block_tokens) * dim + c * W;
    Elems<S, W>::put(dst, layer_src[l] + r * W, sc);
  }
}

// Batched append through a slot mapping, for one layer or for every layer
// of a step at once.  Source rows are [layers, batch, heads, tokens, dim]
// (tokens = 1 for a decode step, the chunk length for chunked prefill);
// token t of sequence b goes to physical slot slots[b * tokens + t] =
// block * block_tokens + offset (negative: skipped) of every layer, whose
// pools lie layer_stride page elements apart.  The all-layer form is the
// batched CudaPagedKvCache::append (src/kv_cache/cuda_paged.cpp:491-611),
// which commits one token's [layers, kv_heads, dim] rows after the forward
// pass.  The (layer, sequence, token) row comes from the workgroup index,
// so each lane divides only for its (head, vector) pair.
template <typename S, int W>
__global__ __launch_bounds__(256) void append_slots_kernel(
    const float* __restrict__ keys, const float* __restrict__ values, S* key_pool, S* value_pool,
    std::size_t layer_stride, unsigned heads, unsigned block_tokens, unsigned dim,
    const std::int64_t* __restrict__ slots, unsigned count, unsigned tokens, float2 scale) {
  // Grid: x covers one row group's heads * dim / W vectors, y walks the
  // (sequence, token) rows, z = 2 * layer + (0: K, 1: V).  Everything but
  // the lane's (head, vector) pair is uniform across the workgroup.
  const unsigned dv = dim / W;
  const unsigned i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= heads * dv) return;
  const unsigned h = i / dv;
  const unsigned c = i - h * dv;
  const bool is_value = (blockIdx.z & 1u) != 0;
  const std::size_t l = blockIdx.z >> 1;
  const float* src = is_value ? values : keys;
  const float sc = is_value ? scale.y : scale.x;
  S* pool = (is_value ? value_pool : key_pool) + l * layer_stride;
  const unsigned rows = count * tokens;
  for (unsigned bt = blockIdx.y; bt < rows; bt += gridDim.y) {
    const std::int64_t slot = slots[bt];
    if (slot < 0) continue;
    const unsigned b = bt / tokens;
    const unsigned t = bt - b * tokens;
    const std::size_t block = static_cast<std::size_t>(slot) / block_tokens;
    const std::size_t off = static_cast<std::size_t>(slot) % block_tokens;
    const std::size_t e = (((l * count + b) * heads + h) * tokens + t) * dv + c;
    Elems<S, W>::put(pool + ((block * heads + h) * block_tokens + off) * dim + c * W, src + e * W,
                     sc);
  }
}

// ---------------------------------------------------------------- rope ----
// Rotary embedding of adjacent pairs (2i, 2i+1) of head vectors, as
// cpu::rope_out (src/kernels/cpu/reference.cpp:490-533): out[2i] =
// x[2i]*cos - x[2i+1]*sin, out[2i+1] = x[2i]*sin + x[2i+1]*cos, every
// product and sum rounded to fp32 on its own (no fused multiply-add), so the
// result is bit-identical to the reference's CPU path.  Up to two tensors
// [rows, vectors, dim] that share the rows' positions go in one launch (a
// decode step's query and key); row r uses cache row positions[r] (or r), and
// a position outside [0, cache_rows) yields a NaN row.  One thread per pair;
// in place is allowed.
struct RopeSegment {
  const float* in;
  float* out;
  unsigned vectors;
};

__global__ void rope_kernel(RopeSegment s0, RopeSegment s1, unsigned rows, unsigned pairs,
                            const float* __restrict__ cosine, const float* __restrict__ sine,
                            const std::int32_t* __restrict__ positions, long long cache_rows) {
  // Products and sums stay separately rounded: no contraction into fma.
#pragma clang fp contract(off)
  const unsigned per_row0 = s0.vectors * pairs;
  const unsigned per_row1 = s1.vectors * pairs;
  const unsigned total0 = rows * per_row0;
  const unsigned total = total0 + rows * per_row1;
  for (unsigned e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += gridDim.x * blockDim.x) {
    const bool second = e >= total0;
    const unsigned f = second ? e - total0 : e;
    const unsigned per_row = second ? per_row1 : per_row0;
    const unsigned r = f / per_row;
    const unsigned rem = f - r * per_row;  // vector * pairs + pair
    const unsigned pair = rem % pairs;
    const long long pos = positions != nullptr ? positions[r] : static_cast<long long>(r);
    const std::size_t off = (static_cast<std::size_t>(r) * per_row + rem) * 2;
    const float2 x = *reinterpret_cast<const float2*>((second ? s1.in : s0.in) + off);
    float2 y;
    if (pos < 0 || pos >= cache_rows) {
      y = make_float2(NAN, NAN);
    } else {
      const std::size_t c_off = static_cast<std::size_t>(pos) * pairs + pair;
      const float c = cosine[c_off];
      const float sn = sine[c_off];
      y.x = x.x * c - x.y * sn;
      y.y = x.x * sn + x.y * c;
    }
    *reinterpret_cast<float2*>((second ? s1.out : s0.out) + off) = y;
  }
}

// Reference: PagedKvCache copy_layer / copy_layer_prefix_out
// (src/kv_cache/paged.cpp:242-280, 895-950).  Tokens [first, first + length)
// of the sequence land at rows [0, length) of the outputs.
template <typename S, int W>
__global__ void gather_kernel(const S* __restrict__ key_pool, const S* __restrict__ value_pool,
                              std::size_t heads, std::size_t block_tokens, std::size_t dim,
                              const std::uint32_t* __restrict__ blocks, std::size_t length,
                              float* keys_out, float* values_out, std::size_t dest_tokens,
                              float2 scale, std::size_t first) {
  const std::size_t dv = dim / W;
  const std::size_t total = heads * length * dv;
  const S* pool = blockIdx.y == 0 ? key_pool : value_pool;
  float* out = blockIdx.y == 0 ? keys_out : values_out;
  const float sc = blockIdx.y == 0 ? scale.x : scale.y;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t c = e % dv;
    const std::size_t ht = e / dv;
    const std::size_t t = ht % length;
    const std::size_t h = ht / length;
    const std::size_t src = first + t;
    const std::size_t phys = blocks[src / block_tokens];
    Elems<S, W>::get(out + (h * dest_tokens + t) * dim + c * W,
                     pool + ((phys * heads + h) * block_tokens + src % block_tokens) * dim + c * W,
                     sc);
  }
}

template <typename S, int W>
__global__ void page_copy_kernel(S* key_base, S* value_base, std::size_t layer_stride,
                                 std::size_t layers, std::size_t heads, std::size_t block_tokens,
                                 std::size_t dim, std::uint32_t from, std::uint32_t to,
                                 std::size_t tokens) {
  const std::size_t dv = dim / W;
  const std::size_t run = tokens * dv;  // contiguous prefix of one (block, head) page
  const std::size_t total = layers * heads * run;
  S* base = blockIdx.y == 0 ? key_base : value_base;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t i = e % run;
    const std::size_t lh = e / run;
    const std::size_t h = lh % heads;
    const std::size_t l = lh / heads;
    const std::size_t page = block_tokens * dim;
    S* layer = base + l * layer_stride;
    Elems<S, W>::copy(layer + (static_cast<std::size_t>(to) * heads + h) * page + i * W,
                      layer + (static_cast<std::size_t>(from) * heads + h) * page + i * W);
  }
}

__global__ void table_update_kernel(std::uint32_t* tables, std::size_t cols,
                                    const std::uint32_t* __restrict__ updates,
                                    std::size_t count) {
  const std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
  if (i < count) {
    tables[static_cast<std::size_t>(updates[3 * i]) * cols + updates[3 * i + 1]] =
        updates[3 * i + 2];
  }
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------- decode ----
// Cross-lane helpers, all VALU (no LDS pipe):
//   DPP within a 16-lane row: row_ror:8 pairs lane i with i ^ 8, row_ror:4
//   with (i + 4) mod 16, the row half-mirror pairs i with 7 - i inside each
//   8-lane group, quad permutes give i ^ 1 and i ^ 2;
//   v_permlane16_swap exchanges the odd 16-lane rows of its first operand
//   with the even rows of its second, v_permlane32_swap the upper 32 lanes of
//   the first with the lower 32 of the second.
constexpr int kDppQuadXor1 = 0xB1;       // quad_perm [1, 0, 3, 2]
constexpr int kDppQuadXor2 = 0x4E;       // quad_perm [2, 3, 0, 1]
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
constexpr int kDppRowHalfMirror = 0x141;

// Raw buffer descriptor word 3 for plain dword access on CDNA.
constexpr int kBufferWord3 = 0x00020000;
// Cache policy of the page loads: non-temporal.  Each page byte is read once
// per launch; marking the loads streaming measured 6.94 TB/s against
// 6.21 TB/s for default loads on a random-order 8 KiB chunk-pair read of
// 45 GiB.
constexpr int kStreamLoad = 2;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 as_float4(u32x4 v) {
  return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]),
                     __uint_as_float(v[3]));
}
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 as_uint2(u32x2 v) { return make_uint2(v[0], v[1]); }


template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float half_xor(float x) { return __shfl_xor(x, 32, 64); }

// Recursive halving: N values per lane; each step keeps the half selected by
// a lane bit and adds the partner lane's copy of that half, so after k steps
// a lane holds N / 2^k values summed over 2^k lanes.  The partner of a step
// must differ from the lane in that step's bit only among the bits used so
// far; the kept value index is the sequence of the lane's bits 4, 3, 2, 1, 0.
template <int N>
__device__ __forceinline__ void halve16(float* x) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x[i]),
                                                    __float_as_uint(x[i + N / 2]), false, false);
    x[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  }
}
template <int N, int CTRL>
__device__ __forceinline__ void halve_dpp(float* x, bool hi) {
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float lo_sum = x[i] + dpp<CTRL>(x[i]);
    const float hi_sum = x[i + N / 2] + dpp<CTRL>(x[i + N / 2]);
    x[i] = hi ? hi_sum : lo_sum;
  }
}

// Reduces 8*G partial dot products (8 tokens x G heads per lane) over the 32
// lanes of a half.  Afterwards lane j holds R = max(1, G/4) complete scores,
// value index v = (j >> DUPB) * R + r (v = local_token * G + head).
template <int G>
__device__ __forceinline__ void reduce_scores(float* x, int j) {
  constexpr int NV = 8 * G;
  halve16<NV>(x);
  halve_dpp<NV / 2, kDppRowRor8>(x, (j & 8) != 0);
  halve_dpp<NV / 4, kDppRowHalfMirror>(x, (j & 4) != 0);
  if constexpr (NV / 8 >= 2) {
    halve_dpp<NV / 8, kDppQuadXor2>(x, (j & 2) != 0);
  } else {
    x[0] += dpp<kDppQuadXor2>(x[0]);
  }
  if constexpr (NV / 16 >= 2) {
    halve_dpp<NV / 16, kDppQuadXor1>(x, (j & 1) != 0);
  } else {
    x[0] += dpp<kDppQuadXor1>(x[0]);
  }
}

// Max / sum over the lanes that hold the same head: the token bits of the
// lane index are bits 2..4 plus the half (bit 5).
__device__ __forceinline__ float token_max(float v) {
  v = fmaxf(v, dpp<kDppRowRor8>(v));
  v = fmaxf(v, dpp<kDppRowRor4>(v));
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float token_sum(float v) {
  v += dpp<kDppRowRor8>(v);
  v += dpp<kDppRowRor4>(v);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

__device__ __forceinline__ float exp2_ratio(float a, float b) {
  // exp2(a - b) with a == b (including +inf == +inf or -inf == -inf) -> 1.
  return a == b ? 1.0f : exp2f(a - b);
}

// The same with v_exp_f32 directly: results below 2^-126 flush to zero, far
// under the tolerance of a probability normalised by a sum >= 1.  Used by
// the stream kernel on bf16 and fp8 pages, whose time follows the
// instruction count per page (it saves exp2f's subnormal-range fix-up, four
// instructions per call).
__device__ __forceinline__ float exp2_ratio_raw(float a, float b) {
  return a == b ? 1.0f : __builtin_amdgcn_exp2f(a - b);
}

struct DecodeKernelArgs {
  const float* query;
  const float* key_pool;
  const float* value_pool;
  const std::uint32_t* tables;
  const std::int32_t* lengths;
  const float* tail_key;
  const float* tail_value;
  float* out;
  float* part_o;        // [batch * kv_heads * max_splits, G, 128]
  float* part_ml;       // [batch * kv_heads * max_splits, G, 2]
  int batch;
  int q_heads;
  int kv_heads;
  int max_blocks;
  int max_splits;
  int pages_per_split;
  std::uint32_t physical_blocks;
  float qscale;
  int stream_waves;     // grid size of the stream kernel (stream mode)
  int* segments;        // [units] (first wavefront, wavefront count), stream mode
  int first_page;       // stream mode: pages before this are covered by the cascade
  long long prefix_slot0;  // cascade: chunk c of unit u at prefix_slot0 + c * units + u
  int prefix_chunks;    // cascade: key chunks of the shared prefix
  // Fused append (stream mode): the tail row of sequence b is also written
  // to physical slot append_slots[b] of these pools (negative: skipped).
  const std::int64_t* append_slots;
  float* append_key_pool;
  float* append_value_pool;
  // fp8 pages: scales of the key and value codes (the key scale is also
  // folded into qscale).
  float k_scale;
  float v_scale;
};

__device__ __forceinline__ int clamp_length(int hist, int max_blocks) {
  return (hist < 0 || hist > max_blocks * 16) ? -1 : hist;
}

// Page splits of one (sequence, kv head) unit; an invalid length (-1)
// attends to the tail only.
__device__ __forceinline__ int unit_splits(int hist, int pages_per_split) {
  const int pages = hist < 0 ? 0 : (hist + 15) / 16;
  const int s = (pages + pages_per_split - 1) / pages_per_split;
  return s < 1 ? 1 : s;
}

// Wave-wide inclusive prefix sum.
__device__ __forceinline__ int wave_incl_scan(int v, int lane) {
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(v, o, 64);
    if (lane >= o) v += t;
  }
  return v;
}

// Split-K decode.  Work items are page splits of the (sequence, kv head)
// units: every full split of every unit first (sequence major), then the
// last split of each unit, which also attends to the uncommitted tail token.
// One wavefront runs one item and the hardware dispatcher hands out items as
// wavefronts retire, so faster waves take more items and the short last
// splits fill the end of the launch.  A unit with one split is finished in
// place; otherwise every split leaves a partial (m, l, o) for
// decode_merge_kernel.  (Merging inside this kernel would need a device-scope
// release per split, which on a multi-XCD part writes back the L2 and costs
// far more than the separate launch.)
//
// The G = q_heads / kv_heads query heads of the unit stay in registers, so
// each K/V byte is read from HBM once per kv head.
//
// Lane layout: lane = 32 * parity + j.  A 128-bit load at float4 index
// i * 64 + lane of a page covers token 2i + parity, dims 4j..4j+3, so each
// load instruction of the wave reads 1 KiB of contiguous page memory.
//
// Per page: partial dots (8 tokens x G heads per lane) -> recursive-halving
// reduction -> online softmax in the exp2 domain (max/sum across token
// lanes) -> probabilities broadcast through LDS -> P.V into 4G accumulators.
//
// Softmax special cases follow src/kernels/cpu/reference.cpp:264-316: a NaN
// score makes the row NaN (it propagates through exp2 into the sum), +inf
// scores take all the mass uniformly (exp2_ratio treats inf == inf as 1 and
// resets finite history), and a row whose maximum stays -inf is NaN.  A page
// ID >= physical_blocks yields NaN, like the reference kernels
// (src/attention/cuda_paged.cu:58-61), and is never dereferenced; so does a
// history length the table row cannot cover.
template <int G>
__global__ __launch_bounds__(64) void decode_split_kernel(DecodeKernelArgs a) {
  constexpr int D = 128;
  constexpr int P = 16;
  constexpr int R = G >= 4 ? G / 4 : 1;
  constexpr int DUPB = G >= 4 ? 0 : (G == 2 ? 1 : 2);
  constexpr int NV = 8 * G;

  __shared__ __align__(16) float s_p[2][NV];
  __shared__ __align__(16) float s_head[3][G];  // alpha / m / l per head

  const int lane = threadIdx.x;
  const int parity = lane >> 5;
  const int j = lane & 31;
  const int item = blockIdx.x;
  const int CP = a.pages_per_split;

  // ---- locate (sequence b, kv head, split) of this item ----------------
  long long fulls = 0;  // full (non-last) split items over all sequences
  for (int c0 = 0; c0 < a.batch; c0 += 64) {
    const int bb = c0 + lane;
    int w = 0;
    if (bb < a.batch) w = (unit_splits(clamp_length(a.lengths[bb], a.max_blocks), CP) - 1) * a.kv_heads;
    fulls += __shfl(wave_incl_scan(w, lane), 63, 64);
  }
  int b = 0, kvh = 0, split = 0;
  if (item < fulls) {
    long long base = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
      const int bb = c0 + lane;
      int w = 0;
      if (bb < a.batch) {
        w = (unit_splits(clamp_length(a.lengths[bb], a.max_blocks), CP) - 1) * a.kv_heads;
      }
      const int incl = wave_incl_scan(w, lane);
      const long long lo = base + incl - w;
      const unsigned long long hit = __ballot(bb < a.batch && lo <= item && item < base + incl);
      if (hit != 0) {
        const int src = __ffsll(static_cast<long long>(hit)) - 1;
        b = c0 + src;
        const long long r = item - __shfl(lo, src, 64);
        const int per = unit_splits(clamp_length(a.lengths[b], a.max_blocks), CP) - 1;
        kvh = static_cast<int>(r / per);
        split = static_cast<int>(r % per);
        break;
      }
      base += __shfl(incl, 63, 64);
    }
  } else {
    const long long r = item - fulls;
    if (r >= static_cast<long long>(a.batch) * a.kv_heads) return;
    b = static_cast<int>(r / a.kv_heads);
    kvh = static_cast<int>(r % a.kv_heads);
    split = unit_splits(clamp_length(a.lengths[b], a.max_blocks), CP) - 1;
  }

  b = __builtin_amdgcn_readfirstlane(b);
  kvh = __builtin_amdgcn_readfirstlane(kvh);
  split = __builtin_amdgcn_readfirstlane(split);
  const int hist = __builtin_amdgcn_readfirstlane(clamp_length(a.lengths[b], a.max_blocks));
  const int hist_ok = hist < 0 ? 0 : hist;
  const int pages = (hist_ok + P - 1) / P;
  const int splits = unit_splits(hist, CP);
  const bool last = split == splits - 1;
  const int pg0 = split * CP;
  const int pg1 = min(pages, pg0 + CP);
  const std::uint32_t* table = a.tables + static_cast<std::size_t>(b) * a.max_blocks;
  const std::size_t qrow0 = static_cast<std::size_t>(b) * a.q_heads + kvh * G;
  const std::size_t page_elems = static_cast<std::size_t>(P) * D;

  float4 q[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    float4 v = reinterpret_cast<const float4*>(a.query + (qrow0 + h) * D)[j];
    q[h] = make_float4(v.x * a.qscale, v.y * a.qscale, v.z * a.qscale, v.w * a.qscale);
  }
  float acc[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.0f;
  float m[R], l[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
  }
  bool bad_page = hist < 0;

  // One page (or the tail as a 1-token page) through score, softmax and P.V.
  auto process = [&](const float4 (&k)[8], float4 (&v)[8], int valid) {
    float xs[NV];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        xs[i * G + h] = q[h].x * k[i].x + q[h].y * k[i].y + q[h].z * k[i].z + q[h].w * k[i].w;
      }
    }
    reduce_scores<G>(xs, j);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int vi = (j >> DUPB) * R + r;
      const int tok = 2 * (vi / G) + parity;
      const bool ok = tok < valid;
      const float s = ok ? xs[r] : -INFINITY;
      const float mn = fmaxf(m[r], token_max(s));
      const float alpha = exp2_ratio(m[r], mn);
      const float p = ok ? exp2_ratio(s, mn) : 0.0f;
      l[r] = l[r] * alpha + token_sum(p);
      m[r] = mn;
      if ((j & ((1 << DUPB) - 1)) == 0) s_p[parity][vi] = p;
      if (parity == 0 && vi < G && (j & ((1 << DUPB) - 1)) == 0) s_head[0][vi] = alpha;
    }
    __syncthreads();
    float pp[NV];
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) {
      const float4 t4 = reinterpret_cast<const float4*>(s_p[parity])[i];
      pp[4 * i] = t4.x;
      pp[4 * i + 1] = t4.y;
      pp[4 * i + 2] = t4.z;
      pp[4 * i + 3] = t4.w;
    }
    float al[G];
#pragma unroll
    for (int h = 0; h < G; ++h) al[h] = s_head[0][h];
    __syncthreads();
    if (valid < P) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        if (2 * i + parity >= valid) v[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      acc[h][0] *= al[h];
      acc[h][1] *= al[h];
      acc[h][2] *= al[h];
      acc[h][3] *= al[h];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pv = pp[i * G + h];
        acc[h][0] += pv * v[i].x;
        acc[h][1] += pv * v[i].y;
        acc[h][2] += pv * v[i].z;
        acc[h][3] += pv * v[i].w;
      }
    }
  };

  // Loads are issued unconditionally (page index clamped by the caller, an
  // out-of-range page ID redirected to page 0 and flagged), so the compiler
  // can count outstanding loads exactly and never drains the queue early.
  auto load_page = [&](int pg, float4 (&k)[8], float4 (&v)[8]) {
    std::uint32_t phys = table[pg];
    if (phys >= a.physical_blocks) {
      bad_page = true;
      phys = 0;
    }
    const std::size_t off = (static_cast<std::size_t>(phys) * a.kv_heads + kvh) * page_elems;
    const float4* kp = reinterpret_cast<const float4*>(a.key_pool + off);
    const float4* vp = reinterpret_cast<const float4*>(a.value_pool + off);
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = kp[i * 64 + lane];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = vp[i * 64 + lane];
  };

  // History pages [pg0, pg1) through a two-buffer ping-pong pipeline: while
  // one page is reduced the loads of the next two are in flight.
  if (pg0 < pg1) {
    float4 ka[8], va[8], kb[8], vb[8];
    load_page(pg0, ka, va);
    load_page(min(pg0 + 1, pg1 - 1), kb, vb);
    for (int pg = pg0; pg < pg1; pg += 2) {
      process(ka, va, min(P, hist_ok - pg * P));
      load_page(min(pg + 2, pg1 - 1), ka, va);
      if (pg + 1 < pg1) process(kb, vb, min(P, hist_ok - (pg + 1) * P));
      load_page(min(pg + 3, pg1 - 1), kb, vb);
    }
  }
  if (last) {
    // The uncommitted current token: lanes of half 0 hold its 128 dims.
    float4 kt[8], vt[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      kt[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      vt[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if (parity == 0) {
      const std::size_t trow = static_cast<std::size_t>(b) * a.kv_heads + kvh;
      kt[0] = reinterpret_cast<const float4*>(a.tail_key + trow * D)[j];
      vt[0] = reinterpret_cast<const float4*>(a.tail_value + trow * D)[j];
    }
    process(kt, vt, 1);
  }

  // Combine the two token halves, then publish m / l per head.
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[h][c] += half_xor(acc[h][c]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int vi = (j >> DUPB) * R + r;
    if (parity == 0 && vi < G && (j & ((1 << DUPB) - 1)) == 0) {
      s_head[1][vi] = m[r];
      s_head[2][vi] = bad_page ? NAN : l[r];
    }
  }
  __syncthreads();

  if (splits == 1) {
    if (parity == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float mh = s_head[1][h];
        const float lh = s_head[2][h];
        float4 o;
        if (mh == -INFINITY) {
          o = make_float4(NAN, NAN, NAN, NAN);
        } else {
          const float inv = 1.0f / lh;
          o = make_float4(acc[h][0] * inv, acc[h][1] * inv, acc[h][2] * inv, acc[h][3] * inv);
        }
        reinterpret_cast<float4*>(a.out + (qrow0 + h) * D)[j] = o;
      }
    }
    return;
  }

  const std::size_t slot = (static_cast<std::size_t>(b) * a.kv_heads + kvh) * a.max_splits + split;
  if (parity == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
      reinterpret_cast<float4*>(a.part_o + (slot * G + h) * D)[j] =
          make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    }
    if (j < G) {
      a.part_ml[(slot * G + j) * 2] = s_head[1][j];
      a.part_ml[(slot * G + j) * 2 + 1] = s_head[2][j];
    }
  }
}

// Merges the split partials of every unit with more than one split:
// O_h = sum_s o_sh 2^(m_sh - M_h) / sum_s l_sh 2^(m_sh - M_h).  One
// workgroup per (sequence, kv head); the per-split weights are formed once
// in LDS, then every thread sums its outputs over the splits with
// independent loads in flight.
template <int G>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecodeKernelArgs a) {
  constexpr int D = 128;
  extern __shared__ float s_w[];  // [G][max_splits] weights, then [G] 1/den
  const int unit = blockIdx.x;
  const int b = unit / a.kv_heads;
  const int hist = clamp_length(a.lengths[b], a.max_blocks);
  const int splits = unit_splits(hist, a.pages_per_split);
  if (splits <= 1) return;
  float* s_inv = s_w + G * a.max_splits;
  __shared__ float s_max[G];
  const std::size_t slot0 = static_cast<std::size_t>(unit) * a.max_splits;
  const int tid = threadIdx.x;
  // Per head: the largest split maximum (one wave per head, G <= 8 heads
  // over four waves).
  for (int h = tid / 64; h < G; h += 4) {
    float mx = -INFINITY;
    for (int s = tid % 64; s < splits; s += 64) mx = fmaxf(mx, a.part_ml[((slot0 + s) * G + h) * 2]);
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (tid % 64 == 0) s_max[h] = mx;
  }
  __syncthreads();
  for (int t = tid; t < G * splits; t += 256) {
    const int h = t / splits;
    const int s = t % splits;
    s_w[h * a.max_splits + s] = exp2_ratio(a.part_ml[((slot0 + s) * G + h) * 2], s_max[h]);
  }
  __syncthreads();
  for (int h = tid / 64; h < G; h += 4) {
    float den = 0.0f;
    for (int s = tid % 64; s < splits; s += 64) {
      den += s_w[h * a.max_splits + s] * a.part_ml[((slot0 + s) * G + h) * 2 + 1];
    }
    for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
    if (tid % 64 == 0) s_inv[h] = s_max[h] == -INFINITY ? NAN : 1.0f / den;
  }
  __syncthreads();
  const std::size_t qrow0 = static_cast<std::size_t>(b) * a.q_heads +
                            static_cast<std::size_t>(unit % a.kv_heads) * G;
  for (int t = tid; t < G * (D / 4); t += 256) {
    const int h = t / (D / 4);
    const int d4 = t % (D / 4);
    const float* w = s_w + h * a.max_splits;
    float4 n0 = make_float4(0.f, 0.f, 0.f, 0.f), n1 = n0;
    int s = 0;
    for (; s + 1 < splits; s += 2) {
      const float4 o0 = reinterpret_cast<const float4*>(a.part_o + ((slot0 + s) * G + h) * D)[d4];
      const float4 o1 =
          reinterpret_cast<const float4*>(a.part_o + ((slot0 + s + 1) * G + h) * D)[d4];
      n0.x += w[s] * o0.x; n0.y += w[s] * o0.y; n0.z += w[s] * o0.z; n0.w += w[s] * o0.w;
      n1.x += w[s + 1] * o1.x; n1.y += w[s + 1] * o1.y;
      n1.z += w[s + 1] * o1.z; n1.w += w[s + 1] * o1.w;
    }
    if (s < splits) {
      const float4 o0 = reinterpret_cast<const float4*>(a.part_o + ((slot0 + s) * G + h) * D)[d4];
      n0.x += w[s] * o0.x; n0.y += w[s] * o0.y; n0.z += w[s] * o0.z; n0.w += w[s] * o0.w;
    }
    const float inv = s_inv[h];
    reinterpret_cast<float4*>(a.out + (qrow0 + h) * D)[d4] =
        make_float4((n0.x + n1.x) * inv, (n0.y + n1.y) * inv, (n0.z + n1.z) * inv,
                    (n0.w + n1.w) * inv);
  }
}

// ------------------------------------------------------ stream decode ----
// Persistent decode: the grid is one wavefront per resident slot, and the
// work is the flat list of pages of all (sequence, kv head) units, kv head
// major (unit index kvh * batch + b), each unit contributing its history
// pages plus one pseudo-page for the uncommitted tail.  Kv-head-major order
// keeps the wavefronts that run side by side on different sequences, i.e.
// on unrelated physical blocks, rather than on the neighbouring kv-head
// pages of one block.  Wavefront w takes the contiguous range
// [w * C, (w + 1) * C) of that list, C = ceil(total / waves), so every
// wavefront moves the same bytes and keeps its two-page prefetch running
// across unit boundaries: a wavefront pays the start-up latency (length
// scan, table, first pages) once per launch instead of once per split, and
// the launch has no tail of short items.  Each page buffer carries its
// unit's query rows, so switching units never waits on a load.
//
// A unit that one wavefront covers completely is finished in place.
// Otherwise each wavefront touching unit u leaves a partial at slot u + w;
// the slots of one unit are contiguous (u + w_first .. u + w_last) and no two
// units share a slot, since the next unit starts at or after w_last.
// decode_stream_merge_kernel combines them.
// Stream-mode pages of a unit: its history pages from `first` on, plus the
// tail pseudo-page.
__device__ __forceinline__ int unit_pages(int hist, int first) {
  const int pages = (hist < 0 ? 0 : (hist + 15) / 16) - first;
  return (pages < 0 ? 0 : pages) + 1;
}

// Marks a wave-uniform 64-bit value as such (scalar registers), so control
// flow on it stays uniform and dependent loads stay scalar.
__device__ __forceinline__ long long uniform64(long long v) {
  const unsigned lo = __builtin_amdgcn_readfirstlane(static_cast<unsigned>(v));
  const unsigned hi =
      __builtin_amdgcn_readfirstlane(static_cast<unsigned>(static_cast<unsigned long long>(v) >> 32));
  return static_cast<long long>((static_cast<unsigned long long>(hi) << 32) | lo);
}

__device__ __forceinline__ long long wave_sum(long long v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Pages of sequences [from, upto) for one kv head: sum of unit_pages.
__device__ __forceinline__ long long stream_pages_between(const DecodeKernelArgs& a, int from,
                                                          int upto, int lane) {
  long long sum = 0;
  for (int c0 = from; c0 < upto; c0 += 64) {
    const int bb = c0 + lane;
    const int w = bb < upto ? unit_pages(clamp_length(a.lengths[bb], a.max_blocks), a.first_page) : 0;
    sum += wave_sum(w);
  }
  return sum;
}

struct PageDesc {
  int b, kvh, p, np, hist;
  long long g;
  bool skip;
};

// PF (page format, the PageType value): fp32 pages (0); bf16 pages (1, 4
// per 64-bit lane load); fp8 E4M3 pages (2, 4 per 32-bit lane load).
// Reduced-precision pages stay packed in registers and each row is widened
// where it is used.  The fp32 tail row is rounded onto the page grid as it
// is read (it is the value the page will hold once appended).  fp8 scales:
// the key scale is folded into the score scale on the host and the value
// scale is applied to each result, so rows widen to bare code values.
// LDS of one stream wavefront.  Results are staged until the wavefront's
// last page: on this architecture a store counts in the same in-order
// counter as the loads, so a store issued between prefetches would make the
// next page's wait also wait for the store to complete; staging keeps every
// global store after the last load.  A full stage is flushed early (many
// short units per wavefront).
constexpr int kStreamStage = 4;
// fp8 stream wavefronts: four per SIMD with a one-deep result stage (the
// extra wavefront hides more per-page latency than its spills cost).
constexpr int kFp8StreamWaves = 4;
constexpr int kFp8StreamStage = 1;


// One token row's 4 dims of a page buffer as fp32: fp32 pages as loaded,
// bf16 pages (4 per 64-bit lane load) widened where the row is used, so a
// buffer never holds a widened copy of its page.
__device__ __forceinline__ float4 page_row(const float4& x) { return x; }
// First word of an fp8 page buffer row (the LDS query path orders on it).
__device__ __forceinline__ unsigned first_word(const unsigned& x) { return x; }
__device__ __forceinline__ float4 page_row(const uint2& x) { return bf16_widen(x.x, x.y); }
__device__ __forceinline__ float4 page_row(const unsigned& x) { return fp8_widen4(x, 1.0f); }
__device__ __forceinline__ float4 masked_row(const float4& x, bool keep) {
  return make_float4(keep ? x.x : 0.0f, keep ? x.y : 0.0f, keep ? x.z : 0.0f, keep ? x.w : 0.0f);
}
__device__ __forceinline__ unsigned masked_row(const unsigned& x, bool keep) { return keep ? x : 0u; }
// A tail row as staged for its page write: fp32 and bf16 rows as values
// (bf16-exact, repacked without rounding), fp8 rows as their codes in .x.
__device__ __forceinline__ float4 staged_row(const float4& x) { return x; }
__device__ __forceinline__ float4 staged_row(const uint2& x) { return page_row(x); }
__device__ __forceinline__ float4 staged_row(const unsigned& x) {
  return make_float4(__uint_as_float(x), 0.0f, 0.0f, 0.0f);
}
__device__ __forceinline__ uint2 masked_row(const uint2& x, bool keep) {
  return make_uint2(keep ? x.x : 0u, keep ? x.y : 0u);
}
template <int G>
struct StreamShared {
  __align__(16) float p[2][8 * G];
  __align__(16) float head[3][G];
  __align__(16) float4 res_o[kStreamStage][G][32];
  float res_ml[kStreamStage][G][2];
  long long res_dst[kStreamStage];  // >= 0: first output row; < 0: -1 - partial slot
  int2 seg[kStreamStage];
  int seg_unit[kStreamStage];
  __align__(16) float4 app_k[kStreamStage][32];
  __align__(16) float4 app_v[kStreamStage][32];
  long long app_dst[kStreamStage];  // element offset of the row, < 0: none
};

// References to one stream wavefront's LDS arrays.  The stream kernel binds
// them to separate __shared__ arrays: as distinct objects they are known not
// to overlap, which the dynamically indexed fields of one struct are not
// (the struct form cost 70 extra LDS reads and spills in the loop).
// S: results staged before a flush.  qslot: query rows loaded straight
// into LDS, one area per page buffer (reduced-precision pages), or null.
template <int G, int S = kStreamStage>
struct StreamLds {
  float (&p)[2][8 * G];
  float (&head)[3][G];
  float4 (&res_o)[S][G][32];
  float (&res_ml)[S][G][2];
  long long (&res_dst)[S];
  int2 (&seg)[S];
  int (&seg_unit)[S];
  float4 (&app_k)[S][32];
  float4 (&app_v)[S][32];
  long long (&app_dst)[S];
  float4 (*qslot)[G][32];
};
template <int G>
__device__ __forceinline__ StreamLds<G> stream_lds(StreamShared<G>& s) {
  return StreamLds<G>{s.p, s.head, s.res_o, s.res_ml, s.res_dst,
                      s.seg, s.seg_unit, s.app_k, s.app_v, s.app_dst, nullptr};
}

// fp8 pages in the stream kernel: query rows loaded straight into LDS (three
// areas used by units in turn) and read from there at every page, with no register
// copy; one result staged; four wavefronts per SIMD, which their small page
// buffers then allow (119-127 VGPRs, at most 2 spilled).  Config 3, one
// box: 104.0 us per layer against 108.5 with a register copy per unit
// (6-13 spilled), 116.3 with three wavefronts and two staged results and
// 140.4 with two wavefronts.  bf16 pages stay at two wavefronts: with the
// same arrangement three ran 128.4-128.8 against 125.4 us (161 VGPRs, no
// spills) and four 161.6 us (21-27 spilled).
constexpr bool stream_lds_query_type(PageType t) { return t == PageType::kFP8; }
template <int PF, int G>
constexpr bool stream_lds_query() {
  return G <= 4 && stream_lds_query_type(static_cast<PageType>(PF));
}

// LDS hand-off inside one wavefront.  In the stream kernel a workgroup is a
// single wavefront, so a workgroup barrier is that; when several independent
// stream wavefronts share a workgroup (the fused cascade launch) each orders
// only its own LDS accesses, which execute in order within a wavefront.
template <bool SHARED_BLOCK>
__device__ __forceinline__ void stream_sync() {
  if constexpr (SHARED_BLOCK) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  } else {
    __syncthreads();
  }
}

// The body of one stream wavefront: `wave` is its index among
// a.stream_waves, `lane` its lane, `sh` its LDS.
template <int G, bool APPEND, int PF, bool SHARED_BLOCK, int S = kStreamStage>
__device__ __forceinline__ void decode_stream_body(
    DecodeKernelArgs a, const std::uint32_t* __restrict__ tables,
    const std::int32_t* __restrict__ lengths, float* __restrict__ out,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ segments,
    const std::int64_t* __restrict__ append_slots, int wave, int lane, StreamLds<G, S> sh) {
  // The block table and lengths are read-only here and do not alias the
  // outputs; with the restrict-qualified parameters their uniform reads
  // become scalar loads.
  a.tables = tables;
  a.lengths = lengths;
  a.out = out;
  a.part_o = part_o;
  a.part_ml = part_ml;
  a.segments = segments;
  a.append_slots = APPEND ? append_slots : nullptr;
  constexpr int D = 128;
  constexpr int P = 16;
  constexpr int R = G >= 4 ? G / 4 : 1;
  constexpr int DUPB = G >= 4 ? 0 : (G == 2 ? 1 : 2);
  constexpr int NV = 8 * G;
  constexpr int kStage = S;
  constexpr bool QLDS = !SHARED_BLOCK && stream_lds_query<PF, G>();
  // fp8 and bf16 pages, and stream wavefronts beside prefix workgroups: the
  // raw exp2 and a ballot for the rescale test (measured: config 3 fp8
  // 110.7 -> 108.4 us per layer, config 4 fused cascade 79.9 -> 79.3 us;
  // bf16 within its box-to-box spread; the plain fp32 stream kernel, bound
  // by HBM, showed no gain and keeps exp2f).
  constexpr bool LEAN = PF != 0 || SHARED_BLOCK;
  auto& s_p = sh.p;
  auto& s_head = sh.head;
  auto& s_res_o = sh.res_o;
  auto& s_res_ml = sh.res_ml;
  auto& s_res_dst = sh.res_dst;
  auto& s_seg = sh.seg;
  auto& s_seg_unit = sh.seg_unit;
  auto& s_app_k = sh.app_k;
  auto& s_app_v = sh.app_v;
  auto& s_app_dst = sh.app_dst;

  const int parity = lane >> 5;
  const int j = lane & 31;

  // The lengths of the first kScanChunks * 64 sequences are loaded at once
  // (lane l holds sequences l, l + 64, ...), so finding the first unit costs
  // one load latency; only larger batches load further chunks in turn.
  constexpr int kScanChunks = 4;
  int histc[kScanChunks];
  int npc[kScanChunks];
#pragma unroll
  for (int c = 0; c < kScanChunks; ++c) {
    const int bb = c * 64 + lane;
    histc[c] = bb < a.batch ? clamp_length(a.lengths[bb], a.max_blocks) : -1;
  }
  long long lane_pages = 0;
#pragma unroll
  for (int c = 0; c < kScanChunks; ++c) {
    npc[c] = c * 64 + lane < a.batch ? unit_pages(histc[c], a.first_page) : 0;
    lane_pages += npc[c];
  }
  long long per_head = wave_sum(lane_pages);
  if (a.batch > kScanChunks * 64) {
    per_head += stream_pages_between(a, kScanChunks * 64, a.batch, lane);
  }
  per_head = uniform64(per_head);
  const long long total = per_head * a.kv_heads;
  const long long C = uniform64((total + a.stream_waves - 1) / a.stream_waves);
  const long long g0 = uniform64(static_cast<long long>(wave) * C);
  if (g0 >= total) return;
  const long long g1 = uniform64(g0 + C < total ? g0 + C : total);

  // Unit and page of g0: kv head = g0 / per_head, then scan sequences.
  PageDesc cur{};
  cur.kvh = static_cast<int>(g0 / per_head);
  {
    const long long rem0 = g0 - static_cast<long long>(cur.kvh) * per_head;
    long long base = 0;
    for (int c0 = 0; c0 < a.batch; c0 += 64) {
      const int bb = c0 + lane;
      int hist, np;
      if (c0 < kScanChunks * 64) {
        // Select the preloaded chunk (wave-uniform index into registers).
        hist = histc[0];
        np = npc[0];
#pragma unroll
        for (int c = 1; c < kScanChunks; ++c) {
          if (c0 == c * 64) {
            hist = histc[c];
            np = npc[c];
          }
        }
      } else {
        hist = bb < a.batch ? clamp_length(a.lengths[bb], a.max_blocks) : -1;
        np = bb < a.batch ? unit_pages(hist, a.first_page) : 0;
      }
      long long incl = np;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const long long t = __shfl_up(incl, o, 64);
        if (lane >= o) incl += t;
      }
      const unsigned long long hit =
          __ballot(bb < a.batch && base + incl - np <= rem0 && rem0 < base + incl);
      if (hit != 0) {
        const int src = __ffsll(static_cast<long long>(hit)) - 1;
        cur.b = c0 + src;
        cur.p = static_cast<int>(rem0 - (base + __shfl(incl - np, src, 64)));
        cur.np = __shfl(np, src, 64);
        cur.hist = __shfl(hist, src, 64);
        break;
      }
      base += __shfl(incl, 63, 64);
    }
  }
  cur.b = __builtin_amdgcn_readfirstlane(cur.b);
  cur.kvh = __builtin_amdgcn_readfirstlane(cur.kvh);
  cur.p = __builtin_amdgcn_readfirstlane(cur.p);
  cur.np = __builtin_amdgcn_readfirstlane(cur.np);
  cur.hist = __builtin_amdgcn_readfirstlane(cur.hist);
  cur.g = g0;
  cur.skip = false;

  const std::size_t page_elems = static_cast<std::size_t>(P) * D;
  PageDesc last = cur;
  // Descriptor of the next page to load; past the range it repeats the last
  // real page (a valid address) marked skip.
  auto next_desc = [&]() -> PageDesc {
    if (cur.g >= g1) {
      PageDesc d = last;
      d.skip = true;
      return d;
    }
    PageDesc d = cur;
    last = cur;
    ++cur.g;
    if (++cur.p == cur.np) {
      cur.p = 0;
      if (++cur.b == a.batch) {
        cur.b = 0;
        ++cur.kvh;
      }
      if (cur.g < g1) {
        cur.b = __builtin_amdgcn_readfirstlane(cur.b);
        cur.hist = __builtin_amdgcn_readfirstlane(
            clamp_length(a.lengths[cur.b], a.max_blocks));
        cur.np = unit_pages(cur.hist, a.first_page);
      }
    }
    return d;
  };

  // Loads of one page (or the tail row, every lane reading its 4 dims for
  // all 8 slots) through per-page buffer descriptors: the lane offset is a
  // constant register and the slot offset a scalar, so no per-load address
  // arithmetic is needed.  The first page of a unit in this wavefront also
  // brings the unit's query rows, issued ahead of the page so that waiting
  // for the page covers them.
  constexpr bool BF16 = PF == 1;
  constexpr bool FP8 = PF == 2;
  const int lane_off = lane * (FP8 ? 4 : BF16 ? 8 : 16);
  const int row_off = j * 16;
  using Raw = std::conditional_t<FP8, unsigned, std::conditional_t<BF16, uint2, float4>>;
  // Query rows through LDS: a unit's rows go to area (kvh * batch + b) % 3.
  // Units are visited in that flat order, every unit has a page (its
  // tail) and loads run two pages ahead, so the unit that reuses an area
  // (three units later) starts loading at least one page after the last
  // read of the area's previous rows.  (Two areas would already reload an
  // area only after its last read in program order; the third adds a page
  // of margin.)
  auto query_area = [&](const PageDesc& d) {
    return static_cast<int>(
        static_cast<unsigned>(__builtin_amdgcn_readfirstlane(d.kvh * a.batch + d.b)) % 3u);
  };
  // slot: the page buffer (0 or 1).
  auto load_page = [&](const PageDesc& d, Raw (&k)[8], Raw (&v)[8], float4 (&q)[G], bool& bad,
                       int slot) {
    const int b = __builtin_amdgcn_readfirstlane(d.b);
    const int kvh = __builtin_amdgcn_readfirstlane(d.kvh);
    const int p = __builtin_amdgcn_readfirstlane(d.p);
    const bool tail = p == __builtin_amdgcn_readfirstlane(d.np) - 1;
    const void* kb;
    const void* vb;
    bad = d.hist < 0;
    if (tail) {
      const std::size_t row = (static_cast<std::size_t>(b) * a.kv_heads + kvh) * D;
      kb = a.tail_key + row;
      vb = a.tail_value + row;
    } else {
      std::uint32_t phys = __builtin_amdgcn_readfirstlane(
          a.tables[static_cast<std::size_t>(b) * a.max_blocks + p + a.first_page]);
      if (phys >= a.physical_blocks) {
        bad = true;
        phys = 0;
      }
      const std::size_t off = (static_cast<std::size_t>(phys) * a.kv_heads + kvh) * page_elems;
      if constexpr (FP8) {
        kb = reinterpret_cast<const unsigned char*>(a.key_pool) + off;
        vb = reinterpret_cast<const unsigned char*>(a.value_pool) + off;
      } else if constexpr (BF16) {
        kb = reinterpret_cast<const unsigned short*>(a.key_pool) + off;
        vb = reinterpret_cast<const unsigned short*>(a.value_pool) + off;
      } else {
        kb = a.key_pool + off;
        vb = a.value_pool + off;
      }
    }
    if (p == 0 || d.g == g0) {
      const float* qsrc = a.query + (static_cast<std::size_t>(b) * a.q_heads + kvh * G) * D;
      if constexpr (QLDS) {
        // The G rows (G * 32 vectors of 16 bytes) straight into this
        // buffer's LDS area, issued ahead of the page: the wait for the
        // page's first key load covers them.
#pragma unroll
        for (int i = 0; i < (G * 32 + 63) / 64; ++i) {
          if (i * 64 + lane < G * 32) {
            prefill_detail::lds_load16(qsrc + (i * 64 + lane) * 4,
                                       prefill_detail::lds_address(&sh.qslot[query_area(d)][0][0]) +
                                           i * 1024);
          }
        }
      } else {
        const __amdgpu_buffer_rsrc_t qr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(qsrc), 0, d.skip ? 0 : G * D * 4, kBufferWord3);
#pragma unroll
        for (int h = 0; h < G; ++h) q[h] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(qr, row_off, h * D * 4, 0));
      }
    }
    // A skip descriptor (past the end of the range) gets an empty buffer
    // range: its loads return zeros without touching memory, and the step
    // that consumes them does nothing.  The instruction stream is the same
    // either way, so the prefetch waits stay static.
    const int bytes =
        d.skip ? 0 : (tail ? D * 4 : P * D * static_cast<int>(sizeof(float) >> (FP8 ? 2 : BF16 ? 1 : 0)));
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(kb), 0, bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(vb), 0, bytes, kBufferWord3);
    if constexpr (FP8) {
      if (tail) {
        // The fp32 row's 4 dims of this lane: four 32-bit words in slots 0-3.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          k[i] = __builtin_amdgcn_raw_buffer_load_b32(kr, row_off, i * 4, 0);
          v[i] = __builtin_amdgcn_raw_buffer_load_b32(vr, row_off, i * 4, 0);
        }
#pragma unroll
        for (int i = 4; i < 8; ++i) k[i] = v[i] = 0u;
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) k[i] = __builtin_amdgcn_raw_buffer_load_b32(kr, lane_off, i * 256, kStreamLoad);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b32(vr, lane_off, i * 256, kStreamLoad);
      }
    } else if constexpr (BF16) {
      if (tail) {
        // The fp32 row's 4 dims of this lane: two 64-bit halves in slots 0, 1.
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          k[i] = as_uint2(__builtin_amdgcn_raw_buffer_load_b64(kr, row_off, i * 8, 0));
          v[i] = as_uint2(__builtin_amdgcn_raw_buffer_load_b64(vr, row_off, i * 8, 0));
        }
#pragma unroll
        for (int i = 2; i < 8; ++i) k[i] = v[i] = make_uint2(0u, 0u);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) k[i] = as_uint2(__builtin_amdgcn_raw_buffer_load_b64(kr, lane_off, i * 512, kStreamLoad));
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = as_uint2(__builtin_amdgcn_raw_buffer_load_b64(vr, lane_off, i * 512, kStreamLoad));
      }
    } else {
      const int voff = tail ? row_off : lane_off;
      const int step = tail ? 0 : 1024;
#pragma unroll
      for (int i = 0; i < 8; ++i) k[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(kr, voff, i * step, kStreamLoad));
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(vr, voff, i * step, kStreamLoad));
    }
  };

  float acc[G][4];
  float m[R], l[R];
  bool unit_bad = false;
  auto reset = [&]() {
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      m[r] = -INFINITY;
      l[r] = 0.0f;
    }
    unit_bad = false;
  };
  reset();

  auto process = [&](const auto& k, auto& v, const float4 (&q)[G], int valid) {
    float xs[NV];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 ki = page_row(k[i]);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        xs[i * G + h] = q[h].x * ki.x + q[h].y * ki.y + q[h].z * ki.z + q[h].w * ki.w;
      }
    }
    reduce_scores<G>(xs, j);
    bool moved = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int vi = (j >> DUPB) * R + r;
      const int tok = 2 * (vi / G) + parity;
      const bool ok = tok < valid;
      const float s = ok ? xs[r] * a.qscale : -INFINITY;
      const float mn = fmaxf(m[r], token_max(s));
      const float alpha = LEAN ? exp2_ratio_raw(m[r], mn) : exp2_ratio(m[r], mn);
      const float pr = ok ? (LEAN ? exp2_ratio_raw(s, mn) : exp2_ratio(s, mn)) : 0.0f;
      l[r] = l[r] * alpha + token_sum(pr);
      moved = moved || !(mn == m[r]);
      m[r] = mn;
      if ((j & ((1 << DUPB) - 1)) == 0) s_p[parity][vi] = pr;
      if (parity == 0 && vi < G && (j & ((1 << DUPB) - 1)) == 0) s_head[0][vi] = alpha;
    }
    stream_sync<SHARED_BLOCK>();
    float pp[NV];
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) {
      const float4 t4 = reinterpret_cast<const float4*>(s_p[parity])[i];
      pp[4 * i] = t4.x;
      pp[4 * i + 1] = t4.y;
      pp[4 * i + 2] = t4.z;
      pp[4 * i + 3] = t4.w;
    }
    float al[G];
#pragma unroll
    for (int h = 0; h < G; ++h) al[h] = s_head[0][h];
    stream_sync<SHARED_BLOCK>();
    if (valid < P) {  // wave-uniform: only partial pages and the tail
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = masked_row(v[i], 2 * i + parity < valid);
    }
    // Some head's factor differs from 1 only where its running maximum
    // moved (a factor that rounds to 1 leaves acc unchanged either way).
    bool rescale = false;
    if constexpr (LEAN) {
      rescale = __ballot(moved) != 0;
    } else {
#pragma unroll
      for (int h = 0; h < G; ++h) rescale = rescale || al[h] != 1.0f;
    }
    if (rescale) {  // wave-uniform: some head's running maximum moved
#pragma unroll
      for (int h = 0; h < G; ++h) {
        acc[h][0] *= al[h];
        acc[h][1] *= al[h];
        acc[h][2] *= al[h];
        acc[h][3] *= al[h];
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float4 vi = page_row(v[i]);
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pv = pp[i * G + h];
        acc[h][0] += pv * vi.x;
        acc[h][1] += pv * vi.y;
        acc[h][2] += pv * vi.z;
        acc[h][3] += pv * vi.w;
      }
    }
  };

  int nres = 0;
  int nseg = 0;
  int napp = 0;
  auto flush = [&]() {
    for (int r = 0; r < (APPEND ? napp : 0); ++r) {
      const long long dst = s_app_dst[r];
      if (parity == 0 && dst >= 0) {
        if constexpr (FP8) {
          // Staged rows hold the codes in .x.
          reinterpret_cast<unsigned*>(reinterpret_cast<unsigned char*>(a.append_key_pool) + dst)[j] =
              __float_as_uint(s_app_k[r][j].x);
          reinterpret_cast<unsigned*>(reinterpret_cast<unsigned char*>(a.append_value_pool) + dst)[j] =
              __float_as_uint(s_app_v[r][j].x);
        } else if constexpr (BF16) {
          // Staged values are already bf16-exact: packing does not round.
          const float4 kk = s_app_k[r][j];
          const float4 vv = s_app_v[r][j];
          reinterpret_cast<uint2*>(reinterpret_cast<unsigned short*>(a.append_key_pool) + dst)[j] =
              make_uint2(bf16_pack(kk.x, kk.y), bf16_pack(kk.z, kk.w));
          reinterpret_cast<uint2*>(reinterpret_cast<unsigned short*>(a.append_value_pool) + dst)[j] =
              make_uint2(bf16_pack(vv.x, vv.y), bf16_pack(vv.z, vv.w));
        } else {
          reinterpret_cast<float4*>(a.append_key_pool + dst)[j] = s_app_k[r][j];
          reinterpret_cast<float4*>(a.append_value_pool + dst)[j] = s_app_v[r][j];
        }
      }
    }
    for (int r = 0; r < nres; ++r) {
      const long long dst = s_res_dst[r];
      if (parity == 0) {
        if (dst >= 0) {
#pragma unroll
          for (int h = 0; h < G; ++h) {
            reinterpret_cast<float4*>(a.out + (static_cast<std::size_t>(dst) + h) * D)[j] =
                s_res_o[r][h][j];
          }
        } else {
          const std::size_t slot = static_cast<std::size_t>(-1 - dst);
#pragma unroll
          for (int h = 0; h < G; ++h) {
            reinterpret_cast<float4*>(a.part_o + (slot * G + h) * D)[j] = s_res_o[r][h][j];
          }
          if (j < G) {
            a.part_ml[(slot * G + j) * 2] = s_res_ml[r][j][0];
            a.part_ml[(slot * G + j) * 2 + 1] = s_res_ml[r][j][1];
          }
        }
      }
    }
    if (lane == 0) {
      for (int r = 0; r < nseg; ++r) reinterpret_cast<int2*>(a.segments)[s_seg_unit[r]] = s_seg[r];
    }
    nres = 0;
    nseg = 0;
    napp = 0;
    stream_sync<SHARED_BLOCK>();
  };

  // Publishes the unit's result: the output itself when this wavefront saw
  // the whole unit, else a partial (m, l, o) at slot unit + wave.
  auto finalize = [&](const PageDesc& d) {
#pragma unroll
    for (int h = 0; h < G; ++h) {
#pragma unroll
      for (int c = 0; c < 4; ++c) acc[h][c] += half_xor(acc[h][c]);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int vi = (j >> DUPB) * R + r;
      if (parity == 0 && vi < G && (j & ((1 << DUPB) - 1)) == 0) {
        s_head[1][vi] = m[r];
        s_head[2][vi] = unit_bad ? NAN : l[r];
      }
    }
    if (nres == kStage) flush();
    stream_sync<SHARED_BLOCK>();
    const std::size_t unit = static_cast<std::size_t>(d.kvh) * a.batch + d.b;
    // With a cascade prefix every unit also has a prefix partial to merge.
    const bool complete = a.first_page == 0 && d.p == d.np - 1 && d.g - d.p >= g0;
    if (parity == 0) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        float4 o = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
        if constexpr (FP8) o = make_float4(o.x * a.v_scale, o.y * a.v_scale, o.z * a.v_scale, o.w * a.v_scale);
        if (complete) {
          const float mh = s_head[1][h];
          const float lh = s_head[2][h];
          if (mh == -INFINITY) {
            o = make_float4(NAN, NAN, NAN, NAN);
          } else {
            const float inv = 1.0f / lh;
            o = make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
          }
        }
        s_res_o[nres][h][j] = o;
      }
      if (j < G) {
        s_res_ml[nres][j][0] = s_head[1][j];
        s_res_ml[nres][j][1] = s_head[2][j];
      }
    }
    if (lane == 0) {
      s_res_dst[nres] = complete
                            ? static_cast<long long>(static_cast<std::size_t>(d.b) * a.q_heads +
                                                     d.kvh * G)
                            : -1 - static_cast<long long>(unit + wave);
    }
    ++nres;
    stream_sync<SHARED_BLOCK>();
    reset();
  };

  float4 qc[G];  // query rows of the unit being processed
  auto step_body = [&](const PageDesc& d, const auto& k, auto& v, const float4 (&qn)[G], int slot,
                       bool bad) {
    int valid = 0;
    if (!d.skip) {
      valid = d.p == d.np - 1 ? 1 : min(P, d.hist - (d.p + a.first_page) * P);
      unit_bad = unit_bad || bad;
      if constexpr (!QLDS) {
        if (d.p == 0 || d.g == g0) {
#pragma unroll
          for (int h = 0; h < G; ++h) qc[h] = qn[h];
        }
      }
      if (d.p == 0) {
        // This wavefront holds the unit's first page: record which
        // wavefronts hold its partials for the merge.
        if (nseg == kStage) flush();
        if (lane == 0) {
          const long long last_wave = (d.g + d.np - 1) / C;
          s_seg[nseg] = make_int2(wave, static_cast<int>(last_wave - wave + 1));
          s_seg_unit[nseg] = d.kvh * a.batch + d.b;
        }
        ++nseg;
      }
      if (APPEND && d.p == d.np - 1) {
        // The tail row is this step's new token: stage its page write.
        if (napp == kStage) flush();
        if (parity == 0) {
          s_app_k[napp][j] = staged_row(k[0]);
          s_app_v[napp][j] = staged_row(v[0]);
        }
        if (lane == 0) {
          const std::int64_t slot = a.append_slots[d.b];
          s_app_dst[napp] =
              slot < 0 ? -1
                       : ((slot / P * static_cast<long long>(a.kv_heads) + d.kvh) * P + slot % P) * D;
        }
        ++napp;
        stream_sync<SHARED_BLOCK>();
      }
    }
    if constexpr (QLDS) {
      // The query rows are read from the unit's LDS area at every page, so
      // no register copy lives across the unit's pages.  The index depends
      // (through an empty asm) on the page's first key word, so the read
      // waits for that load, which was issued after the unit's query loads.
      int dep = 0;
      asm volatile("" : "+v"(dep) : "v"(first_word(k[0])));
      float4 qv[G];
      const int qa = query_area(d);
#pragma unroll
      for (int h = 0; h < G; ++h) qv[h] = sh.qslot[qa][h][j + dep];
      process(k, v, qv, valid);
    } else {
      process(k, v, qc, valid);
    }
    if (!d.skip && (d.p == d.np - 1 || d.g == g1 - 1)) finalize(d);
  };
  auto step = [&](const PageDesc& d, Raw (&kr)[8], Raw (&vr)[8], const float4 (&qn)[G], bool bad,
                  int slot) {
    if constexpr (FP8) {
      if (!d.skip && d.p == d.np - 1) {
        // The tail row arrived as fp32 in slots 0-3: its codes (the values
        // its page will hold) go to slot 0 like a page row.
        kr[0] = fp8_pack4(__uint_as_float(kr[0]) / a.k_scale, __uint_as_float(kr[1]) / a.k_scale,
                          __uint_as_float(kr[2]) / a.k_scale, __uint_as_float(kr[3]) / a.k_scale);
        vr[0] = fp8_pack4(__uint_as_float(vr[0]) / a.v_scale, __uint_as_float(vr[1]) / a.v_scale,
                          __uint_as_float(vr[2]) / a.v_scale, __uint_as_float(vr[3]) / a.v_scale);
      }
    }
    if constexpr (BF16) {
      if (!d.skip && d.p == d.np - 1) {
        // The tail row arrived as fp32 in slots 0 and 1: round it onto the
        // bf16 grid (the value its page will hold) and pack it into slot 0
        // like a page row; the other slots are masked.
        kr[0] = make_uint2(bf16_pack(__uint_as_float(kr[0].x), __uint_as_float(kr[0].y)),
                           bf16_pack(__uint_as_float(kr[1].x), __uint_as_float(kr[1].y)));
        vr[0] = make_uint2(bf16_pack(__uint_as_float(vr[0].x), __uint_as_float(vr[0].y)),
                           bf16_pack(__uint_as_float(vr[1].x), __uint_as_float(vr[1].y)));
      }
    }
    step_body(d, kr, vr, qn, slot, bad);
  };

  // Two pages in flight, each in its own register buffer.  More did not
  // help the reduced-precision pages, whose kernels are held by their
  // per-page instruction latency at two wavefronts per SIMD: bf16 with 3
  // pages 130 against 125 us per config-3 layer (query rows moved to LDS to
  // fit the registers), with 4 pages 191 us (LDS-limited occupancy); fp8
  // with 3 and 4 pages 146 and 150 against 140 us.
  Raw ka[8], va[8], kb[8], vb[8];
  bool bada, badb;
  if constexpr (QLDS) {
#pragma unroll
    for (int h = 0; h < G; ++h) qc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    PageDesc da = next_desc();
    load_page(da, ka, va, qc, bada, 0);
    PageDesc db = next_desc();
    load_page(db, kb, vb, qc, badb, 1);
    for (long long g = g0; g < g1; g += 2) {
      step(da, ka, va, qc, bada, 0);
      da = next_desc();
      load_page(da, ka, va, qc, bada, 0);
      step(db, kb, vb, qc, badb, 1);
      db = next_desc();
      load_page(db, kb, vb, qc, badb, 1);
    }
  } else {
    float4 qa[G], qb[G];
#pragma unroll
    for (int h = 0; h < G; ++h) qa[h] = qb[h] = qc[h] = make_float4(0.f, 0.f, 0.f, 0.f);
    PageDesc da = next_desc();
    load_page(da, ka, va, qa, bada, 0);
    PageDesc db = next_desc();
    load_page(db, kb, vb, qb, badb, 1);
    for (long long g = g0; g < g1; g += 2) {
      step(da, ka, va, qa, bada, 0);
      da = next_desc();
      load_page(da, ka, va, qa, bada, 0);
      step(db, kb, vb, qb, badb, 1);
      db = next_desc();
      load_page(db, kb, vb, qb, badb, 1);
    }
  }
  flush();
}

template <int G, bool APPEND, int PF>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(
    G > 4 ? 1 : (stream_lds_query<PF, G>() ? kFp8StreamWaves : 2))))
void decode_stream_kernel(
    DecodeKernelArgs a, const std::uint32_t* __restrict__ tables,
    const std::int32_t* __restrict__ lengths, float* __restrict__ out,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ segments,
    const std::int64_t* __restrict__ append_slots) {
  constexpr bool QLDS = stream_lds_query<PF, G>();
  constexpr int S = QLDS ? kFp8StreamStage : kStreamStage;
  __shared__ __align__(16) float s_p[2][8 * G];
  __shared__ __align__(16) float s_head[3][G];
  __shared__ __align__(16) float4 s_res_o[S][G][32];
  __shared__ float s_res_ml[S][G][2];
  __shared__ long long s_res_dst[S];
  __shared__ int2 s_seg[S];
  __shared__ int s_seg_unit[S];
  __shared__ __align__(16) float4 s_app_k[S][32];
  __shared__ __align__(16) float4 s_app_v[S][32];
  __shared__ long long s_app_dst[S];
  __shared__ __align__(16) float4 s_qslot[QLDS ? 3 : 1][G][32];
  decode_stream_body<G, APPEND, PF, false, S>(
      a, tables, lengths, out, part_o, part_ml, segments, append_slots, blockIdx.x, threadIdx.x,
      StreamLds<G, S>{s_p, s_head, s_res_o, s_res_ml, s_res_dst, s_seg, s_seg_unit, s_app_k,
                      s_app_v, s_app_dst, QLDS ? s_qslot : nullptr});
}

// Cascade decode in one launch.  Blocks [0, prefix_blocks) are the cascade
// prefix pass's workgroups (4 wavefronts, the prefill kernel's two-tile
// shape) and every later block is 4 independent stream wavefronts, so a CU
// holds one of each (256 VGPRs per wavefront, two wavefronts per SIMD) and
// the matrix-core prefix work runs beside the HBM-bound stream without a
// second stream and the fork and join between them.  LDS is one buffer
// carved either way.
template <int G>
union CascadeShared {
  StreamShared<G> stream[4];
  prefill_detail::CascadePrefixShared prefill;
};

template <int G, bool APPEND, int PF>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void cascade_decode_kernel(
    DecodeKernelArgs a, const std::uint32_t* __restrict__ tables,
    const std::int32_t* __restrict__ lengths, float* __restrict__ out,
    float* __restrict__ part_o, float* __restrict__ part_ml, int* __restrict__ segments,
    const std::int64_t* __restrict__ append_slots, prefill_detail::PrefillKernelArgs prefix,
    unsigned prefix_blocks) {
  __shared__ __align__(16) unsigned char lds[sizeof(CascadeShared<G>)];
  auto& sh = *reinterpret_cast<CascadeShared<G>*>(lds);
  if (blockIdx.x < prefix_blocks) {
    prefill_detail::prefill_body<G, true, PF, 2>(prefix, tables, nullptr, blockIdx.x,
                                                   sh.prefill);
    return;
  }
  const int w = static_cast<int>(__builtin_amdgcn_readfirstlane(threadIdx.x >> 6));
  // The stream wavefronts issue ahead of the prefix wavefronts that share
  // their SIMDs (the prefix work is short and not on the critical path).
  __builtin_amdgcn_s_setprio(3);
  decode_stream_body<G, APPEND, PF, true>(
      a, tables, lengths, out, part_o, part_ml, segments, append_slots,
      static_cast<int>(blockIdx.x - prefix_blocks) * 4 + w, static_cast<int>(threadIdx.x & 63),
      stream_lds(sh.stream[w]));
}

// Combines the partials of units that span several stream wavefronts.  One
// workgroup of G * 32 threads per unit (kv head major: unit = kvh * batch +
// b); thread (h, d4) owns 4 output dims of query head h.  The unit's
// wavefront range was recorded by the stream kernel, so the partial loads
// are issued at once.
template <int G>
__global__ __launch_bounds__(256) void decode_stream_merge_kernel(DecodeKernelArgs a) {
  constexpr int D = 128;
  const int unit = blockIdx.x;
  const int2 seg = reinterpret_cast<const int2*>(a.segments)[unit];
  const bool cascade = a.first_page > 0;
  if (seg.y <= 1 && !cascade) return;
  const int kvh = unit / a.batch;
  const int b = unit % a.batch;
  const int tid = threadIdx.x;
  const int h = tid / (D / 4);
  const int d4 = tid % (D / 4);
  const std::size_t slot0 = static_cast<std::size_t>(unit) + seg.x;
  // Online merge over chunks of 8 partials; each chunk's loads issue together.
  constexpr int kChunk = 8;
  float mx = -INFINITY;
  float den = 0.0f;
  float4 num = make_float4(0.f, 0.f, 0.f, 0.f);
  // Partials: the unit's stream segments, then (cascade) its prefix chunks.
  const int nparts = seg.y + (cascade ? a.prefix_chunks : 0);
  const long long units = static_cast<long long>(a.batch) * a.kv_heads;
  for (int s0 = 0; s0 < nparts; s0 += kChunk) {
    float ms[kChunk], ls[kChunk];
    float4 os[kChunk];
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const bool in = s0 + i < nparts;
      const std::size_t slot =
          !in ? slot0
              : (s0 + i < seg.y
                     ? slot0 + s0 + i
                     : static_cast<std::size_t>(a.prefix_slot0 + (s0 + i - seg.y) * units + unit));
      ms[i] = in ? a.part_ml[(slot * G + h) * 2] : -INFINITY;
      ls[i] = in ? a.part_ml[(slot * G + h) * 2 + 1] : 0.0f;
      os[i] = in ? reinterpret_cast<const float4*>(a.part_o + (slot * G + h) * D)[d4]
                 : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float cm = mx;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) cm = fmaxf(cm, ms[i]);
    const float sc = exp2_ratio(mx, cm);
    den *= sc;
    num.x *= sc;
    num.y *= sc;
    num.z *= sc;
    num.w *= sc;
#pragma unroll
    for (int i = 0; i < kChunk; ++i) {
      const float w = s0 + i < nparts ? exp2_ratio(ms[i], cm) : 0.0f;
      den += w * ls[i];
      num.x += w * os[i].x;
      num.y += w * os[i].y;
      num.z += w * os[i].z;
      num.w += w * os[i].w;
    }
    mx = cm;
  }
  float4 r;
  if (mx == -INFINITY) {
    r = make_float4(NAN, NAN, NAN, NAN);
  } else {
    const float inv = 1.0f / den;
    r = make_float4(num.x * inv, num.y * inv, num.z * inv, num.w * inv);
  }
  const std::size_t qrow = static_cast<std::size_t>(b) * a.q_heads + kvh * G + h;
  reinterpret_cast<float4*>(a.out + qrow * D)[d4] = r;
}

__global__ void zero_words_kernel(unsigned* p, std::size_t n) {
  const std::size_t i = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// ------------------------------------------------------------ generic ----
// One workgroup per (q head, query row).  Pass 1 writes scaled scores (or
// -inf for causally masked keys, NaN for an out-of-range page) to the row of
// the workspace, pass 2 applies the reference softmax rules in place
// (src/kernels/cpu/reference.cpp:264-316), pass 3 computes P.V with the
// probabilities staged through LDS.  Each thread only re-reads workspace
// entries it wrote itself, so no cross-thread global visibility is assumed.
__device__ float block_reduce_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}
__device__ float block_reduce_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x / 64;
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float r = 0.0f;
  for (int i = 0; i < kThreads / 64; ++i) r += red[i];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kThreads) void generic_attention_kernel(GenericArgs a) {
  __shared__ float red[kThreads / 64];
  __shared__ float tile[kThreads];
  const std::size_t qi = blockIdx.x;
  const std::size_t h = blockIdx.y;
  const std::size_t group = a.q_heads / a.kv_heads;
  const std::size_t kvh = h / group;
  const std::size_t keys = a.history + a.tail;
  const std::size_t qpos = a.offset + qi;
  const std::size_t visible = qpos + 1 < keys ? qpos + 1 : keys;
  const float scale = 1.0f / sqrtf(static_cast<float>(a.key_dim));
  const float* qrow = a.query + (h * a.queries + qi) * a.key_dim;
  float* srow = a.workspace + (h * a.queries + qi) * keys;

  float local_max = -INFINITY;
  float nan_seen = 0.0f;
  float pinf = 0.0f;
  for (std::size_t k = threadIdx.x; k < keys; k += kThreads) {
    float s;
    if (k > qpos) {
      s = -INFINITY;
    } else {
      const float* krow = nullptr;
      if (k < a.history) {
        const std::size_t phys = a.table[k / a.block_tokens];
        if (phys < a.physical_blocks) {
          krow = a.key_blocks +
                 ((phys * a.kv_heads + kvh) * a.block_tokens + k % a.block_tokens) * a.key_dim;
        }
      } else {
        krow = a.tail_key + (kvh * a.tail + (k - a.history)) * a.key_dim;
      }
      if (krow == nullptr) {
        s = NAN;
      } else {
        float dot = 0.0f;
        for (std::size_t d = 0; d < a.key_dim; ++d) dot += qrow[d] * krow[d];
        s = dot * scale;
      }
    }
    srow[k] = s;
    if (isnan(s)) nan_seen = 1.0f;
    if (isinf(s) && s > 0.0f) pinf += 1.0f;
    local_max = fmaxf(local_max, s);
  }
  const float mx = block_reduce_max(local_max, red);
  const bool row_nan = block_reduce_max(nan_seen, red) > 0.0f;
  const float inf_count = block_reduce_sum(pinf, red);

  float local_sum = 0.0f;
  if (!row_nan && mx != -INFINITY && inf_count == 0.0f) {
    for (std::size_t k = threadIdx.x; k < keys; k += kThreads) local_sum += expf(srow[k] - mx);
  }
  const float den = block_reduce_sum(local_sum, red);
  for (std::size_t k = threadIdx.x; k < keys; k += kThreads) {
    float p;
    if (row_nan || mx == -INFINITY) {
      p = NAN;
    } else if (inf_count > 0.0f) {
      p = srow[k] == INFINITY ? 1.0f / inf_count : 0.0f;
    } else {
      p = expf(srow[k] - mx) / den;
    }
    srow[k] = p;
  }

  // Pass 3: P.V over the visible keys, 256 keys per tile.  The tile's
  // probabilities are staged in LDS by the threads that wrote them.  With
  // value_dim <= 256 the threads split into kThreads / value_dim key lanes:
  // thread (lane, d) sums lane's keys of the tile for output dim d, the loads
  // of different keys independent of each other, and the lanes are summed
  // through LDS at the end.  Wider values keep one thread per dim (up to 4
  // dims per thread) over every key.
  const std::size_t dv_count = a.value_dim;
  auto value_row = [&](std::size_t key) -> const float* {
    if (key >= a.history) return a.tail_value + (kvh * a.tail + (key - a.history)) * a.value_dim;
    const std::size_t phys = a.table[key / a.block_tokens];
    if (phys >= a.physical_blocks) return nullptr;
    return a.value_blocks +
           ((phys * a.kv_heads + kvh) * a.block_tokens + key % a.block_tokens) * a.value_dim;
  };
  if (dv_count <= kThreads) {
    const std::size_t lanes = kThreads / dv_count;
    const std::size_t d = threadIdx.x % dv_count;
    const std::size_t lane = threadIdx.x / dv_count;
    float acc = 0.0f;
    for (std::size_t k0 = 0; k0 < visible; k0 += kThreads) {
      const std::size_t k = k0 + threadIdx.x;
      tile[threadIdx.x] = k < visible ? srow[k] : 0.0f;
      __syncthreads();
      const std::size_t n = visible - k0 < kThreads ? visible - k0 : kThreads;
      if (lane < lanes) {
        for (std::size_t kk = lane; kk < n; kk += lanes) {
          const float* vrow = value_row(k0 + kk);
          acc += vrow == nullptr ? NAN : tile[kk] * vrow[d];
        }
      }
      __syncthreads();
    }
    // Sum the key lanes of each dim (tile is free again).
    tile[threadIdx.x] = lane < lanes ? acc : 0.0f;
    __syncthreads();
    if (lane == 0) {
      float sum = 0.0f;
      for (std::size_t l = 0; l < lanes; ++l) sum += tile[l * dv_count + d];
      a.out[(h * a.queries + qi) * a.value_dim + d] = sum;
    }
    return;
  }
  float acc[4] = {0.f, 0.f, 0.f, 0.f};  // up to 4 output dims per thread
  for (std::size_t k0 = 0; k0 < visible; k0 += kThreads) {
    const std::size_t k = k0 + threadIdx.x;
    tile[threadIdx.x] = k < visible ? srow[k] : 0.0f;
    __syncthreads();
    const std::size_t n = visible - k0 < kThreads ? visible - k0 : kThreads;
    for (int part = 0; part < 4; ++part) {
      const std::size_t d = threadIdx.x + part * kThreads;
      if (d >= dv_count) break;
      float s = acc[part];
      for (std::size_t kk = 0; kk < n; ++kk) {
        const float* vrow = value_row(k0 + kk);
        s += vrow == nullptr ? NAN : tile[kk] * vrow[d];
      }
      acc[part] = s;
    }
    __syncthreads();
  }
  for (int part = 0; part < 4; ++part) {
    const std::size_t d = threadIdx.x + part * kThreads;
    if (d < dv_count) a.out[(h * a.queries + qi) * a.value_dim + d] = acc[part];
  }
}


// ------------------------------------- reference-shaped one-sequence decode ----
// paged_scaled_dot_product_attention{,_with_tail}_out with one query row per
// head (the reference model's per-layer decode call, src/model/
// cuda_llama.cpp:361-367), in one launch that also leaves the softmax
// probabilities in the caller's score workspace as the reference does
// (src/attention/cuda_paged.cu:420-548).
//
// Work: the pages of each kv head (its history pages plus, with a tail, one
// pseudo-page holding the tail row) are cut into chunks of 4 * ppw pages;
// one workgroup of 4 wavefronts runs one chunk, each wavefront ppw
// consecutive pages with the stream kernel's lane layout and online
// softmax, writing every score (log2 domain) to its workspace entry.  The
// workgroup merges its wavefronts through LDS.  With one workgroup per kv
// head it finishes in place; otherwise it leaves one partial (m, l, o) per
// query head in the scratch for ref_decode_merge_kernel.  Finishing means
// the output rows and the kv head's workspace rows rewritten from scores to
// probabilities, exp2(x - m) / l with the reference's softmax rules
// (src/kernels/cpu/reference.cpp:264-316): a NaN score or a row without a
// finite maximum gives a NaN row, +inf scores share the mass, masked keys
// get 0.
struct RefDecodeKernelArgs {
  const float* query;        // [q_heads, 128]
  const float* key_pool;     // [physical, kv_heads, 16, 128]
  const float* value_pool;
  const std::uint32_t* table;
  const float* tail_key;     // [kv_heads, 128] or null
  const float* tail_value;
  float* out;                // [q_heads, 128]
  float* probs;              // [q_heads, keys]
  float4* part_o;            // [kv_heads * chunks, G, 32]
  float* part_ml;            // [kv_heads * chunks, G, 2]
  int visible;               // page tokens the query row sees
  int keys;                  // workspace row length
  int tail;                  // 1: the tail row is key `visible`
  int kv_heads;
  int chunks;                // workgroups per kv head
  int ppw;                   // pages per wavefront
  std::uint32_t physical_blocks;
  float qscale;              // log2(e) / sqrt(128)
};

template <int G>
__global__ __launch_bounds__(256) void ref_decode_kernel(RefDecodeKernelArgs a) {
  constexpr int D = 128;
  constexpr int P = 16;
  constexpr int R = G >= 4 ? G / 4 : 1;
  constexpr int DUPB = G >= 4 ? 0 : (G == 2 ? 1 : 2);
  constexpr int NV = 8 * G;
  __shared__ __align__(16) float s_p[4][2][NV];
  __shared__ float s_alpha[4][G];
  __shared__ __align__(16) float4 s_o[4][G][32];
  __shared__ float s_ml[4][G][2];
  __shared__ float s_fin[G][2];

  const int unit = static_cast<int>(blockIdx.x) / a.chunks;
  const int chunk = static_cast<int>(blockIdx.x) % a.chunks;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int parity = lane >> 5;
  const int j = lane & 31;
  const bool owner = (j & ((1 << DUPB) - 1)) == 0;
  const int hp = (a.visible + P - 1) / P;
  const int np = hp + a.tail;
  const int p0 = (chunk * 4 + w) * a.ppw;
  const int p1 = min(p0 + a.ppw, np);

  float4 q[G];
#pragma unroll
  for (int h = 0; h < G; ++h) {
    q[h] = reinterpret_cast<const float4*>(a.query + static_cast<std::size_t>(unit * G + h) * D)[j];
  }
  float acc[G][4];
#pragma unroll
  for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = acc[h][2] = acc[h][3] = 0.0f;
  float m[R], l[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    m[r] = -INFINITY;
    l[r] = 0.0f;
  }
  bool bad = false;
  float* prow = a.probs + static_cast<std::size_t>(unit) * G * a.keys;

  // K/V rows of page p: slot i holds token 2i + parity, dims 4j..4j+3; the
  // tail pseudo-page holds the tail row in every slot (masked to token 0).
  auto load = [&](int p, float4 (&k)[8], float4 (&v)[8]) {
    const bool tail = p >= hp;
    const bool skip = p >= p1;
    const void* kb;
    const void* vb;
    if (tail) {
      kb = a.tail_key + static_cast<std::size_t>(unit) * D;
      vb = a.tail_value + static_cast<std::size_t>(unit) * D;
    } else {
      std::uint32_t phys = a.table[p];
      if (phys >= a.physical_blocks) {
        bad = true;
        phys = 0;
      }
      const std::size_t off = (static_cast<std::size_t>(phys) * a.kv_heads + unit) * P * D;
      kb = a.key_pool + off;
      vb = a.value_pool + off;
    }
    const int bytes = skip ? 0 : (tail ? D * 4 : P * D * 4);
    const __amdgpu_buffer_rsrc_t kr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(kb), 0, bytes, kBufferWord3);
    const __amdgpu_buffer_rsrc_t vr =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(vb), 0, bytes, kBufferWord3);
    const int voff = tail ? j * 16 : lane * 16;
    const int step = tail ? 0 : 1024;
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(kr, voff, i * step, kStreamLoad));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = as_float4(__builtin_amdgcn_raw_buffer_load_b128(vr, voff, i * step, kStreamLoad));
  };

  auto process = [&](int p, const float4 (&k)[8], float4 (&v)[8]) {
    const bool tail = p >= hp;
    const int valid = tail ? 1 : min(P, a.visible - p * P);
    float xs[NV];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        xs[i * G + h] = q[h].x * k[i].x + q[h].y * k[i].y + q[h].z * k[i].z + q[h].w * k[i].w;
      }
    }
    reduce_scores<G>(xs, j);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int vi = (j >> DUPB) * R + r;
      const int tok = 2 * (vi / G) + parity;
      const int head = vi % G;
      const bool ok = tok < valid;
      const float s = ok ? xs[r] * a.qscale : -INFINITY;
      if (ok && owner) prow[static_cast<std::size_t>(head) * a.keys + (tail ? a.visible : p * P + tok)] = s;
      const float mn = fmaxf(m[r], token_max(s));
      const float alpha = exp2_ratio(m[r], mn);
      const float pr = ok ? exp2_ratio(s, mn) : 0.0f;
      l[r] = l[r] * alpha + token_sum(pr);
      m[r] = mn;
      if (owner) s_p[w][parity][vi] = pr;
      if (parity == 0 && vi < G && owner) s_alpha[w][vi] = alpha;
    }
    stream_sync<true>();
    float pp[NV];
#pragma unroll
    for (int i = 0; i < NV / 4; ++i) {
      const float4 t4 = reinterpret_cast<const float4*>(s_p[w][parity])[i];
      pp[4 * i] = t4.x;
      pp[4 * i + 1] = t4.y;
      pp[4 * i + 2] = t4.z;
      pp[4 * i + 3] = t4.w;
    }
    float al[G];
#pragma unroll
    for (int h = 0; h < G; ++h) al[h] = s_alpha[w][h];
    stream_sync<true>();
    if (valid < P) {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = masked_row(v[i], 2 * i + parity < valid);
    }
#pragma unroll
    for (int h = 0; h < G; ++h) {
      acc[h][0] *= al[h];
      acc[h][1] *= al[h];
      acc[h][2] *= al[h];
      acc[h][3] *= al[h];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        const float pv = pp[i * G + h];
        acc[h][0] += pv * v[i].x;
        acc[h][1] += pv * v[i].y;
        acc[h][2] += pv * v[i].z;
        acc[h][3] += pv * v[i].w;
      }
    }
  };

  // Two pages in flight.
  float4 ka[8], va[8], kb[8], vb[8];
  for (int p = p0; p < p1; p += 2) {
    load(p, ka, va);
    load(p + 1, kb, vb);
    process(p, ka, va);
    if (p + 1 < p1) process(p + 1, kb, vb);
  }

  // This wavefront's partial into LDS (waves without pages leave m = -inf,
  // l = 0, o = 0), then the workgroup's merge of its four wavefronts.
#pragma unroll
  for (int h = 0; h < G; ++h) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[h][c] += half_xor(acc[h][c]);
  }
  if (parity == 0) {
#pragma unroll
    for (int h = 0; h < G; ++h) s_o[w][h][j] = make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int vi = (j >> DUPB) * R + r;
    if (parity == 0 && vi < G && owner) {
      s_ml[w][vi][0] = m[r];
      s_ml[w][vi][1] = bad ? NAN : l[r];
    }
  }
  __syncthreads();
  const int h = tid >> 5;
  const int d4 = tid & 31;
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
  float mx = -INFINITY, den = 0.0f;
  if (h < G) {
#pragma unroll
    for (int x = 0; x < 4; ++x) mx = fmaxf(mx, s_ml[x][h][0]);
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const float wgt = exp2_ratio(s_ml[x][h][0], mx);
      den += wgt * s_ml[x][h][1];
      const float4 ox = s_o[x][h][d4];
      o.x += wgt * ox.x;
      o.y += wgt * ox.y;
      o.z += wgt * ox.z;
      o.w += wgt * ox.w;
    }
  }
  if (a.chunks > 1) {
    // One partial per head for ref_decode_merge_kernel.
    const std::size_t slot = static_cast<std::size_t>(unit) * a.chunks + chunk;
    if (h < G) {
      a.part_o[(slot * G + h) * 32 + d4] = o;
      if (d4 == 0) {
        a.part_ml[(slot * G + h) * 2] = mx;
        a.part_ml[(slot * G + h) * 2 + 1] = den;
      }
    }
    return;
  }
  // Output rows and the final (m, l) of each head.
  if (h < G) {
    const bool nan_row = mx == -INFINITY || isnan(den);
    const float inv = 1.0f / den;
    const float4 r = nan_row ? make_float4(NAN, NAN, NAN, NAN)
                             : make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
    reinterpret_cast<float4*>(a.out + static_cast<std::size_t>(unit * G + h) * D)[d4] = r;
    if (d4 == 0) {
      s_fin[h][0] = mx;
      s_fin[h][1] = den;
    }
  }
  __syncthreads();
  // Scores -> probabilities over the kv head's G workspace rows.
  const int seen = a.visible + a.tail;
  for (int hh = 0; hh < G; ++hh) {
    const float fm = s_fin[hh][0];
    const float fl = s_fin[hh][1];
    const bool nan_row = fm == -INFINITY || isnan(fl);
    float* row = prow + static_cast<std::size_t>(hh) * a.keys;
    for (int k = tid; k < a.keys; k += 256) {
      float p;
      if (nan_row) {
        p = NAN;
      } else if (k < seen) {
        p = exp2_ratio(row[k], fm) / fl;
      } else {
        p = 0.0f;
      }
      row[k] = p;
    }
  }
}

// Finishes a call whose kv heads took several workgroups.  Workgroup
// (row, s) with row = kv head * G + query head: every workgroup of a row
// merges the row's (m, l) over the kv head's partials, rewrites its share
// of the row's workspace entries (kRefNormKeys keys from s * kRefNormKeys)
// from scores to probabilities, and workgroup s = 0 also merges the output
// row (eight groups of 32 threads over the partials, combined through LDS).
// All loads of a step are issued together: the data was written by other
// XCDs in the previous launch, so every round trip goes to memory.  The
// split of ref_decode_kernel and this merge into two launches is
// deliberate: merging in the last workgroup to finish would need a
// device-scope release per workgroup, which on a multi-XCD part writes back
// the L2 each time (measured per config-3 call in one launch: 63 us with a
// fence in every wavefront of 4-wavefront workgroups, 29 us with one fence
// per 8-wavefront workgroup after each wavefront's own store wait, against
// 12.4 us for the two launches).
constexpr int kRefNormUnroll = static_cast<int>(kRefNormKeys / 256);

template <int G>
__global__ __launch_bounds__(256) void ref_decode_merge_kernel(RefDecodeKernelArgs a) {
  constexpr int D = 128;
  constexpr int kOPer = 8;  // partials per group loaded in the first round
  __shared__ float s_red[4];
  __shared__ __align__(16) float4 s_o[8][32];
  const int row = blockIdx.x;
  const int unit = row / G;
  const int h = row % G;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wv = tid >> 6;
  const bool out_group = blockIdx.y == 0;
  const std::size_t slot0 = static_cast<std::size_t>(unit) * a.chunks;
  auto ml = [&](int c, int i) { return a.part_ml[((slot0 + c) * G + h) * 2 + i]; };
  const int g = tid >> 5;
  const int d4 = tid & 31;
  auto part_o = [&](int c) { return a.part_o[((slot0 + c) * G + h) * 32 + d4]; };

  // One round of loads: this share's scores, the first (m, l) pair per
  // thread and (output workgroup) the first kOPer partial rows per group.
  const int seen = a.visible + a.tail;
  float* prow = a.probs + static_cast<std::size_t>(row) * a.keys;
  const int k0 = static_cast<int>(blockIdx.y) * static_cast<int>(kRefNormKeys) + tid;
  float x[kRefNormUnroll];
#pragma unroll
  for (int u = 0; u < kRefNormUnroll; ++u) {
    const int k = k0 + u * 256;
    x[u] = k < seen ? prow[k] : 0.0f;
  }
  const float m0 = tid < a.chunks ? ml(tid, 0) : -INFINITY;
  const float l0 = tid < a.chunks ? ml(tid, 1) : 0.0f;
  float4 oc[kOPer];
  float om[kOPer];
#pragma unroll
  for (int i = 0; i < kOPer; ++i) {
    const int c = g + 8 * i;
    const bool in = out_group && c < a.chunks;
    om[i] = in ? ml(c, 0) : -INFINITY;
    oc[i] = in ? part_o(c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }

  // Final (m, l) of the row: maximum, then the rescaled sum.
  float mx = m0;
  for (int c = tid + 256; c < a.chunks; c += 256) mx = fmaxf(mx, ml(c, 0));
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) s_red[wv] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
  __syncthreads();
  float den = tid < a.chunks ? exp2_ratio(m0, mx) * l0 : 0.0f;
  for (int c = tid + 256; c < a.chunks; c += 256) den += exp2_ratio(ml(c, 0), mx) * ml(c, 1);
  for (int o = 32; o > 0; o >>= 1) den += __shfl_xor(den, o, 64);
  if (lane == 0) s_red[wv] = den;
  __syncthreads();
  den = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
  const bool nan_row = mx == -INFINITY || isnan(den);

  if (out_group) {
    // Output row: group g takes partials g, g + 8, ...
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int i = 0; i < kOPer; ++i) {
      const float w1 = g + 8 * i < a.chunks ? exp2_ratio(om[i], mx) : 0.0f;
      o.x += w1 * oc[i].x;
      o.y += w1 * oc[i].y;
      o.z += w1 * oc[i].z;
      o.w += w1 * oc[i].w;
    }
    for (int c = g + 8 * kOPer; c < a.chunks; c += 8) {
      const float w1 = exp2_ratio(ml(c, 0), mx);
      const float4 v = part_o(c);
      o.x += w1 * v.x;
      o.y += w1 * v.y;
      o.z += w1 * v.z;
      o.w += w1 * v.w;
    }
    s_o[g][d4] = o;
    __syncthreads();
    if (tid < 32) {
      float4 r = s_o[0][tid];
#pragma unroll
      for (int i = 1; i < 8; ++i) {
        r.x += s_o[i][tid].x;
        r.y += s_o[i][tid].y;
        r.z += s_o[i][tid].z;
        r.w += s_o[i][tid].w;
      }
      const float inv = 1.0f / den;
      r = nan_row ? make_float4(NAN, NAN, NAN, NAN)
                  : make_float4(r.x * inv, r.y * inv, r.z * inv, r.w * inv);
      reinterpret_cast<float4*>(a.out + static_cast<std::size_t>(row) * D)[tid] = r;
    }
  }

  // This workgroup's share of the row: scores -> probabilities.
#pragma unroll
  for (int u = 0; u < kRefNormUnroll; ++u) {
    const int k = k0 + u * 256;
    if (k < a.keys) prow[k] = nan_row ? NAN : (k < seen ? exp2_ratio(x[u], mx) / den : 0.0f);
  }
}

}  // namespace

// ------------------------------------------------------------ launchers ----
namespace {

using Bf16 = unsigned short;
using Fp8 = unsigned char;

float2 scales(const PageFormat& f) { return make_float2(f.k_scale, f.v_scale); }

// Runs body(S*, W) with the page element type of `type` and the widest
// element group the geometry and the fp32 pointers allow.
template <typename F>
hipError_t with_page_type(const PageFormat& fmt, bool vec, F&& body) {
  if (fmt.type == PageType::kBF16) {
    if (vec) {
      body(Bf16{}, std::integral_constant<int, 4>{});
    } else {
      body(Bf16{}, std::integral_constant<int, 1>{});
    }
  } else if (fmt.type == PageType::kFP8) {
    if (vec) {
      body(Fp8{}, std::integral_constant<int, 4>{});
    } else {
      body(Fp8{}, std::integral_constant<int, 1>{});
    }
  } else if (vec) {
    body(float{}, std::integral_constant<int, 4>{});
  } else {
    body(float{}, std::integral_constant<int, 1>{});
  }
  return hipGetLastError();
}

template <typename S>
S* as_pages(void* p) {
  return static_cast<S*>(p);
}
template <typename S>
const S* as_pages(const void* p) {
  return static_cast<const S*>(p);
}

}  // namespace

hipError_t launch_append_token(const float* keys, const float* values, void* key_base,
                               void* value_base, std::size_t layer_stride, std::size_t layers,
                               const PageGeometry& g, std::uint32_t block, std::size_t offset,
                               hipStream_t stream, PageFormat type) {
  const bool vec = g.head_dim % 4 == 0 && aligned16(keys) && aligned16(values);
  const std::size_t work = layers * g.kv_heads * (vec ? g.head_dim / 4 : g.head_dim);
  const dim3 grid(grid_for(work, kThreads), 2);
  return with_page_type(type, vec, [&](auto s, auto w) {
    using S = decltype(s);
    append_token_kernel<S, decltype(w)::value><<<grid, kThreads, 0, stream>>>(
        keys, values, as_pages<S>(key_base), as_pages<S>(value_base), layer_stride, layers,
        g.kv_heads, g.block_tokens, g.head_dim, block, offset, scales(type));
  });
}

hipError_t launch_append_bulk(const float* const* layer_keys, const float* const* layer_values,
                              void* key_base, void* value_base, std::size_t layer_stride,
                              std::size_t layers, const PageGeometry& g,
                              const std::uint32_t* blocks, std::size_t first_block,
                              std::size_t old_length, std::size_t tokens, hipStream_t stream,
                              bool vec, PageFormat type) {
  const std::size_t work = layers * g.kv_heads * tokens * (vec ? g.head_dim / 4 : g.head_dim);
  const dim3 grid(grid_for(work, kThreads), 2);
  const LayerPointers src{layer_keys, layer_values};
  return with_page_type(type, vec, [&](auto s, auto w) {
    using S = decltype(s);
    append_bulk_kernel<S, decltype(w)::value><<<grid, kThreads, 0, stream>>>(
        src, as_pages<S>(key_base), as_pages<S>(value_base), layer_stride, layers, g.kv_heads,
        g.block_tokens, g.head_dim, blocks, first_block, old_length, tokens, scales(type));
  });
}

hipError_t launch_append_slots(const float* keys, const float* values, void* key_pool,
                               void* value_pool, const PageGeometry& g, const std::int64_t* slots,
                               std::size_t count, hipStream_t stream, std::size_t tokens,
                               PageFormat type, std::size_t layers, std::size_t layer_stride) {
  if (count == 0 || tokens == 0 || layers == 0) return hipSuccess;
  const bool vec = g.head_dim % 4 == 0 && aligned16(keys) && aligned16(values);
  const std::size_t per_row = g.kv_heads * (vec ? g.head_dim / 4 : g.head_dim);
  const std::size_t rows = count * tokens;
  if (rows > 0xffffffffu || layers * 2 > 65535 || per_row > 0xffffffffu) {
    return hipErrorInvalidValue;
  }
  const dim3 grid(static_cast<unsigned>((per_row + kThreads - 1) / kThreads),
                  static_cast<unsigned>(rows < 65535 ? rows : 65535),
                  static_cast<unsigned>(layers * 2));
  return with_page_type(type, vec, [&](auto s, auto w) {
    using S = decltype(s);
    constexpr int W = decltype(w)::value;
    append_slots_kernel<S, W><<<grid, kThreads, 0, stream>>>(
        keys, values, as_pages<S>(key_pool), as_pages<S>(value_pool), layer_stride,
        static_cast<unsigned>(g.kv_heads), static_cast<unsigned>(g.block_tokens),
        static_cast<unsigned>(g.head_dim), slots, static_cast<unsigned>(count),
        static_cast<unsigned>(tokens), scales(type));
  });
}

hipError_t launch_rope(const RopeTensor& a, const RopeTensor& b, std::size_t rows,
                       std::size_t head_dim, const float* cosine, const float* sine,
                       std::size_t cache_rows, const std::int32_t* positions, hipStream_t stream) {
  const std::size_t pairs = head_dim / 2;
  const std::size_t work = rows * (a.vectors + b.vectors) * pairs;
  if (work == 0) return hipSuccess;
  const RopeSegment s0{a.input, a.output, static_cast<unsigned>(a.vectors)};
  const RopeSegment s1{b.input, b.output, static_cast<unsigned>(b.vectors)};
  rope_kernel<<<grid_for(work, kThreads), kThreads, 0, stream>>>(
      s0, s1, static_cast<unsigned>(rows), static_cast<unsigned>(pairs), cosine, sine, positions,
      static_cast<long long>(cache_rows));
  return hipGetLastError();
}

hipError_t launch_gather(const void* key_pool, const void* value_pool, const PageGeometry& g,
                         const std::uint32_t* blocks, std::size_t length, float* keys_out,
                         float* values_out, std::size_t dest_tokens, hipStream_t stream,
                         PageFormat type, std::size_t first_token) {
  if (length == 0) return hipSuccess;
  const bool vec = g.head_dim % 4 == 0 && aligned16(keys_out) && aligned16(values_out);
  const std::size_t work = g.kv_heads * length * (vec ? g.head_dim / 4 : g.head_dim);
  const dim3 grid(grid_for(work, kThreads), 2);
  return with_page_type(type, vec, [&](auto s, auto w) {
    using S = decltype(s);
    gather_kernel<S, decltype(w)::value><<<grid, kThreads, 0, stream>>>(
        as_pages<S>(key_pool), as_pages<S>(value_pool), g.kv_heads, g.block_tokens, g.head_dim,
        blocks, length, keys_out, values_out, dest_tokens, scales(type), first_token);
  });
}

hipError_t launch_page_copy(void* key_base, void* value_base, std::size_t layer_stride,
                            std::size_t layers, const PageGeometry& g, std::uint32_t from,
                            std::uint32_t to, std::size_t tokens, hipStream_t stream,
                            PageFormat type) {
  if (tokens == 0) return hipSuccess;
  const bool vec = g.head_dim % 4 == 0;
  const std::size_t work = layers * g.kv_heads * tokens * (vec ? g.head_dim / 4 : g.head_dim);
  const dim3 grid(grid_for(work, kThreads), 2);
  return with_page_type(type, vec, [&](auto s, auto w) {
    using S = decltype(s);
    page_copy_kernel<S, decltype(w)::value><<<grid, kThreads, 0, stream>>>(
        as_pages<S>(key_base), as_pages<S>(value_base), layer_stride, layers, g.kv_heads,
        g.block_tokens, g.head_dim, from, to, tokens);
  });
}

hipError_t launch_table_updates(std::uint32_t* tables, std::size_t cols,
                                const std::uint32_t* updates, std::size_t count,
                                hipStream_t stream) {
  if (count == 0) return hipSuccess;
  table_update_kernel<<<grid_for(count, kThreads), kThreads, 0, stream>>>(tables, cols, updates,
                                                                         count);
  return hipGetLastError();
}

namespace {

std::size_t align256(std::size_t n) { return (n + 255) & ~std::size_t{255}; }

struct WorkspaceLayout {
  std::size_t part_o, part_ml, total, segments;
};

WorkspaceLayout layout_for(std::size_t batch, std::size_t q_heads, std::size_t kv_heads,
                           std::size_t max_splits) {
  const std::size_t group = q_heads / kv_heads;
  const std::size_t slots = batch * kv_heads * max_splits;
  WorkspaceLayout l{};
  l.part_o = 0;
  l.part_ml = align256(slots * group * kDecodeHeadDim * sizeof(float));
  l.total = l.part_ml + align256(slots * group * 2 * sizeof(float));
  return l;
}

// Stream mode: one partial slot per (sequence, kv head) unit plus one per
// wavefront (slot = unit + wavefront), then `chunks` cascade prefix slots
// per unit, then the per-unit segment records.
WorkspaceLayout stream_layout(std::size_t batch, std::size_t q_heads, std::size_t kv_heads,
                              std::size_t waves, std::size_t chunks) {
  WorkspaceLayout l = layout_for((1 + chunks) * batch * kv_heads + waves, q_heads / kv_heads, 1, 1);
  l.segments = l.total;
  l.total += align256(batch * kv_heads * 2 * sizeof(int));
  return l;
}

WorkspaceLayout stream_layout_for(std::size_t batch, std::size_t q_heads, std::size_t kv_heads) {
  return stream_layout(batch, q_heads, kv_heads, kMaxStreamWaves, kMaxCascadeChunks);
}

}  // namespace

std::size_t decode_max_splits(std::size_t max_blocks, std::size_t pages_per_split) {
  if (pages_per_split == 0) return 1;
  const std::size_t s = (max_blocks + pages_per_split - 1) / pages_per_split;
  return s == 0 ? 1 : s;
}

std::size_t decode_workspace_bytes(std::size_t batch, std::size_t q_heads, std::size_t kv_heads,
                                   std::size_t max_blocks, std::size_t pages_per_split) {
  if (kv_heads == 0 || q_heads % kv_heads != 0) return 0;
  if (pages_per_split == 0) {
    // Stream mode: one partial slot per unit plus one per wavefront.
    return stream_layout_for(batch, q_heads, kv_heads).total;
  }
  return layout_for(batch, q_heads, kv_heads, decode_max_splits(max_blocks, pages_per_split)).total;
}

hipError_t launch_decode_workspace_init(void* workspace, std::size_t bytes, hipStream_t stream) {
  const std::size_t words = bytes / sizeof(unsigned);
  if (words == 0) return hipSuccess;
  zero_words_kernel<<<grid_for(words, kThreads), kThreads, 0, stream>>>(
      static_cast<unsigned*>(workspace), words);
  return hipGetLastError();
}

bool decode_group_supported(std::size_t group) {
  return group == 1 || group == 2 || group == 4 || group == 8;
}

std::size_t decode_items(const std::int32_t* lengths, std::size_t batch, std::size_t kv_heads,
                         std::size_t max_blocks, std::size_t pages_per_split) {
  if (pages_per_split == 0) return 0;  // stream mode sizes its own grid
  std::size_t items = 0;
  for (std::size_t b = 0; b < batch; ++b) {
    const std::int64_t h = lengths[b];
    const std::size_t pages =
        (h < 0 || h > static_cast<std::int64_t>(max_blocks * 16)) ? 0 : (h + 15) / 16;
    const std::size_t s = (pages + pages_per_split - 1) / pages_per_split;
    items += kv_heads * (s < 1 ? 1 : s);
  }
  return items;
}

namespace {



// Wavefronts the stream kernel launches: every resident slot of the device
// (fp32 and bf16 pages: two per SIMD up to four query heads per kv head, one
// for eight; fp8 pages: four per SIMD up to four query heads, as the
// kernels' register and LDS use allows), at most kMaxStreamWaves.
// beside_prefix: one per SIMD whatever the group, so the concurrent cascade
// prefix pass finds registers on every SIMD.
std::size_t stream_waves(std::size_t group, bool beside_prefix,
                         PageType type = PageType::kF32) {
  const int n = device_cus();
  const std::size_t per_simd =
      group >= 8 || beside_prefix ? 1 : (stream_lds_query_type(type) ? kFp8StreamWaves : 2);
  const std::size_t w = static_cast<std::size_t>(n) * 4 * per_simd;
  return w < kMaxStreamWaves ? w : kMaxStreamWaves;
}

}  // namespace

namespace {

template <int G, bool APPEND, int PF>
void launch_stream_variant(const dim3& grid, hipStream_t stream, const DecodeKernelArgs& k) {
  decode_stream_kernel<G, APPEND, PF><<<grid, 64, 0, stream>>>(
      k, k.tables, k.lengths, k.out, k.part_o, k.part_ml, k.segments,
      APPEND ? k.append_slots : nullptr);
}

template <int G, bool APPEND, int PF>
void launch_cascade_variant(const dim3& grid, hipStream_t stream, const DecodeKernelArgs& k,
                            const prefill_detail::PrefillKernelArgs& prefix,
                            unsigned prefix_blocks) {
  cascade_decode_kernel<G, APPEND, PF><<<grid, 256, 0, stream>>>(
      k, k.tables, k.lengths, k.out, k.part_o, k.part_ml, k.segments,
      APPEND ? k.append_slots : nullptr, prefix, prefix_blocks);
}

// Runs body(APPEND, PF) with the compile-time forms of append and type.
template <typename F>
void with_stream_variant(bool append, PageType type, F&& body) {
  using std::integral_constant;
  const auto pick = [&](auto ap) {
    switch (type) {
      case PageType::kBF16: body(ap, integral_constant<int, 1>{}); break;
      case PageType::kFP8: body(ap, integral_constant<int, 2>{}); break;
      default: body(ap, integral_constant<int, 0>{}); break;
    }
  };
  if (append) {
    pick(integral_constant<bool, true>{});
  } else {
    pick(integral_constant<bool, false>{});
  }
}

template <int G>
void launch_cascade(const dim3& grid, hipStream_t stream, const DecodeKernelArgs& k,
                    const prefill_detail::PrefillKernelArgs& prefix, unsigned prefix_blocks,
                    bool append, PageType type) {
  with_stream_variant(append, type, [&](auto ap, auto pf) {
    launch_cascade_variant<G, decltype(ap)::value, decltype(pf)::value>(grid, stream, k, prefix,
                                                                        prefix_blocks);
  });
}

template <int G>
void launch_stream(const dim3& grid, hipStream_t stream, const DecodeKernelArgs& k, bool append,
                   PageType type) {
  with_stream_variant(append, type, [&](auto ap, auto pf) {
    launch_stream_variant<G, decltype(ap)::value, decltype(pf)::value>(grid, stream, k);
  });
}

}  // namespace

hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream) {
  if (a.batch == 0) return hipSuccess;
  const bool streamed = a.pages_per_split == 0;
  const std::size_t max_splits = decode_max_splits(a.max_blocks, a.pages_per_split);
  const std::size_t group = a.q_heads / a.kv_heads;
  auto* ws = static_cast<unsigned char*>(a.workspace);
  DecodeKernelArgs k{};
  k.query = a.query;
  k.key_pool = a.key_pool;
  k.value_pool = a.value_pool;
  k.tables = a.tables;
  k.lengths = a.lengths;
  k.tail_key = a.tail_key;
  k.tail_value = a.tail_value;
  k.out = a.out;
  k.batch = static_cast<int>(a.batch);
  k.q_heads = static_cast<int>(a.q_heads);
  k.kv_heads = static_cast<int>(a.kv_heads);
  k.max_blocks = static_cast<int>(a.max_blocks);
  k.max_splits = static_cast<int>(max_splits);
  k.pages_per_split = static_cast<int>(a.pages_per_split);
  k.physical_blocks = static_cast<std::uint32_t>(a.physical_blocks);
  k.qscale = kLog2e / sqrtf(static_cast<float>(kDecodeHeadDim));
  k.k_scale = a.page_type.k_scale;
  k.v_scale = a.page_type.v_scale;
  // fp8 keys widen to bare code values: their scale joins the score scale.
  if (a.page_type.type == PageType::kFP8) k.qscale *= a.page_type.k_scale;
  if (a.lengths == nullptr) return hipErrorInvalidValue;
  if (streamed) {
    // Cascade in one launch for groups up to kCascadeFusedMaxGroup (the
    // stream LDS of four wavefronts then fits beside a prefix workgroup's,
    // two blocks per CU); larger groups run the prefix pass on the side
    // stream when the caller provides one.
    const bool fused = a.shared_pages > 0 && group <= kCascadeFusedMaxGroup;
    const bool overlap = !fused && a.shared_pages > 0 && a.side_stream != nullptr &&
                         a.fork_event != nullptr && a.join_event != nullptr;
    const std::size_t waves = stream_waves(group, overlap || fused, a.page_type.type);
    // The compact layout is sized for this launch's wavefront count (which
    // compact_decode_workspace_bytes gives for the same page type).
    if (a.compact_layout && a.shared_pages != 0) return hipErrorInvalidValue;
    const WorkspaceLayout lay =
        a.compact_layout ? stream_layout(a.batch, a.q_heads, a.kv_heads, waves, 0)
                         : stream_layout_for(a.batch, a.q_heads, a.kv_heads);
    k.part_o = reinterpret_cast<float*>(ws + lay.part_o);
    k.part_ml = reinterpret_cast<float*>(ws + lay.part_ml);
    k.segments = reinterpret_cast<int*>(ws + lay.segments);
    k.first_page = static_cast<int>(a.shared_pages);
    k.append_slots = a.append_slots;
    k.append_key_pool = a.append_key_pool;
    k.append_value_pool = a.append_value_pool;
    k.prefix_slot0 = static_cast<long long>(a.batch * a.kv_heads + kMaxStreamWaves);
    if (a.shared_pages > 0) {
      const std::size_t cp = cascade_chunk_pages(a.shared_pages, a.batch, group, a.kv_heads);
      k.prefix_chunks = static_cast<int>((a.shared_pages + cp - 1) / cp);
      CascadePrefixArgs c{};
      c.query = a.query;
      c.key_pool = a.key_pool;
      c.value_pool = a.value_pool;
      c.table = a.tables;
      c.part_o = k.part_o;
      c.part_ml = k.part_ml;
      c.batch = a.batch;
      c.q_heads = a.q_heads;
      c.kv_heads = a.kv_heads;
      c.shared_pages = a.shared_pages;
      c.physical_blocks = a.physical_blocks;
      c.prefix_slot0 = static_cast<std::size_t>(k.prefix_slot0);
      c.page_type = a.page_type;
      if (fused) {
        std::size_t items = 0;
        const prefill_detail::PrefillKernelArgs pk = prefill_detail::cascade_prefix_args(c, &items);
        k.stream_waves = static_cast<int>(waves);
        const dim3 grid(static_cast<unsigned>(items + waves / 4));
        const bool append = k.append_slots != nullptr;
        const PageType pt = a.page_type.type;
        const auto pb = static_cast<unsigned>(items);
        switch (group) {
          case 1: launch_cascade<1>(grid, stream, k, pk, pb, append, pt); break;
          case 2: launch_cascade<2>(grid, stream, k, pk, pb, append, pt); break;
          case 4: launch_cascade<4>(grid, stream, k, pk, pb, append, pt); break;
          default: return hipErrorInvalidValue;
        }
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (a.between_event != nullptr) {
          e = hipEventRecord(a.between_event, stream);
          if (e != hipSuccess) return e;
        }
        const dim3 mgrid(static_cast<unsigned>(a.batch * a.kv_heads));
        switch (group) {
          case 1: decode_stream_merge_kernel<1><<<mgrid, 1 * 32, 0, stream>>>(k); break;
          case 2: decode_stream_merge_kernel<2><<<mgrid, 2 * 32, 0, stream>>>(k); break;
          case 4: decode_stream_merge_kernel<4><<<mgrid, 4 * 32, 0, stream>>>(k); break;
          default: return hipErrorInvalidValue;
        }
        return hipGetLastError();
      }
      if (overlap) {
        hipError_t e = hipEventRecord(a.fork_event, stream);
        if (e == hipSuccess) e = hipStreamWaitEvent(a.side_stream, a.fork_event, 0);
        if (e == hipSuccess) e = launch_cascade_prefix(c, a.side_stream);
        if (e == hipSuccess) e = hipEventRecord(a.join_event, a.side_stream);
        if (e != hipSuccess) return e;
        // The stream kernel then runs one wavefront per SIMD: with two,
        // the prefix workgroups find no registers until stream waves
        // retire, and the late-starting waves of the static partition
        // stretch the kernel (128 sequences sharing 64 pages, per layer:
        // overlapped 103 us, back to back 111 us, overlapped with two
        // waves per SIMD 124 us).
      } else {
        const hipError_t e = launch_cascade_prefix(c, stream);
        if (e != hipSuccess) return e;
      }
    }
    k.stream_waves = static_cast<int>(waves);
    const dim3 grid(static_cast<unsigned>(waves));
    const bool append = k.append_slots != nullptr;
    const PageType pt = a.page_type.type;
    switch (group) {
      case 1: launch_stream<1>(grid, stream, k, append, pt); break;
      case 2: launch_stream<2>(grid, stream, k, append, pt); break;
      case 4: launch_stream<4>(grid, stream, k, append, pt); break;
      case 8: launch_stream<8>(grid, stream, k, append, pt); break;
      default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // The timing event goes before the join: recorded after a cross-stream
    // wait it cost about 5 us per launch.
    if (a.between_event != nullptr) {
      e = hipEventRecord(a.between_event, stream);
      if (e != hipSuccess) return e;
    }
    if (overlap) {
      e = hipStreamWaitEvent(stream, a.join_event, 0);
      if (e != hipSuccess) return e;
    }
    const dim3 mgrid(static_cast<unsigned>(a.batch * a.kv_heads));
    switch (group) {
      case 1: decode_stream_merge_kernel<1><<<mgrid, 1 * 32, 0, stream>>>(k); break;
      case 2: decode_stream_merge_kernel<2><<<mgrid, 2 * 32, 0, stream>>>(k); break;
      case 4: decode_stream_merge_kernel<4><<<mgrid, 4 * 32, 0, stream>>>(k); break;
      case 8: decode_stream_merge_kernel<8><<<mgrid, 8 * 32, 0, stream>>>(k); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  const WorkspaceLayout lay = layout_for(a.batch, a.q_heads, a.kv_heads, max_splits);
  k.part_o = reinterpret_cast<float*>(ws + lay.part_o);
  k.part_ml = reinterpret_cast<float*>(ws + lay.part_ml);
  // Items beyond the real work (when the caller passes no exact count)
  // return at once.
  const std::size_t items = a.items != 0 ? a.items : a.batch * a.kv_heads * max_splits;
  const dim3 grid(static_cast<unsigned>(items));
  switch (group) {
    case 1: decode_split_kernel<1><<<grid, 64, 0, stream>>>(k); break;
    case 2: decode_split_kernel<2><<<grid, 64, 0, stream>>>(k); break;
    case 4: decode_split_kernel<4><<<grid, 64, 0, stream>>>(k); break;
    case 8: decode_split_kernel<8><<<grid, 64, 0, stream>>>(k); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e == hipSuccess && a.between_event != nullptr) e = hipEventRecord(a.between_event, stream);
  if (e != hipSuccess || max_splits == 1) return e;
  const dim3 mgrid(static_cast<unsigned>(a.batch * a.kv_heads));
  const std::size_t lds = (group * max_splits + group) * sizeof(float);
  switch (group) {
    case 1: decode_merge_kernel<1><<<mgrid, 256, lds, stream>>>(k); break;
    case 2: decode_merge_kernel<2><<<mgrid, 256, lds, stream>>>(k); break;
    case 4: decode_merge_kernel<4><<<mgrid, 256, lds, stream>>>(k); break;
    case 8: decode_merge_kernel<8><<<mgrid, 256, lds, stream>>>(k); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

std::size_t compact_decode_workspace_bytes(std::size_t batch, std::size_t q_heads,
                                           std::size_t kv_heads, PageType type) {
  if (kv_heads == 0 || q_heads % kv_heads != 0) return 0;
  return stream_layout(batch, q_heads, kv_heads, stream_waves(q_heads / kv_heads, false, type), 0)
      .total;
}


RefDecodePlan ref_decode_plan(std::size_t q_heads, std::size_t kv_heads, std::size_t visible,
                              bool tail) {
  RefDecodePlan p{};
  if (kv_heads == 0 || q_heads % kv_heads != 0) return p;
  const std::size_t group = q_heads / kv_heads;
  const std::size_t pages = (visible + kDecodeBlockTokens - 1) / kDecodeBlockTokens + (tail ? 1 : 0);
  // About four wavefronts per CU over the whole call, whole pages each
  // (config-3 calls: 12.4 us against 12.8 at three or six per CU, 13.2 at
  // eight and 13.8 at two).
  const std::size_t target = static_cast<std::size_t>(device_cus()) * 4;
  const std::size_t total = kv_heads * pages;
  p.ppw = total <= target ? 1 : (total + target - 1) / target;
  p.chunks = (pages + 4 * p.ppw - 1) / (4 * p.ppw);
  if (p.chunks == 0) p.chunks = 1;
  const std::size_t slots = p.chunks > 1 ? kv_heads * p.chunks : 0;
  p.scratch_bytes = align256(slots * group * 2 * sizeof(float)) +
                    slots * group * kDecodeHeadDim * sizeof(float);
  return p;
}

hipError_t launch_ref_decode(const RefDecodeArgs& a, const RefDecodePlan& plan,
                             hipStream_t stream) {
  if (a.q_heads == 0) return hipSuccess;
  const std::size_t group = a.q_heads / a.kv_heads;
  auto* ws = static_cast<unsigned char*>(a.scratch);
  const std::size_t slots = a.kv_heads * plan.chunks;
  RefDecodeKernelArgs k{};
  k.query = a.query;
  k.key_pool = a.key_pool;
  k.value_pool = a.value_pool;
  k.table = a.table;
  k.tail_key = a.tail_key;
  k.tail_value = a.tail_value;
  k.out = a.out;
  k.probs = a.probs;
  k.part_ml = reinterpret_cast<float*>(ws);
  k.part_o = reinterpret_cast<float4*>(ws + align256(slots * group * 2 * sizeof(float)));
  k.visible = static_cast<int>(a.visible);
  k.keys = static_cast<int>(a.keys);
  k.tail = a.tail ? 1 : 0;
  k.kv_heads = static_cast<int>(a.kv_heads);
  k.chunks = static_cast<int>(plan.chunks);
  k.ppw = static_cast<int>(plan.ppw);
  k.physical_blocks = static_cast<std::uint32_t>(a.physical_blocks);
  k.qscale = kLog2e / sqrtf(static_cast<float>(kDecodeHeadDim));
  const dim3 grid(static_cast<unsigned>(slots));
  switch (group) {
    case 1: ref_decode_kernel<1><<<grid, 256, 0, stream>>>(k); break;
    case 2: ref_decode_kernel<2><<<grid, 256, 0, stream>>>(k); break;
    case 4: ref_decode_kernel<4><<<grid, 256, 0, stream>>>(k); break;
    case 8: ref_decode_kernel<8><<<grid, 256, 0, stream>>>(k); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || plan.chunks == 1) return e;
  if (a.between_event != nullptr) {
    e = hipEventRecord(a.between_event, stream);
    if (e != hipSuccess) return e;
  }
  const dim3 mgrid(static_cast<unsigned>(a.q_heads),
                   static_cast<unsigned>((a.keys + kRefNormKeys - 1) / kRefNormKeys));
  switch (group) {
    case 1: ref_decode_merge_kernel<1><<<mgrid, 256, 0, stream>>>(k); break;
    case 2: ref_decode_merge_kernel<2><<<mgrid, 256, 0, stream>>>(k); break;
    case 4: ref_decode_merge_kernel<4><<<mgrid, 256, 0, stream>>>(k); break;
    case 8: ref_decode_merge_kernel<8><<<mgrid, 256, 0, stream>>>(k); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_generic(const GenericArgs& a, hipStream_t stream) {
  if (a.queries == 0 || a.q_heads == 0) return hipSuccess;
  dim3 grid(static_cast<unsigned>(a.queries), static_cast<unsigned>(a.q_heads));
  generic_attention_kernel<<<grid, kThreads, 0, stream>>>(a);
  return hipGetLastError();
}

// CUs of the current device, looked up once per device (host threads may
// launch at once).
int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        n <= 0) {
      n = 256;
    }
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

}  // namespace helix::hip
