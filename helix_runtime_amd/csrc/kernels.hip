// Paged-KV kernels for CDNA4 (gfx950): page append / gather / copy-on-write,
// batched split-K decode attention with an uncommitted tail, the split
// combine, and a reference-shaped generic attention kernel.
//
// Data layout in HBM: one layer pool is [physical_blocks, kv_heads,
// block_tokens, head_dim] fp32, so one (block, head) page of 16 tokens x 128
// dims is one contiguous 8 KiB run.  Key and value pools of all layers live
// in one allocation (see paged_cache.cpp).
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <limits>

namespace helix::hip {
namespace {

constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

inline unsigned grid_for(std::size_t work, std::size_t per_block, std::size_t cap = 1u << 20) {
  std::size_t blocks = (work + per_block - 1) / per_block;
  if (blocks == 0) blocks = 1;
  return static_cast<unsigned>(blocks < cap ? blocks : cap);
}

template <typename T>
__device__ __forceinline__ T load_vec(const float* p) {
  return *reinterpret_cast<const T*>(p);
}
template <typename T>
__device__ __forceinline__ void store_vec(float* p, const T& v) {
  *reinterpret_cast<T*>(p) = v;
}
template <typename T>
constexpr int vec_width() {
  return sizeof(T) / sizeof(float);
}

// ------------------------------------------------------------- append ----
// Reference: CudaPagedKvCache::append issues 2 * layers * kv_heads
// cudaMemcpyAsync D2D copies of one head vector (src/kv_cache/cuda_paged.cpp:
// 561-577).  Here one launch moves every (layer, head) vector of K and V with
// 128-bit accesses; blockIdx.y selects keys (0) or values (1).
template <typename V>
__global__ void append_token_kernel(const float* __restrict__ keys,
                                    const float* __restrict__ values, float* key_base,
                                    float* value_base, std::size_t layer_stride,
                                    std::size_t layers, std::size_t heads, std::size_t block_tokens,
                                    std::size_t dim, std::uint32_t block, std::size_t offset) {
  constexpr int W = vec_width<V>();
  const std::size_t dv = dim / W;
  const std::size_t total = layers * heads * dv;
  const float* src = blockIdx.y == 0 ? keys : values;
  float* base = blockIdx.y == 0 ? key_base : value_base;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t c = e % dv;
    const std::size_t lh = e / dv;
    const std::size_t h = lh % heads;
    const std::size_t l = lh / heads;
    float* dst = base + l * layer_stride +
                 ((static_cast<std::size_t>(block) * heads + h) * block_tokens + offset) * dim +
                 c * W;
    store_vec<V>(dst, load_vec<V>(src + e * W));
  }
}

// Reference: PagedKvCache::append_layer_major span copies
// (src/kv_cache/paged.cpp:819-843), token range [old_length, old_length+T).
struct LayerPointers {
  const float* const* keys;
  const float* const* values;
};

template <typename V>
__global__ void append_bulk_kernel(LayerPointers src, float* key_base, float* value_base,
                                   std::size_t layer_stride, std::size_t layers,
                                   std::size_t heads, std::size_t block_tokens, std::size_t dim,
                                   const std::uint32_t* __restrict__ blocks,
                                   std::size_t first_block, std::size_t old_length,
                                   std::size_t tokens) {
  constexpr int W = vec_width<V>();
  const std::size_t dv = dim / W;
  const std::size_t per_layer = heads * tokens * dv;
  const std::size_t total = layers * per_layer;
  float* base = blockIdx.y == 0 ? key_base : value_base;
  const float* const* layer_src = blockIdx.y == 0 ? src.keys : src.values;
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
    float* dst = base + l * layer_stride +
                 ((phys * heads + h) * block_tokens + pos % block_tokens) * dim + c * W;
    store_vec<V>(dst, load_vec<V>(layer_src[l] + r * W));
  }
}

// Batched per-layer append through a slot mapping (decode step: one new
// token per sequence).
template <typename V>
__global__ void append_slots_kernel(const float* __restrict__ keys,
                                    const float* __restrict__ values, float* key_pool,
                                    float* value_pool, std::size_t heads, std::size_t block_tokens,
                                    std::size_t dim, const std::int64_t* __restrict__ slots,
                                    std::size_t count) {
  constexpr int W = vec_width<V>();
  const std::size_t dv = dim / W;
  const std::size_t total = count * heads * dv;
  const float* src = blockIdx.y == 0 ? keys : values;
  float* pool = blockIdx.y == 0 ? key_pool : value_pool;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t c = e % dv;
    const std::size_t rh = e / dv;
    const std::size_t h = rh % heads;
    const std::size_t row = rh / heads;
    const std::int64_t slot = slots[row];
    if (slot < 0) continue;
    const std::size_t block = static_cast<std::size_t>(slot) / block_tokens;
    const std::size_t off = static_cast<std::size_t>(slot) % block_tokens;
    store_vec<V>(pool + ((block * heads + h) * block_tokens + off) * dim + c * W,
                 load_vec<V>(src + e * W));
  }
}

// Reference: PagedKvCache copy_layer / copy_layer_prefix_out
// (src/kv_cache/paged.cpp:242-280, 895-950).
template <typename V>
__global__ void gather_kernel(const float* __restrict__ key_pool,
                              const float* __restrict__ value_pool, std::size_t heads,
                              std::size_t block_tokens, std::size_t dim,
                              const std::uint32_t* __restrict__ blocks, std::size_t length,
                              float* keys_out, float* values_out, std::size_t dest_tokens) {
  constexpr int W = vec_width<V>();
  const std::size_t dv = dim / W;
  const std::size_t total = heads * length * dv;
  const float* pool = blockIdx.y == 0 ? key_pool : value_pool;
  float* out = blockIdx.y == 0 ? keys_out : values_out;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t c = e % dv;
    const std::size_t ht = e / dv;
    const std::size_t t = ht % length;
    const std::size_t h = ht / length;
    const std::size_t phys = blocks[t / block_tokens];
    store_vec<V>(out + (h * dest_tokens + t) * dim + c * W,
                 load_vec<V>(pool + ((phys * heads + h) * block_tokens + t % block_tokens) * dim +
                             c * W));
  }
}

template <typename V>
__global__ void page_copy_kernel(float* key_base, float* value_base, std::size_t layer_stride,
                                 std::size_t layers, std::size_t heads, std::size_t block_tokens,
                                 std::size_t dim, std::uint32_t from, std::uint32_t to,
                                 std::size_t tokens) {
  constexpr int W = vec_width<V>();
  const std::size_t dv = dim / W;
  const std::size_t run = tokens * dv;  // contiguous prefix of one (block, head) page
  const std::size_t total = layers * heads * run;
  float* base = blockIdx.y == 0 ? key_base : value_base;
  for (std::size_t e = blockIdx.x * static_cast<std::size_t>(blockDim.x) + threadIdx.x; e < total;
       e += static_cast<std::size_t>(gridDim.x) * blockDim.x) {
    const std::size_t i = e % run;
    const std::size_t lh = e / run;
    const std::size_t h = lh % heads;
    const std::size_t l = lh / heads;
    const std::size_t page = block_tokens * dim;
    float* layer = base + l * layer_stride;
    store_vec<V>(layer + (static_cast<std::size_t>(to) * heads + h) * page + i * W,
                 load_vec<V>(layer + (static_cast<std::size_t>(from) * heads + h) * page + i * W));
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
// Cross-lane helpers.  ds_swizzle in bit mode exchanges with lane ^ MASK
// inside each 32-lane half; the two halves are combined with ds_bpermute.
template <int MASK>
__device__ __forceinline__ float swz_xor(float x) {
  static_assert(MASK >= 1 && MASK <= 16, "swizzle masks stay inside a 32-lane half");
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(x), (MASK << 10) | 0x1F));
}
__device__ __forceinline__ float half_xor(float x) { return __shfl_xor(x, 32, 64); }

// Recursive halving: N values per lane, exchanged over xor masks 16, 8, ...
// Each step keeps the half selected by the lane's mask bit and adds the
// partner's copy of it, so after k steps a lane holds N / 2^k values summed
// over 2^k lanes.
template <int N, int MASK>
__device__ __forceinline__ void halve(float* x, int j) {
  const bool hi = (j & MASK) != 0;
#pragma unroll
  for (int i = 0; i < N / 2; ++i) {
    const float send = hi ? x[i] : x[i + N / 2];
    const float keep = hi ? x[i + N / 2] : x[i];
    x[i] = keep + swz_xor<MASK>(send);
  }
}

// Reduces 8*G partial dot products (8 tokens x G heads per lane) over the 32
// lanes of a half.  Afterwards lane j holds R = max(1, G/4) complete scores,
// value index v = (j >> DUPB) * R + r (v = local_token * G + head).
template <int G>
__device__ __forceinline__ void reduce_scores(float* x, int j) {
  constexpr int NV = 8 * G;
  halve<NV, 16>(x, j);
  halve<NV / 2, 8>(x, j);
  halve<NV / 4, 4>(x, j);
  if constexpr (NV / 8 >= 2) {
    halve<NV / 8, 2>(x, j);
  } else {
    x[0] += swz_xor<2>(x[0]);
  }
  if constexpr (NV / 16 >= 2) {
    halve<NV / 16, 1>(x, j);
  } else {
    x[0] += swz_xor<1>(x[0]);
  }
}

// Max / sum over the lanes that hold the same head: the token bits of the
// lane index are bits 2..4 plus the half (bit 5).
__device__ __forceinline__ float token_max(float v) {
  v = fmaxf(v, swz_xor<4>(v));
  v = fmaxf(v, swz_xor<8>(v));
  v = fmaxf(v, swz_xor<16>(v));
  return fmaxf(v, half_xor(v));
}
__device__ __forceinline__ float token_sum(float v) {
  v += swz_xor<4>(v);
  v += swz_xor<8>(v);
  v += swz_xor<16>(v);
  return v + half_xor(v);
}

__device__ __forceinline__ float exp2_ratio(float a, float b) {
  // exp2(a - b) with a == b (including +inf == +inf or -inf == -inf) -> 1.
  return a == b ? 1.0f : exp2f(a - b);
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
  float* part_o;   // [batch, q_heads, max_splits, 128]
  float* part_ml;  // [batch, q_heads, max_splits, 2]
  int q_heads;
  int kv_heads;
  int max_blocks;
  int max_splits;
  int pages_per_split;
  std::uint32_t physical_blocks;
  float qscale;
};

// Split-K decode.  One wavefront per (sequence, kv head, split of pages);
// the G = q_heads / kv_heads query heads that share the kv head are held in
// registers, so every K/V byte is read from HBM once per kv head.
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
// (src/attention/cuda_paged.cu:58-61), and is never dereferenced.
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
  const int split = blockIdx.x;
  const int item = blockIdx.y;
  const int b = item / a.kv_heads;
  const int kvh = item % a.kv_heads;

  int hist = a.lengths[b];
  bool bad_page = false;
  if (hist < 0 || hist > a.max_blocks * P) {
    // A length the table cannot cover: attend to the tail only and return
    // NaN rather than reading past the table row.
    hist = 0;
    bad_page = true;
  }
  const int hist_pages = (hist + P - 1) / P;
  int splits = (hist_pages + a.pages_per_split - 1) / a.pages_per_split;
  if (splits < 1) splits = 1;
  if (split >= splits) return;
  const int pg0 = split * a.pages_per_split;
  const int pg1 = min(hist_pages, pg0 + a.pages_per_split);
  const bool last = split == splits - 1;

  const std::size_t qrow0 = static_cast<std::size_t>(b) * a.q_heads + kvh * G;
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

  const std::uint32_t* table = a.tables + static_cast<std::size_t>(b) * a.max_blocks;
  const std::size_t page_elems = static_cast<std::size_t>(P) * D;

  auto page_ptr = [&](const float* pool, std::uint32_t phys) {
    return pool + (static_cast<std::size_t>(phys) * a.kv_heads + kvh) * page_elems;
  };

  // One page (or the tail as a 1-token page) through score, softmax and P.V.
  auto process = [&](const float4 (&k)[8], float4 (&v)[8], int valid) {
    float x[NV];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
      for (int h = 0; h < G; ++h) {
        x[i * G + h] = q[h].x * k[i].x + q[h].y * k[i].y + q[h].z * k[i].z + q[h].w * k[i].w;
      }
    }
    reduce_scores<G>(x, j);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int vi = (j >> DUPB) * R + r;
      const int tok = 2 * (vi / G) + parity;
      const bool ok = tok < valid;
      const float s = ok ? x[r] : -INFINITY;
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

  auto load_page = [&](int pg, float4 (&k)[8], float4 (&v)[8]) -> bool {
    const std::uint32_t phys = table[pg];
    if (phys >= a.physical_blocks) return false;
    const float4* kp = reinterpret_cast<const float4*>(page_ptr(a.key_pool, phys));
    const float4* vp = reinterpret_cast<const float4*>(page_ptr(a.value_pool, phys));
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = kp[i * 64 + lane];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = vp[i * 64 + lane];
    return true;
  };

  if (pg0 < pg1) {
    float4 kc[8], vc[8];
    bool okc = load_page(pg0, kc, vc);
    for (int pg = pg0; pg < pg1; ++pg) {
      float4 kn[8], vn[8];
      bool okn = true;
      if (pg + 1 < pg1) okn = load_page(pg + 1, kn, vn);
      if (okc) {
        process(kc, vc, min(P, hist - pg * P));
      } else {
        bad_page = true;
      }
      if (pg + 1 < pg1) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          kc[i] = kn[i];
          vc[i] = vn[i];
        }
        okc = okn;
      }
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
  if (parity != 0) return;

  const std::size_t out_row0 = qrow0;
  if (splits == 1) {
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
      reinterpret_cast<float4*>(a.out + (out_row0 + h) * D)[j] = o;
    }
    return;
  }
#pragma unroll
  for (int h = 0; h < G; ++h) {
    const std::size_t pidx = (out_row0 + h) * a.max_splits + split;
    reinterpret_cast<float4*>(a.part_o + pidx * D)[j] =
        make_float4(acc[h][0], acc[h][1], acc[h][2], acc[h][3]);
    if (j == 0) {
      a.part_ml[2 * pidx] = s_head[1][h];
      a.part_ml[2 * pidx + 1] = s_head[2][h];
    }
  }
}

// Merges the per-split (m, l, o) of every (sequence, q head) row that used
// more than one split: O = sum_c o_c * 2^(m_c - M) / sum_c l_c * 2^(m_c - M).
__global__ __launch_bounds__(64) void decode_combine_kernel(DecodeKernelArgs a) {
  constexpr int D = 128;
  constexpr int P = 16;
  const int row = blockIdx.x;  // b * q_heads + h
  const int b = row / a.q_heads;
  int hist = a.lengths[b];
  if (hist < 0 || hist > a.max_blocks * P) hist = 0;
  const int hist_pages = (hist + P - 1) / P;
  const int splits = (hist_pages + a.pages_per_split - 1) / a.pages_per_split;
  if (splits <= 1) return;
  const std::size_t base = static_cast<std::size_t>(row) * a.max_splits;
  float mx = -INFINITY;
  for (int c = 0; c < splits; ++c) mx = fmaxf(mx, a.part_ml[2 * (base + c)]);
  float den = 0.0f;
  float2 num = make_float2(0.f, 0.f);
  for (int c = 0; c < splits; ++c) {
    const float w = exp2_ratio(a.part_ml[2 * (base + c)], mx);
    den += w * a.part_ml[2 * (base + c) + 1];
    const float2 o = reinterpret_cast<const float2*>(a.part_o + (base + c) * D)[threadIdx.x];
    num.x += w * o.x;
    num.y += w * o.y;
  }
  float2 res;
  if (mx == -INFINITY) {
    res = make_float2(NAN, NAN);
  } else {
    const float inv = 1.0f / den;
    res = make_float2(num.x * inv, num.y * inv);
  }
  reinterpret_cast<float2*>(a.out + static_cast<std::size_t>(row) * D)[threadIdx.x] = res;
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

  // Pass 3: thread d accumulates sum_k p_k * V[k][d]; probabilities of a
  // 256-key tile are staged in LDS by the threads that wrote them.
  const std::size_t dv_count = a.value_dim;
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
        const std::size_t key = k0 + kk;
        const float* vrow;
        if (key < a.history) {
          const std::size_t phys = a.table[key / a.block_tokens];
          if (phys >= a.physical_blocks) {
            s = NAN;
            continue;
          }
          vrow = a.value_blocks +
                 ((phys * a.kv_heads + kvh) * a.block_tokens + key % a.block_tokens) * a.value_dim;
        } else {
          vrow = a.tail_value + (kvh * a.tail + (key - a.history)) * a.value_dim;
        }
        s += tile[kk] * vrow[d];
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

}  // namespace

// ------------------------------------------------------------ launchers ----
hipError_t launch_append_token(const float* keys, const float* values, float* key_base,
                               float* value_base, std::size_t layer_stride, std::size_t layers,
                               const PageGeometry& g, std::uint32_t block, std::size_t offset,
                               hipStream_t stream) {
  const bool vec = g.head_dim % 4 == 0 && aligned16(keys) && aligned16(values);
  const std::size_t work = layers * g.kv_heads * (vec ? g.head_dim / 4 : g.head_dim);
  dim3 grid(grid_for(work, kThreads), 2);
  if (vec) {
    append_token_kernel<float4><<<grid, kThreads, 0, stream>>>(
        keys, values, key_base, value_base, layer_stride, layers, g.kv_heads, g.block_tokens,
        g.head_dim, block, offset);
  } else {
    append_token_kernel<float><<<grid, kThreads, 0, stream>>>(
        keys, values, key_base, value_base, layer_stride, layers, g.kv_heads, g.block_tokens,
        g.head_dim, block, offset);
  }
  return hipGetLastError();
}

hipError_t launch_append_bulk(const float* const* layer_keys, const float* const* layer_values,
                              float* key_base, float* value_base, std::size_t layer_stride,
                              std::size_t layers, const PageGeometry& g,
                              const std::uint32_t* blocks, std::size_t first_block,
                              std::size_t old_length, std::size_t tokens, hipStream_t stream,
                              bool vec) {
  const std::size_t work = layers * g.kv_heads * tokens * (vec ? g.head_dim / 4 : g.head_dim);
  dim3 grid(grid_for(work, kThreads), 2);
  LayerPointers src{layer_keys, layer_values};
  if (vec) {
    append_bulk_kernel<float4><<<grid, kThreads, 0, stream>>>(
        src, key_base, value_base, layer_stride, layers, g.kv_heads, g.block_tokens, g.head_dim,
        blocks, first_block, old_length, tokens);
  } else {
    append_bulk_kernel<float><<<grid, kThreads, 0, stream>>>(
        src, key_base, value_base, layer_stride, layers, g.kv_heads, g.block_tokens, g.head_dim,
        blocks, first_block, old_length, tokens);
  }
  return hipGetLastError();
}

hipError_t launch_append_slots(const float* keys, const float* values, float* key_pool,
                               float* value_pool, const PageGeometry& g, const std::int64_t* slots,
                               std::size_t count, hipStream_t stream) {
  if (count == 0) return hipSuccess;
  const bool vec = g.head_dim % 4 == 0 && aligned16(keys) && aligned16(values);
  const std::size_t work = count * g.kv_heads * (vec ? g.head_dim / 4 : g.head_dim);
  dim3 grid(grid_for(work, kThreads), 2);
  if (vec) {
    append_slots_kernel<float4><<<grid, kThreads, 0, stream>>>(
        keys, values, key_pool, value_pool, g.kv_heads, g.block_tokens, g.head_dim, slots, count);
  } else {
    append_slots_kernel<float><<<grid, kThreads, 0, stream>>>(
        keys, values, key_pool, value_pool, g.kv_heads, g.block_tokens, g.head_dim, slots, count);
  }
  return hipGetLastError();
}

hipError_t launch_gather(const float* key_pool, const float* value_pool, const PageGeometry& g,
                         const std::uint32_t* blocks, std::size_t length, float* keys_out,
                         float* values_out, std::size_t dest_tokens, hipStream_t stream) {
  if (length == 0) return hipSuccess;
  const bool vec = g.head_dim % 4 == 0 && aligned16(keys_out) && aligned16(values_out);
  const std::size_t work = g.kv_heads * length * (vec ? g.head_dim / 4 : g.head_dim);
  dim3 grid(grid_for(work, kThreads), 2);
  if (vec) {
    gather_kernel<float4><<<grid, kThreads, 0, stream>>>(key_pool, value_pool, g.kv_heads,
                                                         g.block_tokens, g.head_dim, blocks,
                                                         length, keys_out, values_out, dest_tokens);
  } else {
    gather_kernel<float><<<grid, kThreads, 0, stream>>>(key_pool, value_pool, g.kv_heads,
                                                        g.block_tokens, g.head_dim, blocks, length,
                                                        keys_out, values_out, dest_tokens);
  }
  return hipGetLastError();
}

hipError_t launch_page_copy(float* key_base, float* value_base, std::size_t layer_stride,
                            std::size_t layers, const PageGeometry& g, std::uint32_t from,
                            std::uint32_t to, std::size_t tokens, hipStream_t stream) {
  if (tokens == 0) return hipSuccess;
  const bool vec = g.head_dim % 4 == 0;
  const std::size_t work = layers * g.kv_heads * tokens * (vec ? g.head_dim / 4 : g.head_dim);
  dim3 grid(grid_for(work, kThreads), 2);
  if (vec) {
    page_copy_kernel<float4><<<grid, kThreads, 0, stream>>>(key_base, value_base, layer_stride,
                                                            layers, g.kv_heads, g.block_tokens,
                                                            g.head_dim, from, to, tokens);
  } else {
    page_copy_kernel<float><<<grid, kThreads, 0, stream>>>(key_base, value_base, layer_stride,
                                                           layers, g.kv_heads, g.block_tokens,
                                                           g.head_dim, from, to, tokens);
  }
  return hipGetLastError();
}

hipError_t launch_table_updates(std::uint32_t* tables, std::size_t cols,
                                const std::uint32_t* updates, std::size_t count,
                                hipStream_t stream) {
  if (count == 0) return hipSuccess;
  table_update_kernel<<<grid_for(count, kThreads), kThreads, 0, stream>>>(tables, cols, updates,
                                                                         count);
  return hipGetLastError();
}

std::size_t decode_max_splits(std::size_t max_blocks, std::size_t pages_per_split) {
  const std::size_t s = (max_blocks + pages_per_split - 1) / pages_per_split;
  return s == 0 ? 1 : s;
}

std::size_t decode_workspace_bytes(std::size_t batch, std::size_t q_heads, std::size_t max_blocks,
                                   std::size_t pages_per_split) {
  const std::size_t splits = decode_max_splits(max_blocks, pages_per_split);
  return batch * q_heads * splits * (kDecodeHeadDim + 2) * sizeof(float);
}

bool decode_group_supported(std::size_t group) {
  return group == 1 || group == 2 || group == 4 || group == 8;
}

hipError_t launch_decode(const DecodeArgs& a, hipStream_t stream) {
  if (a.batch == 0) return hipSuccess;
  const std::size_t splits = decode_max_splits(a.max_blocks, a.pages_per_split);
  DecodeKernelArgs k{};
  k.query = a.query;
  k.key_pool = a.key_pool;
  k.value_pool = a.value_pool;
  k.tables = a.tables;
  k.lengths = a.lengths;
  k.tail_key = a.tail_key;
  k.tail_value = a.tail_value;
  k.out = a.out;
  k.part_o = static_cast<float*>(a.workspace);
  k.part_ml = k.part_o + a.batch * a.q_heads * splits * kDecodeHeadDim;
  k.q_heads = static_cast<int>(a.q_heads);
  k.kv_heads = static_cast<int>(a.kv_heads);
  k.max_blocks = static_cast<int>(a.max_blocks);
  k.max_splits = static_cast<int>(splits);
  k.pages_per_split = static_cast<int>(a.pages_per_split);
  k.physical_blocks = static_cast<std::uint32_t>(a.physical_blocks);
  k.qscale = kLog2e / sqrtf(static_cast<float>(kDecodeHeadDim));
  dim3 grid(static_cast<unsigned>(splits), static_cast<unsigned>(a.batch * a.kv_heads));
  switch (a.q_heads / a.kv_heads) {
    case 1: decode_split_kernel<1><<<grid, 64, 0, stream>>>(k); break;
    case 2: decode_split_kernel<2><<<grid, 64, 0, stream>>>(k); break;
    case 4: decode_split_kernel<4><<<grid, 64, 0, stream>>>(k); break;
    case 8: decode_split_kernel<8><<<grid, 64, 0, stream>>>(k); break;
    default: return hipErrorInvalidValue;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (splits > 1) {
    decode_combine_kernel<<<static_cast<unsigned>(a.batch * a.q_heads), 64, 0, stream>>>(k);
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_generic(const GenericArgs& a, hipStream_t stream) {
  if (a.queries == 0 || a.q_heads == 0) return hipSuccess;
  dim3 grid(static_cast<unsigned>(a.queries), static_cast<unsigned>(a.q_heads));
  generic_attention_kernel<<<grid, kThreads, 0, stream>>>(a);
  return hipGetLastError();
}

}  // namespace helix::hip
