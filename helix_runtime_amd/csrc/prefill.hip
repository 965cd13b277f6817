// Chunked-prefill attention on the CDNA4 matrix cores (fp32 MFMA): the
// standalone kernel and its launches.  The workgroup code, its design notes
// and the special-value rules are in prefill_body.hpp.
#include "prefill_body.hpp"
#include "prefill_bmma.hpp"

#include <hip/hip_runtime.h>

#include <cstdint>

namespace helix::hip {
namespace {

using namespace prefill_detail;

template <int G, bool CASCADE, int PF, int RT>
__global__ __launch_bounds__(512 / RT, 6 - 2 * RT)
void prefill_kernel(PrefillKernelArgs a, const std::uint32_t* __restrict__ tables,
                    const std::uint32_t* __restrict__ order) {
  __shared__ PrefillShared sh;
  prefill_body<G, CASCADE, PF, RT>(a, tables, order, blockIdx.x, sh);
}

// The exact kernel that also leaves the softmax probabilities (the
// reference-shaped chunk call, fp32 pages).
template <int G>
__global__ __launch_bounds__(512 / kTilesPerWave, 6 - 2 * kTilesPerWave)
void prefill_probs_kernel(PrefillKernelArgs a, const std::uint32_t* __restrict__ tables,
                          const std::uint32_t* __restrict__ order) {
  __shared__ PrefillShared sh;
  prefill_body<G, false, 0, kTilesPerWave, false, PrefillShared, true>(a, tables, order,
                                                                       blockIdx.x, sh);
}

// Finishes the reference-shaped chunk call.  Workgroup (row, s), row =
// q head * tokens + position: merges the row's key-range partials into its
// maximum and sum, rewrites keys [s * 2048, s * 2048 + 2048) of the row's
// workspace entries from scores to probabilities (keys the row sees,
// [0, history + position + 1), become exp2(x - m) / l, the rest 0; a row
// without a finite maximum or with a NaN sum is NaN throughout,
// src/kernels/cpu/reference.cpp:264-316), and workgroup s = 0 writes the
// output row.  All of a thread's loads are issued at once.
constexpr int kNormUnroll = static_cast<int>(kRefNormKeys / 256);
constexpr int kMaxProbSplits = 8;
__global__ __launch_bounds__(256) void prob_normalize_kernel(float* __restrict__ probs,
                                                             const float* __restrict__ ml,
                                                             const float* __restrict__ po,
                                                             float* __restrict__ out,
                                                             int splits, int tokens, int history,
                                                             int keys) {
  const std::size_t row = blockIdx.x;
  const int pos = static_cast<int>(row % static_cast<std::size_t>(tokens));
  const int seen = history + pos + 1;
  float* pr = probs + row * static_cast<std::size_t>(keys);
  const int k0 = static_cast<int>(blockIdx.y) * 256 * kNormUnroll + threadIdx.x;
  float x[kNormUnroll];
#pragma unroll
  for (int u = 0; u < kNormUnroll; ++u) {
    const int k = k0 + u * 256;
    x[u] = k < seen ? pr[k] : 0.0f;
  }
  float ms[kMaxProbSplits], ls[kMaxProbSplits];
  float m = -INFINITY;
#pragma unroll
  for (int s = 0; s < kMaxProbSplits; ++s) {
    ms[s] = s < splits ? ml[(row * splits + s) * 2] : -INFINITY;
    ls[s] = s < splits ? ml[(row * splits + s) * 2 + 1] : 0.0f;
    m = fmaxf(m, ms[s]);
  }
  float l = 0.0f;
#pragma unroll
  for (int s = 0; s < kMaxProbSplits; ++s) {
    if (s < splits) l += exp2_ratio(ms[s], m) * ls[s];
  }
  const bool nan_row = m == -INFINITY || isnan(l);
  if (blockIdx.y == 0 && threadIdx.x < D / 4) {
    float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int s = 0; s < kMaxProbSplits; ++s) {
      if (s < splits) {
        const float w = exp2_ratio(ms[s], m);
        const float4 v = reinterpret_cast<const float4*>(po + (row * splits + s) * D)[threadIdx.x];
        o.x += w * v.x;
        o.y += w * v.y;
        o.z += w * v.z;
        o.w += w * v.w;
      }
    }
    const float inv = 1.0f / l;
    reinterpret_cast<float4*>(out + row * D)[threadIdx.x] =
        nan_row ? make_float4(NAN, NAN, NAN, NAN)
                : make_float4(o.x * inv, o.y * inv, o.z * inv, o.w * inv);
  }
#pragma unroll
  for (int u = 0; u < kNormUnroll; ++u) {
    const int k = k0 + u * 256;
    if (k < keys) pr[k] = nan_row ? NAN : (k < seen ? exp2_ratio(x[u], m) / l : 0.0f);
  }
}

// The exact kernel over the blocks the matrix-core launch flagged (every
// other block returns at once).
template <int G, int PF, int RT>
__global__ __launch_bounds__(512 / RT, 6 - 2 * RT)
void prefill_redo_kernel(PrefillKernelArgs a, const std::uint32_t* __restrict__ tables,
                         const std::uint32_t* __restrict__ order,
                         const std::uint32_t* __restrict__ redo) {
  if (redo[blockIdx.x] == 0) return;
  __shared__ PrefillShared sh;
  prefill_body<G, false, PF, RT>(a, tables, order, blockIdx.x, sh);
}

// Tiles per wavefront of the bf16 matrix-core prefill: one (8 wavefronts
// of 16 rows) keeps two of the query operand's three terms (the third is
// in LDS), the accumulators and the staging of a wavefront within 128
// VGPRs, four wavefronts per SIMD.
constexpr int kBmmaTilesPerWave = 1;

template <int G, int PF, int RT>
__global__ __launch_bounds__(512 / RT, 6 - 2 * RT)
void prefill_bmma_kernel(PrefillKernelArgs a, const std::uint32_t* __restrict__ tables,
                         const std::uint32_t* __restrict__ order,
                         std::uint32_t* __restrict__ redo) {
  __shared__ PrefillBmmaShared sh;
  prefill_body_bmma<G, PF, RT>(a, tables, order, redo, blockIdx.x, sh);
}

// fp32 pages with a redo array: the fast variant of the fp32 kernel (no
// exact paths, one tile per wavefront, four wavefronts per SIMD), then the
// exact kernel over the work items it flagged.
constexpr int kFastTilesPerWave = 1;
template <int G>
__global__ __launch_bounds__(512 / kFastTilesPerWave, 6 - 2 * kFastTilesPerWave)
void prefill_fast_kernel(PrefillKernelArgs a, const std::uint32_t* __restrict__ tables,
                         const std::uint32_t* __restrict__ order,
                         std::uint32_t* __restrict__ redo) {
  __shared__ PrefillShared sh;
  prefill_body<G, false, 0, kFastTilesPerWave, true>(a, tables, order, blockIdx.x, sh, redo);
}

template <int G>
void launch_fast(const dim3& grid, hipStream_t stream, const PrefillKernelArgs& k,
                 const std::uint32_t* tables, const std::uint32_t* order, std::uint32_t* redo) {
  prefill_fast_kernel<G><<<grid, 512 / kFastTilesPerWave, 0, stream>>>(k, tables, order, redo);
  prefill_redo_kernel<G, 0, kTilesPerWave><<<grid, 512 / kTilesPerWave, 0, stream>>>(
      k, tables, order, redo);
}

// bf16 / fp8 pages with a redo array: the bf16 matrix-core kernel, then the
// exact kernel over the work items it flagged.
template <int G, int PF>
void launch_bmma(const dim3& grid, hipStream_t stream, const PrefillKernelArgs& k,
                 const std::uint32_t* tables, const std::uint32_t* order,
                 std::uint32_t* redo) {
  constexpr int BRT = kBmmaTilesPerWave;
  prefill_bmma_kernel<G, PF, BRT><<<grid, 512 / BRT, 0, stream>>>(k, tables, order, redo);
  prefill_redo_kernel<G, PF, kTilesPerWave><<<grid, 512 / kTilesPerWave, 0, stream>>>(
      k, tables, order, redo);
}

template <int G, bool CASCADE, int RT = kTilesPerWave>
void launch_variant(const dim3& grid, hipStream_t stream, const PrefillKernelArgs& k,
                    const std::uint32_t* tables, const std::uint32_t* order, PageType type) {
  switch (type) {
    case PageType::kBF16:
      prefill_kernel<G, CASCADE, 1, RT><<<grid, 512 / RT, 0, stream>>>(k, tables, order);
      break;
    case PageType::kFP8:
      prefill_kernel<G, CASCADE, 2, RT><<<grid, 512 / RT, 0, stream>>>(k, tables, order);
      break;
    default:
      prefill_kernel<G, CASCADE, 0, RT><<<grid, 512 / RT, 0, stream>>>(k, tables, order);
      break;
  }
}

}  // namespace

std::size_t prefill_position_block(std::size_t group) { return kRows / group; }

std::size_t prefill_prob_splits(std::size_t q_heads, std::size_t kv_heads, std::size_t tokens,
                                std::size_t keys, int cus) {
  // About two workgroups per CU (the exact kernel's occupancy), with at
  // least four 16-key blocks per range on average.  Config-5 calls (128
  // items per sequence): 4 ranges 338 us per call, 3 ranges 379, 6 ranges
  // 383, 8 ranges 366.
  const std::size_t pw = kRows / (q_heads / kv_heads);
  const std::size_t items = kv_heads * ((tokens + pw - 1) / pw);
  const std::size_t target = 2 * static_cast<std::size_t>(cus > 0 ? cus : 256);
  std::size_t s = (target + items - 1) / items;
  const std::size_t by_keys = (keys + 63) / 64;
  if (s > by_keys) s = by_keys;
  if (s > static_cast<std::size_t>(kMaxProbSplits)) s = kMaxProbSplits;
  return s == 0 ? 1 : s;
}

// Key pages per cascade work item: enough chunks that the launch has about
// one workgroup per CU, at most kMaxCascadeChunks chunks.  Every extra chunk
// re-loads the query tile, writes one more partial per row and adds merge
// work; beyond one workgroup per CU that costs more than the added
// parallelism gains (128 sequences x 32 heads: 8 chunks beat both 16 and 4).
std::size_t cascade_chunk_pages(std::size_t shared_pages, std::size_t batch, std::size_t group,
                                std::size_t kv_heads) {
  // Work items the key chunks aim for.  Beside a side-stream stream kernel:
  // one prefix workgroup per CU.  In the fused launch, where every CU also
  // holds stream wavefronts, fewer and longer prefix items do better: they
  // reload fewer query tiles and leave fewer partials to merge (config 4,
  // 32-layer step: 4 chunks 2.65 ms, 5 chunks 2.62 ms, 6 chunks 2.67 ms,
  // 8 chunks 2.84 ms, 16 chunks 3.38 ms).
  const std::size_t kCascadeTarget = group <= kCascadeFusedMaxGroup ? 160 : 256;
  const std::size_t items = ((batch * group + kRows - 1) / kRows) * kv_heads;
  std::size_t chunks = (kCascadeTarget + items - 1) / items;
  if (chunks > kMaxCascadeChunks) chunks = kMaxCascadeChunks;
  if (chunks > shared_pages) chunks = shared_pages;
  if (chunks == 0) chunks = 1;
  return (shared_pages + chunks - 1) / chunks;
}

bool prefill_group_supported(std::size_t group) {
  return group == 1 || group == 2 || group == 4 || group == 8;
}

hipError_t launch_prefill(const PrefillArgs& a, hipStream_t stream) {
  if (a.batch == 0 || a.tokens == 0) return hipSuccess;
  const std::size_t group = a.q_heads / a.kv_heads;
  const std::size_t pw = kRows / group;
  PrefillKernelArgs k{};
  k.query = a.query;
  k.key_pool = a.key_pool;
  k.value_pool = a.value_pool;
  k.lengths = a.lengths;
  k.chunk_key = a.chunk_key;
  k.chunk_value = a.chunk_value;
  k.out = a.out;
  k.q_heads = static_cast<int>(a.q_heads);
  k.kv_heads = static_cast<int>(a.kv_heads);
  k.tokens = static_cast<int>(a.tokens);
  k.max_blocks = static_cast<int>(a.max_blocks);
  k.pos_blocks = static_cast<int>((a.tokens + pw - 1) / pw);
  k.physical_blocks = static_cast<std::uint32_t>(a.physical_blocks);
  k.qscale = kLog2e / sqrtf(static_cast<float>(D));
  k.batch = static_cast<int>(a.batch);
  k.k_scale = a.page_type.k_scale;
  k.v_scale = a.page_type.v_scale;
  k.single_length = a.single_length;
  k.probs = a.probs;
  k.prob_keys = static_cast<int>(a.prob_keys);
  k.prob_ml = a.prob_ml;
  dim3 grid(static_cast<unsigned>(k.pos_blocks * a.kv_heads * a.batch));
  if (a.probs != nullptr) {
    if (a.page_type.type != PageType::kF32 || a.redo != nullptr || a.batch != 1 ||
        a.lengths != nullptr || a.prob_ml == nullptr || a.prob_o == nullptr ||
        a.prob_splits < 1 || a.prob_splits > static_cast<std::size_t>(kMaxProbSplits)) {
      return hipErrorInvalidValue;
    }
    k.prob_splits = static_cast<int>(a.prob_splits);
    k.prob_o = a.prob_o;
    grid.x *= static_cast<unsigned>(a.prob_splits);
    constexpr unsigned threads = 512 / kTilesPerWave;
    switch (group) {
      case 1: prefill_probs_kernel<1><<<grid, threads, 0, stream>>>(k, a.tables, a.order); break;
      case 2: prefill_probs_kernel<2><<<grid, threads, 0, stream>>>(k, a.tables, a.order); break;
      case 4: prefill_probs_kernel<4><<<grid, threads, 0, stream>>>(k, a.tables, a.order); break;
      case 8: prefill_probs_kernel<8><<<grid, threads, 0, stream>>>(k, a.tables, a.order); break;
      default: return hipErrorInvalidValue;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 ngrid(static_cast<unsigned>(a.q_heads * a.tokens),
                     static_cast<unsigned>((a.prob_keys + 256 * kNormUnroll - 1) /
                                           (256 * kNormUnroll)));
    prob_normalize_kernel<<<ngrid, 256, 0, stream>>>(
        a.probs, a.prob_ml, a.prob_o, a.out, static_cast<int>(a.prob_splits),
        static_cast<int>(a.tokens), a.single_length, static_cast<int>(a.prob_keys));
    return hipGetLastError();
  }
  if (a.redo != nullptr && a.page_type.type == PageType::kF32) {
    switch (group) {
      case 1: launch_fast<1>(grid, stream, k, a.tables, a.order, a.redo); break;
      case 2: launch_fast<2>(grid, stream, k, a.tables, a.order, a.redo); break;
      case 4: launch_fast<4>(grid, stream, k, a.tables, a.order, a.redo); break;
      case 8: launch_fast<8>(grid, stream, k, a.tables, a.order, a.redo); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  if (a.redo != nullptr) {
    const bool fp8 = a.page_type.type == PageType::kFP8;
    switch (group) {
      case 1: fp8 ? launch_bmma<1, 2>(grid, stream, k, a.tables, a.order, a.redo)
                  : launch_bmma<1, 1>(grid, stream, k, a.tables, a.order, a.redo); break;
      case 2: fp8 ? launch_bmma<2, 2>(grid, stream, k, a.tables, a.order, a.redo)
                  : launch_bmma<2, 1>(grid, stream, k, a.tables, a.order, a.redo); break;
      case 4: fp8 ? launch_bmma<4, 2>(grid, stream, k, a.tables, a.order, a.redo)
                  : launch_bmma<4, 1>(grid, stream, k, a.tables, a.order, a.redo); break;
      case 8: fp8 ? launch_bmma<8, 2>(grid, stream, k, a.tables, a.order, a.redo)
                  : launch_bmma<8, 1>(grid, stream, k, a.tables, a.order, a.redo); break;
      default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
  }
  switch (group) {
    case 1: launch_variant<1, false>(grid, stream, k, a.tables, a.order, a.page_type.type); break;
    case 2: launch_variant<2, false>(grid, stream, k, a.tables, a.order, a.page_type.type); break;
    case 4: launch_variant<4, false>(grid, stream, k, a.tables, a.order, a.page_type.type); break;
    case 8: launch_variant<8, false>(grid, stream, k, a.tables, a.order, a.page_type.type); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

prefill_detail::PrefillKernelArgs prefill_detail::cascade_prefix_args(const CascadePrefixArgs& a,
                                                     std::size_t* work_items) {
  const std::size_t group = a.q_heads / a.kv_heads;
  PrefillKernelArgs k{};
  k.query = a.query;
  k.key_pool = a.key_pool;
  k.value_pool = a.value_pool;
  k.q_heads = static_cast<int>(a.q_heads);
  k.kv_heads = static_cast<int>(a.kv_heads);
  k.tokens = 1;
  k.max_blocks = static_cast<int>(a.shared_pages);
  k.pos_blocks = static_cast<int>((a.batch * group + kRows - 1) / kRows);
  k.physical_blocks = static_cast<std::uint32_t>(a.physical_blocks);
  k.qscale = kLog2e / sqrtf(static_cast<float>(D));
  k.batch = static_cast<int>(a.batch);
  k.cascade_keys = static_cast<int>(a.shared_pages * P);
  k.cascade_chunk_pages = static_cast<int>(cascade_chunk_pages(a.shared_pages, a.batch, group,
                                                               a.kv_heads));
  k.part_o = a.part_o;
  k.part_ml = a.part_ml;
  k.prefix_slot0 = static_cast<long long>(a.prefix_slot0);
  k.k_scale = a.page_type.k_scale;
  k.v_scale = a.page_type.v_scale;
  const std::size_t chunks =
      (a.shared_pages + k.cascade_chunk_pages - 1) / k.cascade_chunk_pages;
  k.cascade_chunks = static_cast<int>(chunks);
  *work_items = static_cast<std::size_t>(k.pos_blocks) * a.kv_heads * chunks;
  return k;
}

hipError_t launch_cascade_prefix(const CascadePrefixArgs& a, hipStream_t stream) {
  if (a.batch == 0 || a.shared_pages == 0) return hipSuccess;
  const std::size_t group = a.q_heads / a.kv_heads;
  std::size_t items = 0;
  const PrefillKernelArgs k = cascade_prefix_args(a, &items);
  const dim3 grid(static_cast<unsigned>(items));
  switch (group) {
    case 1: launch_variant<1, true, kCascadeTilesPerWave>(grid, stream, k, a.table, nullptr, a.page_type.type); break;
    case 2: launch_variant<2, true, kCascadeTilesPerWave>(grid, stream, k, a.table, nullptr, a.page_type.type); break;
    case 4: launch_variant<4, true, kCascadeTilesPerWave>(grid, stream, k, a.table, nullptr, a.page_type.type); break;
    case 8: launch_variant<8, true, kCascadeTilesPerWave>(grid, stream, k, a.table, nullptr, a.page_type.type); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace helix::hip
