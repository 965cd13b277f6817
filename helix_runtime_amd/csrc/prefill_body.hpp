// Device code of the chunked-prefill attention workgroup (fp32 MFMA on the
// CDNA4 matrix cores), shared by the standalone prefill kernel and the fused
// cascade decode launch.
//
// The reference runs prefill through the same paged attention as decode,
// with T query rows and a T-token uncommitted tail
// (src/attention/paged_reference.cpp:173-384, cuda_paged.cu:483-548): query
// row q sees every history token and tail tokens 0..q.  For T = 512 that is
// dense work, so it is computed as a flash-attention style tiled product on
// v_mfma_f32_16x16x4_f32 with fp32 operands and fp32 accumulation.
//
// Work decomposition.  A workgroup (4 wavefronts) owns one (sequence, kv
// head) and 128 query rows: the G = q_heads / kv_heads query heads of that
// kv head times 128 / G consecutive chunk positions, so every K/V byte
// staged in LDS feeds all G heads.  Each wavefront holds 32 of those rows
// (two 16-row tiles) and keeps its Q rows in registers.  Keys stream through
// LDS one page (16 keys) at a time: history pages through the block table,
// then the chunk rows.  With fp32 pages the stages are filled by direct
// global -> LDS loads three blocks ahead; bf16 pages and the cascade
// prefix pass stage through registers into two stages.
//
// Layout trick.  Scores are computed transposed, S^T = K Q^T, so the MFMA
// result leaves each lane holding 4 keys of one query row; the row's max and
// sum then need only two cross-lane steps, and the transposed product
// O^T = V^T P^T takes those probabilities as its B operand unchanged and
// accumulates O with the same row per lane, so the online-softmax rescale is
// lane local.  The reduction dimension of each MFMA is visited in a permuted
// order (the same for both operands), which lets every operand fetch be one
// 128-bit LDS read.
//
// Special values follow src/kernels/cpu/reference.cpp:264-316 as in the
// decode kernel.  A masked (future) chunk value row must not reach the rows
// that do not see it: 0 * inf would be NaN where the reference skips the
// key.  Staging flags non-finite value rows that some row of the workgroup
// masks, and such a block takes an exact per-key path for P.V.
#pragma once

#include "kernels.hpp"

#include "bf16.hpp"
#include "fp8.hpp"

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <type_traits>

namespace helix::hip::prefill_detail {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v4f_a4 __attribute__((ext_vector_type(4), aligned(4)));

constexpr int D = 128;
constexpr int P = 16;
constexpr int kRows = 128;      // query rows per workgroup
// 16-row tiles per wavefront of the exact kernel: 2 (4 waves per workgroup,
// 256 VGPRs, two workgroups per CU).  With its exact paths the kernel also
// builds with 1 (8 waves, 128 VGPRs, four waves per SIMD), but then spills
// (21 VGPRs even with the direct-load staging) and measured 103.7 against
// 113.1 TFLOP/s at config 5; the fast variant (FAST below) drops those paths
// and runs one tile per wave at 118 VGPRs.
constexpr int kTilesPerWave = 2;
// The cascade prefix pass has few keys per work item and runs beside the
// stream decode kernel: 8 waves of one tile (108 VGPRs, no spills) fit two
// waves per SIMD next to a stream wavefront (107.0 against 108.1 us per
// layer back to back at config 4).
constexpr int kCascadeTilesPerWave = 1;
constexpr int kKeys = 16;       // keys per LDS stage (one page)
constexpr int kKStride = D + 4; // padded K row: 8 consecutive rows hit distinct banks
constexpr float kLog2e = 1.4426950408889634f;

struct PrefillKernelArgs {
  const float* query;
  const float* key_pool;
  const float* value_pool;
  const std::int32_t* lengths;
  const float* chunk_key;
  const float* chunk_value;
  float* out;
  int q_heads;
  int kv_heads;
  int tokens;
  int max_blocks;
  int pos_blocks;
  std::uint32_t physical_blocks;
  float qscale;
  // Cascade mode (shared-prefix decode): rows are (sequence, head) pairs of
  // one kv head, keys are the first cascade_keys tokens of table row 0, and
  // each row leaves a partial (m, l, o) at slot prefix_slot0 + kvh * batch +
  // sequence.
  int batch;
  int cascade_keys;
  int cascade_chunk_pages;  // key pages per work item (the prefix is split)
  int cascade_chunks;       // key chunks of the shared prefix
  float* part_o;
  float* part_ml;
  long long prefix_slot0;
  // fp8 pages: scales of the key and value codes.
  float k_scale;
  float v_scale;
  // History of a one-sequence launch whose length is a host value
  // (lengths == nullptr).
  int single_length;
  // Probabilities (the PROBS kernels): row (head * tokens + position) of
  // probs, prob_keys entries long, receives the softmax probabilities of
  // that query row over keys [0, prob_keys); keys the row does not see get 0.
  float* probs;
  int prob_keys;
  // PROBS: each work item's key blocks are split into prob_splits ranges,
  // one per work item; every (row, split) leaves its maximum and sum in
  // prob_ml [rows, prob_splits, 2] and its unnormalised output in prob_o
  // [rows, prob_splits, 128] for prob_normalize_kernel to merge.
  int prob_splits;
  float* prob_ml;
  float* prob_o;
};

// exp2(a - b), with a == b (also +inf == +inf, -inf == -inf) giving 1 and
// a = -inf < b giving 0.  v_exp_f32 directly: results below 2^-126 flush to
// zero, far under the tolerance of a probability normalised by a sum >= 1.
__device__ __forceinline__ float exp2_ratio(float a, float b) {
  return a == b ? 1.0f : __builtin_amdgcn_exp2f(a - b);
}

// Max / sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one query row's
// four key groups) with the cross-row lane swaps.
__device__ __forceinline__ float row_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(t[0]), __uint_as_float(t[1]));
}
__device__ __forceinline__ float row_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto t = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(t[0]) + __uint_as_float(t[1]);
}

__device__ __forceinline__ float comp(const float4& v, int c) {
  return c == 0 ? v.x : c == 1 ? v.y : c == 2 ? v.z : v.w;
}

__device__ __forceinline__ bool finite4(const float4& v) {
  return isfinite(v.x) && isfinite(v.y) && isfinite(v.z) && isfinite(v.w);
}

// PF (page format, the PageType value): fp32 (0), bf16 (1) or fp8 E4M3 (2)
// pages.  For bf16 and fp8 the staging widens history rows (fp8: times the
// pool's scale) and rounds the fp32 chunk rows onto the same grid (the
// values their pages will hold), so the math is the fp32 kernel's on
// operands exact on that grid.
// RT: 16-row tiles per wavefront (1 or 2); the workgroup has 8 / RT waves
// and each SIMD runs 6 - 2 * RT of them.
// LDS of one prefill workgroup.  fp32 pages: three K and three V stages
// filled by direct global -> LDS loads; K rows unpadded with their 16-byte
// chunks XOR-swizzled by row (chunk j of row r at j ^ (r & 15)), so the
// MFMA operand reads (16 rows, one chunk) hit distinct banks.  bf16 and fp8
// pages: two register-staged stages (the widening happens on the way), K rows
// padded to kKStride floats.
constexpr int kDmaStages = 4;
struct PrefillRegStages {
  __align__(16) float k[2][kKeys * kKStride];
  __align__(16) float v[2][kKeys * D];
};
struct PrefillDmaStages {
  __align__(16) float k[kDmaStages][kKeys * D];
  __align__(16) float v[kDmaStages][kKeys * D];
};
// The standalone prefill kernel holds either layout; the cascade prefix
// pass (register staging only) holds just the smaller one.
struct PrefillShared {
  union {
    PrefillDmaStages dma;
    PrefillRegStages reg;
  };
};
struct CascadePrefixShared {
  PrefillRegStages reg;
};
__device__ __forceinline__ PrefillDmaStages* dma_stages(PrefillShared& s) { return &s.dma; }
__device__ __forceinline__ PrefillDmaStages* dma_stages(CascadePrefixShared&) { return nullptr; }

// 64 zero float4: the source of the direct loads of rows past the key range.
__device__ const float4 kZeroRows[64] = {};

// One direct global -> LDS load of 16 bytes per lane: lane i's bytes land at
// LDS byte address lds + 16 i.  Issued from inline assembly so that the
// compiler does not order its own LDS reads behind every pending load; the
// caller waits with an explicit vmcnt before reading the stage and joins
// the workgroup at a barrier.
__device__ __forceinline__ void lds_load16(const void* src, unsigned lds) {
  // M0 (the LDS base of the load) is an operand the compiler sets; the
  // nop is the wait state a write of M0 needs before an LDS-DMA load.
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ unsigned lds_address(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<unsigned>(reinterpret_cast<std::uintptr_t>(p)));
}

// The body of one prefill (or cascade prefix) workgroup; `block` is its
// work-item index (the block index of the standalone kernel).
// FAST (standalone prefill with a redo array): no exact P.V path and no
// non-finite check per block; a work item whose rows end with a NaN in
// their accumulators or sum (where a masked non-finite value row met a zero
// probability, or the exact result is NaN anyway) is flagged in
// redo[block] for the exact kernel.  Without the exact path the kernel
// fits one 16-row tile per wavefront at four wavefronts per SIMD.
// PROBS (the reference-shaped chunk call, one sequence): the key blocks of
// each (kv head, position block) are split into prob_splits ranges, one
// work item each, so a single sequence still fills the GPU.  Every score of
// the range is written (log2 domain, -inf where masked) to its probability
// entry as it is computed, and each row leaves the range's maximum, sum
// (NaN for a work item that met a bad page) and unnormalised output;
// prob_normalize_kernel merges the ranges into the output row and turns the
// scores into probabilities.
template <int G, bool CASCADE, int PF, int RT, bool FAST = false, class Shared,
          bool PROBS = false>
__device__ __forceinline__ void prefill_body(PrefillKernelArgs a,
                                             const std::uint32_t* __restrict__ tables,
                                             const std::uint32_t* __restrict__ order,
                                             std::uint32_t block, Shared& sh,
                                             std::uint32_t* __restrict__ redo = nullptr) {
  static_assert(!FAST || !CASCADE, "the fast prefill is the standalone one");
  static_assert(!PROBS || (!FAST && !CASCADE), "probabilities come from the exact kernel");
  constexpr int PW = kRows / G;  // chunk positions per workgroup
  constexpr bool BF16 = PF == 1;
  constexpr bool FP8 = PF == 2;
  constexpr bool DMA = PF == 0 && !CASCADE;
  constexpr int kKRow = DMA ? D : kKStride;  // K row stride in LDS
  PrefillDmaStages* const ds = dma_stages(sh);  // null where DMA is off
  float (&s_k)[2][kKeys * kKStride] = sh.reg.k;
  float (&s_v)[2][kKeys * D] = sh.reg.v;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;  // MFMA column: query row of the tile / dim group
  const int grp = lane >> 4;  // MFMA k group
  // Work item = (sequence, kv head, position block), packed as
  // (b * kv_heads + kvh) * pos_blocks + pb.  The caller may pass a
  // longest-first order; by default later position blocks (more keys) of a
  // (sequence, kv head) go first.
  std::uint32_t item = block;
  int split = 0;
  if constexpr (PROBS) {
    split = static_cast<int>(block % static_cast<std::uint32_t>(a.prob_splits));
    item = block / static_cast<std::uint32_t>(a.prob_splits);
  }
  int pb, kvh, b, chunk;
  if constexpr (CASCADE) {
    // Cascade items, kv head major: (kvh * chunks + chunk) * pos_blocks +
    // pb.  Every item of a kv head reads the same shared pages (each row
    // block) and the same query rows (each key chunk), so the items of one
    // kv head are given to workgroups that land on one XCD, whose L2 then
    // serves the repeats: workgroup `block` runs on XCD block % kXcds.
    const std::uint32_t n =
        static_cast<std::uint32_t>(a.pos_blocks * a.kv_heads * a.cascade_chunks);
    if (n % kXcds == 0) item = (block % kXcds) * (n / kXcds) + block / kXcds;
    pb = static_cast<int>(item % a.pos_blocks);
    chunk = static_cast<int>((item / a.pos_blocks) % a.cascade_chunks);
    kvh = static_cast<int>(item / a.pos_blocks / a.cascade_chunks);
    b = 0;
  } else {
    if (order != nullptr) {
      item = order[block];
    } else {
      const std::uint32_t x = item % a.pos_blocks;
      item = item - x + (a.pos_blocks - 1 - x);
    }
    pb = static_cast<int>(item % a.pos_blocks);
    kvh = static_cast<int>((item / a.pos_blocks) % a.kv_heads);
    b = static_cast<int>(item / a.pos_blocks / a.kv_heads);
    chunk = 0;
  }
  const int T = a.tokens;
  const int pos0 = pb * PW;

  int hist = CASCADE ? a.cascade_keys : (a.lengths != nullptr ? a.lengths[b] : a.single_length);
  bool bad = hist < 0 || hist > a.max_blocks * P;
  if (bad) hist = 0;
  int key_begin = CASCADE ? chunk * a.cascade_chunk_pages * P : 0;
  int key_end =
      CASCADE ? min(hist, (chunk + 1) * a.cascade_chunk_pages * P) : hist + min(T, pos0 + PW);
  if constexpr (PROBS) {
    // This item's share of the key blocks (possibly none).
    const int nb = (key_end + kKeys - 1) / kKeys;
    const int b0 = static_cast<int>(static_cast<long long>(nb) * split / a.prob_splits);
    const int b1 = static_cast<int>(static_cast<long long>(nb) * (split + 1) / a.prob_splits);
    key_begin = b0 * kKeys;
    key_end = min(key_end, b1 * kKeys);
  }
  // Read-only and indexed by workgroup-uniform values: scalar loads.
  const std::uint32_t* __restrict__ table = tables + static_cast<std::size_t>(b) * a.max_blocks;
  const std::size_t chunk_row0 = (static_cast<std::size_t>(b) * a.kv_heads + kvh) * T;

  // Rows of this lane: tile t holds workgroup row wave * 16 * RT + t * 16 + col.
  // Prefill: G heads x PW chunk positions of sequence b.  Cascade: row R of
  // the kv head is (sequence R / G, head R % G), one query token each.
  int qpos[RT];
  bool qvalid[RT];
  std::size_t qrow[RT];
  int r_head[RT];  // query head within the kv head's group (PROBS)
  float4 q[RT][8];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int r = wave * (16 * RT) + t * 16 + col;
    if constexpr (CASCADE) {
      const int row = pb * kRows + r;
      const int seq = row / G;
      qvalid[t] = seq < a.batch;
      qpos[t] = 0x3fffffff;  // no causal limit: every prefix key is visible
      qrow[t] = (static_cast<std::size_t>(qvalid[t] ? seq : 0) * a.q_heads + kvh * G + row % G) * D;
    } else {
      const int head = kvh * G + r / PW;
      r_head[t] = r / PW;
      qpos[t] = pos0 + r % PW;
      qvalid[t] = qpos[t] < T;
      qrow[t] = ((static_cast<std::size_t>(b) * a.q_heads + head) * T + qpos[t]) * D;
    }
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (qvalid[t]) v = *reinterpret_cast<const float4*>(a.query + qrow[t] + 16 * c + 4 * grp);
      q[t][c] = make_float4(v.x * a.qscale, v.y * a.qscale, v.z * a.qscale, v.w * a.qscale);
    }
  }

  v4f o[RT][2][4];  // [tile][dim half][component]: O^T tiles
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int c = 0; c < 4; ++c) o[t][h][c] = v4f{0.f, 0.f, 0.f, 0.f};
  float m[RT], l[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m[t] = -INFINITY;
    l[t] = 0.f;
  }

  // Staging: thread tid moves float4 column tid % 32 of key rows
  // tid / 32 + RP * r (r < RT) of a 16-key block, for K and V.
  constexpr int RP = 16 / RT;  // rows per staging pass
  const int srow = tid >> 5;
  const int scol = tid & 31;
  float4 stk[RT], stv[RT];
  // A 16-key block is exactly one page, so a history block needs one
  // (uniform) table entry.  The non-finite check runs at store time, when
  // the values have arrived, so the loads stay in flight across the block's
  // compute.
  // lane_off: this lane's float offset inside a 16-row block (page or chunk).
  const int lane_off = srow * D + scol * 4;
  auto stage_load = [&](int blk) {
    const int key0 = blk * kKeys;
    // Uniform bases: the history page of this block and the chunk rows.
    std::size_t page_off = 0;  // element offset of this block's page in the layer pool
    bool page_ok = false;
    if (key0 < hist) {
      const std::uint32_t page = table[blk];
      page_ok = page < a.physical_blocks;
      bad = bad || !page_ok;
      page_off = page_ok ? (static_cast<std::size_t>(page) * a.kv_heads + kvh) * P * D : 0;
    }
    const long long crow = static_cast<long long>(chunk_row0) + key0 - hist;
    const float* kchunk = a.chunk_key + crow * D;
    const float* vchunk = a.chunk_value + crow * D;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int key = key0 + srow + RP * r;
      const bool in_hist = key < hist;
      const bool valid = key < key_end && (!in_hist || page_ok);
      const int o = lane_off + RP * r * D;
      if constexpr (FP8) {
        // History rows: 4 fp8 codes in the low word; chunk rows: fp32.
        stk[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        stv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid && in_hist) {
          const std::size_t e = page_off + o;
          stk[r].x = __uint_as_float(*reinterpret_cast<const unsigned*>(
              reinterpret_cast<const unsigned char*>(a.key_pool) + e));
          stv[r].x = __uint_as_float(*reinterpret_cast<const unsigned*>(
              reinterpret_cast<const unsigned char*>(a.value_pool) + e));
        } else if (valid) {
          stk[r] = *reinterpret_cast<const float4*>(kchunk + o);
          stv[r] = *reinterpret_cast<const float4*>(vchunk + o);
        }
      } else if constexpr (BF16) {
        // History rows: 4 bf16 in the low two words; chunk rows: fp32.
        stk[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        stv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (valid && in_hist) {
          const std::size_t e = page_off + o;
          const uint2 kw = *reinterpret_cast<const uint2*>(
              reinterpret_cast<const unsigned short*>(a.key_pool) + e);
          const uint2 vw = *reinterpret_cast<const uint2*>(
              reinterpret_cast<const unsigned short*>(a.value_pool) + e);
          stk[r] = make_float4(__uint_as_float(kw.x), __uint_as_float(kw.y), 0.f, 0.f);
          stv[r] = make_float4(__uint_as_float(vw.x), __uint_as_float(vw.y), 0.f, 0.f);
        } else if (valid) {
          stk[r] = *reinterpret_cast<const float4*>(kchunk + o);
          stv[r] = *reinterpret_cast<const float4*>(vchunk + o);
        }
      } else {
        const float* kp = (in_hist ? a.key_pool + page_off : kchunk) + o;
        const float* vp = (in_hist ? a.value_pool + page_off : vchunk) + o;
        stk[r] = valid ? *reinterpret_cast<const float4*>(kp) : make_float4(0.f, 0.f, 0.f, 0.f);
        stv[r] = valid ? *reinterpret_cast<const float4*>(vp) : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
  };
  // Returns whether a staged value row is non-finite and some query row of
  // this workgroup masks it (a chunk row past the first position).
  auto stage_store = [&](int buf, int blk) {
    bool nonfinite = false;
#pragma unroll
    for (int r = 0; r < RT; ++r) {
      const int kr = srow + RP * r;
      const int key = blk * kKeys + kr;
      float4 kv = stk[r];
      float4 vv = stv[r];
      if constexpr (FP8) {
        if (key < hist) {
          kv = fp8_widen4(__float_as_uint(kv.x), a.k_scale);
          vv = fp8_widen4(__float_as_uint(vv.x), a.v_scale);
        } else {
          kv = fp8_rounded(kv, a.k_scale);
          vv = fp8_rounded(vv, a.v_scale);
        }
      } else if constexpr (BF16) {
        if (key < hist) {
          kv = bf16_widen(__float_as_uint(kv.x), __float_as_uint(kv.y));
          vv = bf16_widen(__float_as_uint(vv.x), __float_as_uint(vv.y));
        } else {
          kv = bf16_rounded(kv);
          vv = bf16_rounded(vv);
        }
      }
      *reinterpret_cast<float4*>(&s_k[buf][kr * kKStride + scol * 4]) = kv;
      *reinterpret_cast<float4*>(&s_v[buf][kr * D + scol * 4]) = vv;
      if (!CASCADE && key >= hist + pos0 + 1 && key < key_end && !finite4(vv)) {
        nonfinite = true;
      }
    }
    return nonfinite;
  };

  // Only a block holding chunk rows past the workgroup's first position can
  // carry a masked value row; every other block needs a plain barrier
  // (__syncthreads_or costs two more).
  auto staged_barrier = [&](bool nonfinite, int blk) -> int {
    if (!FAST && !CASCADE && blk * kKeys + kKeys > hist + pos0 + 1) {
      return __syncthreads_or(nonfinite);
    }
    __syncthreads();
    return 0;
  };
  // Direct-load staging (fp32 pages).  A block's 8 KiB of K (and of V) is
  // 8 wave loads of 1 KiB = 2 rows; wave w issues loads w * IPW .. + IPW - 1
  // of each, lane i covering row 2 c + i / 32, LDS chunk i % 32.
  constexpr int kWaves = 8 / RT;
  constexpr int IPW = 8 / kWaves;
  auto dma_issue = [&](int blk) {
    const int sbuf = blk % kDmaStages;
    const int key0 = blk * kKeys;
    std::size_t page_off = 0;
    bool page_ok = false;
    if (key0 < hist) {
      const std::uint32_t page = table[blk];
      page_ok = page < a.physical_blocks;
      bad = bad || !page_ok;
      page_off = page_ok ? (static_cast<std::size_t>(page) * a.kv_heads + kvh) * P * D : 0;
    }
    const long long crow = static_cast<long long>(chunk_row0) + key0 - hist;
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int c = wave * IPW + i;
      const int row = 2 * c + (lane >> 5);
      const int phys = lane & 31;
      const int key = key0 + row;
      const bool in_hist = key < hist;
      const bool valid = key < key_end && (!in_hist || page_ok);
      const std::size_t rk = in_hist ? page_off + static_cast<std::size_t>(row) * D : 0;
      const float* kr = in_hist ? a.key_pool + rk : a.chunk_key + (crow + row) * D;
      const float* vr = in_hist ? a.value_pool + rk : a.chunk_value + (crow + row) * D;
      const float* ks = valid ? kr + 4 * (phys ^ (row & 15)) : &kZeroRows[lane].x;
      const float* vs = valid ? vr + 4 * phys : &kZeroRows[lane].x;
      lds_load16(ks, lds_address(&ds->k[sbuf][c * 256]));
      lds_load16(vs, lds_address(&ds->v[sbuf][c * 256]));
    }
  };
  // After a block's stage has landed: does a value row that some query row
  // of the workgroup masks hold a non-finite value?
  auto dma_nonfinite = [&](int blk) {
    bool nf = false;
    const int sbuf = blk % kDmaStages;
#pragma unroll
    for (int i = 0; i < IPW; ++i) {
      const int c = wave * IPW + i;
      const int key = blk * kKeys + 2 * c + (lane >> 5);
      if (key >= hist + pos0 + 1 && key < key_end) {
        nf = nf || !finite4(*reinterpret_cast<const float4*>(&ds->v[sbuf][c * 256 + 4 * lane]));
      }
    }
    return nf;
  };
  // Wait for this wavefront's loads of block n (those of block n + 1 may
  // stay in flight), then meet the workgroup; LDS writes of this wave are
  // complete too.
  static_assert(kDmaStages == 4, "the waits below keep up to two later blocks in flight");
  auto dma_wait = [&](int later_in_flight) {
    if (later_in_flight >= 2) {
      if constexpr (IPW == 2) {
        asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
    } else if (later_in_flight == 1) {
      if constexpr (IPW == 2) {
        asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      } else {
        asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
    } else {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    }
  };

  const int nblocks = (key_end + kKeys - 1) / kKeys;
  const int nfirst = key_begin / kKeys;
  int exact_pv = 0;
  if constexpr (DMA) {
#pragma unroll
    for (int i = 0; i < kDmaStages - 1; ++i) {
      if (nblocks > nfirst + i) dma_issue(nfirst + i);
    }
  } else {
    if (nblocks > nfirst) {
      stage_load(nfirst);
      exact_pv = staged_barrier(stage_store(nfirst & 1, nfirst), nfirst);
    }
  }
  for (int n = nfirst; n < nblocks; ++n) {
    const float* K;
    const float* V;
    if constexpr (DMA) {
      const int sbuf = n % kDmaStages;
      dma_wait(min(nblocks - 1 - n, kDmaStages - 2));
      // Only a block holding chunk rows past the workgroup's first
      // position can carry a masked value row.
      exact_pv = 0;
      if (!FAST && !CASCADE && n * kKeys + kKeys > hist + pos0 + 1) {
        exact_pv = __syncthreads_or(dma_nonfinite(n));
      }
      // The stage of block n - 1 is free: every wave has passed the barrier.
      if (n + kDmaStages - 1 < nblocks) dma_issue(n + kDmaStages - 1);
      K = ds->k[sbuf];
      V = ds->v[sbuf];
    } else {
      const int buf = n & 1;
      if (n + 1 < nblocks) stage_load(n + 1);
      K = s_k[buf];
      V = s_v[buf];
    }

    // S^T = K Q^T: st[t] holds keys 4*grp + i (i = vector component) of
    // query row t*16 + col.
    v4f st[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      st[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const int kc = DMA ? ((4 * c + grp) ^ (col & 15)) : 4 * c + grp;
        const float4 kk = *reinterpret_cast<const float4*>(&K[col * kKRow + 4 * kc]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          st[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(comp(kk, e), comp(q[t][c], e), st[t], 0,
                                                       0, 0);
        }
      }
    }

    // Online softmax (exp2 domain), lane-local rescale of O.  A block whose
    // keys every row of the workgroup sees (all but the last blocks) skips
    // the mask.
    float p[RT][4];
    const bool full = (n + 1) * kKeys <= min(key_end, hist + pos0 + 1);
    auto softmax = [&](auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        float x[4];
        bool vis[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = n * kKeys + 4 * grp + i;
          vis[i] = FULL || (key < key_end && (key < hist || key - hist <= qpos[t]));
          x[i] = vis[i] ? st[t][i] : -INFINITY;
        }
        if constexpr (PROBS) {
          if (qvalid[t]) {
            float* pr = a.probs + (static_cast<std::size_t>(kvh * G + r_head[t]) * T + qpos[t]) *
                                      static_cast<std::size_t>(a.prob_keys);
            const int key = n * kKeys + 4 * grp;
            if (key + 4 <= key_end) {
              // Rows are prob_keys floats long: the four keys are 4-byte
              // aligned only; one dwordx4 store either way.
              *reinterpret_cast<v4f_a4*>(pr + key) = v4f_a4{x[0], x[1], x[2], x[3]};
            } else {
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                if (key + i < key_end) pr[key + i] = x[i];
              }
            }
          }
        }
        const float mx = row_max(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
        const float mn = fmaxf(m[t], mx);
        const float alpha = exp2_ratio(m[t], mn);
#pragma unroll
        for (int i = 0; i < 4; ++i) p[t][i] = vis[i] ? exp2_ratio(x[i], mn) : 0.f;
        const float sum = row_sum((p[t][0] + p[t][1]) + (p[t][2] + p[t][3]));
        l[t] = l[t] * alpha + sum;
        m[t] = mn;
        // Branch-free rescale (alpha is 1 for rows whose maximum held).
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int c = 0; c < 4; ++c) o[t][h][c] *= alpha;
      }
    };
    if (full) {
      softmax(std::true_type{});
    } else {
      softmax(std::false_type{});
    }

    if (FAST || !exact_pv) {
      // O^T += V^T P^T: k step i covers keys 4*g + i over the four lane
      // groups g; A = V rows of those keys at dims 64h + 4*col + c.
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float4 vv =
              *reinterpret_cast<const float4*>(&V[(4 * grp + i) * D + 64 * h + 4 * col]);
#pragma unroll
          for (int c = 0; c < 4; ++c) {
#pragma unroll
            for (int t = 0; t < RT; ++t) {
              o[t][h][c] = __builtin_amdgcn_mfma_f32_16x16x4f32(comp(vv, c), p[t][i], o[t][h][c],
                                                                0, 0, 0);
            }
          }
        }
      }
    } else {
      // Exact path: every key's term is added only to the rows that see it.
      // Lane holds O[row][64h + 16*grp + 4*ii + c] in o[t][h][c][ii].
#pragma unroll 1
      for (int kk = 0; kk < kKeys; ++kk) {
        const int i = kk & 3;
        const int src = col + 16 * (kk >> 2);
        const int key = n * kKeys + kk;
        float pk[RT];
        bool vis[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
          const float sel = i == 0 ? p[t][0] : i == 1 ? p[t][1] : i == 2 ? p[t][2] : p[t][3];
          pk[t] = __shfl(sel, src, 64);
          vis[t] = key < key_end && (key < hist || key - hist <= qpos[t]);
        }
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int ii = 0; ii < 4; ++ii) {
            const float4 vv =
                *reinterpret_cast<const float4*>(&V[kk * D + 64 * h + 16 * grp + 4 * ii]);
#pragma unroll
            for (int t = 0; t < RT; ++t) {
              if (vis[t]) {
                o[t][h][0][ii] += pk[t] * vv.x;
                o[t][h][1][ii] += pk[t] * vv.y;
                o[t][h][2][ii] += pk[t] * vv.z;
                o[t][h][3][ii] += pk[t] * vv.w;
              }
            }
          }
        }
      }
    }

    if constexpr (!DMA) {
      const bool nonfinite = n + 1 < nblocks && stage_store((n & 1) ^ 1, n + 1);
      exact_pv = staged_barrier(nonfinite, n + 1);
    }
  }

  if constexpr (FAST) {
    bool nan_row = false;
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      nan_row = nan_row || !(l[t] < INFINITY);  // NaN, or a sum that overflowed
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
          for (int i = 0; i < 4; ++i) nan_row = nan_row || isnan(o[t][h][c][i]);
    }
    // Any NaN row of the workgroup; bad (NaN rows by design) is folded in
    // by the barrier below anyway.
    const int nan_any = __syncthreads_or(nan_row);
    if (threadIdx.x == 0) redo[block] = nan_any != 0 ? 1u : 0u;
  }
  const int any_bad = __syncthreads_or(bad);
  if constexpr (CASCADE) {
    // Partial (m, l, o) per row; lanes of the four k groups hold the row's
    // 128 dims, the (m, l) pair is written by group 0.
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      if (!qvalid[t]) continue;
      const int row = pb * kRows + wave * (16 * RT) + t * 16 + col;
      const long long units = static_cast<long long>(a.kv_heads) * a.batch;
      const std::size_t slot = static_cast<std::size_t>(
          a.prefix_slot0 + chunk * units + static_cast<long long>(kvh) * a.batch + row / G);
      const std::size_t base = (slot * G + row % G);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          *reinterpret_cast<float4*>(a.part_o + base * D + 64 * h + 16 * grp + 4 * ii) =
              make_float4(o[t][h][0][ii], o[t][h][1][ii], o[t][h][2][ii], o[t][h][3][ii]);
        }
      }
      if (grp == 0) {
        a.part_ml[base * 2] = m[t];
        a.part_ml[base * 2 + 1] = any_bad ? NAN : l[t];
      }
    }
    return;
  }
  if constexpr (PROBS) {
#pragma unroll
    for (int t = 0; t < RT; ++t) {
      if (qpos[t] >= T) continue;
      const std::size_t slot =
          (static_cast<std::size_t>(kvh * G + r_head[t]) * T + qpos[t]) * a.prob_splits + split;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
          *reinterpret_cast<float4*>(a.prob_o + slot * D + 64 * h + 16 * grp + 4 * ii) =
              make_float4(o[t][h][0][ii], o[t][h][1][ii], o[t][h][2][ii], o[t][h][3][ii]);
        }
      }
      if (grp == 0) {
        a.prob_ml[slot * 2] = m[t];
        a.prob_ml[slot * 2 + 1] = any_bad ? NAN : l[t];
      }
    }
    return;
  }
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    if (qpos[t] >= T) continue;
    const bool nan_row = any_bad || m[t] == -INFINITY;
    const float inv = nan_row ? NAN : 1.0f / l[t];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int ii = 0; ii < 4; ++ii) {
        float4 r = make_float4(o[t][h][0][ii] * inv, o[t][h][1][ii] * inv, o[t][h][2][ii] * inv,
                               o[t][h][3][ii] * inv);
        if (nan_row) r = make_float4(NAN, NAN, NAN, NAN);
        *reinterpret_cast<float4*>(a.out + qrow[t] + 64 * h + 16 * grp + 4 * ii) = r;
      }
    }
  }
}

// Kernel arguments of the cascade prefix pass and its work-item count
// (defined with the prefill launches).
PrefillKernelArgs cascade_prefix_args(const CascadePrefixArgs& a, std::size_t* work_items);

}  // namespace helix::hip::prefill_detail
