// Chunked-prefill attention for bf16 and fp8 pages on the bf16 matrix cores.
//
// The decomposition, masks, online softmax and special-value rules are those
// of prefill_body (one workgroup per (sequence, kv head) and 128 query rows,
// 16-row tiles, scores computed transposed so each lane holds keys of one
// query row).  What differs is the matrix
// arithmetic.  A bf16 page element is exact in bf16, and so is the bare code
// value of an fp8 element (the key scale joins the score scale and the value
// scale multiplies the output, as in the decode kernel).  The fp32 operand
// of each product (the scaled query, the probabilities) is split by
// truncation into three bf16 terms, hi + mid + lo, which hold its 24
// significant bits exactly.  Every product term is then exact in fp32, and
// three v_mfma_f32_16x16x32_bf16 replace each fp32 instruction (scores and
// P.V) at about five times the matrix throughput;
// only the order of the fp32 accumulation differs from the fp32 kernel.
//
// Special values.  A non-finite operand keeps only its hi term.  The split
// can only go wrong by giving NaN where fp32 does not: a zero term of one
// operand times an infinite element of the other (a query term against an
// infinite key, a probability of exactly 1 against an infinite value), and
// a value row that some row masks reaching that row (0 * inf).  Each such
// NaN reaches the row's accumulators or sum, so a work item whose rows end
// with a NaN there (or with a sum that is not finite) is flagged in
// redo[block], and the launcher runs
// prefill_body (fp32 operands, exact paths for these cases) over the
// flagged items only.  An item whose exact result is NaN anyway is just
// computed twice.
//
// Blocks of 32 keys (two pages) per LDS stage, so that both products run on
// the K = 32 instruction.  Scores come out as two 16-key tiles, keys
// 4 g + i and 16 + 4 g + i of row col in lane (g = lane / 16, col = lane %
// 16).  P.V contracts over the keys in any order, so its 32-key operand
// takes them in the order the scores left them: contraction index 8 g + j
// is key 4 g + j for j < 4 and key 16 + 4 g + j - 4 otherwise, and V is
// staged in the same order.
//
// LDS: K rows as bf16, padded to kBKStride elements (16 bytes) so the 16
// rows one operand read touches start in distinct banks; V transposed,
// [dim][contraction index] with rows of kVtStride elements, so one 16-byte
// read gives a lane the 8 keys of one dim that the P.V operand needs.
#pragma once

#include "prefill_body.hpp"

namespace helix::hip::prefill_detail {

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef short v8s __attribute__((ext_vector_type(8)));

constexpr int kBKeys = 2 * P;          // keys per LDS stage
constexpr int kBKStride = D + 8;       // bf16 elements per K row in LDS
constexpr int kVtStride = kBKeys + 8;  // bf16 elements per transposed V row

struct PrefillBmmaShared {
  __align__(16) unsigned short k[2][kBKeys * kBKStride];
  __align__(16) unsigned short vt[2][D * kVtStride];
  // The low bf16 term of each lane's query operand, [wave][step][lane]:
  // kept here rather than in registers, which the other two terms, the
  // accumulators and the staging fill.
  __align__(16) uint4 qlo[kRows / 16][4][64];
};

// Position of key kr (0 .. 31 within a stage) on the P.V contraction axis.
__device__ __forceinline__ int bmma_key_slot(int kr) {
  return 8 * ((kr & 15) >> 2) + 4 * (kr >> 4) + (kr & 3);
}

// x = hi + mid + lo exactly (truncating splits of a finite fp32); a
// non-finite x is hi alone.  Results are bf16 bit patterns.  Range: lo's
// exponent is 16 or more below x's, so for |x| < 2^-109 lo can be a bf16
// subnormal, which the matrix cores may flush; mid likewise for |x| <
// 2^-117.  Then the terms sum to x within |x| * 2^-7 (an absolute error
// below 2^-116), far under any tolerance of the products they enter (the
// scaled query and the probabilities of a row whose sum is at least 1);
// such items are not flagged for the exact redo.
__device__ __forceinline__ void split3(float x, short& hi, short& mid, short& lo) {
  const unsigned u = __float_as_uint(x);
  hi = static_cast<short>(u >> 16);
  if (!isfinite(x)) {
    mid = 0;
    lo = 0;
    return;
  }
  const float r1 = x - __uint_as_float(u & 0xffff0000u);
  const unsigned u1 = __float_as_uint(r1);
  mid = static_cast<short>(u1 >> 16);
  const float r2 = r1 - __uint_as_float(u1 & 0xffff0000u);
  lo = static_cast<short>(__float_as_uint(r2) >> 16);
}

// split3 for a probability (in [0, 1], or NaN): no finiteness test.  For
// a finite p the terms are split3's.  A NaN p still gives a NaN middle term,
// so the row's accumulators end NaN as they must (the item is redone).
__device__ __forceinline__ void split3_prob(float x, short& hi, short& mid, short& lo) {
  const unsigned u = __float_as_uint(x);
  hi = static_cast<short>(u >> 16);
  const float r1 = x - __uint_as_float(u & 0xffff0000u);
  const unsigned u1 = __float_as_uint(r1);
  mid = static_cast<short>(u1 >> 16);
  const float r2 = r1 - __uint_as_float(u1 & 0xffff0000u);
  lo = static_cast<short>(__float_as_uint(r2) >> 16);
}

// Four fp8 code values (one word, lowest byte first) as four bf16 bit
// patterns, lowest first, two to a word.  Exact: every E4M3 value is a bf16
// value, and the scale is 1.
__device__ __forceinline__ uint2 fp8_codes_bf16(unsigned w) {
  const auto lo = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
  const auto hi = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true);
  return make_uint2(__builtin_bit_cast(unsigned, lo), __builtin_bit_cast(unsigned, hi));
}

__device__ __forceinline__ float bf16_bits_value(unsigned short h) {
  return __uint_as_float(static_cast<unsigned>(h) << 16);
}

// PF: 1 bf16 pages, 2 fp8 pages.  Standalone prefill only (no cascade).
// RT: 16-row tiles per wavefront; the workgroup has 8 / RT wavefronts.
// redo[block] is written for every block: 1 when the item must be redone
// exactly.
template <int G, int PF, int RT>
__device__ __forceinline__ void prefill_body_bmma(PrefillKernelArgs a,
                                                  const std::uint32_t* __restrict__ tables,
                                                  const std::uint32_t* __restrict__ order,
                                                  std::uint32_t* __restrict__ redo,
                                                  std::uint32_t block, PrefillBmmaShared& sh) {
  static_assert(PF == 1 || PF == 2, "bf16 matrix-core prefill is for bf16 and fp8 pages");
  constexpr int RP = 16 / RT;  // key rows per staging pass
  constexpr int PW = kRows / G;
  constexpr bool FP8 = PF == 2;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int col = lane & 15;
  const int grp = lane >> 4;

  std::uint32_t item = block;
  if (order != nullptr) {
    item = order[block];
  } else {
    const std::uint32_t x = item % a.pos_blocks;
    item = item - x + (a.pos_blocks - 1 - x);
  }
  const int pb = static_cast<int>(item % a.pos_blocks);
  const int kvh = static_cast<int>((item / a.pos_blocks) % a.kv_heads);
  const int b = static_cast<int>(item / a.pos_blocks / a.kv_heads);
  const int T = a.tokens;
  const int pos0 = pb * PW;

  int hist = a.lengths[b];
  bool bad = hist < 0 || hist > a.max_blocks * P;
  if (bad) hist = 0;
  const int key_end = hist + min(T, pos0 + PW);
  const std::uint32_t* __restrict__ table = tables + static_cast<std::size_t>(b) * a.max_blocks;
  const std::size_t chunk_row0 = (static_cast<std::size_t>(b) * a.kv_heads + kvh) * T;
  // fp8: keys are bare code values, their scale joins the score scale.
  const float qs = FP8 ? a.qscale * a.k_scale : a.qscale;

  // Query operand: tile t, step s covers dims 32 s + 8 grp .. + 7 of row
  // t * 16 + col (B operand of S^T = K Q^T), as three bf16 terms.
  int qpos[RT];
  std::size_t qrow[RT];
  v8s qv[RT][2][4];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    const int r = wave * (16 * RT) + t * 16 + col;
    const int head = kvh * G + r / PW;
    qpos[t] = pos0 + r % PW;
    const bool valid = qpos[t] < T;
    qrow[t] = ((static_cast<std::size_t>(b) * a.q_heads + head) * T + qpos[t]) * D;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
      if (valid) {
        x0 = *reinterpret_cast<const float4*>(a.query + qrow[t] + 32 * s + 8 * grp);
        x1 = *reinterpret_cast<const float4*>(a.query + qrow[t] + 32 * s + 8 * grp + 4);
      }
      const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
      v8s lo;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        short h, m, l;
        split3(xs[j] * qs, h, m, l);
        qv[t][0][s][j] = h;
        qv[t][1][s][j] = m;
        lo[j] = l;
      }
      sh.qlo[wave * RT + t][s][lane] = __builtin_bit_cast(uint4, lo);
    }
  }

  v4f o[RT][8];  // O^T tiles: o[t][dt][i] = O[row t*16 + col][dim 16 dt + 4 grp + i]
#pragma unroll
  for (int t = 0; t < RT; ++t)
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) o[t][dt] = v4f{0.f, 0.f, 0.f, 0.f};
  float m[RT], l[RT];
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    m[t] = -INFINITY;
    l[t] = 0.f;
  }

  // Staging: thread tid moves dims 4 scol .. + 3 of key rows srow + RP r
  // (r < NR) of one 16-key half (one page) of a 32-key block, for K and V
  // (as loaded: bf16 words, fp8 code words or fp32 chunk rows).  The two
  // halves of the next block are staged one after the other, so only one
  // page is held in registers.
  constexpr int NR = P / RP;
  const int srow = tid >> 5;
  const int scol = tid & 31;
  float4 stk[NR], stv[NR];
  auto stage_load = [&](int blk, int half) {
    const int pkey0 = blk * kBKeys + half * P;
    std::size_t page_off = 0;
    bool page_ok = false;
    if (pkey0 < hist) {
      const std::uint32_t page = table[pkey0 / P];
      page_ok = page < a.physical_blocks;
      bad = bad || !page_ok;
      page_off = page_ok ? (static_cast<std::size_t>(page) * a.kv_heads + kvh) * P * D : 0;
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int key = pkey0 + srow + RP * r;
      const bool in_hist = key < hist;
      const bool valid = key < key_end && (!in_hist || page_ok);
      const int off = (srow + RP * r) * D + scol * 4;
      stk[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      stv[r] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (valid && in_hist) {
        const std::size_t e = page_off + off;
        if constexpr (FP8) {
          stk[r].x = __uint_as_float(*reinterpret_cast<const unsigned*>(
              reinterpret_cast<const unsigned char*>(a.key_pool) + e));
          stv[r].x = __uint_as_float(*reinterpret_cast<const unsigned*>(
              reinterpret_cast<const unsigned char*>(a.value_pool) + e));
        } else {
          const uint2 kw = *reinterpret_cast<const uint2*>(
              reinterpret_cast<const unsigned short*>(a.key_pool) + e);
          const uint2 vw = *reinterpret_cast<const uint2*>(
              reinterpret_cast<const unsigned short*>(a.value_pool) + e);
          stk[r] = make_float4(__uint_as_float(kw.x), __uint_as_float(kw.y), 0.f, 0.f);
          stv[r] = make_float4(__uint_as_float(vw.x), __uint_as_float(vw.y), 0.f, 0.f);
        }
      } else if (valid) {
        const std::size_t crow = chunk_row0 + static_cast<std::size_t>(key - hist);
        stk[r] = *reinterpret_cast<const float4*>(a.chunk_key + crow * D + scol * 4);
        stv[r] = *reinterpret_cast<const float4*>(a.chunk_value + crow * D + scol * 4);
      }
    }
  };
  // Stores a staged half as bf16 (K rows, V transposed in contraction order).
  auto stage_store = [&](int buf, int blk, int half) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int kr = half * P + srow + RP * r;
      const int key = blk * kBKeys + kr;
      uint2 kb, vb;  // 4 bf16 each, low half first (fp8: the bare code values)
      if (key < hist) {
        if constexpr (FP8) {
          kb = fp8_codes_bf16(__float_as_uint(stk[r].x));
          vb = fp8_codes_bf16(__float_as_uint(stv[r].x));
        } else {
          kb = make_uint2(__float_as_uint(stk[r].x), __float_as_uint(stk[r].y));
          vb = make_uint2(__float_as_uint(stv[r].x), __float_as_uint(stv[r].y));
        }
      } else {
        // Chunk rows (zeros past the key range): onto the page grid.
        if constexpr (FP8) {
          kb = fp8_codes_bf16(fp8_pack4_scaled(stk[r], a.k_scale));
          vb = fp8_codes_bf16(fp8_pack4_scaled(stv[r], a.v_scale));
        } else {
          kb = make_uint2(bf16_pack(stk[r].x, stk[r].y), bf16_pack(stk[r].z, stk[r].w));
          vb = make_uint2(bf16_pack(stv[r].x, stv[r].y), bf16_pack(stv[r].z, stv[r].w));
        }
      }
      *reinterpret_cast<uint2*>(&sh.k[buf][kr * kBKStride + scol * 4]) = kb;
      unsigned short* vt = &sh.vt[buf][(scol * 4) * kVtStride + bmma_key_slot(kr)];
      vt[0] = static_cast<unsigned short>(vb.x & 0xffffu);
      vt[kVtStride] = static_cast<unsigned short>(vb.x >> 16);
      vt[2 * kVtStride] = static_cast<unsigned short>(vb.y & 0xffffu);
      vt[3 * kVtStride] = static_cast<unsigned short>(vb.y >> 16);
    }
  };

  __shared__ int s_redo;
  if (tid == 0) s_redo = 0;  // published by the first barrier below
  const int nblocks = (key_end + kBKeys - 1) / kBKeys;
  if (nblocks > 0) {
    stage_load(0, 0);
    stage_store(0, 0, 0);
    stage_load(0, 1);
    stage_store(0, 0, 1);
  }
  __syncthreads();
  for (int n = 0; n < nblocks; ++n) {
    const int buf = n & 1;
    const bool next = n + 1 < nblocks;
    if (next) stage_load(n + 1, 0);
    const unsigned short* K = sh.k[buf];
    const unsigned short* VT = sh.vt[buf];

    // S^T = K Q^T on the bf16 matrix cores: st[t][h] holds keys
    // 16 h + 4 grp + i of query row t * 16 + col.
    v4f st[RT][2];
#pragma unroll
    for (int t = 0; t < RT; ++t) st[t][0] = st[t][1] = v4f{0.f, 0.f, 0.f, 0.f};
    // Raised wave priority over the matrix instructions: the waves of one
    // workgroup reach them together (barriers), and the softmax and staging
    // of the other workgroup on the CU fill the gaps.
    __builtin_amdgcn_s_setprio(1);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        const v8bf qlo = __builtin_bit_cast(v8bf, sh.qlo[wave * RT + t][s][lane]);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const v8bf kop = __builtin_bit_cast(
              v8bf,
              *reinterpret_cast<const v8s*>(&K[(16 * h + col) * kBKStride + 32 * s + 8 * grp]));
          st[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qlo, st[t][h], 0, 0, 0);
#pragma unroll
          for (int term = 1; term >= 0; --term) {
            st[t][h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                kop, __builtin_bit_cast(v8bf, qv[t][term][s]), st[t][h], 0, 0, 0);
          }
        }
      }
    }
    __builtin_amdgcn_s_setprio(0);
    float p[RT][8];  // p[t][4 h + i]: key 16 h + 4 grp + i
    const bool full = (n + 1) * kBKeys <= min(key_end, hist + pos0 + 1);
    auto softmax = [&](auto full_tag) {
      constexpr bool FULL = decltype(full_tag)::value;
#pragma unroll
      for (int t = 0; t < RT; ++t) {
        float x[8];
        bool vis[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int key = n * kBKeys + 16 * (j >> 2) + 4 * grp + (j & 3);
          vis[j] = FULL || (key < key_end && (key < hist || key - hist <= qpos[t]));
          x[j] = vis[j] ? st[t][j >> 2][j & 3] : -INFINITY;
        }
        const float mx = row_max(fmaxf(fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])),
                                       fmaxf(fmaxf(x[4], x[5]), fmaxf(x[6], x[7]))));
        const float mn = fmaxf(m[t], mx);
        // Branch-free rescale (alpha is 1 for rows whose maximum held).
        const float alpha = exp2_ratio(m[t], mn);
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) o[t][dt] *= alpha;
        if (FULL && __ballot(!(fabsf(mn) < INFINITY)) == 0) {
#pragma unroll
          for (int j = 0; j < 8; ++j) p[t][j] = __builtin_amdgcn_exp2f(x[j] - mn);
        } else {
#pragma unroll
          for (int j = 0; j < 8; ++j) p[t][j] = vis[j] ? exp2_ratio(x[j], mn) : 0.f;
        }
        const float sum = row_sum(((p[t][0] + p[t][1]) + (p[t][2] + p[t][3])) +
                                  ((p[t][4] + p[t][5]) + (p[t][6] + p[t][7])));
        l[t] = l[t] * alpha + sum;
        m[t] = mn;
      }
    };
    if (full) {
      softmax(std::true_type{});
    } else {
      softmax(std::false_type{});
    }

    if (next) {
      stage_store(buf ^ 1, n + 1, 0);
      stage_load(n + 1, 1);
    }

    {
      // O^T += V^T P^T: A = V^T rows (dims 16 dt + col) at contraction
      // indices 8 grp .. + 7, B = the lane's own 8 probabilities of row col
      // in the same order, as three bf16 terms.
      v8s pv[RT][3];
#pragma unroll
      for (int t = 0; t < RT; ++t) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          short h, mm, lo;
          split3_prob(p[t][j], h, mm, lo);
          pv[t][0][j] = h;
          pv[t][1][j] = mm;
          pv[t][2][j] = lo;
        }
      }
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int dt = 0; dt < 8; ++dt) {
        const v8bf vop = __builtin_bit_cast(
            v8bf, *reinterpret_cast<const v8s*>(&VT[(16 * dt + col) * kVtStride + 8 * grp]));
#pragma unroll
        for (int t = 0; t < RT; ++t) {
#pragma unroll
          for (int term = 2; term >= 0; --term) {
            o[t][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                vop, __builtin_bit_cast(v8bf, pv[t][term]), o[t][dt], 0, 0, 0);
          }
        }
      }
    }

    __builtin_amdgcn_s_setprio(0);
    if (next) stage_store(buf ^ 1, n + 1, 1);
    __syncthreads();
  }

  bool nan_row = false;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    nan_row = nan_row || !(l[t] < INFINITY);  // NaN, or a sum that overflowed
#pragma unroll
    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) nan_row = nan_row || isnan(o[t][dt][i]);
  }
  if (__ballot(nan_row) != 0 && lane == 0) s_redo = 1;
  const int any_bad = __syncthreads_or(bad);
  if (tid == 0) redo[block] = s_redo != 0 ? 1u : 0u;
  const float vscale = FP8 ? a.v_scale : 1.0f;
#pragma unroll
  for (int t = 0; t < RT; ++t) {
    if (qpos[t] >= T) continue;
    const bool nan_row = any_bad || m[t] == -INFINITY;
    const float inv = nan_row ? NAN : vscale / l[t];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) {
      float4 r = make_float4(o[t][dt][0] * inv, o[t][dt][1] * inv, o[t][dt][2] * inv,
                             o[t][dt][3] * inv);
      if (nan_row) r = make_float4(NAN, NAN, NAN, NAN);
      *reinterpret_cast<float4*>(a.out + qrow[t] + 16 * dt + 4 * grp) = r;
    }
  }
}

}  // namespace helix::hip::prefill_detail
