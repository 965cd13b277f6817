// CPU oracle for the paged-KV hot path.  TEST INFRASTRUCTURE ONLY.
//
// This file restates, in plain C++, the algorithm of the reference's CPU
// paged KV cache and CPU paged attention so that tests can check the HIP
// product path against it.  Only tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py may load this library; the product library
// (helix_runtime_amd/csrc) never links or calls it.
//
// Restated reference behaviour (paths relative to the reference root):
//   - pool geometry and byte formulas        src/kv_cache/paged.cpp:53-106
//   - FIFO free-block queue                   src/kv_cache/paged.cpp:139-188
//   - pool offset [block, layer, head, tok]   src/kv_cache/paged.cpp:236-240
//   - gather (copy_layer)                     src/kv_cache/paged.cpp:242-280
//   - create_sequence                         src/kv_cache/paged.cpp:509-533
//   - fork_sequence (block aligned)           src/kv_cache/paged.cpp:535-620
//   - append (one token, all layers)          src/kv_cache/paged.cpp:622-719
//   - append_layer_major (bulk)               src/kv_cache/paged.cpp:721-871
//   - copy_layer_prefix_out                   src/kv_cache/paged.cpp:895-950
//   - release_sequence                        src/kv_cache/paged.cpp:952-1001
//   - paged SDPA (+ uncommitted tail)         src/attention/paged_reference.cpp:173-384
//   - row softmax with NaN / +inf rules       src/kernels/cpu/reference.cpp:264-316
//   - contiguous SDPA (the reference's own
//     test oracle for paged attention)        src/attention/reference.cpp:124-226
//   - Tensor::random_uniform fixture inputs   src/tensor/tensor.cpp:169-189
//
// Extensions that the reference does not have (no reference citation exists):
//   - GQA: query head h reads KV head h / (Hq / Hkv), i.e. MHA over KV heads
//     repeated Hq / Hkv times.
//   - copy-on-write fork at a non-block-aligned prefix.
//   - a seeded standard-normal generator (Box-Muller) for synthetic inputs.
//
// Errors are reported as int status codes with the same numbering as the
// product C-ABI: 0 ok, 1 invalid argument, 2 out of range, 3 unsupported,
// 4 resource exhausted, 5 runtime, 6 internal.

#include <algorithm>
#include <array>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <limits>
#include <random>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

enum Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kOutOfRange = 2,
  kUnsupported = 3,
  kResourceExhausted = 4,
  kRuntime = 5,
  kInternal = 6,
};

struct Stats {
  std::uint64_t bytes_reserved, bytes_used, bytes_free, peak_bytes_used;
  std::uint64_t total_blocks, used_blocks, free_blocks, active_sequence_count;
  std::uint64_t active_tokens, resident_tokens, allocated_token_slots;
  std::uint64_t block_reference_count, shared_blocks;
  std::uint64_t sequence_create_count, sequence_fork_count, append_count, release_count;
  std::uint64_t block_allocation_count, block_reuse_count;
};

// Circular FIFO of free physical block IDs, initialised 0..N-1; released
// blocks are pushed at the tail (src/kv_cache/paged.cpp:139-188).
class Fifo {
public:
  explicit Fifo(std::size_t n) : slots_(n), count_(n) {
    for (std::size_t i = 0; i < n; ++i) slots_[i] = static_cast<std::uint32_t>(i);
  }
  std::size_t size() const { return count_; }
  std::uint32_t at(std::size_t i) const { return slots_[(head_ + i) % slots_.size()]; }
  std::uint32_t pop() {
    std::uint32_t v = slots_[head_];
    head_ = (head_ + 1) % slots_.size();
    --count_;
    return v;
  }
  void push(std::uint32_t b) {
    slots_[tail_] = b;
    tail_ = (tail_ + 1) % slots_.size();
    ++count_;
  }

private:
  std::vector<std::uint32_t> slots_;
  std::size_t head_ = 0, tail_ = 0, count_ = 0;
};

struct Sequence {
  std::size_t length = 0;
  std::vector<std::uint32_t> blocks;
};

struct Pool {
  std::size_t L, H, D, P, N;
  std::size_t head_elems, layer_elems, block_elems, block_bytes;
  std::vector<float> keys, values;  // [N, L, H, P, D]
  Fifo fifo;
  std::vector<std::size_t> refs, tokens;
  std::vector<std::uint8_t> was_allocated;
  std::unordered_map<std::uint64_t, Sequence> seqs;
  std::uint64_t next_id = 1;
  Stats st{};

  Pool(std::size_t l, std::size_t h, std::size_t d, std::size_t p, std::size_t n)
      : L(l), H(h), D(d), P(p), N(n), fifo(n), refs(n, 0), tokens(n, 0), was_allocated(n, 0) {
    head_elems = P * D;
    layer_elems = H * head_elems;
    block_elems = L * layer_elems;
    block_bytes = 2 * block_elems * sizeof(float);
    keys.assign(N * block_elems, 0.0F);
    values.assign(N * block_elems, 0.0F);
    st.bytes_reserved = N * block_bytes;
    st.bytes_free = st.bytes_reserved;
    st.total_blocks = N;
    st.free_blocks = N;
  }

  std::size_t offset(std::uint32_t block, std::size_t layer, std::size_t head,
                     std::size_t tok) const {
    return block * block_elems + layer * layer_elems + head * head_elems + tok * D;
  }

  void take_block(Sequence& s, std::uint32_t b) {
    s.blocks.push_back(b);
    refs[b] = 1;
    if (was_allocated[b]) ++st.block_reuse_count;
    was_allocated[b] = 1;
    ++st.used_blocks;
    --st.free_blocks;
    st.bytes_used += block_bytes;
    st.bytes_free -= block_bytes;
    st.peak_bytes_used = std::max(st.peak_bytes_used, st.bytes_used);
    st.allocated_token_slots += P;
    ++st.block_reference_count;
    ++st.block_allocation_count;
  }
};

Sequence* find(Pool* p, std::uint64_t id) {
  auto it = p->seqs.find(id);
  return it == p->seqs.end() ? nullptr : &it->second;
}

// ---------------------------------------------------------------------------
// Softmax over one row (src/kernels/cpu/reference.cpp:264-316): a NaN or an
// all -inf row becomes all NaN; any +inf gives a uniform distribution over
// the +inf entries; otherwise exp(double(x - max)) / sum, cast to float.
void softmax_row(float* row, std::size_t width) {
  bool nan = false;
  std::size_t pinf = 0;
  float mx = -std::numeric_limits<float>::infinity();
  for (std::size_t c = 0; c < width; ++c) {
    const float v = row[c];
    nan = nan || std::isnan(v);
    pinf += static_cast<std::size_t>(std::isinf(v) && v > 0.0F);
    mx = std::max(mx, v);
  }
  if (nan || mx == -std::numeric_limits<float>::infinity()) {
    std::fill_n(row, width, std::numeric_limits<float>::quiet_NaN());
    return;
  }
  if (pinf != 0) {
    const float prob = 1.0F / static_cast<float>(pinf);
    for (std::size_t c = 0; c < width; ++c)
      row[c] = row[c] == std::numeric_limits<float>::infinity() ? prob : 0.0F;
    return;
  }
  double den = 0.0;
  for (std::size_t c = 0; c < width; ++c) den += std::exp(static_cast<double>(row[c] - mx));
  for (std::size_t c = 0; c < width; ++c)
    row[c] = static_cast<float>(std::exp(static_cast<double>(row[c] - mx)) / den);
}

// Paged SDPA over pages in the per-layer GPU layout [N, Hkv, P, D] (the same
// spans LayerReadView::key_block hands out, src/kv_cache/paged.cpp:475-498),
// with an optional uncommitted tail.  Follows
// src/attention/paged_reference.cpp:173-384: double dot products scaled by
// 1/sqrt(double D) and cast to float; causal mask key > offset + q -> -inf;
// row softmax; P.V accumulated in double over 32-wide coordinate tiles, page
// by page, then the tail.  Query head h reads KV head h / (Hq / Hkv).
void paged_attention(const float* q, std::size_t Hq, std::size_t Hkv, std::size_t T,
                     std::size_t D, std::size_t DV, const float* kb, const float* vb,
                     std::size_t P, const std::uint32_t* table, std::size_t history,
                     const float* tk, const float* tv, std::size_t tail, std::size_t offset,
                     float* out, float* ws) {
  const std::size_t keys = history + tail;
  const std::size_t group = Hq / Hkv;
  const double scale = 1.0 / std::sqrt(static_cast<double>(D));
  const std::size_t blocks = history == 0 ? 0 : (history - 1) / P + 1;
  for (std::size_t h = 0; h < Hq; ++h) {
    const std::size_t kvh = h / group;
    for (std::size_t qi = 0; qi < T; ++qi) {
      const float* qrow = q + (h * T + qi) * D;
      float* srow = ws + (h * T + qi) * keys;
      const std::size_t qpos = offset + qi;
      std::size_t key_start = 0;
      for (std::size_t lb = 0; lb < blocks; ++lb) {
        const std::size_t in_block = std::min(P, history - key_start);
        const float* kpage = kb + (static_cast<std::size_t>(table[lb]) * Hkv + kvh) * P * D;
        for (std::size_t t = 0; t < in_block; ++t) {
          const std::size_t key = key_start + t;
          if (key > qpos) {
            srow[key] = -std::numeric_limits<float>::infinity();
            continue;
          }
          double dot = 0.0;
          for (std::size_t d = 0; d < D; ++d)
            dot += static_cast<double>(qrow[d]) * static_cast<double>(kpage[t * D + d]);
          srow[key] = static_cast<float>(dot * scale);
        }
        key_start += in_block;
      }
      for (std::size_t t = 0; t < tail; ++t) {
        const std::size_t key = history + t;
        if (key > qpos) {
          srow[key] = -std::numeric_limits<float>::infinity();
          continue;
        }
        const float* krow = tk + (kvh * tail + t) * D;
        double dot = 0.0;
        for (std::size_t d = 0; d < D; ++d)
          dot += static_cast<double>(qrow[d]) * static_cast<double>(krow[d]);
        srow[key] = static_cast<float>(dot * scale);
      }
    }
  }
  for (std::size_t r = 0; r < Hq * T; ++r) softmax_row(ws + r * keys, keys);

  constexpr std::size_t kTile = 32;
  for (std::size_t h = 0; h < Hq; ++h) {
    const std::size_t kvh = h / group;
    for (std::size_t qi = 0; qi < T; ++qi) {
      const float* prow = ws + (h * T + qi) * keys;
      float* orow = out + (h * T + qi) * DV;
      const std::size_t visible = offset + qi + 1;
      for (std::size_t d0 = 0; d0 < DV; d0 += kTile) {
        const std::size_t td = std::min(kTile, DV - d0);
        std::array<double, kTile> acc{};
        std::size_t start = 0;
        for (std::size_t lb = 0; lb < blocks; ++lb) {
          const std::size_t in_block = std::min(P, history - start);
          const float* vpage = vb + (static_cast<std::size_t>(table[lb]) * Hkv + kvh) * P * DV;
          for (std::size_t t = 0; t < in_block; ++t) {
            const std::size_t key = start + t;
            if (key >= visible) continue;
            const double p = static_cast<double>(prow[key]);
            for (std::size_t j = 0; j < td; ++j)
              acc[j] += p * static_cast<double>(vpage[t * DV + d0 + j]);
          }
          start += in_block;
        }
        for (std::size_t t = 0; t < tail; ++t) {
          const std::size_t key = history + t;
          if (key >= visible) continue;
          const double p = static_cast<double>(prow[key]);
          const float* vrow = tv + (kvh * tail + t) * DV;
          for (std::size_t j = 0; j < td; ++j) acc[j] += p * static_cast<double>(vrow[d0 + j]);
        }
        for (std::size_t j = 0; j < td; ++j) orow[d0 + j] = static_cast<float>(acc[j]);
      }
    }
  }
}

}  // namespace

extern "C" {

// ---------------------------------------------------------------- pool ----
void* oracle_pool_create(std::size_t layers, std::size_t kv_heads, std::size_t head_dim,
                         std::size_t block_tokens, std::size_t physical_blocks, int* status) {
  if (layers == 0 || kv_heads == 0 || head_dim == 0 || block_tokens == 0 ||
      physical_blocks == 0) {
    *status = kInvalidArgument;
    return nullptr;
  }
  if (physical_blocks > std::numeric_limits<std::uint32_t>::max()) {
    *status = kOutOfRange;
    return nullptr;
  }
  *status = kOk;
  return new Pool(layers, kv_heads, head_dim, block_tokens, physical_blocks);
}

void oracle_pool_destroy(void* pool) { delete static_cast<Pool*>(pool); }

std::size_t oracle_bytes_per_token(void* pool) {
  auto* p = static_cast<Pool*>(pool);
  return p->L * 2 * p->H * p->D * sizeof(float);
}
std::size_t oracle_block_bytes(void* pool) { return static_cast<Pool*>(pool)->block_bytes; }

std::uint64_t oracle_create_sequence(void* pool) {
  auto* p = static_cast<Pool*>(pool);
  const std::uint64_t id = p->next_id++;
  p->seqs.emplace(id, Sequence{});
  ++p->st.active_sequence_count;
  ++p->st.sequence_create_count;
  return id;
}

// Block-aligned fork (src/kv_cache/paged.cpp:535-620).  When allow_cow is
// nonzero a non-aligned prefix is accepted (extension): the full blocks are
// shared and the partial block's first prefix % P tokens are copied into a
// fresh exclusive block taken from the FIFO head.
int oracle_fork_sequence(void* pool, std::uint64_t source, std::size_t prefix, int allow_cow,
                         std::uint64_t* out) {
  auto* p = static_cast<Pool*>(pool);
  Sequence* src = find(p, source);
  if (src == nullptr) return kInvalidArgument;
  if (prefix == 0) return kInvalidArgument;
  if (prefix > src->length) return kOutOfRange;
  const std::size_t rem = prefix % p->P;
  if (rem != 0 && !allow_cow) return kInvalidArgument;
  if (rem != 0 && p->fifo.size() == 0) return kResourceExhausted;
  const std::size_t shared = prefix / p->P;
  std::size_t newly_shared = 0;
  for (std::size_t i = 0; i < shared; ++i) newly_shared += p->refs[src->blocks[i]] == 1;
  Sequence f;
  f.length = prefix;
  f.blocks.assign(src->blocks.begin(), src->blocks.begin() + static_cast<std::ptrdiff_t>(shared));
  for (std::size_t i = 0; i < shared; ++i) ++p->refs[src->blocks[i]];
  p->st.block_reference_count += shared;
  p->st.shared_blocks += newly_shared;
  if (rem != 0) {
    const std::uint32_t from = src->blocks[shared];
    const std::uint32_t to = p->fifo.pop();
    p->take_block(f, to);
    for (std::size_t l = 0; l < p->L; ++l)
      for (std::size_t h = 0; h < p->H; ++h) {
        std::memcpy(&p->keys[p->offset(to, l, h, 0)], &p->keys[p->offset(from, l, h, 0)],
                    rem * p->D * sizeof(float));
        std::memcpy(&p->values[p->offset(to, l, h, 0)], &p->values[p->offset(from, l, h, 0)],
                    rem * p->D * sizeof(float));
      }
    p->tokens[to] = rem;
    p->st.resident_tokens += rem;
  }
  const std::uint64_t id = p->next_id++;
  p->seqs.emplace(id, std::move(f));
  ++p->st.active_sequence_count;
  p->st.active_tokens += prefix;
  ++p->st.sequence_create_count;
  ++p->st.sequence_fork_count;
  *out = id;
  return kOk;
}

// One token for every layer: keys/values are [L, H, D] (paged.cpp:622-719).
int oracle_append(void* pool, std::uint64_t seq, const float* keys, const float* values) {
  auto* p = static_cast<Pool*>(pool);
  Sequence* s = find(p, seq);
  if (s == nullptr) return kInvalidArgument;
  std::uint32_t block;
  if (s->length % p->P == 0) {
    if (p->fifo.size() == 0) return kResourceExhausted;
    block = p->fifo.pop();
    p->take_block(*s, block);
  } else {
    block = s->blocks.back();
    if (p->refs[block] != 1) return kInternal;
  }
  const std::size_t off = s->length % p->P;
  for (std::size_t l = 0; l < p->L; ++l)
    for (std::size_t h = 0; h < p->H; ++h) {
      const std::size_t src = (l * p->H + h) * p->D;
      std::memcpy(&p->keys[p->offset(block, l, h, off)], keys + src, p->D * sizeof(float));
      std::memcpy(&p->values[p->offset(block, l, h, off)], values + src, p->D * sizeof(float));
    }
  ++s->length;
  ++p->st.active_tokens;
  ++p->st.resident_tokens;
  p->tokens[block] = off + 1;
  ++p->st.append_count;
  return kOk;
}

// Bulk append of T tokens from per-layer [H, T, D] tensors stored back to
// back as [L, H, T, D] (paged.cpp:721-871).  Transactional: nothing changes
// when the pool cannot hold the new blocks.
int oracle_append_layer_major(void* pool, std::uint64_t seq, const float* keys,
                              const float* values, std::size_t T) {
  auto* p = static_cast<Pool*>(pool);
  Sequence* s = find(p, seq);
  if (s == nullptr) return kInvalidArgument;
  if (T == 0) return kInvalidArgument;
  const std::size_t result = s->length + T;
  const std::size_t need = (result + p->P - 1) / p->P;
  const std::size_t extra = need - s->blocks.size();
  if (extra > p->fifo.size()) return kResourceExhausted;
  if (s->length % p->P != 0 && p->refs[s->blocks.back()] != 1) return kInternal;
  for (std::size_t i = 0; i < extra; ++i) p->take_block(*s, p->fifo.pop());
  const std::size_t old = s->length;
  std::size_t st = 0;
  while (st < T) {
    const std::size_t dst = old + st;
    const std::size_t lb = dst / p->P, off = dst % p->P;
    const std::size_t n = std::min(T - st, p->P - off);
    const std::uint32_t block = s->blocks[lb];
    for (std::size_t l = 0; l < p->L; ++l)
      for (std::size_t h = 0; h < p->H; ++h) {
        const std::size_t src = ((l * p->H + h) * T + st) * p->D;
        std::memcpy(&p->keys[p->offset(block, l, h, off)], keys + src, n * p->D * sizeof(float));
        std::memcpy(&p->values[p->offset(block, l, h, off)], values + src,
                    n * p->D * sizeof(float));
      }
    st += n;
  }
  s->length = result;
  for (std::size_t lb = old / p->P; lb < s->blocks.size(); ++lb)
    p->tokens[s->blocks[lb]] = std::min(p->P, result - lb * p->P);
  p->st.active_tokens += T;
  p->st.resident_tokens += T;
  p->st.append_count += T;
  return kOk;
}

int oracle_release_sequence(void* pool, std::uint64_t seq) {
  auto* p = static_cast<Pool*>(pool);
  Sequence* s = find(p, seq);
  if (s == nullptr) return kInvalidArgument;
  std::size_t released = 0, resident = 0, unshared = 0;
  for (std::uint32_t b : s->blocks) {
    if (p->refs[b] == 1) {
      ++released;
      resident += p->tokens[b];
    } else if (p->refs[b] == 2) {
      ++unshared;
    }
  }
  for (std::uint32_t b : s->blocks) {
    if (--p->refs[b] == 0) {
      p->tokens[b] = 0;
      p->fifo.push(b);
    }
  }
  p->st.used_blocks -= released;
  p->st.free_blocks += released;
  p->st.bytes_used -= released * p->block_bytes;
  p->st.bytes_free += released * p->block_bytes;
  --p->st.active_sequence_count;
  p->st.active_tokens -= s->length;
  p->st.resident_tokens -= resident;
  p->st.allocated_token_slots -= released * p->P;
  p->st.block_reference_count -= s->blocks.size();
  p->st.shared_blocks -= unshared;
  ++p->st.release_count;
  p->seqs.erase(seq);
  return kOk;
}

std::size_t oracle_length(void* pool, std::uint64_t seq) {
  Sequence* s = find(static_cast<Pool*>(pool), seq);
  return s == nullptr ? 0 : s->length;
}

std::size_t oracle_block_table(void* pool, std::uint64_t seq, std::uint32_t* out,
                               std::size_t capacity) {
  Sequence* s = find(static_cast<Pool*>(pool), seq);
  if (s == nullptr) return 0;
  for (std::size_t i = 0; i < s->blocks.size() && i < capacity; ++i) out[i] = s->blocks[i];
  return s->blocks.size();
}

void oracle_stats(void* pool, Stats* out) { *out = static_cast<Pool*>(pool)->st; }

// Gather one layer into compact [H, dest_tokens, D] outputs; dest_tokens ==
// length is copy_layer (paged.cpp:242-280), larger is copy_layer_prefix_out
// (paged.cpp:895-950), which leaves the trailing rows untouched.
int oracle_copy_layer(void* pool, std::uint64_t seq, std::size_t layer, float* keys_out,
                      float* values_out, std::size_t dest_tokens) {
  auto* p = static_cast<Pool*>(pool);
  Sequence* s = find(p, seq);
  if (s == nullptr) return kInvalidArgument;
  if (layer >= p->L) return kOutOfRange;
  if (dest_tokens < s->length) return kInvalidArgument;
  for (std::size_t h = 0; h < p->H; ++h)
    for (std::size_t lb = 0; lb < s->blocks.size(); ++lb) {
      const std::size_t start = lb * p->P;
      const std::size_t n = std::min(p->P, s->length - start);
      const std::size_t src = p->offset(s->blocks[lb], layer, h, 0);
      const std::size_t dst = (h * dest_tokens + start) * p->D;
      std::memcpy(keys_out + dst, &p->keys[src], n * p->D * sizeof(float));
      std::memcpy(values_out + dst, &p->values[src], n * p->D * sizeof(float));
    }
  return kOk;
}

// Export one layer of the pool in the GPU per-layer layout [N, H, P, D].
void oracle_layer_pages(void* pool, std::size_t layer, float* keys_out, float* values_out) {
  auto* p = static_cast<Pool*>(pool);
  for (std::size_t b = 0; b < p->N; ++b)
    for (std::size_t h = 0; h < p->H; ++h) {
      const std::size_t src = p->offset(static_cast<std::uint32_t>(b), layer, h, 0);
      const std::size_t dst = (b * p->H + h) * p->P * p->D;
      std::memcpy(keys_out + dst, &p->keys[src], p->P * p->D * sizeof(float));
      std::memcpy(values_out + dst, &p->values[src], p->P * p->D * sizeof(float));
    }
}

std::size_t oracle_block_token_count(void* pool, std::uint32_t block) {
  return static_cast<Pool*>(pool)->tokens[block];
}
std::size_t oracle_block_refcount(void* pool, std::uint32_t block) {
  return static_cast<Pool*>(pool)->refs[block];
}

// ----------------------------------------------------------- attention ----
// Shapes: query [Hq, T, D]; key_blocks [N, Hkv, P, D]; value_blocks
// [N, Hkv, P, DV]; tail_key [Hkv, tail, D]; tail_value [Hkv, tail, DV];
// output [Hq, T, DV]; workspace [Hq, T, history + tail] receives the
// probabilities.  tail == 0 selects the history-only form with an explicit
// query_position_offset; tail > 0 requires tail == T and offset == history
// (paged_reference.cpp:398-406).
int oracle_paged_attention(const float* query, std::size_t q_heads, std::size_t kv_heads,
                           std::size_t query_tokens, std::size_t head_dim, std::size_t value_dim,
                           const float* key_blocks, const float* value_blocks,
                           std::size_t block_tokens, const std::uint32_t* block_table,
                           std::size_t history, const float* tail_key, const float* tail_value,
                           std::size_t tail, std::size_t offset, float* output,
                           float* workspace) {
  if (q_heads == 0 || kv_heads == 0 || q_heads % kv_heads != 0 || head_dim == 0 ||
      value_dim == 0 || block_tokens == 0)
    return kInvalidArgument;
  if (tail != 0 && (tail != query_tokens || offset != history)) return kInvalidArgument;
  const std::size_t keys = history + tail;
  if (keys == 0) return kInvalidArgument;
  if (offset > keys || query_tokens > keys - offset) return kInvalidArgument;
  if (query_tokens == 0) return kOk;
  paged_attention(query, q_heads, kv_heads, query_tokens, head_dim, value_dim, key_blocks,
                  value_blocks, block_tokens, block_table, history, tail_key, tail_value, tail,
                  offset, output, workspace);
  return kOk;
}

// Batched decode as a per-sequence loop over the single-sequence oracle:
// query [B, Hq, D], tail [B, Hkv, D], tables [B, max_blocks], lengths [B],
// output [B, Hq, D].  Sequences are split over `threads` std::threads.
int oracle_batched_decode(const float* query, std::size_t batch, std::size_t q_heads,
                          std::size_t kv_heads, std::size_t head_dim, const float* key_blocks,
                          const float* value_blocks, std::size_t block_tokens,
                          const std::uint32_t* tables, std::size_t max_blocks,
                          const std::int32_t* lengths, const float* tail_key,
                          const float* tail_value, float* output, int threads) {
  if (threads < 1) threads = 1;
  auto work = [&](std::size_t first, std::size_t stride) {
    std::vector<float> ws;
    for (std::size_t b = first; b < batch; b += stride) {
      const std::size_t hist = static_cast<std::size_t>(lengths[b]);
      ws.resize(q_heads * (hist + 1));
      paged_attention(query + b * q_heads * head_dim, q_heads, kv_heads, 1, head_dim, head_dim,
                      key_blocks, value_blocks, block_tokens, tables + b * max_blocks, hist,
                      tail_key + b * kv_heads * head_dim, tail_value + b * kv_heads * head_dim, 1,
                      hist, output + b * q_heads * head_dim, ws.data());
    }
  };
  if (threads == 1) {
    work(0, 1);
    return kOk;
  }
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t) pool.emplace_back(work, static_cast<std::size_t>(t),
                                                      static_cast<std::size_t>(threads));
  for (auto& t : pool) t.join();
  return kOk;
}

// Contiguous SDPA (src/attention/reference.cpp:124-226): query [H, Q, D],
// key [H, K, D], value [H, K, DV].  Same arithmetic as the paged form.
int oracle_sdpa(const float* query, const float* key, const float* value, std::size_t heads,
                std::size_t queries, std::size_t keys, std::size_t head_dim,
                std::size_t value_dim, std::size_t offset, float* output, float* workspace) {
  if (heads == 0 || head_dim == 0 || keys == 0) return kInvalidArgument;
  if (offset > keys || queries > keys - offset) return kInvalidArgument;
  const double scale = 1.0 / std::sqrt(static_cast<double>(head_dim));
  for (std::size_t h = 0; h < heads; ++h)
    for (std::size_t qi = 0; qi < queries; ++qi) {
      float* srow = workspace + (h * queries + qi) * keys;
      for (std::size_t k = 0; k < keys; ++k) {
        if (k > offset + qi) {
          srow[k] = -std::numeric_limits<float>::infinity();
          continue;
        }
        double dot = 0.0;
        for (std::size_t d = 0; d < head_dim; ++d)
          dot += static_cast<double>(query[(h * queries + qi) * head_dim + d]) *
                 static_cast<double>(key[(h * keys + k) * head_dim + d]);
        srow[k] = static_cast<float>(dot * scale);
      }
    }
  for (std::size_t r = 0; r < heads * queries; ++r) softmax_row(workspace + r * keys, keys);
  for (std::size_t h = 0; h < heads; ++h)
    for (std::size_t qi = 0; qi < queries; ++qi) {
      const float* prow = workspace + (h * queries + qi) * keys;
      const std::size_t visible = offset + qi + 1;
      for (std::size_t d0 = 0; d0 < value_dim; d0 += 32) {
        const std::size_t td = std::min<std::size_t>(32, value_dim - d0);
        std::array<double, 32> acc{};
        for (std::size_t k = 0; k < visible; ++k) {
          const double p = static_cast<double>(prow[k]);
          for (std::size_t j = 0; j < td; ++j)
            acc[j] += p * static_cast<double>(value[(h * keys + k) * value_dim + d0 + j]);
        }
        for (std::size_t j = 0; j < td; ++j)
          output[(h * queries + qi) * value_dim + d0 + j] = static_cast<float>(acc[j]);
      }
    }
  return kOk;
}

void oracle_softmax_rows(float* data, std::size_t rows, std::size_t width) {
  for (std::size_t r = 0; r < rows; ++r) softmax_row(data + r * width, width);
}

// ------------------------------------------------------------ inputs ----
// Tensor::random_uniform (src/tensor/tensor.cpp:169-189): mt19937_64 seeded
// with `seed`, (bits >> 40) * 2^-24 mapped to [lower, upper] in double and
// cast to float.
void oracle_random_uniform(std::uint64_t seed, float lower, float upper, float* out,
                           std::size_t n) {
  std::mt19937_64 gen(seed);
  const double range = static_cast<double>(upper) - static_cast<double>(lower);
  for (std::size_t i = 0; i < n; ++i) {
    const auto bits = gen() >> 40U;
    out[i] = static_cast<float>(static_cast<double>(lower) +
                                range * (static_cast<double>(bits) * (1.0 / 16777216.0)));
  }
}

// Standard normal via Box-Muller on 53-bit uniforms from mt19937_64.
void oracle_random_normal(std::uint64_t seed, float* out, std::size_t n) {
  std::mt19937_64 gen(seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (std::size_t i = 0; i < n; i += 2) {
    const double u1 = (static_cast<double>(gen() >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = static_cast<double>(gen() >> 11) * (1.0 / 9007199254740992.0);
    const double r = std::sqrt(-2.0 * std::log(u1));
    out[i] = static_cast<float>(r * std::cos(two_pi * u2));
    if (i + 1 < n) out[i + 1] = static_cast<float>(r * std::sin(two_pi * u2));
  }
}

std::uint64_t oracle_mt19937_64_nth(std::uint64_t seed, std::size_t n) {
  std::mt19937_64 gen(seed);
  std::uint64_t v = 0;
  for (std::size_t i = 0; i < n; ++i) v = gen();
  return v;
}

}  // extern "C"
