// GPU-resident paged KV cache for one device (the MI355X counterpart of the
// reference's CudaPagedKvCache, include/helix/kv_cache/cuda_paged.hpp:44-120)
// with the CPU cache's sharing features (aligned fork with reference-counted
// pages, src/kv_cache/paged.cpp:535-620) and a copy-on-write extension.
//
// HBM layout: one allocation holds every layer's key and value pool,
// [layers][K|V][physical_blocks][kv_heads][block_tokens][head_dim] fp32, so
// layer l's key pool is the reference's per-layer [N, H, P, D] tensor at
// element offset (2l) * layer_elements and its value pool follows it.
#pragma once

#include "block_manager.hpp"
#include "kernels.hpp"

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <memory>
#include <mutex>
#include <vector>

namespace helix {

// Owning device allocation.
class DeviceBuffer {
public:
  DeviceBuffer() = default;
  DeviceBuffer(std::size_t bytes, int device);
  ~DeviceBuffer();
  DeviceBuffer(const DeviceBuffer&) = delete;
  DeviceBuffer& operator=(const DeviceBuffer&) = delete;
  DeviceBuffer(DeviceBuffer&& o) noexcept;
  DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
  [[nodiscard]] void* data() const noexcept { return ptr_; }
  [[nodiscard]] std::size_t size() const noexcept { return bytes_; }

private:
  void* ptr_ = nullptr;
  std::size_t bytes_ = 0;
};

// Owning pinned host allocation (hipHostMalloc).
class PinnedBuffer {
public:
  PinnedBuffer() = default;
  explicit PinnedBuffer(std::size_t bytes);
  ~PinnedBuffer();
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  PinnedBuffer(PinnedBuffer&& o) noexcept;
  PinnedBuffer& operator=(PinnedBuffer&& o) noexcept;
  [[nodiscard]] void* data() const noexcept { return ptr_; }

private:
  void* ptr_ = nullptr;
};

// Sets the device for the scope and restores the previous one.
class DeviceGuard {
public:
  explicit DeviceGuard(int device);
  ~DeviceGuard();

private:
  int previous_ = -1;
};

void hip_check(hipError_t e, const char* what);

struct CacheState {
  CacheState(const PagedConfig& config, int device, hip::PageFormat page_type = hip::PageFormat());

  BlockManager manager;
  int device;
  hip::PageFormat page_type;  // element type (and fp8 scales) of the pools
  DeviceBuffer slab;
  std::size_t layer_elements = 0;  // physical_blocks * kv_heads * block_tokens * head_dim
  std::mutex mutex;
  bool poisoned = false;
  // Releases through the cache so far: a DecodeBatch compares it with the
  // value at its last prepare() to notice that a member may have been
  // released between the step's calls.
  std::atomic<std::uint64_t> releases{0};
  DeviceBuffer staging;            // transient upload area (grown on demand)

  // Layer pools: fp32 elements, or bf16 / fp8 bits for a reduced-precision
  // cache (the pointer type is nominal then; page_type says which).
  [[nodiscard]] float* key_pool(std::size_t layer) const { return pool_at(2 * layer); }
  [[nodiscard]] float* value_pool(std::size_t layer) const { return pool_at(2 * layer + 1); }
  [[nodiscard]] float* pool_at(std::size_t index) const {
    return reinterpret_cast<float*>(static_cast<unsigned char*>(slab.data()) +
                                    index * layer_elements * hip::page_element_bytes(page_type.type));
  }
  [[nodiscard]] bool bf16() const noexcept { return page_type.type == hip::PageType::kBF16; }
  [[nodiscard]] bool fp8() const noexcept { return page_type.type == hip::PageType::kFP8; }
  [[nodiscard]] bool reduced() const noexcept { return page_type.type != hip::PageType::kF32; }
  [[nodiscard]] std::size_t layer_stride() const noexcept { return 2 * layer_elements; }
  [[nodiscard]] bool overlaps_pool(const void* p, std::size_t bytes) const;
  void require_healthy(const char* op) const;
  void require_sequence(std::uint64_t id, std::uint64_t cache_id, const char* op) const;
  void* staging_bytes(std::size_t bytes);
};

// Every operation takes the cache mutex for its whole duration.  Device work
// is enqueued on the caller's stream and synchronised before metadata is
// committed, as CudaPagedKvCache::append does (src/kv_cache/cuda_paged.cpp:
// 557-611); a failed synchronisation poisons the cache.
class DevicePagedCache {
public:
  DevicePagedCache(const PagedConfig& config, int device,
                   hip::PageFormat page_type = hip::PageFormat());

  [[nodiscard]] const std::shared_ptr<CacheState>& state() const noexcept { return state_; }
  [[nodiscard]] std::uint64_t cache_id() const noexcept { return state_->manager.cache_id(); }

  std::uint64_t create_sequence();
  std::uint64_t fork_sequence(std::uint64_t sequence, std::uint64_t cache_id, std::size_t prefix,
                              bool allow_copy_on_write, hipStream_t stream);
  void append(std::uint64_t sequence, std::uint64_t cache_id, const float* keys,
              const float* values, hipStream_t stream);
  void append_layer_major(std::uint64_t sequence, std::uint64_t cache_id,
                          const float* const* layer_keys, const float* const* layer_values,
                          std::size_t tokens, hipStream_t stream);
  void release(std::uint64_t sequence, std::uint64_t cache_id);
  // Gathers exactly `expected_length` tokens (or the current length when
  // expected_length is SIZE_MAX) of one layer into [kv_heads, dest_tokens,
  // head_dim] device buffers and synchronises the stream.
  void copy_layer_out(std::uint64_t sequence, std::uint64_t cache_id, std::size_t layer,
                      std::size_t expected_length, float* keys_out, float* values_out,
                      std::size_t dest_tokens, hipStream_t stream);

private:
  std::shared_ptr<CacheState> state_;
};

// A read lease: holds the cache mutex and a device copy of one sequence's
// block table (CudaPagedKvCache::DecodeView, cuda_paged.hpp:52-89).
class DecodeView {
public:
  DecodeView(std::shared_ptr<CacheState> state, std::uint64_t sequence, std::uint64_t cache_id);
  [[nodiscard]] std::size_t length() const;
  [[nodiscard]] const std::vector<std::uint32_t>& physical_blocks() const;
  [[nodiscard]] const std::uint32_t* device_table() const;
  [[nodiscard]] float* key_pool(std::size_t layer) const;
  [[nodiscard]] float* value_pool(std::size_t layer) const;
  void poison() noexcept;

private:
  void require_valid(const char* op) const;
  std::shared_ptr<CacheState> state_;
  std::unique_lock<std::mutex> lock_;
  std::size_t length_ = 0;
  std::vector<std::uint32_t> blocks_;
  DeviceBuffer table_;
  bool valid_ = false;
};

// Batched step driver: persistent device block tables [batch, max_blocks]
// and history lengths for a fixed set of sequences, updated incrementally
// each step (one pinned upload + one tiny kernel), plus the split-K
// workspace.  prepare(tokens) reserves and commits `tokens` slots per
// sequence (1 for a decode step, the chunk length for chunked prefill);
// append_layer() must then write those slots for every layer before the
// next prepare().  attention_layer() is the one-token decode,
// prefill_layer() the chunk attention.
//
// Rules the driver enforces:
//  - pages a member gains outside the batch (cache.append /
//    append_layer_major between steps) reach the device tables at the next
//    prepare(): each prepare() uploads every table entry the device copy
//    does not hold yet;
//  - a member released after prepare() makes every later per-step call fail
//    (kInvalidArgument) until the next prepare(), which fails too;
//  - a per-step call on a stream other than prepare()'s waits for the step
//    upload, and prepare() on a stream other than the previous step's last
//    call waits for that call.  Per-step calls of one step on different
//    streams are ordered by the caller (the attention calls share one
//    workspace).
class DecodeBatch {
public:
  DecodeBatch(std::shared_ptr<CacheState> state, const std::uint64_t* sequences,
              const std::uint64_t* cache_ids, std::size_t batch, std::size_t q_heads,
              std::size_t max_tokens, std::size_t pages_per_split);
  ~DecodeBatch();

  void prepare(hipStream_t stream, std::size_t tokens = 1);
  void append_layer(std::size_t layer, const float* keys, const float* values,
                    hipStream_t stream) const;
  // append_layer() for every layer in one launch: rows [layers, batch,
  // kv_heads, tokens, head_dim] (the step's K/V committed after the forward
  // pass, as CudaPagedKvCache::append commits [layers, kv_heads, dim]).
  void append_all_layers(const float* keys, const float* values, hipStream_t stream) const;
  // Rotary embedding of a one-token step's query [batch, q_heads, dim] and
  // key [batch, kv_heads, dim] rows in place, in one launch, each sequence
  // at its position (its length before the step): cosine/sine are
  // [cache_rows, dim / 2] tables as the model's rope cache holds them.
  void rope(float* query, float* key, const float* cosine, const float* sine,
            std::size_t cache_rows, hipStream_t stream) const;
  void attention_layer(std::size_t layer, const float* query, const float* tail_key,
                       const float* tail_value, float* out, hipStream_t stream,
                       bool fused_append = false) const;
  void prefill_layer(std::size_t layer, const float* query, const float* chunk_key,
                     const float* chunk_value, float* out, hipStream_t stream) const;
  // append_layer + attention_layer in one decode launch where the decode
  // kernel supports it (stream mode): the kernel writes each sequence's new
  // token into its slot as it reads the token as the attention tail.
  void append_attention_layer(std::size_t layer, const float* query, const float* keys,
                              const float* values, float* out, hipStream_t stream) const;

  [[nodiscard]] const std::uint32_t* tables() const;
  [[nodiscard]] const std::int32_t* lengths() const;
  [[nodiscard]] const std::int64_t* slots() const;
  [[nodiscard]] std::size_t max_blocks() const noexcept { return max_blocks_; }
  [[nodiscard]] std::size_t pages_per_split() const noexcept { return pages_per_split_; }
  [[nodiscard]] std::size_t batch() const noexcept { return sequences_.size(); }
  [[nodiscard]] std::size_t step_tokens() const noexcept { return step_tokens_; }
  [[nodiscard]] std::size_t shared_pages() const noexcept { return shared_pages_; }
  // Measurement hook: when set, attention_layer() records this event between
  // the main decode kernel and the merge kernel.
  void set_between_event(hipEvent_t e) noexcept { between_event_ = e; }

private:
  std::shared_ptr<CacheState> state_;
  std::vector<std::uint64_t> sequences_;
  std::size_t q_heads_;
  std::size_t max_blocks_;
  std::size_t pages_per_split_;
  std::size_t items_ = 0;      // work items of the prepared step
  std::vector<std::int32_t> host_lengths_;
  DeviceBuffer tables_;
  DeviceBuffer step_;       // lengths [B] int32 | slots [B, tokens] int64 | updates
  DeviceBuffer workspace_;
  PinnedBuffer pinned_[2];
  hipEvent_t uploaded_[2] = {nullptr, nullptr};
  int next_pinned_ = 0;
  std::size_t step_bytes_ = 0;
  std::size_t step_capacity_ = 0;  // tokens per sequence the step buffers hold
  std::size_t step_tokens_ = 0;    // tokens of the prepared step
  bool prepared_ = false;
  hipEvent_t between_event_ = nullptr;
  std::size_t shared_pages_ = 0;  // cascade prefix of the prepared step (0: off)
  // Created with the first cascade step: the prefix pass's stream and the
  // events that fork it from and join it to the caller's stream.
  hipStream_t side_stream_ = nullptr;
  hipEvent_t fork_event_ = nullptr;
  hipEvent_t join_event_ = nullptr;
  // A decode step uses the cascade when at least this many sequences share
  // at least this many leading pages.
  static constexpr std::size_t kMinCascadeBatch = 4;
  static constexpr std::size_t kMinCascadePages = 4;

  // Host mirror of the device tables and the entries of each row that the
  // device copy holds (table rows only grow while a sequence lives).
  std::vector<std::uint32_t> mirror_;
  std::vector<std::size_t> mirrored_;
  mutable std::uint64_t prepared_releases_ = 0;
  hipStream_t prepared_stream_ = nullptr;
  int prepared_event_ = 0;  // uploaded_[prepared_event_] follows the step upload
  mutable hipStream_t last_stream_ = nullptr;
  mutable bool any_call_ = false;
  hipEvent_t order_event_ = nullptr;

  void reserve_step(std::size_t tokens);
  // Checks that the step is prepared and its members still live, and orders
  // `stream` after the step upload.
  void begin_call(hipStream_t stream, const char* op) const;
  [[nodiscard]] std::size_t order_offset(std::size_t tokens) const;
  [[nodiscard]] std::size_t prefill_items(std::size_t tokens) const;
};

}  // namespace helix
