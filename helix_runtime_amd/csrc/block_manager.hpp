// Host-side page bookkeeping of the paged KV pool: the FIFO free-block queue,
// per-sequence block tables, per-block reference and written-token counts and
// the statistics.  No device memory is touched here; the device cache
// (paged_cache.hpp) plans a mutation, performs the page copies on the GPU and
// only then commits the plan, which keeps every operation transactional.
//
// Behaviour follows the reference's PagedKvCache metadata
// (src/kv_cache/paged.cpp): FIFO queue :139-188, create :509-533, aligned
// fork :535-620, append :622-719, bulk append :721-871, release :952-1001,
// invariants :282-393.  Copy-on-write forks at a non-aligned prefix are an
// extension (the reference rejects them, paged.cpp:544-545).
#pragma once

#include <cstddef>
#include <cstdint>
#include <unordered_map>
#include <vector>

namespace helix {

struct PagedConfig {
  std::size_t layers = 0;
  std::size_t kv_heads = 0;
  std::size_t head_dimension = 0;
  std::size_t block_tokens = 0;
  std::size_t physical_blocks = 0;
};

// Field order and meaning of PagedKvCacheStats (include/helix/kv_cache/
// paged.hpp:68-107), all widened to 64 bits.
struct PagedStats {
  std::uint64_t bytes_reserved = 0;
  std::uint64_t bytes_used = 0;
  std::uint64_t bytes_free = 0;
  std::uint64_t peak_bytes_used = 0;
  std::uint64_t total_blocks = 0;
  std::uint64_t used_blocks = 0;
  std::uint64_t free_blocks = 0;
  std::uint64_t active_sequence_count = 0;
  std::uint64_t active_tokens = 0;
  std::uint64_t resident_tokens = 0;
  std::uint64_t allocated_token_slots = 0;
  std::uint64_t block_reference_count = 0;
  std::uint64_t shared_blocks = 0;
  std::uint64_t sequence_create_count = 0;
  std::uint64_t sequence_fork_count = 0;
  std::uint64_t append_count = 0;
  std::uint64_t release_count = 0;
  std::uint64_t block_allocation_count = 0;
  std::uint64_t block_reuse_count = 0;
};

// Pages an append of `tokens` tokens touches: logical blocks first_block ..
// first_block + blocks.size() - 1, of which the last `new_blocks` come from
// the head of the FIFO in order.
struct AppendPlan {
  std::uint64_t sequence = 0;
  std::size_t old_length = 0;
  std::size_t tokens = 0;
  std::size_t first_block = 0;
  std::vector<std::uint32_t> blocks;
  std::size_t new_blocks = 0;
  std::uint64_t reused_blocks = 0;

  // Physical slot (block * block_tokens + offset) of appended token i.
  [[nodiscard]] std::uint64_t slot(std::size_t i, std::size_t block_tokens) const {
    const std::size_t pos = old_length + i;
    return static_cast<std::uint64_t>(blocks[pos / block_tokens - first_block]) * block_tokens +
           pos % block_tokens;
  }
};

struct ForkPlan {
  std::uint64_t source = 0;
  std::size_t prefix = 0;
  std::size_t shared_blocks = 0;
  std::size_t newly_shared = 0;
  bool copy_on_write = false;
  std::uint32_t cow_from = 0;
  std::uint32_t cow_to = 0;
  std::size_t cow_tokens = 0;
};

class BlockManager {
public:
  // element_bytes: 4 for fp32 pages (the reference's), 2 for bf16, 1 for fp8;
  // it scales the byte figures of the geometry and statistics only.
  explicit BlockManager(const PagedConfig& config, std::size_t element_bytes = 4);

  [[nodiscard]] const PagedConfig& config() const noexcept { return config_; }
  [[nodiscard]] std::uint64_t cache_id() const noexcept { return cache_id_; }
  [[nodiscard]] std::size_t bytes_per_token() const noexcept { return bytes_per_token_; }
  [[nodiscard]] std::size_t block_bytes() const noexcept { return block_bytes_; }
  [[nodiscard]] std::size_t token_capacity() const noexcept {
    return config_.physical_blocks * config_.block_tokens;
  }
  [[nodiscard]] const PagedStats& stats() const noexcept { return stats_; }

  std::uint64_t create_sequence();
  [[nodiscard]] AppendPlan plan_append(std::uint64_t sequence, std::size_t tokens) const;
  void commit_append(const AppendPlan& plan);
  [[nodiscard]] ForkPlan plan_fork(std::uint64_t source, std::size_t prefix,
                                   bool allow_copy_on_write) const;
  std::uint64_t commit_fork(const ForkPlan& plan);
  void release(std::uint64_t sequence);

  // Free blocks the FIFO can still hand out.
  [[nodiscard]] std::size_t free_block_count() const noexcept { return free_count_; }
  [[nodiscard]] bool contains(std::uint64_t sequence) const;
  [[nodiscard]] std::size_t length(std::uint64_t sequence) const;
  [[nodiscard]] const std::vector<std::uint32_t>& blocks(std::uint64_t sequence) const;
  [[nodiscard]] std::size_t block_reference_count(std::uint32_t block) const;
  [[nodiscard]] std::size_t block_token_count(std::uint32_t block) const;

  // Re-derives every invariant from the tables (paged.cpp:282-393); throws
  // Status::kInternal on the first inconsistency.
  void validate() const;

private:
  struct Sequence {
    std::size_t length = 0;
    std::vector<std::uint32_t> blocks;
  };

  [[nodiscard]] const Sequence& require(std::uint64_t id, const char* op) const;
  [[nodiscard]] std::uint32_t fifo_at(std::size_t i) const {
    return fifo_[(fifo_head_ + i) % fifo_.size()];
  }
  void take_block(Sequence& s, std::uint32_t block);

  PagedConfig config_;
  std::uint64_t cache_id_ = 0;
  std::size_t bytes_per_token_ = 0;
  std::size_t block_bytes_ = 0;
  std::vector<std::uint32_t> fifo_;
  std::size_t fifo_head_ = 0;
  std::size_t fifo_tail_ = 0;
  std::size_t free_count_ = 0;
  std::vector<std::size_t> refs_;
  std::vector<std::size_t> tokens_;
  std::vector<std::uint8_t> was_allocated_;
  std::unordered_map<std::uint64_t, Sequence> sequences_;
  std::uint64_t next_id_ = 1;
  PagedStats stats_;
};

}  // namespace helix
