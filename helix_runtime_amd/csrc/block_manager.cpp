#include "block_manager.hpp"

#include "status.hpp"

#include <algorithm>
#include <atomic>
#include <limits>
#include <string>

namespace helix {
namespace {

std::uint64_t next_cache_id() {
  static std::atomic<std::uint64_t> next{1};
  return next.fetch_add(1, std::memory_order_relaxed);
}

std::size_t checked_mul(std::size_t a, std::size_t b, const char* what) {
  if (a != 0 && b > std::numeric_limits<std::size_t>::max() / a) {
    fail(Status::kOutOfRange, std::string(what) + " overflows size_t");
  }
  return a * b;
}

std::size_t blocks_for(std::size_t tokens, std::size_t block_tokens) {
  return tokens / block_tokens + (tokens % block_tokens != 0 ? 1 : 0);
}

}  // namespace

// Pool geometry checks and byte formulas of make_layout
// (src/kv_cache/paged.cpp:53-106).
BlockManager::BlockManager(const PagedConfig& config, std::size_t element_bytes)
    : config_(config) {
  check(element_bytes == 4 || element_bytes == 2 || element_bytes == 1, Status::kInvalidArgument,
        "paged KV cache page elements are 4 (fp32), 2 (bf16) or 1 (fp8) bytes");
  check(config.layers != 0, Status::kInvalidArgument, "paged KV cache layer count must be positive");
  check(config.kv_heads != 0, Status::kInvalidArgument, "paged KV cache head count must be positive");
  check(config.head_dimension != 0, Status::kInvalidArgument,
        "paged KV cache head dimension must be positive");
  check(config.block_tokens != 0, Status::kInvalidArgument,
        "paged KV cache block token count must be positive");
  check(config.physical_blocks != 0, Status::kInvalidArgument,
        "paged KV cache physical block count must be positive");
  check(config.physical_blocks <= std::numeric_limits<std::uint32_t>::max(), Status::kOutOfRange,
        "paged KV cache physical block count exceeds the uint32 block-ID capacity");
  std::size_t token_elems = checked_mul(config.layers, 2, "bytes per token");
  token_elems = checked_mul(token_elems, config.kv_heads, "bytes per token");
  token_elems = checked_mul(token_elems, config.head_dimension, "bytes per token");
  bytes_per_token_ = checked_mul(token_elems, element_bytes, "bytes per token");
  block_bytes_ = checked_mul(bytes_per_token_, config.block_tokens, "block bytes");
  const std::size_t pool = checked_mul(block_bytes_, config.physical_blocks, "pool bytes");
  static_cast<void>(checked_mul(config.physical_blocks, config.block_tokens, "token capacity"));

  cache_id_ = next_cache_id();
  fifo_.resize(config.physical_blocks);
  for (std::size_t i = 0; i < fifo_.size(); ++i) fifo_[i] = static_cast<std::uint32_t>(i);
  free_count_ = config.physical_blocks;
  refs_.assign(config.physical_blocks, 0);
  tokens_.assign(config.physical_blocks, 0);
  was_allocated_.assign(config.physical_blocks, 0);
  stats_.bytes_reserved = pool;
  stats_.bytes_free = pool;
  stats_.total_blocks = config.physical_blocks;
  stats_.free_blocks = config.physical_blocks;
}

const BlockManager::Sequence& BlockManager::require(std::uint64_t id, const char* op) const {
  const auto it = sequences_.find(id);
  check(id != 0 && it != sequences_.end(), Status::kInvalidArgument,
        std::string(op) + ": sequence is unknown or was already released");
  return it->second;
}

bool BlockManager::contains(std::uint64_t sequence) const {
  return sequences_.find(sequence) != sequences_.end();
}

std::size_t BlockManager::length(std::uint64_t sequence) const {
  return require(sequence, "length").length;
}

const std::vector<std::uint32_t>& BlockManager::blocks(std::uint64_t sequence) const {
  return require(sequence, "block_table").blocks;
}

std::size_t BlockManager::block_reference_count(std::uint32_t block) const {
  check(block < refs_.size(), Status::kOutOfRange, "block ID is out of range");
  return refs_[block];
}

std::size_t BlockManager::block_token_count(std::uint32_t block) const {
  check(block < tokens_.size(), Status::kOutOfRange, "block ID is out of range");
  return tokens_[block];
}

std::uint64_t BlockManager::create_sequence() {
  check(next_id_ != std::numeric_limits<std::uint64_t>::max(), Status::kResourceExhausted,
        "paged KV sequence id space exhausted");
  const std::uint64_t id = next_id_;
  sequences_.emplace(id, Sequence{});
  ++next_id_;
  ++stats_.active_sequence_count;
  ++stats_.sequence_create_count;
  return id;
}

void BlockManager::take_block(Sequence& s, std::uint32_t block) {
  s.blocks.push_back(block);
  refs_[block] = 1;
  was_allocated_[block] = 1;
  ++stats_.used_blocks;
  --stats_.free_blocks;
  stats_.bytes_used += block_bytes_;
  stats_.bytes_free -= block_bytes_;
  stats_.peak_bytes_used = std::max(stats_.peak_bytes_used, stats_.bytes_used);
  stats_.allocated_token_slots += config_.block_tokens;
  ++stats_.block_reference_count;
  ++stats_.block_allocation_count;
}

// append (paged.cpp:622-719) and append_layer_major (paged.cpp:721-871):
// validation and reservation happen before any state changes.
AppendPlan BlockManager::plan_append(std::uint64_t sequence, std::size_t tokens) const {
  const Sequence& s = require(sequence, "append");
  check(tokens != 0, Status::kInvalidArgument, "append token count must be positive");
  check(tokens <= std::numeric_limits<std::size_t>::max() - s.length, Status::kResourceExhausted,
        "append: sequence length would overflow");
  const std::size_t P = config_.block_tokens;
  const std::size_t result = s.length + tokens;
  const std::size_t need = blocks_for(result, P);
  const std::size_t extra = need - s.blocks.size();
  check(extra <= free_count_, Status::kResourceExhausted,
        "append: the pool has no free physical KV block for the new tokens");
  if (s.length % P != 0) {
    check(refs_[s.blocks.back()] == 1, Status::kInternal,
          "append would mutate a shared partial block");
  }
  AppendPlan plan;
  plan.sequence = sequence;
  plan.old_length = s.length;
  plan.tokens = tokens;
  plan.first_block = s.length / P;
  plan.new_blocks = extra;
  for (std::size_t lb = plan.first_block; lb < s.blocks.size(); ++lb) {
    plan.blocks.push_back(s.blocks[lb]);
  }
  for (std::size_t i = 0; i < extra; ++i) {
    const std::uint32_t b = fifo_at(i);
    plan.blocks.push_back(b);
    plan.reused_blocks += was_allocated_[b] != 0 ? 1 : 0;
  }
  return plan;
}

void BlockManager::commit_append(const AppendPlan& plan) {
  auto it = sequences_.find(plan.sequence);
  check(it != sequences_.end() && it->second.length == plan.old_length, Status::kInternal,
        "append plan is stale");
  Sequence& s = it->second;
  for (std::size_t i = 0; i < plan.new_blocks; ++i) {
    const std::uint32_t b = fifo_[fifo_head_];
    check(b == plan.blocks[plan.blocks.size() - plan.new_blocks + i], Status::kInternal,
          "append plan disagrees with the free queue");
    fifo_head_ = (fifo_head_ + 1) % fifo_.size();
    --free_count_;
    if (was_allocated_[b] != 0) ++stats_.block_reuse_count;
    take_block(s, b);
  }
  const std::size_t P = config_.block_tokens;
  s.length = plan.old_length + plan.tokens;
  for (std::size_t lb = plan.first_block; lb < s.blocks.size(); ++lb) {
    tokens_[s.blocks[lb]] = std::min(P, s.length - lb * P);
  }
  stats_.active_tokens += plan.tokens;
  stats_.resident_tokens += plan.tokens;
  stats_.append_count += plan.tokens;
}

// fork_sequence (paged.cpp:535-620) plus the copy-on-write extension.
ForkPlan BlockManager::plan_fork(std::uint64_t source, std::size_t prefix,
                                 bool allow_copy_on_write) const {
  const Sequence& s = require(source, "fork_sequence");
  check(prefix != 0, Status::kInvalidArgument, "fork_sequence prefix must contain at least one token");
  check(prefix <= s.length, Status::kOutOfRange,
        "fork_sequence prefix exceeds the source sequence length");
  const std::size_t P = config_.block_tokens;
  const std::size_t rem = prefix % P;
  check(rem == 0 || allow_copy_on_write, Status::kInvalidArgument,
        "fork_sequence prefix must end on a KV block boundary");
  ForkPlan plan;
  plan.source = source;
  plan.prefix = prefix;
  plan.shared_blocks = prefix / P;
  for (std::size_t i = 0; i < plan.shared_blocks; ++i) {
    const std::uint32_t b = s.blocks[i];
    check(tokens_[b] == P, Status::kInternal, "fork encountered a partial physical block");
    plan.newly_shared += refs_[b] == 1 ? 1 : 0;
  }
  if (rem != 0) {
    check(free_count_ != 0, Status::kResourceExhausted,
          "fork_sequence has no free physical KV block for the copy-on-write page");
    plan.copy_on_write = true;
    plan.cow_from = s.blocks[plan.shared_blocks];
    plan.cow_to = fifo_at(0);
    plan.cow_tokens = rem;
  }
  return plan;
}

std::uint64_t BlockManager::commit_fork(const ForkPlan& plan) {
  const Sequence& src = require(plan.source, "fork_sequence");
  Sequence f;
  f.length = plan.prefix;
  f.blocks.assign(src.blocks.begin(),
                  src.blocks.begin() + static_cast<std::ptrdiff_t>(plan.shared_blocks));
  for (std::size_t i = 0; i < plan.shared_blocks; ++i) ++refs_[src.blocks[i]];
  stats_.block_reference_count += plan.shared_blocks;
  stats_.shared_blocks += plan.newly_shared;
  if (plan.copy_on_write) {
    const std::uint32_t b = fifo_[fifo_head_];
    check(b == plan.cow_to, Status::kInternal, "fork plan disagrees with the free queue");
    fifo_head_ = (fifo_head_ + 1) % fifo_.size();
    --free_count_;
    if (was_allocated_[b] != 0) ++stats_.block_reuse_count;
    take_block(f, b);
    tokens_[b] = plan.cow_tokens;
    stats_.resident_tokens += plan.cow_tokens;
  }
  const std::uint64_t id = next_id_++;
  sequences_.emplace(id, std::move(f));
  ++stats_.active_sequence_count;
  stats_.active_tokens += plan.prefix;
  ++stats_.sequence_create_count;
  ++stats_.sequence_fork_count;
  return id;
}

// release_sequence (paged.cpp:952-1001): zero-reference blocks return to the
// FIFO tail in table order.
void BlockManager::release(std::uint64_t sequence) {
  const Sequence& s = require(sequence, "release_sequence");
  std::size_t released = 0, resident = 0, unshared = 0;
  for (const std::uint32_t b : s.blocks) {
    if (refs_[b] == 1) {
      ++released;
      resident += tokens_[b];
    } else if (refs_[b] == 2) {
      ++unshared;
    }
  }
  for (const std::uint32_t b : s.blocks) {
    if (--refs_[b] == 0) {
      tokens_[b] = 0;
      fifo_[fifo_tail_] = b;
      fifo_tail_ = (fifo_tail_ + 1) % fifo_.size();
      ++free_count_;
    }
  }
  stats_.used_blocks -= released;
  stats_.free_blocks += released;
  stats_.bytes_used -= released * block_bytes_;
  stats_.bytes_free += released * block_bytes_;
  --stats_.active_sequence_count;
  stats_.active_tokens -= s.length;
  stats_.resident_tokens -= resident;
  stats_.allocated_token_slots -= released * config_.block_tokens;
  stats_.block_reference_count -= s.blocks.size();
  stats_.shared_blocks -= unshared;
  ++stats_.release_count;
  sequences_.erase(sequence);
}

void BlockManager::validate() const {
  auto expect = [](bool ok, const char* what) { check(ok, Status::kInternal, what); };
  const std::size_t P = config_.block_tokens;
  std::vector<std::size_t> derived(config_.physical_blocks, 0);
  std::size_t logical_tokens = 0, mapped = 0;
  for (const auto& [id, s] : sequences_) {
    expect(id != 0, "sequence uses the reserved zero identity");
    expect(s.blocks.size() == blocks_for(s.length, P), "block-table length disagrees with length");
    logical_tokens += s.length;
    mapped += s.blocks.size();
    for (std::size_t lb = 0; lb < s.blocks.size(); ++lb) {
      const std::uint32_t b = s.blocks[lb];
      expect(b < config_.physical_blocks, "block table holds an invalid physical block");
      expect(refs_[b] != 0, "block table references an unowned block");
      expect(tokens_[b] == std::min(P, s.length - lb * P), "block payload length disagrees");
      for (std::size_t prior = 0; prior < lb; ++prior) {
        expect(s.blocks[prior] != b, "sequence maps one physical block twice");
      }
      ++derived[b];
    }
  }
  std::size_t referenced = 0, resident = 0, shared = 0, free_members = 0;
  for (std::size_t b = 0; b < config_.physical_blocks; ++b) {
    expect(refs_[b] == derived[b], "reference count disagrees with the block tables");
    if (derived[b] == 0) {
      ++free_members;
      expect(tokens_[b] == 0, "free block retains a written-token count");
    } else {
      ++referenced;
      resident += tokens_[b];
      shared += derived[b] > 1 ? 1 : 0;
      expect(was_allocated_[b] != 0, "referenced block lacks allocation history");
      expect(tokens_[b] != 0 && tokens_[b] <= P, "referenced block has an invalid token count");
      expect(derived[b] == 1 || tokens_[b] == P, "a partially written block is shared");
    }
  }
  std::vector<std::uint8_t> seen(config_.physical_blocks, 0);
  for (std::size_t i = 0; i < free_count_; ++i) {
    const std::uint32_t b = fifo_at(i);
    expect(b < config_.physical_blocks && refs_[b] == 0, "free queue holds a referenced block");
    expect(seen[b] == 0, "free queue holds a duplicate block");
    seen[b] = 1;
  }
  expect(free_members == free_count_, "free membership and queue disagree");
  expect(referenced + free_count_ == config_.physical_blocks, "accounting does not cover the pool");
  expect(stats_.used_blocks == referenced && stats_.free_blocks == free_count_,
         "used/free block statistics are inconsistent");
  expect(stats_.active_sequence_count == sequences_.size(), "sequence statistic is inconsistent");
  expect(stats_.active_tokens == logical_tokens, "active-token statistic is inconsistent");
  expect(stats_.resident_tokens == resident, "resident-token statistic is inconsistent");
  expect(stats_.block_reference_count == mapped, "block-reference statistic is inconsistent");
  expect(stats_.shared_blocks == shared, "shared-block statistic is inconsistent");
  expect(stats_.allocated_token_slots == referenced * P, "token-slot statistic is inconsistent");
  expect(stats_.bytes_used == referenced * block_bytes_, "used-byte statistic is inconsistent");
  expect(stats_.bytes_free == free_count_ * block_bytes_, "free-byte statistic is inconsistent");
  expect(stats_.bytes_used + stats_.bytes_free == stats_.bytes_reserved,
         "byte statistics do not cover the pool");
}

}  // namespace helix
