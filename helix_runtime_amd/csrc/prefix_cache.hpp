// Bounded prefix index over persistent anchor sequences of a paged pool: the
// counterpart of helix::kv_cache::PagedPrefixCache
// (include/helix/kv_cache/prefix.hpp:66-112, src/kv_cache/prefix.cpp).
//
// Behaviour follows the reference: keys are (namespace, exact token IDs) of
// a block-aligned prefix; insert() forks the source at the key length into
// an anchor the cache owns; lookup_longest() forks the anchor of the longest
// stored prefix of the query (bounded by a token limit) for the caller;
// entries live in most-recently-used order and are evicted from the least
// recent end when the entry or block-reference budget would be exceeded.
//
// Structure (ours): one trie per namespace whose edges are whole pages of
// token IDs.  A key of n pages is the node n edges below the root, so the
// longest lookup is one walk down the query's pages with no digest and no
// candidate verification; recency is a monotonically increasing tick per
// entry, ordered in a map.
//
// Locking: every public method takes the prefix-cache mutex, then the pool's
// own lock inside each pool call (the reference's order, prefix.hpp:62-63).
#pragma once

#include <cstddef>
#include <cstdint>
#include <map>
#include <memory>
#include <mutex>
#include <vector>

namespace helix {

// The sequences a prefix cache anchors into: the host block manager or the
// device cache.  Calls throw helix::Error like the pool's own entry points.
class AnchorPool {
public:
  virtual ~AnchorPool() = default;
  [[nodiscard]] virtual std::size_t block_tokens() const = 0;
  // Length of a live sequence of this pool (throws for a foreign or released
  // handle).
  [[nodiscard]] virtual std::size_t length(std::uint64_t id, std::uint64_t cache_id) = 0;
  // Block-aligned fork sharing the first `tokens` tokens.
  [[nodiscard]] virtual std::uint64_t fork(std::uint64_t id, std::size_t tokens) = 0;
  virtual void release(std::uint64_t id) = 0;
  [[nodiscard]] virtual std::uint64_t cache_id() const = 0;
};

struct PrefixCacheConfig {
  std::size_t maximum_entries = 0;
  std::size_t maximum_block_references = 0;
};

enum class PrefixInsert : int { kInserted = 0, kAlreadyPresent = 1, kRejectedTooLarge = 2 };

// Field-for-field PagedPrefixCacheStats (prefix.hpp:47-63).
struct PrefixStats {
  std::size_t maximum_entries = 0;
  std::size_t maximum_block_references = 0;
  std::size_t entry_count = 0;
  std::size_t retained_tokens = 0;
  std::size_t retained_block_references = 0;
  std::size_t peak_entries = 0;
  std::size_t peak_block_references = 0;
  std::uint64_t lookup_count = 0;
  std::uint64_t hit_count = 0;
  std::uint64_t miss_count = 0;
  std::uint64_t insertion_count = 0;
  std::uint64_t duplicate_insertion_count = 0;
  std::uint64_t rejected_insertion_count = 0;
  std::uint64_t eviction_count = 0;
  std::uint64_t erase_count = 0;
};

class PrefixCache {
public:
  PrefixCache(std::unique_ptr<AnchorPool> pool, PrefixCacheConfig config);
  ~PrefixCache();
  PrefixCache(const PrefixCache&) = delete;
  PrefixCache& operator=(const PrefixCache&) = delete;

  PrefixInsert insert(std::uint64_t namespace_id, const std::uint32_t* tokens, std::size_t count,
                      std::uint64_t source, std::uint64_t source_cache_id);
  // True on a hit: *sequence is a new fork the caller must release.
  bool lookup_longest(std::uint64_t namespace_id, const std::uint32_t* tokens, std::size_t count,
                      std::size_t maximum_prefix_tokens, std::uint64_t* sequence,
                      std::size_t* matched_tokens);
  bool contains(std::uint64_t namespace_id, const std::uint32_t* tokens, std::size_t count);
  bool erase(std::uint64_t namespace_id, const std::uint32_t* tokens, std::size_t count);
  bool evict_lru();
  void clear();
  [[nodiscard]] PrefixStats stats();
  [[nodiscard]] const PrefixCacheConfig& config() const noexcept { return config_; }
  [[nodiscard]] std::size_t block_tokens() const noexcept { return page_; }
  [[nodiscard]] std::uint64_t cache_id() const { return pool_->cache_id(); }

private:
  using Page = std::vector<std::uint32_t>;
  static constexpr std::uint32_t kNone = 0xffffffffu;
  struct Node {
    std::uint32_t parent = kNone;
    std::uint64_t namespace_id = 0;  // set on roots
    Page label;                      // the page of token IDs on the edge from the parent
    std::map<Page, std::uint32_t> children;
    std::uint32_t entry = kNone;
  };
  struct Entry {
    std::uint32_t node = kNone;
    std::size_t tokens = 0;
    std::size_t blocks = 0;
    std::uint64_t anchor = 0;
    std::uint64_t tick = 0;
  };

  void validate_key(std::uint64_t namespace_id, const std::uint32_t* tokens, std::size_t count,
                    const char* op) const;
  // Node of the exact key, or kNone.
  [[nodiscard]] std::uint32_t find_node(std::uint64_t namespace_id, const std::uint32_t* tokens,
                                        std::size_t pages) const;
  std::uint32_t make_path(std::uint64_t namespace_id, const std::uint32_t* tokens,
                          std::size_t pages);
  void prune(std::uint32_t node);
  void touch(std::uint32_t entry);
  void drop(std::uint32_t entry, bool eviction);
  [[nodiscard]] std::uint32_t new_node();
  [[nodiscard]] std::uint32_t new_entry();

  std::unique_ptr<AnchorPool> pool_;
  PrefixCacheConfig config_;
  std::size_t page_ = 0;
  std::mutex mutex_;
  std::map<std::uint64_t, std::uint32_t> roots_;  // namespace -> root node
  std::vector<Node> nodes_;
  std::vector<std::uint32_t> free_nodes_;
  std::vector<Entry> entries_;
  std::vector<std::uint32_t> free_entries_;
  std::map<std::uint64_t, std::uint32_t> recency_;  // tick -> entry, oldest first
  std::uint64_t clock_ = 0;
  PrefixStats stats_;
};

}  // namespace helix
