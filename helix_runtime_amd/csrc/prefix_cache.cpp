#include "prefix_cache.hpp"

#include "status.hpp"

#include <algorithm>
#include <limits>
#include <new>
#include <string>
#include <utility>

namespace helix {
namespace {

void bump(std::uint64_t& counter) noexcept {
  if (counter != std::numeric_limits<std::uint64_t>::max()) ++counter;
}

}  // namespace

// Constructor checks of prefix.cpp:124-139.
PrefixCache::PrefixCache(std::unique_ptr<AnchorPool> pool, PrefixCacheConfig config)
    : pool_(std::move(pool)), config_(config) {
  check(pool_ != nullptr, Status::kInvalidArgument, "prefix cache: paged cache must not be null");
  check(config_.maximum_entries != 0, Status::kInvalidArgument,
        "prefix cache: maximum entry count must be positive");
  check(config_.maximum_block_references != 0, Status::kInvalidArgument,
        "prefix cache: maximum block-reference count must be positive");
  page_ = pool_->block_tokens();
  check(config_.maximum_block_references <= std::numeric_limits<std::size_t>::max() / page_,
        Status::kOutOfRange, "prefix cache: retained token accounting would overflow");
  stats_.maximum_entries = config_.maximum_entries;
  stats_.maximum_block_references = config_.maximum_block_references;
}

// The destructor releases every anchor it still holds (prefix.cpp:277-287).
PrefixCache::~PrefixCache() {
  try {
    clear();
  } catch (...) {
    // Destructors must not throw; an anchor the pool refused stays with it.
  }
}

// prefix.cpp:151-161: namespace 0 is reserved, keys are non-empty and end
// on a page boundary.
void PrefixCache::validate_key(std::uint64_t namespace_id, const std::uint32_t* tokens,
                               std::size_t count, const char* op) const {
  check(namespace_id != 0, Status::kInvalidArgument,
        std::string("prefix cache ") + op + ": prefix namespace zero is reserved as invalid");
  check(count != 0 && tokens != nullptr, Status::kInvalidArgument,
        std::string("prefix cache ") + op + ": prefix must contain at least one token");
  check(count % page_ == 0, Status::kInvalidArgument,
        std::string("prefix cache ") + op + ": prefix must end on a KV block boundary");
}

std::uint32_t PrefixCache::new_node() {
  if (!free_nodes_.empty()) {
    const std::uint32_t n = free_nodes_.back();
    free_nodes_.pop_back();
    nodes_[n] = Node{};
    return n;
  }
  nodes_.emplace_back();
  return static_cast<std::uint32_t>(nodes_.size() - 1);
}

std::uint32_t PrefixCache::new_entry() {
  if (!free_entries_.empty()) {
    const std::uint32_t e = free_entries_.back();
    free_entries_.pop_back();
    entries_[e] = Entry{};
    return e;
  }
  entries_.emplace_back();
  return static_cast<std::uint32_t>(entries_.size() - 1);
}

std::uint32_t PrefixCache::find_node(std::uint64_t namespace_id, const std::uint32_t* tokens,
                                     std::size_t pages) const {
  const auto root = roots_.find(namespace_id);
  if (root == roots_.end()) return kNone;
  std::uint32_t node = root->second;
  Page key(page_);
  for (std::size_t p = 0; p < pages; ++p) {
    std::copy(tokens + p * page_, tokens + (p + 1) * page_, key.begin());
    const auto child = nodes_[node].children.find(key);
    if (child == nodes_[node].children.end()) return kNone;
    node = child->second;
  }
  return node;
}

// Creates the missing nodes of a key's path; returns the key's node.  On an
// allocation failure the partial path is pruned and the failure rethrown.
std::uint32_t PrefixCache::make_path(std::uint64_t namespace_id, const std::uint32_t* tokens,
                                     std::size_t pages) {
  std::uint32_t node = kNone;
  try {
    auto root = roots_.find(namespace_id);
    if (root == roots_.end()) {
      const std::uint32_t r = new_node();
      nodes_[r].namespace_id = namespace_id;
      root = roots_.emplace(namespace_id, r).first;
    }
    node = root->second;
    for (std::size_t p = 0; p < pages; ++p) {
      Page key(tokens + p * page_, tokens + (p + 1) * page_);
      const auto child = nodes_[node].children.find(key);
      if (child != nodes_[node].children.end()) {
        node = child->second;
        continue;
      }
      const std::uint32_t c = new_node();
      nodes_[c].parent = node;
      nodes_[c].label = key;
      nodes_[node].children.emplace(std::move(key), c);
      node = c;
    }
    return node;
  } catch (const std::bad_alloc&) {
    if (node != kNone) prune(node);
    throw;
  }
}

// Removes entry-less leaves from `node` upwards, the root included when its
// namespace becomes empty.
void PrefixCache::prune(std::uint32_t node) {
  while (node != kNone && nodes_[node].entry == kNone && nodes_[node].children.empty()) {
    const std::uint32_t parent = nodes_[node].parent;
    if (parent == kNone) {
      roots_.erase(nodes_[node].namespace_id);
    } else {
      nodes_[parent].children.erase(nodes_[node].label);
    }
    nodes_[node] = Node{};
    free_nodes_.push_back(node);
    node = parent;
  }
}

void PrefixCache::touch(std::uint32_t entry) {
  Entry& e = entries_[entry];
  if (e.tick != 0) recency_.erase(e.tick);
  e.tick = ++clock_;
  recency_.emplace(e.tick, entry);
}

// prefix.cpp:164-186: the anchor is released first; a pool that refuses it
// leaves the entry in place.
void PrefixCache::drop(std::uint32_t entry, bool eviction) {
  Entry& e = entries_[entry];
  pool_->release(e.anchor);
  nodes_[e.node].entry = kNone;
  prune(e.node);
  recency_.erase(e.tick);
  stats_.retained_tokens -= e.tokens;
  stats_.retained_block_references -= e.blocks;
  --stats_.entry_count;
  bump(eviction ? stats_.eviction_count : stats_.erase_count);
  e = Entry{};
  free_entries_.push_back(entry);
}

// prefix.cpp:296-358.
PrefixInsert PrefixCache::insert(std::uint64_t namespace_id, const std::uint32_t* tokens,
                                 std::size_t count, std::uint64_t source,
                                 std::uint64_t source_cache_id) {
  std::scoped_lock lock(mutex_);
  validate_key(namespace_id, tokens, count, "insert");
  const std::size_t source_length = pool_->length(source, source_cache_id);
  check(count <= source_length, Status::kOutOfRange,
        "prefix cache insert: prefix exceeds the source sequence length");

  const std::size_t pages = count / page_;
  const std::uint32_t existing = find_node(namespace_id, tokens, pages);
  if (existing != kNone && nodes_[existing].entry != kNone) {
    touch(nodes_[existing].entry);
    bump(stats_.duplicate_insertion_count);
    return PrefixInsert::kAlreadyPresent;
  }
  if (pages > config_.maximum_block_references) {
    bump(stats_.rejected_insertion_count);
    return PrefixInsert::kRejectedTooLarge;
  }

  const std::uint64_t anchor = pool_->fork(source, count);
  std::uint32_t entry = kNone;
  try {
    const std::uint32_t node = make_path(namespace_id, tokens, pages);
    try {
      entry = new_entry();
    } catch (const std::bad_alloc&) {
      prune(node);
      throw;
    }
    entries_[entry].node = node;
    entries_[entry].tokens = count;
    entries_[entry].blocks = pages;
    entries_[entry].anchor = anchor;
    nodes_[node].entry = entry;
    touch(entry);
  } catch (const std::bad_alloc&) {
    if (entry != kNone) {
      nodes_[entries_[entry].node].entry = kNone;
      prune(entries_[entry].node);
      entries_[entry] = Entry{};
      free_entries_.push_back(entry);
    }
    pool_->release(anchor);
    fail(Status::kResourceExhausted, "prefix cache insert could not allocate its index entry");
  }

  // Least recent entries go first until both budgets hold with the new entry
  // counted (prefix.cpp:188-198); the new entry is the most recent one.
  while (stats_.entry_count + 1 > config_.maximum_entries ||
         stats_.retained_block_references > config_.maximum_block_references - pages) {
    const std::uint32_t oldest = recency_.begin()->second;
    check(oldest != entry, Status::kInternal, "prefix cache eviction reached the new entry");
    drop(oldest, true);
  }
  ++stats_.entry_count;
  stats_.retained_tokens += count;
  stats_.retained_block_references += pages;
  stats_.peak_entries = std::max(stats_.peak_entries, stats_.entry_count);
  stats_.peak_block_references =
      std::max(stats_.peak_block_references, stats_.retained_block_references);
  bump(stats_.insertion_count);
  return PrefixInsert::kInserted;
}

// prefix.cpp:360-403: the deepest stored page-aligned prefix within the
// token bound wins; a hit forks that anchor for the caller.
bool PrefixCache::lookup_longest(std::uint64_t namespace_id, const std::uint32_t* tokens,
                                 std::size_t count, std::size_t maximum_prefix_tokens,
                                 std::uint64_t* sequence, std::size_t* matched_tokens) {
  std::scoped_lock lock(mutex_);
  check(namespace_id != 0, Status::kInvalidArgument,
        "prefix cache lookup_longest: prefix namespace zero is reserved as invalid");
  check(count == 0 || tokens != nullptr, Status::kInvalidArgument,
        "prefix cache lookup_longest: tokens must not be NULL");
  const std::size_t bounded = std::min(count, maximum_prefix_tokens);
  const std::size_t pages = bounded / page_;
  std::uint32_t best = kNone;
  const auto root = roots_.find(namespace_id);
  if (root != roots_.end()) {
    std::uint32_t node = root->second;
    Page key(page_);
    for (std::size_t p = 0; p < pages; ++p) {
      std::copy(tokens + p * page_, tokens + (p + 1) * page_, key.begin());
      const auto child = nodes_[node].children.find(key);
      if (child == nodes_[node].children.end()) break;
      node = child->second;
      if (nodes_[node].entry != kNone) best = nodes_[node].entry;
    }
  }
  if (best == kNone) {
    bump(stats_.lookup_count);
    bump(stats_.miss_count);
    return false;
  }
  const std::uint64_t forked = pool_->fork(entries_[best].anchor, entries_[best].tokens);
  touch(best);
  bump(stats_.lookup_count);
  bump(stats_.hit_count);
  *sequence = forked;
  *matched_tokens = entries_[best].tokens;
  return true;
}

bool PrefixCache::contains(std::uint64_t namespace_id, const std::uint32_t* tokens,
                           std::size_t count) {
  std::scoped_lock lock(mutex_);
  validate_key(namespace_id, tokens, count, "contains");
  const std::uint32_t node = find_node(namespace_id, tokens, count / page_);
  return node != kNone && nodes_[node].entry != kNone;
}

bool PrefixCache::erase(std::uint64_t namespace_id, const std::uint32_t* tokens,
                        std::size_t count) {
  std::scoped_lock lock(mutex_);
  validate_key(namespace_id, tokens, count, "erase");
  const std::uint32_t node = find_node(namespace_id, tokens, count / page_);
  if (node == kNone || nodes_[node].entry == kNone) return false;
  drop(nodes_[node].entry, false);
  return true;
}

bool PrefixCache::evict_lru() {
  std::scoped_lock lock(mutex_);
  if (recency_.empty()) return false;
  drop(recency_.begin()->second, true);
  return true;
}

void PrefixCache::clear() {
  std::scoped_lock lock(mutex_);
  while (!recency_.empty()) drop(recency_.begin()->second, false);
}

PrefixStats PrefixCache::stats() {
  std::scoped_lock lock(mutex_);
  return stats_;
}

}  // namespace helix
