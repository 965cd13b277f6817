// The host-only part of the extern "C" boundary: error strings, the host
// block manager (the reference's PagedKvCache bookkeeping,
// src/kv_cache/paged.cpp) and the prefix cache (src/kv_cache/prefix.cpp) over
// either pool.  No HIP header is included, so this file, block_manager.cpp
// and prefix_cache.cpp also build with a plain C++ compiler under the
// address, undefined-behaviour and thread sanitizers (tests/cpp/Makefile).
#include "abi_common.hpp"

using namespace helix_abi;

std::string& helix_abi::last_error() {
  thread_local std::string message;
  return message;
}

namespace {

void require_manager_handle(const helix::BlockManager& m, helix_sequence s, const char* op) {
  check(s.id != 0 && s.cache_id == m.cache_id(), Status::kInvalidArgument,
        std::string(op) + ": sequence handle belongs to another cache or is empty");
}

// Anchor pool of a prefix cache over the host block manager: every call
// under the manager handle's mutex.
class ManagerAnchors final : public helix::AnchorPool {
public:
  explicit ManagerAnchors(helix_block_manager* m) : m_(m) {}
  std::size_t block_tokens() const override { return m_->manager.config().block_tokens; }
  std::uint64_t cache_id() const override { return m_->manager.cache_id(); }
  std::size_t length(std::uint64_t id, std::uint64_t cache_id) override {
    std::scoped_lock lock(m_->mutex);
    check(id != 0 && cache_id == m_->manager.cache_id(), Status::kInvalidArgument,
          "prefix cache: sequence handle belongs to another cache or is empty");
    return m_->manager.length(id);
  }
  std::uint64_t fork(std::uint64_t id, std::size_t tokens) override {
    std::scoped_lock lock(m_->mutex);
    return m_->manager.commit_fork(m_->manager.plan_fork(id, tokens, false));
  }
  void release(std::uint64_t id) override {
    std::scoped_lock lock(m_->mutex);
    m_->manager.release(id);
  }

private:
  helix_block_manager* m_;
};

}  // namespace

extern "C" {

const char* helix_last_error(void) { return last_error().c_str(); }

const char* helix_status_name(int status) {
  switch (status) {
    case HELIX_OK: return "ok";
    case HELIX_INVALID_ARGUMENT: return "invalid_argument";
    case HELIX_OUT_OF_RANGE: return "out_of_range";
    case HELIX_UNSUPPORTED: return "unsupported";
    case HELIX_RESOURCE_EXHAUSTED: return "resource_exhausted";
    case HELIX_RUNTIME: return "runtime";
    case HELIX_INTERNAL: return "internal";
    default: return "unknown";
  }
}

// --------------------------------------------------------- block manager ----
int helix_block_manager_create(const helix_paged_config* config, helix_block_manager** out) {
  return guarded([&] {
    require_out(out);
    *out = nullptr;
    *out = new helix_block_manager(to_config(config));
  });
}

void helix_block_manager_destroy(helix_block_manager* m) { delete m; }

int helix_block_manager_create_sequence(helix_block_manager* m, helix_sequence* out) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    require_out(out);
    std::scoped_lock lock(m->mutex);
    *out = helix_sequence{m->manager.create_sequence(), m->manager.cache_id()};
  });
}

int helix_block_manager_fork_sequence(helix_block_manager* m, helix_sequence source,
                                      size_t prefix_tokens, int allow_cow, helix_sequence* out,
                                      helix_cow_copy* copy) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    require_out(out);
    std::scoped_lock lock(m->mutex);
    require_manager_handle(m->manager, source, "fork_sequence");
    const helix::ForkPlan plan = m->manager.plan_fork(source.id, prefix_tokens, allow_cow != 0);
    const std::uint64_t id = m->manager.commit_fork(plan);
    *out = helix_sequence{id, m->manager.cache_id()};
    if (copy != nullptr) {
      *copy = helix_cow_copy{plan.cow_from, plan.cow_to,
                             plan.copy_on_write ? plan.cow_tokens : 0};
    }
  });
}

int helix_block_manager_append(helix_block_manager* m, helix_sequence sequence, size_t tokens,
                               uint64_t* slots) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    std::scoped_lock lock(m->mutex);
    require_manager_handle(m->manager, sequence, "append");
    const helix::AppendPlan plan = m->manager.plan_append(sequence.id, tokens);
    if (slots != nullptr) {
      for (std::size_t i = 0; i < tokens; ++i) {
        slots[i] = plan.slot(i, m->manager.config().block_tokens);
      }
    }
    m->manager.commit_append(plan);
  });
}

int helix_block_manager_release_sequence(helix_block_manager* m, helix_sequence sequence) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    std::scoped_lock lock(m->mutex);
    require_manager_handle(m->manager, sequence, "release_sequence");
    m->manager.release(sequence.id);
  });
}

int helix_block_manager_contains(const helix_block_manager* m, helix_sequence sequence,
                                 int* out) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    require_out(out);
    auto* mm = const_cast<helix_block_manager*>(m);
    std::scoped_lock lock(mm->mutex);
    *out = sequence.id != 0 && sequence.cache_id == m->manager.cache_id() &&
           m->manager.contains(sequence.id);
  });
}

int helix_block_manager_length(const helix_block_manager* m, helix_sequence sequence,
                               size_t* out) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    require_out(out);
    auto* mm = const_cast<helix_block_manager*>(m);
    std::scoped_lock lock(mm->mutex);
    require_manager_handle(m->manager, sequence, "length");
    *out = m->manager.length(sequence.id);
  });
}

int helix_block_manager_block_table(const helix_block_manager* m, helix_sequence sequence,
                                    uint32_t* out, size_t capacity, size_t* count) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    require_out(count);
    auto* mm = const_cast<helix_block_manager*>(m);
    std::scoped_lock lock(mm->mutex);
    require_manager_handle(m->manager, sequence, "block_table");
    const auto& blocks = m->manager.blocks(sequence.id);
    *count = blocks.size();
    for (std::size_t i = 0; i < blocks.size() && i < capacity; ++i) out[i] = blocks[i];
  });
}

int helix_block_manager_stats(const helix_block_manager* m, helix_paged_stats* out) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    auto* mm = const_cast<helix_block_manager*>(m);
    std::scoped_lock lock(mm->mutex);
    copy_stats(m->manager.stats(), out);
  });
}

int helix_block_manager_block_info(const helix_block_manager* m, uint32_t block,
                                   size_t* reference_count, size_t* token_count) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    auto* mm = const_cast<helix_block_manager*>(m);
    std::scoped_lock lock(mm->mutex);
    if (reference_count != nullptr) *reference_count = m->manager.block_reference_count(block);
    if (token_count != nullptr) *token_count = m->manager.block_token_count(block);
  });
}

int helix_block_manager_validate(const helix_block_manager* m) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    auto* mm = const_cast<helix_block_manager*>(m);
    std::scoped_lock lock(mm->mutex);
    m->manager.validate();
  });
}

int helix_block_manager_geometry(const helix_block_manager* m, size_t* bytes_per_token,
                                 size_t* block_bytes, size_t* token_capacity) {
  return guarded([&] {
    check(m != nullptr, Status::kInvalidArgument, "manager must not be NULL");
    if (bytes_per_token != nullptr) *bytes_per_token = m->manager.bytes_per_token();
    if (block_bytes != nullptr) *block_bytes = m->manager.block_bytes();
    if (token_capacity != nullptr) *token_capacity = m->manager.token_capacity();
  });
}

// ------------------------------------------------------------ prefix cache

int helix_prefix_cache_create_host(helix_block_manager* manager, const helix_prefix_config* config,
                                   helix_prefix_cache** out) {
  return guarded([&] {
    check(manager != nullptr, Status::kInvalidArgument,
          "prefix cache: paged cache must not be null");
    require_out(out);
    *out = new helix_prefix_cache(std::make_unique<helix::PrefixCache>(
        std::make_unique<ManagerAnchors>(manager), to_prefix_config(config)));
  });
}

void helix_prefix_cache_destroy(helix_prefix_cache* prefixes) { delete prefixes; }

int helix_prefix_cache_insert(helix_prefix_cache* prefixes, uint64_t namespace_id,
                              const uint32_t* tokens, size_t count, helix_sequence source,
                              int* status) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(status);
    *status = static_cast<int>(
        prefixes->index->insert(namespace_id, tokens, count, source.id, source.cache_id));
  });
}

int helix_prefix_cache_lookup_longest(helix_prefix_cache* prefixes, uint64_t namespace_id,
                                      const uint32_t* tokens, size_t count,
                                      size_t maximum_prefix_tokens, int* hit,
                                      helix_sequence* sequence, size_t* matched_tokens) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(hit);
    require_out(sequence);
    require_out(matched_tokens);
    std::uint64_t id = 0;
    std::size_t matched = 0;
    const bool found = prefixes->index->lookup_longest(namespace_id, tokens, count,
                                                       maximum_prefix_tokens, &id, &matched);
    *hit = found ? 1 : 0;
    *sequence = found ? helix_sequence{id, prefixes->index->cache_id()} : helix_sequence{0, 0};
    *matched_tokens = matched;
  });
}

int helix_prefix_cache_contains(helix_prefix_cache* prefixes, uint64_t namespace_id,
                                const uint32_t* tokens, size_t count, int* out) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(out);
    *out = prefixes->index->contains(namespace_id, tokens, count) ? 1 : 0;
  });
}

int helix_prefix_cache_erase(helix_prefix_cache* prefixes, uint64_t namespace_id,
                             const uint32_t* tokens, size_t count, int* erased) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(erased);
    *erased = prefixes->index->erase(namespace_id, tokens, count) ? 1 : 0;
  });
}

int helix_prefix_cache_evict_lru(helix_prefix_cache* prefixes, int* evicted) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(evicted);
    *evicted = prefixes->index->evict_lru() ? 1 : 0;
  });
}

int helix_prefix_cache_clear(helix_prefix_cache* prefixes) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    prefixes->index->clear();
  });
}

int helix_prefix_cache_stats(helix_prefix_cache* prefixes, helix_prefix_stats* out) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(out);
    const helix::PrefixStats s = prefixes->index->stats();
    *out = helix_prefix_stats{s.maximum_entries,       s.maximum_block_references,
                              s.entry_count,           s.retained_tokens,
                              s.retained_block_references, s.peak_entries,
                              s.peak_block_references, s.lookup_count,
                              s.hit_count,             s.miss_count,
                              s.insertion_count,       s.duplicate_insertion_count,
                              s.rejected_insertion_count, s.eviction_count,
                              s.erase_count};
  });
}

int helix_prefix_cache_config(helix_prefix_cache* prefixes, helix_prefix_config* out) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(out);
    const helix::PrefixCacheConfig& c = prefixes->index->config();
    *out = helix_prefix_config{c.maximum_entries, c.maximum_block_references};
  });
}

int helix_prefix_cache_block_tokens(helix_prefix_cache* prefixes, size_t* out) {
  return guarded([&] {
    REQUIRE_PREFIXES();
    require_out(out);
    *out = prefixes->index->block_tokens();
  });
}

}  // extern "C"
