// Pieces of the extern "C" boundary shared by its host-only part
// (host_api.cpp: block manager, host prefix cache, error strings) and its
// device part (c_api.cpp): the handle types both use and the conversion of
// helix::Error into a status code plus a thread-local message.  Nothing here
// includes a HIP header, so the host part builds with a plain C++ compiler
// (and under the sanitizers).
#pragma once

#include "../../include/helix_paged.h"

#include "block_manager.hpp"
#include "prefix_cache.hpp"
#include "status.hpp"

#include <cstdint>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <new>
#include <string>

struct helix_block_manager {
  explicit helix_block_manager(const helix::PagedConfig& c) : manager(c) {}
  helix::BlockManager manager;
  std::mutex mutex;
};

struct helix_prefix_cache {
  explicit helix_prefix_cache(std::unique_ptr<helix::PrefixCache> p) : index(std::move(p)) {}
  std::unique_ptr<helix::PrefixCache> index;
};

namespace helix_abi {

using helix::Error;
using helix::Status;
using helix::check;

// Message of the calling thread's last failed call (host_api.cpp).
std::string& last_error();

template <typename F>
int guarded(F&& body) {
  try {
    body();
    last_error().clear();
    return HELIX_OK;
  } catch (const Error& e) {
    last_error() = e.what();
    return static_cast<int>(e.status());
  } catch (const std::bad_alloc&) {
    last_error() = "host allocation failed";
    return HELIX_RESOURCE_EXHAUSTED;
  } catch (const std::exception& e) {
    last_error() = e.what();
    return HELIX_INTERNAL;
  } catch (...) {
    last_error() = "unknown exception";
    return HELIX_INTERNAL;
  }
}

inline helix::PagedConfig to_config(const helix_paged_config* c) {
  check(c != nullptr, Status::kInvalidArgument, "config must not be NULL");
  return helix::PagedConfig{c->layers, c->kv_heads, c->head_dimension, c->block_tokens,
                            c->physical_blocks};
}

inline void copy_stats(const helix::PagedStats& s, helix_paged_stats* out) {
  check(out != nullptr, Status::kInvalidArgument, "stats output must not be NULL");
  static_assert(sizeof(helix::PagedStats) == sizeof(helix_paged_stats), "stats layout");
  std::memcpy(out, &s, sizeof(s));
}

inline void require_out(const void* p) {
  check(p != nullptr, Status::kInvalidArgument, "output pointer must not be NULL");
}

inline bool overlap(const void* a, std::size_t an, const void* b, std::size_t bn) {
  if (a == nullptr || b == nullptr || an == 0 || bn == 0) return false;
  const auto x = reinterpret_cast<std::uintptr_t>(a);
  const auto y = reinterpret_cast<std::uintptr_t>(b);
  return x < y + bn && y < x + an;
}

inline std::size_t mul(std::size_t a, std::size_t b) {
  check(a == 0 || b <= std::numeric_limits<std::size_t>::max() / a, Status::kOutOfRange,
        "size computation overflows");
  return a * b;
}

inline helix::PrefixCacheConfig to_prefix_config(const helix_prefix_config* c) {
  check(c != nullptr, Status::kInvalidArgument, "prefix cache config must not be NULL");
  return helix::PrefixCacheConfig{c->maximum_entries, c->maximum_block_references};
}

}  // namespace helix_abi

#define REQUIRE_PREFIXES() \
  check(prefixes != nullptr, Status::kInvalidArgument, "prefix cache must not be NULL")
