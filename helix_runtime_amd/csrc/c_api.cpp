// extern "C" boundary (device part; the host-only part is host_api.cpp):
// converts helix::Error (and any other exception) into a
// status code plus a thread-local message; nothing throws across it.
#include "abi_common.hpp"

#include "block_manager.hpp"
#include "kernels.hpp"
#include "paged_cache.hpp"
#include "prefix_cache.hpp"
#include "status.hpp"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <map>
#include <mutex>
#include <tuple>
#include <cstring>
#include <limits>
#include <memory>
#include <new>
#include <string>
#include <vector>

using namespace helix_abi;

struct helix_paged_cache {
  helix_paged_cache(const helix::PagedConfig& c, int device,
                    helix::hip::PageFormat type = helix::hip::PageFormat())
      : cache(c, device, type) {}
  helix::DevicePagedCache cache;
};

struct helix_decode_view {
  helix_decode_view(std::shared_ptr<helix::CacheState> s, std::uint64_t id, std::uint64_t cid)
      : view(std::move(s), id, cid) {}
  helix::DecodeView view;
};

struct helix_block_table {
  helix::DeviceBuffer buffer;
  std::size_t logical = 0;
  std::size_t physical = 0;
  int device = -1;
};

struct helix_decode_batch {
  std::unique_ptr<helix::DecodeBatch> batch;
};

namespace {

hipStream_t as_stream(helix_stream s) { return static_cast<hipStream_t>(s); }

// ------------------------------------------------ attention validation ----
// validate_query_key_and_table / validate_value_blocks / validate_offset of
// src/attention/cuda_paged.cu:211-335.
struct AttentionShape {
  std::size_t q_heads, queries, key_dim, physical, kv_heads, block_tokens, value_dim;
  std::size_t logical, history, tail, keys, offset;
};

void validate_attention(const AttentionShape& s, bool allow_empty_history, const char* op) {
  const std::string o(op);
  check(s.physical > 0 && s.kv_heads > 0 && s.block_tokens > 0 && s.key_dim > 0,
        Status::kInvalidArgument,
        o + ": physical block, head, token, and key dimensions must be positive");
  check(s.value_dim > 0, Status::kInvalidArgument, o + ": value dimension must be positive");
  check(s.q_heads > 0 && s.q_heads % s.kv_heads == 0, Status::kInvalidArgument,
        o + ": query heads must be a positive multiple of the key/value heads");
  check(s.physical <= std::numeric_limits<std::uint32_t>::max(), Status::kInvalidArgument,
        o + ": physical block capacity must fit the uint32 block-ID representation");
  check(allow_empty_history || s.history != 0, Status::kInvalidArgument,
        o + ": KV token count must be positive");
  const std::size_t required = s.history == 0 ? 0 : 1 + (s.history - 1) / s.block_tokens;
  check(s.logical == required, Status::kInvalidArgument,
        o + ": block table length must exactly cover the logical KV token range");
  check(s.offset <= s.keys, Status::kInvalidArgument,
        o + ": query position offset exceeds the KV token count");
  check(s.queries <= s.keys - s.offset, Status::kInvalidArgument,
        o + ": query range extends beyond the KV token count");
  check(s.value_dim <= 1024, Status::kUnsupported, o + ": value dimension above 1024");
}

// Anchor pool of a prefix cache over the device cache: its state under the
// cache mutex (block-aligned forks need no page copy).
class DeviceAnchors final : public helix::AnchorPool {
public:
  explicit DeviceAnchors(std::shared_ptr<helix::CacheState> s) : s_(std::move(s)) {}
  std::size_t block_tokens() const override { return s_->manager.config().block_tokens; }
  std::uint64_t cache_id() const override { return s_->manager.cache_id(); }
  std::size_t length(std::uint64_t id, std::uint64_t cache_id) override {
    std::scoped_lock lock(s_->mutex);
    s_->require_sequence(id, cache_id, "prefix cache insert");
    return s_->manager.length(id);
  }
  std::uint64_t fork(std::uint64_t id, std::size_t tokens) override {
    std::scoped_lock lock(s_->mutex);
    s_->require_healthy("prefix cache fork");
    return s_->manager.commit_fork(s_->manager.plan_fork(id, tokens, false));
  }
  void release(std::uint64_t id) override {
    std::scoped_lock lock(s_->mutex);
    s_->manager.release(id);
  }

private:
  std::shared_ptr<helix::CacheState> s_;
};

}  // namespace

extern "C" {

// ----------------------------------------------------------- device cache ----
int helix_paged_cache_create(const helix_paged_config* config, int device,
                             helix_paged_cache** out) {
  return guarded([&] {
    require_out(out);
    *out = nullptr;
    *out = new helix_paged_cache(to_config(config), device);
  });
}

int helix_paged_cache_create_typed(const helix_paged_config* config, int device, int page_dtype,
                                   helix_paged_cache** out) {
  return guarded([&] {
    require_out(out);
    *out = nullptr;
    check(page_dtype == HELIX_PAGE_F32 || page_dtype == HELIX_PAGE_BF16 ||
              page_dtype == HELIX_PAGE_FP8_E4M3,
          Status::kInvalidArgument,
          "page dtype must be HELIX_PAGE_F32, HELIX_PAGE_BF16 or HELIX_PAGE_FP8_E4M3");
    *out = new helix_paged_cache(to_config(config), device,
                                 static_cast<helix::hip::PageType>(page_dtype));
  });
}

int helix_paged_cache_create_fp8(const helix_paged_config* config, int device, float key_scale,
                                 float value_scale, helix_paged_cache** out) {
  return guarded([&] {
    require_out(out);
    *out = nullptr;
    check(std::isfinite(key_scale) && key_scale > 0.0f && std::isfinite(value_scale) &&
              value_scale > 0.0f,
          Status::kInvalidArgument, "fp8 page scales must be finite and positive");
    *out = new helix_paged_cache(
        to_config(config), device,
        helix::hip::PageFormat(helix::hip::PageType::kFP8, key_scale, value_scale));
  });
}

void helix_paged_cache_destroy(helix_paged_cache* cache) { delete cache; }

#define REQUIRE_CACHE() check(cache != nullptr, Status::kInvalidArgument, "cache must not be NULL")

int helix_paged_cache_page_dtype(helix_paged_cache* cache, int* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    *out = static_cast<int>(cache->cache.state()->page_type.type);
  });
}

int helix_paged_cache_fp8_scales(helix_paged_cache* cache, float* key_scale, float* value_scale) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(key_scale);
    require_out(value_scale);
    *key_scale = cache->cache.state()->page_type.k_scale;
    *value_scale = cache->cache.state()->page_type.v_scale;
  });
}

int helix_paged_cache_create_sequence(helix_paged_cache* cache, helix_sequence* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    *out = helix_sequence{cache->cache.create_sequence(), cache->cache.cache_id()};
  });
}

int helix_paged_cache_fork_sequence(helix_paged_cache* cache, helix_sequence source,
                                    size_t prefix_tokens, int allow_cow, helix_stream stream,
                                    helix_sequence* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    const std::uint64_t id = cache->cache.fork_sequence(source.id, source.cache_id, prefix_tokens,
                                                        allow_cow != 0, as_stream(stream));
    *out = helix_sequence{id, cache->cache.cache_id()};
  });
}

int helix_paged_cache_append(helix_paged_cache* cache, helix_sequence sequence,
                             const float* token_keys, const float* token_values,
                             helix_stream stream) {
  return guarded([&] {
    REQUIRE_CACHE();
    cache->cache.append(sequence.id, sequence.cache_id, token_keys, token_values,
                        as_stream(stream));
  });
}

int helix_paged_cache_append_layer_major(helix_paged_cache* cache, helix_sequence sequence,
                                         const float* const* layer_keys,
                                         const float* const* layer_values, size_t tokens,
                                         helix_stream stream) {
  return guarded([&] {
    REQUIRE_CACHE();
    cache->cache.append_layer_major(sequence.id, sequence.cache_id, layer_keys, layer_values,
                                    tokens, as_stream(stream));
  });
}

int helix_paged_cache_release_sequence(helix_paged_cache* cache, helix_sequence sequence) {
  return guarded([&] {
    REQUIRE_CACHE();
    cache->cache.release(sequence.id, sequence.cache_id);
  });
}

int helix_paged_cache_copy_layer_out(helix_paged_cache* cache, helix_sequence sequence,
                                     size_t layer, float* keys_out, float* values_out,
                                     helix_stream stream) {
  return guarded([&] {
    REQUIRE_CACHE();
    std::size_t length = 0;
    {
      auto& s = *cache->cache.state();
      std::scoped_lock lock(s.mutex);
      s.require_sequence(sequence.id, sequence.cache_id, "copy_layer_out");
      length = s.manager.length(sequence.id);
    }
    cache->cache.copy_layer_out(sequence.id, sequence.cache_id, layer, length, keys_out,
                                values_out, length, as_stream(stream));
  });
}

int helix_paged_cache_copy_layer_prefix_out(helix_paged_cache* cache, helix_sequence sequence,
                                            size_t layer, size_t expected_length,
                                            float* keys_out, float* values_out,
                                            size_t dest_tokens, helix_stream stream) {
  return guarded([&] {
    REQUIRE_CACHE();
    cache->cache.copy_layer_out(sequence.id, sequence.cache_id, layer, expected_length, keys_out,
                                values_out, dest_tokens, as_stream(stream));
  });
}

int helix_paged_cache_contains(helix_paged_cache* cache, helix_sequence sequence, int* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    auto& s = *cache->cache.state();
    std::scoped_lock lock(s.mutex);
    *out = sequence.id != 0 && sequence.cache_id == s.manager.cache_id() &&
           s.manager.contains(sequence.id);
  });
}

int helix_paged_cache_length(helix_paged_cache* cache, helix_sequence sequence, size_t* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    auto& s = *cache->cache.state();
    std::scoped_lock lock(s.mutex);
    s.require_sequence(sequence.id, sequence.cache_id, "length");
    *out = s.manager.length(sequence.id);
  });
}

int helix_paged_cache_block_table(helix_paged_cache* cache, helix_sequence sequence,
                                  uint32_t* out, size_t capacity, size_t* count) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(count);
    auto& s = *cache->cache.state();
    std::scoped_lock lock(s.mutex);
    s.require_sequence(sequence.id, sequence.cache_id, "block_table");
    const auto& blocks = s.manager.blocks(sequence.id);
    *count = blocks.size();
    for (std::size_t i = 0; i < blocks.size() && i < capacity; ++i) out[i] = blocks[i];
  });
}

int helix_paged_cache_stats(helix_paged_cache* cache, helix_paged_stats* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    auto& s = *cache->cache.state();
    std::scoped_lock lock(s.mutex);
    copy_stats(s.manager.stats(), out);
  });
}

int helix_paged_cache_is_healthy(helix_paged_cache* cache, int* out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    auto& s = *cache->cache.state();
    std::scoped_lock lock(s.mutex);
    *out = !s.poisoned;
  });
}

int helix_paged_cache_geometry(helix_paged_cache* cache, size_t* bytes_per_token,
                               size_t* block_bytes, size_t* token_capacity) {
  return guarded([&] {
    REQUIRE_CACHE();
    const auto& m = cache->cache.state()->manager;
    if (bytes_per_token != nullptr) *bytes_per_token = m.bytes_per_token();
    if (block_bytes != nullptr) *block_bytes = m.block_bytes();
    if (token_capacity != nullptr) *token_capacity = m.token_capacity();
  });
}

int helix_paged_cache_layer_pools(helix_paged_cache* cache, size_t layer, float** key_blocks,
                                  float** value_blocks) {
  return guarded([&] {
    REQUIRE_CACHE();
    const auto& s = *cache->cache.state();
    check(layer < s.manager.config().layers, Status::kOutOfRange, "layer index is out of range");
    if (key_blocks != nullptr) *key_blocks = s.key_pool(layer);
    if (value_blocks != nullptr) *value_blocks = s.value_pool(layer);
  });
}

int helix_paged_cache_read_sequence(helix_paged_cache* cache, helix_sequence sequence,
                                    helix_decode_view** out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    *out = nullptr;
    *out = new helix_decode_view(cache->cache.state(), sequence.id, sequence.cache_id);
  });
}

int helix_decode_view_length(const helix_decode_view* view, size_t* out) {
  return guarded([&] {
    check(view != nullptr, Status::kInvalidArgument, "view must not be NULL");
    require_out(out);
    *out = view->view.length();
  });
}

int helix_decode_view_physical_blocks(const helix_decode_view* view, const uint32_t** blocks,
                                      size_t* count) {
  return guarded([&] {
    check(view != nullptr, Status::kInvalidArgument, "view must not be NULL");
    require_out(blocks);
    require_out(count);
    const auto& b = view->view.physical_blocks();
    *blocks = b.data();
    *count = b.size();
  });
}

int helix_decode_view_block_table(const helix_decode_view* view, const uint32_t** device_table) {
  return guarded([&] {
    check(view != nullptr, Status::kInvalidArgument, "view must not be NULL");
    require_out(device_table);
    *device_table = view->view.device_table();
  });
}

int helix_decode_view_layer_pools(const helix_decode_view* view, size_t layer,
                                  float** key_blocks, float** value_blocks) {
  return guarded([&] {
    check(view != nullptr, Status::kInvalidArgument, "view must not be NULL");
    if (key_blocks != nullptr) *key_blocks = view->view.key_pool(layer);
    if (value_blocks != nullptr) *value_blocks = view->view.value_pool(layer);
  });
}

void helix_decode_view_poison(helix_decode_view* view) {
  if (view != nullptr) view->view.poison();
}

void helix_decode_view_release(helix_decode_view* view) { delete view; }

// ------------------------------------------------------------ block table ----
int helix_block_table_create(const uint32_t* physical_blocks, size_t count,
                             size_t physical_block_count, int device, helix_block_table** out) {
  return guarded([&] {
    require_out(out);
    *out = nullptr;
    check(physical_block_count != 0 &&
              physical_block_count <= std::numeric_limits<std::uint32_t>::max(),
          Status::kInvalidArgument,
          "PagedBlockTable: physical block capacity must fit the uint32 block-ID representation");
    check(device >= 0, Status::kInvalidArgument, "PagedBlockTable: device index must be non-negative");
    check(count == 0 || physical_blocks != nullptr, Status::kInvalidArgument,
          "PagedBlockTable: IDs must not be NULL");
    for (std::size_t i = 0; i < count; ++i) {
      check(physical_blocks[i] < physical_block_count, Status::kOutOfRange,
            "PagedBlockTable: physical block ID exceeds the packed block capacity");
    }
    auto table = std::make_unique<helix_block_table>();
    table->logical = count;
    table->physical = physical_block_count;
    table->device = device;
    if (count != 0) {
      table->buffer = helix::DeviceBuffer(count * sizeof(std::uint32_t), device);
      helix::DeviceGuard guard(device);
      helix::hip_check(hipMemcpy(table->buffer.data(), physical_blocks,
                                 count * sizeof(std::uint32_t), hipMemcpyHostToDevice),
                       "PagedBlockTable upload");
    }
    *out = table.release();
  });
}

const uint32_t* helix_block_table_data(const helix_block_table* table) {
  return table == nullptr ? nullptr : static_cast<const uint32_t*>(table->buffer.data());
}

size_t helix_block_table_logical_block_count(const helix_block_table* table) {
  return table == nullptr ? 0 : table->logical;
}

void helix_block_table_destroy(helix_block_table* table) { delete table; }

// -------------------------------------------- reference-shaped attention ----
int helix_paged_score_workspace_bytes(size_t q_heads, size_t queries, size_t kv_heads,
                                      size_t physical_blocks, size_t block_tokens,
                                      size_t logical_blocks, size_t kv_tokens, size_t* out) {
  return guarded([&] {
    require_out(out);
    AttentionShape s{q_heads, queries, 1,  physical_blocks, kv_heads, block_tokens, 1,
                     logical_blocks, kv_tokens, 0, kv_tokens, 0};
    validate_attention(s, false, "paged_score_workspace_bytes");
    *out = mul(mul(mul(q_heads, queries), kv_tokens), sizeof(float));
  });
}

int helix_paged_tail_score_workspace_bytes(size_t q_heads, size_t tail_tokens, size_t kv_heads,
                                           size_t physical_blocks, size_t block_tokens,
                                           size_t logical_blocks, size_t history_tokens,
                                           size_t* out) {
  return guarded([&] {
    require_out(out);
    check(tail_tokens != 0, Status::kInvalidArgument,
          "paged_tail_score_workspace_bytes: tail token count must be positive");
    check(history_tokens <= std::numeric_limits<std::int64_t>::max() - tail_tokens,
          Status::kResourceExhausted,
          "paged_tail_score_workspace_bytes: history plus tail token count overflows shape range");
    AttentionShape s{q_heads, tail_tokens, 1, physical_blocks, kv_heads, block_tokens, 1,
                     logical_blocks, history_tokens, tail_tokens, history_tokens + tail_tokens,
                     history_tokens};
    validate_attention(s, true, "paged_tail_score_workspace_bytes");
    *out = mul(mul(mul(q_heads, tail_tokens), history_tokens + tail_tokens), sizeof(float));
  });
}

namespace {

// Validates the caller's buffers (workspace shape, non-null pointers, no
// aliasing) as cuda_paged.cu:211-352 does; false when there is nothing to
// compute.
bool validate_reference_buffers(const AttentionShape& s, const float* query,
                                const float* key_blocks, const float* value_blocks,
                                const std::uint32_t* block_table, const float* tail_key,
                                const float* tail_value, const float* output,
                                const float* workspace, std::size_t workspace_elements,
                                const char* op) {
  const std::string o(op);
  const std::size_t ws = mul(mul(s.q_heads, s.queries), s.keys);
  check(workspace_elements == ws, Status::kInvalidArgument,
        o + ": score workspace shape does not match [heads, queries, kv tokens]");
  if (s.queries == 0) return false;
  check(query != nullptr && output != nullptr && workspace != nullptr, Status::kInvalidArgument,
        o + ": query, output and workspace must be non-null device pointers");
  check(s.history == 0 || (key_blocks != nullptr && value_blocks != nullptr &&
                           block_table != nullptr),
        Status::kInvalidArgument, o + ": key/value blocks and block table must be non-null");
  check(s.tail == 0 || (tail_key != nullptr && tail_value != nullptr), Status::kInvalidArgument,
        o + ": tail key and value must be non-null");
  const std::size_t qb = mul(ws / s.keys, s.key_dim) * sizeof(float);
  const std::size_t ob = mul(ws / s.keys, s.value_dim) * sizeof(float);
  const std::size_t wb = ws * sizeof(float);
  const std::size_t page = mul(s.physical, mul(s.kv_heads, s.block_tokens));
  const std::size_t kb = mul(page, s.key_dim) * sizeof(float);
  const std::size_t vb = mul(page, s.value_dim) * sizeof(float);
  const std::size_t tkb = mul(mul(s.kv_heads, s.tail), s.key_dim) * sizeof(float);
  const std::size_t tvb = mul(mul(s.kv_heads, s.tail), s.value_dim) * sizeof(float);
  check(!overlap(query, qb, output, ob), Status::kInvalidArgument, o + ": output must not alias query");
  check(!overlap(key_blocks, kb, output, ob), Status::kInvalidArgument,
        o + ": output must not alias key blocks");
  check(!overlap(value_blocks, vb, output, ob), Status::kInvalidArgument,
        o + ": output must not alias value blocks");
  check(!overlap(tail_key, tkb, output, ob), Status::kInvalidArgument,
        o + ": output must not alias tail key");
  check(!overlap(tail_value, tvb, output, ob), Status::kInvalidArgument,
        o + ": output must not alias tail value");
  check(!overlap(query, qb, workspace, wb), Status::kInvalidArgument,
        o + ": score workspace must not alias query");
  check(!overlap(key_blocks, kb, workspace, wb), Status::kInvalidArgument,
        o + ": score workspace must not alias key blocks");
  check(!overlap(value_blocks, vb, workspace, wb), Status::kInvalidArgument,
        o + ": score workspace must not alias value blocks");
  check(!overlap(tail_key, tkb, workspace, wb), Status::kInvalidArgument,
        o + ": score workspace must not alias tail key");
  check(!overlap(tail_value, tvb, workspace, wb), Status::kInvalidArgument,
        o + ": score workspace must not alias tail value");
  check(!overlap(workspace, wb, output, ob), Status::kInvalidArgument,
        o + ": output must not alias score workspace");
  return true;
}

void run_reference_attention(const AttentionShape& s, const float* query,
                             const float* key_blocks, const float* value_blocks,
                             const std::uint32_t* block_table, const float* tail_key,
                             const float* tail_value, float* output, float* workspace,
                             std::size_t workspace_elements, hipStream_t stream, const char* op) {
  if (!validate_reference_buffers(s, query, key_blocks, value_blocks, block_table, tail_key,
                                  tail_value, output, workspace, workspace_elements, op)) {
    return;
  }
  helix::hip::GenericArgs a{};
  a.query = query;
  a.key_blocks = key_blocks;
  a.value_blocks = value_blocks;
  a.table = block_table;
  a.tail_key = tail_key;
  a.tail_value = tail_value;
  a.out = output;
  a.workspace = workspace;
  a.q_heads = s.q_heads;
  a.kv_heads = s.kv_heads;
  a.queries = s.queries;
  a.key_dim = s.key_dim;
  a.value_dim = s.value_dim;
  a.block_tokens = s.block_tokens;
  a.physical_blocks = s.physical;
  a.history = s.history;
  a.tail = s.tail;
  a.offset = s.offset;
  helix::hip_check(helix::hip::launch_generic(a, stream), (std::string(op) + " launch").c_str());
}

// Device scratch of the reference-shaped fast routes, one buffer per
// (device, stream, purpose): calls on one stream run in order and may share
// it, calls on different streams get their own.  It grows on demand (the
// old buffer is freed once the stream has drained).  Buffers live until the
// process ends.  Host threads that issue calls on one stream must order
// those calls themselves, as they must for the stream's work anyway.
enum class ScratchUse : int { kDecode = 0, kChunk = 1, kRowStats = 2 };
void* route_scratch(std::size_t bytes, hipStream_t stream, ScratchUse use) {
  struct Buffer {
    void* ptr = nullptr;
    std::size_t bytes = 0;
  };
  static std::mutex mutex;
  static std::map<std::tuple<int, void*, int>, Buffer> buffers;
  int device = 0;
  helix::hip_check(hipGetDevice(&device), "route scratch: hipGetDevice");
  std::scoped_lock lock(mutex);
  Buffer& b = buffers[{device, static_cast<void*>(stream), static_cast<int>(use)}];
  if (b.bytes < bytes) {
    const std::size_t grown = std::max(bytes, 2 * b.bytes);
    if (b.ptr != nullptr) {
      // Earlier calls on this stream may still read the old buffer.
      helix::hip_check(hipStreamSynchronize(stream), "route scratch: hipStreamSynchronize");
      helix::hip_check(hipFree(b.ptr), "route scratch: hipFree");
      b = Buffer{};
    }
    void* p = nullptr;
    if (hipMalloc(&p, grown) != hipSuccess) {
      (void)hipGetLastError();
      fail(Status::kResourceExhausted, "route scratch: device allocation failed");
    }
    b = Buffer{p, grown};
  }
  return b.ptr;
}

bool aligned16p(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// The reference-shaped call with one query row on the single-sequence decode
// kernel: head_dim 128, 16-token pages, a supported query group and 16-byte
// aligned rows.  The score workspace ends up holding the probabilities, as
// on the reference's own path.  `visible` page tokens, then (tail) the tail
// row.  Returns false (nothing launched) when the call does not qualify.
bool try_ref_decode(const AttentionShape& s, const float* query, const float* key_blocks,
                    const float* value_blocks, const std::uint32_t* block_table,
                    const float* tail_key, const float* tail_value, float* output,
                    float* workspace, std::size_t visible, bool tail, hipStream_t stream,
                    const char* op) {
  namespace hh = helix::hip;
  if (s.queries != 1 || s.key_dim != hh::kDecodeHeadDim || s.value_dim != hh::kDecodeHeadDim ||
      s.block_tokens != hh::kDecodeBlockTokens || s.kv_heads == 0 ||
      s.q_heads % s.kv_heads != 0 || !hh::decode_group_supported(s.q_heads / s.kv_heads) ||
      s.keys > hh::kRefDecodeMaxKeys) {
    return false;
  }
  if (!aligned16p(query) || !aligned16p(output) || (visible > 0 && (!aligned16p(key_blocks) ||
                                                                   !aligned16p(value_blocks))) ||
      (tail && (!aligned16p(tail_key) || !aligned16p(tail_value)))) {
    return false;
  }
  const hh::RefDecodePlan plan = hh::ref_decode_plan(s.q_heads, s.kv_heads, visible, tail);
  hh::RefDecodeArgs a{};
  a.query = query;
  a.key_pool = key_blocks;
  a.value_pool = value_blocks;
  a.table = block_table;
  a.tail_key = tail ? tail_key : nullptr;
  a.tail_value = tail ? tail_value : nullptr;
  a.out = output;
  a.probs = workspace;
  a.q_heads = s.q_heads;
  a.kv_heads = s.kv_heads;
  a.physical_blocks = s.physical;
  a.visible = visible;
  a.keys = s.keys;
  a.tail = tail;
  a.scratch = route_scratch(plan.scratch_bytes, stream, ScratchUse::kDecode);
  helix::hip_check(hh::launch_ref_decode(a, plan, stream), (std::string(op) + " launch").c_str());
  return true;
}

// Whether a reference-shaped call with several query rows (a prefill
// chunk) fits the exact matrix-core prefill kernel: head_dim 128, 16-token
// pages, a supported query group, 16-byte aligned rows and index ranges the
// kernel's 32-bit arithmetic holds.
bool ref_prefill_fits(const AttentionShape& s, const float* query, const float* output,
                      const float* key_blocks, const float* value_blocks, std::size_t history,
                      std::size_t prob_keys) {
  namespace hh = helix::hip;
  constexpr auto kIntMax = static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max());
  return s.queries >= 2 && s.key_dim == hh::kDecodeHeadDim &&
         s.value_dim == hh::kDecodeHeadDim && s.block_tokens == hh::kDecodeBlockTokens &&
         s.kv_heads != 0 && s.q_heads % s.kv_heads == 0 &&
         hh::prefill_group_supported(s.q_heads / s.kv_heads) &&
         prob_keys <= hh::kRefDecodeMaxKeys &&
         s.queries * s.kv_heads <= kIntMax && aligned16p(query) && aligned16p(output) &&
         (history == 0 || (aligned16p(key_blocks) && aligned16p(value_blocks)));
}

// Such a call on that kernel, which also leaves the probabilities in the
// workspace: query row q sees the `history` page tokens and chunk rows
// 0..q; workspace rows are `prob_keys` long.
void run_ref_prefill(const AttentionShape& s, const float* query, const float* key_blocks,
                     const float* value_blocks, const std::uint32_t* block_table,
                     const float* chunk_key, const float* chunk_value, float* output,
                     float* workspace, std::size_t history, std::size_t prob_keys,
                     hipStream_t stream, const char* op) {
  namespace hh = helix::hip;
  hh::PrefillArgs a{};
  a.query = query;
  a.key_pool = key_blocks;
  a.value_pool = value_blocks;
  a.tables = block_table;
  a.lengths = nullptr;
  a.single_length = static_cast<std::int32_t>(history);
  a.chunk_key = chunk_key;
  a.chunk_value = chunk_value;
  a.out = output;
  a.batch = 1;
  a.q_heads = s.q_heads;
  a.kv_heads = s.kv_heads;
  a.tokens = s.queries;
  a.max_blocks = (history + hh::kDecodeBlockTokens - 1) / hh::kDecodeBlockTokens;
  a.physical_blocks = s.physical;
  a.probs = workspace;
  a.prob_keys = prob_keys;
  a.prob_splits = hh::prefill_prob_splits(s.q_heads, s.kv_heads, s.queries, history + s.queries,
                                          hh::device_cus());
  const std::size_t slots = mul(mul(s.q_heads, s.queries), a.prob_splits);
  const std::size_t ml_floats = (slots * 2 + 63) / 64 * 64;  // keeps prob_o 256-byte aligned
  auto* stats = static_cast<float*>(route_scratch(
      mul(ml_floats + mul(slots, hh::kDecodeHeadDim), sizeof(float)), stream,
      ScratchUse::kRowStats));
  a.prob_ml = stats;
  a.prob_o = stats + ml_floats;
  helix::hip_check(hh::launch_prefill(a, stream), (std::string(op) + " launch").c_str());
}

// _with_tail_out with several tail rows: the tail is the chunk.
bool try_ref_prefill(const AttentionShape& s, const float* query, const float* key_blocks,
                     const float* value_blocks, const std::uint32_t* block_table,
                     const float* tail_key, const float* tail_value, float* output,
                     float* workspace, hipStream_t stream, const char* op) {
  if (!ref_prefill_fits(s, query, output, key_blocks, value_blocks, s.history, s.keys) ||
      !aligned16p(tail_key) || !aligned16p(tail_value)) {
    return false;
  }
  run_ref_prefill(s, query, key_blocks, value_blocks, block_table, tail_key, tail_value, output,
                  workspace, s.history, s.keys, stream, op);
  return true;
}

// _out with several query rows: page rows [offset, offset + queries) are
// gathered into this stream's scratch as the chunk (history = offset).
bool try_ref_history_prefill(const AttentionShape& s, const float* query,
                             const float* key_blocks, const float* value_blocks,
                             const std::uint32_t* block_table, float* output, float* workspace,
                             hipStream_t stream, const char* op) {
  namespace hh = helix::hip;
  if (!ref_prefill_fits(s, query, output, key_blocks, value_blocks, s.offset, s.keys) ||
      !aligned16p(key_blocks) || !aligned16p(value_blocks)) {
    return false;
  }
  const std::size_t rows = mul(mul(s.kv_heads, s.queries), hh::kDecodeHeadDim);
  auto* chunk = static_cast<float*>(
      route_scratch(mul(rows, 2 * sizeof(float)), stream, ScratchUse::kChunk));
  const hh::PageGeometry g{s.physical, s.kv_heads, s.block_tokens, s.key_dim};
  helix::hip_check(hh::launch_gather(key_blocks, value_blocks, g, block_table, s.queries, chunk,
                                     chunk + rows, s.queries, stream, hh::PageFormat(),
                                     s.offset),
                   (std::string(op) + " gather").c_str());
  run_ref_prefill(s, query, key_blocks, value_blocks, block_table, chunk, chunk + rows, output,
                  workspace, s.offset, s.keys, stream, op);
  return true;
}

}  // namespace

int helix_paged_attention_out(const float* query, size_t q_heads, size_t queries, size_t key_dim,
                              const float* key_blocks, const float* value_blocks,
                              size_t physical_blocks, size_t kv_heads, size_t block_tokens,
                              size_t value_dim, const uint32_t* block_table,
                              size_t logical_blocks, size_t kv_tokens,
                              size_t query_position_offset, float* output,
                              float* score_workspace, size_t workspace_elements,
                              helix_stream stream) {
  return guarded([&] {
    constexpr const char* op = "paged_scaled_dot_product_attention_out";
    AttentionShape s{q_heads, queries, key_dim, physical_blocks, kv_heads, block_tokens,
                     value_dim, logical_blocks, kv_tokens, 0, kv_tokens, query_position_offset};
    validate_attention(s, false, op);
    if (!validate_reference_buffers(s, query, key_blocks, value_blocks, block_table, nullptr,
                                    nullptr, output, score_workspace, workspace_elements, op)) {
      return;
    }
    if (try_ref_decode(s, query, key_blocks, value_blocks, block_table, nullptr, nullptr, output,
                       score_workspace, query_position_offset + 1, false, as_stream(stream),
                       op) ||
        try_ref_history_prefill(s, query, key_blocks, value_blocks, block_table, output,
                                score_workspace, as_stream(stream), op)) {
      return;
    }
    run_reference_attention(s, query, key_blocks, value_blocks, block_table, nullptr, nullptr,
                            output, score_workspace, workspace_elements, as_stream(stream), op);
  });
}

namespace {

void attention_with_tail(const float* query, size_t q_heads, size_t tail_tokens, size_t key_dim,
                         const float* key_blocks, const float* value_blocks,
                         size_t physical_blocks, size_t kv_heads, size_t block_tokens,
                         size_t value_dim, const uint32_t* block_table, size_t logical_blocks,
                         size_t history_tokens, const float* tail_key, const float* tail_value,
                         float* output, float* score_workspace, size_t workspace_elements,
                         helix_stream stream, bool probabilities, const char* op) {
  check(tail_tokens != 0, Status::kInvalidArgument,
        std::string(op) + ": tail token count must be positive");
  check(history_tokens <= std::numeric_limits<std::int64_t>::max() - tail_tokens,
        Status::kResourceExhausted,
        std::string(op) + ": history plus tail token count overflows shape range");
  AttentionShape s{q_heads, tail_tokens, key_dim, physical_blocks, kv_heads, block_tokens,
                   value_dim, logical_blocks, history_tokens, tail_tokens,
                   history_tokens + tail_tokens, history_tokens};
  validate_attention(s, true, op);
  if (!probabilities) {
    if (!validate_reference_buffers(s, query, key_blocks, value_blocks, block_table, tail_key,
                                    tail_value, output, score_workspace, workspace_elements, op)) {
      return;
    }
    if (try_ref_decode(s, query, key_blocks, value_blocks, block_table, tail_key, tail_value,
                       output, score_workspace, history_tokens, true, as_stream(stream), op) ||
        try_ref_prefill(s, query, key_blocks, value_blocks, block_table, tail_key, tail_value,
                        output, score_workspace, as_stream(stream), op)) {
      return;
    }
  }
  run_reference_attention(s, query, key_blocks, value_blocks, block_table, tail_key, tail_value,
                          output, score_workspace, workspace_elements, as_stream(stream), op);
}

}  // namespace

int helix_paged_attention_with_tail_out(const float* query, size_t q_heads, size_t tail_tokens,
                                        size_t key_dim, const float* key_blocks,
                                        const float* value_blocks, size_t physical_blocks,
                                        size_t kv_heads, size_t block_tokens, size_t value_dim,
                                        const uint32_t* block_table, size_t logical_blocks,
                                        size_t history_tokens, const float* tail_key,
                                        const float* tail_value, float* output,
                                        float* score_workspace, size_t workspace_elements,
                                        helix_stream stream) {
  return guarded([&] {
    attention_with_tail(query, q_heads, tail_tokens, key_dim, key_blocks, value_blocks,
                        physical_blocks, kv_heads, block_tokens, value_dim, block_table,
                        logical_blocks, history_tokens, tail_key, tail_value, output,
                        score_workspace, workspace_elements, stream, false,
                        "paged_scaled_dot_product_attention_with_tail_out");
  });
}

int helix_paged_attention_with_tail_probabilities_out(
    const float* query, size_t q_heads, size_t tail_tokens, size_t key_dim,
    const float* key_blocks, const float* value_blocks, size_t physical_blocks, size_t kv_heads,
    size_t block_tokens, size_t value_dim, const uint32_t* block_table, size_t logical_blocks,
    size_t history_tokens, const float* tail_key, const float* tail_value, float* output,
    float* score_workspace, size_t workspace_elements, helix_stream stream) {
  return guarded([&] {
    attention_with_tail(query, q_heads, tail_tokens, key_dim, key_blocks, value_blocks,
                        physical_blocks, kv_heads, block_tokens, value_dim, block_table,
                        logical_blocks, history_tokens, tail_key, tail_value, output,
                        score_workspace, workspace_elements, stream, true,
                        "paged_scaled_dot_product_attention_with_tail_out");
  });
}

// ---------------------------------------------------------- batched decode ----
namespace {

std::size_t resolve_split(std::size_t pages_per_split) {
  return pages_per_split == 0 ? helix::hip::kDefaultPagesPerSplit : pages_per_split;
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// The batched kernels are compiled for one page geometry.
void require_kernel_geometry(std::size_t head_dim, std::size_t block_tokens, const char* op) {
  if (head_dim != helix::hip::kDecodeHeadDim || block_tokens != helix::hip::kDecodeBlockTokens) {
    fail(Status::kUnsupported,
         std::string(op) + ": pools must have head_dim 128 and 16-token pages (got head_dim " +
             std::to_string(head_dim) + ", " + std::to_string(block_tokens) + "-token pages)");
  }
}

}  // namespace

int helix_paged_decode_workspace_bytes(size_t batch, size_t q_heads, size_t kv_heads,
                                       size_t max_blocks, size_t pages_per_split, size_t* out) {
  return guarded([&] {
    require_out(out);
    check(kv_heads != 0 && q_heads % kv_heads == 0, Status::kInvalidArgument,
          "paged_decode_workspace_bytes: q_heads must be a multiple of kv_heads");
    *out = helix::hip::decode_workspace_bytes(batch, q_heads, kv_heads, max_blocks,
                                              resolve_split(pages_per_split));
  });
}

int helix_paged_decode_workspace_init(void* workspace, size_t workspace_bytes,
                                      helix_stream stream) {
  return guarded([&] {
    check(workspace != nullptr || workspace_bytes == 0, Status::kInvalidArgument,
          "paged_decode_workspace_init: workspace must not be NULL");
    helix::hip_check(helix::hip::launch_decode_workspace_init(workspace, workspace_bytes,
                                                             as_stream(stream)),
                     "paged_decode_workspace_init");
  });
}

}  // extern "C"

namespace {

// Host validation shared by the batched decode entry points (the rules of
// cuda_paged.cu:211-352 for the batched shapes); false when the batch is
// empty.
bool check_decode_call(const char* op, const float* query, size_t batch, size_t q_heads,
                       size_t kv_heads, size_t head_dim, const float* key_blocks,
                       const float* value_blocks, size_t physical_blocks, size_t block_tokens,
                       const uint32_t* tables, size_t max_blocks, const int32_t* lengths,
                       const float* tail_key, const float* tail_value, const float* output,
                       size_t split) {
  require_kernel_geometry(head_dim, block_tokens, op);
  check(kv_heads != 0 && q_heads % kv_heads == 0 &&
            helix::hip::decode_group_supported(q_heads / kv_heads),
        Status::kUnsupported, op, "query groups of 1, 2, 4 or 8 heads only");
  check(physical_blocks != 0 && physical_blocks <= std::numeric_limits<std::uint32_t>::max(),
        Status::kInvalidArgument, op, "physical block count out of range");
  check(max_blocks != 0 && max_blocks <= static_cast<std::size_t>(
                                             std::numeric_limits<std::int32_t>::max() / 16),
        Status::kInvalidArgument, op, "max_blocks out of range");
  check(batch <= static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max()) /
                     (kv_heads * (max_blocks + 1)),
        Status::kInvalidArgument, op, "batch too large");
  if (batch == 0) return false;
  check(kv_heads * batch * helix::hip::decode_max_splits(max_blocks, split) <= (1u << 30),
        Status::kInvalidArgument, op, "too many work items");
  check(helix::hip::decode_max_splits(max_blocks, split) <= helix::hip::kMaxDecodeSplits,
        Status::kUnsupported, op, "max_blocks / pages_per_split above 4096");
  check(query && key_blocks && value_blocks && tables && lengths && tail_key && tail_value &&
            output,
        Status::kInvalidArgument, op, "device pointers must be non-null");
  check(aligned16(query) && aligned16(key_blocks) && aligned16(value_blocks) &&
            aligned16(tail_key) && aligned16(tail_value) && aligned16(output),
        Status::kInvalidArgument, op, "tensors must be 16-byte aligned");
  const std::size_t ob = batch * q_heads * helix::hip::kDecodeHeadDim * sizeof(float);
  check(!overlap(output, ob, query, ob), Status::kInvalidArgument,
        op, "output must not alias query");
  return true;
}

// Largest workspace helix_paged_decode_attention_noalloc can use: the
// partial results of the stream kernel for (units + wavefronts) slots.
constexpr std::size_t kNoAllocScratchBytes = std::size_t{16} << 20;
constexpr int kMaxDevices = 64;

}  // namespace

// The scratch of helix_paged_decode_attention_noalloc.  Every device the
// library runs that entry point on holds its own copy until the process
// ends.  In host code `scratch` is only a handle: its device address comes
// from hipGetSymbolAddress, once per device.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::atomic<void*> g_scratch[kMaxDevices];

// Device address of `scratch` on the current device (looked up on the
// device's first call; concurrent first calls look it up twice, harmlessly).
void* scratch_address(const char* op) {
  int device = -1;
  helix::hip_check(hipGetDevice(&device), op);
  check(device >= 0 && device < kMaxDevices, Status::kUnsupported, op,
        "device index above the scratch table");
  void* p = g_scratch[device].load(std::memory_order_acquire);
  if (p == nullptr) {
    helix::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), op);
    check(p != nullptr, Status::kRuntime, op, "scratch symbol has no device address");
    g_scratch[device].store(p, std::memory_order_release);
  }
  return p;
}

// The page format of a typed entry point's pools: HELIX_PAGE_F32 (the
// reference's), HELIX_PAGE_BF16, or HELIX_PAGE_FP8_E4M3 with the pools'
// finite, positive key and value scales (ignored for the other types).
helix::hip::PageFormat page_format(int page_dtype, float key_scale, float value_scale,
                                   const char* op) {
  check(page_dtype == HELIX_PAGE_F32 || page_dtype == HELIX_PAGE_BF16 ||
            page_dtype == HELIX_PAGE_FP8_E4M3,
        Status::kInvalidArgument,
        std::string(op) + ": page dtype must be HELIX_PAGE_F32, HELIX_PAGE_BF16 or "
                          "HELIX_PAGE_FP8_E4M3");
  if (page_dtype != HELIX_PAGE_FP8_E4M3) {
    return helix::hip::PageFormat(static_cast<helix::hip::PageType>(page_dtype));
  }
  check(std::isfinite(key_scale) && key_scale > 0.0f && std::isfinite(value_scale) &&
            value_scale > 0.0f,
        Status::kInvalidArgument, std::string(op) + ": fp8 page scales must be finite and positive");
  return helix::hip::PageFormat(helix::hip::PageType::kFP8, key_scale, value_scale);
}

helix::hip::DecodeArgs decode_args(const float* query, size_t batch, size_t q_heads,
                                   size_t kv_heads, const float* key_blocks,
                                   const float* value_blocks, size_t physical_blocks,
                                   const uint32_t* tables, size_t max_blocks,
                                   const int32_t* lengths, const float* tail_key,
                                   const float* tail_value, float* output, void* workspace,
                                   size_t split) {
  helix::hip::DecodeArgs a{};
  a.query = query;
  a.key_pool = key_blocks;
  a.value_pool = value_blocks;
  a.tables = tables;
  a.lengths = lengths;
  a.tail_key = tail_key;
  a.tail_value = tail_value;
  a.out = output;
  a.workspace = workspace;
  a.batch = batch;
  a.q_heads = q_heads;
  a.kv_heads = kv_heads;
  a.max_blocks = max_blocks;
  a.physical_blocks = physical_blocks;
  a.pages_per_split = split;
  a.items = 0;
  return a;
}

}  // namespace

extern "C" {

int helix_paged_decode_attention(const float* query, size_t batch, size_t q_heads,
                                 size_t kv_heads, size_t head_dim, const float* key_blocks,
                                 const float* value_blocks, size_t physical_blocks,
                                 size_t block_tokens, const uint32_t* tables, size_t max_blocks,
                                 const int32_t* lengths, const float* tail_key,
                                 const float* tail_value, float* output, void* workspace,
                                 size_t workspace_bytes, size_t pages_per_split,
                                 helix_stream stream) {
  return helix_paged_decode_attention_typed(
      query, batch, q_heads, kv_heads, head_dim, key_blocks, value_blocks, physical_blocks,
      block_tokens, tables, max_blocks, lengths, tail_key, tail_value, output, workspace,
      workspace_bytes, pages_per_split, HELIX_PAGE_F32, 1.0f, 1.0f, stream);
}

int helix_paged_decode_attention_typed(const float* query, size_t batch, size_t q_heads,
                                       size_t kv_heads, size_t head_dim, const void* key_blocks,
                                       const void* value_blocks, size_t physical_blocks,
                                       size_t block_tokens, const uint32_t* tables,
                                       size_t max_blocks, const int32_t* lengths,
                                       const float* tail_key, const float* tail_value,
                                       float* output, void* workspace, size_t workspace_bytes,
                                       size_t pages_per_split, int page_dtype, float key_scale,
                                       float value_scale, helix_stream stream) {
  return guarded([&] {
    constexpr const char* op = "paged_decode_attention";
    const helix::hip::PageFormat fmt = page_format(page_dtype, key_scale, value_scale, op);
    check(fmt.type == helix::hip::PageType::kF32 || pages_per_split == 0, Status::kUnsupported,
          std::string(op) + ": bf16 and fp8 pages run the stream kernel only (pages_per_split 0)");
    const std::size_t split = resolve_split(pages_per_split);
    const auto* kb = static_cast<const float*>(key_blocks);
    const auto* vb = static_cast<const float*>(value_blocks);
    if (!check_decode_call(op, query, batch, q_heads, kv_heads, head_dim, kb, vb,
                           physical_blocks, block_tokens, tables, max_blocks, lengths, tail_key,
                           tail_value, output, split)) {
      return;
    }
    check(workspace != nullptr && aligned16(workspace), Status::kInvalidArgument,
          std::string(op) + ": workspace must be a non-null 16-byte aligned device pointer");
    check(workspace_bytes >=
              helix::hip::decode_workspace_bytes(batch, q_heads, kv_heads, max_blocks, split),
          Status::kInvalidArgument, std::string(op) + ": workspace is too small");
    const std::size_t ob = batch * q_heads * helix::hip::kDecodeHeadDim * sizeof(float);
    check(!overlap(output, ob, workspace, workspace_bytes), Status::kInvalidArgument,
          std::string(op) + ": output must not alias query or workspace");
    helix::hip::DecodeArgs a =
        decode_args(query, batch, q_heads, kv_heads, kb, vb, physical_blocks, tables,
                    max_blocks, lengths, tail_key, tail_value, output, workspace, split);
    a.page_type = fmt;
    helix::hip_check(helix::hip::launch_decode(a, as_stream(stream)), op);
  });
}

int helix_paged_decode_attention_noalloc(const float* query, size_t batch, size_t q_heads,
                                         size_t kv_heads, size_t head_dim, const void* key_blocks,
                                         const void* value_blocks, size_t physical_blocks,
                                         size_t block_tokens, const uint32_t* tables,
                                         size_t max_blocks, const int32_t* lengths,
                                         const float* tail_key, const float* tail_value,
                                         float* output, int page_dtype, float key_scale,
                                         float value_scale, helix_stream stream) {
  return guarded([&] {
    constexpr const char* op = "paged_decode_attention_noalloc";
    const helix::hip::PageFormat fmt = page_format(page_dtype, key_scale, value_scale, op);
    const auto* kb = static_cast<const float*>(key_blocks);
    const auto* vb = static_cast<const float*>(value_blocks);
    if (!check_decode_call(op, query, batch, q_heads, kv_heads, head_dim, kb, vb,
                           physical_blocks, block_tokens, tables, max_blocks, lengths, tail_key,
                           tail_value, output, 0)) {
      return;
    }
    check(helix::hip::compact_decode_workspace_bytes(batch, q_heads, kv_heads, fmt.type) <=
              kNoAllocScratchBytes,
          Status::kOutOfRange, op,
          "batch * kv_heads too large for the 16 MiB scratch (use "
          "helix_paged_decode_attention with a workspace)");
    void* ws = scratch_address(op);
    helix::hip::DecodeArgs a =
        decode_args(query, batch, q_heads, kv_heads, kb, vb, physical_blocks, tables,
                    max_blocks, lengths, tail_key, tail_value, output, ws, 0);
    a.page_type = fmt;
    a.compact_layout = true;
    helix::hip_check(helix::hip::launch_decode(a, as_stream(stream)), op);
  });
}

int helix_rope(const float* input, float* output, size_t tokens, size_t vectors,
               size_t head_dim, const float* cosine, const float* sine, size_t cache_rows,
               const int32_t* positions, helix_stream stream) {
  return guarded([&] {
    constexpr const char* op = "rope";
    check(head_dim != 0 && head_dim % 2 == 0, Status::kInvalidArgument,
          std::string(op) + ": head dimension must be positive and even");
    if (tokens == 0 || vectors == 0) return;
    check(input && output && cosine && sine, Status::kInvalidArgument,
          std::string(op) + ": device pointers must be non-null");
    check(positions != nullptr || cache_rows == tokens, Status::kInvalidArgument,
          std::string(op) + ": without positions the tables need one row per token");
    check(cache_rows != 0, Status::kInvalidArgument, std::string(op) + ": tables have no rows");
    const std::size_t elems = mul(mul(tokens, vectors), head_dim);
    check(elems / 2 < (std::size_t{1} << 31), Status::kOutOfRange,
          std::string(op) + ": too many elements for one launch");
    check(((reinterpret_cast<std::uintptr_t>(input) | reinterpret_cast<std::uintptr_t>(output)) & 7u) == 0,
          Status::kInvalidArgument, std::string(op) + ": input and output must be 8-byte aligned");
    const std::size_t bytes = elems * sizeof(float);
    check(input == output || !overlap(input, bytes, output, bytes), Status::kInvalidArgument,
          std::string(op) + ": output must be the input itself or not overlap it");
    const std::size_t tb = mul(cache_rows, head_dim / 2) * sizeof(float);
    check(!overlap(cosine, tb, output, bytes) && !overlap(sine, tb, output, bytes),
          Status::kInvalidArgument, std::string(op) + ": output must not alias the tables");
    helix::hip_check(helix::hip::launch_rope(helix::hip::RopeTensor{input, output, vectors},
                                             helix::hip::RopeTensor{}, tokens, head_dim, cosine,
                                             sine, cache_rows, positions, as_stream(stream)),
                     op);
  });
}

int helix_paged_append_slots(const float* keys, const float* values, float* key_blocks,
                             float* value_blocks, size_t physical_blocks, size_t kv_heads,
                             size_t block_tokens, size_t head_dim, const int64_t* slots,
                             size_t count, helix_stream stream) {
  return guarded([&] {
    check(physical_blocks != 0 && kv_heads != 0 && block_tokens != 0 && head_dim != 0,
          Status::kInvalidArgument, "append_slots: geometry must be positive");
    if (count == 0) return;
    check(keys && values && key_blocks && value_blocks && slots, Status::kInvalidArgument,
          "append_slots: device pointers must be non-null");
    helix::hip_check(
        helix::hip::launch_append_slots(
            keys, values, key_blocks, value_blocks,
            helix::hip::PageGeometry{physical_blocks, kv_heads, block_tokens, head_dim}, slots,
            count, as_stream(stream)),
        "append_slots");
  });
}

int helix_paged_append_chunk(const float* keys, const float* values, float* key_blocks,
                             float* value_blocks, size_t physical_blocks, size_t kv_heads,
                             size_t block_tokens, size_t head_dim, const int64_t* slots,
                             size_t batch, size_t tokens, helix_stream stream) {
  return guarded([&] {
    check(physical_blocks != 0 && kv_heads != 0 && block_tokens != 0 && head_dim != 0,
          Status::kInvalidArgument, "append_chunk: geometry must be positive");
    if (batch == 0 || tokens == 0) return;
    check(keys && values && key_blocks && value_blocks && slots, Status::kInvalidArgument,
          "append_chunk: device pointers must be non-null");
    helix::hip_check(
        helix::hip::launch_append_slots(
            keys, values, key_blocks, value_blocks,
            helix::hip::PageGeometry{physical_blocks, kv_heads, block_tokens, head_dim}, slots,
            batch, as_stream(stream), tokens),
        "append_chunk");
  });
}

int helix_paged_prefill_attention(const float* query, size_t batch, size_t q_heads,
                                  size_t kv_heads, size_t tokens, size_t head_dim,
                                  const float* key_blocks, const float* value_blocks,
                                  size_t physical_blocks, size_t block_tokens,
                                  const uint32_t* tables, size_t max_blocks,
                                  const int32_t* lengths, const float* chunk_key,
                                  const float* chunk_value, float* output, helix_stream stream) {
  return helix_paged_prefill_attention_typed(query, batch, q_heads, kv_heads, tokens, head_dim,
                                             key_blocks, value_blocks, physical_blocks,
                                             block_tokens, tables, max_blocks, lengths, chunk_key,
                                             chunk_value, output, HELIX_PAGE_F32, 1.0f, 1.0f,
                                             stream);
}

int helix_paged_prefill_attention_typed(const float* query, size_t batch, size_t q_heads,
                                        size_t kv_heads, size_t tokens, size_t head_dim,
                                        const void* key_blocks, const void* value_blocks,
                                        size_t physical_blocks, size_t block_tokens,
                                        const uint32_t* tables, size_t max_blocks,
                                        const int32_t* lengths, const float* chunk_key,
                                        const float* chunk_value, float* output, int page_dtype,
                                        float key_scale, float value_scale, helix_stream stream) {
  return guarded([&] {
    constexpr const char* op = "paged_prefill_attention";
    const helix::hip::PageFormat fmt = page_format(page_dtype, key_scale, value_scale, op);
    require_kernel_geometry(head_dim, block_tokens, op);
    check(kv_heads != 0 && q_heads % kv_heads == 0 &&
              helix::hip::prefill_group_supported(q_heads / kv_heads),
          Status::kUnsupported, std::string(op) + ": query groups of 1, 2, 4 or 8 heads only");
    check(physical_blocks != 0 && physical_blocks <= std::numeric_limits<std::uint32_t>::max(),
          Status::kInvalidArgument, std::string(op) + ": physical block count out of range");
    check(max_blocks != 0 && max_blocks <= static_cast<std::size_t>(
                                               std::numeric_limits<std::int32_t>::max() / 32),
          Status::kInvalidArgument, std::string(op) + ": max_blocks out of range");
    check(tokens <= static_cast<std::size_t>(std::numeric_limits<std::int32_t>::max() / 2),
          Status::kInvalidArgument, std::string(op) + ": chunk too long");
    check(batch <= 65535 && kv_heads <= 65535, Status::kInvalidArgument,
          std::string(op) + ": batch and kv_heads must fit a grid dimension");
    if (batch == 0 || tokens == 0) return;
    check(query && key_blocks && value_blocks && tables && lengths && chunk_key && chunk_value &&
              output,
          Status::kInvalidArgument, std::string(op) + ": device pointers must be non-null");
    check(aligned16(query) && aligned16(key_blocks) && aligned16(value_blocks) &&
              aligned16(chunk_key) && aligned16(chunk_value) && aligned16(output),
          Status::kInvalidArgument, std::string(op) + ": tensors must be 16-byte aligned");
    const std::size_t ob = batch * q_heads * tokens * helix::hip::kDecodeHeadDim * sizeof(float);
    const std::size_t cb = batch * kv_heads * tokens * helix::hip::kDecodeHeadDim * sizeof(float);
    check(!overlap(output, ob, query, ob) && !overlap(output, ob, chunk_key, cb) &&
              !overlap(output, ob, chunk_value, cb),
          Status::kInvalidArgument, std::string(op) + ": output must not alias query or chunk");
    helix::hip::PrefillArgs a{};
    a.query = query;
    a.key_pool = static_cast<const float*>(key_blocks);
    a.value_pool = static_cast<const float*>(value_blocks);
    a.tables = tables;
    a.lengths = lengths;
    a.chunk_key = chunk_key;
    a.chunk_value = chunk_value;
    a.out = output;
    a.batch = batch;
    a.q_heads = q_heads;
    a.kv_heads = kv_heads;
    a.tokens = tokens;
    a.max_blocks = max_blocks;
    a.physical_blocks = physical_blocks;
    a.page_type = fmt;
    helix::hip_check(helix::hip::launch_prefill(a, as_stream(stream)), op);
  });
}

int helix_decode_batch_create(helix_paged_cache* cache, const helix_sequence* sequences,
                              size_t batch, size_t q_heads, size_t max_tokens,
                              size_t pages_per_split, helix_decode_batch** out) {
  return guarded([&] {
    REQUIRE_CACHE();
    require_out(out);
    *out = nullptr;
    check(batch == 0 || sequences != nullptr, Status::kInvalidArgument,
          "decode batch sequences must not be NULL");
    std::vector<std::uint64_t> ids(batch), cids(batch);
    for (std::size_t i = 0; i < batch; ++i) {
      ids[i] = sequences[i].id;
      cids[i] = sequences[i].cache_id;
    }
    auto b = std::make_unique<helix_decode_batch>();
    b->batch = std::make_unique<helix::DecodeBatch>(cache->cache.state(), ids.data(),
                                                    cids.data(), batch, q_heads, max_tokens,
                                                    pages_per_split);
    *out = b.release();
  });
}

int helix_decode_batch_prepare(helix_decode_batch* b, helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->prepare(as_stream(stream));
  });
}

int helix_decode_batch_prepare_chunk(helix_decode_batch* b, size_t tokens, helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->prepare(as_stream(stream), tokens);
  });
}

int helix_decode_batch_append_layer(helix_decode_batch* b, size_t layer, const float* keys,
                                    const float* values, helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->append_layer(layer, keys, values, as_stream(stream));
  });
}

int helix_decode_batch_append_all_layers(helix_decode_batch* b, const float* keys,
                                         const float* values, helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->append_all_layers(keys, values, as_stream(stream));
  });
}

int helix_decode_batch_rope(helix_decode_batch* b, float* query, float* key,
                            const float* cosine, const float* sine, size_t cache_rows,
                            helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    check(((reinterpret_cast<std::uintptr_t>(query) | reinterpret_cast<std::uintptr_t>(key)) & 7u) == 0,
          Status::kInvalidArgument, "decode batch rope: query and key must be 8-byte aligned");
    b->batch->rope(query, key, cosine, sine, cache_rows, as_stream(stream));
  });
}

int helix_decode_batch_attention_layer(helix_decode_batch* b, size_t layer, const float* query,
                                       const float* tail_key, const float* tail_value,
                                       float* output, helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->attention_layer(layer, query, tail_key, tail_value, output, as_stream(stream));
  });
}

int helix_decode_batch_append_attention_layer(helix_decode_batch* b, size_t layer,
                                              const float* query, const float* keys,
                                              const float* values, float* output,
                                              helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    check(keys != nullptr && values != nullptr, Status::kInvalidArgument,
          "decode batch append needs key and value rows");
    b->batch->append_attention_layer(layer, query, keys, values, output, as_stream(stream));
  });
}

int helix_decode_batch_prefill_layer(helix_decode_batch* b, size_t layer, const float* query,
                                     const float* chunk_key, const float* chunk_value,
                                     float* output, helix_stream stream) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->prefill_layer(layer, query, chunk_key, chunk_value, output, as_stream(stream));
  });
}

int helix_decode_batch_tables(const helix_decode_batch* b, const uint32_t** tables,
                              const int32_t** lengths, const int64_t** slots,
                              size_t* max_blocks, size_t* pages_per_split) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    if (tables != nullptr) *tables = b->batch->tables();
    if (lengths != nullptr) *lengths = b->batch->lengths();
    if (slots != nullptr) *slots = b->batch->slots();
    if (max_blocks != nullptr) *max_blocks = b->batch->max_blocks();
    if (pages_per_split != nullptr) *pages_per_split = b->batch->pages_per_split();
  });
}

int helix_decode_batch_shared_pages(const helix_decode_batch* b, size_t* out) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    require_out(out);
    *out = b->batch->shared_pages();
  });
}

int helix_decode_batch_set_timing_event(helix_decode_batch* b, void* event) {
  return guarded([&] {
    check(b != nullptr, Status::kInvalidArgument, "decode batch must not be NULL");
    b->batch->set_between_event(static_cast<hipEvent_t>(event));
  });
}

void helix_decode_batch_destroy(helix_decode_batch* b) { delete b; }

// ------------------------------------------------------------ prefix cache

int helix_prefix_cache_create(helix_paged_cache* cache, const helix_prefix_config* config,
                              helix_prefix_cache** out) {
  return guarded([&] {
    check(cache != nullptr, Status::kInvalidArgument, "prefix cache: paged cache must not be null");
    require_out(out);
    *out = new helix_prefix_cache(std::make_unique<helix::PrefixCache>(
        std::make_unique<DeviceAnchors>(cache->cache.state()), to_prefix_config(config)));
  });
}

}  // extern "C"
