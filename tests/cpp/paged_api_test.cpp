// C++ API tests of libhelix_paged through include/helix_paged.hpp, written
// after the reference's own CUDA tests (tests/cuda_paged_kv_cache_test.cpp,
// tests/cuda_attention_test.cpp:196-556): the same cases, inputs, seeds and
// tolerances, against the HIP path.  Expected attention values come from the
// CPU oracle (oracle/liboracle.so, linked as the checker only); the seeded
// inputs use the oracle's restatement of Tensor::random_uniform, so seeds
// such as 8'101 give the reference tests' values.
//
// Built by tests/cpp/Makefile; run by tests/test_gpu_cpp_api.py on a GPU.
// Without a GPU the host-contract cases run and every GPU case reports
// SKIPPED (the CPU suite runs the binary that way).

#include "helix_paged.hpp"
#include "mini_test.hpp"

#include <algorithm>
#include <array>
#include <chrono>
#include <cstring>
#include <future>
#include <limits>
#include <numeric>
#include <type_traits>

extern "C" {
int oracle_sdpa(const float* query, const float* key, const float* value, std::size_t heads,
                std::size_t queries, std::size_t keys, std::size_t head_dim,
                std::size_t value_dim, std::size_t offset, float* output, float* workspace);
int oracle_batched_decode(const float* query, std::size_t batch, std::size_t q_heads,
                          std::size_t kv_heads, std::size_t head_dim, const float* key_blocks,
                          const float* value_blocks, std::size_t block_tokens,
                          const std::uint32_t* tables, std::size_t max_blocks,
                          const std::int32_t* lengths, const float* tail_key,
                          const float* tail_value, float* output, int threads);
void oracle_random_uniform(std::uint64_t seed, float lower, float upper, float* out,
                           std::size_t n);
int oracle_paged_attention(const float* query, std::size_t q_heads, std::size_t kv_heads,
                           std::size_t query_tokens, std::size_t head_dim, std::size_t value_dim,
                           const float* key_blocks, const float* value_blocks,
                           std::size_t block_tokens, const std::uint32_t* block_table,
                           std::size_t history, const float* tail_key, const float* tail_value,
                           std::size_t tail, std::size_t offset, float* output,
                           float* workspace);
}

namespace {

using namespace helix_amd;
using namespace helix_amd::kv_cache;
using helix_amd::attention::hip::paged_scaled_dot_product_attention;
using helix_amd::attention::hip::paged_scaled_dot_product_attention_out;
using helix_amd::attention::hip::paged_scaled_dot_product_attention_with_tail;
using helix_amd::attention::hip::paged_scaled_dot_product_attention_with_tail_out;
using helix_amd::attention::hip::paged_score_workspace_bytes;
using helix_amd::attention::hip::paged_tail_score_workspace_bytes;
using helix_amd::attention::hip::paged_tail_score_workspace_shape;
using PagedBlockTable = helix_amd::kv_cache::hip::PagedBlockTable;
using Stream = helix_amd::hip::Stream;

static_assert(!std::is_copy_constructible_v<HipPagedKvCache::DecodeView>);
static_assert(!std::is_copy_assignable_v<HipPagedKvCache::DecodeView>);
static_assert(std::is_nothrow_move_constructible_v<HipPagedKvCache::DecodeView>);
static_assert(std::is_nothrow_move_assignable_v<HipPagedKvCache::DecodeView>);
static_assert(
    noexcept(std::declval<HipPagedKvCache::DecodeView&>().poison_after_consumer_failure()));
static_assert(!std::is_copy_constructible_v<PagedBlockTable>);
static_assert(std::is_nothrow_move_constructible_v<PagedBlockTable>);
static_assert(std::is_nothrow_move_assignable_v<PagedBlockTable>);
static_assert(std::is_same_v<CudaPagedKvCache, HipPagedKvCache>);

struct GpuFixture {
  void SetUp() {
    if (!helix_amd::hip::runtime_available()) SKIP("requires a visible AMD GPU");
    helix_amd::hip::set_device(0);
  }
};
struct HostContractTest {
  void SetUp() {}
};
struct HipPagedKvCacheTest : GpuFixture {};
struct HipAttentionTest : GpuFixture {};
struct HipDecodeBatchTest : GpuFixture {};

const Device kGpu = Device::gpu(0);

std::vector<float> host_values(const Tensor& t) {
  const Tensor h = t.to(Device::cpu());
  return std::vector<float>(h.data_as<float>(), h.data_as<float>() + h.numel());
}

Tensor random_uniform(Shape shape, std::uint64_t seed, float lo, float hi) {
  std::vector<float> v(shape_numel(shape));
  oracle_random_uniform(seed, lo, hi, v.data(), v.size());
  return Tensor::from_values(std::move(shape), v);
}

void expect_error_code(const std::function<void()>& operation, ErrorCode code) {
  try {
    operation();
    FAIL("expected helix_amd::Error");
  } catch (const Error& error) {
    EXPECT_EQ(static_cast<int>(error.code()), static_cast<int>(code));
  }
}

// ------------------------------------------ host contracts (no GPU needed) ----
// Validation that happens before any device work, and the status -> Error
// mapping (include/helix/core/error.hpp:10-17: status = code + 1).
TEST_F(HostContractTest, InvalidTablesAndConfigsThrowTheReferenceErrorCodes) {
  constexpr std::array<std::uint32_t, 1> kOutOfRange{3};
  expect_error_code([] { PagedBlockTable t(std::span<const std::uint32_t>{}, 0, 0); },
                    ErrorCode::kInvalidArgument);
  expect_error_code([&] { PagedBlockTable t(kOutOfRange, 3, 0); }, ErrorCode::kOutOfRange);
  expect_error_code([&] { PagedBlockTable t(kOutOfRange, 4, -1); }, ErrorCode::kInvalidArgument);
  expect_error_code([] { HipPagedKvCache c(PagedKvCacheConfig{0, 1, 1, 1, 1}); },
                    ErrorCode::kInvalidArgument);
  expect_error_code([] { HipPagedKvCache c(PagedKvCacheConfig{1, 1, 1, 1, 1}, -1); },
                    ErrorCode::kInvalidArgument);
  EXPECT_TRUE(error_code_name(ErrorCode::kResourceExhausted) == "ResourceExhausted");
  try {
    helix_amd::detail::check(HELIX_OUT_OF_RANGE);
    FAIL("check() must throw on a non-zero status");
  } catch (const Error& e) {
    EXPECT_TRUE(e.code() == ErrorCode::kOutOfRange);
  }
}

TEST_F(HostContractTest, HostTensorsReshapeShareStorageAndCheckCounts) {
  const Tensor t = Tensor::from_values({2, 3}, std::array{1.F, 2.F, 3.F, 4.F, 5.F, 6.F});
  const Tensor r = t.reshape({3, 2});
  EXPECT_TRUE(r.data_as<float>() == t.data_as<float>());
  EXPECT_EQ(r.numel(), 6U);
  EXPECT_EQ(r.nbytes(), 24U);
  EXPECT_THROW(static_cast<void>(t.reshape({4, 2})), Error);
  EXPECT_THROW(static_cast<void>(Tensor::from_values({2, 2}, std::array{1.F, 2.F, 3.F})), Error);
  const Tensor z = Tensor::zeros({0, 5});
  EXPECT_EQ(z.numel(), 0U);
  const HipPagedSequenceHandle empty;
  EXPECT_FALSE(static_cast<bool>(empty));
  EXPECT_EQ(empty.native().id, 0U);
}

// ------------------------------------------------ paged KV cache (device) ----
// tests/cuda_paged_kv_cache_test.cpp:40-66
std::pair<Tensor, Tensor> make_token(const PagedKvCacheConfig& config, std::size_t token) {
  const std::size_t elements = config.layers * config.kv_heads * config.head_dimension;
  std::vector<float> keys(elements), values(elements);
  for (std::size_t layer = 0; layer < config.layers; ++layer)
    for (std::size_t head = 0; head < config.kv_heads; ++head)
      for (std::size_t c = 0; c < config.head_dimension; ++c) {
        const std::size_t index = (layer * config.kv_heads + head) * config.head_dimension + c;
        const float encoded = static_cast<float>(token * 1000 + layer * 100 + head * 10 + c);
        keys[index] = encoded + 0.25F;
        values[index] = -encoded - 0.5F;
      }
  const Shape shape{static_cast<Dimension>(config.layers), static_cast<Dimension>(config.kv_heads),
                    static_cast<Dimension>(config.head_dimension)};
  return {Tensor::from_values(shape, keys, kGpu), Tensor::from_values(shape, values, kGpu)};
}

float expected_value(std::size_t token, std::size_t layer, std::size_t head, std::size_t c,
                     bool keys) {
  const float encoded = static_cast<float>(token * 1000 + layer * 100 + head * 10 + c);
  return keys ? encoded + 0.25F : -encoded - 0.5F;
}

// tests/cuda_paged_kv_cache_test.cpp:77-152
TEST_F(HipPagedKvCacheTest, MapsOddHistoryAcrossPagesAndReportsExactAccounting) {
  const PagedKvCacheConfig config{2, 3, 5, 2, 3};
  HipPagedKvCache cache(config);
  EXPECT_TRUE(cache.is_healthy());
  Stream stream;
  const HipPagedSequenceHandle sequence = cache.create_sequence();
  {
    auto empty = cache.read_sequence(sequence);
    EXPECT_EQ(empty.length(), 0U);
    EXPECT_TRUE(empty.physical_blocks().empty());
    EXPECT_TRUE(empty.block_table().valid());
    EXPECT_TRUE(empty.block_table().data() == nullptr);
    EXPECT_EQ(empty.block_table().logical_block_count(), 0U);
    ASSERT_EQ(empty.layer_key_blocks().size(), config.layers);
    EXPECT_TRUE(empty.layer_key_blocks()[0].shape() == (Shape{3, 3, 2, 5}));
  }
  for (std::size_t token = 0; token < 5; ++token) {
    const auto [keys, values] = make_token(config, token);
    cache.append(sequence, keys, values, stream);
  }
  stream.synchronize();
  {
    auto view = cache.read_sequence(sequence);
    EXPECT_EQ(view.length(), 5U);
    constexpr std::array<std::uint32_t, 3> kExpectedBlocks{0, 1, 2};
    EXPECT_TRUE(std::equal(view.physical_blocks().begin(), view.physical_blocks().end(),
                           kExpectedBlocks.begin(), kExpectedBlocks.end()));
    EXPECT_EQ(view.block_table().logical_block_count(), 3U);
    EXPECT_EQ(view.block_table().physical_block_count(), 3U);
    for (std::size_t layer = 0; layer < config.layers; ++layer) {
      const auto hk = host_values(view.layer_key_blocks()[layer]);
      const auto hv = host_values(view.layer_value_blocks()[layer]);
      for (std::size_t token = 0; token < 5; ++token) {
        const std::size_t block = token / config.block_tokens, slot = token % config.block_tokens;
        for (std::size_t head = 0; head < config.kv_heads; ++head)
          for (std::size_t c = 0; c < config.head_dimension; ++c) {
            const std::size_t i =
                ((block * config.kv_heads + head) * config.block_tokens + slot) *
                    config.head_dimension + c;
            // bit-exact: the append is a copy
            EXPECT_EQ(hk[i], expected_value(token, layer, head, c, true));
            EXPECT_EQ(hv[i], expected_value(token, layer, head, c, false));
          }
      }
    }
  }
  const PagedKvCacheStats stats = cache.stats();
  EXPECT_EQ(cache.bytes_per_token(), 2U * 2U * 3U * 5U * sizeof(float));
  EXPECT_EQ(cache.block_bytes(), cache.bytes_per_token() * config.block_tokens);
  EXPECT_EQ(cache.token_capacity(), 6U);
  EXPECT_EQ(stats.bytes_reserved, cache.block_bytes() * config.physical_blocks);
  EXPECT_EQ(stats.bytes_used, stats.bytes_reserved);
  EXPECT_EQ(stats.bytes_free, 0U);
  EXPECT_EQ(stats.peak_bytes_used, stats.bytes_reserved);
  EXPECT_EQ(stats.total_blocks, 3U);
  EXPECT_EQ(stats.used_blocks, 3U);
  EXPECT_EQ(stats.free_blocks, 0U);
  EXPECT_EQ(stats.active_sequence_count, 1U);
  EXPECT_EQ(stats.active_tokens, 5U);
  EXPECT_EQ(stats.resident_tokens, 5U);
  EXPECT_EQ(stats.allocated_token_slots, 6U);
  EXPECT_EQ(stats.unused_token_slots(), 1U);
  EXPECT_EQ(stats.block_reference_count, 3U);
  EXPECT_EQ(stats.shared_blocks, 0U);
  EXPECT_EQ(stats.sequence_create_count, 1U);
  EXPECT_EQ(stats.append_count, 5U);
  EXPECT_EQ(stats.block_allocation_count, 3U);
  EXPECT_EQ(stats.block_reuse_count, 0U);
}

// tests/cuda_paged_kv_cache_test.cpp:154-192
TEST_F(HipPagedKvCacheTest, ExhaustionIsTransactionalAndReleasedBlocksReuseInFifoOrder) {
  const PagedKvCacheConfig config{1, 2, 3, 2, 3};
  HipPagedKvCache cache(config);
  Stream stream;
  const HipPagedSequenceHandle first = cache.create_sequence();
  const HipPagedSequenceHandle second = cache.create_sequence();
  for (std::size_t token = 0; token < 4; ++token) {
    const auto [keys, values] = make_token(config, token);
    cache.append(first, keys, values, stream);
  }
  const auto [second_keys, second_values] = make_token(config, 10);
  cache.append(second, second_keys, second_values, stream);
  const auto [slack_keys, slack_values] = make_token(config, 11);
  cache.append(second, slack_keys, slack_values, stream);
  ASSERT_EQ(cache.stats().free_blocks, 0U);

  const PagedKvCacheStats before = cache.stats();
  const auto [rejected_keys, rejected_values] = make_token(config, 12);
  expect_error_code([&] { cache.append(second, rejected_keys, rejected_values, stream); },
                    ErrorCode::kResourceExhausted);
  EXPECT_EQ(cache.length(second), 2U);
  EXPECT_EQ(cache.stats().append_count, before.append_count);
  EXPECT_EQ(cache.stats().block_allocation_count, before.block_allocation_count);
  EXPECT_EQ(cache.stats().bytes_used, before.bytes_used);

  cache.release_sequence(first);
  EXPECT_FALSE(cache.contains(first));
  EXPECT_EQ(cache.stats().free_blocks, 2U);
  cache.append(second, rejected_keys, rejected_values, stream);
  {
    auto view = cache.read_sequence(second);
    ASSERT_EQ(view.physical_blocks().size(), 2U);
    EXPECT_EQ(view.physical_blocks()[0], 2U);
    EXPECT_EQ(view.physical_blocks()[1], 0U);
  }
  EXPECT_EQ(cache.stats().block_reuse_count, 1U);
  EXPECT_EQ(cache.stats().release_count, 1U);
  stream.synchronize();
}

// tests/cuda_paged_kv_cache_test.cpp:194-234
TEST_F(HipPagedKvCacheTest, RejectsInvalidConfigurationHandlesTensorsStreamsAndAliasing) {
  EXPECT_THROW(HipPagedKvCache(PagedKvCacheConfig{0, 1, 1, 1, 1}), Error);
  EXPECT_THROW(HipPagedKvCache(PagedKvCacheConfig{1, 0, 1, 1, 1}), Error);
  EXPECT_THROW(HipPagedKvCache(PagedKvCacheConfig{1, 1, 0, 1, 1}), Error);
  EXPECT_THROW(HipPagedKvCache(PagedKvCacheConfig{1, 1, 1, 0, 1}), Error);
  EXPECT_THROW(HipPagedKvCache(PagedKvCacheConfig{1, 1, 1, 1, 0}), Error);
  EXPECT_THROW(HipPagedKvCache(PagedKvCacheConfig{1, 1, 1, 1, 1}, -1), Error);

  const PagedKvCacheConfig config{1, 1, 2, 1, 1};
  HipPagedKvCache first(config);
  HipPagedKvCache second(config);
  const HipPagedSequenceHandle sequence = first.create_sequence();
  const HipPagedSequenceHandle foreign = second.create_sequence();
  Stream stream;
  const auto [keys, values] = make_token(config, 0);

  EXPECT_THROW(first.append(foreign, keys, values, stream), Error);
  EXPECT_THROW(first.append(HipPagedSequenceHandle{}, keys, values, stream), Error);
  EXPECT_THROW(first.append(sequence, Tensor::zeros({1, 1, 2}), values, stream), Error);
  EXPECT_THROW(first.append(sequence, Tensor::zeros({1, 1, 2}, DType::kUInt32, kGpu), values,
                            stream),
               Error);
  EXPECT_THROW(first.append(sequence, Tensor::zeros({1, 2}, DType::kFloat32, kGpu), values,
                            stream),
               Error);

  Stream active_stream = std::move(stream);
  EXPECT_THROW(first.append(sequence, keys, values, stream), Error);

  std::optional<Tensor> aliased_keys;
  {
    auto view = first.read_sequence(sequence);
    aliased_keys.emplace(view.layer_key_blocks()[0].reshape({1, 1, 2}));
  }
  EXPECT_THROW(first.append(sequence, *aliased_keys, values, active_stream), Error);

  first.append(sequence, keys, values, active_stream);
  first.release_sequence(sequence);
  EXPECT_THROW(first.release_sequence(sequence), Error);
  EXPECT_THROW(static_cast<void>(first.read_sequence(sequence)), Error);
  active_stream.synchronize();
}

// tests/cuda_paged_kv_cache_test.cpp:236-267
TEST_F(HipPagedKvCacheTest, DecodeViewPinsMappingAndPoolLifetimeAndMovesSafely) {
  const PagedKvCacheConfig config{1, 1, 3, 2, 2};
  auto cache = std::make_unique<HipPagedKvCache>(config);
  auto replacement_cache = std::make_unique<HipPagedKvCache>(config);
  Stream stream;
  const HipPagedSequenceHandle sequence = cache->create_sequence();
  const HipPagedSequenceHandle replacement_sequence = replacement_cache->create_sequence();
  const auto [keys, values] = make_token(config, 0);
  cache->append(sequence, keys, values, stream);
  replacement_cache->append(replacement_sequence, keys, values, stream);
  stream.synchronize();

  std::optional<HipPagedKvCache::DecodeView> view;
  view.emplace(cache->read_sequence(sequence));
  HipPagedKvCache::DecodeView moved = std::move(*view);
  EXPECT_THROW(static_cast<void>(view->length()), Error);
  view.reset();
  cache.reset();

  EXPECT_EQ(moved.length(), 1U);
  EXPECT_EQ(moved.physical_blocks().front(), 0U);
  EXPECT_TRUE(moved.layer_key_blocks()[0].device() == kGpu);
  EXPECT_TRUE(moved.block_table().valid());
  // the pool outlives the cache object while the view holds it
  const auto hk = host_values(moved.layer_key_blocks()[0]);
  EXPECT_EQ(hk[2], expected_value(0, 0, 0, 2, true));

  auto replacement = replacement_cache->read_sequence(replacement_sequence);
  replacement_cache.reset();
  moved = std::move(replacement);
  EXPECT_THROW(static_cast<void>(replacement.length()), Error);
  EXPECT_EQ(moved.length(), 1U);
  EXPECT_EQ(moved.physical_blocks().front(), 0U);
}

// tests/cuda_paged_kv_cache_test.cpp:269-293
TEST_F(HipPagedKvCacheTest, DecodeViewSerializesReleaseUntilBorrowedPointersExpire) {
  const PagedKvCacheConfig config{1, 1, 2, 2, 1};
  HipPagedKvCache cache(config);
  Stream stream;
  const HipPagedSequenceHandle sequence = cache.create_sequence();
  const auto [keys, values] = make_token(config, 0);
  cache.append(sequence, keys, values, stream);
  stream.synchronize();

  std::optional<HipPagedKvCache::DecodeView> view;
  view.emplace(cache.read_sequence(sequence));
  std::promise<void> started;
  std::future<void> started_future = started.get_future();
  std::future<void> release = std::async(std::launch::async, [&] {
    started.set_value();
    cache.release_sequence(sequence);
  });
  started_future.wait();
  EXPECT_TRUE(release.wait_for(std::chrono::milliseconds(20)) == std::future_status::timeout);
  view.reset();
  EXPECT_TRUE(release.wait_for(std::chrono::seconds(2)) == std::future_status::ready);
  release.get();
  EXPECT_FALSE(cache.contains(sequence));
  EXPECT_EQ(cache.stats().free_blocks, 1U);
}

// tests/cuda_paged_kv_cache_test.cpp:295-327
TEST_F(HipPagedKvCacheTest, FailedConsumerQuarantinesTableAndPreventsPageReuse) {
  const PagedKvCacheConfig config{1, 1, 2, 2, 1};
  HipPagedKvCache cache(config);
  Stream stream;
  const HipPagedSequenceHandle sequence = cache.create_sequence();
  const auto [keys, values] = make_token(config, 0);
  cache.append(sequence, keys, values, stream);
  stream.synchronize();
  {
    auto view = cache.read_sequence(sequence);
    ASSERT_NE(view.block_table().data(), nullptr);
    view.poison_after_consumer_failure();
    EXPECT_THROW(static_cast<void>(view.length()), Error);
  }
  EXPECT_FALSE(cache.is_healthy());
  EXPECT_TRUE(cache.contains(sequence));
  EXPECT_EQ(cache.length(sequence), 1U);
  expect_error_code([&] { static_cast<void>(cache.create_sequence()); }, ErrorCode::kRuntime);
  expect_error_code([&] { static_cast<void>(cache.read_sequence(sequence)); }, ErrorCode::kRuntime);
  expect_error_code([&] { cache.append(sequence, keys, values, stream); }, ErrorCode::kRuntime);

  cache.release_sequence(sequence);
  EXPECT_FALSE(cache.contains(sequence));
  EXPECT_EQ(cache.stats().used_blocks, 0U);
  EXPECT_EQ(cache.stats().free_blocks, 1U);
  expect_error_code([&] { static_cast<void>(cache.create_sequence()); }, ErrorCode::kRuntime);
}

// Extension: copy-on-write fork at a non-aligned prefix, bulk layer-major
// append and the compact gather, each bit-exact.
TEST_F(HipPagedKvCacheTest, ForkBulkAppendAndGatherAreBitExact) {
  const PagedKvCacheConfig config{2, 2, 8, 4, 16};
  HipPagedKvCache cache(config);
  Stream stream;
  const auto source = cache.create_sequence();
  const std::size_t tokens = 10;
  std::vector<Tensor> lk, lv;
  std::vector<std::vector<float>> hk, hv;
  for (std::size_t l = 0; l < config.layers; ++l) {
    lk.push_back(random_uniform({2, static_cast<Dimension>(tokens), 8}, 100 + l, -1, 1).to(kGpu));
    lv.push_back(random_uniform({2, static_cast<Dimension>(tokens), 8}, 200 + l, -1, 1).to(kGpu));
    hk.push_back(host_values(lk.back()));
    hv.push_back(host_values(lv.back()));
  }
  cache.append_layer_major(source, lk, lv, stream);
  EXPECT_THROW(static_cast<void>(cache.fork_sequence(source, 6, false, stream)), Error);
  const auto child = cache.fork_sequence(source, 6, true, stream);
  EXPECT_EQ(cache.length(child), 6U);
  EXPECT_EQ(cache.stats().shared_blocks, 1U);  // the full first page; the second is copied
  for (std::size_t l = 0; l < config.layers; ++l) {
    Tensor k = Tensor::empty({2, 6, 8}, DType::kFloat32, kGpu);
    Tensor v = Tensor::empty({2, 6, 8}, DType::kFloat32, kGpu);
    cache.copy_layer_out(child, l, k, v, stream);
    stream.synchronize();
    const auto gk = host_values(k), gv = host_values(v);
    for (std::size_t h = 0; h < 2; ++h)
      for (std::size_t t = 0; t < 6; ++t)
        for (std::size_t d = 0; d < 8; ++d) {
          EXPECT_EQ(gk[(h * 6 + t) * 8 + d], hk[l][(h * tokens + t) * 8 + d]);
          EXPECT_EQ(gv[(h * 6 + t) * 8 + d], hv[l][(h * tokens + t) * 8 + d]);
        }
  }
  const auto table = cache.block_table(child);
  const auto source_table = cache.block_table(source);
  ASSERT_EQ(table.size(), 2U);
  EXPECT_EQ(table[0], source_table[0]);
  EXPECT_TRUE(table[1] != source_table[1]);
  cache.release_sequence(child);
  cache.release_sequence(source);
  EXPECT_EQ(cache.stats().used_blocks, 0U);
}

// Extension: bf16 pages.  An appended fp32 value is stored rounded to the
// nearest bf16 (ties to even); the gather widens it back exactly, and the
// read view hands out bf16 pools.
float bf16_round(float x) {
  std::uint32_t u;
  std::memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u && (u & 0x007fffffu) != 0) {
    u |= 0x00400000u;  // NaN stays (quiet) NaN
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
  }
  u &= 0xffff0000u;
  float r;
  std::memcpy(&r, &u, 4);
  return r;
}

TEST_F(HipPagedKvCacheTest, Bf16PagesRoundOnAppendAndWidenOnGather) {
  const PagedKvCacheConfig config{2, 2, 8, 4, 8};
  HipPagedKvCache cache(config, 0, PageDType::kBFloat16);
  Stream stream;
  const auto seq = cache.create_sequence();
  std::vector<std::vector<float>> keys, values;  // per token [L, H, D]
  for (std::size_t t = 0; t < 6; ++t) {
    const Tensor k = random_uniform({2, 2, 8}, 900 + t, -3, 3);
    const Tensor v = random_uniform({2, 2, 8}, 950 + t, -3, 3);
    keys.emplace_back(k.data_as<float>(), k.data_as<float>() + k.numel());
    values.emplace_back(v.data_as<float>(), v.data_as<float>() + v.numel());
    cache.append(seq, k.to(kGpu), v.to(kGpu), stream);
  }
  // 1.00390625 = 1 + 2^-8 lies halfway between bf16 1 and 1 + 2^-7: ties to even.
  const std::vector<float> special(32, 1.00390625F);
  cache.append(seq, Tensor::from_values({2, 2, 8}, special, kGpu),
               Tensor::from_values({2, 2, 8}, special, kGpu), stream);
  keys.push_back(special);
  values.push_back(special);
  stream.synchronize();
  EXPECT_EQ(bf16_round(1.00390625F), 1.0F);
  {
    auto view = cache.read_sequence(seq);
    EXPECT_TRUE(view.layer_key_blocks()[0].dtype() == DType::kBFloat16);
    EXPECT_EQ(view.length(), 7U);
  }
  for (std::size_t l = 0; l < 2; ++l) {
    Tensor gk = Tensor::empty({2, 7, 8}, DType::kFloat32, kGpu);
    Tensor gv = Tensor::empty({2, 7, 8}, DType::kFloat32, kGpu);
    cache.copy_layer_out(seq, l, gk, gv, stream);
    stream.synchronize();
    const auto hk = host_values(gk), hv = host_values(gv);
    for (std::size_t h = 0; h < 2; ++h)
      for (std::size_t t = 0; t < 7; ++t)
        for (std::size_t d = 0; d < 8; ++d) {
          const std::size_t src = (l * 2 + h) * 8 + d;
          EXPECT_EQ(hk[(h * 7 + t) * 8 + d], bf16_round(keys[t][src]));
          EXPECT_EQ(hv[(h * 7 + t) * 8 + d], bf16_round(values[t][src]));
        }
  }
}

// Extension: the prefix index over the device cache (prefix.hpp:77-113).
TEST_F(HipPagedKvCacheTest, PrefixCacheHitForksTheAnchorAndSharesItsPages) {
  const PagedKvCacheConfig config{1, 1, 4, 2, 8};
  auto cache = std::make_shared<HipPagedKvCache>(config);
  HipPagedPrefixCache prefixes(cache, PagedPrefixCacheConfig{4, 16});
  EXPECT_EQ(prefixes.block_tokens(), 2U);
  Stream stream;
  const auto anchor = cache->create_sequence();
  for (std::size_t t = 0; t < 4; ++t) {
    const auto [k, v] = make_token(config, t);
    cache->append(anchor, k, v, stream);
  }
  const std::array<std::uint32_t, 4> tokens{7, 8, 9, 10};
  const PrefixNamespaceId ns(3);
  EXPECT_TRUE(prefixes.insert(ns, tokens, anchor) == PrefixInsertStatus::kInserted);
  EXPECT_TRUE(prefixes.insert(ns, tokens, anchor) == PrefixInsertStatus::kAlreadyPresent);
  const std::array<std::uint32_t, 5> query{7, 8, 9, 10, 11};
  const auto match = prefixes.lookup_longest(ns, query);
  ASSERT_TRUE(match.has_value());
  EXPECT_EQ(match->matched_tokens, 4U);
  EXPECT_EQ(cache->length(match->sequence), 4U);
  EXPECT_TRUE(cache->block_table(match->sequence) == cache->block_table(anchor));
  EXPECT_FALSE(prefixes.lookup_longest(PrefixNamespaceId(4), query).has_value());
  EXPECT_EQ(prefixes.stats().hit_count, 1U);
  EXPECT_EQ(prefixes.stats().miss_count, 1U);
  cache->release_sequence(match->sequence);
  EXPECT_TRUE(prefixes.erase(ns, tokens));
  EXPECT_FALSE(prefixes.contains(ns, tokens));
  stream.synchronize();
}

// ------------------------------------------------------- paged attention ----
// tests/cuda_attention_test.cpp:14-99 helpers
void expect_close(const Tensor& actual_device, const std::vector<float>& expected,
                  float tolerance) {
  const auto actual = host_values(actual_device);
  ASSERT_EQ(actual.size(), expected.size());
  for (std::size_t i = 0; i < expected.size(); ++i) EXPECT_NEAR(actual[i], expected[i], tolerance);
}

Tensor pack_logical_blocks(const Tensor& logical, std::span<const std::uint32_t> block_table,
                           Dimension physical_blocks, Dimension block_tokens, float padding) {
  const auto heads = static_cast<std::size_t>(logical.shape()[0]);
  const auto tokens = static_cast<std::size_t>(logical.shape()[1]);
  const auto width = static_cast<std::size_t>(logical.shape()[2]);
  const auto per_block = static_cast<std::size_t>(block_tokens);
  std::vector<float> packed(static_cast<std::size_t>(physical_blocks) * heads * per_block * width,
                            padding);
  const float* source = logical.data_as<float>();
  for (std::size_t h = 0; h < heads; ++h)
    for (std::size_t t = 0; t < tokens; ++t) {
      const std::size_t physical = block_table[t / per_block];
      for (std::size_t d = 0; d < width; ++d)
        packed[((physical * heads + h) * per_block + t % per_block) * width + d] =
            source[(h * tokens + t) * width + d];
    }
  return Tensor::from_values({physical_blocks, logical.shape()[0], block_tokens, logical.shape()[2]},
                             packed);
}

Tensor concatenate_token_axis(const Tensor& prefix, const Tensor& tail) {
  const auto heads = static_cast<std::size_t>(prefix.shape()[0]);
  const auto np = static_cast<std::size_t>(prefix.shape()[1]);
  const auto nt = static_cast<std::size_t>(tail.shape()[1]);
  const auto width = static_cast<std::size_t>(prefix.shape()[2]);
  Tensor result = Tensor::empty({prefix.shape()[0], prefix.shape()[1] + tail.shape()[1],
                                 prefix.shape()[2]});
  for (std::size_t h = 0; h < heads; ++h) {
    float* dst = result.data<float>() + h * (np + nt) * width;
    std::copy_n(prefix.data_as<float>() + h * np * width, np * width, dst);
    std::copy_n(tail.data_as<float>() + h * nt * width, nt * width, dst + np * width);
  }
  return result;
}

std::vector<std::uint32_t> reversed_block_table(std::size_t logical, std::size_t physical) {
  std::vector<std::uint32_t> r(logical);
  for (std::size_t i = 0; i < logical; ++i) r[i] = static_cast<std::uint32_t>(physical - 1 - i);
  return r;
}

/// The oracle's contiguous SDPA: (output, probabilities).
std::pair<std::vector<float>, std::vector<float>> cpu_sdpa(const Tensor& q, const Tensor& k,
                                                           const Tensor& v, std::size_t offset) {
  const auto h = static_cast<std::size_t>(q.shape()[0]), t = static_cast<std::size_t>(q.shape()[1]);
  const auto keys = static_cast<std::size_t>(k.shape()[1]);
  const auto dk = static_cast<std::size_t>(q.shape()[2]), dv = static_cast<std::size_t>(v.shape()[2]);
  std::vector<float> out(h * t * dv), ws(h * t * keys);
  if (oracle_sdpa(q.data_as<float>(), k.data_as<float>(), v.data_as<float>(), h, t, keys, dk, dv,
                  offset, out.data(), ws.data()) != 0) {
    throw std::runtime_error("oracle_sdpa rejected its inputs");
  }
  return {out, ws};
}

// tests/cuda_attention_test.cpp:196-228
TEST_F(HipAttentionTest, PagedPathMatchesKnownReorderedBlocksAndIgnoresTailPadding) {
  constexpr std::array<std::uint32_t, 2> kBlockTable{2, 0};
  const Tensor query_host = Tensor::from_values({1, 2, 2}, std::array{1.0F, 0.0F, 0.0F, 1.0F});
  const Tensor key_host =
      Tensor::from_values({1, 3, 2}, std::array{1.0F, 0.0F, 0.0F, 1.0F, 1.0F, 1.0F});
  const Tensor value_host = Tensor::from_values(
      {1, 3, 3}, std::array{10.0F, 1.0F, -1.0F, 20.0F, 2.0F, -2.0F, 30.0F, 3.0F, -3.0F});
  const auto [expected_output, expected_probabilities] = cpu_sdpa(query_host, key_host, value_host, 1);
  const Tensor query = query_host.to(kGpu);
  const Tensor key_blocks = pack_logical_blocks(key_host, kBlockTable, 3, 2, 10000.0F).to(kGpu);
  const Tensor value_blocks = pack_logical_blocks(value_host, kBlockTable, 3, 2, -10000.0F).to(kGpu);
  PagedBlockTable block_table(kBlockTable, 3, 0);
  Tensor output = Tensor::empty({1, 2, 3}, DType::kFloat32, kGpu);
  Tensor workspace = Tensor::empty({1, 2, 3}, DType::kFloat32, kGpu);
  Stream stream;
  paged_scaled_dot_product_attention_out(query, key_blocks, value_blocks, block_table, 3, 1,
                                         output, workspace, stream);
  stream.synchronize();
  expect_close(output, expected_output, 2.0e-5F);
  expect_close(workspace, expected_probabilities, 2.0e-6F);
}

// tests/cuda_attention_test.cpp:230-273
TEST_F(HipAttentionTest, PagedPathMatchesCpuAcrossOddPagesHeadsAndWidths) {
  struct Problem {
    Dimension heads, queries, keys, key_dimension, value_dimension, block_tokens;
  };
  constexpr std::array kProblems{Problem{1, 1, 3, 1, 2, 2}, Problem{2, 3, 5, 5, 7, 2},
                                 Problem{3, 7, 11, 37, 41, 4}};
  Stream stream;
  for (const Problem p : kProblems) {
    const auto kv_tokens = static_cast<std::size_t>(p.keys);
    const auto per_block = static_cast<std::size_t>(p.block_tokens);
    const std::size_t logical = 1 + (kv_tokens - 1) / per_block;
    const std::size_t physical = logical + 2;
    const auto table = reversed_block_table(logical, physical);
    const auto offset = static_cast<std::size_t>(p.keys - p.queries);
    const Tensor q = random_uniform({p.heads, p.queries, p.key_dimension}, 8101, -1, 1);
    const Tensor k = random_uniform({p.heads, p.keys, p.key_dimension}, 8102, -1, 1);
    const Tensor v = random_uniform({p.heads, p.keys, p.value_dimension}, 8103, -1, 1);
    const auto expected = cpu_sdpa(q, k, v, offset).first;
    const auto pd = static_cast<Dimension>(physical);
    const Tensor kb = pack_logical_blocks(k, table, pd, p.block_tokens, 77.0F).to(kGpu);
    const Tensor vb = pack_logical_blocks(v, table, pd, p.block_tokens, -77.0F).to(kGpu);
    PagedBlockTable block_table(table, physical, 0);
    const Tensor actual = paged_scaled_dot_product_attention(q.to(kGpu), kb, vb, block_table,
                                                             kv_tokens, offset, stream);
    stream.synchronize();
    expect_close(actual, expected, 2.0e-5F + static_cast<float>(p.key_dimension) * 1.0e-6F);
  }
}

// tests/cuda_attention_test.cpp:275-288
TEST_F(HipAttentionTest, PagedPathAcceptsEmptyQueriesWithoutLaunching) {
  constexpr std::array<std::uint32_t, 3> kBlockTable{3, 1, 0};
  const Tensor query = Tensor::zeros({2, 0, 5}, DType::kFloat32, kGpu);
  const Tensor key_blocks = Tensor::zeros({4, 2, 3, 5}, DType::kFloat32, kGpu);
  const Tensor value_blocks = Tensor::zeros({4, 2, 3, 7}, DType::kFloat32, kGpu);
  PagedBlockTable block_table(kBlockTable, 4, 0);
  Stream stream;
  const Tensor output =
      paged_scaled_dot_product_attention(query, key_blocks, value_blocks, block_table, 7, 7, stream);
  EXPECT_TRUE(output.shape() == (Shape{2, 0, 7}));
  EXPECT_EQ(output.numel(), 0U);
  EXPECT_EQ(paged_score_workspace_bytes(query, key_blocks, block_table, 7), 0U);
}

// tests/cuda_attention_test.cpp:290-374
TEST_F(HipAttentionTest, PagedPathRejectsInvalidTablesGeometryOffsetsAndAliasing) {
  constexpr std::array<std::uint32_t, 2> kBlockIds{2, 0};
  constexpr std::array<std::uint32_t, 1> kShortBlockIds{0};
  constexpr std::array<std::uint32_t, 1> kOutOfRangeBlockId{3};
  const Tensor query = Tensor::zeros({1, 2, 2}, DType::kFloat32, kGpu);
  const Tensor key_blocks = Tensor::zeros({3, 1, 2, 2}, DType::kFloat32, kGpu);
  const Tensor value_blocks = Tensor::zeros({3, 1, 2, 2}, DType::kFloat32, kGpu);
  Tensor output = Tensor::zeros({1, 2, 2}, DType::kFloat32, kGpu);
  Tensor workspace = Tensor::zeros({1, 2, 3}, DType::kFloat32, kGpu);
  Stream stream;

  PagedBlockTable empty_table(std::span<const std::uint32_t>{}, 3, 0);
  EXPECT_TRUE(empty_table.valid());
  EXPECT_TRUE(empty_table.data() == nullptr);
  EXPECT_EQ(empty_table.logical_block_count(), 0U);
  EXPECT_EQ(empty_table.size_bytes(), 0U);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, value_blocks, empty_table, 1, 0, stream)),
               Error);
  EXPECT_THROW(static_cast<void>(PagedBlockTable(std::span<const std::uint32_t>{}, 0, 0)), Error);
  EXPECT_THROW(static_cast<void>(PagedBlockTable(kShortBlockIds, 0, 0)), Error);
  EXPECT_THROW(static_cast<void>(PagedBlockTable(kOutOfRangeBlockId, 3, 0)), Error);
  EXPECT_THROW(static_cast<void>(PagedBlockTable(kShortBlockIds, 3, -1)), Error);

  PagedBlockTable original(kBlockIds, 3, 0);
  PagedBlockTable block_table(std::move(original));
  EXPECT_FALSE(original.valid());
  EXPECT_TRUE(block_table.valid());
  EXPECT_EQ(block_table.logical_block_count(), 2U);
  EXPECT_EQ(block_table.physical_block_count(), 3U);
  EXPECT_EQ(block_table.size_bytes(), 2U * sizeof(std::uint32_t));
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, value_blocks, original, 3, 1, stream)),
               Error);
  PagedBlockTable short_table(kShortBlockIds, 3, 0);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, value_blocks, short_table, 3, 1, stream)),
               Error);
  PagedBlockTable wrong_capacity(kBlockIds, 4, 0);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, value_blocks, wrong_capacity, 3, 1, stream)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, value_blocks, block_table, 0, 0, stream)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, value_blocks, block_table, 3, 2, stream)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   Tensor::zeros({1, 2, 2}), key_blocks, value_blocks, block_table, 3, 1, stream)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, Tensor::zeros({3, 2, 2}, DType::kFloat32, kGpu), value_blocks,
                   block_table, 3, 1, stream)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_scaled_dot_product_attention(
                   query, key_blocks, Tensor::zeros({3, 1, 3, 2}, DType::kFloat32, kGpu),
                   block_table, 3, 1, stream)),
               Error);

  Tensor output_alias = query;
  EXPECT_THROW(paged_scaled_dot_product_attention_out(query, key_blocks, value_blocks, block_table,
                                                      3, 1, output_alias, workspace, stream),
               Error);
  Tensor shared = Tensor::zeros({1, 2, 3}, DType::kFloat32, kGpu);
  const Tensor three_value_blocks = Tensor::zeros({3, 1, 2, 3}, DType::kFloat32, kGpu);
  EXPECT_THROW(paged_scaled_dot_product_attention_out(query, key_blocks, three_value_blocks,
                                                      block_table, 3, 1, shared, shared, stream),
               Error);

  PagedBlockTable reassigned(kShortBlockIds, 3, 0);
  reassigned = std::move(block_table);
  EXPECT_FALSE(block_table.valid());
  EXPECT_TRUE(reassigned.valid());
  EXPECT_NO_THROW(paged_scaled_dot_product_attention_out(query, key_blocks, value_blocks,
                                                         reassigned, 3, 1, output, workspace,
                                                         stream));
  stream.synchronize();
}

// tests/cuda_attention_test.cpp:376-449
TEST_F(HipAttentionTest, PagedTailMatchesCpuForEmptyHistoryOddPagesAndChunkedContinuation) {
  struct Problem {
    Dimension heads, history_tokens, tail_tokens, key_dimension, value_dimension, block_tokens;
  };
  constexpr std::array kProblems{Problem{1, 0, 1, 1, 2, 2}, Problem{2, 3, 1, 5, 7, 2},
                                 Problem{3, 5, 3, 37, 41, 4}};
  Stream stream;
  for (const Problem p : kProblems) {
    const auto history = static_cast<std::size_t>(p.history_tokens);
    const auto per_block = static_cast<std::size_t>(p.block_tokens);
    const std::size_t logical = history == 0 ? 0 : 1 + (history - 1) / per_block;
    const std::size_t physical = logical + 2;
    const auto table = reversed_block_table(logical, physical);
    const Tensor q = random_uniform({p.heads, p.tail_tokens, p.key_dimension}, 8201, -1, 1);
    const Tensor hk = random_uniform({p.heads, p.history_tokens, p.key_dimension}, 8202, -1, 1);
    const Tensor hv = random_uniform({p.heads, p.history_tokens, p.value_dimension}, 8203, -1, 1);
    const Tensor tk = random_uniform({p.heads, p.tail_tokens, p.key_dimension}, 8204, -1, 1);
    const Tensor tv = random_uniform({p.heads, p.tail_tokens, p.value_dimension}, 8205, -1, 1);
    const auto [expected_output, expected_workspace] =
        cpu_sdpa(q, concatenate_token_axis(hk, tk), concatenate_token_axis(hv, tv), history);

    const auto pd = static_cast<Dimension>(physical);
    const Tensor query = q.to(kGpu);
    const Tensor kb = pack_logical_blocks(hk, table, pd, p.block_tokens, 10000.0F).to(kGpu);
    const Tensor vb = pack_logical_blocks(hv, table, pd, p.block_tokens, -10000.0F).to(kGpu);
    const Tensor tail_key = tk.to(kGpu), tail_value = tv.to(kGpu);
    PagedBlockTable block_table(table, physical, 0);
    const Shape ws_shape{p.heads, p.tail_tokens, p.history_tokens + p.tail_tokens};
    Tensor output = Tensor::empty({p.heads, p.tail_tokens, p.value_dimension}, DType::kFloat32, kGpu);
    Tensor workspace = Tensor::empty(ws_shape, DType::kFloat32, kGpu);
    EXPECT_TRUE(paged_tail_score_workspace_shape(query, kb, vb, block_table, history, tail_key,
                                                 tail_value) == ws_shape);
    EXPECT_EQ(paged_tail_score_workspace_bytes(query, kb, vb, block_table, history, tail_key,
                                               tail_value),
              shape_numel(ws_shape) * sizeof(float));
    paged_scaled_dot_product_attention_with_tail_out(query, kb, vb, block_table, history, tail_key,
                                                     tail_value, output, workspace, stream);
    stream.synchronize();
    const float tolerance = 2.0e-5F + static_cast<float>(p.key_dimension) * 1.0e-6F;
    expect_close(output, expected_output, tolerance);
    expect_close(workspace, expected_workspace, 2.0e-6F);
    expect_close(paged_scaled_dot_product_attention_with_tail(query, kb, vb, block_table, history,
                                                              tail_key, tail_value, stream),
                 expected_output, tolerance);
  }
}

// tests/cuda_attention_test.cpp:451-531
TEST_F(HipAttentionTest, PagedTailRejectsInvalidGeometryLifetimeAndAliasesBeforeLaunch) {
  constexpr std::array<std::uint32_t, 2> kBlockIds{2, 0};
  const Tensor query = Tensor::zeros({1, 2, 2}, DType::kFloat32, kGpu);
  const Tensor key_blocks = Tensor::zeros({3, 1, 2, 2}, DType::kFloat32, kGpu);
  const Tensor value_blocks = Tensor::zeros({3, 1, 2, 3}, DType::kFloat32, kGpu);
  const Tensor tail_key = Tensor::zeros({1, 2, 2}, DType::kFloat32, kGpu);
  const Tensor tail_value = Tensor::zeros({1, 2, 3}, DType::kFloat32, kGpu);
  Tensor output = Tensor::zeros({1, 2, 3}, DType::kFloat32, kGpu);
  Tensor workspace = Tensor::zeros({1, 2, 5}, DType::kFloat32, kGpu);
  PagedBlockTable block_table(kBlockIds, 3, 0);
  Stream stream;

  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   query, key_blocks, value_blocks, block_table,
                   std::numeric_limits<std::size_t>::max(), tail_key, tail_value)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   Tensor::zeros({1, 0, 2}, DType::kFloat32, kGpu), key_blocks, value_blocks,
                   block_table, 3, Tensor::zeros({1, 0, 2}, DType::kFloat32, kGpu),
                   Tensor::zeros({1, 0, 3}, DType::kFloat32, kGpu))),
               Error);
  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   query, key_blocks, value_blocks, block_table, 3, Tensor::zeros({2, 2}),
                   tail_value)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   query, key_blocks, value_blocks, block_table, 3,
                   Tensor::zeros({1, 1, 2}, DType::kFloat32, kGpu), tail_value)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   query, key_blocks, value_blocks, block_table, 3,
                   Tensor::zeros({1, 2, 3}, DType::kFloat32, kGpu), tail_value)),
               Error);
  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   query, key_blocks, value_blocks, block_table, 3, tail_key,
                   Tensor::zeros({1, 2, 4}, DType::kFloat32, kGpu))),
               Error);
  EXPECT_THROW(static_cast<void>(paged_tail_score_workspace_shape(
                   query, key_blocks, value_blocks, block_table, 3,
                   Tensor::zeros({1, 2, 2}, DType::kUInt32, kGpu), tail_value)),
               Error);

  Tensor output_alias = tail_value;
  EXPECT_THROW(paged_scaled_dot_product_attention_with_tail_out(
                   query, key_blocks, value_blocks, block_table, 3, tail_key, tail_value,
                   output_alias, workspace, stream),
               Error);
  Tensor workspace_alias = tail_key;
  EXPECT_THROW(paged_scaled_dot_product_attention_with_tail_out(
                   query, key_blocks, value_blocks, block_table, 3, tail_key, tail_value, output,
                   workspace_alias, stream),
               Error);
  EXPECT_THROW(paged_scaled_dot_product_attention_with_tail_out(query, key_blocks, value_blocks,
                                                                block_table, 3, tail_key,
                                                                tail_value, output, output, stream),
               Error);

  // A tail value and an output that overlap by half inside one allocation.
  Tensor allocation = Tensor::zeros({192}, DType::kFloat32, kGpu);
  const Tensor wide_value_blocks = Tensor::zeros({3, 1, 2, 64}, DType::kFloat32, kGpu);
  const Tensor partial_tail_value =
      Tensor::borrow(allocation.raw(), {1, 2, 64}, DType::kFloat32, kGpu);
  Tensor partial_output = Tensor::borrow(allocation.data<float>() + 64, {1, 2, 64},
                                         DType::kFloat32, kGpu);
  EXPECT_THROW(paged_scaled_dot_product_attention_with_tail_out(
                   query, key_blocks, wide_value_blocks, block_table, 3, tail_key,
                   partial_tail_value, partial_output, workspace, stream),
               Error);

  Stream active_stream = std::move(stream);
  EXPECT_THROW(paged_scaled_dot_product_attention_with_tail_out(query, key_blocks, value_blocks,
                                                                block_table, 3, tail_key,
                                                                tail_value, output, workspace,
                                                                stream),
               Error);
  EXPECT_NO_THROW(paged_scaled_dot_product_attention_with_tail_out(
      query, key_blocks, value_blocks, block_table, 3, tail_key, tail_value, output, workspace,
      active_stream));
  active_stream.synchronize();
}

// tests/cuda_attention_test.cpp:533-556
TEST_F(HipAttentionTest, PagedTailCausalMaskDoesNotReadFutureNonFiniteValue) {
  const float nan = std::numeric_limits<float>::quiet_NaN();
  const Tensor query = Tensor::zeros({1, 2, 1}, DType::kFloat32, kGpu);
  const Tensor key_blocks = Tensor::zeros({1, 1, 2, 1}, DType::kFloat32, kGpu);
  const Tensor value_blocks = Tensor::zeros({1, 1, 2, 1}, DType::kFloat32, kGpu);
  const Tensor tail_key = Tensor::from_values({1, 2, 1}, std::array{0.0F, nan}, kGpu);
  const Tensor tail_value = Tensor::from_values({1, 2, 1}, std::array{3.0F, nan}, kGpu);
  Tensor output = Tensor::empty({1, 2, 1}, DType::kFloat32, kGpu);
  Tensor workspace = Tensor::empty({1, 2, 2}, DType::kFloat32, kGpu);
  PagedBlockTable block_table(std::span<const std::uint32_t>{}, 1, 0);
  Stream stream;
  paged_scaled_dot_product_attention_with_tail_out(query, key_blocks, value_blocks, block_table, 0,
                                                   tail_key, tail_value, output, workspace, stream);
  stream.synchronize();
  const auto out = host_values(output);
  const auto ws = host_values(workspace);
  EXPECT_FLOAT_EQ(out[0], 3.0F);
  EXPECT_TRUE(std::isnan(out[1]));
  EXPECT_FLOAT_EQ(ws[0], 1.0F);
  EXPECT_FLOAT_EQ(ws[1], 0.0F);
}

// ---------------------------------------------------------- decode batch ----
// Extension: batched GQA decode through DecodeBatch, checked against the
// oracle's per-sequence paged attention (2e-5 abs + 1e-4 rel), then the
// step's rows committed and gathered back bit-exactly; the next step uses
// the fused append + attention launch.
TEST_F(HipDecodeBatchTest, GqaDecodeStepsMatchOracleAndCommitBitExactly) {
  constexpr std::size_t L = 2, H = 2, HQ = 8, D = 128, P = 16, B = 4;
  const PagedKvCacheConfig config{L, H, D, P, 64};
  HipPagedKvCache cache(config);
  Stream stream;
  const std::array<std::size_t, B> lengths{0, 1, 16, 45};
  std::vector<HipPagedSequenceHandle> seqs;
  // per (sequence, layer): host copies of the whole history [H, len, D]
  std::vector<std::vector<std::vector<float>>> hist_k(B), hist_v(B);
  for (std::size_t b = 0; b < B; ++b) {
    seqs.push_back(cache.create_sequence());
    const auto n = static_cast<Dimension>(lengths[b]);
    std::vector<Tensor> lk, lv;
    for (std::size_t l = 0; l < L; ++l) {
      lk.push_back(random_uniform({H, n, D}, 1000 + 10 * b + l, -1, 1));
      lv.push_back(random_uniform({H, n, D}, 2000 + 10 * b + l, -1, 1));
      hist_k[b].emplace_back(lk.back().data_as<float>(), lk.back().data_as<float>() + lk.back().numel());
      hist_v[b].emplace_back(lv.back().data_as<float>(), lv.back().data_as<float>() + lv.back().numel());
      lk.back() = lk.back().to(kGpu);
      lv.back() = lv.back().to(kGpu);
    }
    if (n != 0) cache.append_layer_major(seqs.back(), lk, lv, stream);
  }
  stream.synchronize();
  DecodeBatch batch(cache, seqs, HQ, 64);
  EXPECT_EQ(batch.batch(), B);

  for (int step = 0; step < 2; ++step) {
    batch.prepare(stream);
    std::vector<Tensor> outputs;
    std::vector<std::vector<float>> q_host(L), k_host(L), v_host(L);
    std::vector<Tensor> k_step, v_step;
    for (std::size_t l = 0; l < L; ++l) {
      const Tensor q = random_uniform({B, HQ, D}, 5000 + 10 * step + l, -1, 1);
      const Tensor k = random_uniform({B, H, D}, 6000 + 10 * step + l, -1, 1);
      const Tensor v = random_uniform({B, H, D}, 7000 + 10 * step + l, -1, 1);
      q_host[l].assign(q.data_as<float>(), q.data_as<float>() + q.numel());
      k_host[l].assign(k.data_as<float>(), k.data_as<float>() + k.numel());
      v_host[l].assign(v.data_as<float>(), v.data_as<float>() + v.numel());
      Tensor out = Tensor::empty({B, HQ, D}, DType::kFloat32, kGpu);
      k_step.push_back(k.to(kGpu));
      v_step.push_back(v.to(kGpu));
      if (step == 0) {
        batch.attention_layer(l, q.to(kGpu), k_step[l], v_step[l], out, stream);
        batch.append_layer(l, k_step[l], v_step[l], stream);
      } else {
        batch.append_attention_layer(l, q.to(kGpu), k_step[l], v_step[l], out, stream);
      }
      outputs.push_back(out);
    }
    stream.synchronize();
    // Oracle: a compact pool per sequence, identity tables.
    for (std::size_t l = 0; l < L; ++l) {
      const auto actual = host_values(outputs[l]);
      for (std::size_t b = 0; b < B; ++b) {
        const std::size_t n = lengths[b] + static_cast<std::size_t>(step);
        const std::size_t pages = std::max<std::size_t>(1, (n + P - 1) / P);
        std::vector<float> kb(pages * H * P * D, 0.0F), vb(pages * H * P * D, 0.0F);
        for (std::size_t h = 0; h < H; ++h)
          for (std::size_t t = 0; t < n; ++t)
            for (std::size_t d = 0; d < D; ++d) {
              const std::size_t dst = (((t / P) * H + h) * P + t % P) * D + d;
              kb[dst] = hist_k[b][l][(h * n + t) * D + d];
              vb[dst] = hist_v[b][l][(h * n + t) * D + d];
            }
        std::vector<std::uint32_t> table(pages);
        std::iota(table.begin(), table.end(), 0U);
        const std::int32_t len = static_cast<std::int32_t>(n);
        std::vector<float> expected(HQ * D);
        oracle_batched_decode(q_host[l].data() + b * HQ * D, 1, HQ, H, D, kb.data(), vb.data(), P,
                              table.data(), pages, &len, k_host[l].data() + b * H * D,
                              v_host[l].data() + b * H * D, expected.data(), 1);
        for (std::size_t i = 0; i < HQ * D; ++i) {
          const float a = actual[b * HQ * D + i], e = expected[i];
          EXPECT_TRUE(std::fabs(a - e) <= 2.0e-5F + 1.0e-4F * std::fabs(e));
        }
      }
    }
    // Fold the step's rows into the host history, then check the gather.
    for (std::size_t b = 0; b < B; ++b) {
      const std::size_t n = lengths[b] + static_cast<std::size_t>(step);
      for (std::size_t l = 0; l < L; ++l)
        for (auto* pair : {&hist_k, &hist_v}) {
          const auto& step_rows = pair == &hist_k ? k_host[l] : v_host[l];
          std::vector<float> grown(H * (n + 1) * D);
          for (std::size_t h = 0; h < H; ++h) {
            std::copy_n((*pair)[b][l].data() + h * n * D, n * D, grown.data() + h * (n + 1) * D);
            std::copy_n(step_rows.data() + (b * H + h) * D, D, grown.data() + (h * (n + 1) + n) * D);
          }
          (*pair)[b][l] = std::move(grown);
        }
      EXPECT_EQ(cache.length(seqs[b]), n + 1);
      for (std::size_t l = 0; l < L; ++l) {
        Tensor gk = Tensor::empty({H, static_cast<Dimension>(n + 1), D}, DType::kFloat32, kGpu);
        Tensor gv = Tensor::empty({H, static_cast<Dimension>(n + 1), D}, DType::kFloat32, kGpu);
        cache.copy_layer_out(seqs[b], l, gk, gv, stream);
        stream.synchronize();
        EXPECT_TRUE(host_values(gk) == hist_k[b][l]);
        EXPECT_TRUE(host_values(gv) == hist_v[b][l]);
      }
    }
  }
  // Shape contracts are checked before any launch.
  Tensor wrong = Tensor::empty({B, HQ, D}, DType::kFloat32, kGpu);
  EXPECT_THROW(batch.append_layer(0, wrong, wrong, stream), Error);
  Tensor rows = Tensor::empty({B, H, D}, DType::kFloat32, kGpu);
  EXPECT_THROW(batch.attention_layer(L, wrong, rows, rows, wrong, stream), Error);
}

// Extension: a chunked-prefill step through DecodeBatch (prepare_chunk, the
// chunk rows appended per layer, prefill attention over the pages plus the
// causal chunk) against the oracle's paged attention with a T-token tail,
// the chunk gathered back bit-exactly, then a decode step's RoPE at each
// sequence's position (bit-exact against fp32 arithmetic with every product
// and sum rounded on its own, cpu::rope_out, src/kernels/cpu/reference.cpp:490-533).
TEST_F(HipDecodeBatchTest, ChunkStepMatchesOracleAndDecodeRopeUsesPositions) {
  constexpr std::size_t L = 2, H = 2, HQ = 8, D = 128, P = 16, B = 3, T = 24;
  const PagedKvCacheConfig config{L, H, D, P, 48};
  HipPagedKvCache cache(config);
  Stream stream;
  const std::array<std::size_t, B> hist{0, 5, 37};
  std::vector<HipPagedSequenceHandle> seqs;
  std::vector<std::vector<std::vector<float>>> hk(B), hv(B);  // [b][l] -> [H, n, D]
  for (std::size_t b = 0; b < B; ++b) {
    seqs.push_back(cache.create_sequence());
    const auto n = static_cast<Dimension>(hist[b]);
    std::vector<Tensor> lk, lv;
    for (std::size_t l = 0; l < L; ++l) {
      const Tensor k = random_uniform({H, n, D}, 300 + 10 * b + l, -1, 1);
      const Tensor v = random_uniform({H, n, D}, 400 + 10 * b + l, -1, 1);
      hk[b].emplace_back(k.data_as<float>(), k.data_as<float>() + k.numel());
      hv[b].emplace_back(v.data_as<float>(), v.data_as<float>() + v.numel());
      lk.push_back(k.to(kGpu));
      lv.push_back(v.to(kGpu));
    }
    if (n != 0) cache.append_layer_major(seqs.back(), lk, lv, stream);
  }
  DecodeBatch batch(cache, seqs, HQ, 96);
  batch.prepare_chunk(T, stream);
  for (std::size_t l = 0; l < L; ++l) {
    const Tensor q = random_uniform({B, HQ, T, D}, 500 + l, -1, 1);
    const Tensor ck = random_uniform({B, H, T, D}, 600 + l, -1, 1);
    const Tensor cv = random_uniform({B, H, T, D}, 700 + l, -1, 1);
    const Tensor dk = ck.to(kGpu), dv = cv.to(kGpu);
    Tensor out = Tensor::empty({B, HQ, T, D}, DType::kFloat32, kGpu);
    EXPECT_THROW(batch.append_layer(l, random_uniform({B, H, D}, 1, -1, 1).to(kGpu),
                                    random_uniform({B, H, D}, 2, -1, 1).to(kGpu), stream),
                 Error);  // decode-step rows after prepare_chunk
    batch.append_layer(l, dk, dv, stream);
    batch.prefill_layer(l, q.to(kGpu), dk, dv, out, stream);
    stream.synchronize();
    const auto got = host_values(out);
    for (std::size_t b = 0; b < B; ++b) {
      const std::size_t n = hist[b];
      const std::size_t pages = std::max<std::size_t>(1, (n + P - 1) / P);
      std::vector<float> kb(pages * H * P * D, 0.0F), vb(pages * H * P * D, 0.0F);
      for (std::size_t h = 0; h < H; ++h)
        for (std::size_t t = 0; t < n; ++t)
          for (std::size_t d = 0; d < D; ++d) {
            const std::size_t dst = (((t / P) * H + h) * P + t % P) * D + d;
            kb[dst] = hk[b][l][(h * n + t) * D + d];
            vb[dst] = hv[b][l][(h * n + t) * D + d];
          }
      std::vector<std::uint32_t> table(pages);
      std::iota(table.begin(), table.end(), 0U);
      std::vector<float> want(HQ * T * D), ws(HQ * T * (n + T));
      ASSERT_EQ(oracle_paged_attention(q.data_as<float>() + b * HQ * T * D, HQ, H, T, D, D,
                                       kb.data(), vb.data(), P, table.data(), n,
                                       ck.data_as<float>() + b * H * T * D,
                                       cv.data_as<float>() + b * H * T * D, T, n, want.data(),
                                       ws.data()),
                0);
      for (std::size_t i = 0; i < want.size(); ++i) {
        const float a = got[b * HQ * T * D + i], e = want[i];
        EXPECT_TRUE(std::fabs(a - e) <= 2.0e-5F + 1.0e-4F * std::fabs(e));
      }
      // Fold the chunk into the host history of this layer.
      for (auto* pair : {&hk, &hv}) {
        const float* rows = (pair == &hk ? ck : cv).data_as<float>() + b * H * T * D;
        std::vector<float> grown(H * (n + T) * D);
        for (std::size_t h = 0; h < H; ++h) {
          std::copy_n((*pair)[b][l].data() + h * n * D, n * D, grown.data() + h * (n + T) * D);
          std::copy_n(rows + h * T * D, T * D, grown.data() + (h * (n + T) + n) * D);
        }
        (*pair)[b][l] = std::move(grown);
      }
    }
  }
  for (std::size_t b = 0; b < B; ++b) {
    const std::size_t n = hist[b] + T;
    EXPECT_EQ(cache.length(seqs[b]), n);
    for (std::size_t l = 0; l < L; ++l) {
      Tensor gk = Tensor::empty({H, static_cast<Dimension>(n), D}, DType::kFloat32, kGpu);
      Tensor gv = Tensor::empty({H, static_cast<Dimension>(n), D}, DType::kFloat32, kGpu);
      cache.copy_layer_out(seqs[b], l, gk, gv, stream);
      stream.synchronize();
      EXPECT_TRUE(host_values(gk) == hk[b][l]);
      EXPECT_TRUE(host_values(gv) == hv[b][l]);
    }
  }

  // Decode step: RoPE of the step's query and key at each sequence's length.
  batch.prepare(stream);
  constexpr std::size_t kRows = 96;
  const Tensor cosine = random_uniform({kRows, D / 2}, 801, -1, 1);
  const Tensor sine = random_uniform({kRows, D / 2}, 802, -1, 1);
  const Tensor qh = random_uniform({B, HQ, D}, 803, -2, 2);
  const Tensor kh = random_uniform({B, H, D}, 804, -2, 2);
  Tensor qd = qh.to(kGpu), kd = kh.to(kGpu);
  batch.rope(qd, kd, cosine.to(kGpu), sine.to(kGpu), stream);
  stream.synchronize();
  const auto gq = host_values(qd), gk = host_values(kd);
  auto check_rope = [&](const Tensor& x, const std::vector<float>& got, std::size_t heads) {
    for (std::size_t b = 0; b < B; ++b) {
      const std::size_t pos = hist[b] + T;
      for (std::size_t h = 0; h < heads; ++h)
        for (std::size_t i = 0; i < D / 2; ++i) {
          const std::size_t o = (b * heads + h) * D + 2 * i;
          const float x0 = x.data_as<float>()[o], x1 = x.data_as<float>()[o + 1];
          const float c = cosine.data_as<float>()[pos * (D / 2) + i];
          const float sn = sine.data_as<float>()[pos * (D / 2) + i];
          const float a = x0 * c, bb = x1 * sn, cc = x0 * sn, dd = x1 * c;
          EXPECT_EQ(got[o], a - bb);
          EXPECT_EQ(got[o + 1], cc + dd);
        }
    }
  };
  check_rope(qh, gq, HQ);
  check_rope(kh, gk, H);
}

}  // namespace

int main(int argc, char** argv) {
  return mini_test::run_all(argc > 1 ? argv[1] : nullptr);
}
