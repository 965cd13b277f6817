// C++ API tests of libhelix_paged through include/helix_paged.hpp.
//
// The reference's own expectations enter as data: the fixtures under
// tests/golden/ (the paged-cache scenarios and attention known answers that
// tests/golden/make_fixtures.py transcribed from the reference's tests, the
// same files the Python suites replay) are replayed here through the C++
// API.  Everything else is this repository's own checking: seeded random
// operation programs against the CPU oracle's pool, a table of invalid
// calls that must fail before any launch, the read lease, seeded attention
// sweeps against the oracle, the single-sequence decode route of the decode entry
// point, and the extensions (copy-on-write fork, bulk append, bf16 pages,
// the prefix cache, DecodeBatch decode and chunk steps).
//
// The oracle (oracle/liboracle.so) is linked as the checker only.  Built by
// tests/cpp/Makefile; run by tests/test_gpu_cpp_api.py on a GPU.  Without a
// GPU the host-contract cases run and every GPU case reports SKIPPED (the CPU
// suite runs the binary that way).

#include "helix_paged.hpp"
#include "json_lite.hpp"
#include "mini_test.hpp"

#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <array>
#include <chrono>
#include <cstring>
#include <future>
#include <limits>
#include <map>
#include <numeric>
#include <random>
#include <thread>
#include <type_traits>

extern "C" {
void* oracle_pool_create(std::size_t layers, std::size_t kv_heads, std::size_t head_dim,
                         std::size_t block_tokens, std::size_t physical_blocks, int* status);
void oracle_pool_destroy(void* pool);
std::uint64_t oracle_create_sequence(void* pool);
int oracle_fork_sequence(void* pool, std::uint64_t source, std::size_t prefix, int allow_cow,
                         std::uint64_t* out);
int oracle_append(void* pool, std::uint64_t seq, const float* keys, const float* values);
int oracle_append_layer_major(void* pool, std::uint64_t seq, const float* keys,
                              const float* values, std::size_t tokens);
int oracle_release_sequence(void* pool, std::uint64_t seq);
std::size_t oracle_length(void* pool, std::uint64_t seq);
std::size_t oracle_block_table(void* pool, std::uint64_t seq, std::uint32_t* out,
                               std::size_t capacity);
void oracle_stats(void* pool, helix_paged_stats* out);
int oracle_copy_layer(void* pool, std::uint64_t seq, std::size_t layer, float* keys_out,
                      float* values_out, std::size_t dest_tokens);
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
namespace attn = helix_amd::attention::hip;
using PagedBlockTable = helix_amd::kv_cache::hip::PagedBlockTable;
using Stream = helix_amd::hip::Stream;
using json_lite::Value;

// The lease and table types keep the reference's ownership rules: neither is
// copyable, both move without throwing, poisoning cannot throw, and the
// reference's CUDA spelling names the same class.
static_assert(!std::is_copy_constructible_v<HipPagedKvCache::DecodeView>);
static_assert(std::is_nothrow_move_constructible_v<HipPagedKvCache::DecodeView>);
static_assert(
    noexcept(std::declval<HipPagedKvCache::DecodeView&>().poison_after_consumer_failure()));
static_assert(!std::is_copy_constructible_v<PagedBlockTable>);
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
struct GoldenReplayTest : GpuFixture {};
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

// The ErrorCode a call throws, or nullopt when it returns normally.
std::optional<ErrorCode> thrown_code(const std::function<void()>& call) {
  try {
    call();
  } catch (const Error& e) {
    return e.code();
  }
  return std::nullopt;
}

// tests/golden/<name>, found from this binary's location (tests/cpp/).
std::string golden_path(const char* name) {
  std::vector<char> buf(4096, '\0');
  const ssize_t n = readlink("/proc/self/exe", buf.data(), buf.size() - 1);
  std::string exe = n > 0 ? std::string(buf.data(), static_cast<std::size_t>(n)) : "";
  const auto cut = exe.rfind("/cpp/");
  return (cut == std::string::npos ? std::string("tests") : exe.substr(0, cut)) + "/golden/" +
         name;
}

// ------------------------------------------ host contracts (no GPU needed) ----
// Every C status maps to the reference's ErrorCode (status = code + 1,
// include/helix/core/error.hpp:10-17) with the library's message.
TEST_F(HostContractTest, EveryStatusMapsToItsErrorCode) {
  const std::array<std::pair<int, std::string_view>, 6> table{{{HELIX_INVALID_ARGUMENT, "InvalidArgument"},
                                                               {HELIX_OUT_OF_RANGE, "OutOfRange"},
                                                               {HELIX_UNSUPPORTED, "Unsupported"},
                                                               {HELIX_RESOURCE_EXHAUSTED, "ResourceExhausted"},
                                                               {HELIX_RUNTIME, "Runtime"},
                                                               {HELIX_INTERNAL, "Internal"}}};
  for (const auto& [status, name] : table) {
    const auto code = thrown_code([status = status] { helix_amd::detail::check(status); });
    ASSERT_TRUE(code.has_value());
    EXPECT_EQ(static_cast<int>(*code) + 1, status);
    EXPECT_TRUE(error_code_name(*code) == name);
  }
  EXPECT_FALSE(thrown_code([] { helix_amd::detail::check(HELIX_OK); }).has_value());
  // Unknown statuses are internal errors.
  EXPECT_TRUE(thrown_code([] { helix_amd::detail::check(99); }) == ErrorCode::kInternal);
}

// Validation that runs before any device work: tables checked against the
// pool size, cache configurations, handles and host tensors.
TEST_F(HostContractTest, InvalidArgumentsFailBeforeDeviceWork) {
  const std::vector<std::uint32_t> ids{0, 5, 2};
  struct Row {
    const char* what;
    std::function<void()> call;
    ErrorCode code;
  };
  const std::vector<Row> rows{
      {"empty table of an empty pool", [] { PagedBlockTable t(std::span<const std::uint32_t>{}, 0, 0); },
       ErrorCode::kInvalidArgument},
      {"page id past the pool", [&] { PagedBlockTable t(ids, 5, 0); }, ErrorCode::kOutOfRange},
      {"negative device", [&] { PagedBlockTable t(ids, 6, -1); }, ErrorCode::kInvalidArgument},
      {"zero layers", [] { HipPagedKvCache c(PagedKvCacheConfig{0, 1, 1, 1, 1}); },
       ErrorCode::kInvalidArgument},
      {"zero page tokens", [] { HipPagedKvCache c(PagedKvCacheConfig{1, 1, 1, 0, 1}); },
       ErrorCode::kInvalidArgument},
      {"negative device index", [] { HipPagedKvCache c(PagedKvCacheConfig{1, 1, 1, 1, 1}, -1); },
       ErrorCode::kInvalidArgument},
      {"fp8 scales on bf16 pages",
       [] {
         HipPagedKvCache c(PagedKvCacheConfig{1, 1, 1, 1, 1}, 0, PageDType::kBFloat16,
                           Fp8Scales{2.0F, 1.0F});
       },
       ErrorCode::kInvalidArgument},
      {"zero fp8 key scale",
       [] {
         HipPagedKvCache c(PagedKvCacheConfig{1, 1, 1, 1, 1}, 0, PageDType::kFp8E4M3,
                           Fp8Scales{0.0F, 1.0F});
       },
       ErrorCode::kInvalidArgument},
      {"infinite fp8 value scale",
       [] {
         HipPagedKvCache c(PagedKvCacheConfig{1, 1, 1, 1, 1}, 0, PageDType::kFp8E4M3,
                           Fp8Scales{1.0F, std::numeric_limits<float>::infinity()});
       },
       ErrorCode::kInvalidArgument},
      {"reshape changing the count",
       [] { static_cast<void>(Tensor::zeros({2, 3}).reshape({4, 2})); },
       ErrorCode::kInvalidArgument},
      {"values not matching the shape",
       [] { static_cast<void>(Tensor::from_values({2, 2}, std::array{1.F, 2.F, 3.F})); },
       ErrorCode::kInvalidArgument},
  };
  for (const Row& r : rows) {
    const auto code = thrown_code(r.call);
    if (!code.has_value() || *code != r.code) {
      ::mini_test::fail(__FILE__, __LINE__, std::string("wrong outcome: ") + r.what);
    }
  }
  const Tensor t = Tensor::from_values({2, 3}, std::array{1.F, 2.F, 3.F, 4.F, 5.F, 6.F});
  EXPECT_TRUE(t.reshape({3, 2}).data_as<float>() == t.data_as<float>());  // shared storage
  EXPECT_EQ(Tensor::zeros({0, 5}).numel(), 0U);
  EXPECT_FALSE(static_cast<bool>(HipPagedSequenceHandle{}));
}

#include "host_programs.hpp"

// ------------------------------------------------ golden fixture replay ----
// tests/golden/paged_cache_scenarios.json: op programs with the reference's
// expected tables, page contents, lengths, errors and statistics.
struct ScenarioReplay {
  explicit ScenarioReplay(const Value& scenario)
      : config{scenario["config"][0].index(), scenario["config"][1].index(),
               scenario["config"][2].index(), scenario["config"][3].index(),
               scenario["config"][4].index()},
        cache(config) {}

  // token(base)[l, h, c] = base + flat index
  Tensor encoded_token(double base) const {
    std::vector<float> v(config.layers * config.kv_heads * config.head_dimension);
    for (std::size_t i = 0; i < v.size(); ++i) v[i] = static_cast<float>(base + static_cast<double>(i));
    return Tensor::from_values(shape3(config.layers, config.kv_heads, config.head_dimension), v,
                               kGpu);
  }
  // layer l of a bulk append: [H, count, D] with base + (begin + t) * 100 +
  // (l * H + h) * D + c
  std::vector<Tensor> encoded_layers(std::size_t begin, std::size_t count, double base) const {
    std::vector<Tensor> out;
    for (std::size_t l = 0; l < config.layers; ++l) {
      std::vector<float> v(config.kv_heads * count * config.head_dimension);
      for (std::size_t h = 0; h < config.kv_heads; ++h)
        for (std::size_t t = 0; t < count; ++t)
          for (std::size_t c = 0; c < config.head_dimension; ++c)
            v[(h * count + t) * config.head_dimension + c] = static_cast<float>(
                base + static_cast<double>((begin + t) * 100 +
                                           (l * config.kv_heads + h) * config.head_dimension + c));
      out.push_back(Tensor::from_values(shape3(config.kv_heads, count, config.head_dimension), v,
                                        kGpu));
    }
    return out;
  }
  static Shape shape3(std::size_t a, std::size_t b, std::size_t c) {
    return {static_cast<Dimension>(a), static_cast<Dimension>(b), static_cast<Dimension>(c)};
  }
  std::pair<std::vector<float>, std::vector<float>> layer(const std::string& seq, std::size_t l) {
    const std::size_t n = cache.length(seqs.at(seq));
    Tensor k = Tensor::empty(shape3(config.kv_heads, n, config.head_dimension), DType::kFloat32, kGpu);
    Tensor v = Tensor::empty(shape3(config.kv_heads, n, config.head_dimension), DType::kFloat32, kGpu);
    cache.copy_layer_out(seqs.at(seq), l, k, v, stream);
    stream.synchronize();
    return {host_values(k), host_values(v)};
  }
  std::size_t stat(const std::string& name) const {
    const PagedKvCacheStats s = cache.stats();
    const std::map<std::string, std::size_t> all{
        {"bytes_reserved", s.bytes_reserved}, {"bytes_used", s.bytes_used},
        {"bytes_free", s.bytes_free}, {"peak_bytes_used", s.peak_bytes_used},
        {"total_blocks", s.total_blocks}, {"used_blocks", s.used_blocks},
        {"free_blocks", s.free_blocks}, {"active_sequence_count", s.active_sequence_count},
        {"active_tokens", s.active_tokens}, {"resident_tokens", s.resident_tokens},
        {"allocated_token_slots", s.allocated_token_slots},
        {"block_reference_count", s.block_reference_count}, {"shared_blocks", s.shared_blocks},
        {"sequence_create_count", s.sequence_create_count},
        {"sequence_fork_count", s.sequence_fork_count}, {"append_count", s.append_count},
        {"release_count", s.release_count}, {"block_allocation_count", s.block_allocation_count},
        {"block_reuse_count", s.block_reuse_count}};
    return all.at(name);
  }

  void run(const Value& op) {
    const std::string& kind = op["op"].str();
    auto seq = [&](const char* key = "seq") -> const HipPagedSequenceHandle& {
      return seqs.at(op[key].str());
    };
    if (kind == "create") {
      seqs[op["seq"].str()] = cache.create_sequence();
    } else if (kind == "append_encoded") {
      cache.append(seq(), encoded_token(op["key_base"].num()), encoded_token(op["value_base"].num()),
                   stream);
    } else if (kind == "append_values") {
      const auto s3 = shape3(config.layers, config.kv_heads, config.head_dimension);
      cache.append(seq(), Tensor::from_values(s3, op["keys"].floats(), kGpu),
                   Tensor::from_values(s3, op["values"].floats(), kGpu), stream);
    } else if (kind == "append_layer_major_encoded") {
      const std::size_t begin = op["token_begin"].index(), count = op["count"].index();
      cache.append_layer_major(seq(), encoded_layers(begin, count, op["key_base"].num()),
                               encoded_layers(begin, count, op["value_base"].num()), stream);
    } else if (kind == "fork") {
      seqs[op["new"].str()] = cache.fork_sequence(seq(), op["prefix"].index(), false, stream);
    } else if (kind == "release") {
      cache.release_sequence(seq());
    } else if (kind == "expect_error") {
      const auto code = thrown_code([&] { run(op["inner"]); });
      ASSERT_TRUE(code.has_value());
      const std::string& want = op["status"].str();
      if (want != "any") {
        const std::map<std::string, ErrorCode> names{
            {"invalid_argument", ErrorCode::kInvalidArgument},
            {"out_of_range", ErrorCode::kOutOfRange},
            {"resource_exhausted", ErrorCode::kResourceExhausted}};
        EXPECT_TRUE(*code == names.at(want));
      }
    } else if (kind == "expect_table") {
      const auto want = op["table"].indices();
      const auto got = cache.block_table(seq());
      EXPECT_TRUE(std::vector<std::size_t>(got.begin(), got.end()) == want);
    } else if (kind == "expect_table_size") {
      EXPECT_EQ(cache.block_table(seq()).size(), op["size"].index());
    } else if (kind == "expect_table_last") {
      EXPECT_EQ(cache.block_table(seq()).back(), op["block"].index());
    } else if (kind == "expect_tables_share") {
      const auto a = cache.block_table(seqs.at(op["a"].str()));
      const auto b = cache.block_table(seqs.at(op["b"].str()));
      const std::size_t n = op["count"].index();
      ASSERT_TRUE(a.size() >= n && b.size() >= n);
      EXPECT_TRUE(std::equal(a.begin(), a.begin() + static_cast<std::ptrdiff_t>(n), b.begin()));
    } else if (kind == "expect_tables_differ_at") {
      const std::size_t i = op["index"].index();
      EXPECT_TRUE(cache.block_table(seqs.at(op["a"].str()))[i] !=
                  cache.block_table(seqs.at(op["b"].str()))[i]);
    } else if (kind == "expect_length") {
      EXPECT_EQ(cache.length(seq()), op["length"].index());
    } else if (kind == "expect_layer") {
      const auto [k, v] = layer(op["seq"].str(), op["layer"].index());
      EXPECT_TRUE(k == op["keys"].floats());
      EXPECT_TRUE(v == op["values"].floats());
    } else if (kind == "expect_layer_element") {
      const auto [k, v] = layer(op["seq"].str(), op["layer"].index());
      const std::size_t i = op["index"].index();
      EXPECT_EQ(k.at(i), static_cast<float>(op["key"].num()));
      EXPECT_EQ(v.at(i), static_cast<float>(op["value"].num()));
    } else if (kind == "expect_stats") {
      for (const auto& [name, value] : op["stats"].members) {
        if (stat(name) != value.index()) {
          ::mini_test::fail(__FILE__, __LINE__, "statistic " + name + " differs");
        }
      }
    } else {
      FAIL("unknown fixture op " + kind);
    }
  }

  PagedKvCacheConfig config;
  HipPagedKvCache cache;
  Stream stream;
  std::map<std::string, HipPagedSequenceHandle> seqs;
};

TEST_F(GoldenReplayTest, PagedCacheScenariosReproduceEveryExpectation) {
  const Value scenarios = json_lite::load(golden_path("paged_cache_scenarios.json"));
  ASSERT_TRUE(scenarios.size() >= 7);
  for (const Value& scenario : scenarios.items) {
    std::printf("  scenario: %s\n", scenario["name"].str().c_str());
    ScenarioReplay replay(scenario);
    for (const Value& op : scenario["ops"].items) replay.run(op);
  }
}

// tests/golden/attention_known_answers.json: the reference's closed-form
// attention cases (outputs and probabilities), through the history-only
// entry point and, where the queries are the last keys, through the tail
// entry point with the probability contract.
TEST_F(GoldenReplayTest, AttentionKnownAnswersThroughBothEntryPoints) {
  const Value cases = json_lite::load(golden_path("attention_known_answers.json"));
  ASSERT_TRUE(cases.size() >= 3);
  Stream stream;
  for (const Value& c : cases.items) {
    std::printf("  case: %s\n", c["name"].str().c_str());
    const Value& q = c["query"];
    const Value& k = c["keys"];
    const Value& v = c["values"];
    const std::size_t nq = q.size(), nk = k.size(), dk = q[0].size(), dv = v[0].size();
    const std::size_t bt = c["block_tokens"].index(), phys = c["physical_blocks"].index();
    const std::vector<std::size_t> table_idx = c["table"].indices();
    const std::vector<std::uint32_t> table(table_idx.begin(), table_idx.end());
    auto flat = [](const Value& rows) {
      std::vector<float> out;
      for (const Value& r : rows.items)
        for (float x : r.floats()) out.push_back(x);
      return out;
    };
    const std::vector<float> qf = flat(q), kf = flat(k), vf = flat(v);
    const std::vector<float> want_out = flat(c["output"]), want_p = flat(c["probabilities"]);
    auto pack = [&](const std::vector<float>& rows, std::size_t width, float padding) {
      std::vector<float> pool(phys * bt * width, padding);
      for (std::size_t t = 0; t < nk; ++t)
        std::copy_n(rows.data() + t * width, width, pool.data() + (table[t / bt] * bt + t % bt) * width);
      return Tensor::from_values({static_cast<Dimension>(phys), 1, static_cast<Dimension>(bt),
                                  static_cast<Dimension>(width)},
                                 pool, kGpu);
    };
    const Tensor kp = pack(kf, dk, static_cast<float>(c["key_padding"].num()));
    const Tensor vp = pack(vf, dv, static_cast<float>(c["value_padding"].num()));
    const PagedBlockTable bt_dev(table, phys, 0);
    const Tensor query = Tensor::from_values(
        {1, static_cast<Dimension>(nq), static_cast<Dimension>(dk)}, qf, kGpu);
    Tensor out = Tensor::empty({1, static_cast<Dimension>(nq), static_cast<Dimension>(dv)},
                               DType::kFloat32, kGpu);
    Tensor ws = Tensor::empty({1, static_cast<Dimension>(nq), static_cast<Dimension>(nk)},
                              DType::kFloat32, kGpu);
    attn::paged_scaled_dot_product_attention_out(query, kp, vp, bt_dev, nk, c["offset"].index(),
                                                 out, ws, stream);
    stream.synchronize();
    auto expect_all = [](const std::vector<float>& got, const std::vector<float>& want, float tol) {
      ASSERT_EQ(got.size(), want.size());
      for (std::size_t i = 0; i < want.size(); ++i) EXPECT_NEAR(got[i], want[i], tol);
    };
    expect_all(host_values(out), want_out, 2e-5F);
    expect_all(host_values(ws), want_p, 2e-6F);
    const std::size_t hist = nk - nq;
    if (c["offset"].index() == hist) {
      const Tensor tk = Tensor::from_values(
          {1, static_cast<Dimension>(nq), static_cast<Dimension>(dk)},
          std::vector<float>(kf.begin() + static_cast<std::ptrdiff_t>(hist * dk), kf.end()), kGpu);
      const Tensor tv = Tensor::from_values(
          {1, static_cast<Dimension>(nq), static_cast<Dimension>(dv)},
          std::vector<float>(vf.begin() + static_cast<std::ptrdiff_t>(hist * dv), vf.end()), kGpu);
      std::vector<std::uint32_t> hist_table(table.begin(),
                                            table.begin() + static_cast<std::ptrdiff_t>((hist + bt - 1) / bt));
      const PagedBlockTable ht(hist_table, phys, 0);
      Tensor out2 = Tensor::empty(out.shape(), DType::kFloat32, kGpu);
      Tensor ws2 = Tensor::empty(ws.shape(), DType::kFloat32, kGpu);
      attn::paged_scaled_dot_product_attention_with_tail_probabilities_out(
          query, kp, vp, ht, hist, tk, tv, out2, ws2, stream);
      stream.synchronize();
      expect_all(host_values(out2), want_out, 2e-5F);
      expect_all(host_values(ws2), want_p, 2e-6F);
    }
  }
}

// ------------------------------------------- random programs vs the oracle ----
// Seeded random programs of create / one-token append / bulk append /
// aligned and copy-on-write forks / releases run on the device cache and on
// the oracle pool side by side: every call succeeds or fails on both with
// the same code, and the tables, lengths, statistics and gathered pages stay
// equal throughout.
class OraclePool {
 public:
  OraclePool(std::size_t l, std::size_t h, std::size_t d, std::size_t p, std::size_t n) {
    int status = 0;
    pool_ = oracle_pool_create(l, h, d, p, n, &status);
    if (status != 0) throw std::runtime_error("oracle pool");
  }
  ~OraclePool() { oracle_pool_destroy(pool_); }
  OraclePool(const OraclePool&) = delete;
  OraclePool& operator=(const OraclePool&) = delete;
  [[nodiscard]] void* get() const { return pool_; }

 private:
  void* pool_ = nullptr;
};

// Oracle status (0 ok, else ErrorCode + 1) -> the code the library throws.
std::optional<ErrorCode> oracle_code(int status) {
  if (status == 0) return std::nullopt;
  return static_cast<ErrorCode>(status - 1);
}

TEST_F(HipPagedKvCacheTest, RandomProgramsMatchTheOraclePool) {
  constexpr std::size_t L = 2, H = 2, D = 8, P = 4, N = 40;
  for (std::uint64_t seed : {11U, 12U, 13U}) {
    std::mt19937_64 rng(seed);
    auto pick = [&](std::size_t n) { return static_cast<std::size_t>(rng() % n); };
    HipPagedKvCache cache(PagedKvCacheConfig{L, H, D, P, N});
    OraclePool pool(L, H, D, P, N);
    Stream stream;
    struct Live {
      HipPagedSequenceHandle mine;
      std::uint64_t theirs;
    };
    std::vector<Live> live;
    std::uniform_real_distribution<float> value(-4.0F, 4.0F);
    auto rows = [&](std::size_t n) {
      std::vector<float> v(n);
      for (float& x : v) x = value(rng);
      return v;
    };
    for (int step = 0; step < 160; ++step) {
      const std::size_t what = live.empty() ? 0 : pick(10);
      std::optional<ErrorCode> mine, theirs;
      if (what == 0) {
        live.push_back({cache.create_sequence(), oracle_create_sequence(pool.get())});
      } else if (what <= 3) {  // one token
        Live& s = live[pick(live.size())];
        const auto k = rows(L * H * D), v = rows(L * H * D);
        mine = thrown_code([&] {
          cache.append(s.mine, Tensor::from_values({L, H, D}, k, kGpu),
                       Tensor::from_values({L, H, D}, v, kGpu), stream);
        });
        theirs = oracle_code(oracle_append(pool.get(), s.theirs, k.data(), v.data()));
      } else if (what <= 5) {  // bulk, [L, H, T, D] on the oracle side
        Live& s = live[pick(live.size())];
        const std::size_t t = 1 + pick(11);
        const auto k = rows(L * H * t * D), v = rows(L * H * t * D);
        std::vector<Tensor> lk, lv;
        for (std::size_t l = 0; l < L; ++l) {
          const auto first = static_cast<std::ptrdiff_t>(l * H * t * D);
          const auto last = first + static_cast<std::ptrdiff_t>(H * t * D);
          lk.push_back(Tensor::from_values({H, static_cast<Dimension>(t), D},
                                           std::vector<float>(k.begin() + first, k.begin() + last), kGpu));
          lv.push_back(Tensor::from_values({H, static_cast<Dimension>(t), D},
                                           std::vector<float>(v.begin() + first, v.begin() + last), kGpu));
        }
        mine = thrown_code([&] { cache.append_layer_major(s.mine, lk, lv, stream); });
        theirs = oracle_code(oracle_append_layer_major(pool.get(), s.theirs, k.data(), v.data(), t));
      } else if (what <= 7) {  // fork at an aligned or (with copy-on-write) any prefix
        Live& s = live[pick(live.size())];
        const std::size_t len = cache.length(s.mine);
        const bool cow = pick(2) == 1;
        const std::size_t prefix = len == 0 ? 0 : (cow ? 1 + pick(len) : P * pick(len / P + 1));
        HipPagedSequenceHandle child;
        std::uint64_t other = 0;
        mine = thrown_code([&] { child = cache.fork_sequence(s.mine, prefix, cow, stream); });
        theirs = oracle_code(oracle_fork_sequence(pool.get(), s.theirs, prefix, cow ? 1 : 0, &other));
        if (!mine && !theirs) live.push_back({child, other});
      } else {  // release
        const std::size_t i = pick(live.size());
        cache.release_sequence(live[i].mine);
        ASSERT_EQ(oracle_release_sequence(pool.get(), live[i].theirs), 0);
        live.erase(live.begin() + static_cast<std::ptrdiff_t>(i));
      }
      if (mine != theirs) {
        ::mini_test::fail(__FILE__, __LINE__,
                          "seed " + std::to_string(seed) + " step " + std::to_string(step) +
                              ": library and oracle disagree on success");
        return;
      }
      helix_paged_stats want{};
      oracle_stats(pool.get(), &want);
      const PagedKvCacheStats got = cache.stats();
      EXPECT_EQ(got.used_blocks, want.used_blocks);
      EXPECT_EQ(got.block_reference_count, want.block_reference_count);
      EXPECT_EQ(got.shared_blocks, want.shared_blocks);
      EXPECT_EQ(got.active_tokens, want.active_tokens);
      EXPECT_EQ(got.block_reuse_count, want.block_reuse_count);
      EXPECT_EQ(got.peak_bytes_used, want.peak_bytes_used);
      for (const Live& s : live) {
        std::vector<std::uint32_t> t(N);
        t.resize(oracle_block_table(pool.get(), s.theirs, t.data(), t.size()));
        EXPECT_TRUE(cache.block_table(s.mine) == t);
        EXPECT_EQ(cache.length(s.mine), oracle_length(pool.get(), s.theirs));
      }
      if (step % 20 != 19) continue;
      for (const Live& s : live) {
        const std::size_t n = cache.length(s.mine);
        for (std::size_t l = 0; l < L; ++l) {
          Tensor k = Tensor::empty({H, static_cast<Dimension>(n), D}, DType::kFloat32, kGpu);
          Tensor v = Tensor::empty({H, static_cast<Dimension>(n), D}, DType::kFloat32, kGpu);
          cache.copy_layer_out(s.mine, l, k, v, stream);
          std::vector<float> wk(H * n * D), wv(H * n * D);
          ASSERT_EQ(oracle_copy_layer(pool.get(), s.theirs, l, wk.data(), wv.data(), n), 0);
          EXPECT_TRUE(host_values(k) == wk);
          EXPECT_TRUE(host_values(v) == wv);
        }
      }
    }
  }
}

// ----------------------------------------------------------- read lease ----
// A read view holds the cache: a release issued on another thread waits
// until the view is gone, and a consumer that poisons its view leaves the
// cache unhealthy (every later mutation fails with kRuntime) while the
// view's table and pools stay allocated.
TEST_F(HipPagedKvCacheTest, ReadLeaseDefersMutationsAndPoisonQuarantines) {
  const PagedKvCacheConfig config{1, 2, 4, 2, 6};
  HipPagedKvCache cache(config);
  Stream stream;
  const auto seq = cache.create_sequence();
  const Tensor row = Tensor::zeros({1, 2, 4}, DType::kFloat32, kGpu);
  for (int i = 0; i < 3; ++i) cache.append(seq, row, row, stream);
  auto view = std::make_unique<HipPagedKvCache::DecodeView>(cache.read_sequence(seq));
  EXPECT_EQ(view->length(), 3U);
  EXPECT_EQ(view->physical_blocks().size(), 2U);
  auto released = std::async(std::launch::async, [&] { cache.release_sequence(seq); });
  EXPECT_TRUE(released.wait_for(std::chrono::milliseconds(200)) == std::future_status::timeout);
  view.reset();
  EXPECT_TRUE(released.wait_for(std::chrono::seconds(10)) == std::future_status::ready);
  released.get();
  EXPECT_EQ(cache.stats().used_blocks, 0U);

  const auto other = cache.create_sequence();
  cache.append(other, row, row, stream);
  auto moved = cache.read_sequence(other);
  auto lease = std::move(moved);  // the moved-from view no longer answers
  EXPECT_TRUE(thrown_code([&] { static_cast<void>(moved.length()); }) == ErrorCode::kInvalidArgument);
  const float* pool = lease.layer_key_blocks()[0].data_as<float>();
  lease.poison_after_consumer_failure();
  EXPECT_FALSE(cache.is_healthy());
  EXPECT_TRUE(thrown_code([&] { cache.append(other, row, row, stream); }) == ErrorCode::kRuntime);
  EXPECT_TRUE(thrown_code([&] { static_cast<void>(lease.length()); }) == ErrorCode::kInvalidArgument);
  EXPECT_TRUE(pool != nullptr);
}

// The device cache under contention: four threads, each on its own stream,
// append encoded tokens to their own sequences, fork a shared source and
// release; the cache serialises every call, and afterwards every sequence's
// pages hold exactly its own tokens, bit for bit, with the statistics and
// the free pool consistent.
TEST_F(HipPagedKvCacheTest, ConcurrentAppendsForksAndReleasesStayExact) {
  constexpr std::size_t L = 2, H = 2, D = 8, P = 4;
  HipPagedKvCache cache(PagedKvCacheConfig{L, H, D, P, 128});
  Stream setup;
  const auto source = cache.create_sequence();
  auto token = [&](float base) {
    std::vector<float> v(L * H * D);
    for (std::size_t i = 0; i < v.size(); ++i) v[i] = base + static_cast<float>(i);
    return Tensor::from_values({L, H, D}, v, kGpu);
  };
  for (int t = 0; t < 8; ++t) {
    const Tensor k = token(1000.0F * static_cast<float>(t));
    cache.append(source, k, k, setup);
  }
  constexpr int kThreads = 4, kTokens = 20;
  std::vector<HipPagedSequenceHandle> own(kThreads), forks(kThreads);
  std::vector<std::string> errors(kThreads);
  std::vector<std::thread> threads;
  for (int t = 0; t < kThreads; ++t) {
    threads.emplace_back([&, t] {
      try {
        Stream stream;
        own[t] = cache.create_sequence();
        forks[t] = cache.fork_sequence(source, 8, false, stream);
        for (int i = 0; i < kTokens; ++i) {
          const float base = 100000.0F * static_cast<float>(t + 1) + 100.0F * static_cast<float>(i);
          const Tensor k = token(base);
          cache.append(own[t], k, k, stream);
          cache.append(forks[t], k, k, stream);
          if (i == kTokens / 2) {
            const auto scratch = cache.fork_sequence(forks[t], 8, false, stream);
            cache.release_sequence(scratch);
          }
        }
      } catch (const std::exception& e) {
        errors[t] = e.what();
      }
    });
  }
  for (auto& th : threads) th.join();
  for (const auto& e : errors) EXPECT_TRUE(e.empty());
  for (int t = 0; t < kThreads; ++t) {
    for (const auto* seq : {&own[t], &forks[t]}) {
      const bool forked = seq == &forks[t];
      const std::size_t n = (forked ? 8 : 0) + kTokens;
      ASSERT_EQ(cache.length(*seq), n);
      Tensor k = Tensor::empty({H, static_cast<Dimension>(n), D}, DType::kFloat32, kGpu);
      Tensor v = Tensor::empty({H, static_cast<Dimension>(n), D}, DType::kFloat32, kGpu);
      cache.copy_layer_out(*seq, 1, k, v, setup);
      const auto got = host_values(k);
      for (std::size_t h = 0; h < H; ++h)
        for (std::size_t i = 0; i < n; ++i)
          for (std::size_t c = 0; c < D; ++c) {
            const float base = forked && i < 8 ? 1000.0F * static_cast<float>(i)
                                               : 100000.0F * static_cast<float>(t + 1) +
                                                     100.0F * static_cast<float>(i - (forked ? 8 : 0));
            EXPECT_EQ(got[(h * n + i) * D + c], base + static_cast<float>((1 * H + h) * D + c));
          }
    }
  }
  const PagedKvCacheStats st = cache.stats();
  EXPECT_EQ(st.active_sequence_count, 1U + 2U * kThreads);
  EXPECT_EQ(st.shared_blocks, 2U);  // the source's two pages, held by every fork
  for (int t = 0; t < kThreads; ++t) {
    cache.release_sequence(own[t]);
    cache.release_sequence(forks[t]);
  }
  cache.release_sequence(source);
  EXPECT_EQ(cache.stats().used_blocks, 0U);
}

// ------------------------------------------------------------ extensions ----
// Extension: a copy-on-write fork at a non-aligned prefix shares the full
// pages and copies the partial one; the child's gather equals the source's
// first tokens bit for bit.
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

// Extension: fp8 E4M3 pages with a key and a value scale.  The expected
// value of x is the nearest code of x / scale (ties to the even code,
// saturating at 448) decoded and times the scale, found here by search over
// the format's value table.
float fp8_expected(float x, float scale) {
  const float y = x / scale;
  double best = 0.0;
  int best_code = 0;
  const double a = std::fabs(static_cast<double>(y));
  for (int c = 0; c < 127; ++c) {  // non-negative finite codes, increasing
    const int e = c >> 3, m = c & 7;
    const double v = e == 0 ? m * std::ldexp(1.0, -9) : (1.0 + m / 8.0) * std::ldexp(1.0, e - 7);
    const double d = std::fabs(v - std::min(a, 448.0));
    const double db = std::fabs(best - std::min(a, 448.0));
    if (c == 0 || d < db || (d == db && (c & 1) == 0)) {
      best = v;
      best_code = c;
    }
  }
  static_cast<void>(best_code);
  const float mag = static_cast<float>(best);
  return (std::signbit(y) ? -mag : mag) * scale;
}

TEST_F(HipPagedKvCacheTest, Fp8PagesRoundOnAppendAndWidenOnGather) {
  const PagedKvCacheConfig config{2, 2, 8, 4, 8};
  const Fp8Scales scales{0.05F, 0.02F};
  HipPagedKvCache cache(config, 0, PageDType::kFp8E4M3, scales);
  Stream stream;
  const auto seq = cache.create_sequence();
  std::vector<std::vector<float>> keys, values;  // per token [L, H, D]
  for (std::size_t t = 0; t < 6; ++t) {
    const Tensor k = random_uniform({2, 2, 8}, 1900 + t, -3, 3);
    const Tensor v = random_uniform({2, 2, 8}, 1950 + t, -3, 3);
    keys.emplace_back(k.data_as<float>(), k.data_as<float>() + k.numel());
    values.emplace_back(v.data_as<float>(), v.data_as<float>() + v.numel());
    cache.append(seq, k.to(kGpu), v.to(kGpu), stream);
  }
  // Past the largest code: saturates to 448 * scale.
  const std::vector<float> big(32, 1e6F);
  cache.append(seq, Tensor::from_values({2, 2, 8}, big, kGpu),
               Tensor::from_values({2, 2, 8}, big, kGpu), stream);
  keys.push_back(big);
  values.push_back(big);
  stream.synchronize();
  EXPECT_EQ(fp8_expected(1e6F, 0.05F), 448.0F * 0.05F);
  {
    auto view = cache.read_sequence(seq);
    EXPECT_TRUE(view.layer_key_blocks()[0].dtype() == DType::kFp8E4M3);
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
          EXPECT_EQ(hk[(h * 7 + t) * 8 + d], fp8_expected(keys[t][src], scales.key));
          EXPECT_EQ(hv[(h * 7 + t) * 8 + d], fp8_expected(values[t][src], scales.value));
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
    cache->append(anchor, random_uniform({1, 1, 4}, 60 + t, -1, 1).to(kGpu),
                  random_uniform({1, 1, 4}, 70 + t, -1, 1).to(kGpu), stream);
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
// A seeded paged problem: logical K/V [H, keys, width] scattered over a pool
// of `physical` pages through a permuted table, unused slots filled with a
// large padding value that a wrong index would pick up.
struct PagedProblem {
  std::size_t heads, queries, dk, dv, bt, history, tail, physical;
  std::vector<std::uint32_t> table;
  Tensor query, key_pool, value_pool, tail_key, tail_value;  // host
};

PagedProblem make_problem(std::uint64_t seed, std::size_t heads, std::size_t queries,
                          std::size_t dk, std::size_t dv, std::size_t bt, std::size_t history,
                          std::size_t tail) {
  PagedProblem p{heads, queries, dk, dv, bt, history, tail, 0, {}, {}, {}, {}, {}, {}};
  const std::size_t logical = (history + bt - 1) / bt;
  p.physical = logical + 3;
  std::vector<std::uint32_t> perm(p.physical);
  std::iota(perm.begin(), perm.end(), 0U);
  std::mt19937_64 rng(seed);
  std::shuffle(perm.begin(), perm.end(), rng);
  p.table.assign(perm.begin(), perm.begin() + static_cast<std::ptrdiff_t>(logical));
  const auto H = static_cast<Dimension>(heads);
  p.query = random_uniform({H, static_cast<Dimension>(queries), static_cast<Dimension>(dk)},
                           seed * 10 + 1, -1, 1);
  auto pool = [&](std::size_t width, std::uint64_t s, float padding) {
    const Tensor logical_rows = random_uniform(
        {H, static_cast<Dimension>(history), static_cast<Dimension>(width)}, s, -1, 1);
    std::vector<float> v(p.physical * heads * bt * width, padding);
    for (std::size_t h = 0; h < heads; ++h)
      for (std::size_t t = 0; t < history; ++t)
        std::copy_n(logical_rows.data_as<float>() + (h * history + t) * width, width,
                    v.data() + ((p.table[t / bt] * heads + h) * bt + t % bt) * width);
    return Tensor::from_values({static_cast<Dimension>(p.physical), H,
                                static_cast<Dimension>(bt), static_cast<Dimension>(width)},
                               v);
  };
  p.key_pool = pool(dk, seed * 10 + 2, 9000.0F);
  p.value_pool = pool(dv, seed * 10 + 3, -9000.0F);
  p.tail_key = random_uniform({H, static_cast<Dimension>(tail), static_cast<Dimension>(dk)},
                              seed * 10 + 4, -1, 1);
  p.tail_value = random_uniform({H, static_cast<Dimension>(tail), static_cast<Dimension>(dv)},
                                seed * 10 + 5, -1, 1);
  return p;
}

// Seeded sweep over odd geometries (head and value widths not multiples of
// anything, pages of 1..7 tokens, empty histories, several tail rows): the
// tail entry point with the probability contract and the history-only entry
// point with a query offset both match the oracle (outputs within
// 2e-5 + D * 1e-6, probabilities within 2e-6).
TEST_F(HipAttentionTest, SeededOddGeometriesMatchTheOracle) {
  std::mt19937_64 rng(2024);
  Stream stream;
  for (int trial = 0; trial < 16; ++trial) {
    auto in = [&](std::size_t lo, std::size_t hi) { return lo + rng() % (hi - lo + 1); };
    const std::size_t heads = in(1, 4), dk = in(1, 48), dv = in(1, 48), bt = in(1, 7);
    const std::size_t history = trial % 4 == 0 ? 0 : in(1, 60), tail = in(1, 5);
    const PagedProblem p = make_problem(500 + trial, heads, tail, dk, dv, bt, history, tail);
    const float tol = 2.0e-5F + static_cast<float>(dk) * 1.0e-6F;
    const PagedBlockTable table(p.table, p.physical, 0);
    const Tensor q = p.query.to(kGpu), kp = p.key_pool.to(kGpu), vp = p.value_pool.to(kGpu);
    // Tail form.
    {
      Tensor out = Tensor::empty({static_cast<Dimension>(heads), static_cast<Dimension>(tail),
                                  static_cast<Dimension>(dv)}, DType::kFloat32, kGpu);
      Tensor ws = Tensor::empty(attn::paged_tail_score_workspace_shape(
                                    q, kp, vp, table, history, p.tail_key.to(kGpu),
                                    p.tail_value.to(kGpu)),
                                DType::kFloat32, kGpu);
      attn::paged_scaled_dot_product_attention_with_tail_probabilities_out(
          q, kp, vp, table, history, p.tail_key.to(kGpu), p.tail_value.to(kGpu), out, ws, stream);
      stream.synchronize();
      std::vector<float> want(heads * tail * dv), want_ws(heads * tail * (history + tail));
      ASSERT_EQ(oracle_paged_attention(p.query.data_as<float>(), heads, heads, tail, dk, dv,
                                       p.key_pool.data_as<float>(), p.value_pool.data_as<float>(),
                                       bt, p.table.data(), history, p.tail_key.data_as<float>(),
                                       p.tail_value.data_as<float>(), tail, history, want.data(),
                                       want_ws.data()),
                0);
      const auto got = host_values(out), got_ws = host_values(ws);
      for (std::size_t i = 0; i < want.size(); ++i) EXPECT_NEAR(got[i], want[i], tol);
      for (std::size_t i = 0; i < want_ws.size(); ++i) EXPECT_NEAR(got_ws[i], want_ws[i], 2e-6F);
    }
    // History-only form: the last `tail` history keys are the queries' own.
    if (history >= tail) {
      const std::size_t offset = history - tail;
      Tensor out = Tensor::empty({static_cast<Dimension>(heads), static_cast<Dimension>(tail),
                                  static_cast<Dimension>(dv)}, DType::kFloat32, kGpu);
      Tensor ws = Tensor::empty({static_cast<Dimension>(heads), static_cast<Dimension>(tail),
                                 static_cast<Dimension>(history)}, DType::kFloat32, kGpu);
      attn::paged_scaled_dot_product_attention_out(q, kp, vp, table, history, offset, out, ws,
                                                   stream);
      stream.synchronize();
      std::vector<float> want(heads * tail * dv), want_ws(heads * tail * history);
      ASSERT_EQ(oracle_paged_attention(p.query.data_as<float>(), heads, heads, tail, dk, dv,
                                       p.key_pool.data_as<float>(), p.value_pool.data_as<float>(),
                                       bt, p.table.data(), history, nullptr, nullptr, 0, offset,
                                       want.data(), want_ws.data()),
                0);
      const auto got = host_values(out), got_ws = host_values(ws);
      for (std::size_t i = 0; i < want.size(); ++i) EXPECT_NEAR(got[i], want[i], tol);
      for (std::size_t i = 0; i < want_ws.size(); ++i) EXPECT_NEAR(got_ws[i], want_ws[i], 2e-6F);
    }
  }
}

// Every invalid call of the reference-shaped entry points fails with the
// reference's error code before anything is launched: the output, whose
// sentinel value no kernel would write, is untouched afterwards.  Each row
// changes one thing of a valid call.
TEST_F(HipAttentionTest, InvalidCallsFailBeforeLaunch) {
  const PagedProblem p = make_problem(77, 2, 1, 4, 3, 2, 5, 1);
  Stream stream;
  const PagedBlockTable table(p.table, p.physical, 0);
  const PagedBlockTable short_table(std::span<const std::uint32_t>(p.table).first(2), p.physical, 0);
  const Tensor q = p.query.to(kGpu), kp = p.key_pool.to(kGpu), vp = p.value_pool.to(kGpu);
  const Tensor tk = p.tail_key.to(kGpu), tv = p.tail_value.to(kGpu);
  const std::vector<float> sentinel(2 * 1 * 3, 12345.0F);
  Tensor out = Tensor::from_values({2, 1, 3}, sentinel, kGpu);
  Tensor ws = Tensor::empty({2, 1, 6}, DType::kFloat32, kGpu);
  const Tensor host_q = p.query;
  const Tensor wide_q = random_uniform({2, 1, 5}, 3, -1, 1).to(kGpu);
  const Tensor three_heads = random_uniform({3, 1, 4}, 4, -1, 1).to(kGpu);
  Tensor small_ws = Tensor::empty({2, 1, 5}, DType::kFloat32, kGpu);
  Tensor wrong_out = Tensor::empty({2, 1, 4}, DType::kFloat32, kGpu);
  struct Row {
    const char* what;
    std::function<void()> call;
    ErrorCode code;
  };
  auto tail = [&](const Tensor& query, const PagedBlockTable& t, std::size_t hist, Tensor& o,
                  Tensor& w) {
    attn::paged_scaled_dot_product_attention_with_tail_out(query, kp, vp, t, hist, tk, tv, o, w,
                                                           stream);
  };
  const std::vector<Row> rows{
      {"table shorter than the history", [&] { tail(q, short_table, 5, out, ws); },
       ErrorCode::kInvalidArgument},
      {"history beyond the table", [&] { tail(q, table, 7, out, ws); }, ErrorCode::kInvalidArgument},
      {"query on the host", [&] { tail(host_q, table, 5, out, ws); }, ErrorCode::kInvalidArgument},
      {"query width differs from the keys", [&] { tail(wide_q, table, 5, out, ws); },
       ErrorCode::kInvalidArgument},
      {"query heads not a multiple of kv heads", [&] { tail(three_heads, table, 5, out, ws); },
       ErrorCode::kInvalidArgument},
      {"workspace of the wrong length", [&] { tail(q, table, 5, out, small_ws); },
       ErrorCode::kInvalidArgument},
      {"output of the wrong width", [&] { tail(q, table, 5, wrong_out, ws); },
       ErrorCode::kInvalidArgument},
      {"output aliasing the workspace",
       [&] {
         Tensor alias = ws.reshape({12}).reshape({2, 1, 6});
         Tensor o = Tensor::borrow(alias.raw(), {2, 1, 3}, DType::kFloat32, kGpu);
         tail(q, table, 5, o, ws);
       },
       ErrorCode::kInvalidArgument},
      {"history-only offset past the keys",
       [&] {
         Tensor w5 = Tensor::empty({2, 1, 5}, DType::kFloat32, kGpu);
         attn::paged_scaled_dot_product_attention_out(q, kp, vp, table, 5, 5, out, w5, stream);
       },
       ErrorCode::kInvalidArgument},
  };
  for (const Row& r : rows) {
    const auto code = thrown_code(r.call);
    if (!code.has_value() || *code != r.code) {
      ::mini_test::fail(__FILE__, __LINE__, std::string("wrong outcome: ") + r.what);
    }
  }
  stream.synchronize();
  EXPECT_TRUE(host_values(out) == sentinel);
  // Empty queries are valid and launch nothing.
  Tensor empty_out = Tensor::empty({2, 0, 3}, DType::kFloat32, kGpu);
  Tensor empty_ws = Tensor::empty({2, 0, 5}, DType::kFloat32, kGpu);
  EXPECT_NO_THROW(attn::paged_scaled_dot_product_attention_out(
      Tensor::empty({2, 0, 4}, DType::kFloat32, kGpu), kp, vp, table, 5, 0, empty_out, empty_ws,
      stream));
}

// A non-finite value in a tail row that a query row masks causally must not
// reach that row (the reference skips masked keys; 0 * NaN would not).
TEST_F(HipAttentionTest, MaskedNonFiniteTailRowsDoNotLeak) {
  const PagedProblem p = make_problem(91, 1, 3, 4, 4, 2, 3, 3);
  std::vector<float> tv(p.tail_value.data_as<float>(), p.tail_value.data_as<float>() + 12);
  std::vector<float> tk(p.tail_key.data_as<float>(), p.tail_key.data_as<float>() + 12);
  for (int c = 0; c < 4; ++c) {
    tv[2 * 4 + c] = std::numeric_limits<float>::quiet_NaN();  // row 2: seen by query 2 only
    tk[1 * 4 + c] = std::numeric_limits<float>::infinity();   // row 1: +inf scores from query 1 on
  }
  Stream stream;
  const PagedBlockTable table(p.table, p.physical, 0);
  Tensor out = Tensor::empty({1, 3, 4}, DType::kFloat32, kGpu);
  Tensor ws = Tensor::empty({1, 3, 6}, DType::kFloat32, kGpu);
  attn::paged_scaled_dot_product_attention_with_tail_probabilities_out(
      p.query.to(kGpu), p.key_pool.to(kGpu), p.value_pool.to(kGpu), table, 3,
      Tensor::from_values({1, 3, 4}, tk, kGpu), Tensor::from_values({1, 3, 4}, tv, kGpu), out, ws,
      stream);
  stream.synchronize();
  std::vector<float> want(12), want_ws(18);
  ASSERT_EQ(oracle_paged_attention(p.query.data_as<float>(), 1, 1, 3, 4, 4,
                                   p.key_pool.data_as<float>(), p.value_pool.data_as<float>(), 2,
                                   p.table.data(), 3, tk.data(), tv.data(), 3, 3, want.data(),
                                   want_ws.data()),
            0);
  const auto got = host_values(out);
  for (std::size_t i = 0; i < 12; ++i) {
    EXPECT_EQ(std::isnan(got[i]), std::isnan(want[i]));
    if (!std::isnan(want[i])) EXPECT_NEAR(got[i], want[i], 2e-5F);
  }
  for (std::size_t i = 0; i < 4; ++i) EXPECT_FALSE(std::isnan(got[i]));  // query 0
}

// The model's per-layer call at head_dim 128 and 16-token pages runs the
// single-sequence decode kernel; its output matches the oracle within the
// north-star tolerance and its score workspace holds the same probabilities
// as the exact scalar route's (the reference's workspace contract, within
// the reference test's 2e-6), for MHA and GQA.
TEST_F(HipAttentionTest, DecodeCallsTakeTheSingleSequenceRoute) {
  Stream stream;
  for (const auto& [hkv, group, history] :
       std::vector<std::array<std::size_t, 3>>{{8, 4, 1500}, {4, 1, 700}, {2, 8, 3000}}) {
    const std::size_t hq = hkv * group;
    std::mt19937_64 rng(history);
    const std::size_t logical = (history + 15) / 16, physical = logical + 2;
    std::vector<std::uint32_t> perm(physical);
    std::iota(perm.begin(), perm.end(), 0U);
    std::shuffle(perm.begin(), perm.end(), rng);
    const std::vector<std::uint32_t> ids(perm.begin(), perm.begin() + static_cast<std::ptrdiff_t>(logical));
    const auto P = static_cast<Dimension>(physical), Hk = static_cast<Dimension>(hkv);
    const Tensor kp = random_uniform({P, Hk, 16, 128}, history + 1, -1, 1);
    const Tensor vp = random_uniform({P, Hk, 16, 128}, history + 2, -1, 1);
    const Tensor q = random_uniform({static_cast<Dimension>(hq), 1, 128}, history + 3, -1, 1);
    const Tensor tk = random_uniform({Hk, 1, 128}, history + 4, -1, 1);
    const Tensor tv = random_uniform({Hk, 1, 128}, history + 5, -1, 1);
    const PagedBlockTable table(ids, physical, 0);
    const Tensor dkp = kp.to(kGpu), dvp = vp.to(kGpu), dq = q.to(kGpu);
    const Tensor dtk = tk.to(kGpu), dtv = tv.to(kGpu);
    const Shape os{static_cast<Dimension>(hq), 1, 128};
    const Shape wss{static_cast<Dimension>(hq), 1, static_cast<Dimension>(history + 1)};
    Tensor fast = Tensor::empty(os, DType::kFloat32, kGpu), exact = Tensor::empty(os, DType::kFloat32, kGpu);
    Tensor ws = Tensor::empty(wss, DType::kFloat32, kGpu), ws2 = Tensor::empty(wss, DType::kFloat32, kGpu);
    attn::paged_scaled_dot_product_attention_with_tail_out(dq, dkp, dvp, table, history, dtk, dtv,
                                                           fast, ws, stream);
    attn::paged_scaled_dot_product_attention_with_tail_probabilities_out(
        dq, dkp, dvp, table, history, dtk, dtv, exact, ws2, stream);
    stream.synchronize();
    const std::int32_t len = static_cast<std::int32_t>(history);
    std::vector<float> want(hq * 128);
    oracle_batched_decode(q.data_as<float>(), 1, hq, hkv, 128, kp.data_as<float>(),
                          vp.data_as<float>(), 16, ids.data(), logical, &len, tk.data_as<float>(),
                          tv.data_as<float>(), want.data(), 4);
    const auto a = host_values(fast), b = host_values(exact);
    for (std::size_t i = 0; i < want.size(); ++i) {
      EXPECT_TRUE(std::fabs(a[i] - want[i]) <= 2.0e-5F + 1.0e-4F * std::fabs(want[i]));
      EXPECT_TRUE(std::fabs(b[i] - want[i]) <= 2.0e-5F + 1.0e-4F * std::fabs(want[i]));
    }
    const auto pa = host_values(ws), pb = host_values(ws2);
    for (std::size_t i = 0; i < pa.size(); ++i) EXPECT_TRUE(std::fabs(pa[i] - pb[i]) <= 2.0e-6F);
  }
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
