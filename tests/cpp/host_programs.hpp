// Host-only tests of the library's page bookkeeping through the C ABI
// (block manager and host prefix cache; no device is touched).  Included by
// paged_api_test.cpp (the full C++ API suite) and by host_sanitize_test.cpp,
// which builds the host part of the library (csrc/block_manager.cpp,
// csrc/prefix_cache.cpp, csrc/host_api.cpp) and the oracle with the
// address, undefined-behaviour and thread sanitizers.  The includer defines
// the HostContractTest fixture.
#pragma once

#include "helix_paged.h"
#include "mini_test.hpp"

#include <algorithm>
#include <cstdint>
#include <map>
#include <random>
#include <string>
#include <thread>
#include <vector>

extern "C" {
void* oracle_pool_create(std::size_t layers, std::size_t kv_heads, std::size_t head_dim,
                         std::size_t block_tokens, std::size_t physical_blocks, int* status);
void oracle_pool_destroy(void* pool);
std::uint64_t oracle_create_sequence(void* pool);
int oracle_fork_sequence(void* pool, std::uint64_t source, std::size_t prefix, int allow_cow,
                         std::uint64_t* out);
int oracle_append_layer_major(void* pool, std::uint64_t seq, const float* keys,
                              const float* values, std::size_t tokens);
int oracle_release_sequence(void* pool, std::uint64_t seq);
std::size_t oracle_length(void* pool, std::uint64_t seq);
std::size_t oracle_block_table(void* pool, std::uint64_t seq, std::uint32_t* out,
                               std::size_t capacity);
void oracle_stats(void* pool, helix_paged_stats* out);
}

// Host page bookkeeping under contention: eight threads run random programs
// (create, append, forks of a shared source, releases) on one block manager
// through the C ABI.  Every call is serialised by the manager: each
// sequence ends at the length its own successful appends give it, every
// invariant holds (helix_block_manager_validate), each page's reference count
// equals the number of live tables holding it, and releasing everything
// returns every page.
TEST_F(HostContractTest, BlockManagerSerialisesConcurrentPrograms) {
  const helix_paged_config config{1, 1, 4, 4, 64};
  helix_block_manager* m = nullptr;
  ASSERT_EQ(helix_block_manager_create(&config, &m), HELIX_OK);
  helix_sequence source{};
  ASSERT_EQ(helix_block_manager_create_sequence(m, &source), HELIX_OK);
  ASSERT_EQ(helix_block_manager_append(m, source, 8, nullptr), HELIX_OK);
  constexpr int kThreads = 8;
  struct Owned {
    helix_sequence seq;
    std::size_t length;
  };
  std::vector<std::vector<Owned>> owned(kThreads);
  std::vector<int> unexpected(kThreads, 0);
  std::vector<std::thread> threads;
  for (int t = 0; t < kThreads; ++t) {
    threads.emplace_back([&, t] {
      std::mt19937_64 rng(1000 + t);
      auto& mine = owned[static_cast<std::size_t>(t)];
      for (int i = 0; i < 400; ++i) {
        const int op = static_cast<int>(rng() % 6);
        if (op == 0 || mine.empty()) {
          helix_sequence s{};
          if (helix_block_manager_create_sequence(m, &s) != HELIX_OK) ++unexpected[t];
          mine.push_back({s, 0});
        } else if (op == 1) {
          helix_sequence s{};
          const int rc = helix_block_manager_fork_sequence(m, source, 8, 0, &s, nullptr);
          if (rc == HELIX_OK) {
            mine.push_back({s, 8});
          } else if (rc != HELIX_RESOURCE_EXHAUSTED) {
            ++unexpected[t];
          }
        } else if (op <= 4) {
          Owned& o = mine[rng() % mine.size()];
          const std::size_t n = 1 + rng() % 9;
          const int rc = helix_block_manager_append(m, o.seq, n, nullptr);
          if (rc == HELIX_OK) {
            o.length += n;
          } else if (rc != HELIX_RESOURCE_EXHAUSTED) {
            ++unexpected[t];
          }
        } else {
          const std::size_t k = rng() % mine.size();
          if (helix_block_manager_release_sequence(m, mine[k].seq) != HELIX_OK) ++unexpected[t];
          mine.erase(mine.begin() + static_cast<std::ptrdiff_t>(k));
        }
      }
    });
  }
  for (auto& th : threads) th.join();
  for (int t = 0; t < kThreads; ++t) EXPECT_EQ(unexpected[static_cast<std::size_t>(t)], 0);
  EXPECT_EQ(helix_block_manager_validate(m), HELIX_OK);
  std::map<std::uint32_t, std::size_t> holders;
  std::size_t live = 1;
  auto count_table = [&](helix_sequence s) {
    std::vector<std::uint32_t> ids(64);
    std::size_t n = 0;
    EXPECT_EQ(helix_block_manager_block_table(m, s, ids.data(), ids.size(), &n), HELIX_OK);
    for (std::size_t i = 0; i < n; ++i) ++holders[ids[i]];
  };
  count_table(source);
  for (const auto& mine : owned)
    for (const Owned& o : mine) {
      std::size_t len = 0;
      EXPECT_EQ(helix_block_manager_length(m, o.seq, &len), HELIX_OK);
      EXPECT_EQ(len, o.length);
      count_table(o.seq);
      ++live;
    }
  helix_paged_stats st{};
  EXPECT_EQ(helix_block_manager_stats(m, &st), HELIX_OK);
  EXPECT_EQ(st.active_sequence_count, live);
  EXPECT_EQ(st.used_blocks, holders.size());
  for (const auto& [block, count] : holders) {
    std::size_t refs = 0, tokens = 0;
    EXPECT_EQ(helix_block_manager_block_info(m, block, &refs, &tokens), HELIX_OK);
    EXPECT_EQ(refs, count);
  }
  for (const auto& mine : owned)
    for (const Owned& o : mine) EXPECT_EQ(helix_block_manager_release_sequence(m, o.seq), HELIX_OK);
  EXPECT_EQ(helix_block_manager_release_sequence(m, source), HELIX_OK);
  EXPECT_EQ(helix_block_manager_stats(m, &st), HELIX_OK);
  EXPECT_EQ(st.used_blocks, 0U);
  EXPECT_EQ(st.free_blocks, 64U);
  EXPECT_EQ(helix_block_manager_validate(m), HELIX_OK);
  helix_block_manager_destroy(m);
}

// Seeded random programs (create, appends of 1-9 tokens, aligned and
// copy-on-write forks, releases) on the host block manager and on the
// oracle's restatement of the reference pool (src/kv_cache/paged.cpp): same
// success or error code for every call, the same block tables, lengths and
// statistics after it, every appended token's reported slot inside its
// table page, and every invariant re-derived after every call.
TEST_F(HostContractTest, BlockManagerRandomProgramsMatchTheOraclePool) {
  constexpr std::size_t L = 1, H = 1, D = 2, P = 4, N = 24;
  for (std::uint64_t seed : {21U, 22U, 23U, 24U}) {
    std::mt19937_64 rng(seed);
    auto pick = [&](std::size_t n) { return static_cast<std::size_t>(rng() % n); };
    const helix_paged_config config{L, H, D, P, N};
    helix_block_manager* m = nullptr;
    ASSERT_EQ(helix_block_manager_create(&config, &m), HELIX_OK);
    int st = 0;
    void* pool = oracle_pool_create(L, H, D, P, N, &st);
    ASSERT_EQ(st, 0);
    struct Live {
      helix_sequence mine;
      std::uint64_t theirs;
    };
    std::vector<Live> live;
    for (int step = 0; step < 400; ++step) {
      const std::size_t what = live.empty() ? 0 : pick(10);
      int mine = HELIX_OK, theirs = 0;
      if (what == 0) {
        helix_sequence s{};
        mine = helix_block_manager_create_sequence(m, &s);
        live.push_back({s, oracle_create_sequence(pool)});
      } else if (what <= 4) {
        Live& s = live[pick(live.size())];
        std::size_t before = 0;
        ASSERT_EQ(helix_block_manager_length(m, s.mine, &before), HELIX_OK);
        const std::size_t t = 1 + pick(9);
        std::vector<float> k(L * H * t * D, 1.0F), v(L * H * t * D, 2.0F);
        std::vector<std::uint64_t> slots(t, ~std::uint64_t{0});
        mine = helix_block_manager_append(m, s.mine, t, slots.data());
        theirs = oracle_append_layer_major(pool, s.theirs, k.data(), v.data(), t);
        if (mine == HELIX_OK) {
          std::vector<std::uint32_t> table(N);
          std::size_t n = 0;
          ASSERT_EQ(helix_block_manager_block_table(m, s.mine, table.data(), N, &n), HELIX_OK);
          for (std::size_t i = 0; i < t; ++i) {
            const std::size_t pos = before + i;
            ASSERT_TRUE(pos / P < n);
            EXPECT_EQ(slots[i], std::uint64_t{table[pos / P]} * P + pos % P);
          }
        }
      } else if (what <= 7) {
        Live& s = live[pick(live.size())];
        std::size_t len = 0;
        ASSERT_EQ(helix_block_manager_length(m, s.mine, &len), HELIX_OK);
        const bool cow = pick(2) == 1;
        const std::size_t prefix = len == 0 ? 0 : (cow ? 1 + pick(len) : P * pick(len / P + 1));
        helix_sequence child{};
        helix_cow_copy copy{};
        std::uint64_t other = 0;
        mine = helix_block_manager_fork_sequence(m, s.mine, prefix, cow ? 1 : 0, &child, &copy);
        theirs = oracle_fork_sequence(pool, s.theirs, prefix, cow ? 1 : 0, &other);
        if (mine == HELIX_OK && theirs == 0) {
          live.push_back({child, other});
          // A copy-on-write fork copies exactly the partial last page.
          EXPECT_EQ(copy.tokens, prefix % P == 0 ? std::size_t{0} : prefix % P);
        }
      } else {
        const std::size_t i = pick(live.size());
        mine = helix_block_manager_release_sequence(m, live[i].mine);
        theirs = oracle_release_sequence(pool, live[i].theirs);
        live.erase(live.begin() + static_cast<std::ptrdiff_t>(i));
      }
      if (mine != theirs) {
        ::mini_test::fail(__FILE__, __LINE__,
                          "seed " + std::to_string(seed) + " step " + std::to_string(step) +
                              ": library status " + std::to_string(mine) + ", oracle " +
                              std::to_string(theirs));
        break;
      }
      EXPECT_EQ(helix_block_manager_validate(m), HELIX_OK);
      helix_paged_stats got{}, want{};
      ASSERT_EQ(helix_block_manager_stats(m, &got), HELIX_OK);
      oracle_stats(pool, &want);
      EXPECT_EQ(got.used_blocks, want.used_blocks);
      EXPECT_EQ(got.free_blocks, want.free_blocks);
      EXPECT_EQ(got.block_reference_count, want.block_reference_count);
      EXPECT_EQ(got.shared_blocks, want.shared_blocks);
      EXPECT_EQ(got.active_tokens, want.active_tokens);
      EXPECT_EQ(got.allocated_token_slots, want.allocated_token_slots);
      EXPECT_EQ(got.block_allocation_count, want.block_allocation_count);
      EXPECT_EQ(got.block_reuse_count, want.block_reuse_count);
      EXPECT_EQ(got.peak_bytes_used, want.peak_bytes_used);
      for (const Live& s : live) {
        std::vector<std::uint32_t> a(N), b(N);
        std::size_t n = 0;
        ASSERT_EQ(helix_block_manager_block_table(m, s.mine, a.data(), N, &n), HELIX_OK);
        a.resize(n);
        b.resize(oracle_block_table(pool, s.theirs, b.data(), N));
        EXPECT_TRUE(a == b);
        std::size_t len = 0;
        ASSERT_EQ(helix_block_manager_length(m, s.mine, &len), HELIX_OK);
        EXPECT_EQ(len, oracle_length(pool, s.theirs));
      }
    }
    helix_block_manager_destroy(m);
    oracle_pool_destroy(pool);
  }
}

// The host prefix cache under contention: eight threads insert prompts that
// share page prefixes, look up longest prefixes (and release the forks they
// get), test, erase and evict on one cache over one block manager.  Every
// hit is block aligned, no longer than the query or its limit, and its fork
// has exactly the matched length; the budgets hold throughout; clearing the
// cache and releasing every thread's sequences frees every page.
TEST_F(HostContractTest, HostPrefixCacheUnderContention) {
  constexpr std::size_t P = 4;
  const helix_paged_config config{1, 1, 2, P, 512};
  helix_block_manager* m = nullptr;
  ASSERT_EQ(helix_block_manager_create(&config, &m), HELIX_OK);
  const helix_prefix_config pc{12, 48};
  helix_prefix_cache* cache = nullptr;
  ASSERT_EQ(helix_prefix_cache_create_host(m, &pc, &cache), HELIX_OK);
  // Prompts: prompt i is the first 4 * (1 + i % 8) tokens of family i / 8.
  auto prompt = [](std::size_t i) {
    std::vector<std::uint32_t> t(P * (1 + i % 8));
    for (std::size_t k = 0; k < t.size(); ++k) {
      t[k] = static_cast<std::uint32_t>(1000 * (i / 8) + k);
    }
    return t;
  };
  constexpr int kThreads = 8;
  std::vector<int> unexpected(kThreads, 0);
  std::vector<std::thread> threads;
  for (int th = 0; th < kThreads; ++th) {
    threads.emplace_back([&, th] {
      std::mt19937_64 rng(500 + th);
      int& bad = unexpected[static_cast<std::size_t>(th)];
      for (int i = 0; i < 300; ++i) {
        const std::vector<std::uint32_t> key = prompt(rng() % 24);
        const std::uint64_t ns = 1 + rng() % 2;  // namespace 0 is reserved
        const int op = static_cast<int>(rng() % 7);
        if (op <= 1) {
          helix_sequence s{};
          if (helix_block_manager_create_sequence(m, &s) != HELIX_OK) ++bad;
          const int rc = helix_block_manager_append(m, s, key.size(), nullptr);
          if (rc == HELIX_OK) {
            int status = -1;
            if (helix_prefix_cache_insert(cache, ns, key.data(), key.size(), s, &status) !=
                    HELIX_OK ||
                status < 0 || status > 2) {
              ++bad;
            }
          } else if (rc != HELIX_RESOURCE_EXHAUSTED) {
            ++bad;
          }
          if (helix_block_manager_release_sequence(m, s) != HELIX_OK) ++bad;
        } else if (op <= 3) {
          std::vector<std::uint32_t> query = key;
          query.push_back(7);  // a partial page past the key
          const std::size_t limit = rng() % 3 == 0 ? P * (rng() % 4) : query.size();
          int hit = 0;
          helix_sequence s{};
          std::size_t matched = 0;
          if (helix_prefix_cache_lookup_longest(cache, ns, query.data(), query.size(), limit,
                                                &hit, &s, &matched) != HELIX_OK) {
            ++bad;
            continue;
          }
          if (hit == 0) continue;
          std::size_t len = 0;
          if (matched % P != 0 || matched > limit || matched > key.size() ||
              helix_block_manager_length(m, s, &len) != HELIX_OK || len != matched) {
            ++bad;
          }
          if (helix_block_manager_release_sequence(m, s) != HELIX_OK) ++bad;
        } else if (op == 4) {
          int present = 0;
          if (helix_prefix_cache_contains(cache, ns, key.data(), key.size(), &present) !=
              HELIX_OK) {
            ++bad;
          }
        } else if (op == 5) {
          int erased = 0;
          if (helix_prefix_cache_erase(cache, ns, key.data(), key.size(), &erased) != HELIX_OK) {
            ++bad;
          }
        } else {
          int evicted = 0;
          if (helix_prefix_cache_evict_lru(cache, &evicted) != HELIX_OK) ++bad;
        }
        helix_prefix_stats s{};
        if (helix_prefix_cache_stats(cache, &s) != HELIX_OK || s.entry_count > 12 ||
            s.retained_block_references > 48) {
          ++bad;
        }
      }
    });
  }
  for (auto& t : threads) t.join();
  for (int th = 0; th < kThreads; ++th) EXPECT_EQ(unexpected[static_cast<std::size_t>(th)], 0);
  EXPECT_EQ(helix_block_manager_validate(m), HELIX_OK);
  helix_prefix_stats s{};
  ASSERT_EQ(helix_prefix_cache_stats(cache, &s), HELIX_OK);
  EXPECT_EQ(s.hit_count + s.miss_count, s.lookup_count);
  EXPECT_TRUE(s.peak_entries <= 12 && s.peak_block_references <= 48);
  helix_paged_stats ps{};
  ASSERT_EQ(helix_block_manager_stats(m, &ps), HELIX_OK);
  EXPECT_EQ(ps.active_sequence_count, s.entry_count);  // only the anchors stay live
  ASSERT_EQ(helix_prefix_cache_clear(cache), HELIX_OK);
  ASSERT_EQ(helix_block_manager_stats(m, &ps), HELIX_OK);
  EXPECT_EQ(ps.used_blocks, 0U);
  EXPECT_EQ(ps.active_sequence_count, 0U);
  helix_prefix_cache_destroy(cache);
  EXPECT_EQ(helix_block_manager_validate(m), HELIX_OK);
  helix_block_manager_destroy(m);
}
