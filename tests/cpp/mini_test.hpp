// A minimal test runner with gtest-shaped macros, so that the C++ API tests
// read like the reference's own (gtest is not available in this image).
// Each TEST_F registers a function; EXPECT_* records a failure and goes on,
// ASSERT_* ends the test.  A fixture's SetUp may call SKIP().
#pragma once

#include <cmath>
#include <cstdio>
#include <cstring>
#include <exception>
#include <functional>
#include <sstream>
#include <string>
#include <vector>

namespace mini_test {

struct Case {
  std::string suite, name;
  std::function<void()> run;
};
inline std::vector<Case>& registry() {
  static std::vector<Case> cases;
  return cases;
}
inline int& failures() {
  static int n = 0;
  return n;
}
struct AssertionEnd {};
struct Skipped {
  std::string why;
};
struct Registrar {
  Registrar(const char* suite, const char* name, std::function<void()> run) {
    registry().push_back({suite, name, std::move(run)});
  }
};

inline void fail(const char* file, int line, const std::string& what) {
  ++failures();
  std::fprintf(stderr, "%s:%d: failure: %s\n", file, line, what.c_str());
}

template <class A, class B>
std::string describe(const char* ea, const char* eb, const A& a, const B& b) {
  std::ostringstream s;
  s << ea << " == " << eb << " (" << a << " vs " << b << ")";
  return s.str();
}

inline bool float_eq(float a, float b) {  // within 4 ulps, as gtest's EXPECT_FLOAT_EQ
  if (std::isnan(a) || std::isnan(b)) return false;
  if (a == b) return true;
  std::int32_t ia, ib;
  std::memcpy(&ia, &a, 4);
  std::memcpy(&ib, &b, 4);
  if ((ia < 0) != (ib < 0)) return false;
  return std::abs(static_cast<long long>(ia) - static_cast<long long>(ib)) <= 4;
}

inline int run_all(const char* filter) {
  int failed_cases = 0, ran = 0, skipped = 0;
  for (const Case& c : registry()) {
    const std::string full = c.suite + "." + c.name;
    if (filter != nullptr && full.find(filter) == std::string::npos) continue;
    std::printf("[ RUN      ] %s\n", full.c_str());
    std::fflush(stdout);
    const int before = failures();
    try {
      c.run();
    } catch (const AssertionEnd&) {
    } catch (const Skipped& s) {
      std::printf("[  SKIPPED ] %s: %s\n", full.c_str(), s.why.c_str());
      ++skipped;
      continue;
    } catch (const std::exception& e) {
      fail(__FILE__, __LINE__, std::string("uncaught exception: ") + e.what());
    }
    ++ran;
    const bool ok = failures() == before;
    failed_cases += ok ? 0 : 1;
    std::printf("[ %s ] %s\n", ok ? "      OK" : " FAILED ", full.c_str());
    std::fflush(stdout);
  }
  std::printf("%d ran, %d skipped, %d failed\n", ran, skipped, failed_cases);
  return failed_cases == 0 ? 0 : 1;
}

}  // namespace mini_test

#define MT_CAT2(a, b) a##b
#define MT_CAT(a, b) MT_CAT2(a, b)
#define TEST_F(suite, name)                                                                    \
  struct suite##_##name : suite {                                                              \
    void body();                                                                               \
  };                                                                                           \
  static ::mini_test::Registrar MT_CAT(mt_reg_, MT_CAT(suite##_##name, __LINE__))(             \
      #suite, #name, [] {                                                                      \
        suite##_##name t;                                                                      \
        t.SetUp();                                                                             \
        t.body();                                                                              \
      });                                                                                      \
  void suite##_##name::body()

#define SKIP(why) throw ::mini_test::Skipped{why}
#define MT_CHECK(cond, text, fatal)                                                            \
  do {                                                                                         \
    if (!(cond)) {                                                                             \
      ::mini_test::fail(__FILE__, __LINE__, text);                                             \
      if (fatal) throw ::mini_test::AssertionEnd{};                                            \
    }                                                                                          \
  } while (false)
#define EXPECT_TRUE(c) MT_CHECK((c), #c, false)
#define EXPECT_FALSE(c) MT_CHECK(!(c), "!(" #c ")", false)
#define ASSERT_TRUE(c) MT_CHECK((c), #c, true)
#define EXPECT_EQ(a, b) MT_CHECK((a) == (b), ::mini_test::describe(#a, #b, (a), (b)), false)
#define ASSERT_EQ(a, b) MT_CHECK((a) == (b), ::mini_test::describe(#a, #b, (a), (b)), true)
#define ASSERT_NE(a, b) MT_CHECK((a) != (b), #a " != " #b, true)
#define EXPECT_FLOAT_EQ(a, b) \
  MT_CHECK(::mini_test::float_eq((a), (b)), ::mini_test::describe(#a, #b, (a), (b)), false)
#define EXPECT_NEAR(a, b, tol) \
  MT_CHECK(std::fabs((a) - (b)) <= (tol), ::mini_test::describe(#a, #b, (a), (b)), false)
#define EXPECT_THROW(stmt, type)                                                               \
  do {                                                                                         \
    bool mt_thrown = false;                                                                    \
    try {                                                                                      \
      stmt;                                                                                    \
    } catch (const type&) {                                                                    \
      mt_thrown = true;                                                                        \
    } catch (...) {                                                                            \
    }                                                                                          \
    MT_CHECK(mt_thrown, "expected " #type " from " #stmt, false);                              \
  } while (false)
#define EXPECT_NO_THROW(stmt)                                                                  \
  do {                                                                                         \
    try {                                                                                      \
      stmt;                                                                                    \
    } catch (const std::exception& mt_e) {                                                     \
      MT_CHECK(false, std::string("unexpected exception from " #stmt ": ") + mt_e.what(),      \
               false);                                                                         \
    }                                                                                          \
  } while (false)
#define FAIL(text) MT_CHECK(false, text, true)
