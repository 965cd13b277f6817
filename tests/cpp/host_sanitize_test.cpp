// Host-only test driver built under the sanitizers (tests/cpp/Makefile
// targets host_sanitize_asan and host_sanitize_tsan): the host part of the
// library (block manager, prefix cache, their C ABI) and the oracle pool
// compiled with g++ -fsanitize=address,undefined or -fsanitize=thread, with
// no HIP runtime involved.  The cases are those of host_programs.hpp:
// contention on one block manager, random programs against the oracle pool
// and the host prefix cache under contention.
#include "mini_test.hpp"

struct HostContractTest {
  void SetUp() {}
};

#include "host_programs.hpp"

int main(int argc, char** argv) { return mini_test::run_all(argc > 1 ? argv[1] : nullptr); }
