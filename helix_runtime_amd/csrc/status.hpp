// Error codes and the internal exception type.  The numbering follows
// helix::ErrorCode (include/helix/core/error.hpp:10-17 of the reference):
// 0 is success and 1..6 are the six reference codes in declaration order.
// Exceptions never cross the C ABI: c_api.cpp converts them into an int
// status plus a thread-local message.
#pragma once

#include <stdexcept>
#include <string>

namespace helix {

enum class Status : int {
  kOk = 0,
  kInvalidArgument = 1,
  kOutOfRange = 2,
  kUnsupported = 3,
  kResourceExhausted = 4,
  kRuntime = 5,
  kInternal = 6,
};

class Error final : public std::runtime_error {
public:
  Error(Status status, const std::string& message)
      : std::runtime_error(message), status_(status) {}
  [[nodiscard]] Status status() const noexcept { return status_; }

private:
  Status status_;
};

[[noreturn]] inline void fail(Status status, const std::string& message) {
  throw Error(status, message);
}

inline void check(bool condition, Status status, const std::string& message) {
  if (!condition) fail(status, message);
}

// "op: what", composed only on failure (no host allocation on success).
inline void check(bool condition, Status status, const char* op, const char* what) {
  if (!condition) fail(status, std::string(op) + ": " + what);
}

}  // namespace helix
