// common.hpp — errors, status names and small helpers shared by every layer.
#pragma once

#include <xvram/xvram.h>
#include <xvram/xvram_amd_ext.h>
#include <xvram/xvram_v2.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <limits>
#include <string>
#include <string_view>

namespace xvram {

using Clock = std::chrono::steady_clock;

// One failure, as published through xvram_error_info_v1 (the reference's
// sdk::Error, src/sdk/status.cpp:26-45).
struct Error {
  xvram_status status = XVRAM_STATUS_SUCCESS;
  xvram_native_error_domain native_domain = XVRAM_NATIVE_ERROR_NONE;
  int64_t native_code = 0;
  std::string stage;
  std::string operation;
  std::string native_name;
  std::string message;

  explicit operator bool() const noexcept { return status != XVRAM_STATUS_SUCCESS; }
};

inline Error make_error(xvram_status status, std::string_view stage, std::string_view operation,
                        std::string_view message) {
  Error e;
  e.status = status;
  e.stage.assign(stage);
  e.operation.assign(operation);
  e.message.assign(message);
  return e;
}

inline Error invalid(std::string_view operation, std::string_view message) {
  return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "sdk", operation, message);
}

inline Error incompatible(std::string_view operation, std::string_view message) {
  return make_error(XVRAM_STATUS_INCOMPATIBLE_ABI, "sdk", operation, message);
}

// Status names, identical strings to the reference (src/sdk/status.cpp:83-128).
const char* status_name(xvram_status status) noexcept;

// Copies `error` into a public record, preserving the caller's struct_size
// (src/sdk/status.cpp:130-141).
void write_error_info(const Error& error, xvram_error_info_v1& output) noexcept;

// Maps the active exception to an Error (bad_alloc -> HOST_OUT_OF_MEMORY,
// anything else -> INTERNAL), as the reference boundary does.
Error exception_error(std::string_view operation) noexcept;

inline bool checked_add(uint64_t a, uint64_t b, uint64_t& out) {
  if (b > std::numeric_limits<uint64_t>::max() - a) return false;
  out = a + b;
  return true;
}

inline bool checked_mul(uint64_t a, uint64_t b, uint64_t& out) {
  if (a != 0 && b > std::numeric_limits<uint64_t>::max() / a) return false;
  out = a * b;
  return true;
}

inline uint64_t round_up(uint64_t v, uint64_t m) { return (v + m - 1) / m * m; }
inline uint64_t ceil_div(uint64_t v, uint64_t d) { return (v + d - 1) / d; }

// A submission-relative deadline (src/sdk/deadline.hpp:14-63): zero disables
// it; expiry is now >= submitted + deadline_ms; an unrepresentable deadline is
// rejected at submission.
class Deadline {
public:
  static bool create(uint64_t deadline_ms, Clock::time_point submitted, Deadline& out) {
    out = Deadline{};
    out.submitted_ = submitted;
    if (deadline_ms == 0) return true;
    const auto remaining = Clock::time_point::max() - submitted;
    const auto remaining_ms = std::chrono::duration_cast<std::chrono::milliseconds>(remaining).count();
    if (remaining_ms < 0 || deadline_ms > static_cast<uint64_t>(remaining_ms)) return false;
    out.at_ = submitted + std::chrono::duration_cast<Clock::duration>(
                              std::chrono::milliseconds(static_cast<int64_t>(deadline_ms)));
    out.has_ = true;
    return true;
  }
  bool expired(Clock::time_point now = Clock::now()) const { return has_ && now >= at_; }
  Clock::time_point submitted() const { return submitted_; }
  Error timeout_error(const char* stage, const char* operation) const {
    return make_error(XVRAM_STATUS_TIMEOUT, stage, operation,
                      "operation missed its submission-relative deadline before a safe launch "
                      "boundary");
  }

private:
  Clock::time_point submitted_{};
  Clock::time_point at_{};
  bool has_ = false;
};

inline Error validate_deadline(uint64_t deadline_ms, const char* operation) {
  Deadline ignored;
  if (!Deadline::create(deadline_ms, Clock::now(), ignored))
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "deadline", operation,
                      "deadline_ms cannot be represented by the monotonic clock");
  return {};
}

} // namespace xvram
