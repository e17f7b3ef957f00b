// common.hpp — errors, status names and small helpers shared by every layer.
#pragma once

#include <xvram/xvram.h>
#include <xvram/xvram_amd_ext.h>
#include <xvram/xvram_v2.h>

#include <chrono>
#include <cstdint>
#include <cstring>
#include <limits>
#include <optional>
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

// The status names of the ABI (the strings are interface: reference
// src/sdk/status.cpp:83-128 returns the same name for each code).
const char* status_name(xvram_status status) noexcept;

// Copies `error` into a public record, preserving the caller's struct_size
// (reference src/sdk/status.cpp:130-141).
void write_error_info(const Error& error, xvram_error_info_v1& output) noexcept;

// Maps the exception being handled to an Error: bad_alloc ->
// HOST_OUT_OF_MEMORY, anything else -> INTERNAL (the reference ABI boundary's
// mapping, src/sdk/api.cpp:109-122). Call only inside a catch block.
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

// The submission-relative deadline of an operation (a descriptor's
// deadline_ms): due that many milliseconds after submission, never for 0.
// Once it has passed the operation starts no more device work: the worker
// checks it when it takes the operation off the queue and before each launch.
class Deadline {
public:
  Deadline() = default;
  // nullopt when submission + ms lies beyond the steady clock's range.
  static std::optional<Deadline> after(uint64_t ms, Clock::time_point submitted) {
    using Ms = std::chrono::milliseconds;
    Deadline d;
    d.submitted_ = submitted;
    if (ms == 0) return d;
    const int64_t room = std::chrono::duration_cast<Ms>(Clock::time_point::max() - submitted).count();
    if (room < 0 || ms > static_cast<uint64_t>(room)) return std::nullopt;
    d.due_ = submitted + std::chrono::duration_cast<Clock::duration>(Ms(static_cast<int64_t>(ms)));
    return d;
  }
  bool passed(Clock::time_point now = Clock::now()) const { return due_ && now >= *due_; }
  Clock::time_point submitted() const { return submitted_; }
  Error missed(const char* stage, const char* where) const {
    return make_error(XVRAM_STATUS_TIMEOUT, stage, where,
                      "deadline_ms passed before the operation reached its next launch boundary");
  }

private:
  Clock::time_point submitted_{};
  std::optional<Clock::time_point> due_;
};

// INVALID_ARGUMENT when a descriptor's deadline_ms cannot be represented.
inline Error check_deadline_ms(uint64_t ms, const char* operation) {
  if (Deadline::after(ms, Clock::now())) return {};
  return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "deadline", operation,
                    "deadline_ms lies beyond the range of the monotonic clock");
}

} // namespace xvram
