// errors.cpp — status names, the public error record and the mapping of C++
// exceptions to statuses at the ABI boundary.
#include <algorithm>
#include <array>
#include <exception>
#include <new>

#include "common.hpp"

namespace xvram {

namespace {

// Indexed by status code; the codes are the contiguous range 0..19 of
// include/xvram/xvram.h. The names are interface (the reference's
// status_name, src/sdk/status.cpp:83-128, returns the same string per code).
constexpr std::array<const char*, 20> kStatusNames{
    "success",         "invalid_argument", "incompatible_abi",     "unsupported",
    "unavailable",     "host_out_of_memory", "device_out_of_memory", "budget_pressure",
    "busy",            "not_ready",        "timeout",              "corruption",
    "callback_failed", "cuda_error",       "cublas_error",         "poisoned",
    "cleanup_failed",  "closed",           "cancelled",            "internal"};
static_assert(XVRAM_STATUS_SUCCESS == 0 && XVRAM_STATUS_TIMEOUT == 10 &&
              XVRAM_STATUS_INTERNAL == kStatusNames.size() - 1);

// NUL-terminated, truncated to the field, the rest of the field zeroed.
template <size_t N>
void put_text(char (&field)[N], const std::string& text) noexcept {
  const size_t n = std::min(text.size(), N - 1);
  std::fill(std::copy_n(text.data(), n, field), field + N, '\0');
}

} // namespace

const char* status_name(xvram_status status) noexcept {
  return status < kStatusNames.size() ? kStatusNames[status] : "unknown";
}

void write_error_info(const Error& error, xvram_error_info_v1& output) noexcept {
  xvram_error_info_v1 record = XVRAM_ERROR_INFO_V1_INIT;
  record.struct_size = output.struct_size;
  record.status = error.status;
  record.native_domain = error.native_domain;
  record.native_code = error.native_code;
  put_text(record.stage, error.stage);
  put_text(record.operation, error.operation);
  put_text(record.native_name, error.native_name);
  put_text(record.message, error.message);
  output = record;
}

Error exception_error(std::string_view operation) noexcept {
  Error e;
  e.status = XVRAM_STATUS_INTERNAL;
  try {
    try {
      throw;
    } catch (const std::bad_alloc&) {
      e.status = XVRAM_STATUS_HOST_OUT_OF_MEMORY;
      e.message = "host memory allocation failed";
    } catch (const std::exception& ex) {
      e.message = ex.what();
    } catch (...) {
      e.message = "a C++ exception of unknown type reached the ABI boundary";
    }
    e.stage = "abi";
    e.operation.assign(operation);
  } catch (...) {
    // Building the text needed memory that was not there: the status stands.
  }
  return e;
}

} // namespace xvram
