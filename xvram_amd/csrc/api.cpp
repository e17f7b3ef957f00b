// api.cpp — the C-ABI boundary: xvram_get_api and the v1 function table.
//
// Replaces src/sdk/api.cpp of the reference. Kept identical because callers
// depend on it: argument validation order and the status each failure maps
// to (api.cpp:124-344), struct_size preservation on outputs (:459-475), the
// exception firewall (:109-122: bad_alloc -> HOST_OUT_OF_MEMORY, anything
// else -> INTERNAL), per-session last-error recording (:18-47), handle
// ownership (allocation handles may outlive their session, :644-661) and the
// synchronous wrappers = submit + wait + release (:782-806, :876-900).
#include <xvram/xvram.h>

#include <atomic>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <vector>

#include "common.hpp"
#include "session.hpp"

namespace xvram {
namespace {

struct SessionState {
  SessionState(std::shared_ptr<Session> s, uint64_t chunk, uint64_t workspace)
      : backend(std::move(s)), chunk_bytes(chunk), workspace_cap_bytes(workspace) {}
  void record(const Error& e) noexcept {
    if (!e) return;
    try {
      std::lock_guard<std::mutex> lock(mutex);
      last_error = e;
    } catch (...) {
    }
  }
  Error error() const {
    std::lock_guard<std::mutex> lock(mutex);
    return last_error;
  }
  std::shared_ptr<Session> backend;
  uint64_t chunk_bytes = 0;
  uint64_t workspace_cap_bytes = 0;
  mutable std::mutex mutex;
  Error last_error;
  std::atomic<bool> closed{false};
};

} // namespace
} // namespace xvram

struct xvram_session_t {
  std::shared_ptr<xvram::SessionState> state;
};
struct xvram_allocation_t {
  std::shared_ptr<xvram::SessionState> owner;
  std::shared_ptr<xvram::AllocationRecord> backend;
};
struct xvram_operation_t {
  std::shared_ptr<xvram::SessionState> owner;
  std::shared_ptr<xvram::Operation> backend;
};
struct xvram_gemm_plan_t {
  std::shared_ptr<xvram::SessionState> owner;
  std::shared_ptr<xvram::GemmPlanRecord> backend;
};

namespace xvram {

// ---- status helpers ----------------------------------------------------------

const char* status_name(xvram_status s) noexcept {
  switch (s) {
  case XVRAM_STATUS_SUCCESS: return "success";
  case XVRAM_STATUS_INVALID_ARGUMENT: return "invalid_argument";
  case XVRAM_STATUS_INCOMPATIBLE_ABI: return "incompatible_abi";
  case XVRAM_STATUS_UNSUPPORTED: return "unsupported";
  case XVRAM_STATUS_UNAVAILABLE: return "unavailable";
  case XVRAM_STATUS_HOST_OUT_OF_MEMORY: return "host_out_of_memory";
  case XVRAM_STATUS_DEVICE_OUT_OF_MEMORY: return "device_out_of_memory";
  case XVRAM_STATUS_BUDGET_PRESSURE: return "budget_pressure";
  case XVRAM_STATUS_BUSY: return "busy";
  case XVRAM_STATUS_NOT_READY: return "not_ready";
  case XVRAM_STATUS_TIMEOUT: return "timeout";
  case XVRAM_STATUS_CORRUPTION: return "corruption";
  case XVRAM_STATUS_CALLBACK_FAILED: return "callback_failed";
  case XVRAM_STATUS_CUDA_ERROR: return "cuda_error";
  case XVRAM_STATUS_CUBLAS_ERROR: return "cublas_error";
  case XVRAM_STATUS_POISONED: return "poisoned";
  case XVRAM_STATUS_CLEANUP_FAILED: return "cleanup_failed";
  case XVRAM_STATUS_CLOSED: return "closed";
  case XVRAM_STATUS_CANCELLED: return "cancelled";
  case XVRAM_STATUS_INTERNAL: return "internal";
  default: return "unknown";
  }
}

namespace {

template <size_t N>
void copy_text(char (&dst)[N], const std::string& src) noexcept {
  const size_t n = std::min(src.size(), N - 1);
  std::memset(dst, 0, N);
  if (n) std::memcpy(dst, src.data(), n);
}

} // namespace

void write_error_info(const Error& e, xvram_error_info_v1& out) noexcept {
  const uint32_t caller_size = out.struct_size;
  out = XVRAM_ERROR_INFO_V1_INIT;
  out.struct_size = caller_size;
  out.status = e.status;
  out.native_domain = e.native_domain;
  out.native_code = e.native_code;
  copy_text(out.stage, e.stage);
  copy_text(out.operation, e.operation);
  copy_text(out.native_name, e.native_name);
  copy_text(out.message, e.message);
}

Error exception_error(std::string_view operation) noexcept {
  Error e;
  try {
    throw;
  } catch (const std::bad_alloc&) {
    e.status = XVRAM_STATUS_HOST_OUT_OF_MEMORY;
    try {
      e.message = "host allocation failed";
    } catch (...) {
    }
  } catch (const std::exception& ex) {
    e.status = XVRAM_STATUS_INTERNAL;
    try {
      e.message = ex.what();
    } catch (...) {
    }
  } catch (...) {
    e.status = XVRAM_STATUS_INTERNAL;
    try {
      e.message = "unknown C++ exception at ABI boundary";
    } catch (...) {
    }
  }
  try {
    e.stage = "sdk";
    e.operation.assign(operation);
  } catch (...) {
  }
  return e;
}

namespace {

xvram_status publish(const std::shared_ptr<SessionState>& state, const Error& e) noexcept {
  if (e && state) state->record(e);
  return e.status;
}

template <typename F>
xvram_status boundary(const std::shared_ptr<SessionState>& state, std::string_view operation,
                      F&& f) noexcept {
  try {
    return publish(state, f());
  } catch (const std::bad_alloc&) {
    return publish(state, make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, "sdk", operation,
                                     "host allocation failed"));
  } catch (...) {
    return publish(state, exception_error(operation));
  }
}

template <typename S>
bool has_v1_size(const S* s) noexcept {
  return s != nullptr && s->struct_size >= sizeof(S);
}

bool all_zero(const uint64_t* v, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (v[i] != 0) return false;
  return true;
}

bool valid_access_mode(xvram_access_mode m) {
  return m == XVRAM_ACCESS_READ || m == XVRAM_ACCESS_READ_WRITE || m == XVRAM_ACCESS_WRITE_ONLY;
}

// src/sdk/api.cpp:173-207.
Error validate_session_config(const xvram_session_config_v1* c) {
  if (!has_v1_size(c)) return incompatible("session_create", "session config is null or smaller than v1");
  if (c->flags != 0 || c->reserved0 != 0 || !all_zero(c->reserved, 4))
    return invalid("session_create", "unknown flags or non-zero reserved field");
  if (c->context_mode != XVRAM_CONTEXT_ISOLATED && c->context_mode != XVRAM_CONTEXT_ATTACH_CURRENT)
    return invalid("session_create", "invalid context mode");
  if (c->cache_policy != XVRAM_CACHE_POLICY_CLOCK && c->cache_policy != XVRAM_CACHE_POLICY_LRU)
    return invalid("session_create", "invalid cache policy");
  if (c->device_ordinal < 0) return invalid("session_create", "device ordinal must be non-negative");
  if (c->chunk_size_bytes == 0) return invalid("session_create", "chunk size must be non-zero");
  if (c->staging_slots < 2 || c->staging_slots > 8)
    return invalid("session_create", "staging slot count must be in [2, 8]");
  if (c->prefetch_distance > 8) return invalid("session_create", "prefetch distance must be in [0, 8]");
  const uint64_t int64_max = static_cast<uint64_t>(INT64_MAX);
  if (c->budget_poll_ms == 0 || c->budget_poll_ms > int64_max || c->max_transaction_ms > int64_max)
    return invalid("session_create", "budget and transaction durations are out of range");
  return {};
}

// src/sdk/api.cpp:236-276.
Error collect_accesses(const std::shared_ptr<SessionState>& owner, const xvram_access_range_v1* ranges,
                       uint64_t count, const char* operation, std::vector<Session::Access>& out) {
  if (count == 0) return invalid(operation, "at least one access range is required");
  if (ranges == nullptr) return invalid(operation, "range array is null");
  if (count > out.max_size()) return invalid(operation, "range count is too large");
  out.reserve(static_cast<size_t>(count));
  for (uint64_t i = 0; i < count; ++i) {
    const xvram_access_range_v1& r = ranges[i];
    if (r.allocation == nullptr || !r.allocation->backend)
      return invalid(operation, "access range contains a null allocation");
    if (r.allocation->owner.get() != owner.get())
      return invalid(operation, "all access ranges must belong to the session");
    if (!valid_access_mode(r.mode) || r.reserved0 != 0)
      return invalid(operation, "access range has an invalid mode or reserved field");
    if (r.length_bytes == 0) return invalid(operation, "access range length must be non-zero");
    if (r.offset_bytes > UINT64_MAX - r.length_bytes)
      return invalid(operation, "access range overflows uint64");
    out.push_back(Session::Access{r.allocation->backend, r.offset_bytes, r.length_bytes, r.mode});
  }
  return {};
}

// src/sdk/api.cpp:278-302.
Error convert_matrix(const std::shared_ptr<SessionState>& owner, const xvram_matrix_v1& in,
                     MatrixSpec& out) {
  if (in.struct_size < sizeof(xvram_matrix_v1))
    return incompatible("gemm_plan_create", "matrix descriptor is smaller than v1");
  if (in.allocation == nullptr || !in.allocation->backend)
    return invalid("gemm_plan_create", "matrix allocation is null");
  if (in.allocation->owner.get() != owner.get())
    return invalid("gemm_plan_create", "matrix allocation belongs to another session");
  const bool type_ok = in.data_type <= XVRAM_DATA_FP64;
  const bool layout_ok = in.layout == XVRAM_MATRIX_ROW_MAJOR || in.layout == XVRAM_MATRIX_COLUMN_MAJOR;
  if (!type_ok || !layout_ok || in.reserved0 != 0 || !all_zero(in.reserved, 2))
    return invalid("gemm_plan_create", "matrix descriptor has invalid enum or reserved fields");
  if (in.rows == 0 || in.columns == 0 || in.leading_dimension == 0)
    return invalid("gemm_plan_create", "matrix dimensions and leading dimension must be non-zero");
  out.offset_bytes = in.offset_bytes;
  out.rows = in.rows;
  out.columns = in.columns;
  out.leading_dimension = in.leading_dimension;
  out.layout = in.layout;
  out.data_type = in.data_type;
  return {};
}

// ---- entries -----------------------------------------------------------------

const char* XVRAM_CALL status_name_entry(xvram_status s) noexcept { return status_name(s); }

xvram_status XVRAM_CALL session_create_entry(const xvram_session_config_v1* config,
                                             xvram_session* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  return boundary({}, "session_create", [&]() -> Error {
    if (Error e = validate_session_config(config)) return e;
    xvram_session_config_v1 effective = *config;
    if (config->context_mode == XVRAM_CONTEXT_ATTACH_CURRENT) {
      // Reference src/sdk/runtime.cpp:1369-1383: the session runs on what is
      // current on the calling thread at creation (in HIP, the thread's
      // current device and its primary context); device_ordinal is ignored.
      int current = -1;
      if (current_device(&current) != 0 || current < 0)
        return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "session", "capture_context",
                          "no HIP device is current on the calling thread");
      effective.device_ordinal = current;
    }
    auto session = std::make_shared<Session>(effective);
    if (Error e = session->start()) {
      (void)session->close(XVRAM_TIMEOUT_INFINITE);
      return e;
    }
    if (session->chunk_size_bytes() == 0)
      return make_error(XVRAM_STATUS_INTERNAL, "sdk", "session_create",
                        "backend reported a zero effective chunk size");
    auto state = std::make_shared<SessionState>(session, session->chunk_size_bytes(),
                                                config->workspace_cap_bytes);
    auto* handle = new (std::nothrow) xvram_session_t{std::move(state)};
    if (handle == nullptr)
      return make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, "sdk", "session_create",
                        "failed to allocate session handle");
    *out = handle;
    return {};
  });
}

// src/sdk/api.cpp:209-233.
Error validate_session_config_v2(const xvram_session_config_v2* c) {
  if (!has_v1_size(c))
    return incompatible("session_create_v2", "session config is null or smaller than v2");
  if (c->flags != 0 || !all_zero(c->reserved, 8))
    return invalid("session_create_v2", "unknown flags or non-zero reserved field");
  if (Error e = validate_session_config(&c->v1)) return e;
  if (c->compression_mode != XVRAM_COMPRESSION_DISABLED &&
      c->compression_mode != XVRAM_COMPRESSION_ADAPTIVE &&
      c->compression_mode != XVRAM_COMPRESSION_CAPACITY)
    return invalid("session_create_v2", "invalid compression mode");
  if (c->compression_codec != XVRAM_COMPRESSION_CODEC_AUTO &&
      c->compression_codec != XVRAM_COMPRESSION_CODEC_LZ4)
    return invalid("session_create_v2", "invalid compression codec");
  if (c->compression_workspace_cap_bytes == 0 || c->codec_slots < 2 || c->codec_slots > 8 ||
      c->codec_workers == 0 || c->codec_workers > 8)
    return invalid("session_create_v2", "invalid compression workspace, slots, or workers");
  return {};
}

// src/sdk/api.cpp:399-447 and sdk/runtime.cpp:1393-1397: a DISABLED session is
// exactly a v1 session; compression modes are not provided on this device path.
xvram_status XVRAM_CALL session_create_v2_entry(const xvram_session_config_v2* config,
                                                xvram_session* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  const xvram_status checked = boundary({}, "session_create_v2", [&]() -> Error {
    if (Error e = validate_session_config_v2(config)) return e;
    if (config->compression_mode != XVRAM_COMPRESSION_DISABLED)
      return make_error(XVRAM_STATUS_UNSUPPORTED, "session", "session_create_v2",
                        "host compression is not provided on this device path; use "
                        "XVRAM_COMPRESSION_DISABLED");
    return {};
  });
  if (checked != XVRAM_STATUS_SUCCESS) return checked;
  return session_create_entry(&config->v1, out);
}

xvram_status XVRAM_CALL session_get_telemetry_v2_entry(xvram_session s,
                                                       xvram_session_telemetry_v2* out) noexcept {
  if (s == nullptr || !s->state || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "session_get_telemetry_v2", [&]() -> Error {
    const uint32_t caller = out->struct_size;
    xvram_session_telemetry_v2 local{};
    local.struct_size = sizeof(local);
    if (Error e = s->state->backend->telemetry_v2(local)) return e;
    local.struct_size = caller;
    *out = local;
    return {};
  });
}

xvram_status XVRAM_CALL session_get_error_entry(xvram_session s, xvram_error_info_v1* out) noexcept {
  if (s == nullptr || !s->state || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "session_get_error", [&]() -> Error {
    write_error_info(s->state->error(), *out);
    return {};
  });
}

xvram_status XVRAM_CALL session_get_telemetry_entry(xvram_session s,
                                                    xvram_session_telemetry_v1* out) noexcept {
  if (s == nullptr || !s->state || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "session_get_telemetry", [&]() -> Error {
    const uint32_t caller = out->struct_size;
    xvram_session_telemetry_v1 local{};
    local.struct_size = sizeof(local);
    if (Error e = s->state->backend->telemetry(local)) return e;
    local.struct_size = caller;
    *out = local;
    return {};
  });
}

xvram_status XVRAM_CALL session_drain_entry(xvram_session s, uint64_t timeout_ms) noexcept {
  if (s == nullptr || !s->state) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "session_drain", [&]() { return s->state->backend->drain(timeout_ms); });
}

xvram_status XVRAM_CALL session_close_entry(xvram_session s, uint64_t timeout_ms) noexcept {
  if (s == nullptr || !s->state) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "session_close", [&]() -> Error {
    if (s->state->closed.load(std::memory_order_acquire)) return {};
    Error e = s->state->backend->close(timeout_ms);
    if (!e) s->state->closed.store(true, std::memory_order_release);
    return e;
  });
}

void XVRAM_CALL session_release_entry(xvram_session s) noexcept {
  if (s == nullptr) return;
  try {
    if (s->state && !s->state->closed.load(std::memory_order_acquire)) {
      Error e = s->state->backend->close(XVRAM_TIMEOUT_INFINITE);
      if (!e) s->state->closed.store(true, std::memory_order_release);
      else s->state->record(e);
    }
  } catch (...) {
  }
  delete s;
}

xvram_status XVRAM_CALL allocation_create_entry(xvram_session s, const xvram_allocation_desc_v1* d,
                                                xvram_allocation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (s == nullptr || !s->state) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "allocation_create", [&]() -> Error {
    if (!has_v1_size(d))
      return incompatible("allocation_create", "allocation descriptor is null or smaller than v1");
    if (d->size_bytes == 0) return invalid("allocation_create", "allocation size must be non-zero");
    if ((d->flags & ~static_cast<uint32_t>(XVRAM_ALLOCATION_FLAG_ZERO_INITIALIZE)) != 0 ||
        d->reserved0 != 0 || !all_zero(d->reserved, 2))
      return invalid("allocation_create", "unknown flags or non-zero reserved field");
    if (d->priority > XVRAM_ALLOCATION_STREAMING)
      return invalid("allocation_create", "invalid allocation priority");
    if (d->alignment_bytes != 0 && (d->alignment_bytes & (d->alignment_bytes - 1)) != 0)
      return invalid("allocation_create", "alignment must be zero or a power of two");
    if (d->alignment_bytes > s->state->chunk_bytes ||
        (d->alignment_bytes != 0 && s->state->chunk_bytes % d->alignment_bytes != 0))
      return invalid("allocation_create", "alignment must divide the effective runtime chunk size");
    std::shared_ptr<AllocationRecord> rec;
    if (Error e = s->state->backend->allocate(*d, rec)) return e;
    auto* handle = new (std::nothrow) xvram_allocation_t{s->state, rec};
    if (handle == nullptr) {
      try {
        (void)s->state->backend->release(*rec);
      } catch (...) {
      }
      return make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, "sdk", "allocation_create",
                        "failed to allocate handle");
    }
    *out = handle;
    return {};
  });
}

xvram_status XVRAM_CALL allocation_get_info_entry(xvram_allocation a,
                                                  xvram_allocation_info_v1* out) noexcept {
  if (a == nullptr || !a->owner || !a->backend || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(a->owner, "allocation_get_info", [&]() -> Error {
    if (a->backend->released)
      return make_error(XVRAM_STATUS_CLOSED, "allocation", "info", "allocation is released");
    const uint32_t caller = out->struct_size;
    xvram_allocation_info_v1 local{};
    local.struct_size = caller;
    local.allocation_id = a->backend->id;
    local.size_bytes = a->backend->bytes;
    local.alignment_bytes = a->backend->desc.alignment_bytes;
    local.priority = a->backend->desc.priority;
    local.flags = 0;
    // Transactions see each allocation at one device VA reserved on first use
    // and kept until release.
    local.stable_virtual_address = 1;
    *out = local;
    return {};
  });
}

Error live_allocation(xvram_allocation a, const char* op, std::shared_ptr<Session>& session) {
  session = a->backend->owner.lock();
  if (!session || a->backend->released)
    return make_error(XVRAM_STATUS_CLOSED, "allocation", op, "allocation is released");
  return {};
}

xvram_status XVRAM_CALL allocation_write_entry(xvram_allocation a, uint64_t offset, const void* src,
                                               uint64_t bytes) noexcept {
  if (a == nullptr || !a->owner || !a->backend || (bytes != 0 && src == nullptr))
    return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(a->owner, "allocation_write", [&]() -> Error {
    std::shared_ptr<Session> session;
    if (Error e = live_allocation(a, "write", session)) return e;
    if (bytes == 0) return {};
    return session->write(*a->backend, offset, src, bytes);
  });
}

xvram_status XVRAM_CALL allocation_read_entry(xvram_allocation a, uint64_t offset, void* dst,
                                              uint64_t bytes) noexcept {
  if (a == nullptr || !a->owner || !a->backend || (bytes != 0 && dst == nullptr))
    return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(a->owner, "allocation_read", [&]() -> Error {
    std::shared_ptr<Session> session;
    if (Error e = live_allocation(a, "read", session)) return e;
    if (bytes == 0) return {};
    return session->read(*a->backend, offset, dst, bytes);
  });
}

xvram_status XVRAM_CALL allocation_release_entry(xvram_allocation a) noexcept {
  if (a == nullptr || !a->owner || !a->backend) return XVRAM_STATUS_INVALID_ARGUMENT;
  if (a->owner->closed.load(std::memory_order_acquire)) {
    delete a;
    return XVRAM_STATUS_SUCCESS;
  }
  const xvram_status result = boundary(a->owner, "allocation_release", [&]() -> Error {
    bool expected = false;
    if (!a->backend->released.compare_exchange_strong(expected, true)) return {};
    auto session = a->backend->owner.lock();
    if (!session) return {};
    Error e = session->release(*a->backend);
    if (e.status == XVRAM_STATUS_CLOSED) return {};
    if (e) a->backend->released.store(false);
    return e;
  });
  if (result == XVRAM_STATUS_SUCCESS) delete a;
  return result;
}

xvram_status XVRAM_CALL operation_wait_entry(xvram_operation op, uint64_t timeout_ms,
                                             xvram_operation_info_v1* out) noexcept;
void XVRAM_CALL operation_release_entry(xvram_operation op) noexcept;

Error wrap_operation(const std::shared_ptr<SessionState>& owner, std::shared_ptr<Operation> backend,
                     xvram_operation* out) {
  if (!backend)
    return make_error(XVRAM_STATUS_INTERNAL, "sdk", "operation_create",
                      "backend returned success without an operation");
  auto* handle = new (std::nothrow) xvram_operation_t{owner, backend};
  if (handle == nullptr) {
    try {
      (void)backend->cancel();
    } catch (...) {
    }
    return make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, "sdk", "operation_create",
                      "failed to allocate operation handle");
  }
  *out = handle;
  return {};
}

xvram_status XVRAM_CALL prefetch_submit_entry(xvram_session s, const xvram_prefetch_desc_v1* d,
                                              xvram_operation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (s == nullptr || !s->state) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "prefetch_submit", [&]() -> Error {
    if (!has_v1_size(d)) return incompatible("prefetch_submit", "prefetch descriptor is null or smaller than v1");
    if (d->flags != 0 || !all_zero(d->reserved, 2))
      return invalid("prefetch_submit", "unknown flags or non-zero reserved field");
    if (Error e = validate_deadline(d->deadline_ms, "prefetch_submit")) return e;
    std::vector<Session::Access> accesses;
    if (Error e = collect_accesses(s->state, d->ranges, d->range_count, "prefetch_submit", accesses))
      return e;
    std::shared_ptr<Operation> op;
    if (Error e = s->state->backend->submit_prefetch(std::move(accesses), d->deadline_ms, op)) return e;
    return wrap_operation(s->state, std::move(op), out);
  });
}

xvram_status XVRAM_CALL transaction_submit_entry(xvram_session s, const xvram_transaction_desc_v1* d,
                                                 xvram_operation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (s == nullptr || !s->state) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "transaction_submit", [&]() -> Error {
    if (!has_v1_size(d))
      return incompatible("transaction_submit", "transaction descriptor is null or smaller than v1");
    if (d->flags != 0 || !all_zero(d->reserved, 2))
      return invalid("transaction_submit", "unknown flags or non-zero reserved field");
    if (d->callback == nullptr) return invalid("transaction_submit", "transaction callback is null");
    if (d->workspace_bytes > s->state->workspace_cap_bytes)
      return invalid("transaction_submit", "transaction workspace exceeds the session cap");
    if (Error e = validate_deadline(d->deadline_ms, "transaction_submit")) return e;
    std::vector<Session::Access> accesses;
    if (Error e = collect_accesses(s->state, d->ranges, d->range_count, "transaction_submit", accesses))
      return e;
    std::shared_ptr<Operation> op;
    if (Error e = s->state->backend->submit_transaction(std::move(accesses), d->workspace_bytes,
                                                        d->deadline_ms, d->callback, d->user_data, op))
      return e;
    return wrap_operation(s->state, std::move(op), out);
  });
}

xvram_status XVRAM_CALL transaction_execute_entry(xvram_session s, const xvram_transaction_desc_v1* d,
                                                  uint64_t timeout_ms) noexcept {
  xvram_operation op = nullptr;
  const xvram_status submit = transaction_submit_entry(s, d, &op);
  if (submit != XVRAM_STATUS_SUCCESS) return submit;
  xvram_operation_info_v1 info = XVRAM_OPERATION_INFO_V1_INIT;
  const xvram_status wait = operation_wait_entry(op, timeout_ms, &info);
  if (wait != XVRAM_STATUS_SUCCESS) {
    operation_release_entry(op);
    return wait;
  }
  xvram_status result = info.result;
  if (result != XVRAM_STATUS_SUCCESS) {
    result = boundary(op->owner, "transaction_execute", [&]() -> Error {
      Error e = op->backend->error();
      return e ? e : make_error(info.result, "transaction", "execute", "transaction operation failed");
    });
  }
  operation_release_entry(op);
  return result;
}

// gemm_plan_create, with an optional fused epilogue (extension table).
xvram_status create_plan(xvram_session s, const xvram_gemm_desc_v1* d,
                         const xvram_amd_epilogue_v1* epilogue, xvram_gemm_plan* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (s == nullptr || !s->state) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(s->state, "gemm_plan_create", [&]() -> Error {
    if (!has_v1_size(d)) return incompatible("gemm_plan_create", "GEMM descriptor is null or smaller than v1");
    std::shared_ptr<AllocationRecord> bias;
    EpilogueSpec ep;
    if (epilogue != nullptr) {
      if (epilogue->struct_size < sizeof(xvram_amd_epilogue_v1))
        return incompatible("gemm_plan_create", "epilogue descriptor is smaller than v1");
      if (epilogue->flags != 0 || !all_zero(epilogue->reserved, 2))
        return invalid("gemm_plan_create", "unknown epilogue flags or non-zero reserved field");
      if (epilogue->bias != nullptr) {
        if (!epilogue->bias->backend || epilogue->bias->owner.get() != s->state.get())
          return invalid("gemm_plan_create", "bias allocation belongs to another session");
        bias = epilogue->bias->backend;
      }
      ep.bias_offset_bytes = epilogue->bias_offset_bytes;
      ep.bias_axis = epilogue->bias_axis;
      ep.activation = epilogue->activation;
      if (ep.bias_axis != XVRAM_AMD_BIAS_NONE && !bias)
        return invalid("gemm_plan_create", "bias axis given without a bias allocation");
      if (ep.bias_axis == XVRAM_AMD_BIAS_NONE && bias)
        return invalid("gemm_plan_create", "a bias allocation needs a bias axis");
    }
    if (d->flags != 0 || d->reserved0 != 0 || !all_zero(d->reserved, 3))
      return invalid("gemm_plan_create", "unknown GEMM flags or non-zero reserved field");
    const bool ops_ok = d->operation_a <= XVRAM_MATRIX_OP_T && d->operation_b <= XVRAM_MATRIX_OP_T;
    if (!ops_ok || d->compute_mode > XVRAM_COMPUTE_FP64)
      return invalid("gemm_plan_create", "invalid GEMM operation or compute mode");
    if (Error e = validate_deadline(d->deadline_ms, "gemm_plan_create")) return e;
    GemmSpec spec;
    if (Error e = convert_matrix(s->state, d->a, spec.a)) return e;
    if (Error e = convert_matrix(s->state, d->b, spec.b)) return e;
    if (Error e = convert_matrix(s->state, d->c, spec.c)) return e;
    spec.operation_a = d->operation_a;
    spec.operation_b = d->operation_b;
    spec.compute_mode = d->compute_mode;
    spec.alpha = d->alpha;
    spec.beta = d->beta;
    spec.tile_m_hint = d->tile_m_hint;
    spec.tile_n_hint = d->tile_n_hint;
    spec.tile_k_hint = d->tile_k_hint;
    spec.epilogue = ep;
    std::shared_ptr<GemmPlanRecord> rec;
    if (Error e = s->state->backend->create_gemm_plan(spec, d->a.allocation->backend,
                                                      d->b.allocation->backend,
                                                      d->c.allocation->backend, d->deadline_ms, rec,
                                                      bias))
      return e;
    auto* handle = new (std::nothrow) xvram_gemm_plan_t{s->state, rec};
    if (handle == nullptr)
      return make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, "sdk", "gemm_plan_create",
                        "failed to allocate plan handle");
    *out = handle;
    return {};
  });
}

xvram_status XVRAM_CALL gemm_plan_create_entry(xvram_session s, const xvram_gemm_desc_v1* d,
                                               xvram_gemm_plan* out) noexcept {
  return create_plan(s, d, nullptr, out);
}

xvram_status XVRAM_CALL gemm_plan_create_epilogue_entry(xvram_session s,
                                                        const xvram_gemm_desc_v1* d,
                                                        const xvram_amd_epilogue_v1* epilogue,
                                                        xvram_gemm_plan* out) noexcept {
  if (epilogue == nullptr) {
    if (out != nullptr) *out = nullptr;
    return XVRAM_STATUS_INVALID_ARGUMENT;
  }
  return create_plan(s, d, epilogue, out);
}

xvram_status XVRAM_CALL gemm_plan_get_info_entry(xvram_gemm_plan p, xvram_gemm_plan_info_v1* out) noexcept {
  if (p == nullptr || !p->owner || !p->backend || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(p->owner, "gemm_plan_get_info", [&]() -> Error {
    const uint32_t caller = out->struct_size;
    xvram_gemm_plan_info_v1 local = XVRAM_GEMM_PLAN_INFO_V1_INIT;
    const GemmPlanData& plan = p->backend->plan;
    uint64_t m, n, k;
    problem_dims(p->backend->spec, m, n, k);
    local.m = m;
    local.n = n;
    local.k = k;
    // Tile extents in the caller's orientation (m/n swap back for row-major C).
    local.tile_m = plan.problem.swapped ? plan.tn : plan.tm;
    local.tile_n = plan.problem.swapped ? plan.tm : plan.tn;
    local.tile_k = plan.bk;
    // One launch's working set: its C tile and an A and a B panel frame per
    // K panel it covers.
    auto session = p->backend->owner.lock();
    local.maximum_working_set_bytes =
        session ? (1 + 2 * uint64_t{plan.panels_per_launch}) * session->chunk_size_bytes() : 0;
    local.workspace_bytes = 0;
    // Tiles of the plan's geometry (reference planner.cpp:163 tile_count):
    // C tiles x K panels, however many K panels one launch covers.
    local.tile_count = plan.tiles_m * plan.tiles_n * plan.panels_k;
    local.effective_compute_mode = XVRAM_COMPUTE_FP32_STRICT;
    local.uses_cublas_lt = 0;
    local.struct_size = caller;
    *out = local;
    return {};
  });
}

xvram_status XVRAM_CALL gemm_submit_entry(xvram_gemm_plan p, xvram_operation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (p == nullptr || !p->owner || !p->backend) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(p->owner, "gemm_submit", [&]() -> Error {
    auto session = p->backend->owner.lock();
    if (!session) return make_error(XVRAM_STATUS_CLOSED, "gemm", "submit", "session is closed");
    std::shared_ptr<Operation> op;
    if (Error e = session->submit_gemm(p->backend, op)) return e;
    return wrap_operation(p->owner, std::move(op), out);
  });
}

xvram_status XVRAM_CALL gemm_execute_entry(xvram_gemm_plan p, uint64_t timeout_ms) noexcept {
  xvram_operation op = nullptr;
  const xvram_status submit = gemm_submit_entry(p, &op);
  if (submit != XVRAM_STATUS_SUCCESS) return submit;
  xvram_operation_info_v1 info = XVRAM_OPERATION_INFO_V1_INIT;
  const xvram_status wait = operation_wait_entry(op, timeout_ms, &info);
  if (wait != XVRAM_STATUS_SUCCESS) {
    operation_release_entry(op);
    return wait;
  }
  xvram_status result = info.result;
  if (result != XVRAM_STATUS_SUCCESS) {
    result = boundary(op->owner, "gemm_execute", [&]() -> Error {
      Error e = op->backend->error();
      return e ? e : make_error(info.result, "gemm", "execute", "GEMM operation failed");
    });
  }
  operation_release_entry(op);
  return result;
}

void XVRAM_CALL gemm_plan_release_entry(xvram_gemm_plan p) noexcept {
  try {
    delete p;
  } catch (...) {
  }
}

xvram_status XVRAM_CALL operation_poll_entry(xvram_operation op, xvram_operation_info_v1* out) noexcept {
  if (op == nullptr || !op->owner || !op->backend || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(op->owner, "operation_poll", [&]() -> Error {
    const uint32_t caller = out->struct_size;
    xvram_operation_info_v1 local = XVRAM_OPERATION_INFO_V1_INIT;
    Error e = op->backend->poll(local);
    local.struct_size = caller;
    *out = local;
    return e;
  });
}

xvram_status XVRAM_CALL operation_wait_entry(xvram_operation op, uint64_t timeout_ms,
                                             xvram_operation_info_v1* out) noexcept {
  if (op == nullptr || !op->owner || !op->backend || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(op->owner, "operation_wait", [&]() -> Error {
    const uint32_t caller = out->struct_size;
    xvram_operation_info_v1 local = XVRAM_OPERATION_INFO_V1_INIT;
    Error e = op->backend->wait(timeout_ms, local);
    local.struct_size = caller;
    *out = local;
    return e;
  });
}

xvram_status XVRAM_CALL operation_cancel_entry(xvram_operation op) noexcept {
  if (op == nullptr || !op->owner || !op->backend) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(op->owner, "operation_cancel", [&]() { return op->backend->cancel(); });
}

xvram_status XVRAM_CALL operation_get_error_entry(xvram_operation op, xvram_error_info_v1* out) noexcept {
  if (op == nullptr || !op->owner || !op->backend || !has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return boundary(op->owner, "operation_get_error", [&]() -> Error {
    write_error_info(op->backend->error(), *out);
    return {};
  });
}

void XVRAM_CALL operation_release_entry(xvram_operation op) noexcept {
  try {
    delete op;
  } catch (...) {
  }
}

const xvram_api_v1& api_v1() noexcept {
  static const xvram_api_v1 api = [] {
    xvram_api_v1 v{};
    v.struct_size = sizeof(v);
    v.abi_version = XVRAM_ABI_VERSION_1;
    v.status_name = &status_name_entry;
    v.session_create = &session_create_entry;
    v.session_get_error = &session_get_error_entry;
    v.session_get_telemetry = &session_get_telemetry_entry;
    v.session_drain = &session_drain_entry;
    v.session_close = &session_close_entry;
    v.session_release = &session_release_entry;
    v.allocation_create = &allocation_create_entry;
    v.allocation_get_info = &allocation_get_info_entry;
    v.allocation_write = &allocation_write_entry;
    v.allocation_read = &allocation_read_entry;
    v.allocation_release = &allocation_release_entry;
    v.prefetch_submit = &prefetch_submit_entry;
    v.transaction_submit = &transaction_submit_entry;
    v.transaction_execute = &transaction_execute_entry;
    v.gemm_plan_create = &gemm_plan_create_entry;
    v.gemm_plan_get_info = &gemm_plan_get_info_entry;
    v.gemm_submit = &gemm_submit_entry;
    v.gemm_execute = &gemm_execute_entry;
    v.gemm_plan_release = &gemm_plan_release_entry;
    v.operation_poll = &operation_poll_entry;
    v.operation_wait = &operation_wait_entry;
    v.operation_cancel = &operation_cancel_entry;
    v.operation_get_error = &operation_get_error_entry;
    v.operation_release = &operation_release_entry;
    return v;
  }();
  return api;
}

// src/sdk/api.cpp:1002-1013: the v1 table first (its struct_size and
// abi_version describing the v2 table), then the two v2 entries.
const xvram_api_v2& api_v2() {
  static const xvram_api_v2 api = [] {
    xvram_api_v2 v{};
    v.v1 = api_v1();
    v.v1.struct_size = sizeof(v);
    v.v1.abi_version = XVRAM_ABI_VERSION_2;
    v.session_create_v2 = &session_create_v2_entry;
    v.session_get_telemetry_v2 = &session_get_telemetry_v2_entry;
    return v;
  }();
  return api;
}

xvram_status XVRAM_CALL device_get_info_entry(int32_t ordinal,
                                              xvram_amd_device_info_v1* out) noexcept {
  if (!has_v1_size(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  try {
    DeviceInfo info;
    if (int rc = describe_device(ordinal, info)) {
      return rc == 101 /* hipErrorInvalidDevice */ ? XVRAM_STATUS_INVALID_ARGUMENT
                                                   : XVRAM_STATUS_CUDA_ERROR;
    }
    const uint32_t caller = out->struct_size;
    xvram_amd_device_info_v1 local{};
    local.struct_size = caller;
    local.ordinal = ordinal;
    copy_text(local.name, info.name);
    copy_text(local.arch, info.arch);
    copy_text(local.pci_bus_id, info.pci_bus_id);
    local.total_memory_bytes = info.total_memory;
    local.free_memory_bytes = info.free_memory;
    local.granularity_minimum_bytes = info.granularity_minimum;
    local.granularity_recommended_bytes = info.granularity_recommended;
    local.compute_major = static_cast<uint32_t>(info.compute_major);
    local.compute_minor = static_cast<uint32_t>(info.compute_minor);
    local.multiprocessor_count = static_cast<uint32_t>(info.multiprocessors);
    local.vmm_supported = info.vmm_supported ? 1u : 0u;
    local.driver_version = info.driver_version;
    local.runtime_version = info.runtime_version;
    *out = local;
    return XVRAM_STATUS_SUCCESS;
  } catch (...) {
    return exception_error("device_get_info").status;
  }
}

const xvram_amd_ext_v1& ext_v1() {
  static const xvram_amd_ext_v1 ext = [] {
    xvram_amd_ext_v1 v{};
    v.struct_size = sizeof(v);
    v.ext_version = XVRAM_AMD_EXT_VERSION_1;
    v.gemm_plan_create_epilogue = &gemm_plan_create_epilogue_entry;
    v.device_get_info = &device_get_info_entry;
    return v;
  }();
  return ext;
}

} // namespace
} // namespace xvram

extern "C" XVRAM_API xvram_status XVRAM_CALL xvram_get_api(uint32_t requested_abi_version,
                                                           uint32_t caller_api_size, void* out_api) {
  // One table per version; the same argument rules for each (reference
  // src/sdk/api.cpp:967-1035).
  const void* table = nullptr;
  size_t size = 0;
  switch (requested_abi_version) {
  case XVRAM_ABI_VERSION_1:
    table = &xvram::api_v1();
    size = sizeof(xvram_api_v1);
    break;
  case XVRAM_ABI_VERSION_2:
    table = &xvram::api_v2();
    size = sizeof(xvram_api_v2);
    break;
  case XVRAM_AMD_EXT_ABI_VERSION_1:
    // This build's extension table (no reference counterpart), reached
    // through the one export so the library's symbol set stays the
    // reference's.
    table = &xvram::ext_v1();
    size = sizeof(xvram_amd_ext_v1);
    break;
  default:
    return XVRAM_STATUS_INCOMPATIBLE_ABI;
  }
  if (out_api == nullptr || caller_api_size < size) return XVRAM_STATUS_INVALID_ARGUMENT;
  std::memcpy(out_api, table, size);
  return XVRAM_STATUS_SUCCESS;
}
