// api.cpp — the C-ABI boundary: xvram_get_api and the v1, v2 and extension
// function tables.
//
// Stands in for the reference's SDK entry layer (src/sdk/api.cpp). What a
// caller can observe is interface and is kept: which argument mistakes are
// reported, in which order and with which status (api.cpp:124-344); outputs
// that keep the caller's struct_size (:459-475); exceptions that never cross
// the boundary (bad_alloc -> HOST_OUT_OF_MEMORY, anything else -> INTERNAL,
// :109-122); a per-session last-error record; allocation handles that may
// outlive their session (:644-661); synchronous forms = submit + wait +
// release (:782-806, :876-900).
//
// The structure is this build's own:
//  * a handle is the Session itself plus the object it names (`Bound`); the
//    Session keeps the last-error record and the closed flag;
//  * each descriptor is checked against an ordered table of rules, the first
//    broken rule deciding the error;
//  * every entry point runs its body through `guarded`, which turns
//    exceptions into statuses and records failures on the session.
#include <xvram/xvram.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <memory>
#include <new>
#include <utility>
#include <vector>

#include "common.hpp"
#include "session.hpp"

namespace xvram::abi {

// A handle: the session that issued it (kept alive by the handle) and the
// object it names.
template <class Object>
struct Bound {
  std::shared_ptr<Session> session;
  std::shared_ptr<Object> object;
};

} // namespace xvram::abi

struct xvram_session_t {
  std::shared_ptr<xvram::Session> session;
};
struct xvram_allocation_t : xvram::abi::Bound<xvram::AllocationRecord> {};
struct xvram_operation_t : xvram::abi::Bound<xvram::Operation> {};
struct xvram_gemm_plan_t : xvram::abi::Bound<xvram::GemmPlanRecord> {};

namespace xvram::abi {
namespace {

constexpr const char* kStage = "abi";

Error bad_argument(const char* entry, const char* what) {
  return make_error(XVRAM_STATUS_INVALID_ARGUMENT, kStage, entry, what);
}

Error too_old(const char* entry, const char* what) {
  return make_error(XVRAM_STATUS_INCOMPATIBLE_ABI, kStage, entry, what);
}

Error no_host_memory(const char* entry) {
  return make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, kStage, entry,
                    "no host memory left for the handle");
}

// ---- the firewall ----------------------------------------------------------

// Runs an entry point's body. An escaping exception becomes a status
// (exception_error), and a failure is recorded as the session's last error
// when the call names a session.
template <class Body>
xvram_status guarded(Session* session, const char* entry, Body&& body) noexcept {
  Error outcome;
  try {
    outcome = body();
  } catch (...) {
    outcome = exception_error(entry);
  }
  if (outcome && session != nullptr) session->note_failure(outcome);
  return outcome.status;
}

// Writes a whole output record but keeps the struct_size the caller put there
// (a caller with a newer, larger struct keeps its own size).
template <class T>
void deliver(T* out, T value) noexcept {
  value.struct_size = out->struct_size;
  *out = value;
}

// ---- descriptor rules ------------------------------------------------------

template <class T>
bool versioned(const T* p) noexcept {
  return p != nullptr && p->struct_size >= sizeof(T);
}

template <class W, size_t N>
bool zeroed(const W (&words)[N]) noexcept {
  return std::all_of(words, words + N, [](W w) { return w == 0; });
}

// One rule of a descriptor check; a value that breaks it is INVALID_ARGUMENT
// with `complaint` as the message.
template <class T>
struct Rule {
  bool (*holds)(const T&);
  const char* complaint;
};

template <class T, size_t N>
Error first_broken(const Rule<T> (&rules)[N], const T& value, const char* entry) {
  for (const Rule<T>& rule : rules)
    if (!rule.holds(value)) return bad_argument(entry, rule.complaint);
  return {};
}

constexpr uint64_t kLongestMs = static_cast<uint64_t>(INT64_MAX);

using SessionConfig = xvram_session_config_v1;
const Rule<SessionConfig> kSessionConfigRules[] = {
    {[](const SessionConfig& c) { return c.flags == 0 && c.reserved0 == 0 && zeroed(c.reserved); },
     "flags, reserved0 and reserved[] must be zero"},
    {[](const SessionConfig& c) { return c.context_mode <= XVRAM_CONTEXT_ATTACH_CURRENT; },
     "context_mode is neither ISOLATED nor ATTACH_CURRENT"},
    {[](const SessionConfig& c) { return c.cache_policy <= XVRAM_CACHE_POLICY_LRU; },
     "cache_policy is neither CLOCK nor LRU"},
    {[](const SessionConfig& c) { return c.device_ordinal >= 0; }, "device_ordinal is negative"},
    {[](const SessionConfig& c) { return c.chunk_size_bytes != 0; }, "chunk_size_bytes is zero"},
    {[](const SessionConfig& c) { return c.staging_slots >= 2 && c.staging_slots <= 8; },
     "staging_slots lies outside 2..8"},
    {[](const SessionConfig& c) { return c.prefetch_distance <= 8; },
     "prefetch_distance is larger than 8"},
    {[](const SessionConfig& c) {
       return c.budget_poll_ms != 0 && c.budget_poll_ms <= kLongestMs &&
              c.max_transaction_ms <= kLongestMs;
     },
     "budget_poll_ms must lie in 1..INT64_MAX and max_transaction_ms at most INT64_MAX"},
};

Error check_session_config(const SessionConfig* c, const char* entry) {
  if (!versioned(c)) return too_old(entry, "the session config is missing or older than v1");
  return first_broken(kSessionConfigRules, *c, entry);
}

using SessionConfig2 = xvram_session_config_v2;
const Rule<SessionConfig2> kSessionConfig2Rules[] = {
    {[](const SessionConfig2& c) { return c.compression_mode <= XVRAM_COMPRESSION_CAPACITY; },
     "compression_mode is not a known mode"},
    {[](const SessionConfig2& c) { return c.compression_codec <= XVRAM_COMPRESSION_CODEC_LZ4; },
     "compression_codec is not a known codec"},
    {[](const SessionConfig2& c) {
       return c.compression_workspace_cap_bytes != 0 && c.codec_slots >= 2 && c.codec_slots <= 8 &&
              c.codec_workers >= 1 && c.codec_workers <= 8;
     },
     "compression_workspace_cap_bytes must be non-zero, codec_slots 2..8, codec_workers 1..8"},
};

Error check_session_config_v2(const SessionConfig2* c) {
  constexpr const char* entry = "session_create_v2";
  if (!versioned(c)) return too_old(entry, "the v2 session config is missing or older than v2");
  if (c->flags != 0 || !zeroed(c->reserved))
    return bad_argument(entry, "flags and reserved[] of the v2 config must be zero");
  if (Error e = check_session_config(&c->v1, "session_create")) return e;
  return first_broken(kSessionConfig2Rules, *c, entry);
}

using AllocationDesc = xvram_allocation_desc_v1;
const Rule<AllocationDesc> kAllocationRules[] = {
    {[](const AllocationDesc& d) { return d.size_bytes != 0; }, "size_bytes is zero"},
    {[](const AllocationDesc& d) {
       return (d.flags & ~uint32_t{XVRAM_ALLOCATION_FLAG_ZERO_INITIALIZE}) == 0 &&
              d.reserved0 == 0 && zeroed(d.reserved);
     },
     "unknown allocation flags, or reserved fields not zero"},
    {[](const AllocationDesc& d) { return d.priority <= XVRAM_ALLOCATION_STREAMING; },
     "priority is not NORMAL, HOT or STREAMING"},
    {[](const AllocationDesc& d) { return (d.alignment_bytes & (d.alignment_bytes - 1)) == 0; },
     "alignment_bytes is neither zero nor a power of two"},
};

using Matrix = xvram_matrix_v1;
const Rule<Matrix> kMatrixRules[] = {
    {[](const Matrix& m) {
       return m.data_type <= XVRAM_DATA_FP64 && m.layout <= XVRAM_MATRIX_COLUMN_MAJOR &&
              m.reserved0 == 0 && zeroed(m.reserved);
     },
     "a matrix has an unknown data type or layout, or non-zero reserved fields"},
    {[](const Matrix& m) { return m.rows != 0 && m.columns != 0 && m.leading_dimension != 0; },
     "a matrix has zero rows, columns or leading dimension"},
};

using GemmDesc = xvram_gemm_desc_v1;
const Rule<GemmDesc> kGemmRules[] = {
    {[](const GemmDesc& d) { return d.flags == 0 && d.reserved0 == 0 && zeroed(d.reserved); },
     "GEMM flags, reserved0 and reserved[] must be zero"},
    {[](const GemmDesc& d) {
       return d.operation_a <= XVRAM_MATRIX_OP_T && d.operation_b <= XVRAM_MATRIX_OP_T &&
              d.compute_mode <= XVRAM_COMPUTE_FP64;
     },
     "operation_a/operation_b is not N or T, or compute_mode is unknown"},
};

using AccessRange = xvram_access_range_v1;
const Rule<AccessRange> kAccessRules[] = {
    {[](const AccessRange& r) { return r.mode <= XVRAM_ACCESS_WRITE_ONLY && r.reserved0 == 0; },
     "an access range has an unknown mode or a non-zero reserved0"},
    {[](const AccessRange& r) { return r.length_bytes != 0; }, "an access range is empty"},
    {[](const AccessRange& r) { return r.offset_bytes <= UINT64_MAX - r.length_bytes; },
     "an access range ends beyond 2^64"},
};

// The access list of a prefetch or transaction: at least one range, every
// range naming a live handle of `session`.
Error gather_accesses(Session* session, const AccessRange* ranges, uint64_t count,
                      const char* entry, std::vector<Session::Access>& out) {
  if (count == 0) return bad_argument(entry, "range_count is zero");
  if (ranges == nullptr) return bad_argument(entry, "ranges is NULL");
  if (count > out.max_size()) return bad_argument(entry, "range_count is too large");
  out.reserve(static_cast<size_t>(count));
  for (uint64_t i = 0; i < count; ++i) {
    const AccessRange& r = ranges[i];
    if (r.allocation == nullptr || !r.allocation->object)
      return bad_argument(entry, "an access range names no allocation");
    if (r.allocation->session.get() != session)
      return bad_argument(entry, "an access range names an allocation of another session");
    if (Error e = first_broken(kAccessRules, r, entry)) return e;
    out.push_back(Session::Access{r.allocation->object, r.offset_bytes, r.length_bytes, r.mode});
  }
  return {};
}

Error read_matrix(Session* session, const Matrix& in, MatrixSpec& out) {
  constexpr const char* entry = "gemm_plan_create";
  if (in.struct_size < sizeof(Matrix)) return too_old(entry, "a matrix descriptor is older than v1");
  if (in.allocation == nullptr || !in.allocation->object)
    return bad_argument(entry, "a matrix names no allocation");
  if (in.allocation->session.get() != session)
    return bad_argument(entry, "a matrix names an allocation of another session");
  if (Error e = first_broken(kMatrixRules, in, entry)) return e;
  out.offset_bytes = in.offset_bytes;
  out.rows = in.rows;
  out.columns = in.columns;
  out.leading_dimension = in.leading_dimension;
  out.layout = in.layout;
  out.data_type = in.data_type;
  return {};
}

// The extension's epilogue descriptor (no reference counterpart).
Error read_epilogue(Session* session, const xvram_amd_epilogue_v1& in, EpilogueSpec& out,
                    std::shared_ptr<AllocationRecord>& bias) {
  constexpr const char* entry = "gemm_plan_create";
  if (in.struct_size < sizeof(xvram_amd_epilogue_v1))
    return too_old(entry, "the epilogue descriptor is older than v1");
  if (in.flags != 0 || !zeroed(in.reserved))
    return bad_argument(entry, "epilogue flags and reserved[] must be zero");
  if (in.bias != nullptr) {
    if (!in.bias->object || in.bias->session.get() != session)
      return bad_argument(entry, "the bias names an allocation of another session");
    bias = in.bias->object;
  }
  if (in.bias_axis != XVRAM_AMD_BIAS_NONE && !bias)
    return bad_argument(entry, "a bias axis is given without a bias allocation");
  if (in.bias_axis == XVRAM_AMD_BIAS_NONE && bias)
    return bad_argument(entry, "a bias allocation is given without a bias axis");
  out.bias_offset_bytes = in.bias_offset_bytes;
  out.bias_axis = in.bias_axis;
  out.activation = in.activation;
  return {};
}

// The extension's device-memory GEMM descriptor (no reference counterpart).
using DeviceGemm = xvram_amd_sgemm_v1;
constexpr uint64_t kInt32Max = static_cast<uint64_t>(INT32_MAX);
bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }
const Rule<DeviceGemm> kDeviceGemmRules[] = {
    {[](const DeviceGemm& d) { return d.flags == 0 && zeroed(d.reserved); },
     "flags and reserved[] must be zero"},
    {[](const DeviceGemm& d) {
       return d.operation_a <= XVRAM_MATRIX_OP_T && d.operation_b <= XVRAM_MATRIX_OP_T &&
              d.bias_axis <= XVRAM_AMD_BIAS_PER_COLUMN && d.activation <= XVRAM_AMD_ACTIVATION_RELU;
     },
     "an operation, bias axis or activation is not a known value"},
    {[](const DeviceGemm& d) { return d.a != nullptr && d.b != nullptr && d.c != nullptr; },
     "a, b and c must be device pointers"},
    {[](const DeviceGemm& d) {
       return d.m > 0 && d.n > 0 && d.k > 0 && d.m <= kInt32Max && d.n <= kInt32Max &&
              d.k <= kInt32Max;
     },
     "m, n and k must lie in 1..2^31-1"},
    {[](const DeviceGemm& d) {
       const uint64_t a_rows = d.operation_a == XVRAM_MATRIX_OP_N ? d.m : d.k;
       const uint64_t b_rows = d.operation_b == XVRAM_MATRIX_OP_N ? d.k : d.n;
       return d.lda >= a_rows && d.ldb >= b_rows && d.ldc >= d.m && d.lda % 4 == 0 &&
              d.ldb % 4 == 0 && d.ldc % 4 == 0;
     },
     "leading dimensions must cover the stored rows and be multiples of 4 floats"},
    {[](const DeviceGemm& d) {
       return aligned16(d.a) && aligned16(d.b) && aligned16(d.c) && aligned16(d.workspace);
     },
     "a, b, c and the workspace must be 16-byte aligned"},
    {[](const DeviceGemm& d) { return (d.bias_axis != XVRAM_AMD_BIAS_NONE) == (d.bias != nullptr); },
     "a bias vector needs a bias axis and a bias axis needs a bias vector"},
    {[](const DeviceGemm& d) { return d.workspace != nullptr || d.workspace_bytes == 0; },
     "workspace_bytes is given without a workspace"},
};

Error read_device_gemm(const DeviceGemm* d, const char* entry, kernels::SgemmLaunch& out) {
  if (!versioned(d)) return too_old(entry, "the device GEMM descriptor is missing or older than v1");
  if (Error e = first_broken(kDeviceGemmRules, *d, entry)) return e;
  out.a = d->a;
  out.b = d->b;
  out.c = d->c;
  out.lda = static_cast<int64_t>(d->lda);
  out.ldb = static_cast<int64_t>(d->ldb);
  out.ldc = static_cast<int64_t>(d->ldc);
  out.m = static_cast<int>(d->m);
  out.n = static_cast<int>(d->n);
  out.k = static_cast<int>(d->k);
  out.alpha = static_cast<float>(d->alpha);
  out.beta = static_cast<float>(d->beta);
  out.a_kcontig = d->operation_a == XVRAM_MATRIX_OP_T;
  out.b_ncontig = d->operation_b == XVRAM_MATRIX_OP_T;
  out.padded = true;
  if (d->bias_axis == XVRAM_AMD_BIAS_PER_ROW) out.bias_row = d->bias;
  if (d->bias_axis == XVRAM_AMD_BIAS_PER_COLUMN) out.bias_col = d->bias;
  out.relu = d->activation == XVRAM_AMD_ACTIVATION_RELU;
  out.workspace = static_cast<float*>(d->workspace);
  out.workspace_bytes = d->workspace_bytes;
  return {};
}

Error device_gemm_failure(int rc, const char* entry) {
  if (rc == kNoDevice)
    return make_error(XVRAM_STATUS_UNSUPPORTED, kStage, entry,
                      "this build has no GPU (host simulation)");
  if (rc == kScratchTooSmall)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, kStage, entry,
                      "the split's partials exceed the 64 MiB static scratch; pass a workspace");
  Error e = make_error(rc == 2 /* hipErrorOutOfMemory */ ? XVRAM_STATUS_DEVICE_OUT_OF_MEMORY
                                                          : XVRAM_STATUS_CUDA_ERROR,
                       kStage, entry, "the HIP runtime refused the launch or its workspace");
  e.native_domain = XVRAM_NATIVE_ERROR_CUDA;
  e.native_code = rc;
  return e;
}

// ---- handles -----------------------------------------------------------------

bool live(const xvram_session_t* h) { return h != nullptr && h->session; }
template <class Object>
bool live(const Bound<Object>* h) {
  return h != nullptr && h->session && h->object;
}

Error hand_out_operation(const std::shared_ptr<Session>& session, std::shared_ptr<Operation> op,
                         xvram_operation* out, const char* entry) {
  auto* handle = new (std::nothrow) xvram_operation_t{{session, op}};
  if (handle == nullptr) {
    (void)op->cancel(); // queued work nobody can wait for; a running one drains normally
    return no_host_memory(entry);
  }
  *out = handle;
  return {};
}

// The synchronous form of a submission: submit, wait, release the operation.
// A wait that runs out returns TIMEOUT and leaves the operation running.
template <class Submit>
xvram_status run_to_end(Submit&& submit, uint64_t timeout_ms, const char* entry) {
  xvram_operation handle = nullptr;
  if (const xvram_status s = submit(&handle); s != XVRAM_STATUS_SUCCESS) return s;
  std::unique_ptr<xvram_operation_t> owned(handle);
  return guarded(owned->session.get(), entry, [&]() -> Error {
    Operation& op = *owned->object;
    if (!op.settled_within(timeout_ms))
      return make_error(XVRAM_STATUS_TIMEOUT, "operation", "wait",
                        "the operation did not finish within the timeout");
    if (Error e = op.failure()) return e;
    const xvram_operation_info_v1 info = op.snapshot();
    if (info.result == XVRAM_STATUS_SUCCESS) return {};
    return make_error(info.result, "operation", entry, "the operation failed");
  });
}

// ---- entry points ------------------------------------------------------------

namespace entry {

const char* XVRAM_CALL status_name(xvram_status status) noexcept {
  return xvram::status_name(status);
}

xvram_status XVRAM_CALL session_create(const xvram_session_config_v1* config,
                                       xvram_session* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  return guarded(nullptr, "session_create", [&]() -> Error {
    if (Error e = check_session_config(config, "session_create")) return e;
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
      return make_error(XVRAM_STATUS_INTERNAL, kStage, "session_create",
                        "the runtime set up a zero frame size");
    auto* handle = new (std::nothrow) xvram_session_t{std::move(session)};
    if (handle == nullptr) return no_host_memory("session_create");
    *out = handle;
    return {};
  });
}

// A v2 session with compression DISABLED is exactly a v1 session (reference
// src/sdk/runtime.cpp:1393-1397); the host-compression modes are not
// provided on this device path.
xvram_status XVRAM_CALL session_create_v2(const xvram_session_config_v2* config,
                                          xvram_session* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  const xvram_status checked = guarded(nullptr, "session_create_v2", [&]() -> Error {
    if (Error e = check_session_config_v2(config)) return e;
    if (config->compression_mode != XVRAM_COMPRESSION_DISABLED)
      return make_error(XVRAM_STATUS_UNSUPPORTED, "session", "session_create_v2",
                        "host compression is not provided on this device path; use "
                        "XVRAM_COMPRESSION_DISABLED");
    return {};
  });
  if (checked != XVRAM_STATUS_SUCCESS) return checked;
  return session_create(&config->v1, out);
}

xvram_status XVRAM_CALL session_get_error(xvram_session s, xvram_error_info_v1* out) noexcept {
  if (!live(s) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(s->session.get(), "session_get_error", [&]() -> Error {
    write_error_info(s->session->last_failure(), *out);
    return {};
  });
}

xvram_status XVRAM_CALL session_get_telemetry(xvram_session s,
                                              xvram_session_telemetry_v1* out) noexcept {
  if (!live(s) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(s->session.get(), "session_get_telemetry", [&]() -> Error {
    xvram_session_telemetry_v1 t{};
    if (Error e = s->session->telemetry(t)) return e;
    deliver(out, t);
    return {};
  });
}

xvram_status XVRAM_CALL session_get_telemetry_v2(xvram_session s,
                                                 xvram_session_telemetry_v2* out) noexcept {
  if (!live(s) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(s->session.get(), "session_get_telemetry_v2", [&]() -> Error {
    xvram_session_telemetry_v2 t{};
    if (Error e = s->session->telemetry_v2(t)) return e;
    deliver(out, t);
    return {};
  });
}

xvram_status XVRAM_CALL session_drain(xvram_session s, uint64_t timeout_ms) noexcept {
  if (!live(s)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(s->session.get(), "session_drain",
                 [&]() { return s->session->drain(timeout_ms); });
}

xvram_status XVRAM_CALL session_close(xvram_session s, uint64_t timeout_ms) noexcept {
  if (!live(s)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(s->session.get(), "session_close",
                 [&]() { return s->session->close(timeout_ms); });
}

// Closes without a bound when the caller has not, then frees the handle;
// other handles keep the closed session's records alive until released.
void XVRAM_CALL session_release(xvram_session s) noexcept {
  if (s == nullptr) return;
  if (s->session) (void)guarded(s->session.get(), "session_release", [&]() {
    return s->session->close(XVRAM_TIMEOUT_INFINITE);
  });
  delete s;
}

xvram_status XVRAM_CALL allocation_create(xvram_session s, const xvram_allocation_desc_v1* d,
                                          xvram_allocation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (!live(s)) return XVRAM_STATUS_INVALID_ARGUMENT;
  constexpr const char* entry = "allocation_create";
  return guarded(s->session.get(), entry, [&]() -> Error {
    if (!versioned(d)) return too_old(entry, "the allocation descriptor is missing or older than v1");
    if (Error e = first_broken(kAllocationRules, *d, entry)) return e;
    const uint64_t frame = s->session->chunk_size_bytes();
    if (d->alignment_bytes > frame || (d->alignment_bytes != 0 && frame % d->alignment_bytes != 0))
      return bad_argument(entry, "alignment_bytes does not divide the session's frame size");
    std::shared_ptr<AllocationRecord> record;
    if (Error e = s->session->allocate(*d, record)) return e;
    auto* handle = new (std::nothrow) xvram_allocation_t{{s->session, record}};
    if (handle == nullptr) {
      // The host backing exists already: give it back rather than leak it.
      record->released = true;
      (void)s->session->release(*record);
      return no_host_memory(entry);
    }
    *out = handle;
    return {};
  });
}

xvram_status XVRAM_CALL allocation_get_info(xvram_allocation a,
                                            xvram_allocation_info_v1* out) noexcept {
  if (!live(a) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(a->session.get(), "allocation_get_info", [&]() -> Error {
    const AllocationRecord& r = *a->object;
    if (r.released)
      return make_error(XVRAM_STATUS_CLOSED, "allocation", "info", "the allocation was released");
    xvram_allocation_info_v1 info{};
    info.allocation_id = r.id;
    info.size_bytes = r.bytes;
    info.alignment_bytes = r.desc.alignment_bytes;
    info.priority = r.desc.priority;
    // Transactions see each allocation at one device VA, reserved on first
    // use and kept until release.
    info.stable_virtual_address = 1;
    deliver(out, info);
    return {};
  });
}

// Host copies into and out of an allocation's authoritative host store.
template <class Copy>
xvram_status host_copy(xvram_allocation a, const char* entry, const char* verb, Copy&& copy) {
  return guarded(a->session.get(), entry, [&]() -> Error {
    std::shared_ptr<Session> owner = a->object->owner.lock();
    if (!owner || a->object->released)
      return make_error(XVRAM_STATUS_CLOSED, "allocation", verb, "the allocation was released");
    return copy(*owner);
  });
}

xvram_status XVRAM_CALL allocation_write(xvram_allocation a, uint64_t offset, const void* src,
                                         uint64_t bytes) noexcept {
  if (!live(a) || (bytes != 0 && src == nullptr)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return host_copy(a, "allocation_write", "write", [&](Session& owner) -> Error {
    return bytes == 0 ? Error{} : owner.write(*a->object, offset, src, bytes);
  });
}

xvram_status XVRAM_CALL allocation_read(xvram_allocation a, uint64_t offset, void* dst,
                                        uint64_t bytes) noexcept {
  if (!live(a) || (bytes != 0 && dst == nullptr)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return host_copy(a, "allocation_read", "read", [&](Session& owner) -> Error {
    return bytes == 0 ? Error{} : owner.read(*a->object, offset, dst, bytes);
  });
}

// After a successful session close every allocation is gone with the
// runtime, so releasing a handle is then local and always succeeds. Before
// that, the first release frees the host store; the handle is freed only on
// success, so a failed release can be retried.
xvram_status XVRAM_CALL allocation_release(xvram_allocation a) noexcept {
  if (!live(a)) return XVRAM_STATUS_INVALID_ARGUMENT;
  if (a->session->closed()) {
    delete a;
    return XVRAM_STATUS_SUCCESS;
  }
  const xvram_status status = guarded(a->session.get(), "allocation_release", [&]() -> Error {
    AllocationRecord& r = *a->object;
    if (r.released.exchange(true)) return {};
    Error e = a->session->release(r);
    if (e.status == XVRAM_STATUS_CLOSED) return {};
    if (e) r.released = false;
    return e;
  });
  if (status == XVRAM_STATUS_SUCCESS) delete a;
  return status;
}

xvram_status XVRAM_CALL prefetch_submit(xvram_session s, const xvram_prefetch_desc_v1* d,
                                        xvram_operation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (!live(s)) return XVRAM_STATUS_INVALID_ARGUMENT;
  constexpr const char* entry = "prefetch_submit";
  return guarded(s->session.get(), entry, [&]() -> Error {
    if (!versioned(d)) return too_old(entry, "the prefetch descriptor is missing or older than v1");
    if (d->flags != 0 || !zeroed(d->reserved))
      return bad_argument(entry, "prefetch flags and reserved[] must be zero");
    if (Error e = check_deadline_ms(d->deadline_ms, entry)) return e;
    std::vector<Session::Access> accesses;
    if (Error e = gather_accesses(s->session.get(), d->ranges, d->range_count, entry, accesses))
      return e;
    std::shared_ptr<Operation> op;
    if (Error e = s->session->submit_prefetch(std::move(accesses), d->deadline_ms, op)) return e;
    return hand_out_operation(s->session, std::move(op), out, entry);
  });
}

xvram_status XVRAM_CALL transaction_submit(xvram_session s, const xvram_transaction_desc_v1* d,
                                           xvram_operation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (!live(s)) return XVRAM_STATUS_INVALID_ARGUMENT;
  constexpr const char* entry = "transaction_submit";
  return guarded(s->session.get(), entry, [&]() -> Error {
    if (!versioned(d))
      return too_old(entry, "the transaction descriptor is missing or older than v1");
    if (d->flags != 0 || !zeroed(d->reserved))
      return bad_argument(entry, "transaction flags and reserved[] must be zero");
    if (d->callback == nullptr) return bad_argument(entry, "callback is NULL");
    if (d->workspace_bytes > s->session->config().workspace_cap_bytes)
      return bad_argument(entry, "workspace_bytes exceeds the session's workspace_cap_bytes");
    if (Error e = check_deadline_ms(d->deadline_ms, entry)) return e;
    std::vector<Session::Access> accesses;
    if (Error e = gather_accesses(s->session.get(), d->ranges, d->range_count, entry, accesses))
      return e;
    std::shared_ptr<Operation> op;
    if (Error e = s->session->submit_transaction(std::move(accesses), d->workspace_bytes,
                                                 d->deadline_ms, d->callback, d->user_data, op))
      return e;
    return hand_out_operation(s->session, std::move(op), out, entry);
  });
}

xvram_status XVRAM_CALL transaction_execute(xvram_session s, const xvram_transaction_desc_v1* d,
                                            uint64_t timeout_ms) noexcept {
  return run_to_end([&](xvram_operation* op) { return transaction_submit(s, d, op); }, timeout_ms,
                    "transaction_execute");
}

// gemm_plan_create, with the extension's epilogue when `epilogue` is given.
xvram_status create_plan(xvram_session s, const xvram_gemm_desc_v1* d,
                         const xvram_amd_epilogue_v1* epilogue, xvram_gemm_plan* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (!live(s)) return XVRAM_STATUS_INVALID_ARGUMENT;
  constexpr const char* entry = "gemm_plan_create";
  return guarded(s->session.get(), entry, [&]() -> Error {
    if (!versioned(d)) return too_old(entry, "the GEMM descriptor is missing or older than v1");
    if (Error e = first_broken(kGemmRules, *d, entry)) return e;
    if (Error e = check_deadline_ms(d->deadline_ms, entry)) return e;
    GemmSpec spec;
    const std::pair<const Matrix*, MatrixSpec*> operands[] = {
        {&d->a, &spec.a}, {&d->b, &spec.b}, {&d->c, &spec.c}};
    for (const auto& [in, spec_out] : operands)
      if (Error e = read_matrix(s->session.get(), *in, *spec_out)) return e;
    std::shared_ptr<AllocationRecord> bias;
    if (epilogue != nullptr)
      if (Error e = read_epilogue(s->session.get(), *epilogue, spec.epilogue, bias)) return e;
    spec.operation_a = d->operation_a;
    spec.operation_b = d->operation_b;
    spec.compute_mode = d->compute_mode;
    spec.alpha = d->alpha;
    spec.beta = d->beta;
    spec.tile_m_hint = d->tile_m_hint;
    spec.tile_n_hint = d->tile_n_hint;
    spec.tile_k_hint = d->tile_k_hint;
    std::shared_ptr<GemmPlanRecord> plan;
    if (Error e = s->session->create_gemm_plan(spec, d->a.allocation->object,
                                               d->b.allocation->object, d->c.allocation->object,
                                               d->deadline_ms, plan, bias))
      return e;
    auto* handle = new (std::nothrow) xvram_gemm_plan_t{{s->session, plan}};
    if (handle == nullptr) return no_host_memory(entry);
    *out = handle;
    return {};
  });
}

xvram_status XVRAM_CALL gemm_plan_create(xvram_session s, const xvram_gemm_desc_v1* d,
                                         xvram_gemm_plan* out) noexcept {
  return create_plan(s, d, nullptr, out);
}

xvram_status XVRAM_CALL gemm_plan_create_epilogue(xvram_session s, const xvram_gemm_desc_v1* d,
                                                  const xvram_amd_epilogue_v1* epilogue,
                                                  xvram_gemm_plan* out) noexcept {
  if (epilogue == nullptr) {
    if (out != nullptr) *out = nullptr;
    return XVRAM_STATUS_INVALID_ARGUMENT;
  }
  return create_plan(s, d, epilogue, out);
}

xvram_status XVRAM_CALL gemm_plan_get_info(xvram_gemm_plan p,
                                           xvram_gemm_plan_info_v1* out) noexcept {
  if (!live(p) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(p->session.get(), "gemm_plan_get_info", [&]() -> Error {
    const GemmPlanRecord& record = *p->object;
    const GemmPlanData& plan = record.plan;
    xvram_gemm_plan_info_v1 info = XVRAM_GEMM_PLAN_INFO_V1_INIT;
    problem_dims(record.spec, info.m, info.n, info.k);
    // Tile extents in the caller's orientation (m/n swap back for row-major C).
    info.tile_m = plan.problem.swapped ? plan.tn : plan.tm;
    info.tile_n = plan.problem.swapped ? plan.tm : plan.tn;
    info.tile_k = plan.bk;
    // One launch's working set: its C tile, an A and a B panel frame per K
    // panel it covers, and the frame of split-K partials when the plan's
    // launches split K (all from the cache's frames; the workspace cap stays
    // unused by GEMMs).
    info.maximum_working_set_bytes =
        (1 + 2 * uint64_t{plan.panels_per_launch} + (plan.scratch ? 1 : 0)) *
        p->session->chunk_size_bytes();
    info.workspace_bytes = 0;
    // Tiles of the plan's geometry (reference planner.cpp:163 tile_count):
    // C tiles x K panels, however many K panels one launch covers.
    info.tile_count = record.tile_count();
    info.effective_compute_mode = XVRAM_COMPUTE_FP32_STRICT;
    info.uses_cublas_lt = 0;
    deliver(out, info);
    return {};
  });
}

xvram_status XVRAM_CALL gemm_submit(xvram_gemm_plan p, xvram_operation* out) noexcept {
  if (out == nullptr) return XVRAM_STATUS_INVALID_ARGUMENT;
  *out = nullptr;
  if (!live(p)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(p->session.get(), "gemm_submit", [&]() -> Error {
    std::shared_ptr<Operation> op;
    if (Error e = p->session->submit_gemm(p->object, op)) return e;
    return hand_out_operation(p->session, std::move(op), out, "gemm_submit");
  });
}

xvram_status XVRAM_CALL gemm_execute(xvram_gemm_plan p, uint64_t timeout_ms) noexcept {
  return run_to_end([&](xvram_operation* op) { return gemm_submit(p, op); }, timeout_ms,
                    "gemm_execute");
}

void XVRAM_CALL gemm_plan_release(xvram_gemm_plan p) noexcept { delete p; }

xvram_status XVRAM_CALL operation_poll(xvram_operation op, xvram_operation_info_v1* out) noexcept {
  if (!live(op) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(op->session.get(), "operation_poll", [&]() -> Error {
    deliver(out, op->object->snapshot());
    return {};
  });
}

// Fills `out` whether or not the operation finished; TIMEOUT when it did not.
xvram_status XVRAM_CALL operation_wait(xvram_operation op, uint64_t timeout_ms,
                                       xvram_operation_info_v1* out) noexcept {
  if (!live(op) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(op->session.get(), "operation_wait", [&]() -> Error {
    const bool settled = op->object->settled_within(timeout_ms);
    deliver(out, op->object->snapshot());
    if (settled) return {};
    return make_error(XVRAM_STATUS_TIMEOUT, "operation", "wait",
                      "the operation did not finish within the timeout");
  });
}

xvram_status XVRAM_CALL operation_cancel(xvram_operation op) noexcept {
  if (!live(op)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(op->session.get(), "operation_cancel", [&]() { return op->object->cancel(); });
}

xvram_status XVRAM_CALL operation_get_error(xvram_operation op, xvram_error_info_v1* out) noexcept {
  if (!live(op) || !versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  return guarded(op->session.get(), "operation_get_error", [&]() -> Error {
    write_error_info(op->object->failure(), *out);
    return {};
  });
}

void XVRAM_CALL operation_release(xvram_operation op) noexcept { delete op; }

xvram_status XVRAM_CALL sgemm_device(const xvram_amd_sgemm_v1* desc, void* stream) noexcept {
  constexpr const char* entry = "sgemm_device";
  return guarded(nullptr, entry, [&]() -> Error {
    kernels::SgemmLaunch launch;
    if (Error e = read_device_gemm(desc, entry, launch)) return e;
    if (const int rc = direct_sgemm(launch, stream)) return device_gemm_failure(rc, entry);
    return {};
  });
}

// sgemm_device without any allocation (the static per-GPU scratch serves a
// split the caller's workspace cannot hold).
xvram_status XVRAM_CALL sgemm_device_no_alloc(const xvram_amd_sgemm_v1* desc, void* stream) noexcept {
  constexpr const char* entry = "sgemm_device_no_alloc";
  return guarded(nullptr, entry, [&]() -> Error {
    kernels::SgemmLaunch launch;
    if (Error e = read_device_gemm(desc, entry, launch)) return e;
    if (const int rc = direct_sgemm_no_alloc(launch, stream)) return device_gemm_failure(rc, entry);
    return {};
  });
}

xvram_status XVRAM_CALL device_get_info(int32_t ordinal, xvram_amd_device_info_v1* out) noexcept {
  if (!versioned(out)) return XVRAM_STATUS_INVALID_ARGUMENT;
  try {
    DeviceInfo d;
    if (const int rc = describe_device(ordinal, d))
      return rc == 101 /* hipErrorInvalidDevice */ ? XVRAM_STATUS_INVALID_ARGUMENT
                                                   : XVRAM_STATUS_CUDA_ERROR;
    xvram_amd_device_info_v1 info{};
    info.ordinal = ordinal;
    std::snprintf(info.name, sizeof info.name, "%s", d.name.c_str());
    std::snprintf(info.arch, sizeof info.arch, "%s", d.arch.c_str());
    std::snprintf(info.pci_bus_id, sizeof info.pci_bus_id, "%s", d.pci_bus_id.c_str());
    info.total_memory_bytes = d.total_memory;
    info.free_memory_bytes = d.free_memory;
    info.granularity_minimum_bytes = d.granularity_minimum;
    info.granularity_recommended_bytes = d.granularity_recommended;
    info.compute_major = static_cast<uint32_t>(d.compute_major);
    info.compute_minor = static_cast<uint32_t>(d.compute_minor);
    info.multiprocessor_count = static_cast<uint32_t>(d.multiprocessors);
    info.vmm_supported = d.vmm_supported ? 1u : 0u;
    info.driver_version = d.driver_version;
    info.runtime_version = d.runtime_version;
    deliver(out, info);
    return XVRAM_STATUS_SUCCESS;
  } catch (...) {
    return exception_error("device_get_info").status;
  }
}

} // namespace entry

// ---- the tables ----------------------------------------------------------------

// The v1 table with its header describing a table of `size` bytes, version
// `version` (the v2 table embeds v1 first, headed with v2's size and version).
xvram_api_v1 table_v1(uint32_t size, uint32_t version) {
  return xvram_api_v1{
      .struct_size = size,
      .abi_version = version,
      .status_name = entry::status_name,
      .session_create = entry::session_create,
      .session_get_error = entry::session_get_error,
      .session_get_telemetry = entry::session_get_telemetry,
      .session_drain = entry::session_drain,
      .session_close = entry::session_close,
      .session_release = entry::session_release,
      .allocation_create = entry::allocation_create,
      .allocation_get_info = entry::allocation_get_info,
      .allocation_write = entry::allocation_write,
      .allocation_read = entry::allocation_read,
      .allocation_release = entry::allocation_release,
      .prefetch_submit = entry::prefetch_submit,
      .transaction_submit = entry::transaction_submit,
      .transaction_execute = entry::transaction_execute,
      .gemm_plan_create = entry::gemm_plan_create,
      .gemm_plan_get_info = entry::gemm_plan_get_info,
      .gemm_submit = entry::gemm_submit,
      .gemm_execute = entry::gemm_execute,
      .gemm_plan_release = entry::gemm_plan_release,
      .operation_poll = entry::operation_poll,
      .operation_wait = entry::operation_wait,
      .operation_cancel = entry::operation_cancel,
      .operation_get_error = entry::operation_get_error,
      .operation_release = entry::operation_release,
      .reserved = {},
  };
}

const xvram_api_v1 kApiV1 = table_v1(sizeof(xvram_api_v1), XVRAM_ABI_VERSION_1);

const xvram_api_v2 kApiV2 = {
    .v1 = table_v1(sizeof(xvram_api_v2), XVRAM_ABI_VERSION_2),
    .session_create_v2 = entry::session_create_v2,
    .session_get_telemetry_v2 = entry::session_get_telemetry_v2,
    .reserved = {},
};

// This build's extension table (no reference counterpart), reached through
// the one export so the library's symbol set stays the reference's.
const xvram_amd_ext_v1 kExtV1 = {
    .struct_size = sizeof(xvram_amd_ext_v1),
    .ext_version = XVRAM_AMD_EXT_VERSION_2,
    .gemm_plan_create_epilogue = entry::gemm_plan_create_epilogue,
    .device_get_info = entry::device_get_info,
    .sgemm_device = entry::sgemm_device,
    .sgemm_device_no_alloc = entry::sgemm_device_no_alloc,
    .reserved = {},
};

struct TableRef {
  const void* table;
  size_t size;
};

// NULL for a version this library does not serve.
TableRef table_for(uint32_t version) {
  switch (version) {
  case XVRAM_ABI_VERSION_1: return {&kApiV1, sizeof kApiV1};
  case XVRAM_ABI_VERSION_2: return {&kApiV2, sizeof kApiV2};
  case XVRAM_AMD_EXT_ABI_VERSION_1: return {&kExtV1, sizeof kExtV1};
  default: return {nullptr, 0};
  }
}

} // namespace
} // namespace xvram::abi

// The library's one export (reference include/xvram/xvram.h:532-533): an
// unknown version is INCOMPATIBLE_ABI; a known one needs a buffer at least
// as large as its table, else INVALID_ARGUMENT.
extern "C" XVRAM_API xvram_status XVRAM_CALL xvram_get_api(uint32_t requested_abi_version,
                                                           uint32_t caller_api_size, void* out_api) {
  const xvram::abi::TableRef t = xvram::abi::table_for(requested_abi_version);
  if (t.table == nullptr) return XVRAM_STATUS_INCOMPATIBLE_ABI;
  if (out_api == nullptr || caller_api_size < t.size) return XVRAM_STATUS_INVALID_ARGUMENT;
  std::memcpy(out_api, t.table, t.size);
  return XVRAM_STATUS_SUCCESS;
}
