// session.cpp — session worker, operations, allocations and GEMM plans.
#include "session.hpp"

#include <algorithm>

namespace xvram {

// ---- Operation (reference RuntimeOperation, src/sdk/runtime.cpp:146-279) ----

Operation::Operation(uint64_t id, uint64_t units_total, Deadline deadline)
    : deadline_(deadline), id_(id) {
  info_ = XVRAM_OPERATION_INFO_V1_INIT;
  info_.operation_id = id;
  info_.units_total = units_total;
}

Error Operation::poll(xvram_operation_info_v1& out) {
  std::lock_guard<std::mutex> lock(mutex_);
  out = info_;
  return {};
}

Error Operation::wait(uint64_t timeout_ms, xvram_operation_info_v1& out) {
  std::unique_lock<std::mutex> lock(mutex_);
  const auto terminal = [&]() {
    return info_.state == XVRAM_OPERATION_COMPLETED || info_.state == XVRAM_OPERATION_CANCELLED ||
           info_.state == XVRAM_OPERATION_FAILED;
  };
  bool completed = true;
  if (!terminal()) {
    if (timeout_ms == XVRAM_TIMEOUT_INFINITE) {
      done_.wait(lock, terminal);
    } else {
      completed = done_.wait_for(lock, std::chrono::milliseconds(timeout_ms), terminal);
    }
  }
  out = info_;
  return completed ? Error{}
                   : make_error(XVRAM_STATUS_TIMEOUT, "operation", "wait",
                                "operation did not finish before the timeout");
}

Error Operation::cancel() {
  std::lock_guard<std::mutex> lock(mutex_);
  if (info_.state == XVRAM_OPERATION_QUEUED) {
    cancel_requested_ = true;
    return {};
  }
  if (info_.state == XVRAM_OPERATION_RUNNING)
    return make_error(XVRAM_STATUS_BUSY, "operation", "cancel",
                      "a running device operation cannot be cancelled safely");
  return {};
}

Error Operation::error() const {
  std::lock_guard<std::mutex> lock(mutex_);
  return error_;
}

bool Operation::begin() {
  std::lock_guard<std::mutex> lock(mutex_);
  if (cancel_requested_) {
    info_.state = XVRAM_OPERATION_CANCELLED;
    info_.result = XVRAM_STATUS_CANCELLED;
    error_ = make_error(XVRAM_STATUS_CANCELLED, "operation", "cancel", "operation cancelled");
    done_.notify_all();
    return false;
  }
  const auto now = Clock::now();
  if (deadline_.expired(now)) {
    info_.state = XVRAM_OPERATION_FAILED;
    info_.result = XVRAM_STATUS_TIMEOUT;
    error_ = deadline_.timeout_error("operation", "queue_deadline");
    info_.elapsed_ms = std::chrono::duration<double, std::milli>(now - deadline_.submitted()).count();
    done_.notify_all();
    return false;
  }
  info_.state = XVRAM_OPERATION_RUNNING;
  started_ = now;
  return true;
}

Error Operation::deadline_error(const char* stage, const char* operation) const {
  return deadline_.expired() ? deadline_.timeout_error(stage, operation) : Error{};
}

void Operation::finish(const Error& error, const xvram_session_telemetry_v1& before,
                       const xvram_session_telemetry_v1& after) {
  std::lock_guard<std::mutex> lock(mutex_);
  error_ = error;
  info_.result = error.status;
  info_.state = error ? XVRAM_OPERATION_FAILED : XVRAM_OPERATION_COMPLETED;
  if (!error) info_.units_completed = info_.units_total;
  info_.elapsed_ms = std::chrono::duration<double, std::milli>(Clock::now() - started_).count();
  info_.bytes_h2d = after.bytes_h2d - before.bytes_h2d;
  info_.bytes_d2h = after.bytes_d2h - before.bytes_d2h;
  info_.cache_hits = after.cache_hits - before.cache_hits;
  info_.cache_misses = after.cache_misses - before.cache_misses;
  done_.notify_all();
}

void Operation::advance(uint64_t completed) {
  std::lock_guard<std::mutex> lock(mutex_);
  if (info_.state == XVRAM_OPERATION_RUNNING)
    info_.units_completed = std::min(completed, info_.units_total);
}

// ---- Session --------------------------------------------------------------

namespace {

RuntimeConfig runtime_config(const xvram_session_config_v1& c) {
  RuntimeConfig r;
  r.device_ordinal = c.device_ordinal;
  r.chunk_bytes = c.chunk_size_bytes;
  r.cache_target_bytes = c.cache_target_bytes;
  r.device_headroom_bytes = c.device_headroom_bytes;
  r.workspace_reserve_bytes = c.workspace_cap_bytes;
  r.prefetch_distance = c.prefetch_distance;
  r.cache_policy = c.cache_policy;
  r.max_transaction_ms = c.max_transaction_ms == 0 ? 250 : c.max_transaction_ms;
  r.budget_poll_ms = c.budget_poll_ms;
  return r;
}

} // namespace

Session::Session(const xvram_session_config_v1& config)
    : config_(config), runtime_(runtime_config(config)) {
  close_operation_ = std::make_shared<Operation>(0, 1, Deadline{});
  telemetry_ = xvram_session_telemetry_v1{};
  telemetry_.struct_size = sizeof(telemetry_);
}

Session::~Session() { (void)close(XVRAM_TIMEOUT_INFINITE); }

Error Session::start() {
  try {
    worker_ = std::thread([this]() { worker_main(); });
  } catch (...) {
    Error e = exception_error("worker_start");
    std::lock_guard<std::mutex> lock(queue_mutex_);
    setup_error_ = e;
    setup_finished_ = true;
    worker_exited_ = true;
    return e;
  }
  std::unique_lock<std::mutex> lock(queue_mutex_);
  setup_cv_.wait(lock, [&]() { return setup_finished_; });
  return setup_error_;
}

void Session::refresh_telemetry() {
  xvram_session_telemetry_v1 t{};
  runtime_.telemetry(t);
  std::lock_guard<std::mutex> lock(telemetry_mutex_);
  telemetry_ = t;
  logical_bytes_ = runtime_.logical_bytes();
  host_stored_peak_bytes_ = runtime_.host_stored_peak_bytes();
}

// The v2 view (reference sdk/runtime.cpp:572-620) of a session without host
// compression: the host store holds every logical byte raw, and the logical
// and PCIe traffic counters equal the v1 byte counters.
Error Session::telemetry_v2(xvram_session_telemetry_v2& out) const {
  std::lock_guard<std::mutex> lock(telemetry_mutex_);
  out.v1 = telemetry_;
  out.v1.struct_size = sizeof(out.v1);
  out.logical_bytes = logical_bytes_;
  out.host_stored_bytes = logical_bytes_;
  out.host_stored_peak_bytes = host_stored_peak_bytes_;
  out.host_raw_bytes = logical_bytes_;
  out.logical_h2d_bytes = out.pcie_h2d_bytes = telemetry_.bytes_h2d;
  out.logical_d2h_bytes = out.pcie_d2h_bytes = telemetry_.bytes_d2h;
  return {};
}

void Session::worker_main() {
  Error setup;
  try {
    setup = runtime_.setup();
  } catch (...) {
    setup = exception_error("worker_setup");
  }
  {
    std::lock_guard<std::mutex> lock(queue_mutex_);
    setup_error_ = setup;
    chunk_bytes_ = runtime_.frame_bytes();
    setup_finished_ = true;
  }
  refresh_telemetry();
  setup_cv_.notify_all();
  if (setup) {
    (void)runtime_.close();
    std::lock_guard<std::mutex> lock(queue_mutex_);
    worker_exited_ = true;
    exit_cv_.notify_all();
    return;
  }
  for (;;) {
    WorkItem item;
    {
      std::unique_lock<std::mutex> lock(queue_mutex_);
      queue_cv_.wait(lock, [&]() { return stop_worker_ || close_requested_ || !queue_.empty(); });
      if (stop_worker_ && queue_.empty()) break;
      if (!queue_.empty()) {
        item = std::move(queue_.front());
        queue_.pop_front();
      } else {
        item = WorkItem{close_operation_, {}, true};
        close_requested_ = false;
      }
    }
    if (!item.operation->begin()) continue;
    xvram_session_telemetry_v1 before{}, after{};
    runtime_.telemetry(before);
    Error result;
    try {
      result = item.shutdown ? runtime_.close() : item.action(*item.operation);
    } catch (...) {
      result = exception_error("worker_action");
    }
    runtime_.telemetry(after);
    refresh_telemetry();
    item.operation->finish(result, before, after);
    if (item.shutdown) {
      std::lock_guard<std::mutex> lock(queue_mutex_);
      stop_worker_ = true;
    }
  }
  std::lock_guard<std::mutex> lock(queue_mutex_);
  worker_exited_ = true;
  exit_cv_.notify_all();
}

Error Session::enqueue(Action action, uint64_t units, uint64_t deadline_ms,
                       std::shared_ptr<Operation>& out, std::shared_ptr<GemmPlanRecord> gemm) {
  Deadline deadline;
  if (!Deadline::create(deadline_ms, Clock::now(), deadline))
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "deadline", "submit",
                      "deadline_ms cannot be represented by the monotonic clock");
  auto op = std::make_shared<Operation>(next_operation_id_.fetch_add(1), units, deadline);
  {
    std::lock_guard<std::mutex> lock(queue_mutex_);
    if (closing_) return make_error(XVRAM_STATUS_CLOSED, "session", "submit", "session is closing");
    queue_.push_back(WorkItem{op, std::move(action), false, std::move(gemm)});
  }
  queue_cv_.notify_one();
  out = std::move(op);
  return {};
}

Error Session::invoke_sync(std::function<Error()> action, uint64_t timeout_ms) {
  std::shared_ptr<Operation> op;
  if (Error e = enqueue(
          [action = std::move(action)](Operation& o) -> Error {
            if (Error d = o.deadline_error("operation", "pre_launch_deadline")) return d;
            return action();
          },
          1, 0, op))
    return e;
  xvram_operation_info_v1 info{};
  if (Error e = op->wait(timeout_ms, info)) return e;
  return op->error();
}

Error Session::allocate(const xvram_allocation_desc_v1& desc,
                        std::shared_ptr<AllocationRecord>& out) {
  std::shared_ptr<AllocationRecord> created;
  Error e = invoke_sync([&]() -> Error {
    if (desc.alignment_bytes > runtime_.frame_bytes())
      return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "alignment",
                        "allocation alignment exceeds the runtime chunk alignment");
    HostAllocation* host = nullptr;
    if (Error err = runtime_.allocate(desc.size_bytes, desc.alignment_bytes, desc.priority, host))
      return err;
    created = std::make_shared<AllocationRecord>();
    created->owner = weak_from_this();
    created->id = host->id;
    created->bytes = host->bytes;
    created->desc = desc;
    if (created->desc.alignment_bytes == 0) created->desc.alignment_bytes = runtime_.frame_bytes();
    return {};
  });
  if (e) return e;
  out = std::move(created);
  return {};
}

Error Session::write(AllocationRecord& a, uint64_t offset, const void* src, uint64_t bytes) {
  return invoke_sync([&]() { return runtime_.write(a.id, offset, src, bytes); });
}

Error Session::read(AllocationRecord& a, uint64_t offset, void* dst, uint64_t bytes) {
  return invoke_sync([&]() { return runtime_.read(a.id, offset, dst, bytes); });
}

Error Session::release(AllocationRecord& a) {
  return invoke_sync([&]() { return runtime_.release(a.id); });
}

// Plan creation (reference RuntimeSession::create_gemm_plan,
// src/sdk/runtime.cpp:1277-1364): validate on the worker against live
// allocation sizes, then plan panels against the live frame pool.
Error Session::create_gemm_plan(const GemmSpec& spec_in, std::shared_ptr<AllocationRecord> a,
                                std::shared_ptr<AllocationRecord> b,
                                std::shared_ptr<AllocationRecord> c, uint64_t deadline_ms,
                                std::shared_ptr<GemmPlanRecord>& out,
                                std::shared_ptr<AllocationRecord> bias) {
  if (!a || !b || !c || a->released || b->released || c->released ||
      (bias && bias->released))
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "create_plan",
                      "GEMM allocation is invalid or released");
  std::shared_ptr<GemmPlanRecord> record;
  Error e = invoke_sync([&]() -> Error {
    if (a->released || b->released || c->released || (bias && bias->released))
      return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "create_plan",
                        "GEMM allocation was released before planning");
    GemmSpec spec = spec_in;
    spec.a.allocation_id = a->id;
    spec.a.allocation_bytes = a->bytes;
    spec.b.allocation_id = b->id;
    spec.b.allocation_bytes = b->bytes;
    spec.c.allocation_id = c->id;
    spec.c.allocation_bytes = c->bytes;
    spec.epilogue.bias_allocation_id = bias ? bias->id : 0;
    spec.epilogue.bias_allocation_bytes = bias ? bias->bytes : 0;
    char who = 0;
    const ProblemError pe = validate_problem(spec, &who);
    if (pe != ProblemError::none) {
      std::string msg = std::string("invalid_problem: ") + problem_error_name(pe);
      if (who) msg += std::string(" (") + who + ")";
      return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "make_plan", msg);
    }
    if (Error ee = validate_epilogue(spec)) return ee;
    if (spec.a.data_type != XVRAM_DATA_FP32)
      return make_error(XVRAM_STATUS_UNSUPPORTED, "gemm", "make_plan",
                        "only FP32 GEMM is implemented on this device path");
    record = std::make_shared<GemmPlanRecord>();
    record->owner = weak_from_this();
    record->spec = spec;
    record->a = a;
    record->b = b;
    record->c = c;
    record->bias = bias;
    record->deadline_ms = deadline_ms;
    const double cap = static_cast<double>(runtime_.config().max_transaction_ms) *
                       kGuardPlanningFlopsPerMs;
    return make_gemm_plan(spec, runtime_.frame_bytes(), runtime_.frame_capacity(),
                          config_.prefetch_distance, static_cast<uint64_t>(cap), record->plan);
  });
  if (e) return e;
  out = std::move(record);
  return {};
}

Error Session::submit_gemm(const std::shared_ptr<GemmPlanRecord>& plan,
                           std::shared_ptr<Operation>& out) {
  const uint64_t units = plan->plan.launches.size();
  return enqueue(
      [this, plan](Operation& op) -> Error {
        if (Error d = op.deadline_error("gemm", "pre_launch_deadline")) return d;
        if (plan->a->released || plan->b->released || plan->c->released ||
            (plan->bias && plan->bias->released))
          return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "execute",
                            "a GEMM allocation was released");
        GemmHooks hooks;
        hooks.boundary = [&](const char*) -> Error {
          return op.deadline_error("gemm", "tile_deadline");
        };
        hooks.progress = [&](uint64_t done, uint64_t) { op.advance(done); };
        // Operations run one at a time, so the link would idle while this
        // one's last launches and write-backs finish and the next one starts:
        // start the next queued GEMM's first panel fills behind this one's
        // work instead. prefetch_distance = 0 turns this off.
        hooks.tail = [this]() -> Error {
          if (config_.prefetch_distance == 0) return {};
          const std::shared_ptr<GemmPlanRecord> next = next_queued_gemm();
          if (!next) return {};
          return carry_gemm_head(runtime_, next->plan, uint64_t{next->plan.lookahead} + 1);
        };
        return execute_gemm(runtime_, plan->plan, op.id(), hooks);
      },
      units, plan->deadline_ms, out, plan);
}

std::shared_ptr<GemmPlanRecord> Session::next_queued_gemm() const {
  std::shared_ptr<GemmPlanRecord> next;
  {
    std::lock_guard<std::mutex> lock(queue_mutex_);
    if (queue_.empty()) return nullptr;
    next = queue_.front().gemm;
  }
  if (!next || next->a->released || next->b->released || next->c->released ||
      (next->bias && next->bias->released))
    return nullptr;
  return next;
}

namespace {

// src/sdk/runtime.cpp:827-842: a released allocation cannot be named.
Error convert_accesses(const std::vector<Session::Access>& in, std::vector<AccessSpan>& out,
                       const char* operation) {
  out.clear();
  out.reserve(in.size());
  for (const Session::Access& a : in) {
    if (!a.allocation || a.allocation->released)
      return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "transaction", operation,
                        "allocation is released or belongs to another backend");
    out.push_back(AccessSpan{a.allocation->id, a.offset, a.length, a.mode});
  }
  return {};
}

template <size_t N>
std::string bounded_text(const char (&text)[N]) {
  size_t n = 0;
  while (n < N && text[n] != '\0') ++n;
  return std::string(text, n);
}

} // namespace

// src/sdk/runtime.cpp:394-414.
Error Session::submit_prefetch(std::vector<Access> accesses, uint64_t deadline_ms,
                               std::shared_ptr<Operation>& out) {
  std::vector<AccessSpan> spans;
  if (Error e = convert_accesses(accesses, spans, "prefetch")) return e;
  return enqueue(
      [this, spans = std::move(spans), accesses = std::move(accesses)](Operation& op) -> Error {
        if (Error d = op.deadline_error("operation", "pre_launch_deadline")) return d;
        return runtime_.run_prefetch(spans, op.id());
      },
      1, deadline_ms, out);
}

// src/sdk/runtime.cpp:416-499: the callback runs on the worker with the
// working set resident, sees the resolved stable addresses and the compute
// stream, and its failure is reported with the callback's own status and
// error text (native domain CALLBACK).
Error Session::submit_transaction(std::vector<Access> accesses, uint64_t workspace_bytes,
                                  uint64_t deadline_ms, xvram_transaction_callback_v1 callback,
                                  void* user_data, std::shared_ptr<Operation>& out) {
  if (workspace_bytes > config_.workspace_cap_bytes)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "transaction", "workspace",
                      "transaction workspace exceeds the session workspace cap");
  std::vector<AccessSpan> spans;
  if (Error e = convert_accesses(accesses, spans, "transaction")) return e;
  const uint64_t transaction_id = next_transaction_id_.fetch_add(1);
  return enqueue(
      [this, spans = std::move(spans), accesses = std::move(accesses), workspace_bytes, callback,
       user_data, transaction_id](Operation& op) -> Error {
        if (Error d = op.deadline_error("operation", "pre_launch_deadline")) return d;
        TransactionBody body = [&](const std::vector<ResolvedSpan>& ranges, uint64_t ws_address,
                                   uint64_t ws_bytes, Stream stream, bool& skipped) -> Error {
          if (Error d = op.deadline_error("operation", "post_residency_deadline")) {
            skipped = true;
            return d;
          }
          std::vector<xvram_resolved_range_v1> resolved;
          resolved.reserve(ranges.size());
          for (const ResolvedSpan& r : ranges)
            resolved.push_back(xvram_resolved_range_v1{r.span.allocation_id, r.span.offset,
                                                       r.span.length, r.device_address,
                                                       r.span.mode, 0u});
          xvram_transaction_context_v1 context{};
          context.struct_size = sizeof(context);
          context.operation_id = op.id();
          context.transaction_id = transaction_id;
          context.ranges = resolved.data();
          context.range_count = resolved.size();
          context.workspace_device_address = ws_address;
          context.workspace_bytes = ws_bytes;
          context.native_stream = static_cast<uint64_t>(reinterpret_cast<uintptr_t>(stream));
          xvram_error_info_v1 native = XVRAM_ERROR_INFO_V1_INIT;
          const xvram_status status = callback(&context, user_data, &native);
          if (status == XVRAM_STATUS_SUCCESS) return {};
          Error e;
          e.status = status;
          e.native_domain = XVRAM_NATIVE_ERROR_CALLBACK;
          e.native_code = native.native_code;
          e.stage = bounded_text(native.stage);
          e.operation = bounded_text(native.operation);
          e.native_name = bounded_text(native.native_name);
          e.message = bounded_text(native.message);
          if (e.message.empty()) e.message = "transaction callback failed";
          return e;
        };
        return runtime_.run_transaction(spans, workspace_bytes, body, op.id());
      },
      1, deadline_ms, out);
}

Error Session::telemetry(xvram_session_telemetry_v1& out) const {
  std::lock_guard<std::mutex> lock(telemetry_mutex_);
  out = telemetry_;
  return {};
}

Error Session::drain(uint64_t timeout_ms) {
  return invoke_sync([this]() { return runtime_.drain(); }, timeout_ms);
}

bool Session::wait_worker_exit(uint64_t timeout_ms) {
  std::unique_lock<std::mutex> lock(queue_mutex_);
  const auto exited = [this]() { return worker_exited_; };
  if (worker_exited_) return true;
  if (timeout_ms == XVRAM_TIMEOUT_INFINITE) {
    exit_cv_.wait(lock, exited);
    return true;
  }
  return exit_cv_.wait_for(lock, std::chrono::milliseconds(timeout_ms), exited);
}

// Close (reference RuntimeSession::close, src/sdk/runtime.cpp:637-679): queue
// a shutdown after the pending work, wait for it, join the worker.
Error Session::close(uint64_t timeout_ms) {
  const auto started = Clock::now();
  const auto remaining = [&]() -> uint64_t {
    if (timeout_ms == XVRAM_TIMEOUT_INFINITE) return XVRAM_TIMEOUT_INFINITE;
    const auto el = std::chrono::duration_cast<std::chrono::milliseconds>(Clock::now() - started);
    const uint64_t e = el.count() < 0 ? 0 : static_cast<uint64_t>(el.count());
    return e >= timeout_ms ? 0 : timeout_ms - e;
  };
  Error setup;
  bool has_worker;
  {
    std::lock_guard<std::mutex> lock(queue_mutex_);
    has_worker = worker_.joinable();
    if (!closing_) {
      if (!setup_error_) close_requested_ = true;
      closing_ = true;
    }
    setup = setup_error_;
  }
  queue_cv_.notify_all();
  if (!has_worker) return {};
  if (setup) {
    if (!wait_worker_exit(remaining()))
      return make_error(XVRAM_STATUS_TIMEOUT, "session", "close",
                        "session setup cleanup did not finish before the timeout");
  } else {
    xvram_operation_info_v1 info{};
    if (Error e = close_operation_->wait(remaining(), info)) return e;
    if (!wait_worker_exit(remaining()))
      return make_error(XVRAM_STATUS_TIMEOUT, "session", "close",
                        "worker did not retire after cleanup before the timeout");
  }
  bool join = false;
  {
    std::lock_guard<std::mutex> lock(queue_mutex_);
    if (!joined_) {
      joined_ = true;
      join = true;
    }
  }
  if (join && worker_.joinable()) worker_.join();
  return setup ? setup : close_operation_->error();
}

} // namespace xvram
