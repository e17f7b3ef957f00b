// session.cpp — session worker, operations, allocations and GEMM plans.
#include "session.hpp"

#include <algorithm>
#include <cstdlib>

namespace xvram {

// ---- Operation --------------------------------------------------------------

namespace {

// Internal phases of an operation whose terminal record is being written: a
// snapshot taken meanwhile still shows the phase it is leaving.
constexpr uint32_t kLeavingQueued = 0x100;
constexpr uint32_t kLeavingRunning = 0x101;

bool terminal(uint32_t phase) {
  return phase == XVRAM_OPERATION_COMPLETED || phase == XVRAM_OPERATION_FAILED ||
         phase == XVRAM_OPERATION_CANCELLED;
}

uint32_t visible(uint32_t phase) {
  if (phase == kLeavingQueued) return XVRAM_OPERATION_QUEUED;
  if (phase == kLeavingRunning) return XVRAM_OPERATION_RUNNING;
  return phase;
}

double ms_between(Clock::time_point from, Clock::time_point to) {
  return std::chrono::duration<double, std::milli>(to - from).count();
}

} // namespace

Operation::Operation(uint64_t id, uint64_t units_total, Deadline deadline)
    : id_(id), units_total_(units_total), deadline_(deadline),
      settled_(settled_promise_.get_future().share()) {}

xvram_operation_info_v1 Operation::snapshot() const {
  xvram_operation_info_v1 info = XVRAM_OPERATION_INFO_V1_INIT;
  info.operation_id = id_;
  info.units_total = units_total_;
  const uint32_t phase = phase_.load(std::memory_order_acquire);
  info.state = visible(phase);
  info.units_completed = std::min(units_done_.load(std::memory_order_relaxed), units_total_);
  if (terminal(phase)) {
    // A terminal phase is stored only after the record is complete.
    std::lock_guard<std::mutex> lock(record_mutex_);
    info.result = result_;
    info.elapsed_ms = elapsed_ms_;
    info.bytes_h2d = traffic_.bytes_h2d;
    info.bytes_d2h = traffic_.bytes_d2h;
    info.cache_hits = traffic_.cache_hits;
    info.cache_misses = traffic_.cache_misses;
    if (phase == XVRAM_OPERATION_COMPLETED) info.units_completed = units_total_;
  }
  return info;
}

// Callers mostly wait for an operation right after submitting it, and many
// operations (a resident GEMM, a transaction) end within a few milliseconds.
// Watching the phase word for that long sees the end without a blocked
// thread's sleep and wake-up (tens of microseconds per operation on a busy
// host); a longer wait then blocks on the promise.
constexpr auto kWatchBeforeBlocking = std::chrono::milliseconds(2);

bool Operation::ends_within(Clock::duration limit) const {
  const Clock::time_point until = Clock::now() + limit;
  for (unsigned i = 1;; ++i) {
    if (terminal(phase_.load(std::memory_order_acquire))) return true;
    if (i % 64 == 0 && Clock::now() >= until) return false;
    __builtin_ia32_pause();
  }
}

bool Operation::settled_within(uint64_t timeout_ms) const {
  // Waits longer than the clock can express are waits without bound.
  constexpr uint64_t kLongest = uint64_t{1} << 40; // ~35 years
  const bool bounded = timeout_ms != XVRAM_TIMEOUT_INFINITE && timeout_ms < kLongest;
  const auto watch = bounded ? std::min<Clock::duration>(kWatchBeforeBlocking,
                                                         std::chrono::milliseconds(timeout_ms))
                             : Clock::duration(kWatchBeforeBlocking);
  // A terminal phase is stored after the record and before the promise is set.
  if (ends_within(watch)) return true;
  if (!bounded) {
    settled_.wait();
    return true;
  }
  return settled_.wait_for(std::chrono::milliseconds(timeout_ms) - watch) ==
         std::future_status::ready;
}

Error Operation::cancel() {
  uint32_t expected = XVRAM_OPERATION_QUEUED;
  if (phase_.compare_exchange_strong(expected, kLeavingQueued, std::memory_order_acq_rel)) {
    publish(XVRAM_OPERATION_CANCELLED,
            make_error(XVRAM_STATUS_CANCELLED, "operation", "cancel",
                       "cancelled before the worker started it"),
            0.0, {});
    return {};
  }
  if (visible(expected) == XVRAM_OPERATION_RUNNING)
    return make_error(XVRAM_STATUS_BUSY, "operation", "cancel",
                      "the operation has device work in flight; wait for it instead");
  return {}; // already terminal: nothing to cancel
}

Error Operation::failure() const {
  if (!terminal(phase_.load(std::memory_order_acquire))) return {};
  std::lock_guard<std::mutex> lock(record_mutex_);
  return error_;
}

bool Operation::cancelled() const {
  return phase_.load(std::memory_order_acquire) == XVRAM_OPERATION_CANCELLED;
}

bool Operation::claim() {
  const Clock::time_point now = Clock::now();
  uint32_t expected = XVRAM_OPERATION_QUEUED;
  if (deadline_.passed(now)) {
    if (!phase_.compare_exchange_strong(expected, kLeavingQueued, std::memory_order_acq_rel))
      return false; // cancelled meanwhile
    publish(XVRAM_OPERATION_FAILED, deadline_.missed("operation", "queue_deadline"),
            ms_between(deadline_.submitted(), now), {});
    return false;
  }
  started_ = now;
  return phase_.compare_exchange_strong(expected, XVRAM_OPERATION_RUNNING,
                                        std::memory_order_acq_rel);
}

Error Operation::deadline_check(const char* stage, const char* where) const {
  return deadline_.passed() ? deadline_.missed(stage, where) : Error{};
}

void Operation::progress(uint64_t units_done) {
  units_done_.store(std::min(units_done, units_total_), std::memory_order_relaxed);
}

void Operation::settle(const Error& result, const OperationTraffic& traffic) {
  const xvram_operation_state end = result ? XVRAM_OPERATION_FAILED : XVRAM_OPERATION_COMPLETED;
  phase_.store(kLeavingRunning, std::memory_order_relaxed);
  publish(end, result, ms_between(started_, Clock::now()), traffic);
}

void Operation::publish(xvram_operation_state end, const Error& result, double elapsed_ms,
                        const OperationTraffic& traffic) {
  {
    std::lock_guard<std::mutex> lock(record_mutex_);
    result_ = result.status;
    error_ = result;
    elapsed_ms_ = elapsed_ms;
    traffic_ = traffic;
  }
  phase_.store(end, std::memory_order_release);
  settled_promise_.set_value();
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
  // The session config has no stall deadline field (the reference's SDK
  // uses its runtime default, 5 s); XVRAM_STALL_TIMEOUT_MS overrides it for
  // the whole process.
  if (const char* text = std::getenv("XVRAM_STALL_TIMEOUT_MS"); text != nullptr && *text) {
    char* end = nullptr;
    const unsigned long long ms = std::strtoull(text, &end, 10);
    if (end != text && *end == '\0' && ms > 0) r.stall_timeout_ms = ms;
  }
  return r;
}

} // namespace

Session::Session(const xvram_session_config_v1& config)
    : config_(config), runtime_(runtime_config(config)),
      exited_(exit_promise_.get_future().share()),
      shutdown_(std::make_shared<Operation>(0, 1, Deadline{})) {
  telemetry_.struct_size = sizeof(telemetry_);
}

Session::~Session() {
  try {
    (void)close(XVRAM_TIMEOUT_INFINITE);
  } catch (...) {
    // A destructor cannot report; the runtime's own destructor still frees.
  }
}

Error Session::start() {
  std::future<Error> setup = setup_promise_.get_future();
  try {
    thread_ = std::thread(&Session::worker, this);
    worker_started_ = true;
  } catch (...) {
    Error e = exception_error("worker_start");
    std::lock_guard<std::mutex> lock(jobs_mutex_);
    setup_failed_ = true;
    setup_error_ = e;
    exit_promise_.set_value();
    return e;
  }
  Error e = setup.get();
  if (e) {
    std::lock_guard<std::mutex> lock(jobs_mutex_);
    setup_failed_ = true;
    setup_error_ = e;
  }
  return e;
}

void Session::publish_telemetry() {
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

// The worker: set the runtime up (on this thread, which keeps the device
// current from here on), report the outcome to start(), then run jobs in
// submission order until the shutdown job, which close() queues last.
void Session::worker() {
  Error setup;
  try {
    setup = runtime_.setup();
  } catch (...) {
    setup = exception_error("worker_setup");
  }
  chunk_bytes_ = runtime_.frame_bytes();
  publish_telemetry();
  setup_promise_.set_value(setup);
  if (setup) {
    (void)runtime_.close();
    exit_promise_.set_value();
    return;
  }
  uint64_t taken = 0;
  for (bool running = true; running;) {
    Job job;
    await_job(taken);
    {
      std::lock_guard<std::mutex> lock(jobs_mutex_);
      job = std::move(jobs_.front());
      jobs_.pop_front();
    }
    ++taken;
    running = !job.shutdown;
    execute(job);
  }
  exit_promise_.set_value();
}

// A caller that waited for one operation usually submits the next within
// microseconds: the worker watches the queue counter for a short while before
// it sleeps, so such a job starts without a wake-up.
void Session::await_job(uint64_t taken) {
  constexpr auto kWatch = std::chrono::microseconds(500);
  const Clock::time_point until = Clock::now() + kWatch;
  for (unsigned i = 1; jobs_pushed_.load(std::memory_order_acquire) == taken; ++i) {
    if (i % 64 == 0 && Clock::now() >= until) {
      std::unique_lock<std::mutex> lock(jobs_mutex_);
      jobs_ready_.wait(lock, [this]() { return !jobs_.empty(); });
      return;
    }
    __builtin_ia32_pause();
  }
}

void Session::execute(Job& job) {
  if (!job.operation->claim()) return;
  xvram_session_telemetry_v1 before{}, after{};
  runtime_.telemetry(before);
  Error result;
  try {
    result = job.shutdown ? runtime_.close() : job.body(*job.operation);
  } catch (...) {
    result = exception_error(job.shutdown ? "session_shutdown" : "worker_job");
  }
  runtime_.telemetry(after);
  publish_telemetry();
  job.operation->settle(result, OperationTraffic{after.bytes_h2d - before.bytes_h2d,
                                                 after.bytes_d2h - before.bytes_d2h,
                                                 after.cache_hits - before.cache_hits,
                                                 after.cache_misses - before.cache_misses});
}

Error Session::enqueue(std::function<Error(Operation&)> body, uint64_t units, uint64_t deadline_ms,
                       std::shared_ptr<Operation>& out, std::shared_ptr<GemmPlanRecord> gemm) {
  const std::optional<Deadline> deadline = Deadline::after(deadline_ms, Clock::now());
  if (!deadline) return check_deadline_ms(deadline_ms, "submit");
  auto op = std::make_shared<Operation>(operation_ids_.fetch_add(1), units, *deadline);
  {
    std::lock_guard<std::mutex> lock(jobs_mutex_);
    if (sealed_ || setup_failed_)
      return make_error(XVRAM_STATUS_CLOSED, "session", "submit",
                        "the session is closed or closing; nothing more can be queued");
    jobs_.push_back(Job{op, std::move(body), std::move(gemm), false});
    jobs_pushed_.fetch_add(1, std::memory_order_release);
  }
  jobs_ready_.notify_one();
  out = std::move(op);
  return {};
}

Error Session::run_on_worker(std::function<Error()> body, uint64_t timeout_ms) {
  std::shared_ptr<Operation> op;
  Error e = enqueue(
      [body = std::move(body)](Operation& o) -> Error {
        if (Error d = o.deadline_check("operation", "pre_launch_deadline")) return d;
        return body();
      },
      1, 0, op);
  if (e) return e;
  if (!op->settled_within(timeout_ms))
    return make_error(XVRAM_STATUS_TIMEOUT, "operation", "wait",
                      "the session worker did not finish the call within the timeout");
  return op->failure();
}

Error Session::allocate(const xvram_allocation_desc_v1& desc,
                        std::shared_ptr<AllocationRecord>& out) {
  std::shared_ptr<AllocationRecord> created;
  Error e = run_on_worker([&]() -> Error {
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
  return run_on_worker([&]() { return runtime_.write(a.id, offset, src, bytes); });
}

Error Session::read(AllocationRecord& a, uint64_t offset, void* dst, uint64_t bytes) {
  return run_on_worker([&]() { return runtime_.read(a.id, offset, dst, bytes); });
}

Error Session::release(AllocationRecord& a) {
  return run_on_worker([&]() { return runtime_.release(a.id); });
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
  Error e = run_on_worker([&]() -> Error {
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

// A GEMM operation counts its progress in tiles of the plan's geometry (C
// tiles x K panels, gemm_plan_info_v1.tile_count), as the reference's does
// (src/sdk/runtime.cpp:1227): units_completed reaches tile_count on success
// however many K panels each launch covers.
Error Session::submit_gemm(const std::shared_ptr<GemmPlanRecord>& plan,
                           std::shared_ptr<Operation>& out) {
  return enqueue(
      [this, plan](Operation& op) -> Error {
        if (Error d = op.deadline_check("gemm", "pre_launch_deadline")) return d;
        if (!plan->operands_live())
          return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "execute",
                            "an operand allocation of the plan was released");
        GemmHooks hooks;
        hooks.boundary = [&](const char*) -> Error {
          return op.deadline_check("gemm", "tile_deadline");
        };
        hooks.progress = [&](uint64_t tiles_done, uint64_t) { op.progress(tiles_done); };
        // Operations run one at a time, so the link would idle while this
        // one's last launches and write-backs finish and the next one starts:
        // start the next queued GEMM's first panel fills behind this one's
        // work instead. prefetch_distance = 0 turns this off.
        hooks.tail = [this]() -> Error {
          if (config_.prefetch_distance == 0) return {};
          const std::shared_ptr<GemmPlanRecord> next = gemm_queued_next();
          if (!next) return {};
          return carry_gemm_head(runtime_, next->plan, uint64_t{next->plan.lookahead} + 1);
        };
        return execute_gemm(runtime_, plan->plan, op.id(), hooks);
      },
      plan->tile_count(), plan->deadline_ms, out, plan);
}

std::shared_ptr<GemmPlanRecord> Session::gemm_queued_next() const {
  std::shared_ptr<GemmPlanRecord> next;
  {
    std::lock_guard<std::mutex> lock(jobs_mutex_);
    if (jobs_.empty()) return nullptr;
    next = jobs_.front().gemm;
  }
  return next && next->operands_live() ? next : nullptr;
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
        if (Error d = op.deadline_check("operation", "pre_launch_deadline")) return d;
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
  const uint64_t transaction_id = transaction_ids_.fetch_add(1);
  return enqueue(
      [this, spans = std::move(spans), accesses = std::move(accesses), workspace_bytes, callback,
       user_data, transaction_id](Operation& op) -> Error {
        if (Error d = op.deadline_check("operation", "pre_launch_deadline")) return d;
        TransactionBody body = [&](const std::vector<ResolvedSpan>& ranges, uint64_t ws_address,
                                   uint64_t ws_bytes, Stream stream, bool& skipped) -> Error {
          if (Error d = op.deadline_check("operation", "post_residency_deadline")) {
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
          if (e.message.empty()) e.message = "the transaction callback returned a failure status";
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
  return run_on_worker([this]() { return runtime_.drain(); }, timeout_ms);
}

bool Session::join_worker(uint64_t timeout_ms) {
  if (!worker_started_) return true;
  if (timeout_ms != XVRAM_TIMEOUT_INFINITE &&
      exited_.wait_for(std::chrono::milliseconds(timeout_ms)) != std::future_status::ready)
    return false;
  std::call_once(join_once_, [this]() {
    if (thread_.joinable()) thread_.join();
  });
  return true;
}

// Close (reference RuntimeSession::close, src/sdk/runtime.cpp:637-679): the
// shutdown job is queued once, behind everything already submitted; its
// operation's result is the close result. A session whose set-up failed has
// no runtime to close: its worker has already ended.
Error Session::close(uint64_t timeout_ms) {
  if (closed()) return {};
  const Clock::time_point begun = Clock::now();
  const auto left = [&]() -> uint64_t {
    if (timeout_ms == XVRAM_TIMEOUT_INFINITE) return XVRAM_TIMEOUT_INFINITE;
    const auto spent = std::chrono::duration_cast<std::chrono::milliseconds>(Clock::now() - begun);
    const uint64_t used = spent.count() > 0 ? static_cast<uint64_t>(spent.count()) : 0;
    return used >= timeout_ms ? 0 : timeout_ms - used;
  };
  bool setup_failed = false;
  Error setup_error;
  {
    std::lock_guard<std::mutex> lock(jobs_mutex_);
    setup_failed = setup_failed_;
    setup_error = setup_error_;
    if (!setup_failed && !sealed_ && worker_started_) {
      jobs_.push_back(Job{shutdown_, {}, nullptr, true});
      jobs_pushed_.fetch_add(1, std::memory_order_release);
      jobs_ready_.notify_one();
    }
    sealed_ = true;
  }
  if (!worker_started_) return setup_error;
  if (setup_failed) {
    if (!join_worker(left()))
      return make_error(XVRAM_STATUS_TIMEOUT, "session", "close",
                        "the worker did not finish its failed set-up within the timeout");
    return setup_error;
  }
  if (!shutdown_->settled_within(left()))
    return make_error(XVRAM_STATUS_TIMEOUT, "session", "close",
                      "queued work and the runtime teardown did not finish within the timeout");
  if (!join_worker(left()))
    return make_error(XVRAM_STATUS_TIMEOUT, "session", "close",
                      "the worker did not exit within the timeout after the teardown");
  Error result = shutdown_->failure();
  if (!result) closed_.store(true, std::memory_order_release);
  return result;
}

void Session::note_failure(const Error& error) noexcept {
  if (!error) return;
  try {
    std::lock_guard<std::mutex> lock(failure_mutex_);
    last_failure_ = error;
  } catch (...) {
    // Keeping the previous record is the only option when copying fails.
  }
}

Error Session::last_failure() const {
  std::lock_guard<std::mutex> lock(failure_mutex_);
  return last_failure_;
}

} // namespace xvram
