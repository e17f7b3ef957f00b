// session.hpp — the session backend behind the C ABI: one worker thread per
// session owns the device and executes queued operations in order.
//
// Reference counterpart: src/sdk/runtime.cpp (RuntimeOperation :146-279,
// RuntimeSession :319-1116, RuntimeGemmPlan :1175-1364). What callers observe
// is kept: any thread may call; every call that touches the device runs on the
// worker; submissions return operations with poll/wait/cancel (a cancel is
// accepted only before the operation starts, BUSY while it runs); deadlines are
// submission-relative and are checked when the operation is taken off the
// queue and at safe launch boundaries; close runs after the queued work and
// tears the runtime down.
#pragma once

#include <atomic>
#include <condition_variable>
#include <deque>
#include <functional>
#include <future>
#include <memory>
#include <mutex>
#include <thread>

#include "common.hpp"
#include "gemm.hpp"
#include "runtime.hpp"

namespace xvram {

class Session;

// Traffic an operation caused, from the runtime counters around its run.
struct OperationTraffic {
  uint64_t bytes_h2d = 0, bytes_d2h = 0, cache_hits = 0, cache_misses = 0;
};

// One submitted unit of work. Its phase is one atomic word that the caller
// side (snapshot, settled_within, cancel) and the worker side (claim,
// progress, settle) move with compare-and-swap:
//
//   queued --claim--> running --settle--> completed | failed
//   queued --cancel--> cancelled          (at once: waiters return immediately)
//   queued --claim, deadline passed--> failed (TIMEOUT)
//
// Exactly one of cancel/claim wins a queued operation. The terminal record
// (result, error, elapsed time, traffic) is written once, by the winner, and
// then published through a promise; every waiter holds its shared future.
class Operation {
public:
  Operation(uint64_t id, uint64_t units_total, Deadline deadline);

  // ---- caller side ----
  xvram_operation_info_v1 snapshot() const;
  // True once the operation is terminal; waits at most timeout_ms
  // (XVRAM_TIMEOUT_INFINITE: without bound).
  bool settled_within(uint64_t timeout_ms) const;
  Error cancel();
  Error failure() const;

  // ---- worker side ----
  // Moves a queued operation to running. False when it was cancelled or its
  // deadline had already passed (then it is settled as FAILED/TIMEOUT here).
  bool claim();
  // TIMEOUT error naming `stage`/`where` once the deadline has passed.
  Error deadline_check(const char* stage, const char* where) const;
  void progress(uint64_t units_done);
  void settle(const Error& result, const OperationTraffic& traffic);
  bool cancelled() const;
  uint64_t id() const { return id_; }

private:
  void publish(xvram_operation_state terminal, const Error& result, double elapsed_ms,
               const OperationTraffic& traffic);
  // True if the phase turns terminal within `limit` of watching it.
  bool ends_within(Clock::duration limit) const;

  const uint64_t id_;
  const uint64_t units_total_;
  const Deadline deadline_;
  std::atomic<uint32_t> phase_{XVRAM_OPERATION_QUEUED};
  std::atomic<uint64_t> units_done_{0};
  Clock::time_point started_{};

  mutable std::mutex record_mutex_; // guards the terminal record below
  xvram_status result_ = XVRAM_STATUS_SUCCESS;
  Error error_;
  double elapsed_ms_ = 0.0;
  OperationTraffic traffic_;

  std::promise<void> settled_promise_;
  std::shared_future<void> settled_;
};

struct AllocationRecord {
  std::weak_ptr<Session> owner;
  uint64_t id = 0;
  uint64_t bytes = 0;
  xvram_allocation_desc_v1 desc{};
  std::atomic<bool> released{false};
};

struct GemmPlanRecord {
  std::weak_ptr<Session> owner;
  GemmSpec spec;
  GemmPlanData plan;
  std::shared_ptr<AllocationRecord> a, b, c;
  std::shared_ptr<AllocationRecord> bias; // fused-epilogue bias vector, if any
  uint64_t deadline_ms = 0;
  // Tiles of the plan's geometry: C tiles x K panels (progress units).
  uint64_t tile_count() const { return plan.tiles_m * plan.tiles_n * plan.panels_k; }
  bool operands_live() const {
    return !a->released && !b->released && !c->released && !(bias && bias->released);
  }
};

class Session : public std::enable_shared_from_this<Session> {
public:
  explicit Session(const xvram_session_config_v1& config);
  ~Session();

  // Starts the worker and waits for the runtime set-up it runs.
  Error start();
  uint64_t chunk_size_bytes() const { return chunk_bytes_; }
  const xvram_session_config_v1& config() const { return config_; }

  Error allocate(const xvram_allocation_desc_v1& desc, std::shared_ptr<AllocationRecord>& out);
  Error write(AllocationRecord& a, uint64_t offset, const void* src, uint64_t bytes);
  Error read(AllocationRecord& a, uint64_t offset, void* dst, uint64_t bytes);
  Error release(AllocationRecord& a);

  Error create_gemm_plan(const GemmSpec& spec, std::shared_ptr<AllocationRecord> a,
                         std::shared_ptr<AllocationRecord> b, std::shared_ptr<AllocationRecord> c,
                         uint64_t deadline_ms, std::shared_ptr<GemmPlanRecord>& out,
                         std::shared_ptr<AllocationRecord> bias = nullptr);
  Error submit_gemm(const std::shared_ptr<GemmPlanRecord>& plan, std::shared_ptr<Operation>& out);

  // One access of a transaction or prefetch, with the record kept alive until
  // the operation has run.
  struct Access {
    std::shared_ptr<AllocationRecord> allocation;
    uint64_t offset = 0;
    uint64_t length = 0;
    uint32_t mode = XVRAM_ACCESS_READ;
  };
  Error submit_prefetch(std::vector<Access> accesses, uint64_t deadline_ms,
                        std::shared_ptr<Operation>& out);
  Error submit_transaction(std::vector<Access> accesses, uint64_t workspace_bytes,
                           uint64_t deadline_ms, xvram_transaction_callback_v1 callback,
                           void* user_data, std::shared_ptr<Operation>& out);

  Error telemetry(xvram_session_telemetry_v1& out) const;
  Error telemetry_v2(xvram_session_telemetry_v2& out) const;
  Error drain(uint64_t timeout_ms);
  // Runs after the work already queued; a second call after a successful
  // close returns success at once.
  Error close(uint64_t timeout_ms);
  bool closed() const { return closed_.load(std::memory_order_acquire); }

  // The last failure any ABI call on this session reported (session_get_error).
  void note_failure(const Error& error) noexcept;
  Error last_failure() const;

private:
  // A queued unit of work. `gemm` names the plan of a GEMM execution, so the
  // operation running ahead of it can start its first fills (carry).
  struct Job {
    std::shared_ptr<Operation> operation;
    std::function<Error(Operation&)> body;
    std::shared_ptr<GemmPlanRecord> gemm;
    bool shutdown = false;
  };

  Error enqueue(std::function<Error(Operation&)> body, uint64_t units, uint64_t deadline_ms,
                std::shared_ptr<Operation>& out, std::shared_ptr<GemmPlanRecord> gemm = nullptr);
  // Runs `body` on the worker as an operation of one unit and waits for it.
  Error run_on_worker(std::function<Error()> body, uint64_t timeout_ms = XVRAM_TIMEOUT_INFINITE);
  // The plan of the job queued first, if it is a GEMM whose operands are live.
  std::shared_ptr<GemmPlanRecord> gemm_queued_next() const;
  void worker();
  // Returns once a job is queued: watches jobs_pushed_ for a short while after
  // the last job, then sleeps on jobs_ready_.
  void await_job(uint64_t taken);
  void execute(Job& job);
  void publish_telemetry();
  bool join_worker(uint64_t timeout_ms);

  xvram_session_config_v1 config_{};
  Runtime runtime_;
  uint64_t chunk_bytes_ = 0;

  std::thread thread_;
  std::promise<Error> setup_promise_;
  std::promise<void> exit_promise_;
  std::shared_future<void> exited_;
  std::once_flag join_once_;
  bool worker_started_ = false; // written by start(), before the session is shared

  mutable std::mutex jobs_mutex_;
  std::condition_variable jobs_ready_;
  std::deque<Job> jobs_;
  std::atomic<uint64_t> jobs_pushed_{0}; // jobs ever queued (the idle worker watches it)
  bool sealed_ = false;          // no more jobs; the shutdown job is queued
  bool setup_failed_ = false;
  Error setup_error_;
  std::shared_ptr<Operation> shutdown_;
  std::atomic<bool> closed_{false};
  std::atomic<uint64_t> operation_ids_{1};
  std::atomic<uint64_t> transaction_ids_{1};

  mutable std::mutex failure_mutex_;
  Error last_failure_;

  mutable std::mutex telemetry_mutex_;
  xvram_session_telemetry_v1 telemetry_{};
  uint64_t logical_bytes_ = 0;
  uint64_t host_stored_peak_bytes_ = 0;
};

} // namespace xvram
