// session.hpp — the session backend behind the C ABI: one worker thread per
// session owns the device and executes queued operations in order.
//
// Reference counterpart: src/sdk/runtime.cpp (RuntimeOperation :146-279,
// RuntimeSession :319-1116, RuntimeGemmPlan :1175-1364). Semantics kept: any
// thread may call; every call that touches the device runs on the worker;
// submissions return operations with poll/wait/cancel (cancel succeeds only
// while queued, BUSY while running); deadlines are submission-relative and
// are sampled at safe boundaries; close drains the queue and tears down.
#pragma once

#include <atomic>
#include <condition_variable>
#include <deque>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>

#include "common.hpp"
#include "gemm.hpp"
#include "runtime.hpp"

namespace xvram {

class Session;

class Operation {
public:
  Operation(uint64_t id, uint64_t units_total, Deadline deadline);

  Error poll(xvram_operation_info_v1& out);
  Error wait(uint64_t timeout_ms, xvram_operation_info_v1& out);
  Error cancel();
  Error error() const;

  bool begin();
  Error deadline_error(const char* stage, const char* operation) const;
  void finish(const Error& error, const xvram_session_telemetry_v1& before,
              const xvram_session_telemetry_v1& after);
  void advance(uint64_t completed);
  uint64_t id() const { return id_; }

private:
  mutable std::mutex mutex_;
  std::condition_variable done_;
  xvram_operation_info_v1 info_{};
  Error error_;
  Deadline deadline_;
  Clock::time_point started_{};
  bool cancel_requested_ = false;
  uint64_t id_ = 0;
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
};

class Session : public std::enable_shared_from_this<Session> {
public:
  explicit Session(const xvram_session_config_v1& config);
  ~Session();

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
  Error close(uint64_t timeout_ms);

private:
  using Action = std::function<Error(Operation&)>;
  struct WorkItem {
    std::shared_ptr<Operation> operation;
    Action action;
    bool shutdown = false;
    std::shared_ptr<GemmPlanRecord> gemm; // set for a GEMM execution
  };

  Error enqueue(Action action, uint64_t units, uint64_t deadline_ms,
                std::shared_ptr<Operation>& out,
                std::shared_ptr<GemmPlanRecord> gemm = nullptr);
  // The plan of the GEMM queued next, if the next queued item is one whose
  // allocations are all live.
  std::shared_ptr<GemmPlanRecord> next_queued_gemm() const;
  Error invoke_sync(std::function<Error()> action, uint64_t timeout_ms = XVRAM_TIMEOUT_INFINITE);
  void worker_main();
  void refresh_telemetry();
  bool wait_worker_exit(uint64_t timeout_ms);

  xvram_session_config_v1 config_{};
  Runtime runtime_;
  uint64_t chunk_bytes_ = 0;

  std::thread worker_;
  mutable std::mutex queue_mutex_;
  std::condition_variable queue_cv_;
  std::condition_variable setup_cv_;
  std::condition_variable exit_cv_;
  std::deque<WorkItem> queue_;
  bool setup_finished_ = false;
  bool stop_worker_ = false;
  bool worker_exited_ = false;
  bool closing_ = false;
  bool close_requested_ = false;
  bool joined_ = false;
  Error setup_error_;
  std::shared_ptr<Operation> close_operation_;
  std::atomic<uint64_t> next_operation_id_{1};
  std::atomic<uint64_t> next_transaction_id_{1};

  mutable std::mutex telemetry_mutex_;
  xvram_session_telemetry_v1 telemetry_{};
  uint64_t logical_bytes_ = 0;
  uint64_t host_stored_peak_bytes_ = 0;
};

} // namespace xvram
