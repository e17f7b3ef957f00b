// stress.cpp — several caller threads on one session through the C ABI, built
// together with the host runtime and the host-memory device simulation under
// ThreadSanitizer, and under AddressSanitizer + UndefinedBehaviorSanitizer
// (tests/sanitize/Makefile; run by tests/test_sanitizers.py). CPU only.
//
// Four threads submit, poll, cancel and wait on GEMMs of their own (checked
// against an FP64 loop under |C - C_ref| <= 4*K*2^-24*(|A||B|)_ij + |beta*C0|
// terms), one runs transactions and prefetches on another allocation, one reads
// telemetry and the last error in a loop. Returns 0 when every check held.
#include <xvram/xvram.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <random>
#include <thread>
#include <vector>

namespace {

xvram_api_v1 api;
std::atomic<int> failures{0};

#define CHECK(cond, ...)                                                                  \
  do {                                                                                    \
    if (!(cond)) {                                                                        \
      std::fprintf(stderr, "check failed (%s:%d): ", __FILE__, __LINE__);                 \
      std::fprintf(stderr, __VA_ARGS__);                                                  \
      std::fprintf(stderr, "\n");                                                         \
      ++failures;                                                                         \
      return;                                                                             \
    }                                                                                     \
  } while (0)

constexpr uint64_t kFrame = 16 * 1024;

float uniform(std::mt19937_64& rng) {
  return static_cast<float>(2.0 * static_cast<double>(rng() >> 40) * 0x1p-24 - 1.0);
}

xvram_allocation allocate(xvram_session s, uint64_t bytes) {
  xvram_allocation_desc_v1 d = XVRAM_ALLOCATION_DESC_V1_INIT;
  d.size_bytes = bytes;
  xvram_allocation a = nullptr;
  if (api.allocation_create(s, &d, &a) != XVRAM_STATUS_SUCCESS) return nullptr;
  return a;
}

xvram_matrix_v1 matrix(xvram_allocation a, uint64_t rows, uint64_t cols) {
  xvram_matrix_v1 m = XVRAM_MATRIX_V1_INIT;
  m.allocation = a;
  m.rows = rows;
  m.columns = cols;
  m.leading_dimension = rows;
  m.layout = XVRAM_MATRIX_COLUMN_MAJOR;
  return m;
}

void gemm_thread(xvram_session s, int tid, std::atomic<int>* done, std::atomic<int>* cancelled) {
  std::mt19937_64 rng(100 + tid);
  for (int it = 0; it < 10; ++it) {
    const uint64_t m = 8 + rng() % 90, n = 8 + rng() % 90, k = 8 + rng() % 120;
    const bool ta = rng() & 1, tb = rng() & 1;
    const double beta = (rng() & 1) ? 0.5 : 0.0;
    std::vector<float> a(m * k), b(k * n), c0(m * n);
    for (float& v : a) v = uniform(rng);
    for (float& v : b) v = uniform(rng);
    for (float& v : c0) v = uniform(rng);
    // Logical A(i,p) = a[i + p*m], B(p,j) = b[p + j*k]; stored as op(.) asks.
    std::vector<float> as(m * k), bs(k * n);
    for (uint64_t i = 0; i < m; ++i)
      for (uint64_t p = 0; p < k; ++p) as[ta ? p + i * k : i + p * m] = a[i + p * m];
    for (uint64_t p = 0; p < k; ++p)
      for (uint64_t j = 0; j < n; ++j) bs[tb ? j + p * n : p + j * k] = b[p + j * k];
    xvram_allocation A = allocate(s, m * k * 4), B = allocate(s, k * n * 4), C = allocate(s, m * n * 4);
    CHECK(A && B && C, "allocation_create failed");
    CHECK(api.allocation_write(A, 0, as.data(), m * k * 4) == XVRAM_STATUS_SUCCESS, "write A");
    CHECK(api.allocation_write(B, 0, bs.data(), k * n * 4) == XVRAM_STATUS_SUCCESS, "write B");
    CHECK(api.allocation_write(C, 0, c0.data(), m * n * 4) == XVRAM_STATUS_SUCCESS, "write C");
    xvram_gemm_desc_v1 d = XVRAM_GEMM_DESC_V1_INIT;
    d.a = ta ? matrix(A, k, m) : matrix(A, m, k);
    d.b = tb ? matrix(B, n, k) : matrix(B, k, n);
    d.c = matrix(C, m, n);
    d.operation_a = ta ? XVRAM_MATRIX_OP_T : XVRAM_MATRIX_OP_N;
    d.operation_b = tb ? XVRAM_MATRIX_OP_T : XVRAM_MATRIX_OP_N;
    d.beta = beta;
    xvram_gemm_plan plan = nullptr;
    CHECK(api.gemm_plan_create(s, &d, &plan) == XVRAM_STATUS_SUCCESS, "gemm_plan_create");
    xvram_operation op = nullptr;
    CHECK(api.gemm_submit(plan, &op) == XVRAM_STATUS_SUCCESS, "gemm_submit");
    if (rng() % 4 == 0) {
      const xvram_status st = api.operation_cancel(op);
      CHECK(st == XVRAM_STATUS_SUCCESS || st == XVRAM_STATUS_BUSY, "cancel returned %u", st);
    }
    xvram_operation_info_v1 info = XVRAM_OPERATION_INFO_V1_INIT;
    CHECK(api.operation_poll(op, &info) == XVRAM_STATUS_SUCCESS, "poll");
    CHECK(api.operation_wait(op, XVRAM_TIMEOUT_INFINITE, &info) == XVRAM_STATUS_SUCCESS, "wait");
    const bool was_cancelled = info.result == XVRAM_STATUS_CANCELLED;
    CHECK(was_cancelled || info.result == XVRAM_STATUS_SUCCESS, "gemm result %u", info.result);
    xvram_error_info_v1 err = XVRAM_ERROR_INFO_V1_INIT;
    CHECK(api.operation_get_error(op, &err) == XVRAM_STATUS_SUCCESS, "operation_get_error");
    api.operation_release(op);
    std::vector<float> c(m * n);
    CHECK(api.allocation_read(C, 0, c.data(), m * n * 4) == XVRAM_STATUS_SUCCESS, "read C");
    for (uint64_t j = 0; j < n; ++j) {
      for (uint64_t i = 0; i < m; ++i) {
        const float got = c[i + j * m];
        if (was_cancelled) {
          CHECK(got == c0[i + j * m], "cancelled GEMM changed C");
          continue;
        }
        double ref = 0.0, mag = 0.0;
        for (uint64_t p = 0; p < k; ++p) {
          ref += static_cast<double>(a[i + p * m]) * b[p + j * k];
          mag += std::fabs(static_cast<double>(a[i + p * m]) * b[p + j * k]);
        }
        const double bc = static_cast<float>(beta) * static_cast<double>(c0[i + j * m]);
        ref += bc;
        const double bound = 4.0 * static_cast<double>(k) * 0x1p-24 * (mag + std::fabs(bc));
        CHECK(std::fabs(got - ref) <= bound, "thread %d GEMM %d: C(%llu,%llu) = %g, want %g", tid,
              it, (unsigned long long)i, (unsigned long long)j, got, ref);
      }
    }
    api.gemm_plan_release(plan);
    for (xvram_allocation h : {A, B, C})
      CHECK(api.allocation_release(h) == XVRAM_STATUS_SUCCESS, "allocation_release");
    (was_cancelled ? *cancelled : *done) += 1;
  }
}

xvram_status XVRAM_CALL count_ranges(const xvram_transaction_context_v1* ctx, void* user,
                                     xvram_error_info_v1*) {
  static_cast<std::atomic<uint64_t>*>(user)->fetch_add(ctx->range_count);
  return XVRAM_STATUS_SUCCESS;
}

void transaction_thread(xvram_session s, std::atomic<int>* done) {
  const uint64_t bytes = 6 * kFrame;
  xvram_allocation big = allocate(s, bytes);
  CHECK(big, "allocation_create failed");
  std::vector<uint32_t> data(bytes / 4);
  for (uint64_t i = 0; i < data.size(); ++i) data[i] = static_cast<uint32_t>(i * 2654435761u);
  CHECK(api.allocation_write(big, 0, data.data(), bytes) == XVRAM_STATUS_SUCCESS, "write");
  std::atomic<uint64_t> ranges{0};
  for (int it = 0; it < 16; ++it) {
    xvram_access_range_v1 r{big, (it % 4) * kFrame, 2 * kFrame, XVRAM_ACCESS_READ, 0};
    xvram_operation op = nullptr;
    if (it % 3 == 0) {
      xvram_prefetch_desc_v1 p{sizeof(xvram_prefetch_desc_v1), 0, &r, 1, 0, {0, 0}};
      CHECK(api.prefetch_submit(s, &p, &op) == XVRAM_STATUS_SUCCESS, "prefetch_submit");
    } else {
      xvram_transaction_desc_v1 t{sizeof(xvram_transaction_desc_v1), 0, &r, 1, 0, 0,
                                  count_ranges, &ranges, {0, 0}};
      CHECK(api.transaction_submit(s, &t, &op) == XVRAM_STATUS_SUCCESS, "transaction_submit");
    }
    xvram_operation_info_v1 info = XVRAM_OPERATION_INFO_V1_INIT;
    CHECK(api.operation_wait(op, XVRAM_TIMEOUT_INFINITE, &info) == XVRAM_STATUS_SUCCESS, "wait");
    CHECK(info.result == XVRAM_STATUS_SUCCESS, "transaction result %u", info.result);
    api.operation_release(op);
    *done += 1;
  }
  CHECK(ranges.load() == 10, "callbacks saw %llu ranges", (unsigned long long)ranges.load());
  std::vector<uint32_t> back(bytes / 4);
  CHECK(api.allocation_read(big, 0, back.data(), bytes) == XVRAM_STATUS_SUCCESS, "read");
  CHECK(back == data, "transaction bytes changed");
  CHECK(api.allocation_release(big) == XVRAM_STATUS_SUCCESS, "allocation_release");
}

void observer_thread(xvram_session s, const std::atomic<bool>* stop) {
  while (!stop->load()) {
    xvram_session_telemetry_v1 t{};
    t.struct_size = sizeof(t);
    CHECK(api.session_get_telemetry(s, &t) == XVRAM_STATUS_SUCCESS, "telemetry");
    CHECK(t.resident_bytes <= t.cache_target_bytes, "resident bytes over the target");
    xvram_error_info_v1 e = XVRAM_ERROR_INFO_V1_INIT;
    CHECK(api.session_get_error(s, &e) == XVRAM_STATUS_SUCCESS, "session_get_error");
    std::this_thread::yield();
  }
}

} // namespace

int main() {
  if (xvram_get_api(1, sizeof(api), &api) != XVRAM_STATUS_SUCCESS) return 2;
  xvram_session_config_v1 cfg = XVRAM_SESSION_CONFIG_V1_INIT;
  cfg.chunk_size_bytes = kFrame;
  cfg.cache_target_bytes = 24 * kFrame;
  cfg.workspace_cap_bytes = 0;
  cfg.device_headroom_bytes = 0;
  xvram_session s = nullptr;
  if (api.session_create(&cfg, &s) != XVRAM_STATUS_SUCCESS) return 2;
  std::atomic<int> gemms{0}, cancelled{0}, transactions{0};
  std::atomic<bool> stop{false};
  std::vector<std::thread> threads;
  for (int t = 0; t < 4; ++t) threads.emplace_back(gemm_thread, s, t, &gemms, &cancelled);
  threads.emplace_back(transaction_thread, s, &transactions);
  std::thread observer(observer_thread, s, &stop);
  for (std::thread& t : threads) t.join();
  stop = true;
  observer.join();
  if (api.session_drain(s, XVRAM_TIMEOUT_INFINITE) != XVRAM_STATUS_SUCCESS) ++failures;
  if (api.session_close(s, XVRAM_TIMEOUT_INFINITE) != XVRAM_STATUS_SUCCESS) ++failures;
  xvram_session_telemetry_v1 t{};
  t.struct_size = sizeof(t);
  if (api.session_get_telemetry(s, &t) != XVRAM_STATUS_SUCCESS) ++failures;
  const bool balanced = t.mappings == t.unmaps && t.mappings == t.set_access_calls &&
                        t.physical_handles_created == t.physical_handles_released &&
                        t.unsafe_transitions == 0 && t.unsafe_remaps == 0 &&
                        t.dirty_evictions <= t.writebacks_completed && t.resident_bytes == 0;
  if (!balanced) ++failures;
  api.session_release(s);
  std::printf("gemms %d cancelled %d transactions %d balanced %d failures %d\n", gemms.load(),
              cancelled.load(), transactions.load(), balanced ? 1 : 0, failures.load());
  return failures.load() == 0 && gemms + cancelled == 40 && transactions == 16 ? 0 : 1;
}
