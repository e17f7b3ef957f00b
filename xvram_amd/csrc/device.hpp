// device.hpp — the thin device layer under the residency cache and executor.
//
// Replaces the reference's CUDA Driver API dispatch table
// (src/platform/cuda/cuda_api.hpp:30-80) with the HIP calls the path needs
// (VMM reserve/create/map/set-access, pinned host memory, streams, events,
// 2-D async copies, the tile-kernel launch). Two implementations exist:
//   device_hip.cpp     — the product: HIP on gfx950;
//   device_hostsim.cpp — a host-memory simulation linked only into the test
//                        library libxvram_hostsim.so, so the cache, schedule
//                        and accounting can be tested without a GPU (the role
//                        FakeCuda plays in tests/unit/residency_executor_fake_tests.cpp).
// Every call returns 0 on success or the native error code (a hipError_t).
#pragma once

#include <cstdint>
#include <memory>
#include <string>

#include "sgemm_launch.hpp"

namespace xvram {

using Stream = void*;
using Event = void*;

// event_query's answer for work that has not completed yet (error codes are
// positive).
constexpr int kNotReady = -1;

// What a device reports about itself (for reports and diagnostics).
struct DeviceInfo {
  std::string name;
  std::string arch;       // e.g. "gfx950:sramecc+:xnack-"
  std::string pci_bus_id; // "dddd:bb:dd.f"
  uint64_t total_memory = 0;
  uint64_t free_memory = 0;
  uint64_t granularity_minimum = 0;
  uint64_t granularity_recommended = 0;
  int compute_major = 0;
  int compute_minor = 0;
  int multiprocessors = 0;
  bool vmm_supported = false;
  int driver_version = 0;
  int runtime_version = 0;
};

class Device {
public:
  virtual ~Device() = default;

  virtual int init(int ordinal) = 0;
  virtual int driver_version(int* version) = 0;
  virtual int mem_info(uint64_t* free_bytes, uint64_t* total_bytes) = 0;
  virtual int granularity(uint64_t* minimum, uint64_t* recommended) = 0;

  virtual int va_reserve(uint64_t bytes, uint64_t alignment, uint64_t* address) = 0;
  virtual int va_free(uint64_t address, uint64_t bytes) = 0;
  virtual int mem_create(uint64_t bytes, uint64_t* handle) = 0;
  virtual int mem_release(uint64_t handle) = 0;
  virtual int mem_map(uint64_t address, uint64_t bytes, uint64_t handle) = 0;
  virtual int mem_unmap(uint64_t address, uint64_t bytes) = 0;
  virtual int set_access(uint64_t address, uint64_t bytes) = 0;

  virtual int host_alloc(uint64_t bytes, void** pointer) = 0; // pinned
  virtual int host_free(void* pointer) = 0;

  // There are no blocking waits here: the runtime polls event_query against
  // its stall deadline, so no wait on device work is unbounded.
  virtual int stream_create(Stream* stream) = 0;
  virtual int stream_destroy(Stream stream) = 0;
  virtual int event_create(Event* event) = 0;
  virtual int event_destroy(Event event) = 0;
  virtual int event_record(Event event, Stream stream) = 0;
  // 0 = complete, kNotReady = still pending, otherwise an error code.
  virtual int event_query(Event event) = 0;
  virtual int event_elapsed_ms(float* ms, Event start, Event stop) = 0;
  virtual int stream_wait_event(Stream stream, Event event) = 0;

  // Strided 2-D copies (rows of `width` bytes, `height` rows).
  virtual int copy_h2d_2d(uint64_t dst, uint64_t dst_pitch, const void* src, uint64_t src_pitch,
                          uint64_t width, uint64_t height, Stream stream) = 0;
  virtual int copy_d2h_2d(void* dst, uint64_t dst_pitch, uint64_t src, uint64_t src_pitch,
                          uint64_t width, uint64_t height, Stream stream) = 0;
  virtual int fill_zero(uint64_t dst, uint64_t bytes, Stream stream) = 0;

  virtual int launch_sgemm(const kernels::SgemmLaunch& launch, Stream stream) = 0;

  virtual const char* error_name(int code) = 0;
  // True when this is the host simulation (used only for diagnostics).
  virtual bool simulated() const = 0;
};

// Defined by exactly one of device_hip.cpp / device_hostsim.cpp.
std::unique_ptr<Device> make_device();

// What direct_sgemm returns where there is no device (the host simulation).
constexpr int kNoDevice = -2;
// Enqueues one tile-kernel launch on caller device memory on `stream` (a
// hipStream_t, NULL = the calling thread's default stream). A launch that
// splits K uses launch.workspace when it holds every partial the split wants,
// else a stream-ordered allocation freed behind the kernels. Returns 0, the
// native error code, or kNoDevice (sgemm_direct.hip / device_hostsim.cpp).
int direct_sgemm(const kernels::SgemmLaunch& launch, void* stream);
// What direct_sgemm_no_alloc returns for a split wanting more than its scratch.
constexpr int kScratchTooSmall = -3;
// direct_sgemm that allocates nothing: a split that the launch's own
// workspace cannot hold uses the library's static per-GPU scratch (64 MiB,
// shared by every call on that GPU).
int direct_sgemm_no_alloc(const kernels::SgemmLaunch& launch, void* stream);
// Describes device `ordinal` without disturbing the calling thread's current
// device; returns 0 or the native error code.
int describe_device(int ordinal, DeviceInfo& out);
// The device current on the calling thread (hipGetDevice: the HIP counterpart
// of the CUDA context an XVRAM_CONTEXT_ATTACH_CURRENT session captures);
// returns 0 or the native error code (e.g. no device at all).
int current_device(int* ordinal);

} // namespace xvram
