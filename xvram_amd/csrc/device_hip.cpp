// device_hip.cpp — the HIP implementation of the device layer (product path).
//
// Mapping of the reference's Driver API calls (src/platform/cuda/cuda_api.hpp)
// to HIP: cuMemAddressReserve/Free -> hipMemAddressReserve/Free, cuMemCreate/
// Release -> hipMemCreate/Release (pinned device allocations), cuMemMap/Unmap
// -> hipMemMap/Unmap, cuMemSetAccess -> hipMemSetAccess, cuMemHostAlloc ->
// hipHostMalloc, streams and events one to one, cuMemcpyHtoDAsync/DtoHAsync ->
// hipMemcpy2DAsync (strided panels instead of linear chunks).
#include <hip/hip_runtime_api.h>

#include <cstdio>

#include "device.hpp"

namespace xvram {
namespace {

class HipDevice final : public Device {
public:
  int init(int ordinal) override {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return e;
    if (ordinal < 0 || ordinal >= count) return hipErrorInvalidDevice;
    e = hipSetDevice(ordinal);
    if (e != hipSuccess) return e;
    ordinal_ = ordinal;
    prop_ = {};
    prop_.type = hipMemAllocationTypePinned;
    prop_.location.type = hipMemLocationTypeDevice;
    prop_.location.id = ordinal;
    return hipSuccess;
  }

  int driver_version(int* version) override { return hipDriverGetVersion(version); }

  int mem_info(uint64_t* free_bytes, uint64_t* total_bytes) override {
    size_t f = 0, t = 0;
    const hipError_t e = hipMemGetInfo(&f, &t);
    *free_bytes = f;
    *total_bytes = t;
    return e;
  }

  int granularity(uint64_t* minimum, uint64_t* recommended) override {
    size_t lo = 0, hi = 0;
    hipError_t e = hipMemGetAllocationGranularity(&lo, &prop_, hipMemAllocationGranularityMinimum);
    if (e != hipSuccess) return e;
    e = hipMemGetAllocationGranularity(&hi, &prop_, hipMemAllocationGranularityRecommended);
    if (e != hipSuccess) return e;
    *minimum = lo;
    *recommended = hi;
    return hipSuccess;
  }

  int va_reserve(uint64_t bytes, uint64_t alignment, uint64_t* address) override {
    void* p = nullptr;
    const hipError_t e = hipMemAddressReserve(&p, bytes, alignment, nullptr, 0);
    *address = reinterpret_cast<uint64_t>(p);
    return e;
  }
  int va_free(uint64_t address, uint64_t bytes) override {
    return hipMemAddressFree(reinterpret_cast<void*>(address), bytes);
  }
  int mem_create(uint64_t bytes, uint64_t* handle) override {
    hipMemGenericAllocationHandle_t h{};
    const hipError_t e = hipMemCreate(&h, bytes, &prop_, 0);
    // The caller handles the failure (out of memory: resample and retry);
    // leave no error behind for a later hipGetLastError.
    if (e != hipSuccess) (void)hipGetLastError();
    *handle = reinterpret_cast<uint64_t>(h);
    return e;
  }
  int mem_release(uint64_t handle) override {
    return hipMemRelease(reinterpret_cast<hipMemGenericAllocationHandle_t>(handle));
  }
  int mem_map(uint64_t address, uint64_t bytes, uint64_t handle) override {
    return hipMemMap(reinterpret_cast<void*>(address), bytes, 0,
                     reinterpret_cast<hipMemGenericAllocationHandle_t>(handle), 0);
  }
  int mem_unmap(uint64_t address, uint64_t bytes) override {
    return hipMemUnmap(reinterpret_cast<void*>(address), bytes);
  }
  int set_access(uint64_t address, uint64_t bytes) override {
    hipMemAccessDesc desc{};
    desc.location.type = hipMemLocationTypeDevice;
    desc.location.id = ordinal_;
    desc.flags = hipMemAccessFlagsProtReadWrite;
    return hipMemSetAccess(reinterpret_cast<void*>(address), bytes, &desc, 1);
  }

  int host_alloc(uint64_t bytes, void** pointer) override {
    return hipHostMalloc(pointer, bytes, hipHostMallocDefault);
  }
  int host_free(void* pointer) override { return hipHostFree(pointer); }

  int stream_create(Stream* stream) override {
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = s;
    return e;
  }
  int stream_destroy(Stream stream) override {
    return hipStreamDestroy(static_cast<hipStream_t>(stream));
  }
  int event_create(Event* event) override {
    hipEvent_t ev = nullptr;
    const hipError_t e = hipEventCreateWithFlags(&ev, hipEventDefault);
    *event = ev;
    return e;
  }
  int event_destroy(Event event) override { return hipEventDestroy(static_cast<hipEvent_t>(event)); }
  int event_record(Event event, Stream stream) override {
    return hipEventRecord(static_cast<hipEvent_t>(event), static_cast<hipStream_t>(stream));
  }
  int event_query(Event event) override {
    const hipError_t e = hipEventQuery(static_cast<hipEvent_t>(event));
    if (e == hipSuccess) return 0;
    if (e == hipErrorNotReady) return kNotReady;
    return e;
  }
  int event_elapsed_ms(float* ms, Event start, Event stop) override {
    return hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop));
  }
  int stream_wait_event(Stream stream, Event event) override {
    return hipStreamWaitEvent(static_cast<hipStream_t>(stream), static_cast<hipEvent_t>(event), 0);
  }

  int copy_h2d_2d(uint64_t dst, uint64_t dst_pitch, const void* src, uint64_t src_pitch,
                  uint64_t width, uint64_t height, Stream stream) override {
    return hipMemcpy2DAsync(reinterpret_cast<void*>(dst), dst_pitch, src, src_pitch, width, height,
                            hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
  }
  int copy_d2h_2d(void* dst, uint64_t dst_pitch, uint64_t src, uint64_t src_pitch, uint64_t width,
                  uint64_t height, Stream stream) override {
    return hipMemcpy2DAsync(dst, dst_pitch, reinterpret_cast<const void*>(src), src_pitch, width,
                            height, hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream));
  }
  int fill_zero(uint64_t dst, uint64_t bytes, Stream stream) override {
    return hipMemsetAsync(reinterpret_cast<void*>(dst), 0, bytes,
                          static_cast<hipStream_t>(stream));
  }

  int launch_sgemm(const kernels::SgemmLaunch& launch, Stream stream) override {
    return kernels::launch_sgemm(launch, stream);
  }

  const char* error_name(int code) override {
    return hipGetErrorName(static_cast<hipError_t>(code));
  }
  bool simulated() const override { return false; }

private:
  int ordinal_ = 0;
  hipMemAllocationProp prop_{};
};

} // namespace

std::unique_ptr<Device> make_device() { return std::make_unique<HipDevice>(); }

int current_device(int* ordinal) {
  int count = 0;
  if (hipError_t e = hipGetDeviceCount(&count); e != hipSuccess) return e;
  if (count <= 0) return hipErrorNoDevice;
  return hipGetDevice(ordinal);
}

int describe_device(int ordinal, DeviceInfo& out) {
  int count = 0;
  if (hipError_t e = hipGetDeviceCount(&count); e != hipSuccess) return e;
  if (ordinal < 0 || ordinal >= count) return hipErrorInvalidDevice;
  hipDeviceProp_t p{};
  if (hipError_t e = hipGetDeviceProperties(&p, ordinal); e != hipSuccess) return e;
  out.name = p.name;
  out.arch = p.gcnArchName;
  char bus[32];
  std::snprintf(bus, sizeof(bus), "%04x:%02x:%02x.0", p.pciDomainID, p.pciBusID, p.pciDeviceID);
  out.pci_bus_id = bus;
  out.total_memory = p.totalGlobalMem;
  out.compute_major = p.major;
  out.compute_minor = p.minor;
  out.multiprocessors = p.multiProcessorCount;
  int vmm = 0;
  if (hipDeviceGetAttribute(&vmm, hipDeviceAttributeVirtualMemoryManagementSupported, ordinal) ==
      hipSuccess)
    out.vmm_supported = vmm != 0;
  hipMemAllocationProp prop{};
  prop.type = hipMemAllocationTypePinned;
  prop.location.type = hipMemLocationTypeDevice;
  prop.location.id = ordinal;
  size_t g = 0;
  if (hipMemGetAllocationGranularity(&g, &prop, hipMemAllocationGranularityMinimum) == hipSuccess)
    out.granularity_minimum = g;
  if (hipMemGetAllocationGranularity(&g, &prop, hipMemAllocationGranularityRecommended) ==
      hipSuccess)
    out.granularity_recommended = g;
  (void)hipDriverGetVersion(&out.driver_version);
  (void)hipRuntimeGetVersion(&out.runtime_version);
  int current = 0;
  if (hipGetDevice(&current) == hipSuccess && hipSetDevice(ordinal) == hipSuccess) {
    size_t f = 0, t = 0;
    if (hipMemGetInfo(&f, &t) == hipSuccess) out.free_memory = f;
    (void)hipSetDevice(current);
  }
  return hipSuccess;
}

} // namespace xvram
