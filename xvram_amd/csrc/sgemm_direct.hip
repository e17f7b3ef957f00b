// sgemm_direct.hip — the tile kernels on caller device memory (the extension
// table's sgemm_device). The ABI layer has checked the descriptor; here the
// split-K workspace is settled and the launch enqueued on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <vector>

#include "device.hpp"
#include "sgemm_launch.hpp"

namespace xvram {

namespace {

// The split-K workspace of the allocation-free entry point: one array per
// GPU in this file's code object, held until the process ends and shared by
// every call on that GPU (calls that overlap on one GPU race on it). A split
// never wants more: at most one 256 x 256 partial tile per CU (ring kernels;
// two per CU for a tail split) or one 256 x 128 tile per workgroup of two
// rounds of two per CU (the 256 x 128 kernel). Every partial element the reduction uses is written before it
// is read (the padding rows of a ragged partial are read but not used), so
// nothing in the array needs clearing between calls.
constexpr uint64_t kScratchBytes = 128ull << 20;
static_assert(kScratchBytes >= uint64_t(2 * kernels::kComputeUnits) * 256 * 256 * 4 &&
                  kScratchBytes >= kernels::kSplitMaxPartialBytes,
              "the scratch holds the largest split");
static __device__ __align__(256) float scratch[kScratchBytes / 4];

// Device address of `scratch` on each GPU, looked up once per GPU with that
// GPU current (in host code the array's name is only a stand-in).
std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_address;

int scratch_address(hipStream_t stream, void** out) {
  int device = -1;
  hipError_t e = stream != nullptr ? hipStreamGetDevice(stream, &device) : hipGetDevice(&device);
  if (e != hipSuccess) return static_cast<int>(e);
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (device >= static_cast<int>(g_scratch_address.size()))
    g_scratch_address.resize(static_cast<size_t>(device) + 1, nullptr);
  if (g_scratch_address[device] == nullptr) {
    int current = -1;
    if ((e = hipGetDevice(&current)) != hipSuccess) return static_cast<int>(e);
    if (current != device && (e = hipSetDevice(device)) != hipSuccess) return static_cast<int>(e);
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current != device) (void)hipSetDevice(current);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return static_cast<int>(e);
    }
    g_scratch_address[device] = p;
  }
  *out = g_scratch_address[device];
  return 0;
}

} // namespace

int direct_sgemm_no_alloc(const kernels::SgemmLaunch& launch, void* stream) {
  kernels::SgemmLaunch l = launch;
  l.padded = true;
  const uint64_t wanted = kernels::split_k_bytes_wanted(l);
  if (wanted > 0 && (l.workspace == nullptr || l.workspace_bytes < wanted)) {
    if (wanted > kScratchBytes) return kScratchTooSmall;
    void* p = nullptr;
    if (const int rc = scratch_address(static_cast<hipStream_t>(stream), &p)) return rc;
    l.workspace = static_cast<float*>(p);
    l.workspace_bytes = kScratchBytes;
  }
  return kernels::launch_sgemm(l, stream);
}

int direct_sgemm(const kernels::SgemmLaunch& launch, void* stream) {
  kernels::SgemmLaunch l = launch;
  l.padded = true; // each operand holds ld x (stored columns) floats
  auto* s = static_cast<hipStream_t>(stream);
  // The split this launch wants with room for all of its partials; the
  // caller's workspace serves when it holds them, else a stream-ordered one
  // (the same split either way, so the same result).
  const uint64_t wanted = kernels::split_k_bytes_wanted(l);
  void* own = nullptr;
  if (wanted > 0 && (l.workspace == nullptr || l.workspace_bytes < wanted)) {
    if (const hipError_t e = hipMallocAsync(&own, wanted, s); e != hipSuccess) {
      (void)hipGetLastError();
      return static_cast<int>(e);
    }
    l.workspace = static_cast<float*>(own);
    l.workspace_bytes = wanted;
  }
  const int rc = kernels::launch_sgemm(l, stream);
  if (own != nullptr) {
    // Stream-ordered: released behind the kernels that use it.
    const hipError_t e = hipFreeAsync(own, s);
    if (rc == 0 && e != hipSuccess) return static_cast<int>(e);
  }
  return rc;
}

} // namespace xvram
