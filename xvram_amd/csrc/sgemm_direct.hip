// sgemm_direct.hip — the tile kernels on caller device memory (the extension
// table's sgemm_device). The ABI layer has checked the descriptor; here the
// split-K workspace is settled and the launch enqueued on the caller's stream.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "device.hpp"
#include "sgemm_launch.hpp"

namespace xvram {

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
