// device_hostsim.cpp — host-memory simulation of the device layer.
//
// TEST FIXTURE: linked only into libxvram_hostsim.so, which tests/ load to
// exercise the ABI boundary, session worker, panel cache, schedule and
// accounting on machines without a GPU (the reference does the same with its
// FakeCuda driver, tests/unit/residency_executor_fake_tests.cpp:128-1165).
// The product library libxvram.so never contains this file.
//
// Simulation rules: every call completes synchronously; a reserved VA range is
// backed by host memory so mapped frames are ordinary pointers; accesses to
// unmapped frames are detected and fail the call; the tile "kernel" is a
// plain loop with the SgemmLaunch semantics (beta == 0 never reads C). An
// event records the host clock, so the time between two events is the host
// time of the work done between their records.
// Faults can be injected per call site (xvram_hostsim_inject), and the
// reported device memory can be set (xvram_hostsim_set_memory).
#include <algorithm>
#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <thread>
#include <vector>

#include "device.hpp"
#include "runtime.hpp"

namespace xvram {
namespace {

enum Site {
  kInit, kMemInfo, kVaReserve, kVaFree, kMemCreate, kMemRelease, kMemMap, kMemUnmap, kSetAccess,
  kHostAlloc, kStreamCreate, kEventCreate, kEventRecord, kEventQuery, kCopyH2D, kCopyD2H,
  kLaunch,
  // Not a failure: once this site "fails", the event being recorded never
  // completes (event_query keeps answering kNotReady), as if the work queued
  // before it on its stream hung. Persistent: every later record hangs too.
  kEventHang,
  kSiteCount
};

constexpr int kSimFault = 9001;      // injected failure
constexpr int kSimBadAccess = 9002;  // access to an unmapped or unknown address
constexpr int kSimOutOfMemory = 2;   // same value as hipErrorOutOfMemory

struct Injection {
  long skip = -1; // calls to let through before failing; -1 = disabled
  bool persistent = false;
  long delay_skip = -1; // calls to let through before one call sleeps; -1 = none
  int delay_ms = 0;
};

struct SimState {
  std::mutex mutex;
  Injection sites[kSiteCount];
  uint64_t free_bytes = 16ull << 30;
  uint64_t total_bytes = 16ull << 30;
  uint64_t kernel_launches = 0;
  uint64_t split_launches = 0;  // launches that split K (kernels::split_k_plan)
  uint64_t narrow_splits = 0;   // of those, split on the 256 x 128 kernel
  int last_splits = 0;          // K ranges of the last split launch (or tail split)
  uint64_t tail_splits = 0;     // launches that ran as a head and a split tail
  uint64_t edge_splits = 0;     // launches that ran as an interior and edge strips
  uint64_t k_remainders = 0;    // launches that ran as a rounded K and its remainder
  int device_count = 1;       // simulated devices 0 .. device_count-1
  int current_device = 0;     // what the calling thread sees as current (-1: none)
  int last_init_ordinal = -1; // the device the last session set up on
} g_sim;

int fault(Site site) {
  int sleep_ms = 0;
  {
    std::lock_guard<std::mutex> lock(g_sim.mutex);
    Injection& inj = g_sim.sites[site];
    if (inj.delay_skip == 0) sleep_ms = inj.delay_ms;
    if (inj.delay_skip >= 0) --inj.delay_skip;
  }
  // A slow host call (a descheduled thread, a slow driver call): the host
  // time passes, the simulated device stays idle.
  if (sleep_ms > 0) std::this_thread::sleep_for(std::chrono::milliseconds(sleep_ms));
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  Injection& inj = g_sim.sites[site];
  if (inj.skip < 0) return 0;
  if (inj.skip > 0) {
    --inj.skip;
    return 0;
  }
  if (!inj.persistent) inj.skip = -1;
  return kSimFault;
}

class HostSimDevice final : public Device {
public:
  ~HostSimDevice() override {
    for (auto& r : reservations_) std::free(reinterpret_cast<void*>(r.first));
  }

  int init(int ordinal) override {
    if (int f = fault(kInit)) return f;
    std::lock_guard<std::mutex> lock(g_sim.mutex);
    if (ordinal < 0 || ordinal >= g_sim.device_count) return 101; // hipErrorInvalidDevice
    g_sim.last_init_ordinal = ordinal;
    return 0;
  }
  int driver_version(int* version) override {
    *version = 0;
    return 0;
  }
  int mem_info(uint64_t* free_bytes, uint64_t* total_bytes) override {
    if (int f = fault(kMemInfo)) return f;
    std::lock_guard<std::mutex> lock(g_sim.mutex);
    *free_bytes = g_sim.free_bytes;
    *total_bytes = g_sim.total_bytes;
    return 0;
  }
  int granularity(uint64_t* minimum, uint64_t* recommended) override {
    *minimum = 4096;
    *recommended = 4096;
    return 0;
  }

  int va_reserve(uint64_t bytes, uint64_t alignment, uint64_t* address) override {
    if (int f = fault(kVaReserve)) return f;
    const uint64_t align = alignment < 4096 ? 4096 : alignment;
    void* p = std::aligned_alloc(align, (bytes + align - 1) / align * align);
    if (p == nullptr) return kSimOutOfMemory;
    reservations_[reinterpret_cast<uint64_t>(p)] = bytes;
    *address = reinterpret_cast<uint64_t>(p);
    return 0;
  }
  int va_free(uint64_t address, uint64_t bytes) override {
    if (int f = fault(kVaFree)) return f;
    auto it = reservations_.find(address);
    if (it == reservations_.end() || it->second != bytes) return kSimBadAccess;
    for (auto& m : mappings_)
      if (m.first >= address && m.first < address + bytes) return kSimBadAccess; // still mapped
    std::free(reinterpret_cast<void*>(address));
    reservations_.erase(it);
    return 0;
  }
  int mem_create(uint64_t bytes, uint64_t* handle) override {
    if (int f = fault(kMemCreate)) return f;
    std::lock_guard<std::mutex> lock(g_sim.mutex);
    if (bytes > g_sim.free_bytes) return kSimOutOfMemory;
    g_sim.free_bytes -= bytes;
    *handle = ++next_handle_;
    handles_[*handle] = bytes;
    return 0;
  }
  int mem_release(uint64_t handle) override {
    if (int f = fault(kMemRelease)) return f;
    auto it = handles_.find(handle);
    if (it == handles_.end()) return kSimBadAccess;
    for (auto& m : mappings_)
      if (m.second.handle == handle) return kSimBadAccess; // still mapped
    std::lock_guard<std::mutex> lock(g_sim.mutex);
    g_sim.free_bytes += it->second;
    handles_.erase(it);
    return 0;
  }
  int mem_map(uint64_t address, uint64_t bytes, uint64_t handle) override {
    if (int f = fault(kMemMap)) return f;
    if (!handles_.count(handle) || handles_[handle] != bytes || !inside_reservation(address, bytes))
      return kSimBadAccess;
    if (mappings_.count(address)) return kSimBadAccess;
    mappings_[address] = Mapping{bytes, handle, false};
    return 0;
  }
  int mem_unmap(uint64_t address, uint64_t bytes) override {
    if (int f = fault(kMemUnmap)) return f;
    auto it = mappings_.find(address);
    if (it == mappings_.end() || it->second.bytes != bytes) return kSimBadAccess;
    // Scribble over the frame so a stale read after unmapping is visible.
    std::memset(reinterpret_cast<void*>(address), 0xFF, bytes);
    mappings_.erase(it);
    return 0;
  }
  int set_access(uint64_t address, uint64_t bytes) override {
    if (int f = fault(kSetAccess)) return f;
    uint64_t covered = 0;
    for (auto& m : mappings_) {
      if (m.first >= address && m.first + m.second.bytes <= address + bytes) {
        m.second.accessible = true;
        covered += m.second.bytes;
      }
    }
    return covered == bytes ? 0 : kSimBadAccess;
  }

  int host_alloc(uint64_t bytes, void** pointer) override {
    if (int f = fault(kHostAlloc)) return f;
    *pointer = std::aligned_alloc(4096, (bytes + 4095) / 4096 * 4096);
    return *pointer ? 0 : kSimOutOfMemory;
  }
  int host_free(void* pointer) override {
    std::free(pointer);
    return 0;
  }

  int stream_create(Stream* stream) override {
    if (int f = fault(kStreamCreate)) return f;
    *stream = reinterpret_cast<Stream>(++next_object_);
    return 0;
  }
  int stream_destroy(Stream) override { return 0; }
  int event_create(Event* event) override {
    if (int f = fault(kEventCreate)) return f;
    *event = reinterpret_cast<Event>(++next_object_);
    return 0;
  }
  int event_destroy(Event) override { return 0; }
  int event_record(Event event, Stream) override {
    if (int f = fault(kEventRecord)) return f;
    recorded_[event] = std::chrono::steady_clock::now();
    if (fault(kEventHang)) hung_.insert(event);
    else hung_.erase(event);
    return 0;
  }
  int event_query(Event event) override {
    if (int f = fault(kEventQuery)) return f;
    return hung_.count(event) ? kNotReady : 0;
  }
  int event_elapsed_ms(float* ms, Event start, Event stop) override {
    auto a = recorded_.find(start), b = recorded_.find(stop);
    if (a == recorded_.end() || b == recorded_.end()) return kSimBadAccess;
    *ms = std::chrono::duration<float, std::milli>(b->second - a->second).count();
    return 0;
  }
  int stream_wait_event(Stream, Event) override { return 0; }

  int copy_h2d_2d(uint64_t dst, uint64_t dst_pitch, const void* src, uint64_t src_pitch,
                  uint64_t width, uint64_t height, Stream) override {
    if (int f = fault(kCopyH2D)) return f;
    if (!accessible(dst, dst_pitch * (height - 1) + width)) return kSimBadAccess;
    for (uint64_t r = 0; r < height; ++r)
      std::memcpy(reinterpret_cast<char*>(dst + r * dst_pitch),
                  static_cast<const char*>(src) + r * src_pitch, width);
    return 0;
  }
  int copy_d2h_2d(void* dst, uint64_t dst_pitch, uint64_t src, uint64_t src_pitch, uint64_t width,
                  uint64_t height, Stream) override {
    if (int f = fault(kCopyD2H)) return f;
    if (!accessible(src, src_pitch * (height - 1) + width)) return kSimBadAccess;
    for (uint64_t r = 0; r < height; ++r)
      std::memcpy(static_cast<char*>(dst) + r * dst_pitch,
                  reinterpret_cast<const char*>(src + r * src_pitch), width);
    return 0;
  }
  int fill_zero(uint64_t dst, uint64_t bytes, Stream) override {
    if (!accessible(dst, bytes)) return kSimBadAccess;
    std::memset(reinterpret_cast<void*>(dst), 0, bytes);
    return 0;
  }

  int launch_sgemm(const kernels::SgemmLaunch& l, Stream) override {
    if (int f = fault(kLaunch)) return f;
    // A K remainder runs its two launches one after another, and so does an
    // edge split its parts (sgemm_launch.hpp).
    if (const kernels::KParts kp = kernels::k_remainder_parts(l); kp.count > 0) {
      for (int i = 0; i < kp.count; ++i)
        if (const int rc = dispatch(kp.part[i]); rc != 0) return rc;
      std::lock_guard<std::mutex> lock(g_sim.mutex);
      ++g_sim.k_remainders;
      return 0;
    }
    return dispatch(l);
  }

  int dispatch(const kernels::SgemmLaunch& l) {
    if (const kernels::EdgeParts e = kernels::edge_parts(l); e.count > 0) {
      for (int i = 0; i < e.count; ++i)
        if (const int rc = run_launch(e.part[i]); rc != 0) return rc;
      std::lock_guard<std::mutex> lock(g_sim.mutex);
      ++g_sim.edge_splits;
      return 0;
    }
    return run_launch(l);
  }

  int run_launch(const kernels::SgemmLaunch& l) {
    // Same launch contract as the gfx950 kernel (sgemm_launch.hpp).
    const bool aligned = reinterpret_cast<uintptr_t>(l.a) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(l.b) % 16 == 0 &&
                         reinterpret_cast<uintptr_t>(l.c) % 16 == 0 && l.lda % 4 == 0 &&
                         l.ldb % 4 == 0 && l.ldc % 4 == 0 && l.padded;
    if (l.m <= 0 || l.n <= 0 || l.k <= 0 || !aligned) return 1; // hipErrorInvalidValue
    const bool two = l.a2 != nullptr || l.b2 != nullptr;
    if (two && !kernels::two_panel_valid(l)) return 1; // hipErrorInvalidValue
    const int64_t k1 = two ? l.k_split : l.k; // K rows read from a / b
    const auto span = [](int64_t rows, int64_t cols, int64_t ld) {
      return static_cast<uint64_t>(((cols - 1) * ld + rows) * 4);
    };
    const int64_t a_rows = l.a_kcontig ? k1 : l.m, a_cols = l.a_kcontig ? l.m : k1;
    const int64_t b_rows = l.b_ncontig ? l.n : k1, b_cols = l.b_ncontig ? k1 : l.n;
    if (!accessible(reinterpret_cast<uint64_t>(l.a), span(a_rows, a_cols, l.lda)) ||
        !accessible(reinterpret_cast<uint64_t>(l.b), span(b_rows, b_cols, l.ldb)) ||
        !accessible(reinterpret_cast<uint64_t>(l.c), span(l.m, l.n, l.ldc)))
      return kSimBadAccess;
    const int64_t k2 = l.k - k1; // K rows read from a2 / b2
    if (two && (!accessible(reinterpret_cast<uint64_t>(l.a2),
                            span(l.a_kcontig ? k2 : l.m, l.a_kcontig ? l.m : k2, l.lda)) ||
                !accessible(reinterpret_cast<uint64_t>(l.b2),
                            span(l.b_ncontig ? l.n : k2, l.b_ncontig ? k2 : l.n, l.ldb))))
      return kSimBadAccess;
    if ((l.bias_row && !accessible(reinterpret_cast<uint64_t>(l.bias_row), l.m * 4ull)) ||
        (l.bias_col && !accessible(reinterpret_cast<uint64_t>(l.bias_col), l.n * 4ull)))
      return kSimBadAccess;
    // A split launch writes its partials to the workspace (sgemm_launch.hpp);
    // a tail split runs its head rows unsplit and splits its tail rows.
    const kernels::SplitK sk = two ? kernels::SplitK{} : kernels::split_k_plan(l);
    const kernels::TailSplit ts =
        two || sk.splits > 1 ? kernels::TailSplit{} : kernels::tail_split_plan(l);
    struct Rows {
      int64_t first, count;
      kernels::SplitK split;
    };
    std::vector<Rows> segments;
    if (ts.head_m > 0)
      segments = {Rows{0, ts.head_m, kernels::SplitK{}}, Rows{ts.head_m, l.m - ts.head_m, ts.tail}};
    else
      segments = {Rows{0, l.m, sk}};
    for (const Rows& r : segments) {
      const int64_t partial = kernels::split_partial_ld(r.count) * l.n;
      if (r.split.splits > 1 && !accessible(reinterpret_cast<uint64_t>(l.workspace),
                                            static_cast<uint64_t>(r.split.splits * partial * 4)))
        return kSimBadAccess;
    }
    // Events attached to the dispatch are stamped around the kernel itself.
    if (l.start_event) recorded_[l.start_event] = std::chrono::steady_clock::now();
    // Column by column; each element accumulates its K products in order
    // (p ascending, the second panel after the first), in FP32. A split
    // launch (or tail) accumulates each K range into its partial, then adds
    // the partials in range order.
    std::vector<float> acc(static_cast<size_t>(l.m));
    for (int64_t j = 0; j < l.n; ++j) {
      std::fill(acc.begin(), acc.end(), 0.f);
      for (const Rows& r : segments) {
        const int64_t ldp = kernels::split_partial_ld(r.count);
        const int64_t partial = ldp * l.n;
        const int64_t i0 = r.first, i1 = r.first + r.count;
        for (int s = 0; s < r.split.splits && r.split.splits > 1; ++s) {
          float* part = l.workspace + s * partial + j * ldp;
          std::fill(part, part + r.count, 0.f);
          const int64_t p_end = std::min<int64_t>(l.k, int64_t{s + 1} * r.split.depth);
          for (int64_t p = int64_t{s} * r.split.depth; p < p_end; ++p) {
            const float y = l.b_ncontig ? l.b[j + p * l.ldb] : l.b[p + j * l.ldb];
            for (int64_t i = i0; i < i1; ++i)
              part[i - i0] += (l.a_kcontig ? l.a[p + i * l.lda] : l.a[i + p * l.lda]) * y;
          }
          for (int64_t i = i0; i < i1; ++i)
            acc[i] = s == 0 ? part[i - i0] : acc[i] + part[i - i0];
        }
        for (int64_t p = 0; p < k1 && r.split.splits == 1; ++p) {
          const float y = l.b_ncontig ? l.b[j + p * l.ldb] : l.b[p + j * l.ldb];
          for (int64_t i = i0; i < i1; ++i) {
            const float x = l.a_kcontig ? l.a[p + i * l.lda] : l.a[i + p * l.lda];
            acc[i] += x * y;
          }
        }
      }
      for (int64_t p = 0; p < k2; ++p) { // second panel
        const float y = l.b_ncontig ? l.b2[j + p * l.ldb] : l.b2[p + j * l.ldb];
        for (int64_t i = 0; i < l.m; ++i) {
          const float x = l.a_kcontig ? l.a2[p + i * l.lda] : l.a2[i + p * l.lda];
          acc[i] += x * y;
        }
      }
      for (int64_t i = 0; i < l.m; ++i) {
        float& out = l.c[i + j * l.ldc];
        float v = l.beta != 0.f ? l.alpha * acc[i] + l.beta * out : l.alpha * acc[i];
        if (l.bias_row) v += l.bias_row[i];
        if (l.bias_col) v += l.bias_col[j];
        if (l.relu && v < 0.f) v = 0.f;
        out = v;
      }
    }
    if (l.stop_event) recorded_[l.stop_event] = std::chrono::steady_clock::now();
    std::lock_guard<std::mutex> lock(g_sim.mutex);
    ++g_sim.kernel_launches;
    if (sk.splits > 1) {
      ++g_sim.split_launches;
      if (sk.narrow) ++g_sim.narrow_splits;
      g_sim.last_splits = sk.splits;
    }
    if (ts.head_m > 0) {
      ++g_sim.tail_splits;
      g_sim.last_splits = ts.tail.splits;
    }
    return 0;
  }

  const char* error_name(int code) override {
    switch (code) {
    case kSimFault: return "hostsimInjectedFault";
    case kSimBadAccess: return "hostsimBadAccess";
    case kSimOutOfMemory: return "hipErrorOutOfMemory";
    case 101: return "hipErrorInvalidDevice";
    default: return "hostsimError";
    }
  }
  bool simulated() const override { return true; }

private:
  struct Mapping {
    uint64_t bytes;
    uint64_t handle;
    bool accessible;
  };

  bool inside_reservation(uint64_t address, uint64_t bytes) const {
    for (auto& r : reservations_)
      if (address >= r.first && address + bytes <= r.first + r.second) return true;
    return false;
  }
  // Every byte of [address, address+bytes) must lie in mapped, accessible frames.
  bool accessible(uint64_t address, uint64_t bytes) const {
    uint64_t cursor = address;
    const uint64_t end = address + bytes;
    while (cursor < end) {
      auto it = mappings_.upper_bound(cursor);
      if (it == mappings_.begin()) return false;
      --it;
      if (!it->second.accessible || cursor >= it->first + it->second.bytes) return false;
      cursor = it->first + it->second.bytes;
    }
    return true;
  }

  std::map<uint64_t, uint64_t> reservations_;
  std::map<uint64_t, uint64_t> handles_;
  std::map<uint64_t, Mapping> mappings_;
  std::map<Event, std::chrono::steady_clock::time_point> recorded_;
  std::set<Event> hung_; // recorded while kEventHang fired: never complete
  uint64_t next_handle_ = 0;
  uint64_t next_object_ = 0x1000;
};

} // namespace

std::unique_ptr<Device> make_device() { return std::make_unique<HostSimDevice>(); }

int current_device(int* ordinal) {
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  if (g_sim.current_device < 0) return 100; // hipErrorNoDevice
  *ordinal = g_sim.current_device;
  return 0;
}

int describe_device(int ordinal, DeviceInfo& out) {
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  if (ordinal < 0 || ordinal >= g_sim.device_count) return 101; // hipErrorInvalidDevice
  out.name = "xvram host simulation";
  out.arch = "hostsim";
  out.pci_bus_id.clear();
  out.total_memory = g_sim.total_bytes;
  out.free_memory = g_sim.free_bytes;
  out.granularity_minimum = out.granularity_recommended = 4096;
  out.vmm_supported = true;
  return 0;
}

// Caller device memory does not exist in the simulation.
int direct_sgemm(const kernels::SgemmLaunch&, void*) { return kNoDevice; }
int direct_sgemm_no_alloc(const kernels::SgemmLaunch&, void*) { return kNoDevice; }

} // namespace xvram

// Test-only controls exported by libxvram_hostsim.so.
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_inject(int site, long skip,
                                                                           int persistent) {
  using namespace xvram;
  if (site < 0 || site >= kSiteCount) return -1;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  g_sim.sites[site].skip = skip;
  g_sim.sites[site].persistent = persistent != 0;
  return 0;
}

// After `skip` more calls at `site`, the next one sleeps `ms` on the host
// before it runs (the call itself succeeds).
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_delay(int site, long skip,
                                                                          int ms) {
  using namespace xvram;
  if (site < 0 || site >= kSiteCount || skip < 0 || ms < 0) return -1;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  g_sim.sites[site].delay_skip = skip;
  g_sim.sites[site].delay_ms = ms;
  return 0;
}

extern "C" __attribute__((visibility("default"))) void xvram_hostsim_reset() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  for (auto& s : g_sim.sites) s = Injection{};
  g_sim.free_bytes = g_sim.total_bytes = 16ull << 30;
  g_sim.kernel_launches = 0;
  g_sim.split_launches = 0;
  g_sim.narrow_splits = 0;
  g_sim.last_splits = 0;
  g_sim.tail_splits = 0;
  g_sim.edge_splits = 0;
  g_sim.k_remainders = 0;
  g_sim.device_count = 1;
  g_sim.current_device = 0;
  g_sim.last_init_ordinal = -1;
}

// Simulated device count and the device current on calling threads (-1 = no
// device current, as when the HIP runtime finds no device).
extern "C" __attribute__((visibility("default"))) void xvram_hostsim_set_devices(int count,
                                                                                 int current) {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  g_sim.device_count = count;
  g_sim.current_device = current;
}

// The ordinal the most recent session set up on (-1 before any).
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_last_init_ordinal() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  return g_sim.last_init_ordinal;
}

extern "C" __attribute__((visibility("default"))) void xvram_hostsim_set_memory(uint64_t free_b,
                                                                                uint64_t total_b) {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  g_sim.free_bytes = free_b;
  g_sim.total_bytes = total_b;
}

// Launches that split K since the last reset; *last_splits = the K ranges of
// the last one.
extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_split_launches(
    int* last_splits) {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  if (last_splits != nullptr) *last_splits = g_sim.last_splits;
  return g_sim.split_launches;
}

// The split rule itself (kernels::split_k_shape) for a launch shape: returns
// the number of K ranges (1 = unsplit), their depth and whether they run on
// the 256 x 128 kernel.
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_split_shape(
    int64_t m, int64_t n, int64_t k, int nt, int ring, uint64_t workspace_bytes, int* depth,
    int* narrow) {
  const xvram::kernels::SplitK sk =
      xvram::kernels::split_k_shape(m, n, k, nt != 0, ring != 0, workspace_bytes);
  if (depth != nullptr) *depth = sk.depth;
  if (narrow != nullptr) *narrow = sk.narrow ? 1 : 0;
  return sk.splits;
}

// Of those, the launches whose ranges ran on the 256 x 128 kernel (tiles that
// are not all interior 256 x 256 ones).
// The tail split rule (kernels::tail_split_shape) for a launch shape: returns
// the number of K ranges of the tail (1 = no tail split), *head_m the head's
// rows and *depth the tail's range depth.
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_tail_split_shape(
    int64_t m, int64_t n, int64_t k, int nt, int ring, uint64_t workspace_bytes, int64_t* head_m,
    int* depth) {
  const xvram::kernels::TailSplit ts =
      xvram::kernels::tail_split_shape(m, n, k, nt != 0, ring != 0, workspace_bytes);
  if (head_m != nullptr) *head_m = ts.head_m;
  if (depth != nullptr) *depth = ts.head_m > 0 ? ts.tail.depth : 0;
  return ts.head_m > 0 ? ts.tail.splits : 1;
}

// The edge split rule for a launch shape (panels the ring kernels can
// address): 1 if kernels::edge_split_rated_faster takes it, and *wants = 1 if
// one of its parts would split (kernels::edge_split_wants_workspace).
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_edge_split_shape(
    int64_t m, int64_t n, int64_t k, int nt, int* wants) {
  if (wants != nullptr)
    *wants = xvram::kernels::edge_split_wants_workspace(m, n, k, nt != 0) ? 1 : 0;
  return xvram::kernels::edge_split_rated_faster(m, n, k, nt != 0) ? 1 : 0;
}

// Launches that ran as a rounded K and its remainder since the last reset.
extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_k_remainder_launches() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  return g_sim.k_remainders;
}

// The K remainder rule for a launch shape: the rounded K (0: none).
extern "C" __attribute__((visibility("default"))) int64_t xvram_hostsim_k_remainder_shape(
    int64_t m, int64_t n, int64_t k, int nt) {
  return xvram::kernels::k_remainder_shape(m, n, k, nt != 0);
}

// The partials' bytes a launch wants (kernels::split_k_bytes_wanted) for a
// launch of that shape, form and leading dimensions (pointers unused).
extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_bytes_wanted(
    int m, int n, int k, int a_kcontig, int b_ncontig, int64_t lda, int64_t ldb) {
  xvram::kernels::SgemmLaunch l;
  l.m = m;
  l.n = n;
  l.k = k;
  l.a_kcontig = a_kcontig != 0;
  l.b_ncontig = b_ncontig != 0;
  l.lda = lda;
  l.ldb = ldb;
  l.ldc = m;
  return xvram::kernels::split_k_bytes_wanted(l);
}

// Launches that ran as an interior and edge strips since the last reset.
extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_edge_split_launches() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  return g_sim.edge_splits;
}

// Launches that ran as a head and a split tail since the last reset.
extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_tail_split_launches() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  return g_sim.tail_splits;
}

extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_narrow_split_launches() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  return g_sim.narrow_splits;
}

extern "C" __attribute__((visibility("default"))) uint64_t xvram_hostsim_kernel_launches() {
  using namespace xvram;
  std::lock_guard<std::mutex> lock(g_sim.mutex);
  return g_sim.kernel_launches;
}

// ---- pure host logic of the runtime, exposed for differential tests ----------

// The entry-state transition table (1 = legal).
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_legal_transition(int from,
                                                                                     int to) {
  using xvram::EntryState;
  return xvram::is_legal_transition(static_cast<EntryState>(from), static_cast<EntryState>(to))
             ? 1
             : 0;
}

// normalize_accesses over flat arrays: allocations as (id, bytes) pairs, ranges
// as (id, offset, length, mode) quads. Outputs normalised ranges as quads and
// chunks as (id, index, valid_bytes, requires_h2d, marks_dirty); *n_out_* hold
// the capacities (in records) on entry and the counts on return. Returns 0,
// 1 with the problem's name in `error`, or 2 when a capacity is too small.
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_normalize(
    const uint64_t* allocs, uint64_t n_allocs, const uint64_t* ranges, uint64_t n_ranges,
    uint64_t chunk_bytes, uint64_t* out_ranges, uint64_t* n_out_ranges, uint64_t* out_chunks,
    uint64_t* n_out_chunks, char* error, uint64_t error_len) {
  std::vector<xvram::AllocationExtent> extents;
  for (uint64_t i = 0; i < n_allocs; ++i) extents.push_back({allocs[2 * i], allocs[2 * i + 1]});
  std::vector<xvram::AccessSpan> spans;
  for (uint64_t i = 0; i < n_ranges; ++i)
    spans.push_back({ranges[4 * i], ranges[4 * i + 1], ranges[4 * i + 2],
                     static_cast<uint32_t>(ranges[4 * i + 3])});
  std::vector<xvram::AccessSpan> normalized;
  std::vector<xvram::ChunkPlan> chunks;
  const char* problem = xvram::normalize_accesses(extents, spans, chunk_bytes, normalized, chunks);
  if (problem) {
    std::snprintf(error, error_len, "%s", problem);
    return 1;
  }
  if (normalized.size() > *n_out_ranges || chunks.size() > *n_out_chunks) return 2;
  for (size_t i = 0; i < normalized.size(); ++i) {
    out_ranges[4 * i] = normalized[i].allocation_id;
    out_ranges[4 * i + 1] = normalized[i].offset;
    out_ranges[4 * i + 2] = normalized[i].length;
    out_ranges[4 * i + 3] = normalized[i].mode;
  }
  for (size_t i = 0; i < chunks.size(); ++i) {
    out_chunks[5 * i] = chunks[i].allocation_id;
    out_chunks[5 * i + 1] = chunks[i].index;
    out_chunks[5 * i + 2] = chunks[i].valid_bytes;
    out_chunks[5 * i + 3] = chunks[i].requires_h2d ? 1 : 0;
    out_chunks[5 * i + 4] = chunks[i].marks_dirty ? 1 : 0;
  }
  *n_out_ranges = normalized.size();
  *n_out_chunks = chunks.size();
  return 0;
}

// Runs a command program against a fresh victim policy (kind: 0 CLOCK, 1 LRU).
// Each command is 7 words {op, a, b, c, d, e, f}; one result word per command:
//   op 0 insert(id=a, sequence=b, speculative=c, one_touch=d)           -> 0
//   op 1 touch(id=a, sequence=b, one_touch=c)                           -> 0
//   op 2 erase(id=a)                                                    -> 1 if erased
//   op 3 set candidate id=a: state=b, hot=c, pins=d, in_flight=e, in_working_set=f -> 0
//   op 4 drop candidate id=a                                            -> 0
//   op 5 select_victim(current candidates)                              -> id or ~0
extern "C" __attribute__((visibility("default"))) int xvram_hostsim_policy_run(
    int kind, const uint64_t* program, uint64_t commands, uint64_t* results) {
  std::unique_ptr<xvram::EvictionPolicy> policy =
      xvram::make_policy(kind == 1 ? XVRAM_CACHE_POLICY_LRU : XVRAM_CACHE_POLICY_CLOCK);
  std::vector<xvram::VictimCandidate> candidates;
  for (uint64_t i = 0; i < commands; ++i) {
    const uint64_t* c = program + 7 * i;
    results[i] = 0;
    switch (c[0]) {
    case 0: policy->insert(c[1], c[2], c[3] != 0, c[4] != 0); break;
    case 1: policy->touch(c[1], c[2], c[3] != 0); break;
    case 2: results[i] = policy->erase(c[1]) ? 1 : 0; break;
    case 3: {
      xvram::VictimCandidate v;
      v.id = c[1];
      v.state = static_cast<xvram::EntryState>(c[2]);
      v.hot = c[3] != 0;
      v.pins = static_cast<uint32_t>(c[4]);
      v.in_flight = c[5] != 0;
      v.in_working_set = c[6] != 0;
      bool replaced = false;
      for (auto& existing : candidates)
        if (existing.id == v.id) {
          existing = v;
          replaced = true;
        }
      if (!replaced) candidates.push_back(v);
      break;
    }
    case 4:
      for (size_t k = 0; k < candidates.size(); ++k)
        if (candidates[k].id == c[1]) {
          candidates.erase(candidates.begin() + static_cast<std::ptrdiff_t>(k));
          break;
        }
      break;
    case 5: {
      const auto victim = policy->select_victim(candidates);
      results[i] = victim ? *victim : ~0ull;
      break;
    }
    default: return -1;
    }
  }
  return 0;
}
