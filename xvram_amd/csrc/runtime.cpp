// runtime.cpp — host backing, VRAM frame pool, panel/chunk cache, transactions.
#include "runtime.hpp"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <numeric>
#include <thread>

namespace xvram {

namespace {

uint64_t lcm64(uint64_t a, uint64_t b) { return a / std::gcd(a, b) * b; }

} // namespace

bool is_legal_transition(EntryState from, EntryState to) {
  using S = EntryState;
  if (to == S::poisoned) return true;
  switch (from) {
  case S::host_clean: return to == S::prefetch_queued || to == S::mapping;
  case S::prefetch_queued: return to == S::host_clean || to == S::mapping;
  case S::mapping: return to == S::host_clean || to == S::h2d_in_flight || to == S::resident_clean;
  case S::h2d_in_flight: return to == S::resident_clean;
  case S::resident_clean: return to == S::resident_dirty || to == S::evicting;
  case S::resident_dirty: return to == S::writeback_queued || to == S::evicting;
  case S::writeback_queued: return to == S::d2h_in_flight;
  case S::d2h_in_flight: return to == S::resident_clean;
  case S::evicting: return to == S::host_clean;
  case S::poisoned: return false;
  }
  return false;
}

bool keys_overlap(const PanelKey& a, const PanelKey& b) {
  if (a.allocation_id != b.allocation_id) return false;
  if (a.offset >= b.end() || b.offset >= a.end()) return false;
  if (a.pitch == b.pitch && a.pitch > 0 && a.height > 1 && b.height > 1) {
    const uint64_t P = a.pitch;
    const uint64_t ar = a.offset / P, ac = a.offset % P;
    const uint64_t br = b.offset / P, bc = b.offset % P;
    if (ac + a.width <= P && bc + b.width <= P) {
      const bool rows = ar < br + b.height && br < ar + a.height;
      const bool cols = ac < bc + b.width && bc < ac + a.width;
      return rows && cols;
    }
    return true;
  }
  // A contiguous range against a strided rectangle: test the rectangle's lines.
  const PanelKey* line = a.height == 1 ? &a : (b.height == 1 ? &b : nullptr);
  if (line == nullptr) return true; // different pitches: conservative
  const PanelKey& s = line == &a ? b : a;
  const uint64_t lo = line->offset, hi = line->offset + line->width;
  uint64_t l = 0;
  if (lo > s.offset + s.width && s.pitch > 0) l = (lo - s.offset - s.width) / s.pitch;
  for (; l < s.height; ++l) {
    const uint64_t start = s.offset + l * s.pitch;
    if (start >= hi) break;
    if (lo < start + s.width) return true;
  }
  return false;
}

// Host time between two dispatches on one compute lane after which the second
// kernel takes a start event of its own (Runtime::record_kernel): far below
// any duration-guard limit. A host that keeps ahead of short kernels
// dispatches them well within it; where the host waits longer between
// dispatches, the kernels it waits for are long and a start event (~5 us of
// device time) is small next to them.
constexpr std::chrono::milliseconds kStartEventAfterHostGap{2};

Runtime::Runtime(RuntimeConfig config) : config_(config), device_(make_device()) {
  if (const char* path = std::getenv("XVRAM_TRACE_FILE"); path != nullptr && *path != '\0')
    trace_path_ = path;
  t_.struct_size = sizeof(t_);
}

Runtime::~Runtime() { (void)close(); }

Error Runtime::device_failure(int code, std::string_view stage, std::string_view operation) {
  poisoned_ = true;
  t_.poisoned = 1;
  Error e = make_error(XVRAM_STATUS_CUDA_ERROR, stage, operation, "HIP runtime call failed");
  e.native_domain = XVRAM_NATIVE_ERROR_CUDA;
  e.native_code = code;
  e.native_name = device_->error_name(code);
  return e;
}

Error Runtime::poison(std::string_view stage, std::string_view operation,
                      std::string_view message) {
  poisoned_ = true;
  t_.poisoned = 1;
  return make_error(XVRAM_STATUS_POISONED, stage, operation, message);
}

// Polls rather than blocks (hipEventSynchronize has no time limit). The host
// spins (yielding) through the first 50 ms, the length of the longest waits
// of a running schedule (a frame's last kernel), so completion is seen at
// once; longer waits sleep 100 us between queries.
Error Runtime::await_event(Event event, std::string_view stage, std::string_view operation) {
  if (quarantined_)
    return make_error(XVRAM_STATUS_POISONED, stage, operation,
                      "device work of this session is quarantined after a stalled or failed wait");
  const Clock::time_point begun = Clock::now();
  const Clock::time_point give_up = begun + std::chrono::milliseconds(config_.stall_timeout_ms);
  for (;;) {
    const int q = device_->event_query(event);
    if (q == 0) return {};
    if (q != kNotReady) {
      quarantined_ = true;
      return device_failure(q, stage, operation);
    }
    const Clock::time_point now = Clock::now();
    if (now >= give_up) {
      quarantined_ = true;
      Error e = poison(stage, operation,
                       "device work did not complete within the stall deadline; the frames, "
                       "workspace and host buffers it may still use are quarantined");
      e.status = XVRAM_STATUS_TIMEOUT;
      return e;
    }
    if (now - begun < std::chrono::milliseconds(50)) std::this_thread::yield();
    else std::this_thread::sleep_for(std::chrono::microseconds(100));
  }
}

Error Runtime::await_streams(std::initializer_list<Stream> streams, std::string_view stage,
                             std::string_view operation) {
  if (quarantined_)
    return make_error(XVRAM_STATUS_POISONED, stage, operation,
                      "device work of this session is quarantined after a stalled or failed wait");
  if (streams.size() > static_cast<size_t>(kSyncMarkers))
    return make_error(XVRAM_STATUS_INTERNAL, stage, operation, "too many streams for one wait");
  int used = 0;
  for (Stream s : streams) {
    if (int rc = device_->event_record(sync_markers_[used], s)) {
      quarantined_ = true;
      return device_failure(rc, stage, operation);
    }
    ++used;
  }
  for (int i = 0; i < used; ++i)
    if (Error e = await_event(sync_markers_[i], stage, operation)) return e;
  return {};
}

// Session setup (reference src/residency/runtime.cpp:212-596): bind the
// device, align the frame size to the VMM granularity, derive the budget from
// hipMemGetInfo, reserve the panel arena and create the three streams.
Error Runtime::setup() {
  if (int rc = device_->init(config_.device_ordinal)) return device_failure(rc, "setup", "init");
  int version = 0;
  if (device_->driver_version(&version) == 0 && version > 0)
    t_.cuda_driver_version = static_cast<uint32_t>(version);

  uint64_t gmin = 0, grec = 0;
  if (int rc = device_->granularity(&gmin, &grec))
    return device_failure(rc, "setup", "granularity");
  if (gmin == 0) gmin = 4096;
  if (grec == 0) grec = gmin;
  granularity_ = lcm64(gmin, grec);
  uint64_t aligned = 0;
  if (!checked_add(config_.chunk_bytes, granularity_ - 1, aligned))
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "setup", "chunk_size", "chunk size overflows");
  frame_bytes_ = aligned / granularity_ * granularity_;

  uint64_t free_bytes = 0, total_bytes = 0;
  if (int rc = device_->mem_info(&free_bytes, &total_bytes))
    return device_failure(rc, "setup", "mem_info");
  ++t_.budget_sample_count;
  t_.cuda_free_bytes_minimum = free_bytes;
  t_.cuda_free_bytes_end = free_bytes;
  if (free_bytes <= config_.device_headroom_bytes)
    return make_error(XVRAM_STATUS_DEVICE_OUT_OF_MEMORY, "setup", "budget",
                      "free device memory does not exceed the configured headroom");
  uint64_t target = free_bytes - config_.device_headroom_bytes;
  if (config_.cache_target_bytes != 0) target = std::min(target, config_.cache_target_bytes);
  target = target / frame_bytes_ * frame_bytes_;
  if (target <= config_.workspace_reserve_bytes ||
      (target - config_.workspace_reserve_bytes) / frame_bytes_ < 2)
    return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "setup", "budget",
                      "cache target leaves fewer than two frames");
  target_bytes_ = target;
  capacity_ = (target - config_.workspace_reserve_bytes) / frame_bytes_;
  max_capacity_ = capacity_;
  configured_cap_ = config_.cache_target_bytes != 0 ? config_.cache_target_bytes : total_bytes;
  last_budget_sample_ = Clock::now();
  policy_ = make_policy(config_.cache_policy);
  t_.cache_target_bytes = target_bytes_;
  t_.cache_target_minimum_bytes = target_bytes_;
  t_.cache_target_maximum_bytes = target_bytes_;

  arena_bytes_ = capacity_ * frame_bytes_;
  if (int rc = device_->va_reserve(arena_bytes_, granularity_, &arena_)) {
    arena_ = 0;
    return device_failure(rc, "setup", "va_reserve");
  }
  frames_.resize(capacity_);
  for (uint64_t i = 0; i < capacity_; ++i) {
    frames_[i].index = i;
    frames_[i].slot = arena_ + i * frame_bytes_;
  }
  if (int rc = device_->stream_create(&compute_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->stream_create(&compute2_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->stream_create(&h2d_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->stream_create(&d2h_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->event_create(&op_start_)) return device_failure(rc, "setup", "event");
  if (int rc = device_->event_create(&op_start2_)) return device_failure(rc, "setup", "event");
  if (int rc = device_->event_create(&carry_fence_)) return device_failure(rc, "setup", "event");
  for (Event& marker : sync_markers_)
    if (int rc = device_->event_create(&marker)) return device_failure(rc, "setup", "event");
  t_.flags = XVRAM_TELEMETRY_NO_PHYSICAL_ALIASES | XVRAM_TELEMETRY_STABLE_VIRTUAL_ADDRESSES;
  setup_done_ = true;
  return {};
}

// Drain (reference runtime.cpp:1497-1538 with release_mappings = false): every
// dirty entry is written back and stays cached, clean; then the device idles.
// A poisoned session only waits for its streams.
Error Runtime::drain() {
  if (!setup_done_ || closed_) return {};
  if (!poisoned_)
    if (Error e = flush_all()) return e;
  if (Error e = await_streams({h2d_, compute_, compute2_, d2h_}, "drain", "stream_wait")) return e;
  writebacks_settled();
  return {};
}

Error Runtime::flush_all() {
  bool issued = false;
  for (Frame& f : frames_) {
    if (!f.keyed || !f.dirty) continue;
    if (f.pins > 0)
      return make_error(XVRAM_STATUS_INTERNAL, "cache", "flush", "a dirty entry is still in use");
    if (Error e = writeback(f, false)) return e;
    issued = true;
  }
  if (issued) {
    if (Error e = await_stream(d2h_, "cache", "writeback_wait")) return e;
    writebacks_settled();
  }
  return {};
}

// The D2H stream has drained: every write-back issued so far has landed.
// Outside an operation (read, write, drain, close) the events those copies
// took are complete and go back to the pool at once.
void Runtime::writebacks_settled() {
  pending_writebacks_.clear();
  for (Frame& f : frames_) f.writeback_done = nullptr;
  if (in_operation_) return;
  event_pool_.insert(event_pool_.end(), events_in_use_.begin(), events_in_use_.end());
  events_in_use_.clear();
}

// Teardown (reference runtime.cpp:1540-1857): wait for the device, unmap and
// release every frame, free the VA reservations, streams, events and host
// backing.
Error Runtime::close() {
  if (closed_) return {};
  closed_ = true;
  Error first;
  auto note = [&](int rc, const char* what) {
    if (rc != 0 && !first) first = device_failure(rc, "close", what);
  };
  if (!setup_done_) {
    for (auto& [id, a] : allocations_) device_->host_free(a.host);
    allocations_.clear();
    return {};
  }
  // Dirty entries reach host memory first (reference close writes back each
  // resident_dirty chunk before unmapping it, runtime.cpp:1620-1625).
  for (Frame& f : frames_) f.pins = 0;
  if (!poisoned_)
    if (Error e = flush_all(); e && !first) first = e;
  if (!quarantined_)
    if (Error e = await_streams({h2d_, compute_, compute2_, d2h_}, "close", "stream_wait");
        e && !first)
      first = e;
  if (quarantined_) return abandon_device_resources();
  for (Frame& f : frames_) {
    if (f.keyed) {
      index_.erase(f.key);
      f.keyed = false;
    }
    if (f.mapped_at) {
      note(device_->mem_unmap(f.mapped_at, frame_bytes_), "unmap");
      ++t_.unmaps;
      f.mapped_at = 0;
    }
    if (f.handle) {
      note(device_->mem_release(f.handle), "release");
      ++t_.physical_handles_released;
      f.handle = 0;
    }
    if (f.ready) device_->event_destroy(f.ready);
    if (f.retire) device_->event_destroy(f.retire);
    f.ready = f.retire = f.retire_ref = nullptr;
  }
  if (workspace_va_) {
    note(device_->mem_unmap(workspace_va_, workspace_bytes_), "unmap");
    ++t_.unmaps;
    note(device_->mem_release(workspace_handle_), "release");
    ++t_.physical_handles_released;
    note(device_->va_free(workspace_va_, workspace_bytes_), "va_free");
    workspace_va_ = 0;
  }
  if (arena_) note(device_->va_free(arena_, arena_bytes_), "va_free");
  arena_ = 0;
  for (Event e : event_pool_) device_->event_destroy(e);
  for (Event e : events_in_use_) device_->event_destroy(e);
  for (Event e : carried_events_) device_->event_destroy(e);
  event_pool_.clear();
  events_in_use_.clear();
  carried_events_.clear();
  carried_trace_.clear();
  pending_writebacks_.clear();
  for (Event* e : {&op_start_, &op_start2_, &carry_fence_}) {
    if (*e) device_->event_destroy(*e);
    *e = nullptr;
  }
  for (Event& marker : sync_markers_) {
    if (marker) device_->event_destroy(marker);
    marker = nullptr;
  }
  for (Stream s : {h2d_, compute_, compute2_, d2h_})
    if (s) device_->stream_destroy(s);
  compute_ = compute2_ = h2d_ = d2h_ = nullptr;
  for (auto& [id, a] : allocations_) {
    if (a.va) note(device_->va_free(a.va, a.va_bytes), "va_free");
    device_->host_free(a.host);
  }
  allocations_.clear();
  t_.resident_bytes = 0;
  return first;
}

// Teardown of a quarantined runtime (reference runtime.cpp:1575-1595,
// 1745-1760, and the SDK's abandon at sdk/runtime.cpp:900-915): device work
// whose completion was never observed may still read or write the frames, the
// workspace and the pinned host buffers, so none of them is unmapped,
// released or freed, and the streams and events stay alive. They are given up
// until the process ends; the cache index and the allocation table are
// dropped, so nothing in this session reaches them again. Close reports
// CLEANUP_FAILED.
Error Runtime::abandon_device_resources() {
  uint64_t mapped = 0;
  for (Frame& f : frames_) {
    if (f.mapped_at) ++mapped;
    if (f.keyed) index_.erase(f.key);
    f.keyed = false;
  }
  frames_.clear();
  allocations_.clear();
  event_pool_.clear();
  events_in_use_.clear();
  carried_events_.clear();
  carried_trace_.clear();
  pending_writebacks_.clear();
  compute_ = compute2_ = h2d_ = d2h_ = nullptr;
  op_start_ = op_start2_ = carry_fence_ = nullptr;
  for (Event& marker : sync_markers_) marker = nullptr;
  workspace_va_ = 0;
  arena_ = 0;
  t_.resident_bytes = 0;
  return make_error(XVRAM_STATUS_CLEANUP_FAILED, "close", "quarantine",
                    "device work of this session never completed; " + std::to_string(mapped) +
                        " mapped frames, the workspace and the pinned host buffers were "
                        "abandoned instead of released");
}

// ---- allocations -----------------------------------------------------------

void Runtime::parallel_copy(void* dst, const void* src, uint64_t bytes) {
  constexpr uint64_t kSlice = 64ull << 20;
  if (bytes <= kSlice) {
    if (src) std::memcpy(dst, src, bytes);
    else std::memset(dst, 0, bytes);
    return;
  }
  const unsigned hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const uint64_t slices = ceil_div(bytes, kSlice);
  const unsigned workers = static_cast<unsigned>(std::min<uint64_t>(hw, slices));
  std::vector<std::thread> pool;
  pool.reserve(workers);
  for (unsigned w = 0; w < workers; ++w) {
    pool.emplace_back([=]() {
      for (uint64_t s = w; s < slices; s += workers) {
        const uint64_t begin = s * kSlice;
        const uint64_t n = std::min(kSlice, bytes - begin);
        if (src) std::memcpy(static_cast<char*>(dst) + begin, static_cast<const char*>(src) + begin, n);
        else std::memset(static_cast<char*>(dst) + begin, 0, n);
      }
    });
  }
  for (auto& t : pool) t.join();
}

// Allocation with an authoritative host copy (reference runtime.cpp:598-727
// registers zero-filled chunks; here one pinned buffer, zero-filled, that the
// DMA engines read and write directly — no staging copy, no per-block hash).
Error Runtime::allocate(uint64_t bytes, uint64_t alignment, uint32_t priority,
                        HostAllocation*& out) {
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "allocation", "create", "session is poisoned");
  if (launches_blocked_)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "allocate",
                      "allocation size or runtime state is invalid");
  void* host = nullptr;
  if (int rc = device_->host_alloc(bytes, &host)) {
    if (rc == 2 /* out of memory */)
      return make_error(XVRAM_STATUS_HOST_OUT_OF_MEMORY, "allocation", "host_alloc",
                        "pinned host backing could not be allocated");
    return device_failure(rc, "allocation", "host_alloc");
  }
  parallel_copy(host, nullptr, bytes);
  HostAllocation a;
  a.id = next_allocation_id_++;
  a.bytes = bytes;
  a.alignment = alignment;
  a.priority = priority;
  a.host = static_cast<char*>(host);
  pinned_bytes_ += bytes;
  pinned_peak_bytes_ = std::max(pinned_peak_bytes_, pinned_bytes_);
  auto [it, inserted] = allocations_.emplace(a.id, a);
  (void)inserted;
  out = &it->second;
  return {};
}

HostAllocation* Runtime::find(uint64_t id) {
  auto it = allocations_.find(id);
  return it == allocations_.end() ? nullptr : &it->second;
}

Error Runtime::release(uint64_t id) {
  HostAllocation* a = find(id);
  if (!a) return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "release", "unknown allocation");
  if (Error e = invalidate(id, 0, a->bytes)) return e;
  if (a->va) {
    for (Frame& f : frames_)
      if (f.mapped_at >= a->va && f.mapped_at < a->va + a->va_bytes)
        if (Error e = unmap_frame(f)) return e;
    if (int rc = device_->va_free(a->va, a->va_bytes)) return device_failure(rc, "allocation", "va_free");
    a->va = 0;
  }
  device_->host_free(a->host);
  pinned_bytes_ -= a->bytes;
  allocations_.erase(id);
  lost_.erase(std::remove_if(lost_.begin(), lost_.end(),
                             [id](const PanelKey& k) { return k.allocation_id == id; }),
              lost_.end());
  return {};
}

Error Runtime::write(uint64_t id, uint64_t offset, const void* source, uint64_t bytes) {
  HostAllocation* a = find(id);
  uint64_t end = 0;
  if (!a) return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "write", "unknown allocation");
  if (!checked_add(offset, bytes, end) || end > a->bytes)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "write",
                      "write range exceeds the allocation");
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "allocation", "write", "session is poisoned");
  // Cached entries overlapping the range become stale: drop them first.
  if (Error e = invalidate(id, offset, end)) return e;
  parallel_copy(a->host + offset, source, bytes);
  if (bytes > 0 && !lost_.empty()) {
    PanelKey range;
    range.allocation_id = id;
    range.offset = offset;
    range.width = bytes;
    range.height = 1;
    range.pitch = bytes;
    range.kind = EntryKind::chunk;
    forget_lost_within(range);
  }
  return {};
}

Error Runtime::read(uint64_t id, uint64_t offset, void* destination, uint64_t bytes) {
  HostAllocation* a = find(id);
  uint64_t end = 0;
  if (!a) return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "read", "unknown allocation");
  if (!checked_add(offset, bytes, end) || end > a->bytes)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "allocation", "read",
                      "read range exceeds the allocation");
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "allocation", "read", "session is poisoned");
  // Dirty entries overlapping the range are written back first and stay
  // cached, clean (reference Runtime::read -> flush_overlapping(..., false),
  // runtime.cpp:931-945, 3155-3173).
  if (bytes > 0) {
    PanelKey range;
    range.allocation_id = id;
    range.offset = offset;
    range.width = bytes;
    range.height = 1;
    range.pitch = bytes;
    range.kind = EntryKind::chunk;
    bool issued = false;
    for (Frame& f : frames_) {
      if (!f.keyed || !f.dirty || !keys_overlap(f.key, range)) continue;
      if (f.pins > 0)
        return make_error(XVRAM_STATUS_BUSY, "cache", "read", "entry is in use by an operation");
      if (Error e = writeback(f, false)) return e;
      issued = true;
    }
    if (issued) {
      if (Error e = await_stream(d2h_, "allocation", "writeback_wait")) return e;
      writebacks_settled();
    }
    if (Error e = check_not_lost(range, "allocation", "read")) return e;
  }
  parallel_copy(destination, a->host + offset, bytes);
  return {};
}

// ---- frames ----------------------------------------------------------------

// A frame's handle is mapped at one address at a time: its arena slot while
// it holds a panel, the chunk's address inside the owning allocation's VA
// while it holds a chunk. Moving it waits for its last consumer first.
Error Runtime::map_frame_at(Frame& f, uint64_t address) {
  if (f.mapped_at == address) {
    f.address = address;
    return {};
  }
  if (!f.handle) {
    uint64_t handle = 0;
    int rc = device_->mem_create(frame_bytes_, &handle);
    if (rc == 2 /* out of memory */) {
      // Someone else took device memory: resample the budget once (which may
      // shrink the pool) and retry if this frame is still inside it
      // (reference create_handle, runtime.cpp:3184-3211).
      ++t_.target_oom_retries;
      if (Error e = refresh_budget(0, workspace_bytes_, true)) return e;
      if (f.index >= capacity_)
        return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "cache", "mem_create_retry",
                          "a budget shrink took the frame this allocation was about to use");
      rc = device_->mem_create(frame_bytes_, &handle);
    }
    if (rc == 2)
      return make_error(XVRAM_STATUS_DEVICE_OUT_OF_MEMORY, "cache", "mem_create",
                        "physical frame allocation failed");
    if (rc) return device_failure(rc, "cache", "mem_create");
    f.handle = handle;
    ++t_.physical_handles_created;
  }
  if (f.mapped_at)
    if (Error e = unmap_frame(f)) return e;
  check_generation(f);
  if (int rc = device_->mem_map(address, frame_bytes_, f.handle))
    return device_failure(rc, "cache", "mem_map");
  f.mapped_at = address;
  f.address = address;
  ++t_.mappings;
  if (int rc = device_->set_access(address, frame_bytes_))
    return device_failure(rc, "cache", "set_access");
  ++t_.set_access_calls;
  if (!f.ready)
    if (int rc = device_->event_create(&f.ready)) return device_failure(rc, "cache", "event");
  if (!f.retire)
    if (int rc = device_->event_create(&f.retire)) return device_failure(rc, "cache", "event");
  return {};
}

void Runtime::move(Frame& f, EntryState to) {
  if (!is_legal_transition(f.state, to)) ++t_.unsafe_transitions;
  f.state = to;
}

// Every remap, unmap and refill happens only after the host has seen the
// frame's latest retire event complete; anything else is counted.
void Runtime::check_generation(const Frame& f) {
  if (f.completed != f.generation) ++t_.unsafe_remaps;
}

Error Runtime::record_retire(Frame& f, Stream stream) {
  if (int rc = device_->event_record(f.retire, stream)) return device_failure(rc, "cache", "record");
  adopt_retire(f, f.retire);
  return {};
}

// `done` becomes the frame's retire event: one more event generation.
void Runtime::adopt_retire(Frame& f, Event done) {
  f.retire_ref = done;
  f.retire_pending = true;
  f.retire_seq = ++retire_records_;
  ++f.generation;
}

// A kernel on compute lane `lane` used the frame: it retires after it, and
// after the last kernel on the other lane that used it.
void Runtime::adopt_lane(Frame& f, Event done, int lane) {
  adopt_retire(f, done);
  f.lane_ref[lane] = done;
  f.lane_pending[lane] = true;
}

Error Runtime::unmap_frame(Frame& f) {
  if (!f.mapped_at) return {};
  if (Error e = wait_retired(f)) return e;
  check_generation(f);
  if (int rc = device_->mem_unmap(f.mapped_at, frame_bytes_))
    return device_failure(rc, "cache", "mem_unmap");
  ++t_.unmaps;
  f.mapped_at = 0;
  return {};
}

// A frame is handed out for a new entry only after its last consumer's event
// has retired; the host checks (and if necessary waits for) that event.
Error Runtime::wait_retired(Frame& f) {
  if (!f.retire_pending) return {};
  ++t_.event_boundaries;
  const int q = device_->event_query(f.retire_ref);
  if (q == kNotReady) {
    time_intervals(false); // the host is about to wait anyway
    if (Error e = await_event(f.retire_ref, "cache", "retire_wait")) return e;
  } else if (q != 0) {
    quarantined_ = true;
    return device_failure(q, "cache", "event_query");
  }
  // The other compute lane's last use may finish later than retire_ref.
  for (int lane = 0; lane < kLanes; ++lane) {
    if (!f.lane_pending[lane]) continue;
    if (f.lane_ref[lane] != f.retire_ref)
      if (Error e = await_event(f.lane_ref[lane], "cache", "retire_wait")) return e;
    f.lane_pending[lane] = false;
  }
  f.retire_pending = false;
  f.completed = f.generation;
  f.writeback_done = nullptr; // recorded no later than the retire event
  if (f.state == EntryState::evicting) move(f, EntryState::host_clean);
  return {};
}

Error Runtime::evict_key(Frame& f, bool was_dirty) {
  if (!f.keyed) return {};
  index_.erase(f.key);
  policy_->erase(f.index);
  f.keyed = false;
  f.dirty = false;
  f.unwritten = false;
  f.overwrote_unflushed = false;
  f.ready_pending = false;
  t_.resident_bytes -= frame_bytes_;
  if (was_dirty) ++t_.dirty_evictions;
  if (f.state == EntryState::mapping) {
    move(f, EntryState::host_clean); // never filled: roll back
  } else {
    if (f.state == EntryState::h2d_in_flight) move(f, EntryState::resident_clean);
    move(f, EntryState::evicting);
    if (!f.retire_pending) move(f, EntryState::host_clean);
  }
  // A chunk frame stays mapped at the chunk's address until the frame is
  // reused (map_frame_at moves it) or the chunk is acquired again (it is then
  // taken back without a remap).
  return {};
}

bool Runtime::allocation_hot(uint64_t allocation_id) {
  const HostAllocation* a = find(allocation_id);
  return a && a->priority == XVRAM_ALLOCATION_HOT;
}

bool Runtime::allocation_streaming(uint64_t allocation_id) {
  const HostAllocation* a = find(allocation_id);
  return a && a->priority == XVRAM_ALLOCATION_STREAMING;
}

void Runtime::set_protected(std::vector<PanelKey> keys) {
  std::sort(keys.begin(), keys.end());
  keys.erase(std::unique(keys.begin(), keys.end()), keys.end());
  protected_ = std::move(keys);
}

// Frame choice (reference acquire_frame, runtime.cpp:3470-3529): a free frame
// (the one idle longest), else a not-yet-created frame, else the victim the
// session's policy names among unpinned resident entries (a dirty victim is
// written back first). Only frames inside the live capacity are considered.
// A free frame whose last consumer is still pending (typically a C tile whose
// write-back was just queued) would make the host wait for that consumer while
// launches it could already enqueue sit idle; a clean entry whose last
// consumer was recorded earlier in the schedule is evicted instead when the
// policy names one. Entries the executor declared protected (the panels of its
// next launches) are offered to the policy as part of the working set, i.e.
// not eligible, unless no other entry is: the policy's order of eviction among
// the rest is unchanged, it just never evicts a panel a launch about to run
// needs while something else could go. The choice depends only on the
// schedule (the order of retire records and the declared panels), never on
// how far the device has progressed, so the accounting of a run is
// reproducible.
Error Runtime::select_frame(Frame*& out) {
  Frame* free_frame = nullptr;
  Frame* uncreated = nullptr;
  std::vector<VictimCandidate> candidates;
  candidates.reserve(capacity_);
  for (uint64_t i = 0; i < capacity_; ++i) {
    Frame& f = frames_[i];
    if (!f.handle) {
      if (!uncreated) uncreated = &f;
      continue;
    }
    if (f.pins > 0) continue;
    if (!f.keyed) {
      if (!free_frame || f.last_use < free_frame->last_use) free_frame = &f;
      continue;
    }
    VictimCandidate c;
    c.id = f.index;
    c.state = f.state;
    c.hot = allocation_hot(f.key.allocation_id);
    c.in_working_set = std::binary_search(protected_.begin(), protected_.end(), f.key);
    candidates.push_back(c);
  }
  // The policy with the protected entries held back, then, if that finds
  // nothing, over every candidate.
  const auto choose = [&](std::vector<VictimCandidate>& list) -> std::optional<uint64_t> {
    if (std::optional<uint64_t> v = policy_->select_victim(list)) return v;
    bool any = false;
    for (VictimCandidate& c : list) {
      any = any || c.in_working_set;
      c.in_working_set = false;
    }
    return any ? policy_->select_victim(list) : std::nullopt;
  };
  Frame* chosen = free_frame ? free_frame : uncreated;
  if (free_frame && free_frame->retire_pending) {
    std::vector<VictimCandidate> older;
    for (const VictimCandidate& c : candidates) {
      const Frame& f = frames_[c.id];
      if (!f.dirty && (!f.retire_pending || f.retire_seq < free_frame->retire_seq))
        older.push_back(c);
    }
    if (!older.empty()) {
      // Only an unprotected entry is worth evicting to spare the wait.
      if (const std::optional<uint64_t> victim = policy_->select_victim(older)) {
        Frame& v = frames_[*victim];
        if (Error e = evict_key(v, false)) return e;
        ++t_.clean_evictions;
        chosen = &v;
      }
    }
  }
  if (!chosen) {
    const std::optional<uint64_t> victim = choose(candidates);
    if (!victim)
      return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "cache", "select_frame",
                        "every cache frame is pinned by the current working set");
    Frame& v = frames_[*victim];
    if (v.dirty) {
      if (Error e = writeback_and_evict(v)) return e;
    } else {
      if (Error e = evict_key(v, false)) return e;
      ++t_.clean_evictions;
    }
    chosen = &v;
  }
  if (Error e = wait_retired(*chosen)) return e;
  if (chosen->used_before) ++t_.handle_reuses;
  chosen->used_before = true;
  move(*chosen, EntryState::mapping);
  out = chosen;
  return {};
}

Error Runtime::take_event(Event& out) {
  if (!event_pool_.empty()) {
    out = event_pool_.back();
    event_pool_.pop_back();
  } else if (int rc = device_->event_create(&out)) {
    return device_failure(rc, "cache", "event_create");
  }
  events_in_use_.push_back(out);
  return {};
}

Error Runtime::fill_entry(Frame& f, const PanelKey& key, uint64_t packed_pitch, bool needs_data,
                          const std::vector<PanelPiece>* pieces, std::vector<Event>* piece_ready) {
  ++t_.cache_misses;
  f.keyed = true;
  f.key = key;
  f.packed_pitch = packed_pitch;
  f.pins = 1;
  f.dirty = false;
  f.last_use = ++tick_;
  index_[key] = f.index;
  policy_->insert(f.index, ++policy_sequence_, prefetching_,
                  allocation_streaming(key.allocation_id));
  t_.resident_bytes += frame_bytes_;
  t_.resident_bytes_peak = std::max(t_.resident_bytes_peak, t_.resident_bytes);
  check_generation(f);
  f.unwritten = !needs_data;
  if (!needs_data) {
    move(f, EntryState::resident_clean);
    return {};
  }
  move(f, EntryState::h2d_in_flight);
  for (const auto& [written, done] : pending_writebacks_) {
    // Host bytes this fill reads may still be in flight from a write-back.
    if (!keys_overlap(written, key)) continue;
    if (int rc = device_->stream_wait_event(h2d_, done))
      return device_failure(rc, "cache", "stream_wait");
  }
  HostAllocation* a = find(key.allocation_id);
  if (!a || key.end() > a->bytes)
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "fill", "entry outside its allocation");
  static const std::vector<PanelPiece> kWhole;
  const std::vector<PanelPiece>& parts = pieces ? *pieces : kWhole;
  const size_t copies = parts.empty() ? 1 : parts.size();
  for (size_t i = 0; i < copies; ++i) {
    PanelPiece pc{0, key.height, 0, key.width};
    if (!parts.empty()) pc = parts[i];
    TraceInterval iv;
    iv.kind = 'h';
    iv.bytes = pc.lines * pc.bytes;
    if (Error e = take_event(iv.start)) return e;
    if (int rc = device_->event_record(iv.start, h2d_)) return device_failure(rc, "cache", "record");
    if (int rc = device_->copy_h2d_2d(f.address + pc.line0 * packed_pitch + pc.byte0, packed_pitch,
                                      a->host + key.offset + pc.line0 * key.pitch + pc.byte0,
                                      key.pitch, pc.bytes, pc.lines, h2d_))
      return device_failure(rc, "cache", "copy_h2d");
    if (Error e = take_event(iv.stop)) return e;
    if (int rc = device_->event_record(iv.stop, h2d_)) return device_failure(rc, "cache", "record");
    trace_.push_back(iv);
    // The piece's stop event (an operation-owned event) marks it landed.
    if (piece_ready) piece_ready->push_back(iv.stop);
    f.ready_stamp = iv.stop;
  }
  if (int rc = device_->event_record(f.ready, h2d_)) return device_failure(rc, "cache", "record");
  f.ready_pending = true;
  t_.bytes_h2d += key.bytes();
  return {};
}

Error Runtime::acquire(const PanelKey& key, uint64_t packed_pitch, bool needs_data, Frame*& out) {
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "cache", "acquire", "session is poisoned");
  if (packed_pitch < key.width || packed_pitch * key.height > frame_bytes_)
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "panel does not fit one frame");
  auto it = index_.find(key);
  if (it != index_.end()) {
    Frame& f = frames_[it->second];
    if (f.packed_pitch == packed_pitch) {
      ++f.pins;
      f.last_use = ++tick_;
      ++t_.cache_hits;
      if (!prefetching_)
        policy_->touch(f.index, ++policy_sequence_, allocation_streaming(key.allocation_id));
      out = &f;
      return {};
    }
    // Same rectangle cached with another packing: drop it.
    if (f.pins > 0)
      return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "conflicting pinned packing");
    if (f.dirty) {
      if (Error e = writeback_and_evict(f)) return e;
    } else {
      if (Error e = evict_key(f, false)) return e;
      ++t_.clean_evictions;
    }
  }
  if (Error e = flush_overlapping(key, nullptr)) return e;
  if (needs_data)
    if (Error e = check_not_lost(key, "cache", "fill")) return e;
  Frame* f = nullptr;
  if (Error e = select_frame(f)) return e;
  if (Error e = map_frame_at(*f, f->slot)) return abandon_mapping(*f, e);
  if (Error e = fill_entry(*f, key, packed_pitch, needs_data)) return e;
  out = f;
  return {};
}

// A frame select_frame handed out (state mapping) could not be mapped: it
// goes back to host_clean, so a later selection starts from a legal state.
Error Runtime::abandon_mapping(Frame& f, Error e) {
  if (f.state == EntryState::mapping) move(f, EntryState::host_clean);
  if (!f.handle) f.used_before = false; // its handle was never created
  return e;
}

// The carried entry is inserted like any executor fill (not as a speculative
// prefetch): the next operation pins it before anything else, so the victim
// policy must not rank it below older entries.
Error Runtime::carry_fill(const PanelKey& key, uint64_t packed_pitch, bool& issued) {
  issued = false;
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "cache", "carry", "session is poisoned");
  if (index_.count(key)) return {};
  for (const auto& [written, done] : pending_writebacks_)
    if (keys_overlap(written, key)) return {};
  for (const Frame& f : frames_)
    if (f.keyed && f.dirty && keys_overlap(f.key, key)) return {};
  if (check_not_lost(key, "cache", "carry")) return {}; // its own operation reports it
  if (!carry_active_) {
    if (int rc = device_->event_record(carry_fence_, h2d_)) return device_failure(rc, "cache", "record");
    carry_active_ = true;
    carry_trace_mark_ = trace_.size();
    carry_event_mark_ = events_in_use_.size();
  }
  Frame* f = nullptr;
  if (Error e = acquire(key, packed_pitch, true, f)) return e;
  f->carry_serial = op_serial_;
  issued = true;
  // Retired by its own copy: evicting or unmapping the frame waits for the fill.
  return release_after(*f, h2d_, false);
}

Error Runtime::acquire_pieces(const PanelKey& key, uint64_t packed_pitch,
                              const std::vector<PanelPiece>& pieces, Frame*& out,
                              std::vector<Event>& piece_ready) {
  piece_ready.clear();
  if (pieces.size() < 2 || index_.count(key)) return acquire(key, packed_pitch, true, out);
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "cache", "acquire", "session is poisoned");
  if (packed_pitch < key.width || packed_pitch * key.height > frame_bytes_)
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "panel does not fit one frame");
  uint64_t covered = 0;
  for (const PanelPiece& pc : pieces) {
    if (pc.line0 + pc.lines > key.height || pc.byte0 + pc.bytes > key.width)
      return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "piece outside its panel");
    covered += pc.lines * pc.bytes;
  }
  if (covered != key.bytes())
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "pieces do not tile the panel");
  if (Error e = flush_overlapping(key, nullptr)) return e;
  if (Error e = check_not_lost(key, "cache", "fill")) return e;
  Frame* f = nullptr;
  if (Error e = select_frame(f)) return e;
  if (Error e = map_frame_at(*f, f->slot)) return abandon_mapping(*f, e);
  if (Error e = fill_entry(*f, key, packed_pitch, true, &pieces, &piece_ready)) return e;
  out = f;
  return {};
}

// Orders `stream` after the fill; from then on the entry's bytes are resident
// for everything enqueued on that stream.
// A write-back of the entry still in flight is waited for too: the work on
// `stream` may overwrite the frame.
Error Runtime::wait_ready(Frame& f, Stream stream) {
  if (f.writeback_done) {
    // An operation-owned event (the write-back's stop event).
    if (Error e = stream_wait(stream, f.writeback_done, f.writeback_done)) return e;
    f.writeback_done = nullptr;
  }
  if (!f.ready_pending) return {};
  // A pending fill was issued in this operation or carried into it, so its
  // stamp is one of this operation's events.
  if (Error e = stream_wait(stream, f.ready, f.ready_stamp)) return e;
  if (f.state == EntryState::h2d_in_flight) move(f, EntryState::resident_clean);
  return {};
}

Error Runtime::release_after(Frame& f, Stream stream, bool dirty) {
  if (f.pins <= 0) return make_error(XVRAM_STATUS_INTERNAL, "cache", "release", "frame is not pinned");
  if (Error e = record_retire(f, stream)) return e;
  return unpin(f, dirty);
}

Error Runtime::release_after_event(Frame& f, Event done, bool dirty, int lane) {
  if (f.pins <= 0) return make_error(XVRAM_STATUS_INTERNAL, "cache", "release", "frame is not pinned");
  if (!done) return make_error(XVRAM_STATUS_INTERNAL, "cache", "release", "no retire event");
  if (lane < 0 || lane >= kLanes)
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "release", "no such compute lane");
  adopt_lane(f, done, lane);
  return unpin(f, dirty);
}

Error Runtime::release_after_lanes(Frame& f) {
  if (f.pins <= 0) return make_error(XVRAM_STATUS_INTERNAL, "cache", "release", "frame is not pinned");
  Event e1 = nullptr;
  if (Error e = take_event(e1)) return e;
  if (int rc = device_->event_record(e1, compute2_)) return device_failure(rc, "cache", "record");
  if (Error e = record_retire(f, compute_)) return e;
  f.lane_ref[0] = f.retire;
  f.lane_pending[0] = true;
  f.lane_ref[1] = e1;
  f.lane_pending[1] = true;
  return unpin(f, false);
}

Error Runtime::take_scratch(Frame*& out) {
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "cache", "scratch", "session is poisoned");
  Frame* f = nullptr;
  if (Error e = select_frame(f)) return e;
  if (Error e = map_frame_at(*f, f->slot)) return abandon_mapping(*f, e);
  move(*f, EntryState::resident_clean);
  f->pins = 1;
  f->last_use = ++tick_;
  out = f;
  return {};
}

Error Runtime::release_scratch(Frame& f) {
  if (Error e = release_after_lanes(f)) return e;
  move(f, EntryState::evicting);
  if (!f.retire_pending) move(f, EntryState::host_clean);
  return {};
}

Error Runtime::unpin(Frame& f, bool dirty) {
  --f.pins;
  if (dirty && f.state != EntryState::resident_dirty) {
    if (f.state == EntryState::h2d_in_flight) move(f, EntryState::resident_clean);
    move(f, EntryState::resident_dirty);
  }
  f.last_use = ++tick_;
  if (!dirty) return {};
  if (f.dirty && f.dirty_serial != op_serial_) f.overwrote_unflushed = true;
  f.dirty = true;
  f.unwritten = false;
  f.dirty_serial = op_serial_;
  // Other cached copies of these bytes are stale from now on.
  return drop_overlapping(f.key, &f);
}

// Clean, idle entries whose bytes intersect bytes just written back are stale.
// Dropping the key is enough: the frame itself is reused only after its
// retire event (select_frame waits for it).
Error Runtime::drop_overlapping(const PanelKey& written, const Frame* except) {
  for (Frame& f : frames_) {
    if (&f == except || !f.keyed || f.pins > 0 || f.dirty) continue;
    if (!keys_overlap(f.key, written)) continue;
    if (Error e = evict_key(f, false)) return e;
    ++t_.clean_evictions;
  }
  return {};
}

// Dirty write-back (reference writeback, runtime.cpp:3899-4262): the D2H copy
// is ordered after the frame's last consumer and becomes the frame's retire
// event, so the frame is refilled only after the host bytes are current; a
// fill of overlapping host bytes waits for the copy (pending_writebacks_), and
// so does a later writer of the same frame when the entry stays cached
// (Frame::writeback_done, waited for in wait_ready).
Error Runtime::writeback(Frame& f, bool evict) {
  if (!f.keyed || !f.dirty || f.pins > 0)
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "writeback", "frame is not an idle dirty entry");
  HostAllocation* a = find(f.key.allocation_id);
  if (!a) return make_error(XVRAM_STATUS_INTERNAL, "cache", "writeback", "entry owner is gone");
  if (f.retire_pending)
    if (int rc = device_->stream_wait_event(d2h_, f.retire_ref))
      return device_failure(rc, "cache", "stream_wait");
  for (int lane = 0; lane < kLanes; ++lane)
    if (f.lane_pending[lane] && f.lane_ref[lane] != f.retire_ref)
      if (int rc = device_->stream_wait_event(d2h_, f.lane_ref[lane]))
        return device_failure(rc, "cache", "stream_wait");
  move(f, EntryState::writeback_queued);
  TraceInterval iv;
  iv.kind = 'd';
  iv.bytes = f.key.bytes();
  if (Error e = take_event(iv.start)) return e;
  if (int rc = device_->event_record(iv.start, d2h_)) return device_failure(rc, "cache", "record");
  if (int rc = device_->copy_d2h_2d(a->host + f.key.offset, f.key.pitch, f.address, f.packed_pitch,
                                    f.key.width, f.key.height, d2h_))
    return device_failure(rc, "cache", "copy_d2h");
  move(f, EntryState::d2h_in_flight);
  if (Error e = take_event(iv.stop)) return e;
  if (int rc = device_->event_record(iv.stop, d2h_)) return device_failure(rc, "cache", "record");
  // Intervals are traced per operation; a write-back outside one (read,
  // drain, close) is not.
  if (in_operation_) trace_.push_back(iv);
  if (Error e = record_retire(f, d2h_)) return e;
  // The frame now matches what the host will hold once the copy retires; its
  // retire event (the copy) gates any reuse.
  move(f, EntryState::resident_clean);
  f.dirty = false;
  f.overwrote_unflushed = false;
  const PanelKey written = f.key;
  forget_lost_within(written); // these bytes are whole again once the copy lands
  pending_writebacks_[written] = iv.stop;
  t_.bytes_d2h += written.bytes();
  ++t_.writebacks_completed;
  if (!evict) {
    f.writeback_done = iv.stop;
    return {};
  }
  if (Error e = evict_key(f, true)) return e;
  return drop_overlapping(written, &f);
}

Error Runtime::flush_overlapping(const PanelKey& key, const Frame* except) {
  for (Frame& f : frames_) {
    if (&f == except || !f.keyed || !f.dirty || !keys_overlap(f.key, key)) continue;
    if (f.pins > 0)
      return make_error(XVRAM_STATUS_INTERNAL, "cache", "flush_overlapping",
                        "an entry overlapping the one being filled is written by the operation");
    if (Error e = writeback(f, false)) return e;
  }
  return {};
}

Error Runtime::make_room(uint64_t frames_needed) {
  std::vector<Frame*> idle_dirty;
  for (uint64_t i = 0; i < capacity_; ++i) {
    Frame& f = frames_[i];
    if (f.keyed && f.dirty && f.pins == 0 && f.dirty_serial < op_serial_) idle_dirty.push_back(&f);
  }
  const uint64_t spare = capacity_ > frames_needed ? capacity_ - frames_needed : 0;
  if (idle_dirty.size() <= spare) return {};
  std::sort(idle_dirty.begin(), idle_dirty.end(),
            [](const Frame* x, const Frame* y) { return x->last_use < y->last_use; });
  const size_t excess = idle_dirty.size() - spare;
  for (size_t i = 0; i < excess; ++i)
    if (Error e = writeback(*idle_dirty[i], false)) return e;
  return {};
}

Error Runtime::invalidate(uint64_t allocation_id, uint64_t begin, uint64_t end) {
  if (end <= begin) return {};
  PanelKey range;
  range.allocation_id = allocation_id;
  range.offset = begin;
  range.width = end - begin;
  range.height = 1;
  range.pitch = end - begin;
  range.kind = EntryKind::chunk;
  for (Frame& f : frames_) {
    if (!f.keyed || !keys_overlap(f.key, range)) continue;
    if (f.pins > 0)
      return make_error(XVRAM_STATUS_BUSY, "cache", "invalidate", "entry is in use by an operation");
    if (f.dirty) {
      if (Error e = writeback_and_evict(f)) return e;
      if (Error e = await_stream(d2h_, "cache", "writeback_wait")) return e;
      writebacks_settled();
    } else {
      if (Error e = wait_retired(f)) return e;
      if (Error e = evict_key(f, false)) return e;
      ++t_.clean_evictions;
    }
  }
  return {};
}

// A failed operation drops what it wrote: the host copy stays authoritative.
// Entries it rewrote while they still held an earlier operation's unwritten
// results lose those results too; their rectangles are recorded as lost.
void Runtime::discard_dirty() {
  for (Frame& f : frames_) {
    f.pins = 0;
    if (f.keyed && ((f.dirty && f.dirty_serial == op_serial_) || f.unwritten)) {
      if (f.dirty && f.overwrote_unflushed) lost_.push_back(f.key);
      f.dirty = false;
      (void)evict_key(f, false);
    }
  }
}

Error Runtime::check_not_lost(const PanelKey& range, const char* stage,
                              const char* operation) const {
  for (const PanelKey& k : lost_)
    if (keys_overlap(k, range))
      return make_error(XVRAM_STATUS_CORRUPTION, stage, operation,
                        "these bytes held results of an earlier operation that a failed "
                        "operation overwrote before they were written back; write them again");
  return {};
}

// Lost rectangles that lie inside `rewritten` (same allocation) are whole
// again: a contiguous rewrite covers every line of a rectangle inside its
// byte range; a rectangle rewrite covers one with the same pitch whose lines
// and columns lie inside it.
void Runtime::forget_lost_within(const PanelKey& rewritten) {
  const auto inside = [&](const PanelKey& k) {
    if (k.allocation_id != rewritten.allocation_id) return false;
    if (rewritten.height == 1)
      return k.offset >= rewritten.offset && k.end() <= rewritten.offset + rewritten.width;
    if (k.pitch != rewritten.pitch || rewritten.pitch == 0) return k == rewritten;
    const uint64_t P = rewritten.pitch;
    const uint64_t r0 = rewritten.offset / P, c0 = rewritten.offset % P;
    const uint64_t kr = k.offset / P, kc = k.offset % P;
    return kr >= r0 && kr + k.height <= r0 + rewritten.height && kc >= c0 &&
           kc + k.width <= c0 + rewritten.width;
  };
  lost_.erase(std::remove_if(lost_.begin(), lost_.end(), inside), lost_.end());
}

// ---- transactions and prefetch -----------------------------------------------

Error Runtime::reserve_allocation_va(HostAllocation& a) {
  if (a.va) return {};
  const uint64_t bytes = round_up(a.bytes, frame_bytes_);
  uint64_t va = 0;
  if (int rc = device_->va_reserve(bytes, granularity_, &va))
    return device_failure(rc, "transaction", "va_reserve");
  a.va = va;
  a.va_bytes = bytes;
  return {};
}

// One workspace region of the session's workspace cap, created on first use
// (the cap is already excluded from the frame budget).
Error Runtime::ensure_workspace(uint64_t bytes) {
  if (bytes == 0 || workspace_va_) return {};
  const uint64_t size = round_up(std::max<uint64_t>(config_.workspace_reserve_bytes, 1), granularity_);
  uint64_t va = 0, handle = 0;
  if (int rc = device_->va_reserve(size, granularity_, &va))
    return device_failure(rc, "transaction", "workspace_reserve");
  if (int rc = device_->mem_create(size, &handle)) {
    (void)device_->va_free(va, size);
    return device_failure(rc, "transaction", "workspace_create");
  }
  ++t_.physical_handles_created;
  if (int rc = device_->mem_map(va, size, handle)) return device_failure(rc, "transaction", "workspace_map");
  ++t_.mappings;
  if (int rc = device_->set_access(va, size)) return device_failure(rc, "transaction", "workspace_access");
  ++t_.set_access_calls;
  workspace_va_ = va;
  workspace_bytes_ = size;
  workspace_handle_ = handle;
  t_.workspace_bytes = size;
  return {};
}

const char* normalize_accesses(const std::vector<AllocationExtent>& allocations,
                               const std::vector<AccessSpan>& ranges, uint64_t chunk_bytes,
                               std::vector<AccessSpan>& normalized,
                               std::vector<ChunkPlan>& chunks) {
  normalized.clear();
  chunks.clear();
  std::map<uint64_t, uint64_t> sizes;
  for (const AllocationExtent& a : allocations) sizes[a.id] = a.bytes;
  std::map<uint64_t, std::vector<const AccessSpan*>> by_alloc;
  for (const AccessSpan& r : ranges) {
    if (r.mode != XVRAM_ACCESS_READ && r.mode != XVRAM_ACCESS_READ_WRITE &&
        r.mode != XVRAM_ACCESS_WRITE_ONLY)
      return "invalid_access_mode";
    if (r.length == 0) return "zero_length";
    auto size = sizes.find(r.allocation_id);
    if (size == sizes.end()) return "unknown_allocation";
    uint64_t end = 0;
    if (!checked_add(r.offset, r.length, end)) return "range_overflow";
    if (r.offset >= size->second || end > size->second) return "range_out_of_bounds";
    by_alloc[r.allocation_id].push_back(&r);
  }
  // Per allocation, a sweep over the range boundaries: between two
  // consecutive boundaries the covering ranges are fixed, and their combined
  // mode is the one mode they share, else read-write. Counting the active
  // ranges per mode makes this O((B + R) log R) instead of testing every
  // range against every elementary piece.
  struct Boundary {
    uint64_t at;
    int delta; // +1 a range starts here, -1 one ends here
    uint32_t mode;
  };
  std::vector<Boundary> bounds;
  for (const auto& [id, list] : by_alloc) {
    bounds.clear();
    bounds.reserve(2 * list.size());
    for (const AccessSpan* r : list) {
      bounds.push_back(Boundary{r->offset, +1, r->mode});
      bounds.push_back(Boundary{r->offset + r->length, -1, r->mode});
    }
    std::sort(bounds.begin(), bounds.end(),
              [](const Boundary& a, const Boundary& b) { return a.at < b.at; });
    uint64_t active[3] = {0, 0, 0}; // READ, READ_WRITE, WRITE_ONLY
    for (size_t i = 0; i < bounds.size();) {
      const uint64_t lo = bounds[i].at;
      for (; i < bounds.size() && bounds[i].at == lo; ++i)
        active[bounds[i].mode] += static_cast<uint64_t>(static_cast<int64_t>(bounds[i].delta));
      if (i == bounds.size()) break;
      const uint64_t hi = bounds[i].at;
      const int kinds = (active[0] != 0) + (active[1] != 0) + (active[2] != 0);
      if (kinds == 0) continue;
      uint32_t mode = XVRAM_ACCESS_READ_WRITE;
      if (kinds == 1) mode = active[0] ? XVRAM_ACCESS_READ : (active[1] ? XVRAM_ACCESS_READ_WRITE
                                                                          : XVRAM_ACCESS_WRITE_ONLY);
      AccessSpan* last = normalized.empty() ? nullptr : &normalized.back();
      if (last && last->allocation_id == id && last->offset + last->length == lo &&
          last->mode == mode) {
        last->length += hi - lo;
      } else {
        normalized.push_back(AccessSpan{id, lo, hi - lo, mode});
      }
    }
  }
  for (const AccessSpan& s : normalized) {
    const uint64_t bytes = sizes[s.allocation_id];
    const uint64_t first = s.offset / chunk_bytes, last = (s.offset + s.length - 1) / chunk_bytes;
    for (uint64_t c = first; c <= last; ++c) {
      const uint64_t c_lo = c * chunk_bytes;
      const uint64_t c_hi = std::min(bytes, c_lo + chunk_bytes);
      const uint64_t lo = std::max(s.offset, c_lo), hi = std::min(s.offset + s.length, c_hi);
      const bool full_write_only = s.mode == XVRAM_ACCESS_WRITE_ONLY && lo == c_lo && hi == c_hi;
      if (chunks.empty() || chunks.back().allocation_id != s.allocation_id ||
          chunks.back().index != c) {
        chunks.push_back(ChunkPlan{s.allocation_id, c, c_hi - c_lo, !full_write_only,
                                   s.mode != XVRAM_ACCESS_READ});
      } else {
        // A second span in the chunk: it is no longer one full write-only span.
        chunks.back().requires_h2d = true;
        chunks.back().marks_dirty = chunks.back().marks_dirty || s.mode != XVRAM_ACCESS_READ;
      }
    }
  }
  return nullptr;
}

Error Runtime::plan_chunks(const std::vector<AccessSpan>& ranges, std::vector<ChunkUse>& chunks,
                           std::vector<AccessSpan>& normalized, const char* operation) {
  chunks.clear();
  std::vector<AllocationExtent> extents;
  extents.reserve(allocations_.size());
  for (const auto& [id, a] : allocations_) extents.push_back(AllocationExtent{id, a.bytes});
  std::vector<ChunkPlan> plans;
  const char* problem = ranges.empty()
                            ? "zero_length"
                            : normalize_accesses(extents, ranges, frame_bytes_, normalized, plans);
  if (problem)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "transaction", operation,
                      std::string("invalid access ranges: ") + problem);
  chunks.reserve(plans.size());
  for (const ChunkPlan& p : plans) {
    ChunkUse u;
    u.allocation_id = p.allocation_id;
    u.index = p.index;
    u.needs_data = p.requires_h2d;
    u.writes = p.marks_dirty;
    chunks.push_back(u);
  }
  return {};
}

Error Runtime::acquire_chunk(ChunkUse& use) {
  HostAllocation* a = find(use.allocation_id);
  if (!a) return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "transaction", "acquire", "unknown allocation");
  if (Error e = reserve_allocation_va(*a)) return e;
  PanelKey key;
  key.allocation_id = use.allocation_id;
  key.offset = use.index * frame_bytes_;
  key.width = std::min(frame_bytes_, a->bytes - key.offset);
  key.height = 1;
  key.pitch = key.width;
  key.kind = EntryKind::chunk;
  auto it = index_.find(key);
  if (it != index_.end()) {
    Frame& f = frames_[it->second];
    ++f.pins;
    f.last_use = ++tick_;
    ++t_.cache_hits;
    if (!prefetching_)
      policy_->touch(f.index, ++policy_sequence_, allocation_streaming(key.allocation_id));
    use.frame = &f;
    return {};
  }
  if (Error e = flush_overlapping(key, nullptr)) return e;
  if (use.needs_data)
    if (Error e = check_not_lost(key, "transaction", "fill")) return e;
  const uint64_t address = a->va + key.offset;
  Frame* f = nullptr;
  for (uint64_t i = 0; i < capacity_; ++i) {
    Frame& g = frames_[i];
    // The frame that last held this chunk may still be mapped at its address.
    if (g.mapped_at == address && !g.keyed && g.pins == 0) {
      if (Error e = wait_retired(g)) return e;
      move(g, EntryState::mapping);
      ++t_.handle_reuses;
      f = &g;
      break;
    }
  }
  if (!f)
    if (Error e = select_frame(f)) return e;
  if (Error e = map_frame_at(*f, address)) return abandon_mapping(*f, e);
  use.frame = f;
  use.filled_empty = !use.needs_data;
  return fill_entry(*f, key, key.width, use.needs_data);
}

// A working-set transaction (reference Runtime::execute/acquire_external/
// seal/poll, runtime.cpp:1012-1495): make every touched chunk resident at its
// stable address, run the caller's work on the compute stream, write back what
// it wrote, and measure the work's GPU time against the duration guard.
Error Runtime::run_transaction(const std::vector<AccessSpan>& ranges, uint64_t workspace_bytes,
                               const TransactionBody& body, uint64_t operation_id) {
  if (Error e = begin_operation()) return e;
  std::vector<ChunkUse> chunks;
  std::vector<AccessSpan> normalized;
  Error result = plan_chunks(ranges, chunks, normalized, "normalize_accesses");
  if (!result) result = refresh_budget(chunks.size(), workspace_bytes, false);
  if (!result && chunks.size() > capacity_)
    result = make_error(XVRAM_STATUS_BUDGET_PRESSURE, "transaction", "working_set",
                        "declared working set exceeds the cache target");
  if (!result) result = ensure_workspace(workspace_bytes);
  if (!result) result = make_room(chunks.size());
  for (size_t i = 0; !result && i < chunks.size(); ++i)
    if (Error e = acquire_chunk(chunks[i])) result = e;
  // Leaves the cache as if the callback had never run: unpins, drops every
  // chunk that was mapped without its data and, when work may have been
  // enqueued, every chunk that work may have written (its earlier contents,
  // dirty or not, are gone either way).
  const auto abandon = [&](bool work_enqueued) {
    for (ChunkUse& u : chunks) {
      if (!u.frame) continue;
      if (u.frame->pins > 0) --u.frame->pins;
      if ((work_enqueued && u.writes) || u.filled_empty) {
        u.frame->dirty = false;
        (void)evict_key(*u.frame, false);
      }
    }
  };
  if (result) {
    abandon(false);
    (void)finish_operation(operation_id);
    return result;
  }
  for (ChunkUse& u : chunks)
    if (Error e = wait_ready(*u.frame, compute_)) return e;
  std::vector<ResolvedSpan> resolved;
  resolved.reserve(normalized.size());
  for (const AccessSpan& s : normalized)
    resolved.push_back(ResolvedSpan{s, find(s.allocation_id)->va + s.offset});
  TraceInterval iv;
  iv.kind = 't';
  if (Error e = take_event(iv.start)) return e;
  if (Error e = take_event(iv.stop)) return e;
  if (int rc = device_->event_record(iv.start, compute_)) return device_failure(rc, "transaction", "record");
  bool skipped = false;
  Error body_error;
  try {
    body_error = body(resolved, workspace_bytes ? workspace_va_ : 0, workspace_bytes, compute_, skipped);
  } catch (...) {
    body_error = exception_error("transaction_callback");
    body_error.status = XVRAM_STATUS_CALLBACK_FAILED;
  }
  if (int rc = device_->event_record(iv.stop, compute_)) return device_failure(rc, "transaction", "record");
  if (body_error) {
    // A skipped callback enqueued nothing; a failed one may have enqueued work
    // (the reference's failed_after_possible_submission), which poisons the
    // session once the streams have drained.
    abandon(!skipped);
    (void)finish_operation(operation_id);
    if (!skipped) {
      poisoned_ = true;
      t_.poisoned = 1;
    }
    return body_error;
  }
  trace_.push_back(iv);
  // Written chunks stay resident and dirty (write-back cache).
  for (ChunkUse& u : chunks)
    if (Error e = release_after(*u.frame, compute_, u.writes)) return e;
  ++transactions_in_operation_;
  return finish_operation(operation_id);
}

Error Runtime::run_prefetch(const std::vector<AccessSpan>& ranges, uint64_t operation_id) {
  if (Error e = begin_operation()) return e;
  std::vector<ChunkUse> chunks;
  std::vector<AccessSpan> normalized;
  Error result = plan_chunks(ranges, chunks, normalized, "prefetch");
  if (!result) result = refresh_budget(chunks.size(), 0, false);
  if (!result && chunks.size() > capacity_)
    result = make_error(XVRAM_STATUS_BUDGET_PRESSURE, "transaction", "prefetch",
                        "prefetch working set exceeds the cache target");
  if (!result) result = make_room(chunks.size());
  prefetching_ = true; // fills are speculative until a transaction uses them
  for (size_t i = 0; !result && i < chunks.size(); ++i) {
    chunks[i].needs_data = true; // a prefetched chunk must hold valid data
    if (Error e = acquire_chunk(chunks[i])) result = e;
    else result = release_after(*chunks[i].frame, h2d_, false);
  }
  prefetching_ = false;
  Error finish = finish_operation(operation_id);
  return result ? result : finish;
}

// ---- live budget -------------------------------------------------------------------

// Gives a frame's physical memory back: its entry is written back (dirty) or
// dropped, its mapping removed and its handle released.
Error Runtime::release_frame(Frame& f) {
  if (f.keyed) {
    if (f.dirty) {
      if (Error e = writeback_and_evict(f)) return e;
    } else {
      if (Error e = evict_key(f, false)) return e;
      ++t_.clean_evictions;
    }
  }
  if (Error e = unmap_frame(f)) return e; // waits for the frame's last consumer
  if (f.handle) {
    if (int rc = device_->mem_release(f.handle)) return device_failure(rc, "budget", "mem_release");
    f.handle = 0;
    ++t_.physical_handles_released;
  }
  if (f.state == EntryState::evicting) move(f, EntryState::host_clean);
  f.used_before = false;
  return {};
}

Error Runtime::refresh_budget(uint64_t required_frames, uint64_t required_workspace, bool force) {
  const Clock::time_point now = Clock::now();
  if (!force && config_.budget_poll_ms > 0 &&
      now - last_budget_sample_ < std::chrono::milliseconds(config_.budget_poll_ms))
    return {};
  last_budget_sample_ = now;
  uint64_t free_bytes = 0, total_bytes = 0;
  if (int rc = device_->mem_info(&free_bytes, &total_bytes))
    return device_failure(rc, "budget", "mem_info");
  ++t_.budget_sample_count;
  t_.cuda_free_bytes_end = free_bytes;
  t_.cuda_free_bytes_minimum = std::min(t_.cuda_free_bytes_minimum, free_bytes);

  // Memory this session could hand back counts as available to it.
  uint64_t created = 0;
  for (const Frame& f : frames_)
    if (f.handle) ++created;
  const uint64_t managed = created * frame_bytes_ + workspace_bytes_;
  const uint64_t reclaimable =
      free_bytes > UINT64_MAX - managed ? UINT64_MAX : free_bytes + managed;
  const uint64_t after_headroom = reclaimable > config_.device_headroom_bytes
                                      ? reclaimable - config_.device_headroom_bytes
                                      : 0;
  uint64_t target = std::min(configured_cap_, after_headroom);
  target -= target % frame_bytes_;
  const uint64_t reserve = config_.workspace_reserve_bytes;
  uint64_t frames = target > reserve ? (target - reserve) / frame_bytes_ : 0;
  frames = std::min(frames, max_capacity_);

  if (frames < capacity_) {
    // Shrink now: every tail frame must be idle (checked before anything changes).
    for (uint64_t i = frames; i < capacity_; ++i)
      if (frames_[i].pins > 0)
        return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "budget", "shrink_preflight",
                          "an active working-set frame defers the live target shrink");
    for (uint64_t i = frames; i < capacity_; ++i)
      if (Error e = release_frame(frames_[i])) return e;
    capacity_ = frames;
    target_bytes_ = target;
    t_.cache_target_bytes = target;
    t_.cache_target_minimum_bytes = std::min(t_.cache_target_minimum_bytes, target);
    ++t_.budget_shrinks;
    growth_samples_ = 0;
  }
  if (t_.resident_bytes + workspace_bytes_ > target)
    return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "budget", "managed_device_accounting",
                      "managed residency and workspace exceed the live safe device target");
  uint64_t required = 0;
  if (!checked_mul(required_frames, frame_bytes_, required) ||
      !checked_add(required, required_workspace, required) || target < required ||
      target <= reserve || frames < required_frames)
    return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "budget", "working_set",
                      "live device budget fell below the next working set");
  if (frames > capacity_) {
    // Grow slowly: two frames after ten consecutive samples with room for them.
    if (++growth_samples_ >= 10 && frames >= capacity_ + 2) {
      capacity_ = std::min(frames, capacity_ + 2);
      target_bytes_ = std::min(target, capacity_ * frame_bytes_ + reserve);
      t_.cache_target_bytes = target_bytes_;
      t_.cache_target_maximum_bytes = std::max(t_.cache_target_maximum_bytes, target_bytes_);
      ++t_.budget_grows;
      growth_samples_ = 0;
    }
  } else {
    growth_samples_ = 0;
  }
  return {};
}

// ---- operation bracketing ------------------------------------------------------

Error Runtime::begin_operation() {
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "operation", "begin", "session is poisoned");
  if (launches_blocked_)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "operation", "begin",
                      "runtime is not ready: launches are blocked after device work exceeded "
                      "the transaction duration guard");
  kernels_in_operation_ = 0;
  transactions_in_operation_ = 0;
  in_operation_ = true;
  // Entries the previous operation carried over become ordinary clean
  // entries: a consumer still waits for the fill (ready event) and a reuse of
  // the frame still waits for the copy (retire event), so the policy may pick
  // them as victims like any other (the operation they were carried for may
  // have been cancelled, or need the frames for something else).
  for (Frame& f : frames_)
    if (f.carry_serial != 0 && f.keyed && f.state == EntryState::h2d_in_flight)
      move(f, EntryState::resident_clean);
  ++op_serial_;
  carry_active_ = false;
  // Fills the previous operation carried over belong to this one's trace.
  trace_ = std::move(carried_trace_);
  carried_trace_.clear();
  events_in_use_.insert(events_in_use_.end(), carried_events_.begin(), carried_events_.end());
  carried_events_.clear();
  op_host_start_ = std::chrono::steady_clock::now();
  trace_timed_ = 0;
  op_start_seen_ = false;
  guard_tripped_ = false;
  // Every stream is idle here (the previous operation drained them; carried
  // fills aside), so nothing orders the copy streams after op_start_: a wait
  // on a just-recorded event costs ~16 us of host time. Intervals are timed
  // from op_start_ (a carried fill or a copy issued before op_start_ was
  // processed times as negative). Each compute lane records its own start.
  if (int rc = device_->event_record(op_start_, compute_)) return device_failure(rc, "operation", "record");
  lane_dispatched_at_[0] = Clock::now();
  if (int rc = device_->event_record(op_start2_, compute2_)) return device_failure(rc, "operation", "record");
  lane_dispatched_at_[1] = Clock::now();
  lane_last_[0] = op_start_;
  lane_last_[1] = op_start2_;
  lane_waited_[0] = lane_waited_[1] = false;
  lane_deps_[0].clear();
  lane_deps_[1].clear();
  return {};
}

Error Runtime::record_kernel(TraceInterval& iv, int lane) {
  if (lane < 0 || lane >= kLanes)
    return make_error(XVRAM_STATUS_INTERNAL, "gemm", "launch", "no such compute lane");
  iv.start = iv.start_ref = nullptr;
  iv.deps.clear();
  const Clock::time_point now = Clock::now();
  const bool host_gap = now - lane_dispatched_at_[lane] > kStartEventAfterHostGap;
  lane_dispatched_at_[lane] = now;
  if (lane_waited_[lane] || host_gap) {
    if (Error e = take_event(iv.start)) return e;
  } else {
    iv.start_ref = lane_last_[lane];
    iv.deps.swap(lane_deps_[lane]);
  }
  if (Error e = take_event(iv.stop)) return e;
  lane_last_[lane] = iv.stop;
  lane_waited_[lane] = false;
  lane_deps_[lane].clear();
  return {};
}

Error Runtime::stream_wait(Stream stream, Event event, Event stamp) {
  if (int rc = device_->stream_wait_event(stream, event))
    return device_failure(rc, "cache", "stream_wait");
  for (int lane = 0; lane < kLanes; ++lane) {
    if (stream != compute_stream(lane)) continue;
    if (stamp) lane_deps_[lane].push_back(stamp);
    else lane_waited_[lane] = true;
  }
  return {};
}

void Runtime::time_intervals(bool all) {
  if (!in_operation_ && !all) return;
  // Fills carried into the next operation are timed by that one.
  const size_t own = carry_active_ ? carry_trace_mark_ : trace_.size();
  if (!op_start_seen_) {
    if (!all && (device_->event_query(op_start_) != 0 || device_->event_query(op_start2_) != 0))
      return;
    op_start_seen_ = true;
  }
  while (trace_timed_ < own) {
    TraceInterval& iv = trace_[trace_timed_];
    if (!all && device_->event_query(iv.stop) != 0) return;
    // A kernel without a start event started when the last of its start_ref
    // (an earlier event on the same stream) and its deps (events its stream
    // waited for) completed; all of them completed before its stop did.
    const Event start = iv.start ? iv.start : iv.start_ref;
    float s = 0.f, e = 0.f;
    if (start != op_start_ && device_->event_elapsed_ms(&s, op_start_, start) != 0) s = 0.f;
    for (Event d : iv.deps) {
      float t = 0.f;
      if (device_->event_elapsed_ms(&t, op_start_, d) == 0) s = std::max(s, t);
    }
    if (device_->event_elapsed_ms(&e, op_start_, iv.stop) != 0) e = s;
    iv.start_ms = s;
    iv.stop_ms = e;
    iv.timed = true;
    if (iv.kind == 'k' || iv.kind == 't') {
      const float d = e - s;
      t_.last_transaction_ms = d;
      if (config_.max_transaction_ms > 0 &&
          static_cast<double>(d) > static_cast<double>(config_.max_transaction_ms))
        guard_tripped_ = true;
    }
    ++trace_timed_;
  }
}

// End of an operation: wait for the three streams, fold the kernel, callback
// and copy intervals into telemetry (and the optional trace file), and apply
// the duration guard (reference runtime.cpp:1396-1408: work longer than
// max_transaction_ms blocks further launches and fails with a timeout).
Error Runtime::finish_operation(uint64_t operation_id) {
  const auto host_ms = [&]() {
    return std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() -
                                                     op_host_start_)
        .count();
  };
  const double enqueued_ms = host_ms(); // everything is enqueued: the host waits from here
  Error first;
  if (Error e = await_streams({compute_, compute2_, d2h_}, "operation", "stream_wait"); e)
    first = e;
  // This operation's own fills end at the carry fence; carried fills run on.
  if (Error e = carry_active_ ? await_event(carry_fence_, "operation", "fill_wait")
                              : await_stream(h2d_, "operation", "stream_wait");
      e && !first)
    first = e;
  const bool carrying = carry_active_ && !first;
  for (Frame& f : frames_) {
    if (carrying && f.carry_serial == op_serial_) continue; // still filling for the next one
    f.carry_serial = 0;
    f.ready_pending = false;
    if (first) continue;
    // Every stream has drained: all fills landed and every retire event of
    // this operation has completed (the host has now observed it: an event
    // boundary for each frame that still had one outstanding).
    if (f.retire_pending) ++t_.event_boundaries;
    f.retire_pending = false;
    f.lane_pending[0] = f.lane_pending[1] = false;
    f.completed = f.generation;
    if (f.state == EntryState::h2d_in_flight) move(f, EntryState::resident_clean);
    if (f.state == EntryState::evicting) move(f, EntryState::host_clean);
  }
  const double synced_ms = host_ms();
  // The D2H stream has drained (or the session is poisoned); the copies' stop
  // events go back to the pool below, so nothing may refer to them.
  writebacks_settled();
  in_operation_ = false;
  protected_.clear();
  if (!first) {
    time_intervals(true);
    if (tracing()) {
      // One record per operation: kernel and copy intervals in ms from its
      // start event, then the host timestamps (ms from begin_operation) of the
      // last enqueue and of the device drained.
      const size_t own = carrying ? carry_trace_mark_ : trace_.size();
      std::string line;
      line.reserve(64 + own * 40);
      char buf[96];
      std::snprintf(buf, sizeof buf, "{\"operation_id\": %llu, \"host\": [%.3f, %.3f]",
                    static_cast<unsigned long long>(operation_id), enqueued_ms, synced_ms);
      line += buf;
      const char* names[4] = {"kernels", "h2d", "d2h", "transactions"};
      const char kinds[4] = {'k', 'h', 'd', 't'};
      for (int c = 0; c < 4; ++c) {
        line += ", \"";
        line += names[c];
        line += "\": [";
        bool comma = false;
        for (size_t i = 0; i < own; ++i) {
          const TraceInterval& iv = trace_[i];
          if (iv.kind != kinds[c]) continue;
          std::snprintf(buf, sizeof buf, "%s[%.6f, %.6f, %llu]", comma ? ", " : "", iv.start_ms,
                        iv.stop_ms, static_cast<unsigned long long>(iv.bytes));
          line += buf;
          comma = true;
        }
        line += "]";
      }
      line += "}\n";
      if (FILE* out = std::fopen(trace_path_.c_str(), "a")) {
        std::fwrite(line.data(), 1, line.size(), out);
        std::fclose(out);
      }
    }
    t_.transactions_completed += kernels_in_operation_ + transactions_in_operation_;
    t_.algorithm_selections += kernels_in_operation_;
  }
  // Carried fills are traced with the next operation; their events stay live.
  carried_trace_.clear();
  carried_events_.clear();
  size_t own_events = events_in_use_.size();
  if (carrying) {
    carried_trace_.assign(trace_.begin() + static_cast<std::ptrdiff_t>(carry_trace_mark_),
                          trace_.end());
    carried_events_.assign(events_in_use_.begin() + static_cast<std::ptrdiff_t>(carry_event_mark_),
                           events_in_use_.end());
    own_events = carry_event_mark_;
  }
  carry_active_ = false;
  trace_.clear();
  kernels_in_operation_ = 0;
  transactions_in_operation_ = 0;
  for (size_t i = 0; i < events_in_use_.size(); ++i) {
    // After a failure carried events are returned too: nothing reads them again.
    if (i < own_events || !carrying) event_pool_.push_back(events_in_use_[i]);
  }
  events_in_use_.clear();
  // Free device memory is sampled at setup and by refresh_budget (at most once
  // per budget_poll_ms; reference src/residency/runtime.cpp:3213-3232), not
  // per operation.
  if (!first && guard_tripped_) {
    launches_blocked_ = true;
    ++t_.watchdog_rejections;
    return make_error(XVRAM_STATUS_TIMEOUT, "transaction", "duration_guard",
                      "device work exceeded the configured transaction duration");
  }
  return first;
}

void Runtime::telemetry(xvram_session_telemetry_v1& out) const {
  out = t_;
  out.struct_size = sizeof(out);
  out.pinned_staging_bytes = pinned_bytes_;
  out.poisoned = poisoned_ ? 1u : 0u;
}

} // namespace xvram
