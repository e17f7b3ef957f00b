// runtime.cpp — host backing, VRAM frame pool and panel cache (see runtime.hpp).
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

// Session setup (reference src/residency/runtime.cpp:212-596): bind the
// device, align the frame size to the VMM granularity, derive the budget from
// hipMemGetInfo, reserve the frame arena and create the three streams.
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
    frames_[i].address = arena_ + i * frame_bytes_;
  }
  if (int rc = device_->stream_create(&compute_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->stream_create(&h2d_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->stream_create(&d2h_)) return device_failure(rc, "setup", "stream");
  if (int rc = device_->event_create(&op_start_)) return device_failure(rc, "setup", "event");
  t_.flags = XVRAM_TELEMETRY_NO_PHYSICAL_ALIASES;
  setup_done_ = true;
  return {};
}

Error Runtime::drain() {
  if (!setup_done_ || closed_) return {};
  for (Stream s : {h2d_, compute_, d2h_})
    if (int rc = device_->stream_sync(s)) return device_failure(rc, "drain", "stream_sync");
  return {};
}

// Teardown (reference runtime.cpp:1540-1857): wait for the device, unmap and
// release every frame, free the arena, streams, events and host backing.
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
  for (Stream s : {h2d_, compute_, d2h_})
    if (s) note(device_->stream_sync(s), "stream_sync");
  for (Frame& f : frames_) {
    if (f.keyed) evict_key(f, false);
    if (f.mapped) {
      note(device_->mem_unmap(f.address, frame_bytes_), "unmap");
      ++t_.unmaps;
      f.mapped = false;
    }
    if (f.handle) {
      note(device_->mem_release(f.handle), "release");
      ++t_.physical_handles_released;
      f.handle = 0;
    }
    if (f.ready) device_->event_destroy(f.ready);
    if (f.retire) device_->event_destroy(f.retire);
    f.ready = f.retire = nullptr;
  }
  if (arena_) note(device_->va_free(arena_, arena_bytes_), "va_free");
  arena_ = 0;
  for (Event e : event_pool_) device_->event_destroy(e);
  for (Event e : events_in_use_) device_->event_destroy(e);
  for (auto& [key, e] : pending_writebacks_) (void)key, (void)e;
  event_pool_.clear();
  events_in_use_.clear();
  pending_writebacks_.clear();
  if (op_start_) device_->event_destroy(op_start_);
  for (Stream s : {h2d_, compute_, d2h_})
    if (s) device_->stream_destroy(s);
  compute_ = h2d_ = d2h_ = nullptr;
  for (auto& [id, a] : allocations_) device_->host_free(a.host);
  allocations_.clear();
  t_.resident_bytes = 0;
  return first;
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
  device_->host_free(a->host);
  pinned_bytes_ -= a->bytes;
  allocations_.erase(id);
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
  // Cached panels overlapping the range become stale: drop them first.
  if (Error e = invalidate(id, offset, end)) return e;
  parallel_copy(a->host + offset, source, bytes);
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
  // Operations write their dirty panels back before completing, so the host
  // copy is authoritative here.
  parallel_copy(destination, a->host + offset, bytes);
  return {};
}

// ---- frame pool --------------------------------------------------------------

Error Runtime::ensure_frame_mapped(Frame& f) {
  if (f.mapped) return {};
  if (!f.handle) {
    uint64_t handle = 0;
    if (int rc = device_->mem_create(frame_bytes_, &handle)) {
      if (rc == 2)
        return make_error(XVRAM_STATUS_DEVICE_OUT_OF_MEMORY, "cache", "mem_create",
                          "physical frame allocation failed");
      return device_failure(rc, "cache", "mem_create");
    }
    f.handle = handle;
    ++t_.physical_handles_created;
  }
  if (int rc = device_->mem_map(f.address, frame_bytes_, f.handle))
    return device_failure(rc, "cache", "mem_map");
  f.mapped = true;
  ++t_.mappings;
  if (int rc = device_->set_access(f.address, frame_bytes_))
    return device_failure(rc, "cache", "set_access");
  ++t_.set_access_calls;
  if (!f.ready)
    if (int rc = device_->event_create(&f.ready)) return device_failure(rc, "cache", "event");
  if (!f.retire)
    if (int rc = device_->event_create(&f.retire)) return device_failure(rc, "cache", "event");
  return {};
}

// A frame is handed out for a new panel only after its last consumer's event
// has retired; the host checks (and if necessary waits for) that event.
Error Runtime::wait_retired(Frame& f) {
  if (!f.retire_pending) return {};
  ++t_.event_boundaries;
  const int q = device_->event_query(f.retire);
  if (q == 1) {
    if (int rc = device_->event_sync(f.retire)) return device_failure(rc, "cache", "event_sync");
  } else if (q != 0) {
    return device_failure(q, "cache", "event_query");
  }
  f.retire_pending = false;
  return {};
}

void Runtime::evict_key(Frame& f, bool was_dirty) {
  if (!f.keyed) return;
  index_.erase(f.key);
  f.keyed = false;
  f.dirty = false;
  f.ready_pending = false;
  t_.resident_bytes -= frame_bytes_;
  if (was_dirty) ++t_.dirty_evictions;
}

// Frame choice (reference acquire_frame, runtime.cpp:3470-3529): the free
// frame idle longest, else a not-yet-created frame, else the least-recently-
// used unpinned panel — clean panels before dirty ones (a dirty victim is
// written back first). The choice depends only on the schedule, never on how
// far the device has progressed, so the accounting of a run is reproducible
// (the host-simulation build produces the same counters).
Error Runtime::select_frame(Frame*& out) {
  Frame* free_frame = nullptr;
  Frame* unmapped = nullptr;
  Frame* victim = nullptr;
  for (Frame& f : frames_) {
    if (!f.mapped) {
      if (!unmapped) unmapped = &f;
      continue;
    }
    if (f.pins > 0) continue;
    if (!f.keyed) {
      if (!free_frame || f.last_use < free_frame->last_use) free_frame = &f;
      continue;
    }
    if (!victim) {
      victim = &f;
    } else {
      const bool better = (victim->dirty && !f.dirty) ||
                          (victim->dirty == f.dirty && f.last_use < victim->last_use);
      if (better) victim = &f;
    }
  }
  Frame* chosen = free_frame;
  if (!chosen && unmapped) {
    if (Error e = ensure_frame_mapped(*unmapped)) {
      if (e.status != XVRAM_STATUS_DEVICE_OUT_OF_MEMORY) return e;
    } else {
      chosen = unmapped;
    }
  }
  if (!chosen && victim) {
    if (victim->dirty) {
      if (Error e = writeback_and_evict(*victim)) return e;
    } else {
      evict_key(*victim, false);
      ++t_.clean_evictions;
    }
    chosen = victim;
  }
  if (!chosen)
    return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "cache", "select_frame",
                      "every cache frame is pinned by the current working set");
  if (Error e = wait_retired(*chosen)) return e;
  if (chosen->used_before) ++t_.handle_reuses;
  chosen->used_before = true;
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
      out = &f;
      return {};
    }
    // Same rectangle cached with another packing: drop it.
    if (f.pins > 0)
      return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "conflicting pinned packing");
    if (f.dirty) {
      if (Error e = writeback_and_evict(f)) return e;
    } else {
      evict_key(f, false);
      ++t_.clean_evictions;
    }
  }
  Frame* f = nullptr;
  if (Error e = select_frame(f)) return e;
  ++t_.cache_misses;
  f->keyed = true;
  f->key = key;
  f->packed_pitch = packed_pitch;
  f->pins = 1;
  f->dirty = false;
  f->last_use = ++tick_;
  index_[key] = f->index;
  t_.resident_bytes += frame_bytes_;
  t_.resident_bytes_peak = std::max(t_.resident_bytes_peak, t_.resident_bytes);
  if (auto wb = pending_writebacks_.find(key); wb != pending_writebacks_.end()) {
    // The host copy of this rectangle is still being written back.
    if (int rc = device_->stream_wait_event(h2d_, wb->second))
      return device_failure(rc, "cache", "stream_wait");
  }
  if (needs_data) {
    HostAllocation* a = find(key.allocation_id);
    if (!a || key.end() > a->bytes)
      return make_error(XVRAM_STATUS_INTERNAL, "cache", "acquire", "panel outside its allocation");
    TraceInterval iv;
    iv.kind = 'h';
    iv.bytes = key.bytes();
    if (Error e = take_event(iv.start)) return e;
    if (int rc = device_->event_record(iv.start, h2d_)) return device_failure(rc, "cache", "record");
    if (int rc = device_->copy_h2d_2d(f->address, packed_pitch, a->host + key.offset, key.pitch,
                                      key.width, key.height, h2d_))
      return device_failure(rc, "cache", "copy_h2d");
    if (Error e = take_event(iv.stop)) return e;
    if (int rc = device_->event_record(iv.stop, h2d_)) return device_failure(rc, "cache", "record");
    trace_.push_back(iv);
    if (int rc = device_->event_record(f->ready, h2d_)) return device_failure(rc, "cache", "record");
    f->ready_pending = true;
    t_.bytes_h2d += key.bytes();
  }
  out = f;
  return {};
}

Error Runtime::wait_ready(Frame& f, Stream stream) {
  if (!f.ready_pending) return {};
  if (int rc = device_->stream_wait_event(stream, f.ready))
    return device_failure(rc, "cache", "stream_wait");
  return {};
}

Error Runtime::release_after(Frame& f, Stream stream, bool dirty) {
  if (f.pins <= 0) return make_error(XVRAM_STATUS_INTERNAL, "cache", "release", "frame is not pinned");
  if (int rc = device_->event_record(f.retire, stream)) return device_failure(rc, "cache", "record");
  f.retire_pending = true;
  --f.pins;
  f.dirty = f.dirty || dirty;
  f.last_use = ++tick_;
  return {};
}

// Dirty write-back (reference writeback, runtime.cpp:3899-4262): the D2H copy
// is ordered after the frame's last kernel and becomes the frame's retire
// event, so the frame is refilled only after the host rectangle is current.
Error Runtime::writeback_and_evict(Frame& f) {
  if (!f.keyed || !f.dirty || f.pins > 0)
    return make_error(XVRAM_STATUS_INTERNAL, "cache", "writeback", "frame is not an idle dirty panel");
  HostAllocation* a = find(f.key.allocation_id);
  if (!a) return make_error(XVRAM_STATUS_INTERNAL, "cache", "writeback", "panel owner is gone");
  if (f.retire_pending)
    if (int rc = device_->stream_wait_event(d2h_, f.retire))
      return device_failure(rc, "cache", "stream_wait");
  TraceInterval iv;
  iv.kind = 'd';
  iv.bytes = f.key.bytes();
  if (Error e = take_event(iv.start)) return e;
  if (int rc = device_->event_record(iv.start, d2h_)) return device_failure(rc, "cache", "record");
  if (int rc = device_->copy_d2h_2d(a->host + f.key.offset, f.key.pitch, f.address, f.packed_pitch,
                                    f.key.width, f.key.height, d2h_))
    return device_failure(rc, "cache", "copy_d2h");
  if (Error e = take_event(iv.stop)) return e;
  if (int rc = device_->event_record(iv.stop, d2h_)) return device_failure(rc, "cache", "record");
  trace_.push_back(iv);
  if (int rc = device_->event_record(f.retire, d2h_)) return device_failure(rc, "cache", "record");
  f.retire_pending = true;
  pending_writebacks_[f.key] = iv.stop;
  t_.bytes_d2h += f.key.bytes();
  ++t_.writebacks_completed;
  evict_key(f, true);
  return {};
}

Error Runtime::invalidate(uint64_t allocation_id, uint64_t begin, uint64_t end) {
  for (Frame& f : frames_) {
    if (!f.keyed || f.key.allocation_id != allocation_id) continue;
    if (f.key.offset >= end || f.key.end() <= begin) continue;
    if (f.pins > 0)
      return make_error(XVRAM_STATUS_BUSY, "cache", "invalidate", "panel is in use by an operation");
    if (f.dirty) {
      if (Error e = writeback_and_evict(f)) return e;
      for (Stream s : {d2h_})
        if (int rc = device_->stream_sync(s)) return device_failure(rc, "cache", "stream_sync");
    } else {
      if (Error e = wait_retired(f)) return e;
      evict_key(f, false);
      ++t_.clean_evictions;
    }
  }
  return {};
}

void Runtime::discard_dirty() {
  for (Frame& f : frames_) {
    if (f.keyed && f.dirty) {
      f.pins = 0;
      evict_key(f, false);
    }
    f.pins = 0;
  }
}

Error Runtime::begin_operation() {
  if (poisoned_) return make_error(XVRAM_STATUS_POISONED, "operation", "begin", "session is poisoned");
  kernels_in_operation_ = 0;
  trace_.clear();
  if (int rc = device_->event_record(op_start_, compute_)) return device_failure(rc, "operation", "record");
  for (Stream s : {h2d_, d2h_})
    if (int rc = device_->stream_wait_event(s, op_start_)) return device_failure(rc, "operation", "wait");
  return {};
}

Error Runtime::record_kernel(Event& start, Event& stop) {
  if (Error e = take_event(start)) return e;
  return take_event(stop);
}

// End of an operation: wait for the three streams, then fold the kernel and
// copy intervals into telemetry (and the optional trace file).
Error Runtime::finish_operation(uint64_t operation_id) {
  Error first;
  for (Stream s : {h2d_, compute_, d2h_}) {
    if (int rc = device_->stream_sync(s)) {
      if (!first) first = device_failure(rc, "operation", "stream_sync");
    }
  }
  for (Frame& f : frames_) {
    f.ready_pending = false;
    if (!first) f.retire_pending = false;
  }
  pending_writebacks_.clear();
  if (!first) {
    FILE* out = nullptr;
    if (tracing()) out = std::fopen(trace_path_.c_str(), "a");
    if (out) std::fprintf(out, "{\"operation_id\": %llu", static_cast<unsigned long long>(operation_id));
    const char* names[3] = {"kernels", "h2d", "d2h"};
    const char kinds[3] = {'k', 'h', 'd'};
    for (int c = 0; c < 3; ++c) {
      if (out) std::fprintf(out, ", \"%s\": [", names[c]);
      bool comma = false;
      for (const TraceInterval& iv : trace_) {
        if (iv.kind != kinds[c]) continue;
        float s = 0.f, e = 0.f;
        if (device_->event_elapsed_ms(&s, op_start_, iv.start) != 0) s = 0.f;
        if (device_->event_elapsed_ms(&e, op_start_, iv.stop) != 0) e = s;
        if (iv.kind == 'k') {
          float d = 0.f;
          if (device_->event_elapsed_ms(&d, iv.start, iv.stop) == 0) t_.last_transaction_ms = d;
        }
        if (out) {
          std::fprintf(out, "%s[%.6f, %.6f, %llu]", comma ? ", " : "", s, e,
                       static_cast<unsigned long long>(iv.bytes));
          comma = true;
        }
      }
      if (out) std::fprintf(out, "]");
    }
    if (out) {
      std::fprintf(out, "}\n");
      std::fclose(out);
    }
    t_.transactions_completed += kernels_in_operation_;
    t_.algorithm_selections += kernels_in_operation_;
  }
  trace_.clear();
  kernels_in_operation_ = 0;
  for (Event e : events_in_use_) event_pool_.push_back(e);
  events_in_use_.clear();
  uint64_t free_bytes = 0, total_bytes = 0;
  if (!first && device_->mem_info(&free_bytes, &total_bytes) == 0) {
    ++t_.budget_sample_count;
    t_.cuda_free_bytes_minimum = std::min(t_.cuda_free_bytes_minimum, free_bytes);
    t_.cuda_free_bytes_end = free_bytes;
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
