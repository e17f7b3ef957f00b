// runtime.hpp — host backing, the VRAM frame pool and the panel cache.
//
// Reference counterpart: residency::Runtime (src/residency/runtime.hpp:317-372,
// runtime.cpp:212-596 setup, :3470-3529 acquire_frame, :3531-3897
// ensure_resident, :3899-4262 writeback, :1540-1857 close). The reference
// caches 64 MiB linear chunks of each allocation; a column panel with a large
// leading dimension touches every chunk. This runtime caches *panels*: the
// unit of residency is one packed 2-D sub-matrix (a strided rectangle of an
// allocation), copied with one hipMemcpy2DAsync into one frame.
//
// Frames: `capacity` physical handles of `frame_bytes` each (hipMemCreate),
// created lazily and mapped once into a single hipMemAddressReserve arena
// under the budget `target_bytes`. A frame is refilled only after the host has
// seen the hipEvent of its last consumer (the last kernel that read it, or the
// write-back copy that drained it) complete.
//
// Streams: one compute stream (tile kernels), one H2D copy stream and one D2H
// copy stream, all at the default priority; they are ordered with events only.
#pragma once

#include <cstdint>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "device.hpp"

namespace xvram {

struct RuntimeConfig {
  int device_ordinal = 0;
  uint64_t chunk_bytes = 64ull << 20;
  uint64_t cache_target_bytes = 0;
  uint64_t device_headroom_bytes = 512ull << 20;
  uint64_t workspace_reserve_bytes = 4ull << 20;
  uint32_t prefetch_distance = 2;
  uint32_t cache_policy = XVRAM_CACHE_POLICY_CLOCK;
  uint64_t max_transaction_ms = 250;
};

struct HostAllocation {
  uint64_t id = 0;
  uint64_t bytes = 0;
  uint64_t alignment = 0;
  uint32_t priority = 0;
  char* host = nullptr; // pinned backing store (authoritative copy)
};

// A strided rectangle of an allocation: `height` lines of `width` bytes, the
// first at byte `offset`, consecutive lines `pitch` bytes apart.
struct PanelKey {
  uint64_t allocation_id = 0;
  uint64_t offset = 0;
  uint64_t width = 0;
  uint64_t height = 0;
  uint64_t pitch = 0;

  bool operator==(const PanelKey& o) const {
    return allocation_id == o.allocation_id && offset == o.offset && width == o.width &&
           height == o.height && pitch == o.pitch;
  }
  bool operator<(const PanelKey& o) const {
    if (allocation_id != o.allocation_id) return allocation_id < o.allocation_id;
    if (offset != o.offset) return offset < o.offset;
    if (width != o.width) return width < o.width;
    if (height != o.height) return height < o.height;
    return pitch < o.pitch;
  }
  uint64_t end() const { return offset + (height - 1) * pitch + width; }
  uint64_t bytes() const { return width * height; }
};

struct Frame {
  uint64_t index = 0;
  uint64_t address = 0;
  uint64_t handle = 0;
  bool mapped = false;
  bool keyed = false;
  PanelKey key;
  uint64_t packed_pitch = 0;
  int pins = 0;
  bool dirty = false;
  uint64_t last_use = 0;
  Event ready = nullptr; // recorded on the H2D stream after a fill
  bool ready_pending = false;
  Event retire = nullptr; // recorded after the last consumer (kernel or write-back)
  bool retire_pending = false;
  bool used_before = false;
};

// Per-operation intervals for the optional trace file (XVRAM_TRACE_FILE).
struct TraceInterval {
  Event start = nullptr;
  Event stop = nullptr;
  uint64_t bytes = 0;
  char kind = 'k'; // 'k' kernel, 'h' H2D, 'd' D2H
};

class Runtime {
public:
  explicit Runtime(RuntimeConfig config);
  ~Runtime();

  Error setup();
  Error close();
  Error drain();

  Device& device() { return *device_; }
  uint64_t frame_bytes() const { return frame_bytes_; }
  uint64_t frame_capacity() const { return capacity_; }
  uint64_t target_bytes() const { return target_bytes_; }
  uint64_t granularity() const { return granularity_; }
  const RuntimeConfig& config() const { return config_; }
  bool poisoned() const { return poisoned_; }
  Stream compute_stream() const { return compute_; }

  // ---- allocations (authoritative pinned host copies) ----
  Error allocate(uint64_t bytes, uint64_t alignment, uint32_t priority, HostAllocation*& out);
  Error release(uint64_t id);
  Error write(uint64_t id, uint64_t offset, const void* source, uint64_t bytes);
  Error read(uint64_t id, uint64_t offset, void* destination, uint64_t bytes);
  HostAllocation* find(uint64_t id);

  // ---- panel cache ----
  // Makes `key` resident in a frame with packed line pitch `packed_pitch` and
  // pins it. needs_data=false (a write-only panel) skips the H2D copy.
  Error acquire(const PanelKey& key, uint64_t packed_pitch, bool needs_data, Frame*& out);
  // Orders `stream` after the frame's fill.
  Error wait_ready(Frame& frame, Stream stream);
  // Unpins after the consumer enqueued on `stream`; records the retire event.
  Error release_after(Frame& frame, Stream stream, bool dirty);
  // Writes a dirty panel back to its host rectangle (D2H stream, ordered after
  // the frame's last consumer) and removes it from the cache.
  Error writeback_and_evict(Frame& frame);
  // Drops every cached panel (write-back first if dirty=keep) of an allocation
  // overlapping [begin, end); used by allocation_write and release.
  Error invalidate(uint64_t allocation_id, uint64_t begin, uint64_t end);
  // Discards dirty panels without writing them back (failed operation).
  void discard_dirty();
  // Marks the start of an operation: every stream is ordered after it.
  Error begin_operation();
  // Waits for every stream; records trace intervals of the finished operation.
  Error finish_operation(uint64_t operation_id);

  // Kernel bookkeeping used by the executor.
  Error record_kernel(Event& start, Event& stop);
  Error take_event(Event& out);
  void note_kernel_launched() { ++kernels_in_operation_; }

  // Telemetry snapshot in public form.
  void telemetry(xvram_session_telemetry_v1& out) const;

  Error device_failure(int code, std::string_view stage, std::string_view operation);
  Error poison(std::string_view stage, std::string_view operation, std::string_view message);

  bool tracing() const { return !trace_path_.empty(); }
  void trace_push(const TraceInterval& interval) { trace_.push_back(interval); }

private:
  Error ensure_frame_mapped(Frame& frame);
  Error select_frame(Frame*& out);
  Error wait_retired(Frame& frame);
  void evict_key(Frame& frame, bool was_dirty);
  void parallel_copy(void* dst, const void* src, uint64_t bytes);

  RuntimeConfig config_;
  std::unique_ptr<Device> device_;
  bool setup_done_ = false;
  bool closed_ = false;
  bool poisoned_ = false;

  uint64_t granularity_ = 0;
  uint64_t frame_bytes_ = 0;
  uint64_t capacity_ = 0;
  uint64_t target_bytes_ = 0;
  uint64_t arena_ = 0;
  uint64_t arena_bytes_ = 0;
  std::vector<Frame> frames_;
  std::map<PanelKey, uint64_t> index_; // key -> frame index
  uint64_t tick_ = 0;

  Stream compute_ = nullptr;
  Stream h2d_ = nullptr;
  Stream d2h_ = nullptr;
  Event op_start_ = nullptr;
  std::vector<Event> event_pool_;
  std::vector<Event> events_in_use_;

  std::map<uint64_t, HostAllocation> allocations_;
  uint64_t next_allocation_id_ = 1;
  uint64_t pinned_bytes_ = 0;

  // Write-backs still in flight in this operation: a later refill of the same
  // panel waits for them.
  std::map<PanelKey, Event> pending_writebacks_;

  std::string trace_path_;
  std::vector<TraceInterval> trace_;
  uint64_t kernels_in_operation_ = 0;

  xvram_session_telemetry_v1 t_{};
};

} // namespace xvram
