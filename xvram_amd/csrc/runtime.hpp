// runtime.hpp — host backing, the VRAM frame pool and the residency cache.
//
// Reference counterpart: residency::Runtime (src/residency/runtime.hpp:317-372,
// runtime.cpp:212-596 setup, :598-727 allocate, :1012-1495 transactions,
// :3470-3529 acquire_frame, :3531-3897 ensure_resident, :3899-4262 writeback,
// :1540-1857 close).
//
// Cache entries come in two kinds:
//   * panels — a packed 2-D sub-matrix (a strided rectangle of an allocation)
//     filled with one hipMemcpy2DAsync; the GEMM executor's unit. Panel frames
//     live at their fixed slot in one hipMemAddressReserve arena.
//   * chunks — frame-sized linear pieces of an allocation used by working-set
//     transactions and prefetch; a chunk frame is mapped at the chunk's stable
//     address inside the allocation's own VA reservation (reserved on first
//     use), so a transaction sees each allocation as one contiguous range.
// Frames are `frame_bytes` hipMemCreate handles, created lazily up to the
// budget. A frame is refilled, unmapped or remapped only after the host has
// seen the hipEvent of its last consumer (kernel, callback work or write-back)
// complete.
//
// The cache is write-back (reference runtime.cpp:931-945, 3155-3173): an entry
// an operation wrote stays resident and dirty after the operation, and its
// bytes reach host memory only when it is evicted, when an allocation_read or
// allocation_write overlaps it, when another entry overlapping it is filled,
// or at drain, close or a budget shrink. When an operation begins, dirty
// entries of earlier operations that its schedule will have to evict start
// their write-back at once (make_room), so the eviction waits for nothing.
// Coherence between overlapping entries: an entry that becomes dirty drops
// every other cached entry overlapping it (they are stale), and an entry is
// filled only after every dirty entry overlapping it has been written back.
//
// Streams: two compute lanes (tile kernels; lane 0 also runs transaction
// callbacks), one H2D copy stream and one D2H copy stream, all at the default
// priority; ordered with events only. Short tile launches alternate between
// the lanes so one launch's tail and the next one's start overlap; every
// launch of one C tile stays on one lane.
#pragma once

#include <chrono>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "common.hpp"
#include "device.hpp"
#include "entry_state.hpp"
#include "policy.hpp"

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
  uint64_t budget_poll_ms = 100;
  // How long the host waits for any one piece of device work (an event or a
  // stream's queue) before it gives up on it: then the session is poisoned
  // and its device resources quarantined (reference RuntimeConfig
  // stall_timeout, src/residency/runtime.hpp:65).
  uint64_t stall_timeout_ms = 5000;
};

struct HostAllocation {
  uint64_t id = 0;
  uint64_t bytes = 0;
  uint64_t alignment = 0;
  uint32_t priority = 0;
  char* host = nullptr;  // pinned backing store (authoritative copy)
  uint64_t va = 0;       // stable device VA for chunk mappings (0 until first use)
  uint64_t va_bytes = 0;
};

enum class EntryKind : uint32_t { panel = 0, chunk = 1 };

// A strided rectangle of an allocation: `height` lines of `width` bytes, the
// first at byte `offset`, consecutive lines `pitch` bytes apart (a chunk is one
// line).
struct PanelKey {
  uint64_t allocation_id = 0;
  uint64_t offset = 0;
  uint64_t width = 0;
  uint64_t height = 0;
  uint64_t pitch = 0;
  EntryKind kind = EntryKind::panel;

  bool operator==(const PanelKey& o) const {
    return allocation_id == o.allocation_id && offset == o.offset && width == o.width &&
           height == o.height && pitch == o.pitch && kind == o.kind;
  }
  bool operator<(const PanelKey& o) const {
    if (allocation_id != o.allocation_id) return allocation_id < o.allocation_id;
    if (kind != o.kind) return kind < o.kind;
    if (offset != o.offset) return offset < o.offset;
    if (width != o.width) return width < o.width;
    if (height != o.height) return height < o.height;
    return pitch < o.pitch;
  }
  uint64_t end() const { return offset + (height - 1) * pitch + width; }
  uint64_t bytes() const { return width * height; }
};

// A share of a panel that one copy fills: lines [line0, line0 + lines) and
// bytes [byte0, byte0 + bytes) of each of them, relative to the panel.
struct PanelPiece {
  uint64_t line0 = 0, lines = 0, byte0 = 0, bytes = 0;
};

// True when the byte sets of two rectangles of one allocation intersect
// (exact for rectangles of equal pitch, conservative otherwise).
bool keys_overlap(const PanelKey& a, const PanelKey& b);


struct Frame {
  uint64_t index = 0;
  uint64_t slot = 0;      // this frame's address in the panel arena
  uint64_t address = 0;   // where the current entry is mapped
  uint64_t mapped_at = 0; // current mapping (0 = unmapped)
  uint64_t handle = 0;    // physical handle (0 = not created yet)
  bool keyed = false;
  PanelKey key;
  uint64_t packed_pitch = 0;
  int pins = 0;
  bool dirty = false;
  uint64_t last_use = 0;
  Event ready = nullptr; // recorded on the H2D stream after a fill
  // The fill's last copy's stop event (operation-owned, recorded just before
  // `ready` on the same stream): when the fill landed, for timing.
  Event ready_stamp = nullptr;
  bool ready_pending = false;
  Event retire = nullptr; // this frame's own event for its last consumer
  // The event that marks the last consumer: `retire`, or the stop event of the
  // tile launch that consumed the frame (adopted, not recorded again).
  Event retire_ref = nullptr;
  bool retire_pending = false;
  uint64_t retire_seq = 0; // schedule order of the last retire record
  bool used_before = false;
  EntryState state = EntryState::host_clean;
  // Event generations (reference core.cpp begin/complete_event_generation):
  // `generation` counts retire-event records, `completed` the last one the
  // host has seen finish. A frame is remapped or refilled only when equal.
  uint64_t generation = 0;
  uint64_t completed = 0;
  // Serial of the operation that started this frame's fill for the operation
  // after it (Runtime::carry_fill); 0 when the frame holds no carried fill.
  uint64_t carry_serial = 0;
  // Serial of the operation that last wrote the entry (a failed operation
  // discards only what it wrote itself).
  uint64_t dirty_serial = 0;
  // Mapped for an output without loading its bytes and not written yet: its
  // contents are garbage until the consumer writes them (dropped if the
  // operation fails first).
  bool unwritten = false;
  // The operation that last wrote the entry overwrote results an earlier
  // operation had left in it, not yet written back. If that operation fails,
  // neither result survives: the bytes are recorded as lost.
  bool overwrote_unflushed = false;
  // Stop event of a write-back still in flight that left the entry cached: a
  // later writer of the frame must not overtake the copy.
  Event writeback_done = nullptr;
  // The last kernel on each compute lane that used the frame (pending until
  // the host has seen it complete): launches on the two lanes finish in any
  // order, so the frame is reused only after both.
  Event lane_ref[2] = {nullptr, nullptr};
  bool lane_pending[2] = {false, false};
};

// Per-operation intervals for the optional trace file (XVRAM_TRACE_FILE).
struct TraceInterval {
  Event start = nullptr;
  Event stop = nullptr;
  // A kernel dispatched with no start event starts when the last of
  // `start_ref` (the previous kernel's stop event on its stream, or the
  // stream's operation start) and the events its stream waited for since
  // (`deps`, operation-owned) completed.
  Event start_ref = nullptr;
  std::vector<Event> deps;
  uint64_t bytes = 0;
  char kind = 'k'; // 'k' kernel, 'h' H2D, 'd' D2H, 't' transaction callback work
  // Start and stop in ms from the operation's start event, once both events
  // have completed (Runtime::time_intervals).
  bool timed = false;
  float start_ms = 0.f, stop_ms = 0.f;
};

// One access of a working-set transaction (allocation-relative bytes).
struct AccessSpan {
  uint64_t allocation_id = 0;
  uint64_t offset = 0;
  uint64_t length = 0;
  uint32_t mode = XVRAM_ACCESS_READ;
};

struct ResolvedSpan {
  AccessSpan span;
  uint64_t device_address = 0;
};

struct AllocationExtent {
  uint64_t id = 0;
  uint64_t bytes = 0;
};

// One chunk a transaction touches: the bytes it holds (`valid_bytes`, short
// for an allocation's last chunk), whether its current bytes must be loaded
// (anything but one write-only span over all valid bytes) and whether the
// transaction writes it.
struct ChunkPlan {
  uint64_t allocation_id = 0;
  uint64_t index = 0;
  uint64_t valid_bytes = 0;
  bool requires_h2d = true;
  bool marks_dirty = false;
};

// Access normalisation and chunk split (reference
// core::normalize_and_split_accesses, src/residency/core.cpp:128-276):
// per allocation in id order, the ranges are cut at every boundary, each piece
// takes the combined mode of the ranges covering it (read + write-only =
// read-write), adjacent pieces of equal mode merge; chunks follow in
// (allocation, index) order. Returns nullptr, or the name of the first
// problem in input order: invalid_access_mode, zero_length,
// unknown_allocation, range_overflow, range_out_of_bounds.
const char* normalize_accesses(const std::vector<AllocationExtent>& allocations,
                               const std::vector<AccessSpan>& ranges, uint64_t chunk_bytes,
                               std::vector<AccessSpan>& normalized,
                               std::vector<ChunkPlan>& chunks);

// The work a transaction enqueues with its working set resident. Returns an
// error to fail the transaction; `skipped` reports that nothing was enqueued.
using TransactionBody =
    std::function<Error(const std::vector<ResolvedSpan>& ranges, uint64_t workspace_address,
                        uint64_t workspace_bytes, Stream stream, bool& skipped)>;

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
  bool quarantined() const { return quarantined_; }
  static constexpr int kLanes = 2;
  Stream compute_stream(int lane = 0) const { return lane == 0 ? compute_ : compute2_; }

  // ---- allocations (authoritative pinned host copies) ----
  Error allocate(uint64_t bytes, uint64_t alignment, uint32_t priority, HostAllocation*& out);
  Error release(uint64_t id);
  Error write(uint64_t id, uint64_t offset, const void* source, uint64_t bytes);
  Error read(uint64_t id, uint64_t offset, void* destination, uint64_t bytes);
  HostAllocation* find(uint64_t id);

  // ---- panel cache (GEMM) ----
  // Makes `key` resident in a frame with packed line pitch `packed_pitch` and
  // pins it. needs_data=false (a write-only panel) skips the H2D copy.
  Error acquire(const PanelKey& key, uint64_t packed_pitch, bool needs_data, Frame*& out);
  // acquire() with data, except that a miss is filled by one copy per piece
  // (the pieces must tile the panel), recorded in order on the H2D stream;
  // `piece_ready` receives one event per piece, complete when that piece has
  // landed, so a consumer of one piece need not wait for the whole panel. A
  // hit (or fewer than two pieces) leaves `piece_ready` empty: wait_ready().
  Error acquire_pieces(const PanelKey& key, uint64_t packed_pitch,
                       const std::vector<PanelPiece>& pieces, Frame*& out,
                       std::vector<Event>& piece_ready);
  // Entries the running schedule will use again soon (the executor's next
  // launches): victim selection passes over them while any other entry is
  // eligible. Empty = none; cleared at the end of every operation.
  void set_protected(std::vector<PanelKey> keys);
  // Orders `stream` after the frame's fill.
  Error wait_ready(Frame& frame, Stream stream);
  // Unpins after the consumer enqueued on `stream`; records the retire event.
  Error release_after(Frame& frame, Stream stream, bool dirty);
  // Unpins after a consumer whose completion `done` already marks (the stop
  // event of a tile launch on compute lane `lane`, recorded by its dispatch):
  // no event is recorded. `done` must stay unrecorded until the operation ends.
  Error release_after_event(Frame& frame, Event done, bool dirty, int lane = 0);
  // Unpins after work enqueued on both compute lanes (a frame every launch of
  // an operation reads, such as a bias vector).
  Error release_after_lanes(Frame& frame);
  // A frame of the pool as a kernel workspace for the current operation
  // (split-K partials): not a cache entry (never filled, never written back),
  // mapped at its arena slot and pinned until release_scratch, which retires
  // it after the last kernel of either compute lane.
  Error take_scratch(Frame*& out);
  Error release_scratch(Frame& frame);
  // Writes a dirty entry back to its host bytes (D2H stream, ordered after the
  // frame's last consumer). With `evict` the entry then leaves the cache (and
  // clean entries overlapping the written bytes are dropped); otherwise it
  // stays cached, clean (resident_dirty -> writeback_queued -> d2h_in_flight
  // -> resident_clean).
  Error writeback(Frame& frame, bool evict);
  Error writeback_and_evict(Frame& frame) { return writeback(frame, true); }
  // Drops every cached entry of an allocation overlapping [begin, end);
  // used by allocation_write and release.
  Error invalidate(uint64_t allocation_id, uint64_t begin, uint64_t end);
  // Discards the entries the current operation wrote, without writing them
  // back, and those it mapped for output but never wrote (a failed
  // operation); unpins everything.
  void discard_dirty();

  // ---- working-set transactions and prefetch ----
  Error run_transaction(const std::vector<AccessSpan>& ranges, uint64_t workspace_bytes,
                        const TransactionBody& body, uint64_t operation_id);
  Error run_prefetch(const std::vector<AccessSpan>& ranges, uint64_t operation_id);

  // ---- operation bracketing ----
  // Marks the start of an operation: every stream is ordered after it.
  Error begin_operation();
  // Called when an operation begins with the number of frames its schedule
  // keeps in use: idle dirty entries written by earlier operations that do
  // not fit beside them will be evicted during the operation, so their
  // write-back (least recently used first) starts now and the eviction finds
  // them clean. The entries stay cached until then.
  Error make_room(uint64_t frames_needed);
  // Live budget (reference refresh_budget, runtime.cpp:3213-3468): samples
  // hipMemGetInfo at most every budget_poll_ms (always when forced), shrinks
  // the frame pool at once when the safe target falls (writing back and
  // releasing the tail frames; BUDGET_PRESSURE if one of them is in use), grows
  // it by two frames after ten consecutive samples with room for two more, and
  // fails with BUDGET_PRESSURE when the next working set no longer fits.
  Error refresh_budget(uint64_t required_frames, uint64_t required_workspace, bool force);
  // Waits for every stream; folds kernel/copy intervals into telemetry, applies
  // the duration guard, writes the optional trace line. Fills carried to the
  // next operation (carry_fill) are not waited for: the H2D stream is waited
  // on only up to the carry fence.
  Error finish_operation(uint64_t operation_id);

  // Cross-operation fill: while the current operation's last launches run,
  // starts the H2D fill of a panel the next queued operation will read, behind
  // a fence that marks the end of the current operation's own fills. The entry
  // is left clean and unpinned, with its ready and retire events pending, for
  // the next operation to find. Panels already cached, or overlapping a dirty
  // entry or a write-back still in flight, are skipped (issued = false).
  Error carry_fill(const PanelKey& key, uint64_t packed_pitch, bool& issued);

  // Kernel bookkeeping used by the executor. record_kernel takes the stop
  // event of a kernel about to be dispatched on compute lane `lane`; its
  // start is derived from the events it follows (TraceInterval::start_ref,
  // deps), and a start event is taken only when the lane waited for an event
  // with no operation-owned stamp (a start event in the dispatch costs ~16 us
  // of host time and ~5 us of device time per kernel).
  Error record_kernel(TraceInterval& iv, int lane);
  // stream_wait_event(stream, event). For a compute lane, `stamp` is an
  // operation-owned event that completes with `event` (nullptr: none known,
  // the lane's next kernel takes a start event).
  Error stream_wait(Stream stream, Event event, Event stamp);
  Error take_event(Event& out);
  void note_kernel_launched(uint64_t tiles = 1) { kernels_in_operation_ += tiles; }

  // Telemetry snapshot in public form.
  void telemetry(xvram_session_telemetry_v1& out) const;
  // Host-store figures of the v2 telemetry: every byte is stored raw.
  uint64_t logical_bytes() const { return pinned_bytes_; }
  uint64_t host_stored_peak_bytes() const { return pinned_peak_bytes_; }

  Error device_failure(int code, std::string_view stage, std::string_view operation);
  // Bounded waits: poll until the event (or everything queued on the stream
  // so far) completes, at most stall_timeout_ms; past that, or on a device
  // error, the runtime is quarantined and the call fails (TIMEOUT / the
  // device error).
  Error await_event(Event event, std::string_view stage, std::string_view operation);
  Error await_stream(Stream stream, std::string_view stage, std::string_view operation) {
    return await_streams({stream}, stage, operation);
  }
  // Every queue in `streams` (at most kSyncMarkers): a marker is recorded on
  // each first, so the waits overlap.
  Error await_streams(std::initializer_list<Stream> streams, std::string_view stage,
                      std::string_view operation);
  Error abandon_device_resources();
  Error poison(std::string_view stage, std::string_view operation, std::string_view message);

  bool tracing() const { return !trace_path_.empty(); }
  void trace_push(const TraceInterval& interval) { trace_.push_back(interval); }
  // Times the operation's intervals whose events have completed, in order,
  // from the first untimed one; with `all`, every interval of the operation
  // (its streams have drained). Kernel and callback durations feed the
  // duration guard. Run while the host would otherwise wait, so that little is
  // left when the operation ends.
  void time_intervals(bool all);

private:
  struct ChunkUse {
    uint64_t allocation_id = 0;
    uint64_t index = 0;
    bool needs_data = true;
    bool writes = false;
    bool filled_empty = false; // mapped on a miss without loading its bytes
    Frame* frame = nullptr;
  };

  void move(Frame& frame, EntryState to);
  void check_generation(const Frame& frame);
  Error record_retire(Frame& frame, Stream stream);
  void adopt_retire(Frame& frame, Event done);
  void adopt_lane(Frame& frame, Event done, int lane);
  Error unpin(Frame& frame, bool dirty);
  Error map_frame_at(Frame& frame, uint64_t address);
  Error abandon_mapping(Frame& frame, Error error);
  Error unmap_frame(Frame& frame);
  Error select_frame(Frame*& out);
  bool allocation_hot(uint64_t allocation_id);
  bool allocation_streaming(uint64_t allocation_id);
  Error release_frame(Frame& frame);
  Error fill_entry(Frame& f, const PanelKey& key, uint64_t packed_pitch, bool needs_data,
                   const std::vector<PanelPiece>* pieces = nullptr,
                   std::vector<Event>* piece_ready = nullptr);
  Error wait_retired(Frame& frame);
  Error evict_key(Frame& frame, bool was_dirty);
  Error drop_overlapping(const PanelKey& written, const Frame* except);
  // Writes back (keeping them cached) the dirty entries overlapping `key`
  // other than `except`, before `key` is filled; counts the bytes as
  // write-backs. Fails if such an entry is pinned.
  Error flush_overlapping(const PanelKey& key, const Frame* except);
  // Writes back every dirty entry (drain, close); waits for the copies.
  Error flush_all();
  // After the host has waited for the D2H stream: no write-back is in flight.
  void writebacks_settled();
  Error reserve_allocation_va(HostAllocation& a);
  Error ensure_workspace(uint64_t bytes);
  Error plan_chunks(const std::vector<AccessSpan>& ranges, std::vector<ChunkUse>& chunks,
                    std::vector<AccessSpan>& normalized, const char* operation);
  Error acquire_chunk(ChunkUse& use);
  void parallel_copy(void* dst, const void* src, uint64_t bytes);

  RuntimeConfig config_;
  std::unique_ptr<Device> device_;
  bool setup_done_ = false;
  bool closed_ = false;
  bool poisoned_ = false;
  // Device work whose completion the host could not observe (a wait ran past
  // the stall deadline or a query failed) may still use frames, the
  // workspace and the pinned host buffers: close then abandons them.
  bool quarantined_ = false;
  // Rectangles whose latest results were lost: a failed operation rewrote
  // entries that held an earlier operation's unwritten results, and dropped
  // them. Reading those bytes (allocation_read, a fill) fails with
  // CORRUPTION until the caller writes them again or a later operation's
  // write-back covers them.
  std::vector<PanelKey> lost_;
  Error check_not_lost(const PanelKey& range, const char* stage, const char* operation) const;
  void forget_lost_within(const PanelKey& rewritten);
  // Recorded on streams to wait for their queues (one per stream a single
  // wait covers: all are recorded before any is polled).
  static constexpr int kSyncMarkers = 4;
  Event sync_markers_[kSyncMarkers] = {};
  bool launches_blocked_ = false;

  uint64_t granularity_ = 0;
  uint64_t frame_bytes_ = 0;
  uint64_t capacity_ = 0;       // frames usable now (live budget)
  uint64_t max_capacity_ = 0;   // frames reserved at setup (the arena)
  uint64_t configured_cap_ = 0; // cache_target_bytes, or total device memory when 0
  uint64_t target_bytes_ = 0;
  Clock::time_point last_budget_sample_{};
  uint32_t growth_samples_ = 0;
  std::unique_ptr<EvictionPolicy> policy_;
  uint64_t policy_sequence_ = 0;
  bool prefetching_ = false;
  uint64_t arena_ = 0;
  uint64_t arena_bytes_ = 0;
  std::vector<Frame> frames_;
  std::map<PanelKey, uint64_t> index_; // key -> frame index
  std::vector<PanelKey> protected_;    // sorted; see set_protected
  uint64_t tick_ = 0;
  uint64_t retire_records_ = 0; // retire events recorded so far (schedule order)

  uint64_t workspace_va_ = 0;
  uint64_t workspace_bytes_ = 0;
  uint64_t workspace_handle_ = 0;

  Stream compute_ = nullptr;
  Stream compute2_ = nullptr; // compute lane 1
  Stream h2d_ = nullptr;
  Stream d2h_ = nullptr;
  Event op_start_ = nullptr;  // recorded on compute_ at each operation's start
  Event op_start2_ = nullptr; // recorded on compute2_ at the same time
  // Host clock at begin_operation (the trace's host timestamps count from it).
  std::chrono::steady_clock::time_point op_host_start_{};
  size_t trace_timed_ = 0;     // trace_[0 .. trace_timed_) are timed
  bool op_start_seen_ = false; // op_start_ and op_start2_ have completed (intervals can be timed)
  Event lane_last_[2] = {nullptr, nullptr}; // last kernel stop per lane (its start event at first)
  bool lane_waited_[2] = {false, false};    // a wait without a stamp since lane_last_
  // Host clock at each lane's last dispatch (or the operation's start). A
  // lane the host left alone for longer than kStartEventAfterHostGap may have
  // drained and idled, so its next kernel takes a real start event instead
  // of inheriting the previous stop (an idle gap would otherwise count as
  // kernel time under the duration guard).
  Clock::time_point lane_dispatched_at_[2]{};
  std::vector<Event> lane_deps_[2];         // stamps of the waits since lane_last_
  bool guard_tripped_ = false; // a kernel or callback of the operation exceeded the guard
  std::vector<Event> event_pool_;
  std::vector<Event> events_in_use_;
  uint64_t op_serial_ = 0; // operations begun so far
  bool in_operation_ = false;

  // Fills carried past the current operation (carry_fill): the fence on the
  // H2D stream before the first of them, and where their trace intervals and
  // events start in trace_ / events_in_use_. At the end of the operation they
  // move to carried_trace_ / carried_events_ and join the next operation.
  bool carry_active_ = false;
  Event carry_fence_ = nullptr;
  size_t carry_trace_mark_ = 0;
  size_t carry_event_mark_ = 0;
  std::vector<TraceInterval> carried_trace_;
  std::vector<Event> carried_events_;

  std::map<uint64_t, HostAllocation> allocations_;
  uint64_t next_allocation_id_ = 1;
  uint64_t pinned_bytes_ = 0;      // sum of live allocation sizes (all raw host bytes)
  uint64_t pinned_peak_bytes_ = 0;

  // Write-backs still in flight in this operation: a later refill of the same
  // entry waits for them.
  std::map<PanelKey, Event> pending_writebacks_;

  std::string trace_path_;
  std::vector<TraceInterval> trace_;
  uint64_t kernels_in_operation_ = 0;
  uint64_t transactions_in_operation_ = 0;

  xvram_session_telemetry_v1 t_{};
};

} // namespace xvram
