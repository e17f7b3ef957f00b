// entry_state.hpp — the states of a residency-cache entry.
#pragma once

#include <cstdint>

namespace xvram {

// Entry states and their legal transitions: the reference's chunk state
// machine (src/residency/core.hpp:102-113, core.cpp:304-332) applied to every
// cache entry (panel or chunk), plus one edge of this design:
// resident_dirty -> evicting, the discard of a failed operation's unwritten
// output (the host copy stays authoritative; the reference poisons instead).
// An illegal move is counted in telemetry (unsafe_transitions), never taken
// silently.
enum class EntryState : uint32_t {
  host_clean,
  prefetch_queued,
  mapping,
  h2d_in_flight,
  resident_clean,
  resident_dirty,
  writeback_queued,
  d2h_in_flight,
  evicting,
  poisoned,
};
bool is_legal_transition(EntryState from, EntryState to);

} // namespace xvram
