// policy.cpp — CLOCK and LRU victim selection (reference policy.cpp:88-187).
#include "policy.hpp"

#include <algorithm>
#include <limits>
#include <unordered_map>

#include "xvram/xvram.h"

namespace xvram {

namespace {

class CandidateIndex {
public:
  explicit CandidateIndex(const std::vector<VictimCandidate>& candidates) {
    by_id_.reserve(candidates.size());
    for (const VictimCandidate& c : candidates) by_id_.emplace(c.id, &c);
  }
  const VictimCandidate* find(uint64_t id) const {
    auto it = by_id_.find(id);
    return it == by_id_.end() ? nullptr : it->second;
  }

private:
  std::unordered_map<uint64_t, const VictimCandidate*> by_id_;
};

// Cost classes: dirty +3, hot +4, then one-touch streaming 0, speculative 1,
// everything else 2.
unsigned cost_of(bool speculative, bool one_touch, const VictimCandidate& c) {
  const unsigned base = (c.state == EntryState::resident_dirty ? 3u : 0u) + (c.hot ? 4u : 0u);
  if (one_touch) return base;
  return base + (speculative ? 1u : 2u);
}

} // namespace

bool is_policy_candidate_eligible(const VictimCandidate& c) {
  const bool resident = c.state == EntryState::resident_clean || c.state == EntryState::resident_dirty;
  return resident && c.pins == 0 && !c.in_flight && !c.in_working_set;
}

void ClockPolicy::insert(uint64_t id, uint64_t, bool speculative, bool one_touch) {
  for (Entry& e : entries_) {
    if (e.id == id) {
      e.referenced = e.referenced || !speculative;
      e.speculative = speculative;
      e.one_touch = one_touch;
      return;
    }
  }
  entries_.push_back(Entry{id, !speculative, speculative, one_touch});
}

void ClockPolicy::touch(uint64_t id, uint64_t sequence, bool one_touch) {
  for (Entry& e : entries_) {
    if (e.id == id) {
      e.referenced = true;
      e.speculative = false;
      e.one_touch = one_touch;
      return;
    }
  }
  insert(id, sequence, false, one_touch);
}

bool ClockPolicy::erase(uint64_t id) {
  for (size_t i = 0; i < entries_.size(); ++i) {
    if (entries_[i].id != id) continue;
    entries_.erase(entries_.begin() + static_cast<std::ptrdiff_t>(i));
    if (!entries_.empty() && i < hand_) --hand_;
    if (entries_.empty() || hand_ >= entries_.size()) hand_ = 0;
    return true;
  }
  return false;
}

std::optional<uint64_t> ClockPolicy::select_victim(const std::vector<VictimCandidate>& candidates) {
  if (entries_.empty()) return std::nullopt;
  const CandidateIndex index_of(candidates);
  unsigned cheapest = std::numeric_limits<unsigned>::max();
  for (const Entry& e : entries_) {
    const VictimCandidate* c = index_of.find(e.id);
    if (c && is_policy_candidate_eligible(*c))
      cheapest = std::min(cheapest, cost_of(e.speculative, e.one_touch, *c));
  }
  if (cheapest == std::numeric_limits<unsigned>::max()) return std::nullopt;
  // Sweep 1 clears the reference bits of the cheapest class; sweep 2 then
  // finds an entry whose second chance is used up.
  for (int sweep = 0; sweep < 2; ++sweep) {
    for (size_t step = 0; step < entries_.size(); ++step) {
      const size_t index = (hand_ + step) % entries_.size();
      Entry& e = entries_[index];
      const VictimCandidate* c = index_of.find(e.id);
      if (!c || !is_policy_candidate_eligible(*c) || cost_of(e.speculative, e.one_touch, *c) != cheapest)
        continue;
      if (e.referenced) {
        e.referenced = false;
        continue;
      }
      hand_ = (index + 1) % entries_.size();
      return e.id;
    }
  }
  return std::nullopt;
}

void LruPolicy::insert(uint64_t id, uint64_t sequence, bool, bool) {
  for (Entry& e : entries_) {
    if (e.id == id) {
      e.last_touch = sequence;
      return;
    }
  }
  entries_.push_back(Entry{id, sequence});
}

void LruPolicy::touch(uint64_t id, uint64_t sequence, bool) { insert(id, sequence, false, false); }

bool LruPolicy::erase(uint64_t id) {
  for (size_t i = 0; i < entries_.size(); ++i) {
    if (entries_[i].id == id) {
      entries_.erase(entries_.begin() + static_cast<std::ptrdiff_t>(i));
      return true;
    }
  }
  return false;
}

std::optional<uint64_t> LruPolicy::select_victim(const std::vector<VictimCandidate>& candidates) {
  const CandidateIndex index_of(candidates);
  const Entry* best = nullptr;
  const VictimCandidate* best_c = nullptr;
  for (const Entry& e : entries_) {
    const VictimCandidate* c = index_of.find(e.id);
    if (!c || !is_policy_candidate_eligible(*c)) continue;
    const bool better =
        best == nullptr || (best_c->hot && !c->hot) ||
        (best_c->hot == c->hot &&
         (e.last_touch < best->last_touch || (e.last_touch == best->last_touch && e.id < best->id)));
    if (better) {
      best = &e;
      best_c = c;
    }
  }
  if (!best) return std::nullopt;
  return best->id;
}

std::unique_ptr<EvictionPolicy> make_policy(uint32_t cache_policy) {
  if (cache_policy == XVRAM_CACHE_POLICY_LRU) return std::make_unique<LruPolicy>();
  return std::make_unique<ClockPolicy>();
}

} // namespace xvram
