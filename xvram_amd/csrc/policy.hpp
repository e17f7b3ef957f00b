// policy.hpp — victim selection for the residency cache.
//
// Reference counterpart: residency::ClockPolicy / LruPolicy
// (src/residency/policy.hpp:25-84, policy.cpp:88-187). Kept identical because
// the session's cache_policy selects between them and callers rely on their
// order of eviction:
//   * CLOCK (the default): entries in insertion order with a hand and a
//     reference bit; among eligible entries only the cheapest cost class is
//     considered (dirty +3, hot +4; then one-touch streaming 0, speculative
//     (prefetched, never used) 1, other 2); one sweep clears reference bits of
//     that class, a second picks the first unreferenced entry after the hand.
//   * LRU: the eligible entry with the oldest touch, non-hot first, ties by id.
// An entry is eligible when it is resident (clean or dirty), unpinned, has no
// work in flight and is not part of the working set being acquired.
#pragma once

#include <cstdint>
#include <memory>
#include <optional>
#include <vector>

#include "entry_state.hpp"

namespace xvram {

struct VictimCandidate {
  uint64_t id = 0;
  EntryState state{};
  bool hot = false;
  uint32_t pins = 0;
  bool in_flight = false;
  bool in_working_set = false;
};

bool is_policy_candidate_eligible(const VictimCandidate& candidate);

class EvictionPolicy {
public:
  virtual ~EvictionPolicy() = default;
  virtual const char* name() const = 0;
  virtual void insert(uint64_t id, uint64_t sequence, bool speculative, bool one_touch) = 0;
  virtual void touch(uint64_t id, uint64_t sequence, bool one_touch) = 0;
  virtual bool erase(uint64_t id) = 0;
  virtual std::optional<uint64_t> select_victim(const std::vector<VictimCandidate>& candidates) = 0;
  virtual size_t size() const = 0;
};

class ClockPolicy final : public EvictionPolicy {
public:
  const char* name() const override { return "clock"; }
  void insert(uint64_t id, uint64_t sequence, bool speculative, bool one_touch) override;
  void touch(uint64_t id, uint64_t sequence, bool one_touch) override;
  bool erase(uint64_t id) override;
  std::optional<uint64_t> select_victim(const std::vector<VictimCandidate>& candidates) override;
  size_t size() const override { return entries_.size(); }

private:
  struct Entry {
    uint64_t id;
    bool referenced;
    bool speculative;
    bool one_touch;
  };
  std::vector<Entry> entries_;
  size_t hand_ = 0;
};

class LruPolicy final : public EvictionPolicy {
public:
  const char* name() const override { return "lru"; }
  void insert(uint64_t id, uint64_t sequence, bool speculative, bool one_touch) override;
  void touch(uint64_t id, uint64_t sequence, bool one_touch) override;
  bool erase(uint64_t id) override;
  std::optional<uint64_t> select_victim(const std::vector<VictimCandidate>& candidates) override;
  size_t size() const override { return entries_.size(); }

private:
  struct Entry {
    uint64_t id;
    uint64_t last_touch;
  };
  std::vector<Entry> entries_;
};

// XVRAM_CACHE_POLICY_CLOCK or XVRAM_CACHE_POLICY_LRU.
std::unique_ptr<EvictionPolicy> make_policy(uint32_t cache_policy);

} // namespace xvram
