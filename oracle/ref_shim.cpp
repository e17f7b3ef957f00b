// ref_shim.cpp — C entry points over the reference's own planner and pattern
// sources, compiled in place from /root/reference by oracle/Makefile into
// oracle/_ref/libxvram_ref.so. TEST INFRASTRUCTURE ONLY: used by tests/ to
// pin the oracle's pattern restatement, the library's GEMM-problem
// validation, its access normalisation and its entry-state table against the
// reference implementation itself.
//   - ref_pattern_*      -> src/gemm_bench/pattern.cpp:207-237
//   - ref_validate_problem -> src/gemm/planner.cpp:785-859
//   - ref_legal_transition -> src/residency/core.cpp:304-332
//   - ref_normalize        -> src/residency/core.cpp:128-276
//   - ref_policy_run       -> src/residency/policy.cpp:88-187
#include "gemm/planner.hpp"
#include "gemm_bench/pattern.hpp"
#include "residency/core.hpp"
#include "residency/policy.hpp"

#include <memory>

#include <cstdint>
#include <cstdio>
#include <string>
#include <vector>

extern "C" {

uint64_t ref_pattern_a(uint64_t row, uint64_t k) { return xvram::gemm_bench::pattern_a_value(row, k); }
uint64_t ref_pattern_b(uint64_t k, uint64_t col) { return xvram::gemm_bench::pattern_b_value(k, col); }
int ref_pattern_expected(uint64_t row, uint64_t col, uint64_t k, uint64_t* out) {
  const auto value = xvram::gemm_bench::pattern_expected_value(row, col, k);
  if (!value) return 0;
  *out = *value;
  return 1;
}
void ref_pattern_sums(uint64_t k, uint64_t* p, uint64_t* q, uint64_t* pq) {
  const auto sums = xvram::gemm_bench::pattern_closed_form_sums(k);
  *p = sums.sum_p;
  *q = sums.sum_q;
  *pq = sums.sum_pq;
}

// One matrix: allocation id/size, offset, rows, columns, ld, layout (0 row, 1
// column major), element type (0 fp16, 1 bf16, 2 fp32, 3 fp64).
struct RefMatrix {
  uint64_t allocation_id, allocation_bytes, offset_bytes, rows, columns, leading_dimension;
  uint32_t layout, element_type;
};

// Returns the reference ProblemError enumerator (0 == valid) for a GEMM
// problem whose m/k come from A and op_a, n from B and op_b, exactly as
// src/sdk/runtime.cpp:1303-1309 derives them. compute: 0 strict, 1 tf32, 2 fp64.
int ref_validate_problem(const RefMatrix* a, const RefMatrix* b, const RefMatrix* c, uint32_t op_a,
                         uint32_t op_b, uint32_t compute, double beta) {
  using namespace xvram::gemm;
  const auto view = [](const RefMatrix& m) {
    MatrixView v;
    v.allocation_id = xvram::residency::AllocationId{m.allocation_id};
    v.allocation_bytes = m.allocation_bytes;
    v.offset_bytes = m.offset_bytes;
    v.rows = m.rows;
    v.columns = m.columns;
    v.leading_dimension = m.leading_dimension;
    v.layout = m.layout == 1 ? MatrixLayout::column_major : MatrixLayout::row_major;
    v.element_type = static_cast<ElementType>(m.element_type);
    return v;
  };
  GemmProblem p;
  p.a = view(*a);
  p.b = view(*b);
  p.c = view(*c);
  p.a_operation = op_a ? MatrixOperation::transpose : MatrixOperation::none;
  p.b_operation = op_b ? MatrixOperation::transpose : MatrixOperation::none;
  p.m = op_a ? p.a.columns : p.a.rows;
  p.k = op_a ? p.a.rows : p.a.columns;
  p.n = op_b ? p.b.rows : p.b.columns;
  p.compute_mode = compute == 2 ? ComputeMode::fp64
                                : (compute == 1 ? ComputeMode::fast_tf32 : ComputeMode::strict_fp32);
  p.beta = beta;
  return static_cast<int>(validate_problem(p).error);
}

int ref_legal_transition(int from, int to) {
  using xvram::residency::ChunkState;
  return xvram::residency::is_legal_transition(static_cast<ChunkState>(from),
                                               static_cast<ChunkState>(to))
             ? 1
             : 0;
}

// Same flat-array contract as the library's hostsim hook: allocations as
// (id, bytes), ranges as (id, offset, length, mode); outputs normalised ranges
// as quads and chunks as (id, index, valid_bytes, requires_h2d, marks_dirty).
int ref_normalize(const uint64_t* allocs, uint64_t n_allocs, const uint64_t* ranges,
                  uint64_t n_ranges, uint64_t chunk_bytes, uint64_t* out_ranges,
                  uint64_t* n_out_ranges, uint64_t* out_chunks, uint64_t* n_out_chunks,
                  char* error, uint64_t error_len) {
  using namespace xvram::residency;
  std::vector<AllocationLayout> layouts;
  for (uint64_t i = 0; i < n_allocs; ++i)
    layouts.push_back(AllocationLayout{AllocationId{allocs[2 * i]}, allocs[2 * i + 1]});
  std::vector<AccessRange> in;
  for (uint64_t i = 0; i < n_ranges; ++i)
    in.push_back(AccessRange{AllocationId{ranges[4 * i]}, ranges[4 * i + 1], ranges[4 * i + 2],
                             static_cast<AccessMode>(ranges[4 * i + 3])});
  const AccessPlanResult plan = normalize_and_split_accesses(layouts, in, chunk_bytes);
  if (!plan) {
    std::snprintf(error, error_len, "%s", std::string(access_plan_error_name(plan.error)).c_str());
    return 1;
  }
  if (plan.normalized_ranges.size() > *n_out_ranges || plan.chunks.size() > *n_out_chunks)
    return 2;
  for (size_t i = 0; i < plan.normalized_ranges.size(); ++i) {
    const AccessRange& r = plan.normalized_ranges[i];
    out_ranges[4 * i] = r.allocation_id.value;
    out_ranges[4 * i + 1] = r.offset_bytes;
    out_ranges[4 * i + 2] = r.length_bytes;
    out_ranges[4 * i + 3] = static_cast<uint64_t>(r.mode);
  }
  for (size_t i = 0; i < plan.chunks.size(); ++i) {
    const ChunkAccessPlan& c = plan.chunks[i];
    out_chunks[5 * i] = c.key.allocation_id.value;
    out_chunks[5 * i + 1] = c.key.chunk_index;
    out_chunks[5 * i + 2] = c.valid_bytes;
    out_chunks[5 * i + 3] = c.requires_h2d ? 1 : 0;
    out_chunks[5 * i + 4] = c.marks_dirty ? 1 : 0;
  }
  *n_out_ranges = plan.normalized_ranges.size();
  *n_out_chunks = plan.chunks.size();
  return 0;
}

// The command program of the library's hostsim hook, run against the
// reference's ClockPolicy (kind 0) or LruPolicy (kind 1); ids are chunk
// indices of allocation 1.
int ref_policy_run(int kind, const uint64_t* program, uint64_t commands, uint64_t* results) {
  using namespace xvram::residency;
  std::unique_ptr<VictimPolicy> policy;
  if (kind == 1) policy = std::make_unique<LruPolicy>();
  else policy = std::make_unique<ClockPolicy>();
  std::vector<VictimCandidate> candidates;
  const auto key = [](uint64_t id) { return ChunkKey{AllocationId{1}, id}; };
  for (uint64_t i = 0; i < commands; ++i) {
    const uint64_t* c = program + 7 * i;
    results[i] = 0;
    switch (c[0]) {
    case 0: policy->insert(key(c[1]), c[2], c[3] != 0, c[4] != 0); break;
    case 1: policy->touch(key(c[1]), c[2], c[3] != 0); break;
    case 2: results[i] = policy->erase(key(c[1])) ? 1 : 0; break;
    case 3: {
      VictimCandidate v{key(c[1]), static_cast<ChunkState>(c[2])};
      v.hot = c[3] != 0;
      v.pin_count = static_cast<std::uint32_t>(c[4]);
      v.in_flight = c[5] != 0;
      v.in_current_working_set = c[6] != 0;
      bool replaced = false;
      for (auto& existing : candidates)
        if (existing.key == v.key) {
          existing = v;
          replaced = true;
        }
      if (!replaced) candidates.push_back(v);
      break;
    }
    case 4:
      for (size_t k = 0; k < candidates.size(); ++k)
        if (candidates[k].key == key(c[1])) {
          candidates.erase(candidates.begin() + static_cast<std::ptrdiff_t>(k));
          break;
        }
      break;
    case 5: {
      const auto victim = policy->select_victim(candidates);
      results[i] = victim ? victim->chunk_index : ~0ull;
      break;
    }
    default: return -1;
    }
  }
  return 0;
}
}
