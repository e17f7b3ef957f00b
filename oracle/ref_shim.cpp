// ref_shim.cpp — C entry points over the reference's own planner and pattern
// sources, compiled in place from /root/reference by oracle/Makefile into
// oracle/_ref/libxvram_ref.so. TEST INFRASTRUCTURE ONLY: used by tests/ to
// pin the oracle's pattern restatement and the library's GEMM-problem
// validation against the reference implementation itself.
//   - ref_pattern_*      -> src/gemm_bench/pattern.cpp:207-237
//   - ref_validate_problem -> src/gemm/planner.cpp:785-859
#include "gemm/planner.hpp"
#include "gemm_bench/pattern.hpp"

#include <cstdint>

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
}
