// gemm.hpp — GEMM problem validation, panel planning and the pipelined
// out-of-core executor.
//
// Reference counterparts: src/gemm/planner.hpp/.cpp (validate_problem
// :785-859, make_plan :1005-1153) and src/gemm/executor.cpp:331-454
// (execute_tiled_gemm). Validation reproduces the reference rules and error
// classes exactly; planning and execution are redesigned around panels.
#pragma once

#include <cstdint>
#include <functional>
#include <string>
#include <vector>

#include "common.hpp"
#include "runtime.hpp"

namespace xvram {

struct MatrixSpec {
  uint64_t allocation_id = 0;
  uint64_t allocation_bytes = 0;
  uint64_t offset_bytes = 0;
  uint64_t rows = 0;
  uint64_t columns = 0;
  uint64_t leading_dimension = 0;
  uint32_t layout = XVRAM_MATRIX_ROW_MAJOR;
  uint32_t data_type = XVRAM_DATA_FP32;
};

// Optional fused epilogue, an extension of this build with no reference
// counterpart (the reference's tiled linear is bias-free,
// python/xvram/torch_native.py:1920-1921):
//   C = act(alpha * op(A) * op(B) + beta * C + bias)
// with an FP32 bias vector over the rows (length m) or the columns (length n)
// of the caller's C, and act = identity or ReLU.
struct EpilogueSpec {
  uint64_t bias_allocation_id = 0; // 0 = no bias
  uint64_t bias_allocation_bytes = 0;
  uint64_t bias_offset_bytes = 0;
  uint32_t bias_axis = 0;  // XVRAM_AMD_BIAS_PER_ROW / _PER_COLUMN of the caller's C
  uint32_t activation = 0; // XVRAM_AMD_ACTIVATION_NONE / _RELU
};

struct GemmSpec {
  MatrixSpec a, b, c;
  uint32_t operation_a = XVRAM_MATRIX_OP_N;
  uint32_t operation_b = XVRAM_MATRIX_OP_N;
  uint32_t compute_mode = XVRAM_COMPUTE_AUTO;
  double alpha = 1.0;
  double beta = 0.0;
  uint64_t tile_m_hint = 0, tile_n_hint = 0, tile_k_hint = 0;
  EpilogueSpec epilogue;
};

// Problem error classes in the reference's enumerator order
// (src/gemm/planner.hpp:69-84).
enum class ProblemError : int {
  none = 0,
  zero_dimension,
  invalid_allocation,
  invalid_layout,
  invalid_operation,
  invalid_element_type,
  invalid_compute_mode,
  dimension_mismatch,
  leading_dimension_too_small,
  storage_overflow,
  storage_out_of_bounds,
  unsupported_type_combination,
  output_aliases_input,
  integer_limit_exceeded,
};

const char* problem_error_name(ProblemError error);

// m/k from A and op_a, n from B and op_b (src/sdk/runtime.cpp:1303-1308).
void problem_dims(const GemmSpec& spec, uint64_t& m, uint64_t& n, uint64_t& k);

// The reference's validate_problem, compute mode resolved as
// src/sdk/runtime.cpp:119-135 does (AUTO -> TF32 for FP32 data).
ProblemError validate_problem(const GemmSpec& spec, char* operand);

// One operand of the canonical column-major problem. Element (x, y) of the
// operand's *physical* column-major storage is at base + (x + y*ld)*4; the
// operand's logical (row, col) maps to (x, y) directly unless `transposed`.
struct CanonOperand {
  uint64_t allocation_id = 0;
  uint64_t base = 0;
  uint64_t ld = 0;
  bool transposed = false;
};

// C' (m x n, column-major) = alpha * op(A') * op(B') + beta * C'.
struct CanonProblem {
  uint64_t m = 0, n = 0, k = 0;
  CanonOperand a, b, c;
  float alpha = 1.f, beta = 0.f;
  bool swapped = false; // C was row-major: C' = C^T, A' = B, B' = A
  // Epilogue in canonical terms: the bias runs along C' rows (length m) when
  // bias_rows, else along C' columns (length n).
  uint64_t bias_allocation_id = 0;
  uint64_t bias_base = 0;
  bool bias_rows = false;
  bool relu = false;
  bool has_epilogue() const { return bias_allocation_id != 0 || relu; }
  uint64_t bias_length() const { return bias_rows ? m : n; }
};

// Checks an epilogue against the problem (extension rules: FP32 bias inside
// its allocation, 4-byte aligned, not overlapping C; known axis/activation).
Error validate_epilogue(const GemmSpec& spec);

CanonProblem canonicalize(const GemmSpec& spec);

// One tile-kernel launch of a plan: C' tile (ti, tj), K panels kp ..
// kp + panels - 1 (each its own A and B frame).
struct TileLaunch {
  uint32_t ti = 0, tj = 0, kp = 0;
  uint8_t panels = 1;
  bool first_panel = false; // first K panel applied to this C tile (uses user beta)
  bool last_panel = false;  // C tile final after this launch
  // The C tile is final and its block is not the plan's last: the next
  // blocks' tiles need its frame, so it is written back and evicted as soon
  // as this launch is enqueued. The last block's tiles stay resident, dirty.
  bool evict_c = false;
  uint8_t lane = 0; // compute lane (Runtime::compute_stream); one lane per C tile
};

struct GemmPlanData {
  CanonProblem problem;
  uint64_t tm = 0, tn = 0, bk = 0;         // tile / panel extents
  uint64_t tiles_m = 0, tiles_n = 0, panels_k = 0;
  uint64_t block_m = 0, block_n = 0;       // C block, in tiles
  uint32_t lookahead = 0;                  // launches acquired ahead of the enqueue point
  uint64_t h2d_bytes_planned = 0;          // compulsory traffic of this schedule
  uint64_t d2h_bytes_planned = 0;
  uint64_t frames_in_use = 0;              // frames the schedule keeps busy at once
  int lanes = 1;                           // compute lanes the launches alternate over
  uint32_t panels_per_launch = 1;          // K panels one launch covers (1 or 2)
  // Launches that leave workgroup slots idle split K (kernels::split_k_plan)
  // into partials held in one frame of the pool, taken for the operation.
  bool scratch = false;
  std::vector<TileLaunch> launches;
};

// Launches of at most this many FLOPs (a few ms) alternate between the two
// compute lanes: a short launch's fixed costs (its last workgroups' C tile
// write, the next launch's dispatch and first loads) are then overlapped by
// the neighbouring launch. Longer launches stay on one lane, where each
// launch's HIP-event duration is its own run time.
constexpr double kDualLaneMaxFlops = 3.0e11;

// One-panel launches of at most this many FLOPs take two K panels per launch
// when a two-panel tile kernel accepts them (interior 256 x 256 tiles, at
// least one per CU, panel depth a multiple of 32, K a multiple of 4 for N/T
// and of 8 for the other forms) and the schedule keeps
// its H2D traffic: each launch pays a C-tile read and write through HBM and a
// prologue, ~20 us on a 4096 x 4096 tile (2 % of a 4096-deep launch).
constexpr double kTwoPanelMaxFlops = 1.5e11;

// Floating-point rate assumed when sizing launches against the transaction
// duration guard: well under the tile kernel's sustained FP32 rate, so a launch
// planned at the cap finishes in a fraction of the guard.
constexpr double kGuardPlanningFlopsPerMs = 4.0e10; // 40 TFLOP/s

// max_launch_flops caps 2*tm*tn*bk of every launch (0 = no cap).
Error make_gemm_plan(const GemmSpec& spec, uint64_t frame_bytes, uint64_t frame_count,
                     uint32_t prefetch_distance, uint64_t max_launch_flops, GemmPlanData& out);

struct GemmHooks {
  // Called at safe boundaries (before each launch); a returned error stops
  // execution there.
  std::function<Error(const char* boundary)> boundary;
  std::function<void(uint64_t completed, uint64_t total)> progress;
  // Called once after the last launch is enqueued, while it still runs: the
  // place to start fills for the operation queued next (carry_gemm_head).
  std::function<Error()> tail;
};

Error execute_gemm(Runtime& runtime, const GemmPlanData& plan, uint64_t operation_id,
                   const GemmHooks& hooks);

// Starts, behind the running operation (Runtime::carry_fill), the fills of
// the bias and of the A and B panels of the first `launches` launches of
// `plan`: the panels its executor acquires before its first enqueue. Stops
// quietly when no frame is free of pins; device errors are returned.
Error carry_gemm_head(Runtime& runtime, const GemmPlanData& plan, uint64_t launches);

} // namespace xvram
