// gemm.cpp — validation, panel planning and pipelined execution of one GEMM.
#include "gemm.hpp"

#include <algorithm>
#include <climits>
#include <cmath>
#include <deque>

namespace xvram {

namespace {

uint64_t element_bytes(uint32_t type) {
  switch (type) {
  case XVRAM_DATA_FP16:
  case XVRAM_DATA_BF16: return 2;
  case XVRAM_DATA_FP32: return 4;
  case XVRAM_DATA_FP64: return 8;
  default: return 0;
  }
}

enum class Compute { strict_fp32, fast_tf32, fp64, invalid };

// Compute-mode resolution of the reference session (src/sdk/runtime.cpp:119-135).
Compute resolve_compute(uint32_t mode, uint32_t a_type) {
  switch (mode) {
  case XVRAM_COMPUTE_AUTO:
    if (a_type == XVRAM_DATA_FP64) return Compute::fp64;
    if (a_type == XVRAM_DATA_FP16 || a_type == XVRAM_DATA_BF16) return Compute::strict_fp32;
    return Compute::fast_tf32;
  case XVRAM_COMPUTE_FP32_STRICT: return Compute::strict_fp32;
  case XVRAM_COMPUTE_FP32_TF32: return Compute::fast_tf32;
  case XVRAM_COMPUTE_FP64: return Compute::fp64;
  default: return Compute::invalid;
  }
}

struct Bounds {
  uint64_t begin = 0, end = 0;
};

// Per-operand checks in the reference's order (planner.cpp:50-100).
ProblemError validate_matrix(const MatrixSpec& mx) {
  if (mx.allocation_id == 0 || mx.allocation_bytes == 0) return ProblemError::invalid_allocation;
  if (mx.layout != XVRAM_MATRIX_ROW_MAJOR && mx.layout != XVRAM_MATRIX_COLUMN_MAJOR)
    return ProblemError::invalid_layout;
  const uint64_t eb = element_bytes(mx.data_type);
  if (eb == 0) return ProblemError::invalid_element_type;
  if (mx.rows == 0 || mx.columns == 0) return ProblemError::zero_dimension;
  const bool row = mx.layout == XVRAM_MATRIX_ROW_MAJOR;
  const uint64_t required_ld = row ? mx.columns : mx.rows;
  if (mx.leading_dimension < required_ld) return ProblemError::leading_dimension_too_small;
  if (mx.leading_dimension > static_cast<uint64_t>(INT_MAX))
    return ProblemError::integer_limit_exceeded;
  const uint64_t major = row ? mx.rows : mx.columns;
  const uint64_t minor = row ? mx.columns : mx.rows;
  uint64_t last_major = 0, last = 0, bytes = 0, end = 0;
  if (!checked_mul(major - 1, mx.leading_dimension, last_major))
    return ProblemError::storage_overflow;
  if (!checked_add(last_major, minor - 1, last) || !checked_add(last, 1, last))
    return ProblemError::storage_overflow;
  if (!checked_mul(last, eb, bytes) || !checked_add(mx.offset_bytes, bytes, end))
    return ProblemError::storage_overflow;
  if (mx.offset_bytes >= mx.allocation_bytes || end > mx.allocation_bytes)
    return ProblemError::storage_out_of_bounds;
  return ProblemError::none;
}

bool matrix_bounds(const MatrixSpec& mx, Bounds& out) {
  const uint64_t eb = element_bytes(mx.data_type);
  if (eb == 0 || mx.rows == 0 || mx.columns == 0) return false;
  const bool row = mx.layout == XVRAM_MATRIX_ROW_MAJOR;
  const uint64_t major = row ? mx.rows : mx.columns;
  const uint64_t minor = row ? mx.columns : mx.rows;
  uint64_t elements = 0, bytes = 0, end = 0;
  if (!checked_mul(major - 1, mx.leading_dimension, elements) ||
      !checked_add(elements, minor, elements) || !checked_mul(elements, eb, bytes) ||
      !checked_add(mx.offset_bytes, bytes, end))
    return false;
  out = Bounds{mx.offset_bytes, end};
  return true;
}

uint64_t isqrt(uint64_t v) {
  uint64_t r = static_cast<uint64_t>(std::sqrt(static_cast<double>(v)));
  while (r * r > v) --r;
  while ((r + 1) * (r + 1) <= v) ++r;
  return r;
}

// Geometry of one panel of an operand: x runs along the stored (contiguous)
// dimension, y along lines.
struct PanelGeom {
  uint64_t x0, xn, y0, yn;
};

PanelKey panel_key(const CanonOperand& op, const PanelGeom& g) {
  PanelKey key;
  key.allocation_id = op.allocation_id;
  key.offset = op.base + (g.x0 + g.y0 * op.ld) * 4;
  key.width = g.xn * 4;
  key.height = g.yn;
  key.pitch = op.ld * 4;
  return key;
}

uint64_t packed_ld(const PanelGeom& g) { return round_up(g.xn, 4); }
uint64_t panel_bytes(uint64_t x_extent, uint64_t lines) { return round_up(x_extent, 4) * 4 * lines; }

// Panel of A' rows [i0, i0+h), k [p0, p0+w).
PanelGeom a_geom(const CanonOperand& a, uint64_t i0, uint64_t h, uint64_t p0, uint64_t w) {
  return a.transposed ? PanelGeom{p0, w, i0, h} : PanelGeom{i0, h, p0, w};
}
// Panel of B' k [p0, p0+w), columns [j0, j0+g).
PanelGeom b_geom(const CanonOperand& b, uint64_t p0, uint64_t w, uint64_t j0, uint64_t g) {
  return b.transposed ? PanelGeom{j0, g, p0, w} : PanelGeom{p0, w, j0, g};
}
PanelGeom c_geom(uint64_t i0, uint64_t h, uint64_t j0, uint64_t g) { return PanelGeom{i0, h, j0, g}; }

uint64_t a_panel_bytes(const CanonProblem& p, uint64_t h, uint64_t w) {
  return p.a.transposed ? panel_bytes(w, h) : panel_bytes(h, w);
}
uint64_t b_panel_bytes(const CanonProblem& p, uint64_t w, uint64_t g) {
  return p.b.transposed ? panel_bytes(g, w) : panel_bytes(w, g);
}
uint64_t c_panel_bytes(uint64_t h, uint64_t g) { return panel_bytes(h, g); }

} // namespace

const char* problem_error_name(ProblemError error) {
  switch (error) {
  case ProblemError::none: return "none";
  case ProblemError::zero_dimension: return "zero_dimension";
  case ProblemError::invalid_allocation: return "invalid_allocation";
  case ProblemError::invalid_layout: return "invalid_layout";
  case ProblemError::invalid_operation: return "invalid_operation";
  case ProblemError::invalid_element_type: return "invalid_element_type";
  case ProblemError::invalid_compute_mode: return "invalid_compute_mode";
  case ProblemError::dimension_mismatch: return "dimension_mismatch";
  case ProblemError::leading_dimension_too_small: return "leading_dimension_too_small";
  case ProblemError::storage_overflow: return "storage_overflow";
  case ProblemError::storage_out_of_bounds: return "storage_out_of_bounds";
  case ProblemError::unsupported_type_combination: return "unsupported_type_combination";
  case ProblemError::output_aliases_input: return "output_aliases_input";
  case ProblemError::integer_limit_exceeded: return "integer_limit_exceeded";
  }
  return "invalid";
}

void problem_dims(const GemmSpec& s, uint64_t& m, uint64_t& n, uint64_t& k) {
  const bool ta = s.operation_a == XVRAM_MATRIX_OP_T;
  const bool tb = s.operation_b == XVRAM_MATRIX_OP_T;
  m = ta ? s.a.columns : s.a.rows;
  k = ta ? s.a.rows : s.a.columns;
  n = tb ? s.b.rows : s.b.columns;
}

// GEMM problem validity, rule for rule as the reference's validate_problem
// (src/gemm/planner.cpp:785-859), including which rule reports first.
ProblemError validate_problem(const GemmSpec& s, char* operand) {
  char dummy = 0;
  char& who = operand ? *operand : dummy;
  who = 0;
  uint64_t m, n, k;
  problem_dims(s, m, n, k);
  if (m == 0 || n == 0 || k == 0) return ProblemError::zero_dimension;
  if (s.operation_a != XVRAM_MATRIX_OP_N && s.operation_a != XVRAM_MATRIX_OP_T) {
    who = 'A';
    return ProblemError::invalid_operation;
  }
  if (s.operation_b != XVRAM_MATRIX_OP_N && s.operation_b != XVRAM_MATRIX_OP_T) {
    who = 'B';
    return ProblemError::invalid_operation;
  }
  const Compute compute = resolve_compute(s.compute_mode, s.a.data_type);
  if (compute == Compute::invalid) return ProblemError::invalid_compute_mode;
  const MatrixSpec* mats[3] = {&s.a, &s.b, &s.c};
  const char names[3] = {'A', 'B', 'C'};
  for (int i = 0; i < 3; ++i) {
    const ProblemError e = validate_matrix(*mats[i]);
    if (e != ProblemError::none) {
      who = names[i];
      return e;
    }
  }
  if ((s.a.allocation_id == s.b.allocation_id && s.a.allocation_bytes != s.b.allocation_bytes) ||
      (s.a.allocation_id == s.c.allocation_id && s.a.allocation_bytes != s.c.allocation_bytes) ||
      (s.b.allocation_id == s.c.allocation_id && s.b.allocation_bytes != s.c.allocation_bytes))
    return ProblemError::invalid_allocation;
  const bool tb = s.operation_b == XVRAM_MATRIX_OP_T;
  const uint64_t b_rows = tb ? s.b.columns : s.b.rows;
  const uint64_t b_cols = tb ? s.b.rows : s.b.columns;
  if (b_rows != k || b_cols != n || s.c.rows != m || s.c.columns != n)
    return ProblemError::dimension_mismatch;
  if (s.a.data_type != s.b.data_type) return ProblemError::unsupported_type_combination;
  bool supported = false;
  switch (s.a.data_type) {
  case XVRAM_DATA_FP16:
  case XVRAM_DATA_BF16:
    supported = (s.c.data_type == s.a.data_type || s.c.data_type == XVRAM_DATA_FP32) &&
                compute == Compute::strict_fp32;
    break;
  case XVRAM_DATA_FP32:
    supported = s.c.data_type == XVRAM_DATA_FP32 &&
                (compute == Compute::strict_fp32 || compute == Compute::fast_tf32);
    break;
  case XVRAM_DATA_FP64:
    supported = s.c.data_type == XVRAM_DATA_FP64 && compute == Compute::fp64;
    break;
  }
  if (!supported) return ProblemError::unsupported_type_combination;
  Bounds ab, bb, cb;
  if (!matrix_bounds(s.a, ab) || !matrix_bounds(s.b, bb) || !matrix_bounds(s.c, cb))
    return ProblemError::storage_overflow;
  const auto overlaps = [](const Bounds& l, const Bounds& r) {
    return l.begin < r.end && r.begin < l.end;
  };
  if ((s.a.allocation_id == s.c.allocation_id && overlaps(ab, cb)) ||
      (s.b.allocation_id == s.c.allocation_id && overlaps(bb, cb))) {
    who = 'C';
    return ProblemError::output_aliases_input;
  }
  return ProblemError::none;
}

// Reduces the problem to column-major C. A matrix stored row-major is the
// column-major storage of its transpose, so each operand's effective
// operation is op XOR (layout == row-major); a row-major C is handled as
// C^T = op(B)^T op(A)^T (the operand swap of src/gemm/executor.cpp:191-209).
CanonProblem canonicalize(const GemmSpec& s) {
  CanonProblem p;
  uint64_t m, n, k;
  problem_dims(s, m, n, k);
  const bool eop_a = (s.operation_a == XVRAM_MATRIX_OP_T) != (s.a.layout == XVRAM_MATRIX_ROW_MAJOR);
  const bool eop_b = (s.operation_b == XVRAM_MATRIX_OP_T) != (s.b.layout == XVRAM_MATRIX_ROW_MAJOR);
  const auto operand = [](const MatrixSpec& mx, bool transposed) {
    CanonOperand o;
    o.allocation_id = mx.allocation_id;
    o.base = mx.offset_bytes;
    o.ld = mx.leading_dimension;
    o.transposed = transposed;
    return o;
  };
  p.alpha = static_cast<float>(s.alpha);
  p.beta = static_cast<float>(s.beta);
  p.k = k;
  p.c = operand(s.c, false);
  if (s.c.layout == XVRAM_MATRIX_COLUMN_MAJOR) {
    p.m = m;
    p.n = n;
    p.a = operand(s.a, eop_a);
    p.b = operand(s.b, eop_b);
  } else {
    p.swapped = true;
    p.m = n;
    p.n = m;
    p.a = operand(s.b, !eop_b);
    p.b = operand(s.a, !eop_a);
  }
  const EpilogueSpec& ep = s.epilogue;
  if (ep.bias_axis != XVRAM_AMD_BIAS_NONE) {
    p.bias_allocation_id = ep.bias_allocation_id;
    p.bias_base = ep.bias_offset_bytes;
    // The caller's rows are C' columns when C was swapped.
    p.bias_rows = (ep.bias_axis == XVRAM_AMD_BIAS_PER_ROW) != p.swapped;
  }
  p.relu = ep.activation == XVRAM_AMD_ACTIVATION_RELU;
  return p;
}

Error validate_epilogue(const GemmSpec& s) {
  const EpilogueSpec& ep = s.epilogue;
  const auto bad = [](const char* message) {
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "epilogue", message);
  };
  if (ep.activation != XVRAM_AMD_ACTIVATION_NONE && ep.activation != XVRAM_AMD_ACTIVATION_RELU)
    return bad("unknown activation");
  if (ep.bias_axis == XVRAM_AMD_BIAS_NONE) {
    if (ep.bias_allocation_id != 0) return bad("a bias allocation needs a bias axis");
    return {};
  }
  if (ep.bias_axis != XVRAM_AMD_BIAS_PER_ROW && ep.bias_axis != XVRAM_AMD_BIAS_PER_COLUMN)
    return bad("unknown bias axis");
  if (ep.bias_allocation_id == 0) return bad("bias axis given without a bias allocation");
  if (ep.bias_offset_bytes % 4 != 0) return bad("bias offset must be 4-byte aligned");
  uint64_t m, n, k;
  problem_dims(s, m, n, k);
  const uint64_t length = ep.bias_axis == XVRAM_AMD_BIAS_PER_ROW ? m : n;
  uint64_t bytes = 0, end = 0;
  if (!checked_mul(length, 4, bytes) || !checked_add(ep.bias_offset_bytes, bytes, end) ||
      end > ep.bias_allocation_bytes)
    return bad("bias vector exceeds its allocation");
  if (ep.bias_allocation_id == s.c.allocation_id) {
    // Conservative: the bias must lie outside C's whole storage extent.
    const uint64_t c_lines = s.c.layout == XVRAM_MATRIX_COLUMN_MAJOR ? s.c.columns : s.c.rows;
    const uint64_t c_begin = s.c.offset_bytes;
    const uint64_t c_end = c_begin + (c_lines * s.c.leading_dimension) * 4;
    if (ep.bias_offset_bytes < c_end && c_begin < end) return bad("bias overlaps C");
  }
  return {};
}

// Panel planning. Tiles are sized so that each A, B and C panel fits one
// frame; C blocks (block_m x block_n tiles) stay resident across the whole K
// loop while A and B panels stream through the remaining frames, and the block
// shape minimises the scheduled H2D traffic
//   ceil(tiles_m/block_m)*|B| + ceil(tiles_n/block_n)*|A| (+|C| if beta != 0).
Error make_gemm_plan(const GemmSpec& spec, uint64_t frame_bytes, uint64_t total_frames,
                     uint32_t prefetch_distance, uint64_t max_launch_flops, GemmPlanData& out) {
  out = GemmPlanData{};
  CanonProblem p = canonicalize(spec);
  out.problem = p;
  // A bias vector stays pinned in one frame for the whole operation.
  const bool bias = p.bias_allocation_id != 0;
  if (bias && p.bias_length() * 4 > frame_bytes)
    return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "gemm", "make_plan",
                      "working_set_too_large: the bias vector exceeds one cache frame");
  uint64_t frame_count = total_frames - (bias && total_frames > 0 ? 1 : 0);
  if (frame_count < 3)
    return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "gemm", "make_plan",
                      "working_set_too_large: fewer than three cache frames");
  const uint64_t F = frame_bytes;
  uint64_t tm, tn, bk;
  const bool hinted = spec.tile_m_hint || spec.tile_n_hint || spec.tile_k_hint;
  const auto launch_flops = [](uint64_t a, uint64_t b, uint64_t c) {
    return 2.0 * static_cast<double>(a) * static_cast<double>(b) * static_cast<double>(c);
  };
  const bool over_cap = max_launch_flops != 0 &&
                        launch_flops(p.m, p.n, p.k) > static_cast<double>(max_launch_flops);
  // The 256 x 256 tile kernels address an A or B panel with 32-bit buffer
  // offsets (sgemm_wide.hip), so those panels stay below 2^31 bytes; a larger
  // one would fall back to the slower 256 x 128 kernel.
  constexpr uint64_t kPanelLimit = uint64_t(1) << 31;
  if (!hinted && !over_cap && a_panel_bytes(p, p.m, p.k) <= F && b_panel_bytes(p, p.k, p.n) <= F &&
      c_panel_bytes(p.m, p.n) <= F && a_panel_bytes(p, p.m, p.k) < kPanelLimit &&
      b_panel_bytes(p, p.k, p.n) < kPanelLimit) {
    tm = p.m;
    tn = p.n;
    bk = p.k;
  } else {
    // Start from the largest power of two whose square panel fits a frame:
    // such extents divide the usual problem sizes (no ragged last tile of a
    // 65536 extent, as 11520 would leave), and the growth step below then
    // spends the rest of the frame on a deeper K panel (fewer launches, and
    // fewer passes of each C tile through HBM).
    // An 8192 x 8192 C tile is already 1024 workgroups of the 256 x 256
    // kernel (four per CU): a wider start adds nothing to the kernel, so larger
    // frames go to K instead (below).
    constexpr uint64_t kMaxSquare = 8192;
    uint64_t s = 16;
    while ((s * 2) * (s * 2) <= F / 4) s *= 2;
    s = std::min(s, kMaxSquare);
    tm = std::min(p.m, s);
    tn = std::min(p.n, s);
    bk = std::min(p.k, s);
    // Hints are given for the caller's m/n (swapped when C is row-major).
    const uint64_t hm = p.swapped ? spec.tile_n_hint : spec.tile_m_hint;
    const uint64_t hn = p.swapped ? spec.tile_m_hint : spec.tile_n_hint;
    if (hm) tm = std::min(p.m, hm);
    if (hn) tn = std::min(p.n, hn);
    if (spec.tile_k_hint) bk = std::min(p.k, spec.tile_k_hint);
    const auto fits = [&](uint64_t a, uint64_t b, uint64_t c) {
      return a_panel_bytes(p, a, c) <= F && b_panel_bytes(p, c, b) <= F && c_panel_bytes(a, b) <= F &&
             a_panel_bytes(p, a, c) < kPanelLimit && b_panel_bytes(p, c, b) < kPanelLimit;
    };
    // Shrink the largest extent until every panel fits a frame.
    while (!fits(tm, tn, bk)) {
      uint64_t* largest = &tm;
      if (tn > *largest) largest = &tn;
      if (bk > *largest) largest = &bk;
      if (*largest <= 16) {
        return make_error(XVRAM_STATUS_BUDGET_PRESSURE, "gemm", "make_plan",
                          "working_set_too_large: no tile fits one cache frame");
      }
      *largest = std::max<uint64_t>(16, *largest / 2 / 16 * 16);
    }
    // Grow extents the problem did not clamp while the panels still fit: K
    // first (each doubling halves the passes of a C tile through HBM and the
    // launches' fixed costs), then the tile extents.
    if (!hinted) {
      while (bk < p.k && fits(tm, tn, std::min(p.k, bk * 2))) bk = std::min(p.k, bk * 2);
      bool grew = true;
      while (grew) {
        grew = false;
        if (bk < p.k && fits(tm, tn, std::min(p.k, bk * 2))) {
          bk = std::min(p.k, bk * 2);
          grew = true;
        }
        if (tm < p.m && fits(std::min(p.m, tm * 2), tn, bk)) {
          tm = std::min(p.m, tm * 2);
          grew = true;
        }
        if (tn < p.n && fits(tm, std::min(p.n, tn * 2), bk)) {
          tn = std::min(p.n, tn * 2);
          grew = true;
        }
      }
    }
    // Keep every launch well inside the transaction duration guard: split K
    // first (the C tile stays resident across K panels), then the larger of
    // the tile extents.
    while (max_launch_flops != 0 &&
           launch_flops(tm, tn, bk) > static_cast<double>(max_launch_flops)) {
      uint64_t* cut = bk > 2048 ? &bk : (tm >= tn ? &tm : &tn);
      if (*cut <= 256) break; // a launch this small cannot approach any guard
      *cut = std::max<uint64_t>(256, *cut / 2 / 16 * 16);
    }
  }
  out.tm = tm;
  out.tn = tn;
  out.bk = bk;
  out.tiles_m = ceil_div(p.m, tm);
  out.tiles_n = ceil_div(p.n, tn);
  out.panels_k = ceil_div(p.k, bk);
  // A launch that leaves workgroup slots idle splits its K (or its tail
  // rows' K, or that of the parts of its edge split, or of the first part of
  // its K remainder), its partials in one frame of the pool
  // (kernels::split_k_shape, tail_split_shape, edge_split_wants_workspace and
  // k_remainder_wants_workspace for the plan's tile and panel; its panels are
  // below 2^31 bytes): that frame is taken from the schedule's.
  {
    const int64_t sm = static_cast<int64_t>(tm), sn = static_cast<int64_t>(tn),
                  sk = static_cast<int64_t>(bk);
    const bool nt_form = !p.a.transposed && p.b.transposed;
    out.scratch = frame_count >= 4 &&
                  (kernels::split_k_shape(sm, sn, sk, nt_form, true, F).splits > 1 ||
                   kernels::tail_split_shape(sm, sn, sk, nt_form, true, F).head_m > 0 ||
                   kernels::edge_split_wants_workspace(sm, sn, sk, nt_form) ||
                   kernels::k_remainder_wants_workspace(sm, sn, sk, nt_form));
  }
  if (out.scratch) --frame_count;

  // Lookahead: launches whose panels are acquired (and pinned) before they are
  // enqueued, so copies run ahead of compute. At most 3 frames per one-panel
  // launch are pinned, so keep 3*(lookahead+1) below the frame count (a
  // two-panel launch pins 5 and gets half the lookahead: 5*(lookahead/2+1)
  // stays below it too).
  uint32_t lookahead = std::max<uint32_t>(2, 2 * prefetch_distance);
  lookahead = static_cast<uint32_t>(
      std::min<uint64_t>(lookahead, frame_count >= 6 ? frame_count / 3 - 1 : 0));

  // Block search for `panels` K panels per launch: the block's C tiles, the
  // pass's A and B panels and the frames the lookahead brings in ahead
  // (`ahead` launches); the block minimising the scheduled H2D traffic wins.
  const uint64_t a_bytes = p.m * p.k * 4, b_bytes = p.k * p.n * 4, c_bytes = p.m * p.n * 4;
  struct Block {
    uint64_t gm = 1, gn = 1, h2d = UINT64_MAX, need = 0;
  };
  const auto search = [&](uint64_t panels, uint64_t ahead) {
    Block best;
    for (uint64_t gm = 1; gm <= out.tiles_m; ++gm) {
      for (uint64_t gn = 1; gn <= out.tiles_n; ++gn) {
        const uint64_t need = gm * gn + panels * (gm + gn) + 2ull * ahead;
        if (need > frame_count && !(gm == 1 && gn == 1)) continue;
        const uint64_t h2d = ceil_div(out.tiles_m, gm) * b_bytes +
                             ceil_div(out.tiles_n, gn) * a_bytes + (p.beta != 0.f ? c_bytes : 0);
        if (h2d < best.h2d || (h2d == best.h2d && gm * gn > best.gm * best.gn))
          best = Block{gm, gn, h2d, need};
      }
    }
    return best;
  };
  Block best = search(1, lookahead);
  // Two K panels per launch: the launch is twice as long, so half the
  // lookahead covers the same time. Taken only where the two-panel kernel
  // applies to every launch (no ragged tiles or panels) and the schedule's H2D
  // traffic does not grow. The frames must hold the block, both panels of
  // every A and B of a pass and two new frames per launch acquired ahead; the
  // executor keeps the panels of the coming pass out of victim selection
  // (Runtime::set_protected), without which such a tight budget evicted panels
  // before their last use (32768^3 under 2 GiB of 64 MiB frames: 23 % more H2D).
  // Not with a partials frame: a launch whose tiles leave a last round mostly
  // idle gains more from a tail split than from a second panel.
  uint32_t panels = 1;
  const double one_panel_flops = launch_flops(tm, tn, bk);
  const bool nt = !p.a.transposed && p.b.transposed;
  const bool two_panel_kernel = tm % 256 == 0 && tn % 256 == 0 &&
                                (tm / 256) * (tn / 256) >= 256 && p.m % tm == 0 &&
                                p.n % tn == 0 && bk % 32 == 0 && p.k % (nt ? 4 : 8) == 0 &&
                                out.panels_k >= 2 && !out.scratch;
  if (two_panel_kernel && one_panel_flops <= kTwoPanelMaxFlops &&
      (max_launch_flops == 0 || 2.0 * one_panel_flops <= static_cast<double>(max_launch_flops))) {
    const uint32_t ahead2 = std::max<uint32_t>(1, lookahead / 2);
    const Block two = search(2, ahead2);
    if (two.need <= frame_count && two.h2d <= best.h2d) {
      best = two;
      panels = 2;
      lookahead = ahead2;
    }
  }
  const uint64_t best_gm = best.gm, best_gn = best.gn;
  out.block_m = best_gm;
  out.block_n = best_gn;
  out.panels_per_launch = panels;
  if (best.need > frame_count) {
    // Only the 1 x 1 block is possible: shrink the lookahead to fit.
    const uint64_t spare = frame_count > 3 ? frame_count - 3 : 0;
    lookahead = static_cast<uint32_t>(std::min<uint64_t>(lookahead, spare / 3));
    best.need = 3 + 2ull * lookahead;
  }
  out.lookahead = lookahead;
  out.h2d_bytes_planned = best.h2d;
  out.d2h_bytes_planned = c_bytes;
  // The block's C tiles, one pass's A and B panels and the launches acquired
  // ahead (and the bias frame).
  out.frames_in_use =
      std::min<uint64_t>(total_frames, best.need + (bias ? 1 : 0) + (out.scratch ? 1 : 0));

  // Launch order: blocks in a serpentine; K passes (groups of `panels` K
  // panels, fixed boundaries) alternate direction from block to block so the
  // panels loaded last are the first needed next; inside a pass, tiles row by
  // row so each A panel serves consecutive launches.
  const uint64_t blocks_m = ceil_div(out.tiles_m, best_gm);
  const uint64_t blocks_n = ceil_div(out.tiles_n, best_gn);
  const uint64_t passes = ceil_div(out.panels_k, panels);
  uint64_t total = 0;
  if (!checked_mul(out.tiles_m, out.tiles_n, total) || !checked_mul(total, out.panels_k, total) ||
      total > 100000000ull)
    return make_error(XVRAM_STATUS_INVALID_ARGUMENT, "gemm", "make_plan", "too_many_tiles");
  out.launches.reserve(total);
  // A split launch fills the chip by itself, and its partials' frame serves
  // one launch at a time: one lane.
  out.lanes = !out.scratch && panels * one_panel_flops <= kDualLaneMaxFlops ? 2 : 1;
  uint64_t block_seq = 0;
  for (uint64_t bi = 0; bi < blocks_m; ++bi) {
    for (uint64_t s = 0; s < blocks_n; ++s, ++block_seq) {
      const uint64_t bj = (bi % 2 == 0) ? s : blocks_n - 1 - s;
      const uint64_t i_begin = bi * best_gm, i_end = std::min(out.tiles_m, i_begin + best_gm);
      const uint64_t j_begin = bj * best_gn, j_end = std::min(out.tiles_n, j_begin + best_gn);
      const bool forward = block_seq % 2 == 0;
      for (uint64_t q = 0; q < passes; ++q) {
        const uint64_t pass = forward ? q : passes - 1 - q;
        const uint64_t kp = pass * panels;
        const uint64_t in_pass = std::min<uint64_t>(panels, out.panels_k - kp);
        // The operation's first pass fills the cache with every panel it
        // uses, so the link sets its pace: one panel per launch there needs
        // half the new bytes per launch (a two-panel head left the kernels
        // idle 2.7 ms longer per 32768^3 operation), so it runs as one-panel
        // passes.
        const uint64_t split = (block_seq == 0 && q == 0) ? in_pass : 1;
        for (uint64_t sub = 0; sub < split; ++sub) {
          for (uint64_t i = i_begin; i < i_end; ++i) {
            for (uint64_t j = j_begin; j < j_end; ++j) {
              TileLaunch l;
              l.ti = static_cast<uint32_t>(i);
              l.tj = static_cast<uint32_t>(j);
              l.kp = static_cast<uint32_t>(kp + sub);
              l.panels = static_cast<uint8_t>(split > 1 ? 1 : in_pass);
              l.first_panel = q == 0 && sub == 0;
              l.last_panel = q + 1 == passes && sub + 1 == split;
              l.evict_c = l.last_panel && block_seq + 1 < blocks_m * blocks_n;
              // Consecutive launches in a pass are different C tiles of the
              // block: alternate lanes by the tile's place in the block.
              const uint64_t place = (i - i_begin) * (j_end - j_begin) + (j - j_begin);
              l.lane = static_cast<uint8_t>(out.lanes > 1 ? place % 2 : 0);
              out.launches.push_back(l);
            }
          }
        }
      }
    }
  }
  return {};
}

namespace {

struct Acquired {
  size_t index = 0;
  Frame* a[2] = {nullptr, nullptr}; // one A and one B frame per K panel of the launch
  Frame* b[2] = {nullptr, nullptr};
  Frame* c = nullptr;
  uint64_t slice = 0;                        // K depth of each slice; 0 = unsliced
  std::vector<Event> a_ready[2], b_ready[2]; // per-slice fill events (empty: whole panel)
};

// The first launch of an operation waits for its whole A and B panels before
// any compute can start (37.7 ms for two 1 GiB panels at 57 GB/s). It runs as
// one kernel per K slice of at least this depth (at most kFirstSlices per
// panel); a missing panel is filled by one copy per slice and each kernel
// waits only for its own slices of A and B, so compute starts after the first
// slices land and runs under the rest of the fill. The slicing is part of the
// plan, not of the cache state: a first launch whose panels are cached runs
// the same slices (without waits), so C is bit-identical whichever panels a
// previous operation left behind.
constexpr uint64_t kFirstSliceMin = 2048;
constexpr uint64_t kFirstSlices = 8;

// The K slices of a panel as copy pieces: K runs along its lines (op-N A,
// op-T B) or within them (op-T A, op-N B).
std::vector<PanelPiece> k_slices(const PanelGeom& g, bool k_within_lines, uint64_t slice) {
  std::vector<PanelPiece> out;
  const uint64_t depth = k_within_lines ? g.xn : g.yn;
  for (uint64_t k0 = 0; k0 < depth; k0 += slice) {
    const uint64_t d = std::min(slice, depth - k0);
    if (k_within_lines) out.push_back(PanelPiece{0, g.yn, k0 * 4, d * 4});
    else out.push_back(PanelPiece{k0, d, 0, g.xn * 4});
  }
  return out;
}

// A launch's C tile and its K panels: panel t covers K rows [p0[t], p0[t] + w[t]).
struct LaunchGeom {
  uint64_t i0, h, j0, g;
  uint32_t panels;
  uint64_t p0[2], w[2];
};

LaunchGeom launch_geom(const GemmPlanData& plan, const TileLaunch& l) {
  const CanonProblem& p = plan.problem;
  LaunchGeom g;
  g.i0 = l.ti * plan.tm;
  g.h = std::min(plan.tm, p.m - g.i0);
  g.j0 = l.tj * plan.tn;
  g.g = std::min(plan.tn, p.n - g.j0);
  g.panels = l.panels;
  for (uint32_t t = 0; t < 2; ++t) {
    g.p0[t] = (static_cast<uint64_t>(l.kp) + t) * plan.bk;
    g.w[t] = t < l.panels ? std::min(plan.bk, p.k - g.p0[t]) : 0;
  }
  return g;
}

// One tile-kernel dispatch of a launch: K rows [k0, k0 + depth) of panel
// `panel`, or both panels of a two-panel launch (two == true).
struct KernelPiece {
  uint32_t panel = 0;
  uint64_t k0 = 0, depth = 0;
  bool two = false;
  int slice = -1; // index into the per-slice ready events, -1 = none
};

} // namespace

// Pipelined execution. Panels of the next `lookahead` launches are acquired
// (H2D copies queued on the copy stream) before each launch is enqueued on the
// compute stream; the compute stream waits on the fill events of the launch's
// frames; the launch's stop event, recorded by its dispatch, becomes the
// retire event of those frames. A C tile of any block but the last is written
// back on the D2H stream and evicted as soon as its last K pass is enqueued
// (the next block needs the frame); the last block's tiles stay resident and
// dirty after the operation (write-back cache). The host blocks only when a
// frame it wants to refill still has an unretired consumer. A launch over two
// K panels runs as one dispatch of the two-panel kernel when that kernel's
// contract holds (the planner only makes such launches), else as one
// dispatch per panel.
Error execute_gemm(Runtime& rt, const GemmPlanData& plan, uint64_t operation_id,
                   const GemmHooks& hooks) {
  const CanonProblem& p = plan.problem;
  if (Error e = rt.begin_operation()) return e;
  if (Error e = rt.make_room(plan.frames_in_use)) {
    (void)rt.finish_operation(operation_id);
    return e;
  }
  std::deque<Acquired> window;
  size_t next = 0;
  const size_t total = plan.launches.size();

  // The bias vector, when there is one, is one panel pinned for the whole
  // operation; tile launches index it at their first C' row or column.
  Frame* bias = nullptr;
  if (p.bias_allocation_id != 0) {
    PanelKey key;
    key.allocation_id = p.bias_allocation_id;
    key.offset = p.bias_base;
    key.width = p.bias_length() * 4;
    key.height = 1;
    key.pitch = key.width;
    Error e = rt.acquire(key, round_up(key.width, 16), true, bias);
    for (int lane = 0; !e && lane < plan.lanes; ++lane)
      e = rt.wait_ready(*bias, rt.compute_stream(lane));
    if (e) {
      if (bias) (void)rt.release_after(*bias, rt.compute_stream(), false);
      (void)rt.finish_operation(operation_id);
      return e;
    }
  }

  // Split launches keep their partials in one frame taken for the operation.
  Frame* scratch = nullptr;
  if (plan.scratch) {
    if (Error e = rt.take_scratch(scratch)) {
      if (bias) (void)rt.release_after(*bias, rt.compute_stream(), false);
      (void)rt.finish_operation(operation_id);
      return e;
    }
  }
  const auto release_scratch = [&]() -> Error {
    Frame* f = scratch;
    scratch = nullptr;
    return f ? rt.release_scratch(*f) : Error{};
  };

  // Unpins what an acquisition already holds (its launch never runs).
  const auto drop = [&](Acquired& acq) {
    Stream cs = rt.compute_stream();
    for (Frame* f : {acq.c, acq.a[0], acq.b[0], acq.a[1], acq.b[1]})
      if (f) (void)rt.release_after(*f, cs, false);
  };

  // The panels (and C tiles) of launches idx .. idx + one pass of a block:
  // everything the schedule uses again before a pass goes by, which victim
  // selection then passes over while it has another choice (a tight budget
  // would otherwise evict a panel the pass still needs and load it again).
  const size_t horizon = std::max<uint64_t>(1, plan.block_m * plan.block_n);
  const auto protect_from = [&](size_t idx) {
    std::vector<PanelKey> keys;
    const size_t end = std::min(total, idx + horizon);
    keys.reserve((end - idx) * 5);
    for (size_t i = idx; i < end; ++i) {
      const LaunchGeom g = launch_geom(plan, plan.launches[i]);
      keys.push_back(panel_key(p.c, c_geom(g.i0, g.h, g.j0, g.g)));
      for (uint32_t t = 0; t < g.panels; ++t) {
        keys.push_back(panel_key(p.a, a_geom(p.a, g.i0, g.h, g.p0[t], g.w[t])));
        keys.push_back(panel_key(p.b, b_geom(p.b, g.p0[t], g.w[t], g.j0, g.g)));
      }
    }
    rt.set_protected(std::move(keys));
  };

  const auto acquire_launch = [&](size_t idx) -> Error {
    // Sample the live budget (rate-limited) before each launch's panels.
    if (Error e = rt.refresh_budget(3, 0, false)) return e;
    protect_from(idx);
    const TileLaunch& l = plan.launches[idx];
    const LaunchGeom g = launch_geom(plan, l);
    Acquired acq;
    acq.index = idx;
    const PanelGeom cg = c_geom(g.i0, g.h, g.j0, g.g);
    const bool c_needs_data = !l.first_panel || p.beta != 0.f;
    if (idx == 0 && plan.launches.size() > 1 && g.w[0] >= 2 * kFirstSliceMin)
      acq.slice = std::max(kFirstSliceMin, round_up(ceil_div(g.w[0], kFirstSlices), 16));
    if (Error e = rt.acquire(panel_key(p.c, cg), packed_ld(cg) * 4, c_needs_data, acq.c)) return e;
    // A hit (or an unsliced launch) leaves the per-slice event lists empty.
    const auto operand = [&](const CanonOperand& op, const PanelGeom& pg, bool k_within,
                             Frame*& out, std::vector<Event>& ready) -> Error {
      if (!acq.slice) return rt.acquire(panel_key(op, pg), packed_ld(pg) * 4, true, out);
      return rt.acquire_pieces(panel_key(op, pg), packed_ld(pg) * 4,
                               k_slices(pg, k_within, acq.slice), out, ready);
    };
    for (uint32_t t = 0; t < g.panels; ++t) {
      const PanelGeom ag = a_geom(p.a, g.i0, g.h, g.p0[t], g.w[t]);
      const PanelGeom bg = b_geom(p.b, g.p0[t], g.w[t], g.j0, g.g);
      Error e = operand(p.a, ag, p.a.transposed, acq.a[t], acq.a_ready[t]);
      if (!e) e = operand(p.b, bg, !p.b.transposed, acq.b[t], acq.b_ready[t]);
      if (e) {
        drop(acq);
        return e;
      }
    }
    window.push_back(std::move(acq));
    return {};
  };

  Error result;
  uint64_t tiles_done = 0; // C tiles x K panels enqueued so far (progress units)
  for (size_t idx = 0; idx < total && !result; ++idx) {
    if (hooks.boundary) {
      if (Error e = hooks.boundary("before_tile")) {
        result = e;
        break;
      }
    }
    while (next <= idx) {
      if (Error e = acquire_launch(next++)) {
        result = e;
        break;
      }
    }
    if (result) break;
    Acquired acq = std::move(window.front());
    window.pop_front();
    const TileLaunch& l = plan.launches[idx];
    const LaunchGeom g = launch_geom(plan, l);
    const PanelGeom cg = c_geom(g.i0, g.h, g.j0, g.g);
    const int lane = l.lane;
    Stream cs = rt.compute_stream(lane);
    // Whole-panel fills are waited for up front; sliced ones slice by slice.
    if (Error e = rt.wait_ready(*acq.c, cs)) { result = e; break; }
    for (uint32_t t = 0; t < g.panels && !result; ++t) {
      if (acq.a_ready[t].empty())
        if (Error e = rt.wait_ready(*acq.a[t], cs)) result = e;
      if (!result && acq.b_ready[t].empty())
        if (Error e = rt.wait_ready(*acq.b[t], cs)) result = e;
    }
    if (result) break;
    // Packed leading dimensions of panel t (a K-within-lines panel's depends
    // on its depth; both panels of a two-panel dispatch share theirs).
    const auto lda_of = [&](uint32_t t) {
      return static_cast<int64_t>(packed_ld(a_geom(p.a, g.i0, g.h, g.p0[t], g.w[t])));
    };
    const auto ldb_of = [&](uint32_t t) {
      return static_cast<int64_t>(packed_ld(b_geom(p.b, g.p0[t], g.w[t], g.j0, g.g)));
    };
    // The dispatches of this launch: K slices of each panel (sliced fill),
    // one two-panel dispatch, or one dispatch per panel.
    std::vector<KernelPiece> pieces;
    const bool nt = !p.a.transposed && p.b.transposed;
    const bool two_ok = g.panels == 2 && !acq.slice && g.h % 256 == 0 && g.g % 256 == 0 &&
                        (g.h / 256) * (g.g / 256) >= 256 && g.w[0] % 32 == 0 &&
                        (g.w[0] + g.w[1]) % (nt ? 4 : 8) == 0 && lda_of(0) == lda_of(1) &&
                        ldb_of(0) == ldb_of(1);
    if (two_ok) {
      pieces.push_back(KernelPiece{0, 0, g.w[0] + g.w[1], true, -1});
    } else {
      for (uint32_t t = 0; t < g.panels; ++t) {
        // A sliced launch runs every panel slice by slice (waiting on the
        // slices of those filled in pieces); an unsliced one panel by panel.
        const bool waits = !acq.a_ready[t].empty() || !acq.b_ready[t].empty();
        const uint64_t depth = acq.slice ? acq.slice : g.w[t];
        for (uint64_t k0 = 0, s = 0; k0 < g.w[t]; k0 += depth, ++s)
          pieces.push_back(KernelPiece{t, k0, std::min(depth, g.w[t] - k0), false,
                                       waits ? static_cast<int>(s) : -1});
      }
    }
    Event done = nullptr;
    for (size_t n = 0; n < pieces.size() && !result; ++n) {
      const KernelPiece& kp = pieces[n];
      const uint32_t t = kp.panel;
      if (kp.slice >= 0) {
        for (const std::vector<Event>* ready : {&acq.a_ready[t], &acq.b_ready[t]}) {
          if (ready->empty()) continue;
          if (Error e = rt.stream_wait(cs, (*ready)[kp.slice], (*ready)[kp.slice])) {
            result = e;
            break;
          }
        }
        if (result) break;
      }
      // K rows k0.. of a packed panel: whole lines (op-N A: A(i,p) = a[i + p*lda];
      // op-T B: B(p,j) = b[j + p*ldb]) or a column range of every line.
      const float* a = reinterpret_cast<const float*>(acq.a[t]->address);
      const float* b = reinterpret_cast<const float*>(acq.b[t]->address);
      const int64_t lda = lda_of(t), ldb = ldb_of(t);
      kernels::SgemmLaunch k;
      k.a = a + (p.a.transposed ? kp.k0 : kp.k0 * lda);
      k.b = b + (p.b.transposed ? kp.k0 * ldb : kp.k0);
      if (kp.two) {
        k.a2 = reinterpret_cast<const float*>(acq.a[1]->address);
        k.b2 = reinterpret_cast<const float*>(acq.b[1]->address);
        k.k_split = static_cast<int>(g.w[0]);
      }
      k.c = reinterpret_cast<float*>(acq.c->address);
      k.lda = lda;
      k.ldb = ldb;
      k.ldc = static_cast<int64_t>(packed_ld(cg));
      k.m = static_cast<int>(g.h);
      k.n = static_cast<int>(g.g);
      k.k = static_cast<int>(kp.depth);
      k.alpha = p.alpha;
      k.beta = (n == 0 && l.first_panel) ? p.beta : 1.f;
      if (scratch) {
        k.workspace = reinterpret_cast<float*>(scratch->address);
        k.workspace_bytes = rt.frame_bytes();
      }
      k.a_kcontig = p.a.transposed;
      k.b_ncontig = p.b.transposed;
      k.padded = true;
      if (l.last_panel && n + 1 == pieces.size() && p.has_epilogue()) {
        if (bias) {
          const float* v = reinterpret_cast<const float*>(bias->address);
          if (p.bias_rows) k.bias_row = v + g.i0;
          else k.bias_col = v + g.j0;
        }
        k.relu = p.relu;
      }
      // The launch's stop event is recorded by its dispatch (its start is
      // derived from the events it follows: Runtime::record_kernel); the last
      // dispatch's stop event is also the retire event of the launch's frames
      // (each marker packet between kernels would otherwise cost the compute
      // stream a few microseconds).
      TraceInterval iv;
      iv.kind = 'k';
      if (Error e = rt.record_kernel(iv, lane)) {
        result = e;
        break;
      }
      k.start_event = iv.start;
      k.stop_event = iv.stop;
      if (int rc = rt.device().launch_sgemm(k, cs)) {
        result = rt.device_failure(rc, "gemm", "launch_tile");
        break;
      }
      rt.trace_push(iv);
      done = iv.stop;
    }
    if (result) break;
    // Sliced fills: settle the entries' state (their whole-panel ready events
    // completed no later than the last slices, which the stream already waits for).
    for (uint32_t t = 0; t < g.panels && !result; ++t) {
      if (!acq.a_ready[t].empty())
        if (Error e = rt.wait_ready(*acq.a[t], cs)) result = e;
      if (!result && !acq.b_ready[t].empty())
        if (Error e = rt.wait_ready(*acq.b[t], cs)) result = e;
    }
    if (result) break;
    rt.note_kernel_launched(g.panels); // one retired tile per K panel, however many dispatches
    for (uint32_t t = 0; t < g.panels && !result; ++t) {
      if (Error e = rt.release_after_event(*acq.a[t], done, false, lane)) result = e;
      else if (Error e2 = rt.release_after_event(*acq.b[t], done, false, lane)) result = e2;
    }
    if (result) break;
    if (Error e = rt.release_after_event(*acq.c, done, true, lane)) { result = e; break; }
    if (l.evict_c) {
      if (Error e = rt.writeback_and_evict(*acq.c)) {
        result = e;
        break;
      }
    }
    tiles_done += l.panels;
    if (hooks.progress) hooks.progress(tiles_done, plan.tiles_m * plan.tiles_n * plan.panels_k);
    while (next < total && next <= idx + plan.lookahead) {
      if (Error e = acquire_launch(next++)) {
        result = e;
        break;
      }
    }
  }
  if (bias && !result) result = rt.release_after_lanes(*bias);
  if (Error e = release_scratch(); e && !result) result = e;
  if (!result && hooks.tail) result = hooks.tail();
  if (result) {
    // Unpin what was acquired ahead, drop partial C panels, drain the device.
    rt.discard_dirty();
    (void)rt.finish_operation(operation_id);
    return result;
  }
  return rt.finish_operation(operation_id);
}

Error carry_gemm_head(Runtime& rt, const GemmPlanData& plan, uint64_t launches) {
  const CanonProblem& p = plan.problem;
  const auto carry = [&](const PanelKey& key, uint64_t pitch, bool& stop) -> Error {
    bool issued = false;
    Error e = rt.carry_fill(key, pitch, issued);
    if (e && e.status == XVRAM_STATUS_BUDGET_PRESSURE) {
      stop = true; // every frame is pinned: nothing more can be carried
      return {};
    }
    return e;
  };
  bool stop = false;
  if (p.bias_allocation_id != 0) {
    PanelKey key;
    key.allocation_id = p.bias_allocation_id;
    key.offset = p.bias_base;
    key.width = p.bias_length() * 4;
    key.height = 1;
    key.pitch = key.width;
    if (Error e = carry(key, round_up(key.width, 16), stop)) return e;
  }
  const uint64_t n = std::min<uint64_t>(launches, plan.launches.size());
  for (uint64_t idx = 0; idx < n && !stop; ++idx) {
    const LaunchGeom g = launch_geom(plan, plan.launches[idx]);
    for (uint32_t t = 0; t < g.panels && !stop; ++t) {
      const PanelGeom ag = a_geom(p.a, g.i0, g.h, g.p0[t], g.w[t]);
      const PanelGeom bg = b_geom(p.b, g.p0[t], g.w[t], g.j0, g.g);
      if (Error e = carry(panel_key(p.a, ag), packed_ld(ag) * 4, stop)) return e;
      if (stop) break;
      if (Error e = carry(panel_key(p.b, bg), packed_ld(bg) * 4, stop)) return e;
    }
  }
  return {};
}

} // namespace xvram
