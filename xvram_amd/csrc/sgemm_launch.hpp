// sgemm_launch.hpp — host-side description of one tile-kernel launch.
//
// C (m x n, column-major, ldc) = alpha * op(A) * op(B) + beta * C, where
//   a_kcontig == false: A(i,p) = a[i + p*lda]   (op N on a column-major A)
//   a_kcontig == true : A(i,p) = a[p + i*lda]   (op T)
//   b_ncontig == false: B(p,j) = b[p + j*ldb]   (op N)
//   b_ncontig == true : B(p,j) = b[j + p*ldb]   (op T)
// beta == 0 means C is not read. Optional epilogue, applied after the beta
// term: + bias_row[i] (per row of C), + bias_col[j] (per column), then ReLU
// (negative values become 0; NaN is kept). The kernel requires 16-byte aligned bases,
// leading dimensions that are multiples of 4 floats and `padded` = true (every
// line may be read as whole 16-byte vectors up to its leading dimension), which
// frame-packed panels always satisfy; anything else returns hipErrorInvalidValue.
//
// Two K panels (optional): with a2 / b2 set, k rows [0, k_split) of op(A) and
// op(B) come from a / b and rows [k_split, k) from a2 / b2 (same leading
// dimensions): one launch over two separately stored panels. Only for m and n
// multiples of 256 with at least 256 tiles of 256 x 256, k a multiple of 4
// (N/T: a_kcontig false, b_ncontig true) or of 8 (the other forms), k_split a
// multiple of 32 inside (0, k), 16-byte aligned a2 / b2 and each operand panel
// spanning less than 2^31 bytes from its base (two_panel_valid below);
// anything else returns hipErrorInvalidValue.
//
// Split K (optional, workspace set): a launch that would leave CUs idle may
// cut its K into ranges (split_k_plan below), one workgroup per tile and
// range; each stores the raw partial sums of its range to the workspace
// (`splits` column-major m x n matrices, leading dimension m rounded up to 4,
// split_partial_ld), and a second kernel adds them in range order and applies
// alpha, beta and the epilogue. Launches whose tiles are all interior 256 x
// 256 tiles (m and n multiples of 256, K a multiple of 4 for N/T and of 8 for
// the other forms) split on the ring kernels when they have fewer tiles than
// the chip has CUs; other launches with fewer than 256 tiles of 256 x 256
// split on the 256 x 128 kernel (two workgroups per CU) when they have fewer
// of its tiles than it has slots. The order of the additions is fixed, so C
// is the same from run to run. Without a workspace large enough for two
// partials the launch runs unsplit. One K panel only.
//
// start_event / stop_event (hipEvent_t, optional) are recorded by the dispatch
// itself (hipExtLaunchKernelGGL): no separate marker packets run between
// kernels, and stop_event completes when the kernel does, so it can serve as
// the retire event of every panel the launch reads or writes. A start event
// costs the dispatch ~16 us of host time and ~5 us of device time; the
// executor passes none and derives starts from the events a launch follows.
#pragma once

#include <cstdint>

namespace xvram::kernels {

struct SgemmLaunch {
  const float* a = nullptr;
  const float* b = nullptr;
  float* c = nullptr;
  int64_t lda = 0, ldb = 0, ldc = 0;
  int m = 0, n = 0, k = 0;
  float alpha = 1.f, beta = 0.f;
  bool a_kcontig = false;
  bool b_ncontig = false;
  bool padded = false;
  const float* bias_row = nullptr;
  const float* bias_col = nullptr;
  bool relu = false;
  const float* a2 = nullptr;
  const float* b2 = nullptr;
  int k_split = 0;
  void* start_event = nullptr;
  void* stop_event = nullptr;
  float* workspace = nullptr; // split-K partials (16-byte aligned), nullptr = none
  uint64_t workspace_bytes = 0;
};

// MI355X: 256 compute units; a launch with fewer tiles than this leaves CUs
// idle unless its K is split.
constexpr int64_t kComputeUnits = 256;
// K per workgroup of a split launch, at least (a range this deep keeps the
// ring kernels' prologue and the partial's store small next to its MFMA work).
constexpr int64_t kSplitMinDepth = 256;

struct SplitK {
  int splits = 1;      // 1 = not split
  int depth = 0;       // K per range (multiple of 32); the last range holds the rest
  bool narrow = false; // the ranges run on the 256 x 128 kernel (else the ring kernels)
};

// Leading dimension of a split launch's partials: m rounded up to 4 floats,
// so every column starts 16-byte aligned.
inline int64_t split_partial_ld(int64_t m) { return (m + 3) / 4 * 4; }

// The split of an m x n x k launch of form `nt` (A op N, B op T) or not,
// given a workspace of `workspace_bytes` (see "Split K" above): as many ranges
// as fill the chip's workgroup slots, each at least kSplitMinDepth deep, at
// most as many partials as the workspace holds. `ring` = the ring kernels can
// address the operand panels (each spans less than 2^31 bytes).
inline SplitK split_k_shape(int64_t m, int64_t n, int64_t k, bool nt, bool ring,
                            uint64_t workspace_bytes) {
  if (m <= 0 || n <= 0 || k <= 0) return {};
  const bool interior = ring && m % 256 == 0 && n % 256 == 0 && k % (nt ? 4 : 8) == 0;
  int64_t tiles = 0, slots = 0;
  if (interior) {
    tiles = (m / 256) * (n / 256);
    slots = kComputeUnits;
  } else {
    // At least one 256 x 256 tile per CU runs a 256 x 256 kernel unsplit.
    if (((m + 255) / 256) * ((n + 255) / 256) >= kComputeUnits) return {};
    tiles = ((m + 255) / 256) * ((n + 127) / 128);
    slots = 2 * kComputeUnits;
  }
  if (tiles >= slots) return {};
  const int64_t partial = split_partial_ld(m) * n * 4;
  int64_t s = slots / tiles;
  if (k / kSplitMinDepth < s) s = k / kSplitMinDepth;
  if (static_cast<int64_t>(workspace_bytes / partial) < s)
    s = static_cast<int64_t>(workspace_bytes / partial);
  if (s < 2) return {};
  const int64_t depth = (k + s - 1) / s;
  const int64_t depth32 = (depth + 31) / 32 * 32;
  const int64_t splits = (k + depth32 - 1) / depth32;
  if (splits < 2) return {};
  return SplitK{static_cast<int>(splits), static_cast<int>(depth32), !interior};
}

// The split a launch takes given room for `workspace_bytes` of partials: none
// for a two-panel launch, else split_k_shape (on the ring kernels only when
// each operand panel spans less than 2^31 bytes, their 32-bit buffer offsets).
inline SplitK split_k_for(const SgemmLaunch& l, uint64_t workspace_bytes) {
  constexpr int64_t kLimit = int64_t(1) << 31;
  if (l.a2 != nullptr || l.b2 != nullptr) return {};
  const int64_t a_bytes = (l.a_kcontig ? int64_t{l.m} : int64_t{l.k}) * l.lda * 4;
  const int64_t b_bytes = (l.b_ncontig ? int64_t{l.k} : int64_t{l.n}) * l.ldb * 4;
  return split_k_shape(l.m, l.n, l.k, !l.a_kcontig && l.b_ncontig,
                       a_bytes < kLimit && b_bytes < kLimit, workspace_bytes);
}

// The split of one launch with its own 16-byte aligned workspace.
inline SplitK split_k_plan(const SgemmLaunch& l) {
  if (l.workspace == nullptr || reinterpret_cast<uintptr_t>(l.workspace) % 16 != 0) return {};
  return split_k_for(l, l.workspace_bytes);
}

// Bytes of partials a launch's split wants when the workspace is not the
// limit (0: it does not split).
inline uint64_t split_k_bytes_wanted(const SgemmLaunch& l) {
  const SplitK sk = split_k_for(l, ~uint64_t{0});
  return sk.splits > 1
             ? static_cast<uint64_t>(sk.splits) * uint64_t(split_partial_ld(l.m)) * uint64_t(l.n) * 4
             : 0;
}

// Enqueues the launch on `stream` (a hipStream_t); returns a hipError_t.
int launch_sgemm(const SgemmLaunch& launch, void* stream);

// The two-panel part of the contract (a2 / b2 set); the one-panel part is
// checked separately.
inline bool two_panel_valid(const SgemmLaunch& l) {
  constexpr int64_t kLimit = int64_t(1) << 31;
  if (l.a2 == nullptr || l.b2 == nullptr || reinterpret_cast<uintptr_t>(l.a2) % 16 != 0 ||
      reinterpret_cast<uintptr_t>(l.b2) % 16 != 0)
    return false;
  const bool nt = !l.a_kcontig && l.b_ncontig;
  if (l.m % 256 != 0 || l.n % 256 != 0 || int64_t{l.m / 256} * (l.n / 256) < 256 ||
      l.k % (nt ? 4 : 8) != 0 || l.k_split % 32 != 0 || l.k_split <= 0 || l.k_split >= l.k)
    return false;
  for (const int64_t kk : {int64_t{l.k_split}, int64_t{l.k - l.k_split}}) {
    // Floats from a panel's base to the end of its last line.
    const int64_t a = l.a_kcontig ? (l.m - 1) * l.lda + kk : kk * l.lda;
    const int64_t b = l.b_ncontig ? kk * l.ldb : (l.n - 1) * l.ldb + kk;
    if (a * 4 >= kLimit || b * 4 >= kLimit) return false;
  }
  return true;
}

} // namespace xvram::kernels
