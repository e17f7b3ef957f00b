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
// split on the 256 x 128 kernel (two workgroups per CU) when a split runs
// faster by narrow_time. The order of the additions is fixed, so C
// is the same from run to run. Without a workspace large enough for two
// partials the launch runs unsplit. One K panel only. A launch of at least
// 256 interior tiles whose last round would leave CUs idle may run as a
// head and a split tail instead (tail_split_plan below).
//
// start_event / stop_event (hipEvent_t, optional) are recorded by the dispatch
// itself (hipExtLaunchKernelGGL): no separate marker packets run between
// kernels, and stop_event completes when the kernel does, so it can serve as
// the retire event of every panel the launch reads or writes. A start event
// costs the dispatch ~16 us of host time and ~5 us of device time; the
// executor passes none and derives starts from the events a launch follows.
#pragma once

#include <algorithm>
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
// K per workgroup of a split launch, at least (a shallower range spends more
// of its time on its first loads and on storing its partial than on MFMAs).
constexpr int64_t kSplitMinDepth = 64;
// K per workgroup of a split on the ring kernels, at least: shallower ranges
// of interior tiles run faster as the 256 x 128 kernel's split (1024^3, 64
// deep on the ring kernels: 44.4 against 55.0 us; 512 x 512 x 4096, 64:
// 46.7 against 63.9; 1024 x 1024 x 3072, 192: 76.1 against 82.0), deeper
// ones on the ring kernels (1536^3, 224: 91.3 against 94.1 us; 2048 x 2048 x
// 1024, 256: 99.8 against 102.6; 1024 x 1024 x 8192, 512: 151.2 against
// 159.6).
constexpr int64_t kRingSplitMinDepth = 224;
// Workgroups of one split launch on the 256 x 128 kernel, at most: two rounds
// of its two workgroups per CU. Its partials then hold at most this many
// 256 x 128 tiles (kSplitMaxPartialBytes).
constexpr int64_t kNarrowMaxGroups = 4 * kComputeUnits;
constexpr uint64_t kSplitMaxPartialBytes = uint64_t(kNarrowMaxGroups) * 256 * 128 * 4;

struct SplitK {
  int splits = 1;      // 1 = not split
  int depth = 0;       // K per range (multiple of 32); the last range holds the rest
  bool narrow = false; // the ranges run on the 256 x 128 kernel (else the ring kernels)
};

// Leading dimension of a split launch's partials: m rounded up to 4 floats,
// so every column starts 16-byte aligned.
inline int64_t split_partial_ld(int64_t m) { return (m + 3) / 4 * 4; }

// K ranges of `depth` (ceil(k / s) rounded up to 32) covering k.
inline SplitK split_ranges(int64_t k, int64_t s, bool narrow) {
  const int64_t depth = ((k + s - 1) / s + 31) / 32 * 32;
  return SplitK{static_cast<int>((k + depth - 1) / depth), static_cast<int>(depth), narrow};
}

// Time of an m x n x k launch on the 256 x 128 kernel as `groups` equal
// workgroups of K depth `depth` writing `splits` partials (1 = unsplit, no
// partials), in hundredths of the time a workgroup paired with another on its
// CU takes per unit of K. The dispatcher fills every CU's two slots round
// after round, so full rounds of 2 x CUs workgroups each take a pair's time,
// and so does a last round that pairs workgroups on some CUs; a last round of
// at most one workgroup per CU runs each alone, in 0.65 of a pair's time.
// Each workgroup pays a fixed cost worth 32 units of K, and each partial one
// 8e-6 units per element to write and read back. Fitted to sixteen launches
// of 4 to 384 tiles of 256 x 128 (config 2, seven other ragged shapes and
// eight of interior tiles, each at four to nine split counts from unsplit to
// three rounds): the rule's choice ran within 1.6 % of the fastest measured
// count on every one.
inline int64_t narrow_time(int64_t m, int64_t n, int64_t groups, int64_t depth, int64_t splits) {
  constexpr int64_t slots = 2 * kComputeUnits;
  const int64_t full = (groups - 1) / slots;
  const int64_t last = groups - full * slots;
  const int64_t partials = splits > 1 ? splits * m * n / 1250 : 0;
  return (depth + 32) * (100 * full + (last > kComputeUnits ? 100 : 65)) + partials;
}

// The split of an m x n x k launch of form `nt` (A op N, B op T) or not,
// given a workspace of `workspace_bytes` (see "Split K" above). Ranges are at
// least kSplitMinDepth deep and the workspace holds all their partials.
// `ring` = the ring kernels can address the operand panels (each spans less
// than 2^31 bytes).
//  - Interior tiles on the ring kernels (one workgroup per CU): as many
//    ranges as one round of the CUs takes (more rounds only add each
//    range's fixed costs), when those are at least kRingSplitMinDepth deep.
//  - Otherwise, on the 256 x 128 kernel, when the launch has fewer than
//    kComputeUnits tiles of 256 x 256: the number of ranges, within two rounds
//    of its workgroup slots (kNarrowMaxGroups), that narrow_time rates
//    fastest, the unsplit launch included (ties go to fewer ranges).
inline SplitK split_k_shape(int64_t m, int64_t n, int64_t k, bool nt, bool ring,
                            uint64_t workspace_bytes) {
  if (m <= 0 || n <= 0 || k <= 0) return {};
  const bool interior = ring && m % 256 == 0 && n % 256 == 0 && k % (nt ? 4 : 8) == 0;
  const int64_t partial = split_partial_ld(m) * n * 4;
  const int64_t deepest = k / kSplitMinDepth;
  const int64_t most =
      std::min(deepest, static_cast<int64_t>(std::min<uint64_t>(workspace_bytes / partial, 1 << 30)));
  if (most < 2) return {};
  if (interior) {
    // The kernel family follows from the shape alone, not from the
    // workspace: a launch given exactly the workspace its split wants
    // (split_k_bytes_wanted) takes that same split.
    const int64_t tiles = (m / 256) * (n / 256);
    const int64_t one_round = std::min(deepest, kComputeUnits / tiles);
    if (one_round < 2) return {};
    if (split_ranges(k, one_round, false).depth >= kRingSplitMinDepth) {
      const SplitK sk = split_ranges(k, std::min(one_round, most), false);
      return sk.splits >= 2 ? sk : SplitK{};
    }
  }
  // At least one 256 x 256 tile per CU runs a 256 x 256 kernel unsplit.
  if (((m + 255) / 256) * ((n + 255) / 256) >= kComputeUnits) return {};
  const int64_t tiles = ((m + 255) / 256) * ((n + 127) / 128);
  SplitK best{};
  int64_t best_time = narrow_time(m, n, tiles, k, 1);
  for (int64_t s = 2; s <= most; ++s) {
    const SplitK sk = split_ranges(k, s, true);
    if (sk.splits < 2 || sk.splits == best.splits) continue;
    if (tiles * sk.splits > kNarrowMaxGroups) break;
    const int64_t t = narrow_time(m, n, tiles * sk.splits, sk.depth, sk.splits);
    if (t < best_time) {
      best = sk;
      best_time = t;
    }
  }
  return best;
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

// K below this runs on a plain kernel (each thread four rows of one column of
// C), not the MFMA tiles: a K remainder's last 1-7 rows, or any such launch.
constexpr int kThinK = 8;

// Tail split. A launch of at least kComputeUnits interior 256 x 256 tiles
// runs in rounds of one workgroup per CU, and a last round that fills few
// CUs costs as much as a full one (17 x 17 tiles: 2 rounds for 289 tiles).
// It may run instead as a head, tile rows [0, head_m) unsplit in whole
// rounds, followed by a tail, rows [head_m, m), whose K is split on the ring
// kernels (up to two rounds of ranges at least kRingSplitMinDepth deep, the
// partials in the workspace), when the model below rates that at most 0.9
// of the unsplit launch. Time is counted in units of K of one round: the head
// takes its rounds x K, the tail its rounds x (range depth + 48), plus 128 for
// its extra launch and the reduction.
struct TailSplit {
  int64_t head_m = 0; // rows of the head (a multiple of 256); 0 = no tail split
  SplitK tail;        // the split of the tail's m - head_m rows
};

// The rounds of one workgroup per CU that `groups` workgroups take.
inline int64_t cu_rounds(int64_t groups) { return (groups + kComputeUnits - 1) / kComputeUnits; }

// The tail split of an interior m x n x k launch (none: head_m 0) and, in
// *time, the model's time of the launch as it then runs (tail split or not).
inline TailSplit tail_split_timed(int64_t m, int64_t n, int64_t k, uint64_t workspace_bytes,
                                  int64_t* time) {
  const int64_t tiles_m = m / 256, tiles_n = n / 256;
  const int64_t unsplit = cu_rounds(tiles_m * tiles_n) * k;
  TailSplit best{};
  int64_t best_time = unsplit;
  for (int64_t t = 1; t < tiles_m && 2 * t * tiles_n <= 2 * kComputeUnits; ++t) {
    const int64_t tail_tiles = t * tiles_n;
    const uint64_t partial = uint64_t(t) * 256 * uint64_t(n) * 4;
    const int64_t head_time = cu_rounds((tiles_m - t) * tiles_n) * k;
    for (int64_t s = 2; s <= k / kSplitMinDepth; ++s) {
      const SplitK sk = split_ranges(k, s, false);
      if (sk.depth < kRingSplitMinDepth || tail_tiles * sk.splits > 2 * kComputeUnits ||
          uint64_t(sk.splits) * partial > workspace_bytes)
        break;
      const int64_t time = head_time + cu_rounds(tail_tiles * sk.splits) * (sk.depth + 48) + 128;
      if (time < best_time) {
        best_time = time;
        best = TailSplit{(tiles_m - t) * 256, sk};
      }
    }
  }
  if (10 * best_time > 9 * unsplit) {
    best = TailSplit{};
    best_time = unsplit;
  }
  if (time != nullptr) *time = best_time;
  return best;
}

inline TailSplit tail_split_shape(int64_t m, int64_t n, int64_t k, bool nt, bool ring,
                                  uint64_t workspace_bytes) {
  if (!ring || m <= 0 || n <= 0 || k <= 0 || m % 256 != 0 || n % 256 != 0 || k % (nt ? 4 : 8) != 0)
    return {};
  if ((m / 256) * (n / 256) < kComputeUnits) return {};
  return tail_split_timed(m, n, k, workspace_bytes, nullptr);
}

// The tail split a launch takes given room for `workspace_bytes` of
// partials: none for a two-panel launch or panels the ring kernels cannot
// address, else tail_split_shape.
inline TailSplit tail_split_for(const SgemmLaunch& l, uint64_t workspace_bytes) {
  constexpr int64_t kLimit = int64_t(1) << 31;
  if (l.a2 != nullptr || l.b2 != nullptr) return {};
  const int64_t a_bytes = (l.a_kcontig ? int64_t{l.m} : int64_t{l.k}) * l.lda * 4;
  const int64_t b_bytes = (l.b_ncontig ? int64_t{l.k} : int64_t{l.n}) * l.ldb * 4;
  return tail_split_shape(l.m, l.n, l.k, !l.a_kcontig && l.b_ncontig,
                          a_bytes < kLimit && b_bytes < kLimit, workspace_bytes);
}

// The tail split of one launch with its own 16-byte aligned workspace.
inline TailSplit tail_split_plan(const SgemmLaunch& l) {
  if (l.workspace == nullptr || reinterpret_cast<uintptr_t>(l.workspace) % 16 != 0) return {};
  return tail_split_for(l, l.workspace_bytes);
}

// Bytes of partials a launch's split (or tail split) wants when the
// workspace is not the limit (0: it does not split).
inline uint64_t split_k_bytes_wanted_whole(const SgemmLaunch& l) {
  const SplitK sk = split_k_for(l, ~uint64_t{0});
  if (sk.splits > 1)
    return static_cast<uint64_t>(sk.splits) * uint64_t(split_partial_ld(l.m)) * uint64_t(l.n) * 4;
  const TailSplit ts = tail_split_for(l, ~uint64_t{0});
  return ts.head_m > 0 ? static_cast<uint64_t>(ts.tail.splits) * uint64_t(l.m - ts.head_m) *
                             uint64_t(l.n) * 4
                       : 0;
}

// Edge split. A launch whose m or n is not a multiple of 256 and that has at
// least kComputeUnits tiles of 256 x 256 runs every tile on the ring kernels'
// edge instances (K a multiple of 4 for N/T, of 8 for the other forms), whose
// K loop is the interior one: rounds x (K x 26/25 + 50) in units of K of one
// round, within 4 % of 17 shapes measured. Its last round may fill few CUs. It
// may run instead as up to three launches of its own, one after another on
// its stream: the interior rows [0, mi) x columns [0, ni) (mi, ni = m, n
// rounded down to 256; ring kernels, or their tail split), the right strip
// rows [0, mi) x columns [ni, n) and the bottom strip rows [mi, m) x columns
// [0, n), each split by the rules above (the strips on the 256 x 128 kernel),
// sharing the workspace. Every element of C is computed by one of them. The
// split is modelled as the interior's time (tail_split_timed, one round for
// fewer than kComputeUnits tiles), plus the strips' 256 x 128 tiles x K x
// 2.7 over the 256 x 128 kernel's 512 slots (their split launches' first
// loads, partial stores and reductions, and mostly empty tiles: least squares
// over 20 shapes), plus 150 for the two extra launches, and taken when it
// models faster. On 22 shapes from 4100^2 x 240 to 11500 x 11000 x 1024 the
// model's split / whole ratio came within 7 % of the measured one and picked
// the faster plan every time (split 4100^2 x 4096 1.74x, 7000^3 1.31x, 5000^2
// x 2048 1.09x; whole 8191^2 x 8192 1.17x, 8100^2 x 4096 1.15x, 8000^3 1.07x).
// Only for one-panel launches with K a multiple of 4 (N/T) or 8 (the other
// forms), and panels below 2^31 bytes; when a part would split, only with a
// workspace (a strip unsplit would leave most CUs idle).
inline bool edge_split_rated_faster(int64_t m, int64_t n, int64_t k, bool nt) {
  if (m <= 0 || n <= 0 || k <= 0 || k % (nt ? 4 : 8) != 0) return false;
  const int64_t mi = m / 256 * 256, ni = n / 256 * 256;
  const int64_t whole_tiles = ((m + 255) / 256) * ((n + 255) / 256);
  if ((mi == m && ni == n) || whole_tiles < kComputeUnits || mi == 0 || ni == 0) return false;
  const int64_t whole = cu_rounds(whole_tiles) * (k * 26 / 25 + 50);
  const int64_t interior_tiles = (mi / 256) * (ni / 256);
  int64_t interior = cu_rounds(interior_tiles) * k;
  if (interior_tiles >= kComputeUnits) tail_split_timed(mi, ni, k, ~uint64_t{0}, &interior);
  // The strips' 256 x 128 tiles (the bottom strip's one row of them, the
  // right strip's column of them).
  const int64_t strip_tiles = (m > mi ? (n + 127) / 128 : 0) + (mi / 256) * ((n - ni + 127) / 128);
  const int64_t split = interior + 27 * k * strip_tiles / (20 * kComputeUnits) + 150;
  return split < whole;
}

struct EdgeParts {
  int count = 0; // 0 = no edge split
  SgemmLaunch part[3];
};

// Rows [r0, r0 + rows) x columns [c0, c0 + cols) of a launch as a launch of
// its own (no events).
inline SgemmLaunch sub_launch(const SgemmLaunch& l, int64_t r0, int rows, int64_t c0, int cols) {
  SgemmLaunch s = l;
  s.a = l.a_kcontig ? l.a + r0 * l.lda : l.a + r0;
  s.b = l.b_ncontig ? l.b + c0 : l.b + c0 * l.ldb;
  s.c = l.c + r0 + c0 * l.ldc;
  if (s.bias_row != nullptr) s.bias_row += r0;
  if (s.bias_col != nullptr) s.bias_col += c0;
  s.m = rows;
  s.n = cols;
  s.start_event = nullptr;
  s.stop_event = nullptr;
  return s;
}

// The parts of a launch's edge split by shape alone (count 0: none).
inline EdgeParts edge_parts_shape(const SgemmLaunch& l) {
  constexpr int64_t kLimit = int64_t(1) << 31;
  EdgeParts e;
  if (l.a2 != nullptr || l.b2 != nullptr || l.m <= 0 || l.n <= 0 || l.k <= 0) return e;
  const bool nt = !l.a_kcontig && l.b_ncontig;
  const int64_t a_bytes = (l.a_kcontig ? int64_t{l.m} : int64_t{l.k}) * l.lda * 4;
  const int64_t b_bytes = (l.b_ncontig ? int64_t{l.k} : int64_t{l.n}) * l.ldb * 4;
  if (a_bytes >= kLimit || b_bytes >= kLimit || !edge_split_rated_faster(l.m, l.n, l.k, nt))
    return e;
  const int mi = l.m / 256 * 256, ni = l.n / 256 * 256;
  e.part[e.count++] = sub_launch(l, 0, mi, 0, ni);
  if (ni < l.n) e.part[e.count++] = sub_launch(l, 0, mi, ni, l.n - ni);
  if (mi < l.m) e.part[e.count++] = sub_launch(l, mi, l.m - mi, 0, l.n);
  e.part[0].start_event = l.start_event;
  e.part[e.count - 1].stop_event = l.stop_event;
  return e;
}

// The parts of a launch's edge split (count 0: none): by shape, and without a
// workspace only when no part would split.
inline EdgeParts edge_parts(const SgemmLaunch& l) {
  const EdgeParts e = edge_parts_shape(l);
  if (e.count == 0 || l.workspace != nullptr) return e;
  for (int i = 0; i < e.count; ++i)
    if (split_k_bytes_wanted_whole(e.part[i]) > 0) return {};
  return e;
}

// Whether an m x n x k launch of form `nt` whose panels the ring kernels can
// address would take an edge split one of whose parts splits (the planner
// then gives its launches a workspace).
inline bool edge_split_wants_workspace(int64_t m, int64_t n, int64_t k, bool nt) {
  if (!edge_split_rated_faster(m, n, k, nt)) return false;
  const int64_t mi = m / 256 * 256, ni = n / 256 * 256;
  constexpr uint64_t kAny = ~uint64_t{0};
  return split_k_shape(mi, ni, k, nt, true, kAny).splits > 1 ||
         tail_split_shape(mi, ni, k, nt, true, kAny).head_m > 0 ||
         (ni < n && split_k_shape(mi, n - ni, k, nt, true, kAny).splits > 1) ||
         (mi < m && split_k_shape(m - mi, n, k, nt, true, kAny).splits > 1);
}

// K remainder. The ring kernels need K a multiple of 4 (N/T) or 8 (the other
// forms), and so do the tail and edge splits. A launch whose K is not, whose
// K rounded down to that multiple is at least 512, and which either has
// interior tiles and would take a tail split over the rounded K, or has
// ragged tiles, at least kComputeUnits of them (the rounded K then runs on
// the ring kernels' edge instances or takes an edge split, not the general
// kernel's predicated edge tiles), runs as two launches of its own: the first
// over the rounded K with alpha and beta and no epilogue, the second over the
// remaining 1 to 7 K rows with alpha and beta 1 onto the first's result, then
// the epilogue (one more read and write of C: 4500^3 N/N, 2.30 ms as one
// launch on the general kernel, gains far more from the split first part).
// Returns the rounded K (0: no K remainder).
inline int64_t k_remainder_shape(int64_t m, int64_t n, int64_t k, bool nt) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  const int64_t k1 = k - k % (nt ? 4 : 8);
  if (k1 == k || k1 < 512) return 0;
  const bool interior = m % 256 == 0 && n % 256 == 0;
  const bool gains = interior ? tail_split_shape(m, n, k1, nt, true, ~uint64_t{0}).head_m > 0
                              : ((m + 255) / 256) * ((n + 255) / 256) >= kComputeUnits;
  return gains ? k1 : 0;
}

struct KParts {
  int count = 0; // 0 = no K remainder
  SgemmLaunch part[2];
};

// The two launches of a K remainder by shape (count 0: none); one-panel
// launches whose panels the ring kernels can address only.
inline KParts k_remainder_parts_shape(const SgemmLaunch& l) {
  constexpr int64_t kLimit = int64_t(1) << 31;
  KParts r;
  if (l.a2 != nullptr || l.b2 != nullptr) return r;
  const int64_t a_bytes = (l.a_kcontig ? int64_t{l.m} : int64_t{l.k}) * l.lda * 4;
  const int64_t b_bytes = (l.b_ncontig ? int64_t{l.k} : int64_t{l.n}) * l.ldb * 4;
  if (a_bytes >= kLimit || b_bytes >= kLimit) return r;
  const int64_t k1 = k_remainder_shape(l.m, l.n, l.k, !l.a_kcontig && l.b_ncontig);
  if (k1 == 0) return r;
  SgemmLaunch first = l;
  first.k = static_cast<int>(k1);
  first.bias_row = nullptr;
  first.bias_col = nullptr;
  first.relu = false;
  first.stop_event = nullptr;
  SgemmLaunch rest = l;
  rest.k = l.k - static_cast<int>(k1);
  rest.a = l.a_kcontig ? l.a + k1 : l.a + k1 * l.lda;
  rest.b = l.b_ncontig ? l.b + k1 * l.ldb : l.b + k1;
  rest.beta = 1.f;
  rest.start_event = nullptr;
  r.part[0] = first;
  r.part[1] = rest;
  r.count = 2;
  return r;
}

// Bytes of partials a launch wants when the workspace is not the limit: the
// first part's of a K remainder; else the most any part of its edge split
// wants (they run one after another on the stream, so they share it); else
// its own split's (0: it does not split).
inline uint64_t split_k_bytes_wanted(const SgemmLaunch& l) {
  const KParts kp = k_remainder_parts_shape(l);
  const SgemmLaunch& base = kp.count > 0 ? kp.part[0] : l;
  const EdgeParts e = edge_parts_shape(base);
  if (e.count == 0) return split_k_bytes_wanted_whole(base);
  uint64_t most = 0;
  for (int i = 0; i < e.count; ++i) most = std::max(most, split_k_bytes_wanted_whole(e.part[i]));
  return most;
}

// The two launches of a K remainder (count 0: none): by shape, and without a
// workspace only when the first part would not split.
inline KParts k_remainder_parts(const SgemmLaunch& l) {
  const KParts kp = k_remainder_parts_shape(l);
  if (kp.count == 0 || l.workspace != nullptr || split_k_bytes_wanted(kp.part[0]) == 0) return kp;
  return {};
}

// Whether a plan's m x n x k launch of form `nt` would take a K remainder
// whose first part splits (the planner then gives its launches a workspace).
inline bool k_remainder_wants_workspace(int64_t m, int64_t n, int64_t k, bool nt) {
  const int64_t k1 = k_remainder_shape(m, n, k, nt);
  if (k1 == 0) return false;
  return tail_split_shape(m, n, k1, nt, true, ~uint64_t{0}).head_m > 0 ||
         edge_split_wants_workspace(m, n, k1, nt);
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
