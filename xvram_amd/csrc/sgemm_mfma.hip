// sgemm_mfma.hip — the tile contraction of the out-of-core SGEMM on gfx950.
//
// Replaces the reference's only dense-math call, the cuBLAS/cuBLASLt SGEMM of
// one resident tile (src/gemm/executor.cpp:147-329 ->
// src/platform/cublas/cublas_api.cpp:634-687,920-938):
//
//     C = alpha * op(A) * op(B) + beta * C        (column-major C, FP32)
//
// computed with full-precision FP32 matrix instructions
// (v_mfma_f32_32x32x2_f32; no xf32 / reduced-precision path). beta == 0 means
// C is never read, so stale or NaN contents of a write-only C panel never leak.
// An optional fused epilogue adds a per-row or per-column bias and applies
// ReLU after the beta term (the host requests it on a tile's last K panel).
//
// Operand forms (canonical column-major, decided by the host planner):
//   A is m x k: A_KCONTIG=false -> a[i + p*lda] (op N), true -> a[p + i*lda] (op T)
//   B is k x n: B_NCONTIG=false -> b[p + j*ldb] (op N), true -> b[j + p*ldb] (op T)
// Every base is 16-byte aligned and every leading dimension a multiple of 4
// floats, and each line may be read as whole 16-byte vectors up to its
// leading dimension (frame-packed panels guarantee all three).
//
// Work decomposition:
//   * workgroup = 256 threads = 4 wave64, output tile 256 (m) x 128 (n), two
//     workgroups per CU (2 waves per SIMD);
//   * each wave owns a 128 x 64 sub-tile = 4 x 2 MFMA blocks of 32 x 32; MFMA
//     row r of block b is tile row 4r+b and MFMA column c of block q is tile
//     column 2c+q, so one ds_read_b128 feeds the A operands of all four row
//     blocks and one ds_read_b64 the B operands of both column blocks, and the
//     epilogue writes four consecutive C rows per lane;
//   * K advances in stages of 16 through two LDS buffers ([k][m] and [k][n],
//     rows padded by 4 floats so the transposing stores of K-contiguous
//     operands hit distinct banks); the next stage's 128-bit global loads are
//     issued at the start of a stage, its LDS stores after the stage's seventh
//     k-step; the operand fragments of k-step kk+1 are read while the MFMAs of
//     k-step kk run; the stage barrier sits before the last k-step's MFMAs and
//     the next stage's first fragments are read right after it, so barrier and
//     LDS latency overlap MFMA work;
//   * interior tiles (every row, column and k of a stage in range) run a
//     branch-free steady-state loop with one pointer per operand; edge tiles
//     and the K tail load through predicated paths that produce exact zeros in
//     BOTH operands for out-of-range rows, columns and k (stale frame padding
//     can never produce 0*NaN), and only in-range C elements are stored — no
//     padding copies;
//   * workgroup ids are remapped so each XCD (8 per chip, dispatched
//     round-robin) walks a contiguous range of tiles, grouped GROUP_M tile-rows
//     at a time, keeping its A/B panels in its own L2.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sgemm_device.hpp"
#include "sgemm_launch.hpp"

namespace xvram::kernels {

int wide_tile();
hipError_t launch_wide(const device::Params& p, bool a_kcontig, bool b_ncontig,
                       hipStream_t stream, hipEvent_t start, hipEvent_t stop);
hipError_t launch_splitk_reduce(const device::Params& p, hipStream_t stream, hipEvent_t stop);
hipError_t launch_thin_k(const device::Params& p, bool a_kcontig, bool b_ncontig,
                         hipStream_t stream, hipEvent_t start, hipEvent_t stop);

namespace {

using namespace device;

constexpr int kThreads = 256;
constexpr int kTileM = 256;
constexpr int kTileN = 128;
constexpr int kStageK = 16;
constexpr int kSteps = kStageK / 2; // MFMA k-steps (K = 2 each) per stage
constexpr int kWaveM = 128;
constexpr int kWaveN = 64;
constexpr int kPitchA = kTileM + 4;
constexpr int kPitchN = kTileN + 4;
constexpr int kGroupM = 8;
constexpr int kALoads = kTileM * kStageK / 4 / kThreads; // float4 per thread per stage
constexpr int kBLoads = kTileN * kStageK / 4 / kThreads;

struct Stage {
  float4 a[kALoads];
  float4 b[kBLoads];
};

// Thread -> element maps for one stage (f = tid + r*256):
//   A m-contiguous: k-row f/64,  rows (f%64)*4..+3
//   A k-contiguous: row f/4,     k (f%4)*4..+3
//   B n-contiguous: k-row f/32,  columns (f%32)*4..+3
//   B k-contiguous: column f/4,  k (f%4)*4..+3
template <bool AK, bool BN>
__device__ __forceinline__ void load_edge(const Params& p, int m0, int n0, int k0, int tid,
                                          Stage& s) {
#pragma unroll
  for (int r = 0; r < kALoads; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (!AK) {
      const int kk = f / (kTileM / 4), mm = (f % (kTileM / 4)) * 4, kg = k0 + kk;
      s.a[r] = load4(p.a + (int64_t)kg * p.lda + m0, mm, p.m - m0, kg < p.k);
    } else {
      const int mm = f / (kStageK / 4), kk = (f % (kStageK / 4)) * 4, mg = m0 + mm;
      s.a[r] = load4(p.a + (int64_t)mg * p.lda + k0, kk, p.k - k0, mg < p.m);
    }
  }
#pragma unroll
  for (int r = 0; r < kBLoads; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (BN) {
      const int kk = f / (kTileN / 4), nn = (f % (kTileN / 4)) * 4, kg = k0 + kk;
      s.b[r] = load4(p.b + (int64_t)kg * p.ldb + n0, nn, p.n - n0, kg < p.k);
    } else {
      const int nn = f / (kStageK / 4), kk = (f % (kStageK / 4)) * 4, ng = n0 + nn;
      s.b[r] = load4(p.b + (int64_t)ng * p.ldb + k0, kk, p.k - k0, ng < p.n);
    }
  }
}

// Interior stage: same maps, no predicates, one base pointer per operand.
template <bool AK, bool BN>
__device__ __forceinline__ void load_full(const float* __restrict__ pa,
                                          const float* __restrict__ pb, int64_t lda, int64_t ldb,
                                          Stage& s) {
#pragma unroll
  for (int r = 0; r < kALoads; ++r) {
    const int64_t off = AK ? (int64_t)(r * (kThreads / (kStageK / 4))) * lda
                           : (int64_t)(r * (kThreads / (kTileM / 4))) * lda;
    s.a[r] = *reinterpret_cast<const float4*>(pa + off);
  }
#pragma unroll
  for (int r = 0; r < kBLoads; ++r) {
    const int64_t off = BN ? (int64_t)(r * (kThreads / (kTileN / 4))) * ldb
                           : (int64_t)(r * (kThreads / (kStageK / 4))) * ldb;
    s.b[r] = *reinterpret_cast<const float4*>(pb + off);
  }
}

template <bool AK, bool BN>
__device__ __forceinline__ void store_stage(float* __restrict__ la, float* __restrict__ lb, int tid,
                                            const Stage& s) {
#pragma unroll
  for (int r = 0; r < kALoads; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (!AK) {
      const int kk = f / (kTileM / 4), mm = (f % (kTileM / 4)) * 4;
      *reinterpret_cast<float4*>(la + kk * kPitchA + mm) = s.a[r];
    } else {
      const int mm = f / (kStageK / 4), kk = (f % (kStageK / 4)) * 4;
      la[(kk + 0) * kPitchA + mm] = s.a[r].x;
      la[(kk + 1) * kPitchA + mm] = s.a[r].y;
      la[(kk + 2) * kPitchA + mm] = s.a[r].z;
      la[(kk + 3) * kPitchA + mm] = s.a[r].w;
    }
  }
#pragma unroll
  for (int r = 0; r < kBLoads; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (BN) {
      const int kk = f / (kTileN / 4), nn = (f % (kTileN / 4)) * 4;
      *reinterpret_cast<float4*>(lb + kk * kPitchN + nn) = s.b[r];
    } else {
      const int nn = f / (kStageK / 4), kk = (f % (kStageK / 4)) * 4;
      lb[(kk + 0) * kPitchN + nn] = s.b[r].x;
      lb[(kk + 1) * kPitchN + nn] = s.b[r].y;
      lb[(kk + 2) * kPitchN + nn] = s.b[r].z;
      lb[(kk + 3) * kPitchN + nn] = s.b[r].w;
    }
  }
}

template <bool AK, bool BN>
__global__ __launch_bounds__(kThreads, 2) void sgemm_mfma_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float lds_a[2][kStageK * kPitchA];
  __shared__ __attribute__((aligned(16))) float lds_b[2][kStageK * kPitchN];

  // A split launch (p.splits > 1): each workgroup multiplies one K range of
  // its tile into that range's partial (sgemm_device.hpp).
  int tile_m, tile_n, split = 0;
  if (p.splits > 1) {
    split = split_coords<kGroupM>(p, tile_m, tile_n);
    narrow_to_split(p, split, AK, !BN);
  } else {
    tile_coords<kGroupM>(p, tile_m, tile_n);
  }
  const int m0 = tile_m * kTileM;
  const int n0 = tile_n * kTileN;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave & 1) * kWaveM;
  const int wn = (wave >> 1) * kWaveN;
  const int lrow = lane & 31;  // MFMA row (A) / column (B) of this lane
  const int lhalf = lane >> 5; // which of the MFMA's two k values

  float16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int stages = (p.k + kStageK - 1) / kStageK;
  const int full_stages = p.k / kStageK;
  const bool interior = m0 + kTileM <= p.m && n0 + kTileN <= p.n;
  const float* pa = AK ? p.a + (int64_t)(m0 + tid / (kStageK / 4)) * p.lda + (tid % (kStageK / 4)) * 4
                       : p.a + (int64_t)(tid / (kTileM / 4)) * p.lda + m0 + (tid % (kTileM / 4)) * 4;
  const float* pb = BN ? p.b + (int64_t)(tid / (kTileN / 4)) * p.ldb + n0 + (tid % (kTileN / 4)) * 4
                       : p.b + (int64_t)(n0 + tid / (kStageK / 4)) * p.ldb + (tid % (kStageK / 4)) * 4;
  const int64_t a_step = AK ? kStageK : (int64_t)kStageK * p.lda;
  const int64_t b_step = BN ? (int64_t)kStageK * p.ldb : kStageK;

  Stage s;
  load_edge<AK, BN>(p, m0, n0, 0, tid, s);
  store_stage<AK, BN>(lds_a[0], lds_b[0], tid, s);
  __syncthreads();

  float4 fa[2];
  float2 fb[2];
  auto read_frag = [&](int buf, int kk, int slot) {
    const int krow = kk + lhalf;
    fa[slot] = *reinterpret_cast<const float4*>(lds_a[buf] + wm + 4 * lrow + krow * kPitchA);
    fb[slot] = *reinterpret_cast<const float2*>(lds_b[buf] + wn + 2 * lrow + krow * kPitchN);
  };
  auto mfmas = [&](int slot) {
    const float ao[4] = {fa[slot].x, fa[slot].y, fa[slot].z, fa[slot].w};
    const float bo[2] = {fb[slot].x, fb[slot].y};
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ao[i], bo[j], acc[i][j], 0, 0, 0);
  };

  read_frag(0, 0, 0);
  int st = 0;
  if (interior) {
    // Steady state: this stage and the next are full. Straight-line body.
    for (; st + 1 < full_stages; ++st) {
      const int buf = st & 1;
      load_full<AK, BN>(pa + (st + 1) * a_step, pb + (st + 1) * b_step, p.lda, p.ldb, s);
      // Keep the next stage's global loads here, a whole stage of MFMAs ahead
      // of their use (the scheduler would otherwise sink them next to the LDS
      // stores to shorten register live ranges, exposing their latency).
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int q = 0; q < kSteps - 1; ++q) {
        read_frag(buf, 2 * (q + 1), (q + 1) & 1);
        mfmas(q & 1);
      }
      store_stage<AK, BN>(lds_a[buf ^ 1], lds_b[buf ^ 1], tid, s);
      __syncthreads();
      read_frag(buf ^ 1, 0, 0);
      mfmas((kSteps - 1) & 1);
    }
  }
  for (; st < stages; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < stages;
    if (more) {
      if (interior && st + 1 < full_stages)
        load_full<AK, BN>(pa + (st + 1) * a_step, pb + (st + 1) * b_step, p.lda, p.ldb, s);
      else
        load_edge<AK, BN>(p, m0, n0, (st + 1) * kStageK, tid, s);
    }
#pragma unroll
    for (int q = 0; q < kSteps - 1; ++q) {
      read_frag(buf, 2 * (q + 1), (q + 1) & 1);
      mfmas(q & 1);
    }
    if (more) store_stage<AK, BN>(lds_a[buf ^ 1], lds_b[buf ^ 1], tid, s);
    __syncthreads();
    if (more) read_frag(buf ^ 1, 0, 0);
    mfmas((kSteps - 1) & 1);
  }

  const Params out = p.splits > 1 ? partial_target(p, split) : p;
  store_c_tile<2, false>(out, acc, m0 + wm, n0 + wn, lrow, lhalf);
}

template <bool AK, bool BN>
hipError_t launch_variant(const Params& p, hipStream_t stream, hipEvent_t start, hipEvent_t stop) {
  const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n * p.splits));
  hipExtLaunchKernelGGL((sgemm_mfma_kernel<AK, BN>), grid, dim3(kThreads), 0, stream, start, stop,
                        0, p);
  return hipGetLastError();
}

} // namespace

// A launch with at least this many 256 x 256 tiles (one per CU of the chip)
// runs a 256 x 256 kernel (sgemm_wide.hip picks a barrier-free one for
// launches of interior tiles); smaller ones keep two 256 x 128 tiles per CU.
constexpr int64_t kWideMinTiles = 256;

// The 256 x 256 kernels address each operand panel with 32-bit buffer
// offsets, so every panel must span less than 2^31 bytes.
bool wide_fits(const SgemmLaunch& l) {
  constexpr int64_t kLimit = int64_t(1) << 31;
  const int64_t t = wide_tile();
  const int64_t tiles = ((l.m + t - 1) / t) * ((l.n + t - 1) / t);
  const int64_t a_bytes = (l.a_kcontig ? (int64_t)l.m : (int64_t)l.k) * l.lda * 4;
  const int64_t b_bytes = (l.b_ncontig ? (int64_t)l.k : (int64_t)l.n) * l.ldb * 4;
  return tiles >= kWideMinTiles && a_bytes < kLimit && b_bytes < kLimit;
}

int launch_sgemm(const SgemmLaunch& launch, void* stream) {
  const bool aligned =
      (reinterpret_cast<uintptr_t>(launch.a) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(launch.b) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(launch.c) % 16 == 0) && (launch.lda % 4 == 0) &&
      (launch.ldb % 4 == 0) && (launch.ldc % 4 == 0) && launch.padded;
  if (launch.m <= 0 || launch.n <= 0 || launch.k <= 0 || !aligned)
    return static_cast<int>(hipErrorInvalidValue);
  // The launch's own error is read back with hipGetLastError below, which also
  // returns an error an earlier runtime call on this thread left behind (an
  // out-of-memory hipMemCreate the cache already handled, for one): consume
  // that first so it is not reported as a launch failure.
  (void)hipGetLastError();
  // K not a multiple of the ring kernels' step where a tail or edge split
  // would pay: the rounded K, then the rest (sgemm_launch.hpp).
  if (const KParts kp = k_remainder_parts(launch); kp.count > 0) {
    for (int i = 0; i < kp.count; ++i)
      if (const int rc = launch_sgemm(kp.part[i], stream); rc != 0) return rc;
    return 0;
  }
  // Ragged m or n over many tiles: the interior and the edge strips as
  // launches of their own (sgemm_launch.hpp), one after another.
  if (const EdgeParts e = edge_parts(launch); e.count > 0) {
    for (int i = 0; i < e.count; ++i)
      if (const int rc = launch_sgemm(e.part[i], stream); rc != 0) return rc;
    return 0;
  }
  Params p;
  p.a = launch.a;
  p.b = launch.b;
  p.c = launch.c;
  p.lda = launch.lda;
  p.ldb = launch.ldb;
  p.ldc = launch.ldc;
  p.m = launch.m;
  p.n = launch.n;
  p.k = launch.k;
  p.alpha = launch.alpha;
  p.beta = launch.beta;
  p.bias_row = launch.bias_row;
  p.bias_col = launch.bias_col;
  p.relu = launch.relu ? 1 : 0;
  p.a2 = launch.a2;
  p.b2 = launch.b2;
  p.k_split = launch.k_split;
  p.splits = 1;
  p.split_depth = 0;
  p.partial = nullptr;
  auto* s = static_cast<hipStream_t>(stream);
  auto* e0 = static_cast<hipEvent_t>(launch.start_event);
  auto* e1 = static_cast<hipEvent_t>(launch.stop_event);
  if (launch.a2 != nullptr || launch.b2 != nullptr) {
    // Two K panels: the barrier-free kernels only.
    if (!two_panel_valid(launch)) return static_cast<int>(hipErrorInvalidValue);
    p.tiles_m = launch.m / wide_tile();
    p.tiles_n = launch.n / wide_tile();
    return static_cast<int>(launch_wide(p, launch.a_kcontig, launch.b_ncontig, s, e0, e1));
  }
  p.k_split = 0;
  // K below 8: no MFMA tiles (sgemm_wide.hip, thin_k_kernel).
  if (launch.k < kThinK)
    return static_cast<int>(launch_thin_k(p, launch.a_kcontig, launch.b_ncontig, s, e0, e1));
  // Fewer tiles than workgroup slots: split K when a workspace is given
  // (fixed-order reduction; sgemm_launch.hpp), on the ring kernels for
  // interior 256 x 256 tiles, else on the 256 x 128 kernel.
  if (const SplitK sk = split_k_plan(launch); sk.splits > 1) {
    p.splits = sk.splits;
    p.split_depth = sk.depth;
    p.partial = launch.workspace;
    if (!sk.narrow) {
      p.tiles_m = launch.m / wide_tile();
      p.tiles_n = launch.n / wide_tile();
      return static_cast<int>(launch_wide(p, launch.a_kcontig, launch.b_ncontig, s, e0, e1));
    }
    p.tiles_m = (launch.m + kTileM - 1) / kTileM;
    p.tiles_n = (launch.n + kTileN - 1) / kTileN;
    hipError_t err;
    if (!launch.a_kcontig && !launch.b_ncontig) err = launch_variant<false, false>(p, s, e0, nullptr);
    else if (!launch.a_kcontig && launch.b_ncontig) err = launch_variant<false, true>(p, s, e0, nullptr);
    else if (launch.a_kcontig && !launch.b_ncontig) err = launch_variant<true, false>(p, s, e0, nullptr);
    else err = launch_variant<true, true>(p, s, e0, nullptr);
    if (err != hipSuccess) return static_cast<int>(err);
    return static_cast<int>(launch_splitk_reduce(p, s, e1));
  }
  // A last round of 256 x 256 tiles that would fill few CUs: the head's
  // tile rows unsplit, then the tail's rows split (sgemm_launch.hpp); the
  // start event rides on the head's dispatch, the stop event on the tail's
  // reduction.
  if (const TailSplit ts = tail_split_plan(launch); ts.head_m > 0) {
    Params head = p;
    head.m = static_cast<int>(ts.head_m);
    head.tiles_m = static_cast<int>(ts.head_m / wide_tile());
    head.tiles_n = launch.n / wide_tile();
    if (const hipError_t e = launch_wide(head, launch.a_kcontig, launch.b_ncontig, s, e0, nullptr);
        e != hipSuccess)
      return static_cast<int>(e);
    Params tail = p;
    tail.a = launch.a_kcontig ? launch.a + ts.head_m * launch.lda : launch.a + ts.head_m;
    tail.c = launch.c + ts.head_m;
    if (tail.bias_row != nullptr) tail.bias_row += ts.head_m;
    tail.m = launch.m - static_cast<int>(ts.head_m);
    tail.tiles_m = tail.m / wide_tile();
    tail.tiles_n = launch.n / wide_tile();
    tail.splits = ts.tail.splits;
    tail.split_depth = ts.tail.depth;
    tail.partial = launch.workspace;
    return static_cast<int>(launch_wide(tail, launch.a_kcontig, launch.b_ncontig, s, nullptr, e1));
  }
  if (wide_fits(launch)) {
    p.tiles_m = (launch.m + wide_tile() - 1) / wide_tile();
    p.tiles_n = (launch.n + wide_tile() - 1) / wide_tile();
    return static_cast<int>(launch_wide(p, launch.a_kcontig, launch.b_ncontig, s, e0, e1));
  }
  p.tiles_m = (launch.m + kTileM - 1) / kTileM;
  p.tiles_n = (launch.n + kTileN - 1) / kTileN;
  hipError_t err;
  if (!launch.a_kcontig && !launch.b_ncontig) err = launch_variant<false, false>(p, s, e0, e1);
  else if (!launch.a_kcontig && launch.b_ncontig) err = launch_variant<false, true>(p, s, e0, e1);
  else if (launch.a_kcontig && !launch.b_ncontig) err = launch_variant<true, false>(p, s, e0, e1);
  else err = launch_variant<true, true>(p, s, e0, e1);
  return static_cast<int>(err);
}

} // namespace xvram::kernels
