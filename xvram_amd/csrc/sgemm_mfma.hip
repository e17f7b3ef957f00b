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
//
// Operand forms (canonical column-major, decided by the host planner):
//   A is m x k: A_KCONTIG=false -> a[i + p*lda] (op N), true -> a[p + i*lda] (op T)
//   B is k x n: B_NCONTIG=false -> b[p + j*ldb] (op N), true -> b[j + p*ldb] (op T)
//
// Work decomposition:
//   * workgroup = 256 threads = 4 wave64, output tile 256 (m) x 128 (n);
//   * each wave owns a 128 x 64 sub-tile = 4 x 2 MFMA blocks of 32 x 32; MFMA
//     row r of block b is tile row 4r+b and MFMA column c of block q is tile
//     column 2c+q, so one ds_read_b128 feeds the A operands of all four row
//     blocks and one ds_read_b64 the B operands of both column blocks, and the
//     epilogue writes four consecutive C rows per lane;
//   * K advances in stages of 16, double-buffered in LDS ([k][m] and [k][n]
//     panels, padded so the transposing stores of K-contiguous operands are
//     bank-conflict free); the next stage's global loads are issued before the
//     current stage's MFMAs;
//   * global loads are 128-bit and coalesced along the operand's contiguous
//     dimension for all four N/T forms (VEC=4; requires 16-byte aligned bases
//     and leading dimensions that are multiples of 4, which frame-packed
//     panels always have) or 32-bit (VEC=1, any alignment);
//   * edges are predicated (no padding copies): out-of-range rows, columns and
//     k are loaded as exact zeros in BOTH operands (so garbage in the unused
//     part of a frame can never produce 0*NaN) and never stored;
//   * workgroup ids are remapped so each XCD (8 per chip, dispatched
//     round-robin) walks a contiguous, GROUP_M-grouped range of tiles and keeps
//     its A/B panels in its own L2.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "sgemm_launch.hpp"

namespace xvram::kernels {
namespace {

constexpr int kThreads = 256;
constexpr int kTileM = 256;
constexpr int kTileN = 128;
constexpr int kStageK = 16;
constexpr int kWaveM = 128;
constexpr int kWaveN = 64;
// LDS row pitches (floats). +4 keeps ds_write_b128/ds_read_b128 16-byte
// aligned and spreads the four k-rows written by one transposing store over
// different banks.
constexpr int kPitchA = kTileM + 4;
constexpr int kPitchN = kTileN + 4;
constexpr int kGroupM = 8;

typedef float float16_t __attribute__((ext_vector_type(16)));

struct Params {
  const float* a;
  const float* b;
  float* c;
  int64_t lda, ldb, ldc;
  int m, n, k;
  float alpha, beta;
  int tiles_m, tiles_n;
};

__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// Loads 4 consecutive elements along the contiguous dimension starting at
// element `first` of a line whose valid extent is `limit`, from `line`
// (the line's base). Elements >= limit read as 0. The vector form reads a
// whole float4 when its first element is in range: callers guarantee the
// allocation extends to the padded leading dimension (multiple of 4).
template <int VEC>
__device__ __forceinline__ float4 load4(const float* __restrict__ line, int first, int limit,
                                        bool line_valid) {
  if (!line_valid || first >= limit) return zero4();
  if constexpr (VEC == 4) {
    float4 v = *reinterpret_cast<const float4*>(line + first);
    if (first + 4 > limit) {
      const int left = limit - first;
      if (left < 4) v.w = 0.f;
      if (left < 3) v.z = 0.f;
      if (left < 2) v.y = 0.f;
    }
    return v;
  } else {
    float4 v;
    v.x = line[first];
    v.y = first + 1 < limit ? line[first + 1] : 0.f;
    v.z = first + 2 < limit ? line[first + 2] : 0.f;
    v.w = first + 3 < limit ? line[first + 3] : 0.f;
    return v;
  }
}

// Per-thread staging registers for one K stage.
struct Stage {
  float4 a[4];
  float4 b[2];
};

// Global -> registers for the stage starting at k0.
//
// A tile is 256 (m) x 16 (k) = 1024 float4; B tile is 16 (k) x 128 (n) = 512.
template <bool A_KCONTIG, bool B_NCONTIG, int VEC>
__device__ __forceinline__ void load_stage(const Params& p, int m0, int n0, int k0, int tid,
                                           Stage& s) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (!A_KCONTIG) {
      // 16 columns (k) of 256 contiguous rows: 64 float4 per column.
      const int kk = f >> 6;
      const int mm = (f & 63) * 4;
      const int kg = k0 + kk;
      s.a[r] = load4<VEC>(p.a + (int64_t)kg * p.lda + m0, mm, p.m - m0, kg < p.k);
    } else {
      // 256 rows (m) of 16 contiguous k: 4 float4 per row.
      const int mm = f >> 2;
      const int kk = (f & 3) * 4;
      const int mg = m0 + mm;
      s.a[r] = load4<VEC>(p.a + (int64_t)mg * p.lda + k0, kk, p.k - k0, mg < p.m);
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (B_NCONTIG) {
      // 16 rows (k) of 128 contiguous n: 32 float4 per row.
      const int kk = f >> 5;
      const int nn = (f & 31) * 4;
      const int kg = k0 + kk;
      s.b[r] = load4<VEC>(p.b + (int64_t)kg * p.ldb + n0, nn, p.n - n0, kg < p.k);
    } else {
      // 128 columns (n) of 16 contiguous k: 4 float4 per column.
      const int nn = f >> 2;
      const int kk = (f & 3) * 4;
      const int ng = n0 + nn;
      s.b[r] = load4<VEC>(p.b + (int64_t)ng * p.ldb + k0, kk, p.k - k0, ng < p.n);
    }
  }
}

// Registers -> LDS ([k][m] for A, [k][n] for B).
template <bool A_KCONTIG, bool B_NCONTIG>
__device__ __forceinline__ void store_stage(float* __restrict__ lds_a, float* __restrict__ lds_b,
                                            int tid, const Stage& s) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (!A_KCONTIG) {
      const int kk = f >> 6;
      const int mm = (f & 63) * 4;
      *reinterpret_cast<float4*>(lds_a + kk * kPitchA + mm) = s.a[r];
    } else {
      const int mm = f >> 2;
      const int kk = (f & 3) * 4;
      lds_a[(kk + 0) * kPitchA + mm] = s.a[r].x;
      lds_a[(kk + 1) * kPitchA + mm] = s.a[r].y;
      lds_a[(kk + 2) * kPitchA + mm] = s.a[r].z;
      lds_a[(kk + 3) * kPitchA + mm] = s.a[r].w;
    }
  }
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (B_NCONTIG) {
      const int kk = f >> 5;
      const int nn = (f & 31) * 4;
      *reinterpret_cast<float4*>(lds_b + kk * kPitchN + nn) = s.b[r];
    } else {
      const int nn = f >> 2;
      const int kk = (f & 3) * 4;
      lds_b[(kk + 0) * kPitchN + nn] = s.b[r].x;
      lds_b[(kk + 1) * kPitchN + nn] = s.b[r].y;
      lds_b[(kk + 2) * kPitchN + nn] = s.b[r].z;
      lds_b[(kk + 3) * kPitchN + nn] = s.b[r].w;
    }
  }
}

// Maps the linear workgroup id to a (tile_m, tile_n) pair: first undo the
// round-robin XCD dispatch so that XCD x owns ids [x*per, (x+1)*per), then
// walk tiles in GROUP_M-row groups (column-major inside a group) so that
// concurrently running workgroups share A rows and B columns in L2.
__device__ __forceinline__ void tile_coords(const Params& p, int& tm, int& tn) {
  const int total = p.tiles_m * p.tiles_n;
  int id = blockIdx.x;
  constexpr int kXcds = 8;
  if ((total % kXcds) == 0) {
    const int per = total / kXcds;
    id = (id % kXcds) * per + id / kXcds;
  }
  const int group_span = kGroupM * p.tiles_n;
  const int group = id / group_span;
  const int first_m = group * kGroupM;
  const int group_rows = min(p.tiles_m - first_m, kGroupM);
  const int in_group = id - group * group_span;
  tm = first_m + in_group % group_rows;
  tn = in_group / group_rows;
}

template <bool A_KCONTIG, bool B_NCONTIG, int VEC>
__global__ __launch_bounds__(kThreads, 2) void sgemm_mfma_kernel(Params p) {
  __shared__ __attribute__((aligned(16))) float lds_a[2][kStageK * kPitchA];
  __shared__ __attribute__((aligned(16))) float lds_b[2][kStageK * kPitchN];

  int tile_m, tile_n;
  tile_coords(p, tile_m, tile_n);
  const int m0 = tile_m * kTileM;
  const int n0 = tile_n * kTileN;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = (wave & 1) * kWaveM;  // wave's row offset inside the tile
  const int wn = (wave >> 1) * kWaveN; // wave's column offset inside the tile
  const int lrow = lane & 31;          // MFMA row (A) / column (B) of this lane
  const int lhalf = lane >> 5;         // which of the two k values of an MFMA

  float16_t acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int stages = (p.k + kStageK - 1) / kStageK;
  Stage s;
  load_stage<A_KCONTIG, B_NCONTIG, VEC>(p, m0, n0, 0, tid, s);
  store_stage<A_KCONTIG, B_NCONTIG>(lds_a[0], lds_b[0], tid, s);
  __syncthreads();

  for (int st = 0; st < stages; ++st) {
    const int buf = st & 1;
    const bool more = st + 1 < stages;
    if (more) load_stage<A_KCONTIG, B_NCONTIG, VEC>(p, m0, n0, (st + 1) * kStageK, tid, s);

    const float* la = lds_a[buf] + wm + 4 * lrow;
    const float* lb = lds_b[buf] + wn + 2 * lrow;
#pragma unroll
    for (int kk = 0; kk < kStageK; kk += 2) {
      const int krow = kk + lhalf;
      const float4 av = *reinterpret_cast<const float4*>(la + krow * kPitchA);
      const float2 bv = *reinterpret_cast<const float2*>(lb + krow * kPitchN);
      const float a_ops[4] = {av.x, av.y, av.z, av.w};
      const float b_ops[2] = {bv.x, bv.y};
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a_ops[i], b_ops[j], acc[i][j], 0, 0, 0);
    }

    if (more) store_stage<A_KCONTIG, B_NCONTIG>(lds_a[buf ^ 1], lds_b[buf ^ 1], tid, s);
    __syncthreads();
  }

  // Epilogue. Accumulator element v of block (i, j) for this lane sits at
  // MFMA row 8*(v/4) + 4*lhalf + v%4 and MFMA column lrow, i.e. tile row
  // wm + 4*(that) + i and tile column wn + 2*lrow + j.
  const bool read_c = p.beta != 0.f;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int col = n0 + wn + 2 * lrow + j;
    if (col >= p.n) continue;
    float* cline = p.c + (int64_t)col * p.ldc;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int mrow = 8 * (v >> 2) + 4 * lhalf + (v & 3);
      const int row = m0 + wm + 4 * mrow;
      if (row >= p.m) continue;
      float out[4] = {acc[0][j][v], acc[1][j][v], acc[2][j][v], acc[3][j][v]};
      if (VEC == 4 && row + 4 <= p.m) {
        float4* dst = reinterpret_cast<float4*>(cline + row);
        float4 r;
        if (read_c) {
          const float4 old = *dst;
          r.x = p.alpha * out[0] + p.beta * old.x;
          r.y = p.alpha * out[1] + p.beta * old.y;
          r.z = p.alpha * out[2] + p.beta * old.z;
          r.w = p.alpha * out[3] + p.beta * old.w;
        } else {
          r.x = p.alpha * out[0];
          r.y = p.alpha * out[1];
          r.z = p.alpha * out[2];
          r.w = p.alpha * out[3];
        }
        *dst = r;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (row + t < p.m) {
            const float val = p.alpha * out[t];
            cline[row + t] = read_c ? val + p.beta * cline[row + t] : val;
          }
        }
      }
    }
  }
}

template <bool AK, bool BN, int VEC>
hipError_t launch_variant(const Params& p, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
  hipLaunchKernelGGL((sgemm_mfma_kernel<AK, BN, VEC>), grid, dim3(kThreads), 0, stream, p);
  return hipGetLastError();
}

template <int VEC>
hipError_t dispatch_layout(const Params& p, bool ak, bool bn, hipStream_t stream) {
  if (!ak && !bn) return launch_variant<false, false, VEC>(p, stream);
  if (!ak && bn) return launch_variant<false, true, VEC>(p, stream);
  if (ak && !bn) return launch_variant<true, false, VEC>(p, stream);
  return launch_variant<true, true, VEC>(p, stream);
}

} // namespace

int sgemm_tile_m() { return kTileM; }
int sgemm_tile_n() { return kTileN; }

int launch_sgemm(const SgemmLaunch& launch, void* stream) {
  if (launch.m <= 0 || launch.n <= 0 || launch.k <= 0) return static_cast<int>(hipErrorInvalidValue);
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
  p.tiles_m = (launch.m + kTileM - 1) / kTileM;
  p.tiles_n = (launch.n + kTileN - 1) / kTileN;
  const bool aligned =
      (reinterpret_cast<uintptr_t>(launch.a) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(launch.b) % 16 == 0) &&
      (reinterpret_cast<uintptr_t>(launch.c) % 16 == 0) && (launch.lda % 4 == 0) &&
      (launch.ldb % 4 == 0) && (launch.ldc % 4 == 0) && launch.padded;
  auto* s = static_cast<hipStream_t>(stream);
  const hipError_t err = aligned ? dispatch_layout<4>(p, launch.a_kcontig, launch.b_ncontig, s)
                                 : dispatch_layout<1>(p, launch.a_kcontig, launch.b_ncontig, s);
  return static_cast<int>(err);
}

} // namespace xvram::kernels
