// sgemm_device.hpp — device-side pieces shared by the tile kernels
// (sgemm_mfma.hip: 256 x 128 tiles, two workgroups per CU; sgemm_wide.hip:
// two kernels of 256 x 256 tiles, one workgroup per CU). Compiled only by hipcc.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace xvram::kernels::device {

typedef float float16_t __attribute__((ext_vector_type(16)));

// One launch, canonical column-major form (see sgemm_launch.hpp).
struct Params {
  const float* a;
  const float* b;
  float* c;
  int64_t lda, ldb, ldc;
  int m, n, k;
  float alpha, beta;
  int tiles_m, tiles_n;
  const float* bias_row; // per-row bias (nullptr = none)
  const float* bias_col; // per-column bias (nullptr = none)
  int relu;
  // Second K panel (ring kernel only): k rows [k_split, k) of A and B come
  // from a2 / b2 (same leading dimensions) instead of a / b; nullptr = none.
  const float* a2;
  const float* b2;
  int k_split;
  // Split K: splits > 1 cuts K into ranges of split_depth; blockIdx.x covers
  // tiles x splits and each workgroup stores its range's raw sums to partial
  // `split` (column-major, ld = m rounded up to 4; partial_target).
  int splits;
  int split_depth;
  float* partial;
};

__device__ __forceinline__ float4 zero4() { return make_float4(0.f, 0.f, 0.f, 0.f); }

// Four consecutive elements of a line starting at `first`; elements at or
// beyond `limit` (and the whole vector when !line_ok) read as 0.
__device__ __forceinline__ float4 load4(const float* __restrict__ line, int first, int limit,
                                        bool line_ok) {
  if (!line_ok || first >= limit) return zero4();
  float4 v = *reinterpret_cast<const float4*>(line + first);
  if (first + 4 > limit) {
    const int left = limit - first;
    if (left < 4) v.w = 0.f;
    if (left < 3) v.z = 0.f;
    if (left < 2) v.y = 0.f;
  }
  return v;
}

// Linear workgroup id -> (tile_m, tile_n): undo the round-robin XCD dispatch
// so XCD x owns ids [x*per, (x+1)*per), then walk tiles in kGroupM-row groups
// (column-major inside a group).
template <int kGroupM>
__device__ __forceinline__ void tile_coords(const Params& p, int& tm, int& tn) {
  const int total = p.tiles_m * p.tiles_n;
  int id = blockIdx.x;
  constexpr int kXcds = 8;
  if ((total % kXcds) == 0) {
    const int per = total / kXcds;
    id = (id % kXcds) * per + id / kXcds;
  }
  const int span = kGroupM * p.tiles_n;
  const int group = id / span;
  const int first_m = group * kGroupM;
  const int rows = min(p.tiles_m - first_m, kGroupM);
  const int in_group = id - group * span;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
}

// Split-K launches: workgroup -> (tile_m, tile_n), returning its K range
// index. Ids are remapped per XCD as in tile_coords; the ids of one range are
// consecutive, so each XCD works on whole ranges and keeps their A and B
// K-slices in its own L2.
template <int kGroupM>
__device__ __forceinline__ int split_coords(const Params& p, int& tm, int& tn) {
  const int tiles = p.tiles_m * p.tiles_n;
  const int total = tiles * p.splits;
  int id = blockIdx.x;
  constexpr int kXcds = 8;
  if ((total % kXcds) == 0) {
    const int per = total / kXcds;
    id = (id % kXcds) * per + id / kXcds;
  }
  const int split = id / tiles;
  id -= split * tiles;
  const int span = kGroupM * p.tiles_n;
  const int group = id / span;
  const int first_m = group * kGroupM;
  const int rows = min(p.tiles_m - first_m, kGroupM);
  const int in_group = id - group * span;
  tm = first_m + in_group % rows;
  tn = in_group / rows;
  return split;
}

// The launch parameters of K range `split` of a split launch: operand bases
// moved to the range's first k (k-contiguous operands by k elements, the
// others by k lines), K = the range's depth.
__device__ __forceinline__ void narrow_to_split(Params& p, int split, bool a_kcontig,
                                                bool b_kcontig) {
  const int k0 = split * p.split_depth;
  p.a += a_kcontig ? (int64_t)k0 : (int64_t)k0 * p.lda;
  p.b += b_kcontig ? (int64_t)k0 : (int64_t)k0 * p.ldb;
  p.k = min(p.split_depth, p.k - k0);
}

// Leading dimension of the partials of a split launch (sgemm_launch.hpp's
// split_partial_ld): m rounded up to 4, so every column is 16-byte aligned.
__host__ __device__ __forceinline__ int64_t partial_ld(int m) { return ((int64_t)m + 3) / 4 * 4; }

// Where a workgroup of a split launch stores its raw sums: its range's
// partial (ld = partial_ld(m)) with alpha 1, beta 0 and no epilogue (1 * x
// is exact).
__device__ __forceinline__ Params partial_target(const Params& p, int split) {
  Params o = p;
  o.ldc = partial_ld(p.m);
  o.c = p.partial + (int64_t)split * o.ldc * p.n;
  o.alpha = 1.f;
  o.beta = 0.f;
  o.bias_row = nullptr;
  o.bias_col = nullptr;
  o.relu = 0;
  return o;
}

// Writes one wave's accumulators: acc[i][j] holds MFMA block (row block i,
// column block j) of v_mfma_f32_32x32x2f32; element v of this lane sits at
// MFMA row 8*(v/4) + 4*lhalf + v%4 and MFMA column lrow, i.e. tile row
// row0 + 4*(that) + i and tile column col0 + kNJ*lrow + j (row blocks and
// column blocks interleaved so one float4 covers four consecutive rows).
// C = alpha*acc + beta*C (C not read when beta == 0), then + bias_row[i] +
// bias_col[j], then ReLU (NaN kept: v < 0 is false). Only in-range elements
// are touched.
//
// A wave whose whole 128 x 32*kNJ region lies inside C takes the interior path:
// no per-element bounds, and the loads of old C (beta != 0), of the column
// biases and of the row biases are issued in batches before any is used, so
// the wave waits for memory once per kBatch columns of its lane instead of
// once per float4 (a serial chain of 16*kNJ round trips that every workgroup of
// a launch would otherwise run at the same moment). Same arithmetic, in the
// same order, as the general path. Row biases are loaded ahead only with
// kRowBiasAhead (64 more registers: the 256 x 256 kernels have them, the
// 256 x 128 kernel at two workgroups per CU does not). store_c_tile uses
// batches of one column (two would make the kernels that also compile the
// general path spill); kernels whose tiles are all interior call
// store_c_interior directly.
template <int kNJ, int kBatch, bool kRowBiasAhead>
__device__ __forceinline__ void store_c_interior(const Params& p, const float16_t (&acc)[4][kNJ],
                                                 int row0, int col0, int lrow, int lhalf) {
  const bool read_c = p.beta != 0.f;
  const bool extra = p.bias_row != nullptr || p.bias_col != nullptr || p.relu != 0;
  const auto row_of = [&](int v) { return row0 + 4 * (8 * (v >> 2) + 4 * lhalf + (v & 3)); };
  float brow[16][4];
  if (kRowBiasAhead && p.bias_row != nullptr) {
#pragma unroll
    for (int v = 0; v < 16; ++v)
#pragma unroll
      for (int t = 0; t < 4; ++t) brow[v][t] = p.bias_row[row_of(v) + t];
  }
  const auto finish = [&](float v, int vi, int t, float bias_c) {
    if (p.bias_row != nullptr) v += kRowBiasAhead ? brow[vi][t] : p.bias_row[row_of(vi) + t];
    v += bias_c;
    return (p.relu != 0 && v < 0.f) ? 0.f : v;
  };
  static_assert(kNJ % kBatch == 0, "columns come in whole batches");
#pragma unroll
  for (int j0 = 0; j0 < kNJ; j0 += kBatch) {
    float4 old[kBatch][16];
    float bias_c[kBatch];
#pragma unroll
    for (int jb = 0; jb < kBatch; ++jb) {
      const int col = col0 + kNJ * lrow + j0 + jb;
      bias_c[jb] = p.bias_col != nullptr ? p.bias_col[col] : 0.f;
      if (read_c) {
        const float* cline = p.c + (int64_t)col * p.ldc;
#pragma unroll
        for (int v = 0; v < 16; ++v) old[jb][v] = *reinterpret_cast<const float4*>(cline + row_of(v));
      }
    }
#pragma unroll
    for (int jb = 0; jb < kBatch; ++jb) {
      const int j = j0 + jb;
      float* cline = p.c + (int64_t)(col0 + kNJ * lrow + j) * p.ldc;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float4 r;
        if (read_c) {
          r.x = p.alpha * acc[0][j][v] + p.beta * old[jb][v].x;
          r.y = p.alpha * acc[1][j][v] + p.beta * old[jb][v].y;
          r.z = p.alpha * acc[2][j][v] + p.beta * old[jb][v].z;
          r.w = p.alpha * acc[3][j][v] + p.beta * old[jb][v].w;
        } else {
          r.x = p.alpha * acc[0][j][v];
          r.y = p.alpha * acc[1][j][v];
          r.z = p.alpha * acc[2][j][v];
          r.w = p.alpha * acc[3][j][v];
        }
        if (extra) {
          r.x = finish(r.x, v, 0, bias_c[jb]);
          r.y = finish(r.y, v, 1, bias_c[jb]);
          r.z = finish(r.z, v, 2, bias_c[jb]);
          r.w = finish(r.w, v, 3, bias_c[jb]);
        }
        *reinterpret_cast<float4*>(cline + row_of(v)) = r;
      }
    }
  }
}

template <int kNJ, bool kRowBiasAhead>
__device__ __forceinline__ void store_c_tile(const Params& p, const float16_t (&acc)[4][kNJ],
                                             int row0, int col0, int lrow, int lhalf) {
  if (row0 + 128 <= p.m && col0 + 32 * kNJ <= p.n) {
    store_c_interior<kNJ, 1, kRowBiasAhead>(p, acc, row0, col0, lrow, lhalf);
    return;
  }
  const bool read_c = p.beta != 0.f;
  const bool extra = p.bias_row != nullptr || p.bias_col != nullptr || p.relu != 0;
  const auto finish = [&](float v, int r, float bias_c) {
    if (p.bias_row != nullptr) v += p.bias_row[r];
    v += bias_c;
    return (p.relu != 0 && v < 0.f) ? 0.f : v;
  };
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const int col = col0 + kNJ * lrow + j;
    if (col >= p.n) continue;
    float* cline = p.c + (int64_t)col * p.ldc;
    const float bias_c = p.bias_col != nullptr ? p.bias_col[col] : 0.f;
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      const int mrow = 8 * (v >> 2) + 4 * lhalf + (v & 3);
      const int row = row0 + 4 * mrow;
      if (row >= p.m) continue;
      const float out[4] = {acc[0][j][v], acc[1][j][v], acc[2][j][v], acc[3][j][v]};
      if (row + 4 <= p.m) {
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
        if (extra) {
          r.x = finish(r.x, row, bias_c);
          r.y = finish(r.y, row + 1, bias_c);
          r.z = finish(r.z, row + 2, bias_c);
          r.w = finish(r.w, row + 3, bias_c);
        }
        *dst = r;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          if (row + t < p.m) {
            const float val = p.alpha * out[t];
            const float sum = read_c ? val + p.beta * cline[row + t] : val;
            cline[row + t] = extra ? finish(sum, row + t, bias_c) : sum;
          }
        }
      }
    }
  }
}

} // namespace xvram::kernels::device
