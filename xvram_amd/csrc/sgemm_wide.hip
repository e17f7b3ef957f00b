// sgemm_wide.hip — the 256 x 256 tile kernel used for large launches on gfx950.
//
// Same contract as the 256 x 128 kernel in sgemm_mfma.hip (which dispatches
// here): C = alpha * op(A) * op(B) + beta * C with FP32 matrix instructions
// (v_mfma_f32_32x32x2_f32), the optional bias / ReLU epilogue, exact zeros for
// out-of-range rows, columns and k in both operands, and only in-range C
// elements stored. Organised for one workgroup per CU:
//
//   * workgroup = 4 waves; wave w owns a 128 x 128 sub-tile = 4 x 4 MFMA blocks
//     whose 256 accumulator registers live in AGPRs. Row blocks and column
//     blocks are interleaved (MFMA row r of row block i is wave row 4r+i, MFMA
//     column c of column block j is wave column 4c+j), so one ds_read_b128
//     feeds four blocks of each operand;
//   * K advances in stages of 16 through three LDS buffers: stage s+2 is loaded
//     while stage s is multiplied. An operand whose tile extent is contiguous
//     in memory (m for op-N A, n for op-T B) is loaded straight into LDS
//     (buffer_load_dwordx4 ... lds: one 256-float k-row per wave instruction,
//     rows unpadded); a k-contiguous operand goes through registers and
//     transposing LDS stores into rows padded by 4 floats (distinct banks);
//   * every load of the steady state uses a buffer descriptor over the tile's
//     operand panel: the per-lane offsets are fixed and the stage advance is a
//     scalar offset, so the loop issues no 64-bit vector address arithmetic
//     (which measurably delays MFMA issue on this chip). The descriptor's
//     record count also makes any read past the panel return zeros;
//   * the stage's eight loads are spread over the first MFMAs of the stage
//     rather than issued as a burst; the single barrier per stage sits before
//     the second half of the last k-pair, whose MFMAs cover the next stage's
//     first fragment reads;
//   * edge tiles and the last stages run a register-staged loop with
//     predicated loads; workgroup ids are remapped per XCD as in the 256 x 128
//     kernel.
//
// The host uses this kernel only when every operand panel spans less than
// 2^31 bytes from a tile's base (32-bit buffer offsets) and the launch has at
// least one tile per CU. N/T launches whose tiles are all interior and whose K
// is a multiple of 4 run sgemm_ring_kernel instead (below): the same tile and
// MFMA sequence with each wave streaming its own operand halves through a
// private LDS ring, so its K loop needs no workgroup barrier. Launches of the
// other three forms with interior tiles and K a multiple of 8 run
// sgemm_ring8_kernel, the same ring scheme with k-contiguous halves loaded
// straight into LDS as well.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <type_traits>
#include <utility>

#include "sgemm_device.hpp"

namespace xvram::kernels {
namespace {

using namespace device;

constexpr int kThreads = 256;
constexpr int kTile = 256;     // rows and columns of C per workgroup
constexpr int kStageK = 16;
constexpr int kWave = 128;     // rows and columns of C per wave
constexpr int kGroupM = 8;
constexpr int kLoads = kTile * kStageK / 4 / kThreads; // float4 per thread per operand per stage
constexpr int kLoadStep = 3;   // MFMAs between consecutive loads at the start of a stage
constexpr int kPairs = kStageK / 4;
static_assert(kLoads == 4 && kLoadStep * 2 * kLoads <= 32, "loads fit in the first k-pair");

// LDS row pitch in floats: unpadded for rows written whole (direct loads and
// float4 stores of extent-contiguous operands), padded for transposing stores.
template <bool KC> constexpr int kPitch = KC ? kTile + 4 : kTile;

template <int N> using Int = std::integral_constant<int, N>;

struct Half {
  float4 v[kLoads];
};

// Thread -> element map of one operand's stage (f = tid + r*256):
//   extent-contiguous (KC = false): k-row f/64, elements (f%64)*4..+3
//   k-contiguous      (KC = true) : element f/4, k (f%4)*4..+3
template <bool KC>
__device__ __forceinline__ void load_edge(const float* base, int64_t ld, int e0, int extent, int k0,
                                          int k, int tid, Half& h) {
#pragma unroll
  for (int r = 0; r < kLoads; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (!KC) {
      const int kk = f / (kTile / 4), ee = (f % (kTile / 4)) * 4, kg = k0 + kk;
      h.v[r] = load4(base + (int64_t)kg * ld + e0, ee, extent - e0, kg < k);
    } else {
      const int ee = f / (kStageK / 4), kk = (f % (kStageK / 4)) * 4, eg = e0 + ee;
      h.v[r] = load4(base + (int64_t)eg * ld + k0, kk, k - k0, eg < extent);
    }
  }
}

// Interior stage; `p` points at this thread's first element of the stage.
template <bool KC>
__device__ __forceinline__ void load_full(const float* __restrict__ p, int64_t ld, Half& h) {
#pragma unroll
  for (int r = 0; r < kLoads; ++r) {
    const int64_t off = KC ? (int64_t)(r * (kThreads / (kStageK / 4))) * ld
                           : (int64_t)(r * (kThreads / (kTile / 4))) * ld;
    h.v[r] = *reinterpret_cast<const float4*>(p + off);
  }
}

template <bool KC>
__device__ __forceinline__ void store_half(float* __restrict__ l, int tid, const Half& h) {
  constexpr int P = kPitch<KC>;
#pragma unroll
  for (int r = 0; r < kLoads; ++r) {
    const int f = tid + r * kThreads;
    if constexpr (!KC) {
      const int kk = f / (kTile / 4), ee = (f % (kTile / 4)) * 4;
      *reinterpret_cast<float4*>(l + kk * P + ee) = h.v[r];
    } else {
      const int ee = f / (kStageK / 4), kk = (f % (kStageK / 4)) * 4;
      l[(kk + 0) * P + ee] = h.v[r].x;
      l[(kk + 1) * P + ee] = h.v[r].y;
      l[(kk + 2) * P + ee] = h.v[r].z;
      l[(kk + 3) * P + ee] = h.v[r].w;
    }
  }
}

// Raw buffer descriptor (no stride, 32-bit data format word) over `bytes`
// bytes from `base`; reads at or past `bytes` return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t panel_rsrc(const float* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// One wave-wide direct load: lane l's 16 bytes at rsrc.base + soff + voff land
// at LDS byte address lds_base + kOff + 16*l (lds_base wave-uniform). Counted
// by vmcnt only: the caller waits on vmcnt before the data is read (and, when
// other waves read it, before the barrier that publishes it).
template <int kOff>
__device__ __forceinline__ void load_lds16(uint32_t lds_base, uint32_t voff,
                                           __amdgpu_buffer_rsrc_t rsrc, uint32_t soff) {
  asm volatile("s_add_u32 m0, %0, %4\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :: "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff), "i"(kOff)
               : "memory", "m0", "scc");
}

__device__ __forceinline__ float4 load_reg16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff,
                                             uint32_t soff) {
  return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rsrc, voff, soff, 0));
}

__device__ __forceinline__ uint32_t lds_byte_addr(const float* p) {
  return __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
}

template <bool AK, bool BN>
__global__ __launch_bounds__(kThreads, 1) void sgemm_wide_kernel(Params p) {
  constexpr bool kDirectA = !AK; // m-contiguous A: straight into LDS
  constexpr bool kDirectB = BN;  // n-contiguous B: straight into LDS
  constexpr int kPA = kPitch<AK>;
  constexpr int kPB = kPitch<!BN>;
  constexpr int kBufA = kStageK * kPA;
  constexpr int kBuf = kBufA + kStageK * kPB;
  constexpr int kDirect = (kDirectA ? kLoads : 0) + (kDirectB ? kLoads : 0);
  __shared__ __attribute__((aligned(16))) float lds[3 * kBuf];

  // The MFMAs take their accumulators in AGPRs (256 per lane), leaving the
  // architectural VGPRs to fragments, staging and addresses.
  asm volatile("; accumulators in AGPRs" ::: "a0");

  int tile_m, tile_n;
  tile_coords<kGroupM>(p, tile_m, tile_n);
  const int m0 = tile_m * kTile;
  const int n0 = tile_n * kTile;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave & 1) * kWave;
  const int wn = (wave >> 1) * kWave;
  const int lrow = lane & 31;  // MFMA row (A) / column (B) of this lane
  const int lhalf = lane >> 5; // which of the MFMA's two k values

  float16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int stages = (p.k + kStageK - 1) / kStageK;
  const int full_stages = p.k / kStageK;
  const bool interior = m0 + kTile <= p.m && n0 + kTile <= p.n;
  const float* pa = AK ? p.a + (int64_t)(m0 + tid / (kStageK / 4)) * p.lda + (tid % (kStageK / 4)) * 4
                       : p.a + (int64_t)(tid / (kTile / 4)) * p.lda + m0 + (tid % (kTile / 4)) * 4;
  const float* pb = BN ? p.b + (int64_t)(tid / (kTile / 4)) * p.ldb + n0 + (tid % (kTile / 4)) * 4
                       : p.b + (int64_t)(n0 + tid / (kStageK / 4)) * p.ldb + (tid % (kStageK / 4)) * 4;
  const int64_t a_step = AK ? kStageK : (int64_t)kStageK * p.lda;
  const int64_t b_step = BN ? (int64_t)kStageK * p.ldb : kStageK;

  auto lds_a = [&](int buf) { return lds + buf * kBuf; };
  auto lds_b = [&](int buf) { return lds + buf * kBuf + kBufA; };

  Half ha, hb;
  auto load_any = [&](int stg) {
    load_edge<AK>(p.a, p.lda, m0, p.m, stg * kStageK, p.k, tid, ha);
    load_edge<!BN>(p.b, p.ldb, n0, p.n, stg * kStageK, p.k, tid, hb);
  };
  auto store_any = [&](int buf) {
    store_half<AK>(lds_a(buf), tid, ha);
    store_half<!BN>(lds_b(buf), tid, hb);
  };

  load_any(0);
  store_any(0);
  if (stages > 1) {
    load_any(1);
    store_any(1);
  }
  __syncthreads();

  float4 fa[2][2], fb[2][2];
  // Fragments of the k-pair (kk, kk+2) into `slot`.
  auto read_pair = [&](const float* la, const float* lb, int kk, int slot) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int krow = kk + 2 * t + lhalf;
      fa[slot][t] = *reinterpret_cast<const float4*>(la + wm + 4 * lrow + krow * kPA);
      fb[slot][t] = *reinterpret_cast<const float4*>(lb + wn + 4 * lrow + krow * kPB);
    }
  };
  // MFMAs number from..to-1 of a k-pair: x = 16*t + 4*i + j.
  auto mfma_range = [&](int slot, int from, int to) {
#pragma unroll
    for (int x = 0; x < 32; ++x) {
      if (x < from || x >= to) continue;
      const int t = x / 16, i = (x % 16) / 4, j = x % 4;
      const float4 a = fa[slot][t], b = fb[slot][t];
      const float ao = i == 0 ? a.x : i == 1 ? a.y : i == 2 ? a.z : a.w;
      const float bo = j == 0 ? b.x : j == 1 ? b.y : j == 2 ? b.z : b.w;
      acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ao, bo, acc[i][j], 0, 0, 0);
    }
  };
  read_pair(lds_a(0), lds_b(0), 0, 0);
  int st = 0;

  if (interior) {
    // Buffer descriptors over this tile's panels. A(i, k) sits at byte
    // 4*((i-m0)*lda + k) (op T) or 4*(k*lda + i-m0) (op N) from a + m0*lda or
    // a + m0; B likewise from b + n0 (op T) or b + n0*ldb (op N).
    const float* a_base = AK ? p.a + (int64_t)m0 * p.lda : p.a + m0;
    const float* b_base = BN ? p.b + n0 : p.b + (int64_t)n0 * p.ldb;
    const int64_t a_bytes = AK ? (int64_t)(p.m - m0) * p.lda * 4 : ((int64_t)p.k * p.lda - m0) * 4;
    const int64_t b_bytes = BN ? ((int64_t)p.k * p.ldb - n0) * 4 : (int64_t)(p.n - n0) * p.ldb * 4;
    const __amdgpu_buffer_rsrc_t rs_a = panel_rsrc(a_base, (uint32_t)a_bytes);
    const __amdgpu_buffer_rsrc_t rs_b = panel_rsrc(b_base, (uint32_t)b_bytes);
    // Per-lane byte offsets of load r in stage 0, and the byte advance per stage.
    uint32_t vo_a[kLoads], vo_b[kLoads];
#pragma unroll
    for (int r = 0; r < kLoads; ++r) {
      vo_a[r] = kDirectA ? (uint32_t)(((int64_t)(wave + 4 * r) * p.lda + lane * 4) * 4)
                         : (uint32_t)(((int64_t)(tid / 4 + 64 * r) * p.lda + (tid % 4) * 4) * 4);
      vo_b[r] = kDirectB ? (uint32_t)(((int64_t)(wave + 4 * r) * p.ldb + lane * 4) * 4)
                         : (uint32_t)(((int64_t)(tid / 4 + 64 * r) * p.ldb + (tid % 4) * 4) * 4);
    }
    const uint32_t a_stage_bytes = (uint32_t)(kDirectA ? kStageK * p.lda * 4 : kStageK * 4);
    const uint32_t b_stage_bytes = (uint32_t)(kDirectB ? kStageK * p.ldb * 4 : kStageK * 4);
    // LDS byte address of this wave's first direct-load row in buffer 0.
    const uint32_t lds_a_wave = lds_byte_addr(lds + wave * kPA);
    const uint32_t lds_b_wave = lds_byte_addr(lds + kBufA + wave * kPB);

    // Load r (A for r < kLoads, else B) of stage `stg` into buffer `far`.
    auto issue = [&]<int far, int r>(int stg, Int<far>, Int<r>) {
      if constexpr (r < kLoads) {
        const uint32_t so = __builtin_amdgcn_readfirstlane(a_stage_bytes * (uint32_t)stg);
        if constexpr (kDirectA)
          load_lds16<(far * kBuf + r * 4 * kPA) * 4>(lds_a_wave, vo_a[r], rs_a, so);
        else
          ha.v[r] = load_reg16(rs_a, vo_a[r], so);
      } else {
        const uint32_t so = __builtin_amdgcn_readfirstlane(b_stage_bytes * (uint32_t)stg);
        if constexpr (kDirectB)
          load_lds16<(far * kBuf + (r - kLoads) * 4 * kPB) * 4>(lds_b_wave, vo_b[r - kLoads],
                                                                          rs_b, so);
        else
          hb.v[r - kLoads] = load_reg16(rs_b, vo_b[r - kLoads], so);
      }
    };
    // One stage: multiply stage stg from buffer cur while stage stg+2 loads
    // into buffer far; end with stage stg+1's first fragments read from nxt.
    auto body = [&]<int cur, int nxt, int far>(int stg, Int<cur>, Int<nxt>, Int<far> far_t) {
      auto one_mfma = [&]<int Q, int X>(Int<Q>, Int<X>) {
        constexpr int g = Q * 32 + X;
        if constexpr (g % kLoadStep == 0 && g / kLoadStep < 2 * kLoads) {
          __builtin_amdgcn_sched_barrier(0);
          issue(stg + 2, far_t, Int<g / kLoadStep>{});
          __builtin_amdgcn_sched_barrier(0);
        }
        mfma_range(Q & 1, X, X + 1);
      };
      auto pair = [&]<int Q>(Int<Q> q) {
        read_pair(lds_a(cur), lds_b(cur), 4 * (Q + 1), (Q + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
        [&]<int... X>(std::integer_sequence<int, X...>) {
          (one_mfma(q, Int<X>{}), ...);
        }(std::make_integer_sequence<int, 32>{});
        __builtin_amdgcn_sched_barrier(0);
      };
      [&]<int... Q>(std::integer_sequence<int, Q...>) {
        (pair(Int<Q>{}), ...);
      }(std::make_integer_sequence<int, kPairs - 1>{});
      if constexpr (!kDirectA) store_half<true>(lds_a(far), tid, ha);
      if constexpr (!kDirectB) store_half<true>(lds_b(far), tid, hb);
      mfma_range((kPairs - 1) & 1, 0, 16);
      __builtin_amdgcn_sched_barrier(0);
      // Stage stg+1's direct loads were issued a stage earlier than this
      // stage's kDirect ones; loads complete in order.
      if constexpr (kDirect == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
      else if constexpr (kDirect == 4) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
      __syncthreads();
      read_pair(lds_a(nxt), lds_b(nxt), 0, 0);
      mfma_range((kPairs - 1) & 1, 16, 32);
    };
    // Stages 0 and 1 are in LDS; each body needs stages stg..stg+2 full.
    for (; st + 4 < full_stages; st += 3) {
      body(st, Int<0>{}, Int<1>{}, Int<2>{});
      body(st + 1, Int<1>{}, Int<2>{}, Int<0>{});
      body(st + 2, Int<2>{}, Int<0>{}, Int<1>{});
    }
  }

  // Remaining stages (every stage of an edge tile): stage st+2 is staged
  // through registers while st runs; stage st+1 is in LDS or in flight.
  for (; st < stages; ++st) {
    const int cur = st % 3, nxt = (st + 1) % 3, far = (st + 2) % 3;
    const bool more2 = st + 2 < stages;
    if (more2) {
      if (interior && st + 2 < full_stages) {
        load_full<AK>(pa + (st + 2) * a_step, p.lda, ha);
        load_full<!BN>(pb + (st + 2) * b_step, p.ldb, hb);
      } else {
        load_any(st + 2);
      }
    }
#pragma unroll
    for (int q = 0; q < kPairs - 1; ++q) {
      read_pair(lds_a(cur), lds_b(cur), 4 * (q + 1), (q + 1) & 1);
      mfma_range(q & 1, 0, 32);
    }
    if (more2) store_any(far);
    if constexpr (kDirect > 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (st + 1 < stages) read_pair(lds_a(nxt), lds_b(nxt), 0, 0);
    mfma_range((kPairs - 1) & 1, 0, 32);
  }

  store_c_tile<4, true>(p, acc, m0 + wm, n0 + wn, lrow, lhalf);
}

// ---- barrier-free N/T kernel ------------------------------------------------
//
// When both operands are extent-contiguous (A op N, B op T) every operand load
// can go straight into LDS, and each wave can stream the two 128-wide halves it
// multiplies (its A rows and its B columns) into an LDS ring of its own: no
// data is shared between waves, so the K loop has no workgroup barrier at all,
// only per-wave waits on the wave's own loads. Each half is loaded by the two
// waves that use it (L2 serves the second read; L2 -> LDS traffic doubles, HBM
// traffic does not change). The MFMA sequence per accumulator is the one of
// sgemm_wide_kernel<false, true>, so both produce bit-identical C.
//
// Per wave, a ring of kRing slots; slot s holds one k-pair (4 k-rows) of the
// wave's A half (4 x 128 floats) followed by its B half (4 x 128). Step q
// multiplies pair q from registers, reads pair q+1's fragments from LDS and
// issues pair q+kAhead's four loads (two per operand, each a wave-wide
// buffer_load_dwordx4 ... lds of two 128-float k-rows) into the slot pair q-1
// vacated: pair q-1's fragments were consumed by step q-1's MFMAs, so its reads
// have completed. Loads complete in order, so before reading pair q+1 the wave
// waits until at most the loads of pairs q+2 .. q+kAhead-1 are outstanding.
//
// K must be a multiple of 4. In the instances for interior tiles (m and n
// multiples of 256) every load stays inside the tile's rows and columns and
// inside the K extent (the last load of the last pair ends at or before the
// panel's record count), so no predication is needed. Edge instance (kEdge,
// one panel, unsplit): a tile may reach past row m or column n. A lane whose
// four elements would start past the operand's last whole float4 (rows up to
// m rounded up to 4, which the leading dimension covers) loads that float4
// instead; the copies feed only rows or columns of C past m or n, which the
// predicated store leaves alone. The loads of a lane keep one offset over
// the whole K loop, so the K loop is the interior one.
//
// Two-panel instance (kTwo): the launch's K rows come from two separately
// stored panels with the same leading dimensions, [0, k_split) from a / b and
// [k_split, k) from a2 / b2, one buffer descriptor pair each; a C tile then
// takes two K panels per pass through HBM (one read and one write of C, one
// prologue) instead of one. Only the loads' source changes, so C is bit-identical
// to a one-panel launch over the same K.
//
// Split instance (kSplit): workgroup ids cover tiles x K ranges
// (split_coords); each workgroup narrows its operands to its range and stores
// raw sums to its range's partial (partial_target), which
// splitk_reduce_kernel adds up. The one-panel instance carries none of this.
constexpr int kRing = 8;   // slots (k-pairs) per wave
constexpr int kAhead = 7;  // prefetch distance in k-pairs
constexpr int kSlot = 1024; // floats per slot: A 4 x 128, then B 4 x 128
static_assert(kAhead == kRing - 1, "loads reuse the slot vacated one step earlier");
static_assert(4 * kAhead <= 63, "outstanding loads fit the vmcnt counter");
static_assert(4 * (kAhead - 2) == 20, "steady-state wait below");

// One K panel's buffer descriptors for A and B; pair q of the launch is pair
// q - base of that panel.
struct RingSource {
  __amdgpu_buffer_rsrc_t a, b;
  int base;
  int count = 0;  // sgemm_ring8_kernel: K slots of this panel
  int rotate = 0; // sgemm_ring8_kernel: slot loaded first (< count)
};

// First element of a lane's float4 in an extent-contiguous operand half:
// element w + 4*lrow of the tile, or, for an edge tile with `extent` elements
// left in the operand, at most the last whole float4 below extent rounded up
// to 4 (extent >= 1).
template <bool kEdge>
__device__ __forceinline__ int lane_elem(int w, int lrow, int extent) {
  const int e = w + 4 * lrow;
  if constexpr (kEdge) return min(e, ((extent + 3) & ~3) - 4);
  else return e;
}

template <bool kTwo, bool kSplit, bool kEdge>
__global__ __launch_bounds__(kThreads, 1) void sgemm_ring_kernel(Params p) {
  static_assert(!(kTwo && kSplit), "a two-panel launch never splits");
  static_assert(!(kEdge && (kTwo || kSplit)), "edge tiles run one-panel, unsplit launches");
  __shared__ __attribute__((aligned(16))) float lds[4 * kRing * kSlot];
  asm volatile("; accumulators in AGPRs" ::: "a0");

  int tile_m, tile_n, split = 0;
  if constexpr (kSplit) {
    split = split_coords<kGroupM>(p, tile_m, tile_n);
    narrow_to_split(p, split, false, false); // A op N, B op T: K runs along lines
  } else {
    tile_coords<kGroupM>(p, tile_m, tile_n);
  }
  const int m0 = tile_m * kTile;
  const int n0 = tile_n * kTile;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave & 1) * kWave;
  const int wn = (wave >> 1) * kWave;
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;

  float16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int pairs = p.k / 4;
  // A(i, k) sits at byte 4*(k*lda + i-m0) from a + m0, B(k, j) at
  // 4*(k*ldb + j-n0) from b + n0. kTwo: k rows [0, k_split) come from a / b
  // and rows [k_split, k) from a2 / b2 (row k_split is their row 0); k_split
  // is a multiple of 4 * kRing, so every block of kRing steps below loads from
  // at most two sources, fixed per block.
  const int k1 = kTwo ? p.k_split : p.k;
  const int q_split = k1 / 4;
  const RingSource lo{panel_rsrc(p.a + m0, (uint32_t)(((int64_t)k1 * p.lda - m0) * 4)),
                      panel_rsrc(p.b + n0, (uint32_t)(((int64_t)k1 * p.ldb - n0) * 4)), 0};
  RingSource hi = lo;
  if constexpr (kTwo) {
    const int k2 = p.k - k1;
    hi = RingSource{panel_rsrc(p.a2 + m0, (uint32_t)(((int64_t)k2 * p.lda - m0) * 4)),
                    panel_rsrc(p.b2 + n0, (uint32_t)(((int64_t)k2 * p.ldb - n0) * 4)), q_split};
  }
  // Load h of a pair: lane l brings k-row 2h + l/32 of the pair, elements
  // 4*(l%32) .. +3 of the wave's half; it lands at LDS byte 1024*h + 16*l of
  // the operand's part of the slot, i.e. row-major 4 x 128.
  const int ea = lane_elem<kEdge>(wm, lrow, p.m - m0);
  const int eb = lane_elem<kEdge>(wn, lrow, p.n - n0);
  uint32_t vo_a[2], vo_b[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    vo_a[h] = (uint32_t)(((int64_t)(2 * h + lhalf) * p.lda + ea) * 4);
    vo_b[h] = (uint32_t)(((int64_t)(2 * h + lhalf) * p.ldb + eb) * 4);
  }
  const uint32_t pair_a = (uint32_t)(16 * p.lda);
  const uint32_t pair_b = (uint32_t)(16 * p.ldb);
  float* ring = lds + wave * (kRing * kSlot);
  const uint32_t ring_lds = lds_byte_addr(ring);

  // Load L (0, 1: A halves; 2, 3: B halves) of pair q into slot S.
  auto issue = [&]<int S, int L>(int q, Int<S>, Int<L>, const RingSource& src) {
    constexpr int off = (S * kSlot + (L >> 1) * 512 + (L & 1) * 256) * 4;
    const uint32_t qq = (uint32_t)(q - src.base);
    if constexpr (L < 2) {
      const uint32_t so = __builtin_amdgcn_readfirstlane(pair_a * qq);
      load_lds16<off>(ring_lds, vo_a[L & 1], src.a, so);
    } else {
      const uint32_t so = __builtin_amdgcn_readfirstlane(pair_b * qq);
      load_lds16<off>(ring_lds, vo_b[L & 1], src.b, so);
    }
  };
  // Fragments of one pair: rows 2t + lhalf, four consecutive floats at 4*lrow
  // (the same element map as sgemm_wide_kernel's read_pair).
  float4 fa[2][2], fb[2][2];
  auto read_frag = [&]<int S, int R>(Int<S>, Int<R>) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const float* row = ring + S * kSlot + (2 * t + lhalf) * kWave + 4 * lrow;
      fa[R][t] = *reinterpret_cast<const float4*>(row);
      fb[R][t] = *reinterpret_cast<const float4*>(row + 512);
    }
  };
  auto mfma_one = [&]<int R, int X>(Int<R>, Int<X>) {
    constexpr int t = X / 16, i = (X % 16) / 4, j = X % 4;
    const float4 a = fa[R][t], b = fb[R][t];
    const float ao = i == 0 ? a.x : i == 1 ? a.y : i == 2 ? a.z : a.w;
    const float bo = j == 0 ? b.x : j == 1 ? b.y : j == 2 ? b.z : b.w;
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ao, bo, acc[i][j], 0, 0, 0);
  };

  // Pairs 0 .. kAhead-1 in flight, then pair 0's fragments in registers: with
  // all kAhead pairs issued, only pair 0's four loads need to have landed.
  [&]<int... I>(std::integer_sequence<int, I...>) {
    ((I < pairs ? (issue(I, Int<I % kRing>{}, Int<0>{}, lo), issue(I, Int<I % kRing>{}, Int<1>{}, lo),
                   issue(I, Int<I % kRing>{}, Int<2>{}, lo), issue(I, Int<I % kRing>{}, Int<3>{}, lo), 0)
                : 0),
     ...);
  }(std::make_integer_sequence<int, kAhead>{});
  static_assert(4 * (kAhead - 1) == 24, "prologue wait below");
  if (pairs >= kAhead) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  read_frag(Int<0>{}, Int<0>{});

  // Step q, q % kRing == J. kTail: the last steps, which may issue no loads
  // (and so wait for all outstanding ones) and may have no next pair.
  // Step J of a block (q % kRing == J) loads pair q + kAhead: from `first`
  // for J == 0, from `rest` for the others (pairs q - J + kRing ..).
  auto step = [&]<int J, bool kTail>(int q, Int<J>, std::bool_constant<kTail>,
                                      const RingSource& first, const RingSource& rest) {
    constexpr int cur = J & 1, nxt = (J + 1) & 1;
    constexpr int s_next = (J + 1) % kRing, s_load = (J + kAhead) % kRing;
    if constexpr (!kTail) asm volatile("s_waitcnt vmcnt(20)" ::: "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (!kTail || q + 1 < pairs) read_frag(Int<s_next>{}, Int<nxt>{});
    __builtin_amdgcn_sched_barrier(0);
    const bool load = !kTail || q + kAhead < pairs;
    [&]<int... X>(std::integer_sequence<int, X...>) {
      (([&] {
         if constexpr (X % 8 == 0) {
           if (load) {
             __builtin_amdgcn_sched_barrier(0);
             if constexpr (J == 0) issue(q + kAhead, Int<s_load>{}, Int<X / 8>{}, first);
             else issue(q + kAhead, Int<s_load>{}, Int<X / 8>{}, rest);
             __builtin_amdgcn_sched_barrier(0);
           }
         }
         mfma_one(Int<cur>{}, Int<X>{});
       }()),
       ...);
    }(std::make_integer_sequence<int, 32>{});
    __builtin_amdgcn_sched_barrier(0);
  };

  // The block starting at q (a multiple of kRing) loads pair q + kAhead in its
  // first step and pairs q + kRing .. in the rest; q_split is a multiple of
  // kRing, so each of the two groups lies wholly in one panel: blocks before
  // q_split - kRing load from `lo` only, the block at q_split - kRing loads its
  // first step's pair from `lo` and the rest from `hi`, and later blocks load
  // from `hi` only. Each phase runs its own loop with fixed sources (a choice
  // per block inside one loop cost 0.45 % of the K loop).
  static_assert(kAhead + 1 == kRing, "the first step loads the last pair of its block");
  const auto source = [&](int pair) -> RingSource {
    if constexpr (kTwo) return pair < q_split ? lo : hi;
    else return lo;
  };
  const auto block = [&](int q0, const RingSource& first, const RingSource& rest) {
    [&]<int... J>(std::integer_sequence<int, J...>) {
      (step(q0 + J, Int<J>{}, std::false_type{}, first, rest), ...);
    }(std::make_integer_sequence<int, kRing>{});
  };
  int q = 0;
  // Full blocks of kRing steps whose loads all exist (q + kRing - 1 + kAhead < pairs).
  if constexpr (kTwo) {
    for (; q + kRing < q_split && q + kRing + kAhead <= pairs; q += kRing) block(q, lo, lo);
    if (q + kRing == q_split && q + kRing + kAhead <= pairs) {
      block(q, lo, hi);
      q += kRing;
    }
    if (q >= q_split)
      for (; q + kRing + kAhead <= pairs; q += kRing) block(q, hi, hi);
  } else {
    for (; q + kRing + kAhead <= pairs; q += kRing) block(q, lo, lo);
  }
  for (; q < pairs; q += kRing) {
    const RingSource first = source(q + kAhead);
    const RingSource rest = source(q + kRing);
    [&]<int... J>(std::integer_sequence<int, J...>) {
      ((q + J < pairs ? (step(q + J, Int<J>{}, std::true_type{}, first, rest), 0) : 0), ...);
    }(std::make_integer_sequence<int, kRing>{});
  }

  // Interior tiles: two columns of C per batch of loads. A split launch
  // stores its range's raw sums instead. Edge tiles: only elements of C.
  const Params out = kSplit ? partial_target(p, split) : p;
  if constexpr (kEdge) store_c_tile<4, false>(out, acc, m0 + wm, n0 + wn, lrow, lhalf);
  else store_c_interior<4, 2, true>(out, acc, m0 + wm, n0 + wn, lrow, lhalf);
}

// ---- barrier-free kernel for layouts with a k-contiguous operand ------------
//
// The ring scheme above for N/N, T/N and T/T launches. An extent-contiguous
// half (op-N A, op-T B) is loaded as k-rows as there; a k-contiguous one
// (op-T A, op-N B) as 32-byte pieces of its lines: lane (lrow, h) of load I
// brings k values 4h .. 4h+3 of line 4*lrow + I of the wave's half, so one
// load covers the 32 lines that feed MFMA block I. A slot holds 8 k values
// of both halves of the wave:
//   extent-contiguous: row-major 8 x 128 (k-row, element), as loaded;
//   k-contiguous:      lane (lrow, h)'s piece of block I's line at float
//                      256*I + 128*h + 4*lrow, as loaded.
// The MFMAs of a slot run k-steps s = 0..3 with lane half h supplying k value
// 4h + s (one fixed order of the slot's 8 k values, the same for both
// operands): one ds_read_b128 of a k-contiguous half gives a lane its values
// of one block for all four k-steps, one of an extent-contiguous half its
// values of one k-step for all four blocks. Every fragment read and every
// load covers 64 consecutive 16-byte LDS units in runs of 32 (no bank
// conflicts).
//
// Per wave kRing8 slots of 8 KB (128 KB per workgroup). Step q multiplies
// slot q from registers; during its first 32 MFMAs it issues slot q+kRing8's
// eight loads into the ring slot of q, whose fragments were read half a step
// earlier; after them it waits for slot q+1 and reads its fragments into the
// other register set. A block of kRing8 steps loads the kRing8 slots of the
// next block, so with k_split a multiple of 8 * kRing8 (two-panel instance,
// as in sgemm_ring_kernel) each block's loads come from one K panel.
//
// K must be a multiple of 8. In the instances for interior tiles (m and n
// multiples of 256) every load stays inside the tile's lines and the K
// extent, so no predication is needed. Edge instance (kEdge, one panel,
// unsplit): an extent-contiguous half clamps its lanes' elements as
// sgemm_ring_kernel does, a k-contiguous half its lines to the operand's last
// line (m - 1 or n - 1), and that half's descriptor ends after the last line;
// the copies feed only rows or columns of C that the predicated store skips.
constexpr int kRing8 = 4;       // slots per wave
constexpr int kSlotK = 8;       // k values per slot
constexpr int kHalf8 = 1024;    // floats of one operand half per slot (128 x 8)
constexpr int kTurnClasses = 8; // rotated K order (op-T A): tile rows per cycle of turns
constexpr int kTurnSlots = 8;   // slots between the turns of consecutive tile rows (256 B)
static_assert(4 * kRing8 * 2 * kHalf8 * 4 <= 160 * 1024, "rings fit the LDS");
static_assert(8 * kRing8 <= 63, "outstanding loads fit the vmcnt counter");
static_assert(8 * kRing8 == 32, "two-panel launches split K at multiples of 32");

template <int C>
__device__ __forceinline__ float pick(const float4& v) {
  if constexpr (C == 0) return v.x;
  else if constexpr (C == 1) return v.y;
  else if constexpr (C == 2) return v.z;
  else return v.w;
}

// Waits until at most 8 * `after` vector loads are outstanding.
__device__ __forceinline__ void wait_slots(int after) {
  if (after >= 3) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
  else if (after == 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
  else if (after == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <bool kAKC, bool kBKC, bool kTwo, bool kSplit, bool kEdge>
__global__ __launch_bounds__(kThreads, 1) void sgemm_ring8_kernel(Params p) {
  static_assert(!(kTwo && kSplit), "a two-panel launch never splits");
  static_assert(!(kEdge && (kTwo || kSplit)), "edge tiles run one-panel, unsplit launches");
  __shared__ __attribute__((aligned(16))) float lds[4 * kRing8 * 2 * kHalf8];
  asm volatile("; accumulators in AGPRs" ::: "a0");

  int tile_m, tile_n, split = 0;
  if constexpr (kSplit) {
    split = split_coords<kGroupM>(p, tile_m, tile_n);
    narrow_to_split(p, split, kAKC, kBKC);
  } else {
    tile_coords<kGroupM>(p, tile_m, tile_n);
  }
  const int m0 = tile_m * kTile;
  const int n0 = tile_n * kTile;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = (wave & 1) * kWave;
  const int wn = (wave >> 1) * kWave;
  const int lrow = lane & 31;
  const int lhalf = lane >> 5;

  float16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.f;

  const int slots = p.k / kSlotK;
  const int k1 = kTwo ? p.k_split : p.k;
  const int q_split = k1 / kSlotK;
  // A panel's descriptor from the tile's first element: an extent-contiguous
  // X(e, k) = x[e + k*ld] spans (kk*ld - e0) floats from x + e0 (to the end of
  // k-row kk-1), a k-contiguous X(e, k) = x[k + e*ld] spans 255*ld + kk
  // floats from x + e0*ld (the tile's 256 lines, kk values each).
  // Edge tiles: a k-contiguous panel ends after its last line (`lines` of
  // the tile's 256 lie inside the operand).
  const int a_lines = kEdge ? min(kTile, p.m - m0) : kTile;
  const int b_lines = kEdge ? min(kTile, p.n - n0) : kTile;
  const auto rsrc = [](const float* x, int64_t ld, int e0, int kk, bool kc, int lines) {
    return kc ? panel_rsrc(x + (int64_t)e0 * ld, (uint32_t)(((lines - 1) * ld + kk) * 4))
              : panel_rsrc(x + e0, (uint32_t)(((int64_t)kk * ld - e0) * 4));
  };
  // Rotated K order (op-T A): the tile row's slots are visited from slot
  // `turn` on, wrapping within each panel, so tile rows on one XCD read their
  // k-contiguous lines at different k. With a power-of-two lda every line of
  // every tile row otherwise sits at the same offset modulo the L2's channel
  // interleave at the same moment, which at 8192^3 T/N costs 3 % and at the
  // split 16384 x 256 x 16384 launch 9 % against a padded lda; the tile rows
  // sharing a tile column still read its lines within kTurnClasses *
  // kTurnSlots slots of one another. Each tile sums its slots in one fixed
  // order.
  const int turn = kAKC ? (tile_m % kTurnClasses) * kTurnSlots : 0;
  RingSource lo{rsrc(p.a, p.lda, m0, k1, kAKC, a_lines), rsrc(p.b, p.ldb, n0, k1, kBKC, b_lines), 0};
  lo.count = kTwo ? q_split : slots;
  lo.rotate = turn % lo.count;
  RingSource hi = lo;
  if constexpr (kTwo) {
    const int k2 = p.k - k1;
    hi = RingSource{rsrc(p.a2, p.lda, m0, k2, kAKC, a_lines), rsrc(p.b2, p.ldb, n0, k2, kBKC, b_lines),
                    q_split};
    hi.count = slots - q_split;
    hi.rotate = turn % hi.count;
  }
  // Lane offsets of load I of a half in its panel's first slot: k-row 2I + h,
  // elements w + 4*lrow .. +3 (extent-contiguous), or line w + 4*lrow + I, k
  // values 4h .. 4h+3 (k-contiguous). A slot advances K by 8 rows / values.
  // Edge tiles: elements and lines clamped to the operand (`lines` inside).
  const auto voff = [&](int64_t ld, int w, int i, bool kc, int lines) {
    int line = w + 4 * lrow + i;
    if constexpr (kEdge) line = min(line, lines - 1);
    return kc ? (uint32_t)(((int64_t)line * ld + 4 * lhalf) * 4)
              : (uint32_t)(((int64_t)(2 * i + lhalf) * ld + lane_elem<kEdge>(w, lrow, lines)) * 4);
  };
  uint32_t vo_a[4], vo_b[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    vo_a[i] = voff(p.lda, wm, i, kAKC, a_lines);
    vo_b[i] = voff(p.ldb, wn, i, kBKC, b_lines);
  }
  const uint32_t adv_a = kAKC ? kSlotK * 4 : (uint32_t)(kSlotK * 4 * p.lda);
  const uint32_t adv_b = kBKC ? kSlotK * 4 : (uint32_t)(kSlotK * 4 * p.ldb);
  float* ring = lds + wave * (kRing8 * 2 * kHalf8);
  const uint32_t ring_lds = lds_byte_addr(ring);

  // Load L (0..3: A, 4..7: B; load index L & 3) of slot q into ring slot S.
  auto issue = [&]<int S, int L>(int q, Int<S>, Int<L>, const RingSource& src) {
    constexpr int off = (S * 2 * kHalf8 + (L >> 2) * kHalf8 + (L & 3) * 256) * 4;
    uint32_t qq = (uint32_t)(q - src.base);
    if constexpr (kAKC) {
      qq += (uint32_t)src.rotate;
      if (qq >= (uint32_t)src.count) qq -= (uint32_t)src.count;
    }
    if constexpr (L < 4) {
      const uint32_t so = __builtin_amdgcn_readfirstlane(adv_a * qq);
      load_lds16<off>(ring_lds, vo_a[L & 3], src.a, so);
    } else {
      const uint32_t so = __builtin_amdgcn_readfirstlane(adv_b * qq);
      load_lds16<off>(ring_lds, vo_b[L & 3], src.b, so);
    }
  };
  // Fragments of ring slot S into register set R: x is the k-step of an
  // extent-contiguous half and the block of a k-contiguous one.
  float4 fa[2][4], fb[2][4];
  auto read_frag = [&]<int S, int R>(Int<S>, Int<R>) {
    const float* slot = ring + S * 2 * kHalf8;
#pragma unroll
    for (int x = 0; x < 4; ++x) {
      const int kc_off = 256 * x + 128 * lhalf + 4 * lrow;
      const int ex_off = (4 * lhalf + x) * kWave + 4 * lrow;
      fa[R][x] = *reinterpret_cast<const float4*>(slot + (kAKC ? kc_off : ex_off));
      fb[R][x] = *reinterpret_cast<const float4*>(slot + kHalf8 + (kBKC ? kc_off : ex_off));
    }
  };
  // MFMA X of a slot: k-step X / 16, row block (X / 4) % 4, column block X % 4.
  auto mfma_one = [&]<int R, int X>(Int<R>, Int<X>) {
    constexpr int s = X / 16, i = (X % 16) / 4, j = X % 4;
    float ao, bo;
    if constexpr (kAKC) ao = pick<s>(fa[R][i]);
    else ao = pick<i>(fa[R][s]);
    if constexpr (kBKC) bo = pick<s>(fb[R][j]);
    else bo = pick<j>(fb[R][s]);
    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(ao, bo, acc[i][j], 0, 0, 0);
  };

  // Slots 0 .. kRing8-1 in flight, then slot 0's fragments in registers.
  auto issue_slot = [&]<int S>(Int<S>) {
    [&]<int... L>(std::integer_sequence<int, L...>) {
      (issue(S, Int<S>{}, Int<L>{}, lo), ...);
    }(std::make_integer_sequence<int, 8>{});
  };
  [&]<int... S>(std::integer_sequence<int, S...>) {
    ((S < slots ? (issue_slot(Int<S>{}), 0) : 0), ...);
  }(std::make_integer_sequence<int, kRing8>{});
  wait_slots(min(slots, kRing8) - 1);
  read_frag(Int<0>{}, Int<0>{});

  // Step q (q % kRing8 == J). `load`: issue slot q + kRing8. `after`: slots
  // issued beyond q + 1 when slot q + 1 is waited for (-1: no slot q + 1).
  auto step = [&]<int J, bool kTail>(int q, Int<J>, std::bool_constant<kTail>,
                                      const RingSource& src) {
    constexpr int cur = J & 1, nxt = cur ^ 1;
    const bool load = !kTail || q + kRing8 < slots;
    const int after = !kTail ? kRing8 - 1
                      : q + 1 < slots ? min(q + kRing8, slots - 1) - (q + 1) : -1;
    // Slot q's fragment reads (issued half a step ago) are complete before
    // its ring slot is refilled.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
    [&]<int... X>(std::integer_sequence<int, X...>) {
      (([&] {
         if constexpr (X % 4 == 0 && X < 32) {
           if (load) {
             __builtin_amdgcn_sched_barrier(0);
             issue(q + kRing8, Int<J>{}, Int<X / 4>{}, src);
             __builtin_amdgcn_sched_barrier(0);
           }
         }
         if constexpr (X == 32) {
           if (after >= 0) {
             __builtin_amdgcn_sched_barrier(0);
             if constexpr (!kTail) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
             else wait_slots(after);
             read_frag(Int<(J + 1) % kRing8>{}, Int<nxt>{});
             __builtin_amdgcn_sched_barrier(0);
           }
         }
         mfma_one(Int<cur>{}, Int<X>{});
       }()),
       ...);
    }(std::make_integer_sequence<int, 64>{});
    __builtin_amdgcn_sched_barrier(0);
  };
  static_assert(kRing8 - 1 == 3, "steady-state wait above");

  const auto block = [&](int q0, const RingSource& src) {
    [&]<int... J>(std::integer_sequence<int, J...>) {
      (step(q0 + J, Int<J>{}, std::false_type{}, src), ...);
    }(std::make_integer_sequence<int, kRing8>{});
  };
  int q = 0;
  // Full blocks: the next block's slots all exist (q + 2 * kRing8 <= slots).
  if constexpr (kTwo) {
    for (; q + 2 * kRing8 <= slots && q + kRing8 < q_split; q += kRing8) block(q, lo);
    for (; q + 2 * kRing8 <= slots; q += kRing8) block(q, hi);
  } else {
    for (; q + 2 * kRing8 <= slots; q += kRing8) block(q, lo);
  }
  for (; q < slots; q += kRing8) {
    const RingSource& src = (kTwo && q + kRing8 >= q_split) ? hi : lo;
    [&]<int... J>(std::integer_sequence<int, J...>) {
      ((q + J < slots ? (step(q + J, Int<J>{}, std::true_type{}, src), 0) : 0), ...);
    }(std::make_integer_sequence<int, kRing8>{});
  }

  // The lane id is produced again here instead of being kept live across the
  // K loop: the epilogue needs every register, and addresses derived from a
  // value computed before the loop were hoisted above it and spilled.
  int lane_e;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(lane_e));
  const Params out = kSplit ? partial_target(p, split) : p;
  if constexpr (kEdge) store_c_tile<4, false>(out, acc, m0 + wm, n0 + wn, lane_e & 31, lane_e >> 5);
  else store_c_interior<4, 2, true>(out, acc, m0 + wm, n0 + wn, lane_e & 31, lane_e >> 5);
}

// ---- split-K reduction --------------------------------------------------------
//
// C = alpha * (P_0 + P_1 + ... + P_{S-1}) + beta * C, + bias, ReLU: the
// partials of a split launch added in range order (fixed, so C is the same
// from run to run), then the same epilogue arithmetic as store_c_tile. One
// thread per four consecutive rows of one column (ceil(m / 4) per column, the
// threads of a wave covering 256 consecutive floats of a column): the partials
// (ld = partial_ld(m)) are read as 16-byte vectors, C too where the four rows
// lie inside it, element by element in a column's last, partial quad (m not a
// multiple of 4).
__global__ __launch_bounds__(kThreads) void splitk_reduce_kernel(Params p) {
  const int64_t per_col = ((int64_t)p.m + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x;
  if (idx >= per_col * p.n) return;
  const int col = (int)(idx / per_col);
  const int row = (int)(idx - (int64_t)col * per_col) * 4;
  const int64_t ldp = partial_ld(p.m);
  const int64_t stride = ldp * p.n;
  const float* part = p.partial + (int64_t)col * ldp + row;
  float4 sum = *reinterpret_cast<const float4*>(part);
  for (int s = 1; s < p.splits; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(part + s * stride);
    sum.x += v.x;
    sum.y += v.y;
    sum.z += v.z;
    sum.w += v.w;
  }
  float* cp = p.c + (int64_t)col * p.ldc + row;
  const bool extra = p.bias_row != nullptr || p.bias_col != nullptr || p.relu != 0;
  const float bias_c = p.bias_col != nullptr ? p.bias_col[col] : 0.f;
  const auto finish = [&](float v, int r) {
    if (p.bias_row != nullptr) v += p.bias_row[r];
    v += bias_c;
    return (p.relu != 0 && v < 0.f) ? 0.f : v;
  };
  if (row + 4 <= p.m) {
    float r[4] = {p.alpha * sum.x, p.alpha * sum.y, p.alpha * sum.z, p.alpha * sum.w};
    if (p.beta != 0.f) {
      const float4 old = *reinterpret_cast<const float4*>(cp);
      r[0] = p.alpha * sum.x + p.beta * old.x;
      r[1] = p.alpha * sum.y + p.beta * old.y;
      r[2] = p.alpha * sum.z + p.beta * old.z;
      r[3] = p.alpha * sum.w + p.beta * old.w;
    }
    if (extra) {
#pragma unroll
      for (int t = 0; t < 4; ++t) r[t] = finish(r[t], row + t);
    }
    *reinterpret_cast<float4*>(cp) = make_float4(r[0], r[1], r[2], r[3]);
    return;
  }
  const float v[4] = {sum.x, sum.y, sum.z, sum.w};
  for (int t = 0; t < 4 && row + t < p.m; ++t) {
    const float val = p.alpha * v[t];
    const float out = p.beta != 0.f ? val + p.beta * cp[t] : val;
    cp[t] = extra ? finish(out, row + t) : out;
  }
}

// A launch of K below 8 (a K remainder's last rows): too little work for the
// MFMA tiles, whose prologue and C round trip it would pay in full. Each
// workgroup takes 4 * kThreads rows of C and kThinCols of its columns; each
// thread reads its four rows of the K columns of op(A) once into registers
// (an op-T A's rows are lines, read value by value) and then, column by
// column, forms the four sums with FP32 multiply-adds in K order (B(q, col)
// is the same for every lane) and applies the tile epilogue's arithmetic
// (alpha, beta, bias, ReLU), reading and writing C as 16-byte vectors, the
// old C of four columns loaded together (8192^2 x 7 at beta 1: 99 us, 5.4
// TB/s, against 115 us loading one column at a time). HBM-bound: about 8
// bytes of C per element.
constexpr int kThinCols = 16;
constexpr int kThinBatch = 4; // columns whose old C is loaded together

template <bool AK, bool BN>
__global__ __launch_bounds__(kThreads) void thin_k_kernel(Params p) {
  constexpr int kMaxK = 7;
  const int row_blocks = (p.m + 4 * kThreads - 1) / (4 * kThreads);
  const int block_row = (int)(blockIdx.x % (unsigned)row_blocks);
  const int col0 = (int)(blockIdx.x / (unsigned)row_blocks) * kThinCols;
  const int row = block_row * 4 * kThreads + 4 * (int)threadIdx.x;
  if (row >= p.m) return;
  const int rows = min(4, p.m - row);
  float x[kMaxK][4];
#pragma unroll
  for (int q = 0; q < kMaxK; ++q) {
    if (q < p.k) {
      if (!AK && rows == 4) {
        const float4 v = *reinterpret_cast<const float4*>(p.a + row + (int64_t)q * p.lda);
        x[q][0] = v.x;
        x[q][1] = v.y;
        x[q][2] = v.z;
        x[q][3] = v.w;
      } else {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          x[q][t] = t < rows ? (AK ? p.a[q + (int64_t)(row + t) * p.lda] : p.a[row + t + (int64_t)q * p.lda])
                             : 0.f;
      }
    }
  }
  const bool extra = p.bias_row != nullptr || p.bias_col != nullptr || p.relu != 0;
  float brow[4] = {0.f, 0.f, 0.f, 0.f};
  if (p.bias_row != nullptr)
    for (int t = 0; t < rows; ++t) brow[t] = p.bias_row[row + t];
  const int cols = min(kThinCols, p.n - col0);
  const bool read_c = p.beta != 0.f;
  // Columns in batches of kThinBatch: a batch's old C (beta != 0) is loaded
  // before any of it is used, so a thread has kThinBatch loads in flight.
  for (int j0 = 0; j0 < cols; j0 += kThinBatch) {
    float4 old[kThinBatch] = {};
    if (read_c && rows == 4) {
#pragma unroll
      for (int jb = 0; jb < kThinBatch; ++jb)
        if (j0 + jb < cols)
          old[jb] = *reinterpret_cast<const float4*>(p.c + (int64_t)(col0 + j0 + jb) * p.ldc + row);
    }
#pragma unroll
    for (int jb = 0; jb < kThinBatch; ++jb) {
      if (j0 + jb >= cols) break;
      const int col = col0 + j0 + jb;
      float sum[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int q = 0; q < kMaxK; ++q) {
        if (q < p.k) {
          const float y = BN ? p.b[col + (int64_t)q * p.ldb] : p.b[q + (int64_t)col * p.ldb];
#pragma unroll
          for (int t = 0; t < 4; ++t) sum[t] += x[q][t] * y;
        }
      }
      float* cp = p.c + (int64_t)col * p.ldc + row;
      const float bias_c = p.bias_col != nullptr ? p.bias_col[col] : 0.f;
      const auto finish = [&](float v, int t) {
        if (p.bias_row != nullptr) v += brow[t];
        v += bias_c;
        return (p.relu != 0 && v < 0.f) ? 0.f : v;
      };
      if (rows == 4) {
        float r[4] = {p.alpha * sum[0], p.alpha * sum[1], p.alpha * sum[2], p.alpha * sum[3]};
        if (read_c) {
          r[0] = p.alpha * sum[0] + p.beta * old[jb].x;
          r[1] = p.alpha * sum[1] + p.beta * old[jb].y;
          r[2] = p.alpha * sum[2] + p.beta * old[jb].z;
          r[3] = p.alpha * sum[3] + p.beta * old[jb].w;
        }
        if (extra) {
#pragma unroll
          for (int t = 0; t < 4; ++t) r[t] = finish(r[t], t);
        }
        *reinterpret_cast<float4*>(cp) = make_float4(r[0], r[1], r[2], r[3]);
      } else {
        for (int t = 0; t < rows; ++t) {
          const float val = p.alpha * sum[t];
          const float out = read_c ? val + p.beta * cp[t] : val;
          cp[t] = extra ? finish(out, t) : out;
        }
      }
    }
  }
}

} // namespace

int wide_tile() { return kTile; }

// The reduction of a split launch whose workgroups have been enqueued on
// `stream` (p.splits, p.split_depth and p.partial set); `stop` (optional) is
// recorded by its dispatch.
hipError_t launch_splitk_reduce(const Params& p, hipStream_t stream, hipEvent_t stop) {
  const int64_t quads = (((int64_t)p.m + 3) / 4) * p.n;
  const dim3 grid(static_cast<unsigned>((quads + kThreads - 1) / kThreads));
  hipExtLaunchKernelGGL(splitk_reduce_kernel, grid, dim3(kThreads), 0, stream, nullptr, stop, 0, p);
  return hipGetLastError();
}

// Launches thin_k_kernel for `p` (K below 8); start / stop (optional) are
// recorded by the dispatch.
hipError_t launch_thin_k(const Params& p, bool a_kcontig, bool b_ncontig, hipStream_t stream,
                         hipEvent_t start, hipEvent_t stop) {
  const int64_t row_blocks = ((int64_t)p.m + 4 * kThreads - 1) / (4 * kThreads);
  const int64_t col_groups = ((int64_t)p.n + kThinCols - 1) / kThinCols;
  const dim3 grid(static_cast<unsigned>(row_blocks * col_groups)), block(kThreads);
  if (!a_kcontig && !b_ncontig)
    hipExtLaunchKernelGGL((thin_k_kernel<false, false>), grid, block, 0, stream, start, stop, 0, p);
  else if (!a_kcontig && b_ncontig)
    hipExtLaunchKernelGGL((thin_k_kernel<false, true>), grid, block, 0, stream, start, stop, 0, p);
  else if (a_kcontig && !b_ncontig)
    hipExtLaunchKernelGGL((thin_k_kernel<true, false>), grid, block, 0, stream, start, stop, 0, p);
  else
    hipExtLaunchKernelGGL((thin_k_kernel<true, true>), grid, block, 0, stream, start, stop, 0, p);
  return hipGetLastError();
}

// Launches a 256 x 256 kernel for `p` (tiles_m / tiles_n already in 256s):
// sgemm_ring_kernel (N/T, K a multiple of 4) or sgemm_ring8_kernel (the other
// forms, K a multiple of 8) -- for launches of interior tiles their interior
// instances, or the two-panel ones when p.a2 is set (the caller has checked
// that launch's contract), else their edge instances; sgemm_wide_kernel for
// other K. start / stop (optional) are recorded by the dispatch itself.
hipError_t launch_wide(const Params& p, bool a_kcontig, bool b_ncontig, hipStream_t stream,
                       hipEvent_t start, hipEvent_t stop) {
  const dim3 block(kThreads);
  if (p.splits > 1) {
    // Split K (the caller has checked split_k_plan's conditions): the ring
    // kernel over tiles x ranges into the partials, then the reduction; the
    // start event rides on the first dispatch, the stop event on the second.
    const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n * p.splits));
    if (!a_kcontig && b_ncontig)
      hipExtLaunchKernelGGL((sgemm_ring_kernel<false, true, false>), grid, block, 0, stream, start, nullptr, 0, p);
    else if (!a_kcontig && !b_ncontig)
      hipExtLaunchKernelGGL((sgemm_ring8_kernel<false, true, false, true, false>), grid, block, 0, stream, start, nullptr, 0, p);
    else if (a_kcontig && !b_ncontig)
      hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, true, false, true, false>), grid, block, 0, stream, start, nullptr, 0, p);
    else
      hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, false, false, true, false>), grid, block, 0, stream, start, nullptr, 0, p);
    if (const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    return launch_splitk_reduce(p, stream, stop);
  }
  const dim3 grid(static_cast<unsigned>(p.tiles_m * p.tiles_n));
  const bool interior = p.m % kTile == 0 && p.n % kTile == 0;
  if (interior && !a_kcontig && b_ncontig && p.k % 4 == 0) {
    if (p.a2 != nullptr)
      hipExtLaunchKernelGGL((sgemm_ring_kernel<true, false, false>), grid, block, 0, stream, start, stop, 0, p);
    else
      hipExtLaunchKernelGGL((sgemm_ring_kernel<false, false, false>), grid, block, 0, stream, start, stop, 0, p);
  } else if (interior && p.k % kSlotK == 0) {
    const bool two = p.a2 != nullptr;
    if (!a_kcontig && !b_ncontig)
      two ? hipExtLaunchKernelGGL((sgemm_ring8_kernel<false, true, true, false, false>), grid, block, 0, stream, start, stop, 0, p)
          : hipExtLaunchKernelGGL((sgemm_ring8_kernel<false, true, false, false, false>), grid, block, 0, stream, start, stop, 0, p);
    else if (a_kcontig && !b_ncontig)
      two ? hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, true, true, false, false>), grid, block, 0, stream, start, stop, 0, p)
          : hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, true, false, false, false>), grid, block, 0, stream, start, stop, 0, p);
    else
      two ? hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, false, true, false, false>), grid, block, 0, stream, start, stop, 0, p)
          : hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, false, false, false, false>), grid, block, 0, stream, start, stop, 0, p);
  } else if (!a_kcontig && b_ncontig && p.k % 4 == 0) {
    // Edge tiles (one panel: two-panel launches are interior).
    hipExtLaunchKernelGGL((sgemm_ring_kernel<false, false, true>), grid, block, 0, stream, start, stop, 0, p);
  } else if (p.k % kSlotK == 0) {
    if (!a_kcontig && !b_ncontig)
      hipExtLaunchKernelGGL((sgemm_ring8_kernel<false, true, false, false, true>), grid, block, 0, stream, start, stop, 0, p);
    else if (a_kcontig && !b_ncontig)
      hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, true, false, false, true>), grid, block, 0, stream, start, stop, 0, p);
    else
      hipExtLaunchKernelGGL((sgemm_ring8_kernel<true, false, false, false, true>), grid, block, 0, stream, start, stop, 0, p);
  } else if (!a_kcontig && !b_ncontig)
    hipExtLaunchKernelGGL((sgemm_wide_kernel<false, false>), grid, block, 0, stream, start, stop, 0, p);
  else if (!a_kcontig && b_ncontig)
    hipExtLaunchKernelGGL((sgemm_wide_kernel<false, true>), grid, block, 0, stream, start, stop, 0, p);
  else if (a_kcontig && !b_ncontig)
    hipExtLaunchKernelGGL((sgemm_wide_kernel<true, false>), grid, block, 0, stream, start, stop, 0, p);
  else
    hipExtLaunchKernelGGL((sgemm_wide_kernel<true, true>), grid, block, 0, stream, start, stop, 0, p);
  return hipGetLastError();
}

} // namespace xvram::kernels
