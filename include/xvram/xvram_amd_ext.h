/*
 * xvram_amd extension table — additions of the MI355X build that have no
 * counterpart in the reference ABI. A caller of the reference interface never
 * needs this header. The library still exports exactly one symbol,
 * xvram_get_api@@XVRAM_0.1 (reference include/xvram/xvram.h:532-533,
 * cmake/xvram.exports.map); the extension table is requested through it with
 * the private version number XVRAM_AMD_EXT_ABI_VERSION_1, which lies outside
 * the reference's sequential ABI versions (1, 2, ...):
 *
 *     xvram_amd_ext_v1 ext;
 *     xvram_get_api(XVRAM_AMD_EXT_ABI_VERSION_1, sizeof(ext), &ext);
 *
 * Argument rules are those of the v1/v2 tables: NULL or a buffer smaller than
 * xvram_amd_ext_v1 -> XVRAM_STATUS_INVALID_ARGUMENT; every other unknown
 * version still returns XVRAM_STATUS_INCOMPATIBLE_ABI. The functions work on
 * the same session/allocation/plan handles as include/xvram/xvram.h.
 *
 * Version 1: GEMM plans with a fused epilogue,
 *
 *     C = act(alpha * op(A) * op(B) + beta * C + bias)
 *
 * where bias is an FP32 vector in a session allocation running along the rows
 * (length m) or the columns (length n) of C as the caller describes C, and act
 * is the identity or ReLU (negative values become 0; NaN stays NaN). The
 * epilogue is applied once per element, after the whole K reduction. A linear
 * layer Y = ReLU(X W^T + b) with row-major X (batch x in), W (out x in) and
 * Y (batch x out) is op(A) = X, op(B) = W^T (operation_b = T), C = Y, with a
 * per-column bias.
 *
 * Version 2 adds the tile GEMM on device memory the caller owns:
 *
 *     sgemm_device(&desc, hip_stream)
 *
 * enqueues C = act(alpha * op(A) * op(B) + beta * C + bias) on the stream with
 * the kernels gemm_execute runs on each tile (full-precision FP32 MFMA), for
 * operands already in HBM, e.g. the resolved ranges a transaction callback
 * receives (enqueue on its native_stream). It returns once the work is
 * enqueued. A launch that would leave the GPU's workgroup slots idle splits
 * its K (partial sums in a workspace, added in a fixed order: the same result
 * on every call); the workspace is desc.workspace when it holds every partial,
 * else one the library allocates stream-ordered on the stream
 * (hipMallocAsync, freed behind the kernels).
 *
 * Conventions are those of xvram.h: struct_size first, reserved members and
 * unknown flags must be zero.
 */
#ifndef XVRAM_XVRAM_AMD_EXT_H
#define XVRAM_XVRAM_AMD_EXT_H

#include <xvram/xvram.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The version passed to xvram_get_api for the extension table ('X','A' in the
   top bytes keeps it clear of the reference's small ABI numbers). */
#define XVRAM_AMD_EXT_ABI_VERSION_1 UINT32_C(0x58410001)
/* Values of xvram_amd_ext_v1.ext_version: 2 = the table has sgemm_device. */
#define XVRAM_AMD_EXT_VERSION_1 UINT32_C(1)
#define XVRAM_AMD_EXT_VERSION_2 UINT32_C(2)

typedef uint32_t xvram_amd_bias_axis;
enum {
  XVRAM_AMD_BIAS_NONE = 0,
  XVRAM_AMD_BIAS_PER_ROW = 1,    /* bias[i] added to row i of C (length m) */
  XVRAM_AMD_BIAS_PER_COLUMN = 2  /* bias[j] added to column j of C (length n) */
};

typedef uint32_t xvram_amd_activation;
enum { XVRAM_AMD_ACTIVATION_NONE = 0, XVRAM_AMD_ACTIVATION_RELU = 1 };

typedef struct xvram_amd_epilogue_v1 {
  uint32_t struct_size;
  uint32_t flags;
  xvram_allocation bias;          /* NULL when bias_axis is NONE */
  uint64_t bias_offset_bytes;     /* 4-byte aligned; the vector is FP32 */
  xvram_amd_bias_axis bias_axis;
  xvram_amd_activation activation;
  uint64_t reserved[2];
} xvram_amd_epilogue_v1;

/* What a device reports about itself (no session needed). */
typedef struct xvram_amd_device_info_v1 {
  uint32_t struct_size;
  int32_t ordinal;
  char name[256];
  char arch[64];       /* e.g. "gfx950:sramecc+:xnack-" */
  char pci_bus_id[32]; /* "dddd:bb:dd.f", empty when unknown */
  uint64_t total_memory_bytes;
  uint64_t free_memory_bytes;
  uint64_t granularity_minimum_bytes;
  uint64_t granularity_recommended_bytes;
  uint32_t compute_major;
  uint32_t compute_minor;
  uint32_t multiprocessor_count;
  uint32_t vmm_supported;
  int32_t driver_version;
  int32_t runtime_version;
  uint64_t reserved[4];
} xvram_amd_device_info_v1;

/* One GEMM on device memory, column-major (see sgemm_device above). Every
   pointer is device memory of the stream's GPU, 16-byte aligned; leading
   dimensions are in floats, multiples of 4, at least the stored rows; each
   operand buffer holds ld x (stored columns) floats. The padding rows (stored
   rows .. ld - 1) may be read but hold any values, NaN included: none reaches
   C. m, n, k in 1..2^31-1. */
typedef struct xvram_amd_sgemm_v1 {
  uint32_t struct_size;
  uint32_t flags;
  const float* a;       /* op N: A(i,p) = a[i + p*lda] (m x k); op T: a[p + i*lda] */
  const float* b;       /* op N: B(p,j) = b[p + j*ldb] (k x n); op T: b[j + p*ldb] */
  float* c;             /* C(i,j) = c[i + j*ldc] (m x n) */
  const float* bias;    /* m (PER_ROW) or n (PER_COLUMN) floats; NULL with BIAS_NONE */
  void* workspace;      /* optional split-K workspace; NULL = the library's */
  uint64_t workspace_bytes;
  uint64_t m, n, k;
  uint64_t lda, ldb, ldc;
  double alpha;         /* converted to float */
  double beta;          /* converted to float; 0 = C is not read */
  xvram_matrix_operation operation_a;
  xvram_matrix_operation operation_b;
  xvram_amd_bias_axis bias_axis;
  xvram_amd_activation activation;
  uint64_t reserved[4];
} xvram_amd_sgemm_v1;

typedef struct xvram_amd_ext_v1 {
  uint32_t struct_size;
  uint32_t ext_version;
  /* gemm_plan_create with an epilogue; the plan is used and released with the
     xvram_api_v1 functions (gemm_plan_get_info, gemm_submit, gemm_execute,
     gemm_plan_release). The bias must not overlap C. */
  xvram_status(XVRAM_CALL* gemm_plan_create_epilogue)(xvram_session session,
                                                      const xvram_gemm_desc_v1* desc,
                                                      const xvram_amd_epilogue_v1* epilogue,
                                                      xvram_gemm_plan* out_plan);
  /* Fills `out` (struct_size >= v1, preserved) for device `ordinal`. */
  xvram_status(XVRAM_CALL* device_get_info)(int32_t ordinal, xvram_amd_device_info_v1* out);
  /* ext_version >= 2: one GEMM on device memory, enqueued on `hip_stream` (a
     hipStream_t; NULL = the default stream of the calling thread's device).
     No counterpart in the reference (its tile GEMM is internal). Returns
     INVALID_ARGUMENT for a malformed descriptor, DEVICE_OUT_OF_MEMORY when a
     needed workspace cannot be allocated, CUDA_ERROR (a hipError_t) when the
     enqueue fails, UNSUPPORTED in a build without a GPU. */
  xvram_status(XVRAM_CALL* sgemm_device)(const xvram_amd_sgemm_v1* desc, void* hip_stream);
  /* ext_version >= 2: sgemm_device that allocates nothing, for callers that
     cannot allocate (code under stream capture, tight serving loops). No
     counterpart in the reference. A split that desc->workspace cannot hold
     uses the library's static per-GPU scratch of 128 MiB (the most any split
     wants: one 256 x 256 partial tile per CU, two for a tail split, or one
     256 x 128 tile per workgroup of two rounds of the 256 x 128 kernel's
     slots), held until the process ends and shared by every call on that
     GPU: calls that overlap on one GPU race. A split wanting more returns
     INVALID_ARGUMENT. Same results as sgemm_device. */
  xvram_status(XVRAM_CALL* sgemm_device_no_alloc)(const xvram_amd_sgemm_v1* desc,
                                                  void* hip_stream);
  uint64_t reserved[1];
} xvram_amd_ext_v1;

#ifdef __cplusplus
}
#endif

#endif /* XVRAM_XVRAM_AMD_EXT_H */
