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
/* Value of xvram_amd_ext_v1.ext_version. */
#define XVRAM_AMD_EXT_VERSION_1 UINT32_C(1)

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
  uint64_t reserved[3];
} xvram_amd_ext_v1;

#ifdef __cplusplus
}
#endif

#endif /* XVRAM_XVRAM_AMD_EXT_H */
