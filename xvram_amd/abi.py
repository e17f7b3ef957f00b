"""ctypes mirror of ``include/xvram/xvram.h`` (the xVRAM v1 C ABI).

Every structure reproduces the C layout field for field; ``tests/test_abi_layout``
checks ``ctypes.sizeof``/offsets against the sizes a C compiler computes for
the header (and the reference's published table).
"""
from __future__ import annotations

import ctypes
from ctypes import (CFUNCTYPE, POINTER, Structure, c_char, c_char_p, c_double, c_int32,
                    c_int64, c_uint32, c_uint64, c_void_p)

ABI_VERSION_1 = 1
TIMEOUT_INFINITE = (1 << 64) - 1

STATUS = {
    0: "success", 1: "invalid_argument", 2: "incompatible_abi", 3: "unsupported",
    4: "unavailable", 5: "host_out_of_memory", 6: "device_out_of_memory",
    7: "budget_pressure", 8: "busy", 9: "not_ready", 10: "timeout", 11: "corruption",
    12: "callback_failed", 13: "cuda_error", 14: "cublas_error", 15: "poisoned",
    16: "cleanup_failed", 17: "closed", 18: "cancelled", 19: "internal",
}
SUCCESS, INVALID_ARGUMENT, INCOMPATIBLE_ABI, UNSUPPORTED, UNAVAILABLE = 0, 1, 2, 3, 4
HOST_OUT_OF_MEMORY, DEVICE_OUT_OF_MEMORY, BUDGET_PRESSURE, BUSY, NOT_READY = 5, 6, 7, 8, 9
TIMEOUT, CORRUPTION, CALLBACK_FAILED, CUDA_ERROR, CUBLAS_ERROR = 10, 11, 12, 13, 14
POISONED, CLEANUP_FAILED, CLOSED, CANCELLED, INTERNAL = 15, 16, 17, 18, 19

NATIVE_ERROR_NONE, NATIVE_ERROR_CUDA, NATIVE_ERROR_CUBLAS = 0, 1, 2
NATIVE_ERROR_PLATFORM, NATIVE_ERROR_CALLBACK, NATIVE_ERROR_INTERNAL = 3, 4, 5

CONTEXT_ISOLATED, CONTEXT_ATTACH_CURRENT = 0, 1
CACHE_POLICY_CLOCK, CACHE_POLICY_LRU = 0, 1
ALLOCATION_NORMAL, ALLOCATION_HOT, ALLOCATION_STREAMING = 0, 1, 2
ALLOCATION_FLAG_ZERO_INITIALIZE = 1
ACCESS_READ, ACCESS_READ_WRITE, ACCESS_WRITE_ONLY = 0, 1, 2
OPERATION_QUEUED, OPERATION_RUNNING, OPERATION_COMPLETED = 0, 1, 2
OPERATION_CANCELLED, OPERATION_FAILED = 3, 4
DATA_FP16, DATA_BF16, DATA_FP32, DATA_FP64 = 0, 1, 2, 3
COMPUTE_AUTO, COMPUTE_FP32_STRICT, COMPUTE_FP32_TF32, COMPUTE_FP64 = 0, 1, 2, 3
ROW_MAJOR, COLUMN_MAJOR = 0, 1
OP_N, OP_T = 0, 1


class ErrorInfo(Structure):
    _fields_ = [("struct_size", c_uint32), ("status", c_uint32), ("native_domain", c_uint32),
                ("reserved0", c_uint32), ("native_code", c_int64), ("stage", c_char * 32),
                ("operation", c_char * 64), ("native_name", c_char * 64),
                ("message", c_char * 256)]


class SessionConfig(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("device_ordinal", c_int32),
                ("context_mode", c_uint32), ("chunk_size_bytes", c_uint64),
                ("cache_target_bytes", c_uint64), ("device_headroom_bytes", c_uint64),
                ("workspace_cap_bytes", c_uint64), ("budget_poll_ms", c_uint64),
                ("max_transaction_ms", c_uint64), ("staging_slots", c_uint32),
                ("cache_policy", c_uint32), ("prefetch_distance", c_uint32),
                ("reserved0", c_uint32), ("reserved", c_uint64 * 4)]


class AllocationDesc(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("size_bytes", c_uint64),
                ("alignment_bytes", c_uint64), ("priority", c_uint32), ("reserved0", c_uint32),
                ("reserved", c_uint64 * 2)]


class AllocationInfo(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("allocation_id", c_uint64),
                ("size_bytes", c_uint64), ("alignment_bytes", c_uint64), ("priority", c_uint32),
                ("stable_virtual_address", c_uint32), ("reserved", c_uint64 * 2)]


class AccessRange(Structure):
    _fields_ = [("allocation", c_void_p), ("offset_bytes", c_uint64), ("length_bytes", c_uint64),
                ("mode", c_uint32), ("reserved0", c_uint32)]


class PrefetchDesc(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("ranges", POINTER(AccessRange)),
                ("range_count", c_uint64), ("deadline_ms", c_uint64), ("reserved", c_uint64 * 2)]


class ResolvedRange(Structure):
    _fields_ = [("allocation_id", c_uint64), ("offset_bytes", c_uint64),
                ("length_bytes", c_uint64), ("device_address", c_uint64), ("mode", c_uint32),
                ("reserved0", c_uint32)]


class TransactionContext(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("operation_id", c_uint64),
                ("transaction_id", c_uint64), ("ranges", POINTER(ResolvedRange)),
                ("range_count", c_uint64), ("workspace_device_address", c_uint64),
                ("workspace_bytes", c_uint64), ("native_stream", c_uint64),
                ("reserved", c_uint64 * 2)]


TransactionCallback = CFUNCTYPE(c_uint32, POINTER(TransactionContext), c_void_p, POINTER(ErrorInfo))


class TransactionDesc(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("ranges", POINTER(AccessRange)),
                ("range_count", c_uint64), ("workspace_bytes", c_uint64), ("deadline_ms", c_uint64),
                ("callback", TransactionCallback), ("user_data", c_void_p),
                ("reserved", c_uint64 * 2)]


class OperationInfo(Structure):
    _fields_ = [("struct_size", c_uint32), ("state", c_uint32), ("result", c_uint32),
                ("reserved0", c_uint32), ("operation_id", c_uint64), ("units_completed", c_uint64),
                ("units_total", c_uint64), ("elapsed_ms", c_double), ("bytes_h2d", c_uint64),
                ("bytes_d2h", c_uint64), ("cache_hits", c_uint64), ("cache_misses", c_uint64),
                ("reserved", c_uint64 * 2)]


class Matrix(Structure):
    _fields_ = [("struct_size", c_uint32), ("data_type", c_uint32), ("allocation", c_void_p),
                ("offset_bytes", c_uint64), ("rows", c_uint64), ("columns", c_uint64),
                ("leading_dimension", c_uint64), ("layout", c_uint32), ("reserved0", c_uint32),
                ("reserved", c_uint64 * 2)]


class GemmDesc(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("a", Matrix), ("b", Matrix),
                ("c", Matrix), ("operation_a", c_uint32), ("operation_b", c_uint32),
                ("compute_mode", c_uint32), ("reserved0", c_uint32), ("alpha", c_double),
                ("beta", c_double), ("workspace_cap_bytes", c_uint64), ("deadline_ms", c_uint64),
                ("tile_m_hint", c_uint64), ("tile_n_hint", c_uint64), ("tile_k_hint", c_uint64),
                ("reserved", c_uint64 * 3)]


class GemmPlanInfo(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("m", c_uint64), ("n", c_uint64),
                ("k", c_uint64), ("tile_m", c_uint64), ("tile_n", c_uint64), ("tile_k", c_uint64),
                ("maximum_working_set_bytes", c_uint64), ("workspace_bytes", c_uint64),
                ("tile_count", c_uint64), ("effective_compute_mode", c_uint32),
                ("uses_cublas_lt", c_uint32), ("reserved", c_uint64 * 2)]


_TELEMETRY_U64 = [
    "cache_target_bytes", "cache_target_minimum_bytes", "cache_target_maximum_bytes",
    "resident_bytes", "resident_bytes_peak", "workspace_bytes", "bytes_h2d", "bytes_d2h",
    "cache_hits", "cache_misses", "clean_evictions", "dirty_evictions", "writebacks_completed",
    "mappings", "unmaps", "set_access_calls", "handle_reuses", "unsafe_remaps",
    "unsafe_transitions", "budget_shrinks", "budget_grows"]


class SessionTelemetry(Structure):
    _fields_ = ([("struct_size", c_uint32), ("flags", c_uint32)]
                + [(n, c_uint64) for n in _TELEMETRY_U64]
                + [("cuda_driver_version", c_uint32), ("cublas_version", c_uint32),
                   ("cublas_lt_available", c_uint32), ("poisoned", c_uint32),
                   ("physical_handles_created", c_uint64), ("physical_handles_released", c_uint64),
                   ("event_boundaries", c_uint64), ("pinned_staging_bytes", c_uint64),
                   ("transactions_completed", c_uint64), ("algorithm_selections", c_uint64),
                   ("algorithm_cache_hits", c_uint64), ("last_transaction_ms", c_double),
                   ("budget_sample_count", c_uint64), ("cuda_free_bytes_minimum", c_uint64),
                   ("cuda_free_bytes_end", c_uint64), ("cublas_lt_version", c_uint32),
                   ("cublas_library_source", c_uint32), ("wddm_available_bytes_minimum", c_uint64),
                   ("wddm_available_bytes_end", c_uint64), ("wddm_budget_observed", c_uint32),
                   ("watchdog_rejections", c_uint32), ("target_oom_retries", c_uint64)])


_H = c_void_p  # opaque handles
_F = CFUNCTYPE


class ApiV1(Structure):
    _fields_ = [
        ("struct_size", c_uint32), ("abi_version", c_uint32),
        ("status_name", _F(c_char_p, c_uint32)),
        ("session_create", _F(c_uint32, POINTER(SessionConfig), POINTER(_H))),
        ("session_get_error", _F(c_uint32, _H, POINTER(ErrorInfo))),
        ("session_get_telemetry", _F(c_uint32, _H, POINTER(SessionTelemetry))),
        ("session_drain", _F(c_uint32, _H, c_uint64)),
        ("session_close", _F(c_uint32, _H, c_uint64)),
        ("session_release", _F(None, _H)),
        ("allocation_create", _F(c_uint32, _H, POINTER(AllocationDesc), POINTER(_H))),
        ("allocation_get_info", _F(c_uint32, _H, POINTER(AllocationInfo))),
        ("allocation_write", _F(c_uint32, _H, c_uint64, c_void_p, c_uint64)),
        ("allocation_read", _F(c_uint32, _H, c_uint64, c_void_p, c_uint64)),
        ("allocation_release", _F(c_uint32, _H)),
        ("prefetch_submit", _F(c_uint32, _H, POINTER(PrefetchDesc), POINTER(_H))),
        ("transaction_submit", _F(c_uint32, _H, POINTER(TransactionDesc), POINTER(_H))),
        ("transaction_execute", _F(c_uint32, _H, POINTER(TransactionDesc), c_uint64)),
        ("gemm_plan_create", _F(c_uint32, _H, POINTER(GemmDesc), POINTER(_H))),
        ("gemm_plan_get_info", _F(c_uint32, _H, POINTER(GemmPlanInfo))),
        ("gemm_submit", _F(c_uint32, _H, POINTER(_H))),
        ("gemm_execute", _F(c_uint32, _H, c_uint64)),
        ("gemm_plan_release", _F(None, _H)),
        ("operation_poll", _F(c_uint32, _H, POINTER(OperationInfo))),
        ("operation_wait", _F(c_uint32, _H, c_uint64, POINTER(OperationInfo))),
        ("operation_cancel", _F(c_uint32, _H)),
        ("operation_get_error", _F(c_uint32, _H, POINTER(ErrorInfo))),
        ("operation_release", _F(None, _H)),
        ("reserved", c_uint64 * 16),
    ]


def session_config_init() -> SessionConfig:
    """XVRAM_SESSION_CONFIG_V1_INIT."""
    c = SessionConfig()
    c.struct_size = ctypes.sizeof(SessionConfig)
    c.chunk_size_bytes = 64 << 20
    c.device_headroom_bytes = 512 << 20
    c.workspace_cap_bytes = 4 << 20
    c.budget_poll_ms = 100
    c.staging_slots = 4
    c.cache_policy = CACHE_POLICY_CLOCK
    c.prefetch_distance = 2
    return c


def allocation_desc_init(size: int = 0) -> AllocationDesc:
    d = AllocationDesc()
    d.struct_size = ctypes.sizeof(AllocationDesc)
    d.size_bytes = size
    return d


def matrix_init() -> Matrix:
    m = Matrix()
    m.struct_size = ctypes.sizeof(Matrix)
    m.data_type = DATA_FP32
    m.layout = ROW_MAJOR
    return m


def gemm_desc_init() -> GemmDesc:
    d = GemmDesc()
    d.struct_size = ctypes.sizeof(GemmDesc)
    for name in ("a", "b", "c"):
        setattr(d, name, matrix_init())
    d.alpha = 1.0
    d.beta = 0.0
    return d


def operation_info_init() -> OperationInfo:
    o = OperationInfo()
    o.struct_size = ctypes.sizeof(OperationInfo)
    return o


def error_info_init() -> ErrorInfo:
    e = ErrorInfo()
    e.struct_size = ctypes.sizeof(ErrorInfo)
    return e


def telemetry_init() -> SessionTelemetry:
    t = SessionTelemetry()
    t.struct_size = ctypes.sizeof(SessionTelemetry)
    return t


def plan_info_init() -> GemmPlanInfo:
    p = GemmPlanInfo()
    p.struct_size = ctypes.sizeof(GemmPlanInfo)
    return p


# ---- xvram_amd extension table (include/xvram/xvram_amd_ext.h) -----------------------

# xvram_get_api version number of the extension table (XVRAM_AMD_EXT_ABI_VERSION_1)
# and the table's own ext_version (XVRAM_AMD_EXT_VERSION_1).
EXT_ABI_VERSION_1 = 0x58410001
EXT_VERSION_1 = 1
EXT_VERSION_2 = 2  # the table has sgemm_device
BIAS_NONE, BIAS_PER_ROW, BIAS_PER_COLUMN = 0, 1, 2
ACTIVATION_NONE, ACTIVATION_RELU = 0, 1


class EpilogueV1(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("bias", c_void_p),
                ("bias_offset_bytes", c_uint64), ("bias_axis", c_uint32),
                ("activation", c_uint32), ("reserved", c_uint64 * 2)]


class DeviceInfoV1(Structure):
    _fields_ = [("struct_size", c_uint32), ("ordinal", c_int32), ("name", c_char * 256),
                ("arch", c_char * 64), ("pci_bus_id", c_char * 32),
                ("total_memory_bytes", c_uint64), ("free_memory_bytes", c_uint64),
                ("granularity_minimum_bytes", c_uint64),
                ("granularity_recommended_bytes", c_uint64), ("compute_major", c_uint32),
                ("compute_minor", c_uint32), ("multiprocessor_count", c_uint32),
                ("vmm_supported", c_uint32), ("driver_version", c_int32),
                ("runtime_version", c_int32), ("reserved", c_uint64 * 4)]


class SgemmDeviceV1(Structure):
    """xvram_amd_sgemm_v1: one GEMM on device memory (pointers as integers)."""
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("a", c_void_p),
                ("b", c_void_p), ("c", c_void_p), ("bias", c_void_p), ("workspace", c_void_p),
                ("workspace_bytes", c_uint64), ("m", c_uint64), ("n", c_uint64), ("k", c_uint64),
                ("lda", c_uint64), ("ldb", c_uint64), ("ldc", c_uint64), ("alpha", c_double),
                ("beta", c_double), ("operation_a", c_uint32), ("operation_b", c_uint32),
                ("bias_axis", c_uint32), ("activation", c_uint32), ("reserved", c_uint64 * 4)]


class ExtV1(Structure):
    _fields_ = [("struct_size", c_uint32), ("ext_version", c_uint32),
                ("gemm_plan_create_epilogue",
                 _F(c_uint32, _H, POINTER(GemmDesc), POINTER(EpilogueV1), POINTER(_H))),
                ("device_get_info", _F(c_uint32, c_int32, POINTER(DeviceInfoV1))),
                ("sgemm_device", _F(c_uint32, POINTER(SgemmDeviceV1), c_void_p)),
                ("sgemm_device_no_alloc", _F(c_uint32, POINTER(SgemmDeviceV1), c_void_p)),
                ("reserved", c_uint64 * 1)]


def sgemm_device_init() -> SgemmDeviceV1:
    d = SgemmDeviceV1()
    d.struct_size = ctypes.sizeof(SgemmDeviceV1)
    d.alpha = 1.0
    return d


def epilogue_init() -> EpilogueV1:
    e = EpilogueV1()
    e.struct_size = ctypes.sizeof(EpilogueV1)
    return e


# ---- ABI v2 (include/xvram/xvram_v2.h) ------------------------------------------------

ABI_VERSION_2 = 2
COMPRESSION_DISABLED, COMPRESSION_ADAPTIVE, COMPRESSION_CAPACITY = 0, 1, 2
COMPRESSION_CODEC_AUTO, COMPRESSION_CODEC_LZ4 = 0, 1


class SessionConfigV2(Structure):
    _fields_ = [("struct_size", c_uint32), ("flags", c_uint32), ("v1", SessionConfig),
                ("compression_mode", c_uint32), ("compression_codec", c_uint32),
                ("host_store_cap_bytes", c_uint64), ("host_headroom_bytes", c_uint64),
                ("compression_workspace_cap_bytes", c_uint64), ("codec_slots", c_uint32),
                ("codec_workers", c_uint32), ("reserved", c_uint64 * 8)]


_TELEMETRY_V2_U64 = [
    "logical_bytes", "host_stored_bytes", "host_stored_peak_bytes", "host_raw_bytes",
    "host_compressed_bytes", "host_implicit_zero_bytes", "host_invalid_bytes",
    "logical_h2d_bytes", "pcie_h2d_bytes", "logical_d2h_bytes", "pcie_d2h_bytes",
    "raw_path_decisions", "cpu_lz4_gpu_decode_decisions", "gpu_lz4_decisions",
    "never_compress_decisions", "raw_fallbacks", "cpu_codec_fallbacks", "gpu_codec_fallbacks",
    "compression_attempts", "compression_commits", "decompression_attempts",
    "decompression_commits", "generations_created", "generations_committed",
    "generations_discarded", "codec_workspace_bytes", "codec_workspace_peak_bytes",
    "codec_slot_bytes", "codec_slot_peak_bytes", "spill_reserved_bytes",
    "spill_reserved_peak_bytes", "cpu_encode_nanoseconds", "cpu_decode_nanoseconds",
    "gpu_encode_nanoseconds", "gpu_decode_nanoseconds", "verification_nanoseconds"]


class SessionTelemetryV2(Structure):
    _fields_ = ([("struct_size", c_uint32), ("flags", c_uint32), ("v1", SessionTelemetry)]
                + [(n, c_uint64) for n in _TELEMETRY_V2_U64] + [("reserved", c_uint64 * 8)])


class ApiV2(Structure):
    _fields_ = [("v1", ApiV1),
                ("session_create_v2", _F(c_uint32, POINTER(SessionConfigV2), POINTER(_H))),
                ("session_get_telemetry_v2", _F(c_uint32, _H, POINTER(SessionTelemetryV2))),
                ("reserved", c_uint64 * 14)]


def session_config_v2_init() -> SessionConfigV2:
    """XVRAM_SESSION_CONFIG_V2_INIT (note: it requests ADAPTIVE compression)."""
    c = SessionConfigV2()
    c.struct_size = ctypes.sizeof(SessionConfigV2)
    c.v1 = session_config_init()
    c.compression_mode = COMPRESSION_ADAPTIVE
    c.compression_codec = COMPRESSION_CODEC_AUTO
    c.compression_workspace_cap_bytes = 268435456
    c.codec_slots = 2
    c.codec_workers = 2
    return c
