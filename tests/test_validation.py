"""Boundary validation: session/allocation/GEMM descriptors are rejected with
the reference's statuses, and GEMM-problem validity matches the reference's own
validate_problem (src/gemm/planner.cpp:785-859) on randomly generated
descriptors: against its answers recorded in tests/golden/reference_outputs.json
and, where the reference tree is mounted, against the compiled function itself
(oracle/_ref). Runs over the host-simulation library."""
import ctypes

import numpy as np
import pytest

import generators
import oracle
import xvram_amd as xv
from xvram_amd import abi

KiB = 1 << 10

PROBLEM_ERRORS = ["none", "zero_dimension", "invalid_allocation", "invalid_layout",
                  "invalid_operation", "invalid_element_type", "invalid_compute_mode",
                  "dimension_mismatch", "leading_dimension_too_small", "storage_overflow",
                  "storage_out_of_bounds", "unsupported_type_combination", "output_aliases_input",
                  "integer_limit_exceeded"]


@pytest.fixture()
def session():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    s = xv.Session(lib, chunk_size_bytes=256 * KiB, cache_target_bytes=16 * 256 * KiB,
                   workspace_cap_bytes=0, device_headroom_bytes=0)
    yield s
    s.close()
    s.release()


def create_session(lib, **fields):
    cfg = abi.session_config_init()
    for k, v in fields.items():
        if k == "reserved":
            cfg.reserved[0] = v
        else:
            setattr(cfg, k, v)
    h = ctypes.c_void_p()
    status = lib.api.session_create(ctypes.byref(cfg), ctypes.byref(h))
    if status == abi.SUCCESS:
        lib.api.session_close(h, abi.TIMEOUT_INFINITE)
        lib.api.session_release(h)
    return status


@pytest.mark.parametrize("fields,status", [
    ({}, abi.SUCCESS),
    ({"struct_size": 100}, abi.INCOMPATIBLE_ABI),
    ({"flags": 1}, abi.INVALID_ARGUMENT),
    ({"reserved0": 1}, abi.INVALID_ARGUMENT),
    ({"reserved": 1}, abi.INVALID_ARGUMENT),
    ({"context_mode": 2}, abi.INVALID_ARGUMENT),
    ({"cache_policy": 2}, abi.INVALID_ARGUMENT),
    ({"device_ordinal": -1}, abi.INVALID_ARGUMENT),
    ({"chunk_size_bytes": 0}, abi.INVALID_ARGUMENT),
    ({"staging_slots": 1}, abi.INVALID_ARGUMENT),
    ({"staging_slots": 9}, abi.INVALID_ARGUMENT),
    ({"prefetch_distance": 9}, abi.INVALID_ARGUMENT),
    ({"budget_poll_ms": 0}, abi.INVALID_ARGUMENT),
    ({"max_transaction_ms": 1 << 63}, abi.INVALID_ARGUMENT),
    ({"device_ordinal": 3}, abi.CUDA_ERROR),
    ({"cache_target_bytes": 64 << 20}, abi.BUDGET_PRESSURE),  # fewer than two frames after reserve
])
def test_session_config_rules(fields, status):
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    cfg = dict(chunk_size_bytes=64 << 20, cache_target_bytes=1 << 30)
    cfg.update(fields)
    assert create_session(lib, **cfg) == status


def test_null_pointers(session):
    api = session.api
    assert api.session_create(None, None) == abi.INVALID_ARGUMENT
    h = ctypes.c_void_p()
    assert api.session_create(None, ctypes.byref(h)) == abi.INCOMPATIBLE_ABI
    assert api.allocation_create(None, None, ctypes.byref(h)) == abi.INVALID_ARGUMENT
    assert api.gemm_plan_create(session.handle, None, ctypes.byref(h)) == abi.INCOMPATIBLE_ABI
    assert api.operation_poll(None, None) == abi.INVALID_ARGUMENT
    t = abi.telemetry_init()
    t.struct_size = 8
    assert api.session_get_telemetry(session.handle, ctypes.byref(t)) == abi.INVALID_ARGUMENT


@pytest.mark.parametrize("fields,status", [
    ({"size_bytes": 4096}, abi.SUCCESS),
    ({"size_bytes": 0}, abi.INVALID_ARGUMENT),
    ({"size_bytes": 4096, "flags": 2}, abi.INVALID_ARGUMENT),
    ({"size_bytes": 4096, "flags": 1}, abi.SUCCESS),
    ({"size_bytes": 4096, "priority": 3}, abi.INVALID_ARGUMENT),
    ({"size_bytes": 4096, "alignment_bytes": 3}, abi.INVALID_ARGUMENT),
    ({"size_bytes": 4096, "alignment_bytes": 512 * KiB}, abi.INVALID_ARGUMENT),
    ({"size_bytes": 4096, "alignment_bytes": 4096}, abi.SUCCESS),
    ({"size_bytes": 4096, "struct_size": 40}, abi.INCOMPATIBLE_ABI),
])
def test_allocation_rules(session, fields, status):
    d = abi.allocation_desc_init()
    for k, v in fields.items():
        setattr(d, k, v)
    h = ctypes.c_void_p()
    assert session.api.allocation_create(session.handle, ctypes.byref(d), ctypes.byref(h)) == status
    if status == abi.SUCCESS:
        info = abi.AllocationInfo()
        info.struct_size = 1000  # larger caller struct: preserved on output
        assert session.api.allocation_get_info(h, ctypes.byref(info)) == abi.SUCCESS
        assert info.struct_size == 1000 and info.size_bytes == 4096
        assert session.api.allocation_release(h) == abi.SUCCESS


def test_allocation_io_bounds(session):
    a = session.allocation(4096)
    data = np.arange(1024, dtype=np.float32)
    a.write(data)
    assert np.array_equal(a.read(dtype=np.float32), data)
    assert np.array_equal(a.read(16, offset=4000, dtype=np.float32), data[1000:1004])
    api = session.api
    buf = np.zeros(8, np.float32)
    assert api.allocation_write(a.handle, 4090, buf.ctypes.data_as(ctypes.c_void_p), 8) == abi.INVALID_ARGUMENT
    assert api.allocation_read(a.handle, 0, None, 4) == abi.INVALID_ARGUMENT
    assert api.allocation_read(a.handle, 0, None, 0) == abi.SUCCESS
    a.release()
    # zero-initialised backing
    b = session.allocation(8192)
    assert not b.read().any()


def test_gemm_descriptor_rules(session):
    a = session.allocation(64 * 64 * 4)
    b = session.allocation(64 * 64 * 4)
    c = session.allocation(64 * 64 * 4)
    api = session.api

    def status_of(mutate):
        d = abi.gemm_desc_init()
        d.a = xv.matrix(a, 64, 64, 64)
        d.b = xv.matrix(b, 64, 64, 64)
        d.c = xv.matrix(c, 64, 64, 64)
        mutate(d)
        h = ctypes.c_void_p()
        st = api.gemm_plan_create(session.handle, ctypes.byref(d), ctypes.byref(h))
        if st == abi.SUCCESS:
            api.gemm_plan_release(h)
        return st

    assert status_of(lambda d: None) == abi.SUCCESS
    assert status_of(lambda d: setattr(d, "flags", 1)) == abi.INVALID_ARGUMENT
    assert status_of(lambda d: setattr(d, "operation_a", 2)) == abi.INVALID_ARGUMENT
    assert status_of(lambda d: setattr(d, "compute_mode", 4)) == abi.INVALID_ARGUMENT
    assert status_of(lambda d: setattr(d.a, "struct_size", 8)) == abi.INCOMPATIBLE_ABI
    assert status_of(lambda d: setattr(d.b, "allocation", None)) == abi.INVALID_ARGUMENT
    assert status_of(lambda d: setattr(d.c, "rows", 0)) == abi.INVALID_ARGUMENT
    assert status_of(lambda d: setattr(d.c, "layout", 2)) == abi.INVALID_ARGUMENT
    assert status_of(lambda d: setattr(d, "deadline_ms", 1 << 63)) == abi.INVALID_ARGUMENT
    # valid FP16 problem: accepted by validation, not implemented on this path
    def fp16(d):
        for mx in (d.a, d.b):
            mx.data_type = abi.DATA_FP16
        d.c.data_type = abi.DATA_FP32
        d.compute_mode = abi.COMPUTE_FP32_STRICT
    assert status_of(fp16) == abi.UNSUPPORTED
    # TF32 requests are served by the strict FP32 path and say so
    plan = xv.GemmPlan(session, xv.matrix(a, 64, 64, 64), xv.matrix(b, 64, 64, 64),
                       xv.matrix(c, 64, 64, 64), compute_mode=abi.COMPUTE_FP32_TF32)
    assert plan.info().effective_compute_mode == abi.COMPUTE_FP32_STRICT
    assert plan.info().uses_cublas_lt == 0
    plan.release()


def abi_verdicts(session, cases):
    """gemm_plan_create of each case: (status, last error message)."""
    allocs = [session.allocation(size) for size in generators.VALIDATION_SIZES]
    api = session.api
    out = []
    for c in cases:
        gd = abi.gemm_desc_init()
        gd.a, gd.b, gd.c = [xv.matrix(allocs[al], rows, cols, ld, layout, offset, dtype)
                            for al, offset, rows, cols, ld, layout, dtype in c["mats"]]
        gd.operation_a, gd.operation_b = c["op_a"], c["op_b"]
        gd.compute_mode = c["compute"]
        gd.beta = c["beta"]
        h = ctypes.c_void_p()
        st = api.gemm_plan_create(session.handle, ctypes.byref(gd), ctypes.byref(h))
        msg = session.error().message.decode() if st != abi.SUCCESS else ""
        if st == abi.SUCCESS:
            api.gemm_plan_release(h)
        out.append((st, msg))
    return out


def check_verdicts(cases, verdicts, wants):
    """A reference verdict of 0 (valid) must plan (FP32) or be UNSUPPORTED
    (other types); any other verdict is INVALID_ARGUMENT naming that class."""
    seen = set()
    for c, (st, msg), want in zip(cases, verdicts, wants):
        seen.add(want)
        if want == 0:
            expected = abi.SUCCESS if c["mats"][0][6] == abi.DATA_FP32 else abi.UNSUPPORTED
            assert st == expected, (c, st, msg)
        else:
            assert st == abi.INVALID_ARGUMENT, (c, st)
            assert f"invalid_problem: {PROBLEM_ERRORS[want]}" in msg, (c, msg, PROBLEM_ERRORS[want])
    # every class reachable through the ABI (the ABI itself rejects zero
    # sizes and bad enums first, and one handle cannot have two sizes)
    assert seen >= {0, 7, 8, 9, 10, 11, 12, 13}, sorted(seen)


def test_problem_validation_matches_recorded_reference(session):
    cases = generators.validation_cases(1500, 2024)
    wants = generators.reference_outputs("validation", cases)
    check_verdicts(cases, abi_verdicts(session, cases), wants)


def test_problem_validation_matches_reference(session):
    """The same random descriptors through the compiled reference planner."""
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("reference planner not built here (oracle/_ref needs /root/reference)")
    ref.ref_validate_problem.argtypes = [ctypes.POINTER(generators.RefMatrix)] * 3 + [
        ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double]
    cases = generators.validation_cases(1500, 2024)
    wants = []
    for c in cases:
        mats = [generators.ref_matrix(m) for m in c["mats"]]
        rc = generators.reference_compute_mode(c["compute"], c["mats"][0][6])
        wants.append(ref.ref_validate_problem(*(ctypes.byref(m) for m in mats), c["op_a"],
                                              c["op_b"], rc, c["beta"]))
    assert wants == generators.reference_outputs("validation", cases)
    check_verdicts(cases, abi_verdicts(session, cases), wants)
