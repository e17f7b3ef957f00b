"""Fault matrix over every device call site of the host simulation (the role of
the reference's FakeCuda fault matrix, tests/unit/residency_executor_fake_tests.cpp:84-114
and :4105): each site fails once, after 0, 1, 3, 8 or 30 successful calls,
while a session runs a small workload through the C ABI -- allocations and
writes, an out-of-core analytic-pattern GEMM, a transaction, a prefetch and the
read-back. Whatever the site and moment:

- a failed call reports XVRAM_STATUS_CUDA_ERROR with the injected native code
  (domain CUDA), or POISONED once an earlier failure has poisoned the session;
- after a device failure the session reports poisoned and accepts no more work;
- a GEMM that reports success produced the exact pattern product;
- session close and release always return (no hang, no crash), and a session
  that saw no fault tears down balanced.

Across the matrix the faults fire during session setup, allocation, the GEMM,
the transaction, allocation release and session close. (The device layer has
no blocking wait: every wait polls event_query, whose failures are covered
here and whose never-ending case is tests/test_hostsim_stall.py.)"""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import pattern_operands

KiB = 1 << 10
SITES = ["init", "mem_info", "va_reserve", "va_free", "mem_create", "mem_release", "mem_map",
         "mem_unmap", "set_access", "host_alloc", "stream_create", "event_create",
         "event_record", "event_query", "copy_h2d", "copy_d2h", "launch"]
INJECTED = 9001  # the simulation's injected error code


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_inject.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int]
    yield lib
    lib.dll.xvram_hostsim_reset()


def workload(lib, oracle_mod, log):
    """Runs the workload; returns the session (or None) and records each
    failing call's (status, native code) in `log`."""
    def attempt(fn, what):
        try:
            return fn()
        except xv.XvramError as exc:
            log.append((what, exc.status, exc.info.native_code if exc.info else 0))
            return None

    s = attempt(lambda: xv.Session(lib, chunk_size_bytes=16 * KiB,
                                   cache_target_bytes=8 * 16 * KiB, workspace_cap_bytes=0,
                                   device_headroom_bytes=0), "session_create")
    if s is None:
        return None, None
    m, n, k = 96, 80, 200
    a_op, b_op = pattern_operands(m, n, k)
    A = attempt(lambda: s.allocation(m * k * 4), "allocation A")
    B = attempt(lambda: s.allocation(k * n * 4), "allocation B")
    C = attempt(lambda: s.allocation(m * n * 4), "allocation C")
    T = attempt(lambda: s.allocation(2 * 16 * KiB), "allocation T")
    product = None
    if A and B and C:
        ok = attempt(lambda: A.write(np.asfortranarray(a_op).T.copy()), "write A") is not False
        attempt(lambda: B.write(np.asfortranarray(b_op).T.copy()), "write B")
        plan = attempt(lambda: xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k),
                                           xv.matrix(C, m, n, m)), "plan")
        if plan is not None and ok:
            before = len(log)
            attempt(plan.execute, "gemm_execute")
            if len(log) == before:
                out = attempt(lambda: C.read(dtype=np.float32), "read C")
                if out is not None:
                    product = np.asfortranarray(out.reshape(n, m).T)
            plan.release()
    if T:
        attempt(lambda: T.write(np.arange(2 * 16 * KiB // 4, dtype=np.float32)), "write T")
        attempt(lambda: s.execute_transaction([xv.access(T, 0, 2 * 16 * KiB, abi.ACCESS_READ)],
                                              lambda view: None), "transaction")
        op = attempt(lambda: s.prefetch([xv.access(T, 0, 16 * KiB)]), "prefetch")
        if op is not None:
            st, info = op.wait()
            if info.result != abi.SUCCESS:
                log.append(("prefetch", info.result, op.error().native_code))
            op.release()
    if product is not None:
        expected = oracle_mod.pattern_expected_matrix(m, n, k)
        assert np.array_equal(product.astype(np.float64), expected), "a successful GEMM is exact"
    return s, (A, B, C, T)


@pytest.mark.parametrize("site", range(len(SITES)), ids=SITES)
@pytest.mark.parametrize("skip", [0, 1, 3, 8, 30])
def test_fault_matrix(sim, oracle_mod, site, skip):
    assert sim.dll.xvram_hostsim_inject(site, skip, 0) == 0
    log = []
    s, handles = workload(sim, oracle_mod, log)
    if s is not None:
        if log:
            # A device failure poisons the session: no more work is accepted.
            assert s.telemetry().poisoned == 1
            with pytest.raises(xv.XvramError) as exc:
                s.allocation(4096)
            assert exc.value.status == abi.POISONED
        failed_before_teardown = bool(log)
        # Teardown may hit the injected site too (va_free, mem_unmap,
        # mem_release...): it must still return.
        for h in handles or ():
            if h:
                try:
                    h.release()
                except xv.XvramError as exc:
                    log.append(("allocation_release", exc.status, exc.info.native_code))
        try:
            s.close()
        except xv.XvramError as exc:
            log.append(("session_close", exc.status, exc.info.native_code if exc.info else 0))
        t = s.telemetry()
        if not log:
            assert t.mappings == t.unmaps
            assert t.physical_handles_created == t.physical_handles_released
            assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
            assert t.resident_bytes == 0
        elif not failed_before_teardown:
            assert t.poisoned == 1
        s.release()
    if log:
        first_what, first_status, first_native = log[0]
        # The first failure is the injected device error itself (a failed
        # session_create has no handle to carry the detail: status only).
        assert first_status == abi.CUDA_ERROR, log
        assert first_native == INJECTED or first_what == "session_create", log
        # Later failures: the same error surfacing, or the poisoned session.
        for what, status, native in log[1:]:
            assert status in (abi.CUDA_ERROR, abi.POISONED, abi.INVALID_ARGUMENT,
                              abi.CLEANUP_FAILED), log
