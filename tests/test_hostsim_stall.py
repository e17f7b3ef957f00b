"""CPU tests of the stall deadline on device waits, over libxvram_hostsim.so.

The simulated device can be told that every event recorded from some point on
never completes (xvram_hostsim_inject at the event-hang site), as if the work
queued before it had hung on the GPU. Every host wait on device work polls
against the session's stall deadline (XVRAM_STALL_TIMEOUT_MS, default 5 s;
150 ms here), so a GEMM, a transaction, a drain and a host read each return
TIMEOUT soon after the deadline instead of blocking forever. The session is
then poisoned (later calls fail), and close leaves the frames, the workspace
and the pinned host buffers that hung work may still use mapped and allocated
(CLEANUP_FAILED) instead of releasing them.

Reference behaviour followed: wait_event (src/residency/runtime.cpp:3031-3051:
poll until the stall deadline, then poison with timeout and quarantine the
in-flight generation), wait_external with config_.stall_timeout (:1494, 1508,
1555), the quarantined teardown (:1575-1595, 1745-1760) and the SDK's abandon
at close (src/sdk/runtime.cpp:900-915)."""
import ctypes
import time

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import uniform

KiB = 1 << 10
F = 16 * KiB
SITE_EVENT_HANG = 17
STALL_MS = 150
# Generous bound for one failed call: the first expired wait quarantines the
# session, after which no further wait is attempted.
LATE_MS = 2000


@pytest.fixture()
def sim(monkeypatch):
    monkeypatch.setenv("XVRAM_STALL_TIMEOUT_MS", str(STALL_MS))
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_inject.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int]
    yield lib
    lib.dll.xvram_hostsim_reset()


def hang_after(lib, records):
    """Every event recorded after `records` more records never completes."""
    assert lib.dll.xvram_hostsim_inject(SITE_EVENT_HANG, records, 1) == 0


def make_session(lib):
    return xv.Session(lib, chunk_size_bytes=F, cache_target_bytes=14 * F, workspace_cap_bytes=0,
                      device_headroom_bytes=0)


def gemm_plan(s, oracle_mod, m=96, n=40):
    a, b, c = s.allocation(m * m * 4), s.allocation(m * n * 4), s.allocation(m * n * 4)
    a.write(np.asfortranarray(uniform(oracle_mod, m, m, 61)).T.copy())
    b.write(np.asfortranarray(uniform(oracle_mod, m, n, 62)).T.copy())
    plan = xv.GemmPlan(s, xv.matrix(a, m, m, m), xv.matrix(b, m, n, m), xv.matrix(c, m, n, m))
    assert plan.info().tile_count > 1
    return plan, c


def timed(call):
    t0 = time.monotonic()
    status = call()
    return status, (time.monotonic() - t0) * 1e3


def assert_quarantined(s, lib):
    """Poisoned: later work is refused, and close abandons the mapped frames."""
    t = s.telemetry()
    assert t.poisoned == 1
    desc = abi.allocation_desc_init()
    desc.size_bytes = F
    h = ctypes.c_void_p()
    assert s.api.allocation_create(s.handle, ctypes.byref(desc), ctypes.byref(h)) == abi.POISONED
    mapped_before = t.mappings - t.unmaps
    status, ms = timed(lambda: s.api.session_close(s.handle, abi.TIMEOUT_INFINITE))
    assert status == abi.CLEANUP_FAILED
    assert ms < LATE_MS
    err = s.error()
    assert err.status == abi.CLEANUP_FAILED and err.operation == b"quarantine"
    t = s.telemetry()
    # Nothing that hung work may still touch was unmapped or released.
    assert t.mappings - t.unmaps == mapped_before > 0
    assert t.physical_handles_created > t.physical_handles_released
    return t


@pytest.mark.parametrize("records", [0, 1, 3, 6, 10])
def test_gemm_that_stalls_times_out_and_quarantines(sim, oracle_mod, records):
    s = make_session(sim)
    try:
        plan, _ = gemm_plan(s, oracle_mod)
        hang_after(sim, records)
        status, ms = timed(lambda: s.api.gemm_execute(plan.handle, abi.TIMEOUT_INFINITE))
        assert status == abi.TIMEOUT, abi.STATUS.get(status)
        assert STALL_MS <= ms < LATE_MS
        assert s.error().status == abi.TIMEOUT
        # The next GEMM is refused at once; the queue still drains.
        status, ms = timed(lambda: s.api.gemm_execute(plan.handle, abi.TIMEOUT_INFINITE))
        assert status == abi.POISONED and ms < LATE_MS
        assert_quarantined(s, sim)
        plan.release()
    finally:
        s.release()


def test_transaction_that_stalls_times_out(sim, oracle_mod):
    s = make_session(sim)
    try:
        a = s.allocation(4 * F)
        calls = []
        hang_after(sim, 0)
        t0 = time.monotonic()
        with pytest.raises(xv.XvramError) as e:
            s.execute_transaction([xv.access(a, 0, 4 * F, abi.ACCESS_READ_WRITE)],
                                  lambda view: calls.append(len(view.ranges)))
        ms = (time.monotonic() - t0) * 1e3
        assert e.value.status == abi.TIMEOUT and ms < LATE_MS
        assert_quarantined(s, sim)
    finally:
        s.release()


def test_drain_of_dirty_results_that_stalls_times_out(sim, oracle_mod):
    s = make_session(sim)
    try:
        plan, c = gemm_plan(s, oracle_mod)
        plan.execute()                       # C stays cached and dirty
        assert s.telemetry().writebacks_completed == 0
        hang_after(sim, 0)
        status, ms = timed(lambda: s.api.session_drain(s.handle, abi.TIMEOUT_INFINITE))
        assert status == abi.TIMEOUT and STALL_MS <= ms < LATE_MS
        # A host read of C needs the same write-back: refused at once.
        buf = np.empty(96 * 40 * 4, np.uint8)
        st = s.api.allocation_read(c.handle, 0, buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes)
        assert st == abi.POISONED
        assert_quarantined(s, sim)
        plan.release()
    finally:
        s.release()


def test_host_read_that_stalls_times_out(sim, oracle_mod):
    s = make_session(sim)
    try:
        plan, c = gemm_plan(s, oracle_mod)
        plan.execute()
        hang_after(sim, 0)
        buf = np.empty(96 * 40 * 4, np.uint8)
        status, ms = timed(lambda: s.api.allocation_read(
            c.handle, 0, buf.ctypes.data_as(ctypes.c_void_p), buf.nbytes))
        assert status == abi.TIMEOUT and STALL_MS <= ms < LATE_MS
        assert_quarantined(s, sim)
        plan.release()
    finally:
        s.release()


def test_waits_that_complete_are_not_affected(sim, oracle_mod):
    """Without a hang the same session runs, drains and closes balanced."""
    s = make_session(sim)
    plan, c = gemm_plan(s, oracle_mod)
    plan.execute()
    s.drain()
    plan.release()
    s.close()
    t = s.telemetry()
    assert t.poisoned == 0 and t.mappings == t.unmaps
    assert t.physical_handles_created == t.physical_handles_released
    s.release()
