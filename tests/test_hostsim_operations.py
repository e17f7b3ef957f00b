"""CPU tests of asynchronous operations through the C ABI, over
libxvram_hostsim.so: the lifecycle of an operation (queued -> running ->
completed/failed, queued -> cancelled), cancel while queued, while running and
after the end, the queue deadline, waits that time out, and progress counted in
the plan's tiles.

Reference behaviour followed: RuntimeOperation (src/sdk/runtime.cpp:146-279:
cancel is accepted while queued and BUSY while running; a deadline that has
passed when the operation leaves the queue fails it with TIMEOUT), the
synchronous wrappers (src/sdk/api.cpp:782-806, 876-900) and GEMM progress in
tiles (src/sdk/runtime.cpp:1227; gemm_bench's tiles_retired =
min(units_completed, tile_count))."""
import ctypes
import threading
import time

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import pattern_operands, storage

KiB = 1 << 10
MiB = 1 << 20
F = 4 * KiB


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def session(lib, **extra):
    cfg = dict(chunk_size_bytes=F, cache_target_bytes=8 * F, workspace_cap_bytes=0,
               device_headroom_bytes=0)
    cfg.update(extra)
    return xv.Session(lib, **cfg)


class Gate:
    """A transaction callback that holds the worker until opened."""

    def __init__(self):
        self.entered = threading.Event()
        self.open = threading.Event()

    def __call__(self, _view):
        self.entered.set()
        assert self.open.wait(30)


def test_cancel_of_a_queued_operation_settles_at_once(sim):
    with session(sim) as s:
        a = s.allocation(F)
        gate = Gate()
        held = s.transaction([xv.access(a, 0, F)], gate)
        assert gate.entered.wait(30)
        calls = []
        queued = s.transaction([xv.access(a, 0, F)], lambda v: calls.append("ran"))
        info = queued.poll()
        assert info.state == abi.OPERATION_QUEUED and info.result == abi.SUCCESS
        assert queued.cancel() == abi.SUCCESS
        # Terminal before the worker reaches it: a wait of 0 ms returns now.
        st, info = queued.wait(0)
        assert st == abi.SUCCESS
        assert info.state == abi.OPERATION_CANCELLED and info.result == abi.CANCELLED
        assert queued.error().status == abi.CANCELLED
        # The held operation is running: it cannot be cancelled.
        assert held.poll().state == abi.OPERATION_RUNNING
        assert held.cancel() == abi.BUSY
        assert s.error().status == abi.BUSY
        # A wait that runs out reports TIMEOUT and the state at that moment.
        st, info = held.wait(20)
        assert st == abi.TIMEOUT and info.state == abi.OPERATION_RUNNING
        gate.open.set()
        st, info = held.wait()
        assert st == abi.SUCCESS and info.state == abi.OPERATION_COMPLETED
        assert info.units_completed == info.units_total == 1
        # Cancelling a finished operation changes nothing.
        assert held.cancel() == abi.SUCCESS
        assert held.poll().state == abi.OPERATION_COMPLETED
        # The worker skips the cancelled operation and keeps going.
        s.execute_transaction([xv.access(a, 0, F)], lambda v: calls.append("after"))
        assert calls == ["after"]
        for op in (held, queued):
            op.release()


def test_bounded_waits_last_their_timeout(sim):
    """A waiter watches the phase word for up to 2 ms before it blocks: a
    bounded wait on a running operation still lasts its whole timeout, below
    and above that window, and reports TIMEOUT; an operation that ends while
    waiters watch or block wakes them with SUCCESS."""
    with session(sim) as s:
        a = s.allocation(F)
        gate = Gate()
        held = s.transaction([xv.access(a, 0, F)], gate)
        assert gate.entered.wait(30)
        for timeout_ms in (1, 2, 3, 25):
            t = time.perf_counter()
            st, info = held.wait(timeout_ms)
            elapsed_ms = (time.perf_counter() - t) * 1e3
            assert st == abi.TIMEOUT and info.state == abi.OPERATION_RUNNING
            assert elapsed_ms >= timeout_ms * 0.99, (timeout_ms, elapsed_ms)
        results = []
        waiters = [threading.Thread(target=lambda: results.append(held.wait(10000)[0]))
                   for _ in range(4)]
        for w in waiters:
            w.start()
        time.sleep(0.001)  # some waiters still watching, some perhaps blocked
        gate.open.set()
        for w in waiters:
            w.join(30)
        assert results == [abi.SUCCESS] * 4
        assert held.poll().state == abi.OPERATION_COMPLETED
        held.release()


def test_queue_deadline_fails_with_timeout(sim):
    with session(sim) as s:
        a = s.allocation(F)
        gate = Gate()
        held = s.transaction([xv.access(a, 0, F)], gate)
        assert gate.entered.wait(30)
        late = s.transaction([xv.access(a, 0, F)], lambda v: None, deadline_ms=5)
        time.sleep(0.05)
        gate.open.set()
        st, info = late.wait()
        assert st == abi.SUCCESS
        assert info.state == abi.OPERATION_FAILED and info.result == abi.TIMEOUT
        assert info.elapsed_ms >= 5.0
        assert late.error().operation == b"queue_deadline"
        assert held.wait()[1].result == abi.SUCCESS
        for op in (held, late):
            op.release()


def test_operations_submitted_after_close_are_refused(sim):
    s = session(sim)
    a = s.allocation(F)
    s.close()
    desc, keep = s._transaction_desc([xv.access(a, 0, F)], lambda v: None, 0, 0)
    handle = ctypes.c_void_p()
    assert s.api.transaction_submit(s.handle, ctypes.byref(desc), ctypes.byref(handle)) == abi.CLOSED
    assert not handle.value
    del keep
    # A second close of a closed session succeeds at once.
    assert s.api.session_close(s.handle, 0) == abi.SUCCESS
    a.release()
    s.release()


def test_gemm_progress_counts_plan_tiles(sim):
    """A plan whose launches cover two K panels each (4096 x 4096 C tile,
    six 32-deep panels: two one-panel launches, then two of two): the
    operation has tile_count units and completes all of them."""
    m = n = 4096
    k = 192
    a_op, b_op = pattern_operands(m, n, k)
    with xv.Session(sim, chunk_size_bytes=64 * MiB, cache_target_bytes=12 * 64 * MiB,
                    workspace_cap_bytes=0, device_headroom_bytes=0,
                    max_transaction_ms=600000) as s:
        a_flat, lda = storage(np.ascontiguousarray(a_op), abi.COLUMN_MAJOR)
        b_flat, ldb = storage(np.ascontiguousarray(b_op.T), abi.COLUMN_MAJOR)
        A, B, C = s.allocation(a_flat.nbytes), s.allocation(b_flat.nbytes), s.allocation(m * n * 4)
        A.write(a_flat)
        B.write(b_flat)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, lda), xv.matrix(B, n, k, ldb),
                           xv.matrix(C, m, n, m), abi.OP_N, abi.OP_T,
                           tile_hints=(4096, 4096, 32))
        info = plan.info()
        assert info.tile_count == 6
        op = plan.submit()
        assert op.poll().units_total == info.tile_count
        st, oi = op.wait()
        assert st == abi.SUCCESS and oi.result == abi.SUCCESS
        assert oi.units_total == oi.units_completed == info.tile_count
        op.release()
        plan.release()
