"""CPU tests of working-set transactions and prefetch through the C ABI, over
libxvram_hostsim.so (device addresses there are host pointers, so a callback
can read and write the resident bytes directly).

Reference behaviour followed: access normalisation and the write-only rule
(src/residency/core.cpp:128-276, cases from tests/unit/residency_core_tests.cpp
:38-122), transaction execution, callback failure and the duration guard
(src/residency/runtime.cpp:1012-1495), the SDK wrapper
(src/sdk/runtime.cpp:394-499) and ABI validation (src/sdk/api.cpp:236-276,
:700-806)."""
import ctypes
import random
import time

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import uniform

KiB = 1 << 10
F = 4 * KiB  # hostsim granularity = frame size used here
R, RW, WO = abi.ACCESS_READ, abi.ACCESS_READ_WRITE, abi.ACCESS_WRITE_ONLY
SITE_COPY_H2D = 14


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_inject.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int]
    yield lib
    lib.dll.xvram_hostsim_reset()


def session(lib, frames=8, workspace=0, **extra):
    cfg = dict(chunk_size_bytes=F, cache_target_bytes=frames * F + workspace,
               workspace_cap_bytes=workspace, device_headroom_bytes=0)
    cfg.update(extra)
    return xv.Session(lib, **cfg)


def dev(addr, n):
    return np.ctypeslib.as_array((ctypes.c_uint8 * n).from_address(addr))


def rand_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def test_reference_normalization_case(sim):
    """tests/unit/residency_core_tests.cpp:38-85 scaled from 8-byte to 4 KiB chunks."""
    u = F // 8
    with session(sim) as s:
        first, second = s.allocation(20 * u), s.allocation(8 * u)
        id1, id2 = first.info().allocation_id, second.info().allocation_id
        d1, d2 = rand_bytes(20 * u, 1), rand_bytes(8 * u, 2)
        first.write(d1)
        second.write(d2)
        t0 = s.telemetry()
        seen = []

        def cb(view):
            seen.extend(view.ranges)
            for aid, off, ln, addr, mode in view.ranges:
                if mode == WO:
                    dev(addr, ln)[:] = (aid * 16 + off // u) & 0xFF
                elif mode == RW:
                    dev(addr, ln)[:] ^= 0x5A

        s.execute_transaction([xv.access(first, 0, 16 * u, WO), xv.access(first, 4 * u, 4 * u, R),
                               xv.access(first, 16 * u, 4 * u, WO),
                               xv.access(second, 0, 4 * u, WO), xv.access(second, 4 * u, 4 * u, WO)],
                              cb)
        t1 = s.telemetry()
        got = [(a, o, l, m) for a, o, l, _, m in seen]
        assert got == [(id1, 0, 4 * u, WO), (id1, 4 * u, 4 * u, RW), (id1, 8 * u, 12 * u, WO),
                       (id2, 0, 8 * u, WO)]
        # One contiguous device range per allocation.
        assert seen[1][3] - seen[0][3] == 4 * u and seen[2][3] - seen[0][3] == 8 * u
        # Only the mixed chunk (first, 0) is loaded; the other three are full
        # write-only chunks (including the 4-byte-scaled tail).
        assert t1.bytes_h2d - t0.bytes_h2d == F
        # The four written chunks stay cached, dirty (write-back cache) ...
        assert t1.writebacks_completed == t0.writebacks_completed
        assert t1.bytes_d2h == t0.bytes_d2h
        assert t1.transactions_completed - t0.transactions_completed == 1
        out1, out2 = first.read(), second.read()
        # ... until the reads write them back.
        t2 = s.telemetry()
        assert t2.writebacks_completed - t0.writebacks_completed == 4
        assert t2.bytes_d2h - t0.bytes_d2h == 20 * u + 8 * u
        assert t2.dirty_evictions == t0.dirty_evictions
        exp1 = d1.copy()
        exp1[0:4 * u] = (id1 * 16 + 0) & 0xFF
        exp1[4 * u:8 * u] ^= 0x5A
        exp1[8 * u:20 * u] = (id1 * 16 + 8) & 0xFF
        assert np.array_equal(out1, exp1)
        assert np.array_equal(out2, np.full(8 * u, (id2 * 16) & 0xFF, np.uint8))


def test_partial_write_only_loads_chunk(sim):
    """residency_core_tests.cpp:86-94: a partial write-only span needs the chunk's bytes."""
    with session(sim) as s:
        a = s.allocation(3 * F)
        data = rand_bytes(3 * F, 3)
        a.write(data)
        t0 = s.telemetry()

        def cb(view):
            (_, off, ln, addr, mode), = view.ranges
            dev(addr, ln)[:] = 7

        s.execute_transaction([xv.access(a, F + 100, 200, WO)], cb)
        t1 = s.telemetry()
        assert t1.bytes_h2d - t0.bytes_h2d == F
        exp = data.copy()
        exp[F + 100:F + 300] = 7
        assert np.array_equal(a.read(), exp)


def test_multi_chunk_read_is_contiguous_and_stable(sim):
    with session(sim, frames=8) as s:
        a = s.allocation(5 * F + 100)
        assert a.info().stable_virtual_address == 1
        data = rand_bytes(5 * F + 100, 4)
        a.write(data)
        grabbed = {}

        def cb(view):
            (_, off, ln, addr, mode), = view.ranges
            grabbed["addr"] = addr
            grabbed["bytes"] = dev(addr, ln).copy()

        s.execute_transaction([xv.access(a, 1000, 5 * F + 50 - 1000, R)], cb)
        assert np.array_equal(grabbed["bytes"], data[1000:5 * F + 50])
        first_addr = grabbed["addr"]
        t0 = s.telemetry()
        s.execute_transaction([xv.access(a, 1000, 5 * F + 50 - 1000, R)], cb)
        t1 = s.telemetry()
        assert grabbed["addr"] == first_addr
        assert t1.cache_hits - t0.cache_hits == 6
        assert t1.bytes_h2d == t0.bytes_h2d
        assert t1.bytes_d2h == t0.bytes_d2h  # read-only: nothing written back


def test_random_transactions_match_model(sim):
    """Out-of-core: 24 chunks through 5 frames, random overlapping spans and modes."""
    nchunks, frames = 24, 5
    size = nchunks * F - 300
    rng = random.Random(5)
    with session(sim, frames=frames) as s:
        a = s.allocation(size)
        model = rand_bytes(size, 6)
        a.write(model)
        bases = set()
        for step in range(60):
            ranges = []
            lo_chunk = rng.randrange(nchunks - 4)
            for _ in range(rng.randint(1, 3)):
                off = rng.randrange(lo_chunk * F, min(size - 1, (lo_chunk + 4) * F))
                ln = rng.randint(1, min(size, (lo_chunk + 5) * F) - off)
                ranges.append(xv.access(a, off, ln, rng.choice([R, RW, WO])))
            seed = 1000 + step
            mismatch = []

            def cb(view, seed=seed):
                r2 = np.random.default_rng(seed)
                for _, off, ln, addr, mode in view.ranges:
                    bases.add(addr - off)
                    v = dev(addr, ln)
                    if mode in (R, RW) and not np.array_equal(v, model[off:off + ln]):
                        mismatch.append((step, off, ln))
                    if mode == RW:
                        x = np.uint8(r2.integers(1, 256))
                        v ^= x
                        model[off:off + ln] ^= x
                    elif mode == WO:
                        fill = r2.integers(0, 256, ln, dtype=np.uint8)
                        v[:] = fill
                        model[off:off + ln] = fill

            s.execute_transaction(ranges, cb)
            assert not mismatch, mismatch
        assert np.array_equal(a.read(), model)
        t = s.telemetry()
        assert t.clean_evictions + t.dirty_evictions > 0
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        assert len(bases) == 1  # one base address for the allocation throughout


def test_transactions_and_gemm_stay_coherent(sim, oracle_mod):
    m = n = k = 64
    a_np = uniform(oracle_mod, m, k, 11)
    b_np = uniform(oracle_mod, k, n, 12)
    with session(sim, frames=16) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        A.write(np.asfortranarray(a_np).T.reshape(-1))
        B.write(np.asfortranarray(b_np).T.reshape(-1))
        C.write(np.zeros(m * n, np.float32))
        # Cache C as a clean chunk first, so the GEMM's write-back must drop it.
        s.execute_transaction([xv.access(C, 0, m * n * 4, R)], lambda v: None)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k), xv.matrix(C, m, n, m))
        plan.execute()
        seen = {}

        def grab(view):
            (_, off, ln, addr, mode), = view.ranges
            seen["c"] = dev(addr, ln).view(np.float32).copy()

        s.execute_transaction([xv.access(C, 0, m * n * 4, R)], grab)
        c_host = C.read(dtype=np.float32)
        assert np.array_equal(seen["c"], c_host)
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a_np), np.asfortranarray(b_np),
                                          1.0, 0.0, None)
        bad, _, _ = oracle_mod.check_bound(c_host.reshape(n, m).T, k, ref, absab)
        assert bad == 0

        # Double A inside a transaction; the GEMM's cached A panels must be dropped.
        def double(view):
            (_, off, ln, addr, mode), = view.ranges
            v = dev(addr, ln).view(np.float32)
            v *= 2.0

        s.execute_transaction([xv.access(A, 0, m * k * 4, RW)], double)
        plan.execute()
        c2 = C.read(dtype=np.float32).reshape(n, m).T
        ref2, absab2 = oracle_mod.sgemm_f64(np.asfortranarray(2 * a_np), np.asfortranarray(b_np),
                                            1.0, 0.0, None)
        bad, _, _ = oracle_mod.check_bound(c2, k, ref2, absab2)
        assert bad == 0
        plan.release()


def test_prefetch_then_transaction_hits(sim):
    with session(sim, frames=8) as s:
        a = s.allocation(4 * F)
        data = rand_bytes(4 * F, 7)
        a.write(data)
        t0 = s.telemetry()
        op = s.prefetch([xv.access(a, 0, 4 * F, R)])
        status, info = op.wait()
        assert status == abi.SUCCESS and info.result == abi.SUCCESS
        assert info.state == abi.OPERATION_COMPLETED
        op.release()
        t1 = s.telemetry()
        assert t1.cache_misses - t0.cache_misses == 4 and t1.bytes_h2d - t0.bytes_h2d == 4 * F
        got = {}

        def cb(view):
            (_, off, ln, addr, mode), = view.ranges
            got["b"] = dev(addr, ln).copy()

        s.execute_transaction([xv.access(a, 0, 4 * F, R)], cb)
        t2 = s.telemetry()
        assert t2.cache_hits - t1.cache_hits == 4 and t2.bytes_h2d == t1.bytes_h2d
        assert np.array_equal(got["b"], data)


def test_workspace(sim):
    with session(sim, frames=6, workspace=8 * KiB) as s:
        a = s.allocation(F)
        got = {}

        def cb(view):
            got["ws"] = (view.workspace_address, view.workspace_bytes)
            if view.workspace_bytes:
                dev(view.workspace_address, view.workspace_bytes)[:] = 1

        s.execute_transaction([xv.access(a, 0, F, R)], cb, workspace_bytes=4 * KiB)
        assert got["ws"][0] != 0 and got["ws"][1] == 4 * KiB
        s.execute_transaction([xv.access(a, 0, F, R)], cb, workspace_bytes=0)
        assert got["ws"] == (0, 0)
        with pytest.raises(xv.XvramError) as e:
            s.transaction([xv.access(a, 0, F, R)], cb, workspace_bytes=8 * KiB + 1)
        assert e.value.status == abi.INVALID_ARGUMENT
        assert s.telemetry().workspace_bytes >= 4 * KiB


def test_callback_status_and_error_record_propagate(sim):
    with session(sim) as s:
        a = s.allocation(F)
        data = rand_bytes(F, 8)
        a.write(data)

        def fails(view):
            (_, off, ln, addr, mode), = view.ranges
            dev(addr, ln)[:] = 0  # enqueued work that must not reach the host copy
            raise ValueError("kernel launch refused")

        with pytest.raises(xv.XvramError) as e:
            s.execute_transaction([xv.access(a, 0, F, RW)], fails)
        assert e.value.status == abi.CALLBACK_FAILED
        assert b"kernel launch refused" in e.value.info.message
        assert e.value.info.native_domain == abi.NATIVE_ERROR_CALLBACK
        assert s.telemetry().poisoned == 1
        with pytest.raises(xv.XvramError) as e2:
            s.execute_transaction([xv.access(a, 0, F, R)], lambda v: None)
        assert e2.value.status == abi.POISONED


def test_callback_own_status_is_reported(sim):
    with session(sim) as s:
        a = s.allocation(F)
        with pytest.raises(xv.XvramError) as e:
            s.execute_transaction([xv.access(a, 0, F, R)], lambda v: abi.CORRUPTION)
        assert e.value.status == abi.CORRUPTION
        assert e.value.info.native_domain == abi.NATIVE_ERROR_CALLBACK


def test_duration_guard_blocks_later_launches(sim):
    with session(sim, max_transaction_ms=5) as s:
        a = s.allocation(F)

        def slow(view):
            (_, off, ln, addr, mode), = view.ranges
            dev(addr, ln)[:] = 9
            time.sleep(0.03)

        with pytest.raises(xv.XvramError) as e:
            s.execute_transaction([xv.access(a, 0, F, RW)], slow)
        assert e.value.status == abi.TIMEOUT
        t = s.telemetry()
        assert t.watchdog_rejections == 1 and t.last_transaction_ms >= 5
        # The work completed and was written back before the guard tripped.
        assert np.array_equal(a.read(), np.full(F, 9, np.uint8))
        with pytest.raises(xv.XvramError) as e2:
            s.execute_transaction([xv.access(a, 0, F, R)], lambda v: None)
        assert e2.value.status == abi.INVALID_ARGUMENT


def test_duration_guard_on_gemm_kernels(sim, oracle_mod):
    """The guard also covers tile kernels (dispatched without a start event:
    a kernel's start is derived from the events its lane follows). On the
    simulated device a 128 x 128 x 1024 launch computes on the host for far
    longer than 1 ms: the operation completes, then fails with TIMEOUT, and
    later launches are refused."""
    m, n, k = 128, 128, 1024
    a_op = uniform(oracle_mod, m, k, 61)
    b_op = uniform(oracle_mod, k, n, 62)
    with xv.Session(sim, chunk_size_bytes=1 << 20, workspace_cap_bytes=0,
                    device_headroom_bytes=0, max_transaction_ms=1) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        A.write(np.asfortranarray(a_op).reshape(-1, order="F"))
        B.write(np.asfortranarray(b_op).reshape(-1, order="F"))
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k), xv.matrix(C, m, n, m))
        assert plan.info().tile_count == 1
        with pytest.raises(xv.XvramError) as e:
            plan.execute()
        assert e.value.status == abi.TIMEOUT
        t = s.telemetry()
        assert t.watchdog_rejections == 1 and t.last_transaction_ms >= 1
        out = C.read(dtype=np.float32).reshape(n, m).T
        ref = a_op.astype(np.float64) @ b_op.astype(np.float64)
        bound = 4 * k * 2.0 ** -24 * (np.abs(a_op).astype(np.float64) @ np.abs(b_op).astype(np.float64))
        assert np.all(np.abs(out - ref) <= bound)  # the work completed before the guard tripped
        with pytest.raises(xv.XvramError) as e2:
            plan.execute()
        assert e2.value.status == abi.INVALID_ARGUMENT
        plan.release()


def test_host_stall_between_dispatches_does_not_trip_the_guard(sim):
    """A tile kernel without a start event inherits its start from the event
    its lane last recorded (the previous kernel's stop, or the operation's
    start marker). When the host itself stalls before a dispatch with no fill
    to wait for (here: one event record sleeps 100 ms on the host, at each
    record of a repeated, fully cached 96 x 40 x 96 GEMM in turn), the lane
    may have idled meanwhile: the kernel then takes a real start event, so the
    idle time is not counted as kernel time and a 50 ms guard does not trip.
    (The record after the operation's start marker on lane 0 is such a stall:
    lane 0's first kernel would otherwise inherit that marker.)"""
    sim.dll.xvram_hostsim_delay.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int]
    site_event_record = 12
    m, n = 96, 40
    for skip in range(0, 24):
        sim.dll.xvram_hostsim_reset()
        with xv.Session(sim, chunk_size_bytes=16 * KiB, cache_target_bytes=32 * 16 * KiB,
                        workspace_cap_bytes=0, device_headroom_bytes=0,
                        max_transaction_ms=50) as s:
            a, b, c = s.allocation(m * m * 4), s.allocation(m * n * 4), s.allocation(m * n * 4)
            a.write(np.ones(m * m, np.float32))
            b.write(np.ones(m * n, np.float32))
            plan = xv.GemmPlan(s, xv.matrix(a, m, m, m), xv.matrix(b, m, n, m),
                               xv.matrix(c, m, n, m))
            plan.execute()
            assert sim.dll.xvram_hostsim_delay(site_event_record, skip, 100) == 0
            plan.execute()
            t = s.telemetry()
            assert t.watchdog_rejections == 0 and t.last_transaction_ms < 50, skip
            assert np.array_equal(c.read(dtype=np.float32), np.full(m * n, m, np.float32))
            plan.release()


@pytest.mark.parametrize("max_ms,split", [(0, False), (1, True)])
def test_planner_keeps_launches_under_the_guard(sim, max_ms, split):
    """Plans are sized against max_transaction_ms (at a deliberately low assumed
    rate), so a whole-fit problem is split when one launch could trip the guard."""
    n = 4096
    with xv.Session(sim, chunk_size_bytes=64 << 20, cache_target_bytes=8 * (64 << 20),
                    workspace_cap_bytes=0, device_headroom_bytes=0,
                    max_transaction_ms=max_ms) as s:
        a, b, c = (s.allocation(n * n * 4) for _ in range(3))
        plan = xv.GemmPlan(s, xv.matrix(a, n, n, n), xv.matrix(b, n, n, n), xv.matrix(c, n, n, n))
        info = plan.info()
        flops = 2.0 * info.tile_m * info.tile_n * info.tile_k
        limit = (max_ms or 250) * 4.0e10
        assert flops <= limit
        assert (info.tile_count > 1) == split
        plan.release()


def test_queued_deadline_and_cancel(sim):
    with session(sim) as s:
        a = s.allocation(F)
        calls = []

        def slow(view):
            calls.append("slow")
            time.sleep(0.1)

        first = s.transaction([xv.access(a, 0, F, R)], slow)
        late = s.transaction([xv.access(a, 0, F, R)], lambda v: calls.append("late"),
                             deadline_ms=10)
        cancelled = s.transaction([xv.access(a, 0, F, R)], lambda v: calls.append("cancelled"))
        assert cancelled.cancel() == abi.SUCCESS
        st, info = first.wait()
        assert st == abi.SUCCESS and info.result == abi.SUCCESS
        st, info = late.wait()
        assert info.result == abi.TIMEOUT
        st, info = cancelled.wait()
        assert info.state == abi.OPERATION_CANCELLED
        for op in (first, late, cancelled):
            op.release()
        assert calls == ["slow"]
        assert s.telemetry().poisoned == 0
        s.execute_transaction([xv.access(a, 0, F, R)], lambda v: calls.append("after"))
        assert calls[-1] == "after"


def test_access_validation(sim):
    with session(sim, frames=4) as s:
        a = s.allocation(2 * F)
        other = s.allocation(F)
        cb = lambda v: None

        def status_of(ranges, **kw):
            with pytest.raises(xv.XvramError) as e:
                s.execute_transaction(ranges, cb, **kw)
            return e.value

        err = status_of([xv.access(a, 2 * F - 1, 2, R)])
        assert err.status == abi.INVALID_ARGUMENT
        assert b"range_out_of_bounds" in err.info.message
        assert status_of([xv.access(a, 0, 0, R)]).status == abi.INVALID_ARGUMENT
        assert status_of([xv.access(a, 0, 4, 7)]).status == abi.INVALID_ARGUMENT
        assert status_of([xv.access(a, (1 << 64) - 2, 4, R)]).status == abi.INVALID_ARGUMENT
        assert status_of([]).status == abi.INVALID_ARGUMENT
        # More chunks than frames.
        big = s.allocation(6 * F)
        assert status_of([xv.access(big, 0, 6 * F, R)]).status == abi.BUDGET_PRESSURE
        other.release()
        with pytest.raises(xv.XvramError) as e:
            s.transaction([xv.access(a, 0, F, R)], cb, deadline_ms=(1 << 64) - 1)
        assert e.value.status == abi.INVALID_ARGUMENT
        assert s.telemetry().poisoned == 0
        s.execute_transaction([xv.access(a, 0, 2 * F, R)], cb)


def test_raw_abi_rejections(sim):
    """Null callback, non-zero flags and a released allocation (src/sdk/api.cpp:733-780)."""
    with session(sim) as s:
        a = s.allocation(F)
        rng = (abi.AccessRange * 1)(xv.access(a, 0, F, R))
        desc = abi.TransactionDesc()
        desc.struct_size = ctypes.sizeof(desc)
        desc.ranges = ctypes.cast(rng, ctypes.POINTER(abi.AccessRange))
        desc.range_count = 1
        out = ctypes.c_void_p()
        assert s.api.transaction_submit(s.handle, ctypes.byref(desc), ctypes.byref(out)) == \
            abi.INVALID_ARGUMENT  # null callback
        keep = abi.TransactionCallback(lambda c, u, e: 0)
        desc.callback = keep
        desc.flags = 1
        assert s.api.transaction_submit(s.handle, ctypes.byref(desc), ctypes.byref(out)) == \
            abi.INVALID_ARGUMENT
        desc.flags = 0
        desc.struct_size = ctypes.sizeof(desc) - 8
        assert s.api.transaction_submit(s.handle, ctypes.byref(desc), ctypes.byref(out)) == \
            abi.INCOMPATIBLE_ABI
        desc.struct_size = ctypes.sizeof(desc)
        assert s.api.transaction_execute(s.handle, ctypes.byref(desc), abi.TIMEOUT_INFINITE) == \
            abi.SUCCESS
        pdesc = abi.PrefetchDesc()
        pdesc.struct_size = ctypes.sizeof(pdesc)
        pdesc.ranges = desc.ranges
        pdesc.range_count = 1
        pdesc.reserved[1] = 1
        assert s.api.prefetch_submit(s.handle, ctypes.byref(pdesc), ctypes.byref(out)) == \
            abi.INVALID_ARGUMENT


def test_injected_copy_fault_poisons(sim):
    with session(sim) as s:
        a = s.allocation(F)
        sim.dll.xvram_hostsim_inject(SITE_COPY_H2D, 0, 0)
        with pytest.raises(xv.XvramError) as e:
            s.execute_transaction([xv.access(a, 0, F, R)], lambda v: None)
        assert e.value.status == abi.CUDA_ERROR
        assert s.telemetry().poisoned == 1


def test_teardown_balances_mappings(sim):
    with session(sim, frames=3) as s:
        allocs = [s.allocation(2 * F) for _ in range(3)]
        for i in range(6):
            x = allocs[i % 3]
            s.execute_transaction([xv.access(x, 0, 2 * F, RW)], lambda v: None)
        allocs[0].release()
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps
        assert t.physical_handles_created == t.physical_handles_released
        assert t.resident_bytes == 0
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
