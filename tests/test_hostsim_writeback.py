"""The write-back cache over libxvram_hostsim.so: what an operation wrote stays
cached and dirty after it, and reaches host memory only on eviction, on an
overlapping allocation_read/allocation_write, when an overlapping entry is
filled, at drain/close, or through the background flush (reference
src/residency/runtime.cpp:931-945 read/write -> flush_overlapping :3155-3173,
drain :1497-1538, close :1620-1625).

Every operand is small-integer valued, so every product below is exact in FP32
and results are compared bit for bit."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

KiB = 1 << 10
SITE_LAUNCH = 16  # the host simulation's kernel-launch site (device_hostsim.cpp)
F = 16 * KiB
R, RW, WO = abi.ACCESS_READ, abi.ACCESS_READ_WRITE, abi.ACCESS_WRITE_ONLY


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def session(lib, frames=16, frame=F, **extra):
    cfg = dict(chunk_size_bytes=frame, cache_target_bytes=frames * frame, workspace_cap_bytes=0,
               device_headroom_bytes=0)
    cfg.update(extra)
    return xv.Session(lib, **cfg)


def ints(rows, cols, seed, lo=-3, hi=4):
    return np.asfortranarray(
        np.random.default_rng(seed).integers(lo, hi, (rows, cols)).astype(np.float32))


def put(s, mat):
    """A column-major allocation holding `mat`."""
    a = s.allocation(mat.size * 4)
    a.write(np.asfortranarray(mat).T.copy())
    return a


def get(alloc, rows, cols):
    return np.asfortranarray(alloc.read(dtype=np.float32).reshape(cols, rows).T)


def run(plan):
    op = plan.submit()
    st, info = op.wait()
    assert st == abi.SUCCESS and info.result == abi.SUCCESS, op.error().message
    op.release()
    return info


def test_resident_repeat_writes_nothing_back(sim):
    """A GEMM whose operands fit: C stays cached between executions, so a
    repeated execution moves no bytes at all (operation_info.bytes_d2h = 0)."""
    m, n, k = 60, 50, 40
    a_h, b_h = ints(m, k, 1), ints(k, n, 2)
    with session(sim) as s:
        a, b, c = put(s, a_h), put(s, b_h), s.allocation(m * n * 4)
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
        assert plan.info().tile_count == 1
        first = run(plan)
        assert first.bytes_d2h == 0 and first.bytes_h2d == (m * k + k * n) * 4
        for _ in range(2):
            again = run(plan)
            assert again.bytes_d2h == 0 and again.bytes_h2d == 0
            assert again.cache_hits == 3 and again.cache_misses == 0
        t0 = s.telemetry()
        assert t0.writebacks_completed == 0
        np.testing.assert_array_equal(get(c, m, n), a_h @ b_h)
        t1 = s.telemetry()
        assert t1.writebacks_completed == 1 and t1.bytes_d2h == m * n * 4
        # The read left C cached, clean: reading again moves nothing.
        np.testing.assert_array_equal(get(c, m, n), a_h @ b_h)
        assert s.telemetry().bytes_d2h == t1.bytes_d2h
        # Another execution dirties C again; the old host copy is not served.
        b.write(np.asfortranarray(2 * b_h).T.copy())
        run(plan)
        np.testing.assert_array_equal(get(c, m, n), a_h @ (2 * b_h))
        plan.release()


def test_beta_accumulates_in_the_cache(sim):
    """beta = 1 reads the resident dirty C, never a stale host copy."""
    m, n, k = 40, 30, 20
    a_h, b_h = ints(m, k, 3), ints(k, n, 4)
    with session(sim) as s:
        a, b = put(s, a_h), put(s, b_h)
        c = put(s, np.ones((m, n), np.float32))
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m),
                           beta=1.0)
        for _ in range(3):
            run(plan)
        assert s.telemetry().bytes_d2h == 0
        np.testing.assert_array_equal(get(c, m, n), 1 + 3 * (a_h @ b_h))
        plan.release()


def test_next_gemm_reads_dirty_output_through_another_rectangle(sim):
    """C1 = A B stays dirty; the next GEMM reads C1 transposed, i.e. through
    panels of another shape: each fill first writes the overlapping dirty C1
    tiles back (they stay cached, clean)."""
    m, n, k = 70, 90, 50
    a_h, b_h, d_h = ints(m, k, 5), ints(k, n, 6), ints(m, 30, 7)
    with session(sim, frames=12) as s:
        a, b, c1 = put(s, a_h), put(s, b_h), s.allocation(m * n * 4)
        d, c2 = put(s, d_h), s.allocation(n * 30 * 4)
        p1 = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c1, m, n, m))
        # C2 (n x 30) = C1^T D: C1 stored m x n column-major, used with op T,
        # in 32-deep K panels (C1's tiles are 64 x 64: other rectangles).
        p2 = xv.GemmPlan(s, xv.matrix(c1, m, n, m), xv.matrix(d, m, 30, m),
                         xv.matrix(c2, n, 30, n), op_a=abi.OP_T, tile_hints=(0, 0, 32))
        run(p1)
        t0 = s.telemetry()
        info = run(p2)
        t1 = s.telemetry()
        assert t1.writebacks_completed > t0.writebacks_completed  # flushed C1 tiles
        assert info.bytes_d2h == t1.bytes_d2h - t0.bytes_d2h
        ref1 = a_h @ b_h
        np.testing.assert_array_equal(get(c2, n, 30), ref1.T @ d_h)
        np.testing.assert_array_equal(get(c1, m, n), ref1)
        p1.release()
        p2.release()


def test_chain_hits_the_previous_output(sim):
    """act[l+1] = W act[l]: the next layer's B panels are the previous layer's
    C tiles (same rectangles, same packing), found in the cache; nothing of
    the intermediate activations crosses the link."""
    m, n, layers = 64, 24, 4
    with session(sim, frames=24) as s:
        x = ints(m, n, 8)
        ws = [ints(m, m, 9 + l, -1, 2) for l in range(layers)]
        acts = [put(s, x)] + [s.allocation(m * n * 4) for _ in range(layers)]
        w_allocs = [put(s, w) for w in ws]
        plans = [xv.GemmPlan(s, xv.matrix(w_allocs[l], m, m, m), xv.matrix(acts[l], m, n, m),
                             xv.matrix(acts[l + 1], m, n, m)) for l in range(layers)]
        t0 = s.telemetry()
        for p in plans:
            run(p)
        t1 = s.telemetry()
        assert t1.bytes_d2h == t0.bytes_d2h
        assert t1.bytes_h2d - t0.bytes_h2d == (layers * m * m + m * n) * 4
        ref = x
        for l in range(layers):
            ref = ws[l] @ ref
            np.testing.assert_array_equal(get(acts[l + 1], m, n), ref)
        for p in plans:
            p.release()


def dev(addr, n):
    return np.ctypeslib.as_array((ctypes.c_float * n).from_address(addr))


def test_transaction_output_feeds_a_gemm(sim):
    """A transaction writes A (its chunks stay dirty); the GEMM's A panel
    overlaps them: written back first, then filled."""
    m, n, k = 32, 16, 64
    a_h, b_h = ints(m, k, 10), ints(k, n, 11)
    with session(sim, frame=4 * KiB, frames=24) as s:
        a = s.allocation(m * k * 4)
        b, c = put(s, b_h), s.allocation(m * n * 4)
        src = np.asfortranarray(a_h).T.copy().reshape(-1)

        def fill(view):
            for _, off, ln, addr, _mode in view.ranges:
                dev(addr, ln // 4)[:] = src[off // 4:(off + ln) // 4]

        s.execute_transaction([xv.access(a, 0, m * k * 4, WO)], fill)
        assert s.telemetry().bytes_d2h == 0  # the chunks stay dirty
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
        run(plan)
        assert s.telemetry().bytes_d2h == m * k * 4  # flushed before the A panel fill
        np.testing.assert_array_equal(get(c, m, n), a_h @ b_h)
        plan.release()


def test_gemm_output_feeds_a_transaction(sim):
    m, n, k = 32, 32, 16
    a_h, b_h = ints(m, k, 12), ints(k, n, 13)
    with session(sim, frame=4 * KiB, frames=24) as s:
        a, b, c = put(s, a_h), put(s, b_h), s.allocation(m * n * 4)
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
        run(plan)
        seen = []

        def look(view):
            for _, off, ln, addr, _mode in view.ranges:
                seen.append((off, dev(addr, ln // 4).copy()))
                dev(addr, ln // 4)[:] += 1  # and modify it in place

        s.execute_transaction([xv.access(c, 0, m * n * 4, RW)], look)
        ref = a_h @ b_h
        flat = np.asfortranarray(ref).T.reshape(-1)
        got = np.concatenate([v for _, v in sorted(seen, key=lambda t: t[0])])
        np.testing.assert_array_equal(got, flat)
        np.testing.assert_array_equal(get(c, m, n), ref + 1)
        plan.release()


def test_partial_host_write_over_dirty_output(sim):
    m, n, k = 40, 40, 8
    a_h, b_h = ints(m, k, 14), ints(k, n, 15)
    with session(sim) as s:
        a, b, c = put(s, a_h), put(s, b_h), s.allocation(m * n * 4)
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
        run(plan)
        # Overwrite columns 10..12 of C from the host while C is cached dirty.
        patch = np.full(3 * m, 7.0, np.float32)
        c.write(patch, offset=10 * m * 4)
        ref = a_h @ b_h
        ref[:, 10:13] = 7.0
        np.testing.assert_array_equal(get(c, m, n), ref)
        plan.release()


def test_drain_and_close_write_back(sim):
    m, n, k = 48, 48, 16
    a_h, b_h = ints(m, k, 16), ints(k, n, 17)
    s = session(sim)
    try:
        a, b, c = put(s, a_h), put(s, b_h), s.allocation(m * n * 4)
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
        run(plan)
        assert s.telemetry().writebacks_completed == 0
        s.drain()
        t = s.telemetry()
        assert t.writebacks_completed == 1 and t.bytes_d2h == m * n * 4
        np.testing.assert_array_equal(get(c, m, n), a_h @ b_h)
        assert s.telemetry().bytes_d2h == m * n * 4  # nothing left to flush
        run(plan)
        s.close()  # writes the dirty C back before tearing down
        t = s.telemetry()
        assert t.writebacks_completed == 2 and t.bytes_d2h == 2 * m * n * 4
        assert t.resident_bytes == 0 and t.mappings == t.unmaps
        plan.release()
    finally:
        s.release()


def test_failed_operation_keeps_earlier_outputs(sim):
    """A GEMM that fails part way (its deadline expires between launches)
    discards only what it wrote; an earlier GEMM's output, still cached dirty,
    survives."""
    m1, n1, k1 = 40, 30, 20
    a1, b1 = ints(m1, k1, 18), ints(k1, n1, 19)
    big = 512
    with session(sim, frame=256 * KiB, frames=12) as s:
        A1, B1, C1 = put(s, a1), put(s, b1), s.allocation(m1 * n1 * 4)
        p1 = xv.GemmPlan(s, xv.matrix(A1, m1, k1, m1), xv.matrix(B1, k1, n1, k1),
                         xv.matrix(C1, m1, n1, m1))
        run(p1)
        A2, B2 = put(s, ints(big, big, 20)), put(s, ints(big, big, 21))
        C2 = s.allocation(big * big * 4)
        # Cycle other panels through the frames first, so a frame mapped for a
        # C2 tile without a load holds stale bytes, not zeros.
        other = s.allocation(big * big * 4)
        p0 = xv.GemmPlan(s, xv.matrix(A2, big, big, big), xv.matrix(B2, big, big, big),
                         xv.matrix(other, big, big, big))
        run(p0)
        p0.release()
        # 256^3 tiles; the second launch is held 1.5 s, so the 500 ms deadline
        # expires between launches, after the first one.
        p2 = xv.GemmPlan(s, xv.matrix(A2, big, big, big), xv.matrix(B2, big, big, big),
                         xv.matrix(C2, big, big, big), deadline_ms=500)
        assert p2.info().tile_count == 8
        slow_second_launch(sim)
        op = p2.submit()
        st, info = op.wait()
        assert st == abi.SUCCESS and info.result == abi.TIMEOUT
        where = op.error().operation.decode()
        op.release()
        if where != "tile_deadline":
            pytest.skip(f"the deadline expired at {where}, before any launch")
        assert 0 < info.units_completed < 8
        np.testing.assert_array_equal(get(C1, m1, n1), a1 @ b1)
        # Neither C2 tiles the failed GEMM wrote nor those it had mapped ahead
        # for writing (never written) survive: C2 is its host copy (zeros), so
        # an accumulating GEMM over it yields exactly A2 B2.
        p3 = xv.GemmPlan(s, xv.matrix(A2, big, big, big), xv.matrix(B2, big, big, big),
                         xv.matrix(C2, big, big, big), beta=1.0)
        run(p3)
        a2, b2 = ints(big, big, 20), ints(big, big, 21)
        np.testing.assert_array_equal(get(C2, big, big), a2 @ b2)
        p1.release()
        p2.release()
        p3.release()


def slow_second_launch(sim):
    """The host simulation's next-but-one kernel launch sleeps 1.5 s first."""
    fn = sim.dll.xvram_hostsim_delay
    fn.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int]
    fn.restype = ctypes.c_int
    assert fn(SITE_LAUNCH, 1, 1500) == 0


def failing_repeat(s, A, B, C, big):
    """Runs the same product again under a 500 ms deadline with its second
    launch held 1.5 s; returns the failed operation's info (or skips when the
    deadline expired before any launch: a host too loaded to reach the first
    launch in 500 ms)."""
    p = xv.GemmPlan(s, xv.matrix(A, big, big, big), xv.matrix(B, big, big, big),
                    xv.matrix(C, big, big, big), deadline_ms=500)
    slow_second_launch(s.lib)
    op = p.submit()
    st, info = op.wait()
    assert st == abi.SUCCESS and info.result == abi.TIMEOUT
    where = op.error().operation.decode()
    op.release()
    p.release()
    if where != "tile_deadline":
        pytest.skip(f"the deadline expired at {where}, before any launch")
    assert 0 < info.units_completed < 8
    return info


@pytest.mark.parametrize("drained", [False, True], ids=["unwritten", "written_back"])
def test_failed_repeat_of_a_gemm(sim, drained):
    """The same GEMM run twice, the second run failing part way: C tiles the
    failed run rewrote while they still held the first run's unwritten results
    (the resident pattern: C stays cached and dirty) hold neither result.
    Those bytes are reported lost: reading them, or a GEMM reading them,
    fails with CORRUPTION until the caller writes them again. When the first
    results had been written back (drain) before, nothing is lost: C reads
    back as the first run's result."""
    big = 512
    a_h, b_h = ints(big, big, 26), ints(big, big, 27)
    # 24 frames: the four 256 x 256 C tiles form one block and all stay
    # cached, dirty, after the first run (fewer frames, and the second run
    # writes them back before it starts, as its schedule needs the frames).
    with session(sim, frame=256 * KiB, frames=24) as s:
        A, B, C = put(s, a_h), put(s, b_h), s.allocation(big * big * 4)
        p1 = xv.GemmPlan(s, xv.matrix(A, big, big, big), xv.matrix(B, big, big, big),
                         xv.matrix(C, big, big, big))
        run(p1)
        if drained:
            s.drain()
        failing_repeat(s, A, B, C, big)
        if drained:
            np.testing.assert_array_equal(get(C, big, big), a_h @ b_h)
            p1.release()
            return
        with pytest.raises(xv.XvramError) as e:
            C.read()
        assert e.value.status == abi.CORRUPTION
        # A GEMM that reads C (beta = 1) cannot load the lost bytes either.
        p3 = xv.GemmPlan(s, xv.matrix(A, big, big, big), xv.matrix(B, big, big, big),
                         xv.matrix(C, big, big, big), beta=1.0)
        op = p3.submit()
        st, info = op.wait()
        assert info.result == abi.CORRUPTION
        op.release()
        # Rewriting C makes it whole; the same GEMM then runs as before.
        C.write(np.zeros(big * big, np.float32))
        np.testing.assert_array_equal(get(C, big, big), np.zeros((big, big), np.float32))
        run(p3)
        np.testing.assert_array_equal(get(C, big, big), a_h @ b_h)
        assert s.telemetry().poisoned == 0
        p1.release()
        p3.release()


def test_background_flush_bounds_idle_dirty_frames(sim):
    """Outputs of earlier operations may not crowd the pool: once more than
    half of it is idle and dirty, the least recently used half of those are
    written back and stay cached, clean."""
    frames = 16
    m = n = k = 32  # one 4 KiB tile per C
    with session(sim, frame=4 * KiB, frames=frames) as s:
        a_h, b_h = ints(m, k, 22), ints(k, n, 23)
        a, b = put(s, a_h), put(s, b_h)
        outs = []
        for i in range(12):
            c = s.allocation(m * n * 4)
            plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k),
                               xv.matrix(c, m, n, m), alpha=float(i + 1))
            run(plan)
            plan.release()
            outs.append(c)
        t = s.telemetry()
        # 12 C tiles were written; at most half the pool (8) can stay dirty
        # before the flush, so some were written back without being evicted.
        assert t.writebacks_completed > 0
        assert t.writebacks_completed > t.dirty_evictions
        ref = a_h @ b_h
        for i, c in enumerate(outs):
            np.testing.assert_array_equal(get(c, m, n), (i + 1) * ref)


def test_queued_reads_and_gemms_from_threads(sim):
    """Reads of C queued behind GEMMs on the same session see each result."""
    m = n = k = 24
    with session(sim) as s:
        a_h, b_h = ints(m, k, 24), ints(k, n, 25)
        a, b, c = put(s, a_h), put(s, b_h), s.allocation(m * n * 4)
        plans = [xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k),
                             xv.matrix(c, m, n, m), alpha=float(i + 1)) for i in range(4)]
        got = []
        for i, p in enumerate(plans):
            op = p.submit()
            out = get(c, m, n)  # queued after the GEMM on the worker
            got.append(out)
            st, info = op.wait()
            assert info.result == abi.SUCCESS
            op.release()
        ref = a_h @ b_h
        for i, out in enumerate(got):
            np.testing.assert_array_equal(out, (i + 1) * ref)
        for p in plans:
            p.release()
