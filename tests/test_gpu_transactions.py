"""GPU tests of working-set transactions and prefetch through the C ABI on the
MI355X: the callback enqueues real device work (HIP memset / device-to-device
copies) on the session's compute stream against the resolved stable
addresses, including copies that cross frame boundaries inside one
allocation's VA range. Results are checked bit-exactly against a host model
of the same byte operations."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import uniform

pytestmark = pytest.mark.gpu

MiB = 1 << 20
R, RW, WO = abi.ACCESS_READ, abi.ACCESS_READ_WRITE, abi.ACCESS_WRITE_ONLY
HIP_D2D = 3


@pytest.fixture(scope="module")
def hip():
    h = ctypes.CDLL("libamdhip64.so")
    h.hipMemsetD8Async.argtypes = [ctypes.c_uint64, ctypes.c_ubyte, ctypes.c_size_t, ctypes.c_void_p]
    h.hipMemsetD8Async.restype = ctypes.c_int
    h.hipMemcpyAsync.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int,
                                 ctypes.c_void_p]
    h.hipMemcpyAsync.restype = ctypes.c_int
    return h


@pytest.fixture(scope="module")
def lib():
    return xv.load()


def rand_bytes(n, seed):
    return np.random.default_rng(seed).integers(0, 256, n, dtype=np.uint8)


def small_budget(lib, frames, chunk=2 * MiB, workspace=0):
    return xv.Session(lib, chunk_size_bytes=chunk, cache_target_bytes=frames * chunk + workspace,
                      workspace_cap_bytes=workspace)


def close_balanced(s):
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps == t.set_access_calls
    assert t.physical_handles_created == t.physical_handles_released
    assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    s.release()


def test_device_copies_across_frames(lib, hip):
    s = small_budget(lib, frames=8)
    try:
        F = s.config.chunk_size_bytes
        size = 5 * F + 12345
        a = s.allocation(size)
        model = rand_bytes(size, 21)
        a.write(model)
        src, dst, ln = F // 2 + 7, 3 * F - 999, F + 4096  # both spans cross frame boundaries

        def cb(view):
            (_, off, length, addr, mode), = view.ranges
            base = addr - off
            assert hip.hipMemcpyAsync(base + dst, base + src, ln, HIP_D2D, view.stream) == 0
            assert hip.hipMemsetD8Async(base + 4 * F + 100, 0xA5, 5000, view.stream) == 0

        s.execute_transaction([xv.access(a, 0, size, RW)], cb)
        model[dst:dst + ln] = model[src:src + ln].copy()
        model[4 * F + 100:4 * F + 5100] = 0xA5
        assert np.array_equal(a.read(), model)
        t = s.telemetry()
        assert t.writebacks_completed >= 6 and t.transactions_completed >= 1
    finally:
        close_balanced(s)


def test_out_of_core_sliding_windows(lib, hip):
    """16 chunks through 4 frames; each step copies one chunk-sized window onto
    the next and marks it, so every step depends on the previous write-back."""
    s = small_budget(lib, frames=4)
    try:
        F = s.config.chunk_size_bytes
        n = 16
        a = s.allocation(n * F)
        model = rand_bytes(n * F, 22)
        a.write(model)
        for step in range(n - 1):
            lo = step * F

            def cb(view, lo=lo, step=step):
                (_, off, length, addr, mode), = view.ranges
                base = addr - off
                assert hip.hipMemcpyAsync(base + lo + F, base + lo, F, HIP_D2D, view.stream) == 0
                assert hip.hipMemsetD8Async(base + lo + F + step, step & 0xFF, 1, view.stream) == 0

            s.execute_transaction([xv.access(a, lo, 2 * F, RW)], cb)
            model[lo + F:lo + 2 * F] = model[lo:lo + F]
            model[lo + F + step] = step & 0xFF
        assert np.array_equal(a.read(), model)
        t = s.telemetry()
        assert t.dirty_evictions > 0 or t.writebacks_completed >= n - 1
    finally:
        close_balanced(s)


def test_write_only_and_workspace(lib, hip):
    s = small_budget(lib, frames=6, workspace=2 * MiB)
    try:
        F = s.config.chunk_size_bytes
        a = s.allocation(3 * F)
        model = rand_bytes(3 * F, 23)
        a.write(model)
        t0 = s.telemetry()

        def cb(view):
            assert view.workspace_address != 0 and view.workspace_bytes == MiB
            (_, off, length, addr, mode), = view.ranges
            assert mode == WO
            assert hip.hipMemsetD8Async(view.workspace_address, 0x3C, MiB, view.stream) == 0
            assert hip.hipMemcpyAsync(addr, view.workspace_address, MiB, HIP_D2D, view.stream) == 0
            assert hip.hipMemcpyAsync(addr + MiB, view.workspace_address, F - MiB, HIP_D2D,
                                      view.stream) == 0

        s.execute_transaction([xv.access(a, F, F, WO)], cb, workspace_bytes=MiB)
        t1 = s.telemetry()
        assert t1.bytes_h2d == t0.bytes_h2d  # a full write-only chunk is never loaded
        model[F:2 * F] = 0x3C
        assert np.array_equal(a.read(), model)
    finally:
        close_balanced(s)


def test_prefetch_and_gemm_coherence(lib, hip, oracle_mod):
    m = n = k = 512
    a_np = uniform(oracle_mod, m, k, 31)
    b_np = uniform(oracle_mod, k, n, 32)
    s = small_budget(lib, frames=12)
    try:
        A, B, C, D = (s.allocation(m * n * 4) for _ in range(4))
        A.write(np.asfortranarray(a_np).T.reshape(-1))
        B.write(np.asfortranarray(b_np).T.reshape(-1))
        C.write(np.zeros(m * n, np.float32))
        op = s.prefetch([xv.access(C, 0, m * n * 4, R)])
        st, info = op.wait()
        op.release()
        assert st == abi.SUCCESS and info.result == abi.SUCCESS
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k), xv.matrix(C, m, n, m))
        plan.execute()

        def copy_c(view):
            by_alloc = {r[0]: r for r in view.ranges}
            c_r = by_alloc[C.info().allocation_id]
            d_r = by_alloc[D.info().allocation_id]
            assert hip.hipMemcpyAsync(d_r[3], c_r[3], m * n * 4, HIP_D2D, view.stream) == 0

        # The prefetched C chunk is stale after the GEMM; the copy must see the result.
        s.execute_transaction([xv.access(C, 0, m * n * 4, R), xv.access(D, 0, m * n * 4, WO)],
                              copy_c)
        c_host = C.read(dtype=np.float32)
        assert np.array_equal(D.read(dtype=np.float32), c_host)
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a_np), np.asfortranarray(b_np),
                                          1.0, 0.0, None)
        bad, _, _ = oracle_mod.check_bound(c_host.reshape(n, m).T, k, ref, absab)
        assert bad == 0

        # Zero A on the device through a write-only transaction.
        def zero_a(view):
            (_, off, length, addr, mode), = view.ranges
            assert hip.hipMemsetD8Async(addr, 0, length, view.stream) == 0

        s.execute_transaction([xv.access(A, 0, m * k * 4, WO)], zero_a)
        plan.execute()  # cached A panels must have been dropped: C becomes 0
        assert not np.any(C.read(dtype=np.float32))
        plan.release()
    finally:
        close_balanced(s)
