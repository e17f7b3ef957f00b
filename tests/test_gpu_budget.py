"""Live budget control on the MI355X's real VMM (reference
src/residency/runtime.cpp:3184-3211 create_handle's one OOM retry,
:3213-3468 refresh_budget's immediate shrink and hysteretic grow), and the LRU
policy out of core.

Device memory is taken from the session between operations with a plain
hipMalloc in the test process, the way another tenant of the GPU would take
it; every result is the analytic pattern, compared bit for bit."""
import ctypes
import time

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_configs import FP, closed, fill_pattern, synth  # noqa: F401 (fixture)

pytestmark = pytest.mark.gpu

MiB, GiB = 1 << 20, 1 << 30


def log(msg):
    print(f"[budget] {msg}", flush=True)


@pytest.fixture(scope="module")
def hip():
    h = ctypes.CDLL("libamdhip64.so")
    h.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    h.hipFree.argtypes = [ctypes.c_void_p]
    h.hipMemGetInfo.argtypes = [ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)]
    assert h.hipSetDevice(0) == 0
    return h


def free_bytes(hip):
    f, t = ctypes.c_size_t(), ctypes.c_size_t()
    assert hip.hipMemGetInfo(ctypes.byref(f), ctypes.byref(t)) == 0
    return f.value


class Taken:
    """Device memory held by the test process, in pieces of at most 16 GiB."""

    def __init__(self, hip, nbytes):
        self.hip, self.ptrs = hip, []
        left = nbytes
        while left > 0:
            piece = min(left, 16 * GiB)
            p = ctypes.c_void_p()
            assert hip.hipMalloc(ctypes.byref(p), piece) == 0, "hipMalloc failed"
            self.ptrs.append(p)
            left -= piece

    def release(self):
        for p in self.ptrs:
            assert self.hip.hipFree(p) == 0
        self.ptrs = []


def pattern_gemm(s, synth, size):
    """C = A B^T on the analytic pattern (exact in FP32 while 28 K < 2^24)."""
    m = n = k = size
    a, b, c = s.allocation(m * k * 4), s.allocation(n * k * 4), s.allocation(m * n * 4)
    fill_pattern(a, synth.synth_fill_pattern_a, m, k, 0)
    fill_pattern(b, synth.synth_fill_pattern_b, n, k, 1)
    return a, b, c


def make_plan(s, a, b, c, size):
    m = n = k = size
    return xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, n, k, n), xv.matrix(c, m, n, m),
                       abi.OP_N, abi.OP_T)


def run(plan):
    op = plan.submit()
    st, info = op.wait()
    assert st == abi.SUCCESS
    e = op.error()
    result = info.result
    message = (f"{e.stage.decode()}/{e.operation.decode()} "
               f"{e.native_name.decode()}:{e.native_code} {e.message.decode()}")
    op.release()
    return result, message


def exact(c, size, oracle_mod):
    got = c.read(dtype=np.float32).reshape(size, size).T
    expect = oracle_mod.pattern_expected_matrix(size, size, size).astype(np.float32)
    return int(np.count_nonzero(got != expect))


def test_pool_shrinks_and_grows_with_device_memory(lib_product, hip, synth, oracle_mod):
    size, frame, cap = 24576, 256 * MiB, 6 * GiB
    free0 = free_bytes(hip)
    # A headroom that leaves exactly cap + 768 MiB for the session at setup:
    # taking 2 GiB later must bring the safe target below the pool.
    headroom = free0 - (cap + 768 * MiB)
    s = xv.Session(lib_product, chunk_size_bytes=frame, cache_target_bytes=cap,
                   device_headroom_bytes=headroom, budget_poll_ms=1)
    taken = None
    try:
        frames0 = s.telemetry().cache_target_bytes // frame
        a, b, c = pattern_gemm(s, synth, size)
        plan = make_plan(s, a, b, c, size)
        assert run(plan)[0] == abi.SUCCESS
        assert exact(c, size, oracle_mod) == 0
        t1 = s.telemetry()
        log(f"before: target {t1.cache_target_bytes / GiB:.2f} GiB ({frames0} frames), "
            f"handles {t1.physical_handles_created}")
        taken = Taken(hip, 2 * GiB)
        result, message = run(plan)
        t2 = s.telemetry()
        log(f"after taking 2 GiB: result {result} ({message}), target "
            f"{t2.cache_target_bytes / GiB:.2f} GiB, shrinks {t2.budget_shrinks}, handles "
            f"created {t2.physical_handles_created} released {t2.physical_handles_released}")
        assert result == abi.SUCCESS, message
        assert t2.budget_shrinks > t1.budget_shrinks
        assert t2.cache_target_bytes < t1.cache_target_bytes
        assert t2.physical_handles_released > t1.physical_handles_released
        assert t2.resident_bytes_peak <= cap
        assert exact(c, size, oracle_mod) == 0
        taken.release()
        taken = None
        grows = t2.budget_grows
        for _ in range(6):
            assert run(plan)[0] == abi.SUCCESS
            if s.telemetry().budget_grows > grows:
                break
        t3 = s.telemetry()
        log(f"after freeing: target {t3.cache_target_bytes / GiB:.2f} GiB, grows "
            f"{t3.budget_grows}")
        assert t3.budget_grows > grows
        assert t3.cache_target_bytes > t2.cache_target_bytes
        assert exact(c, size, oracle_mod) == 0
        assert t3.unsafe_remaps == 0 and t3.unsafe_transitions == 0
        plan.release()
    finally:
        if taken is not None:
            taken.release()
        closed(s)


def test_out_of_memory_retry_then_recovery(lib_product, hip, synth, oracle_mod):
    """Another tenant takes almost all device memory before the session has
    created its frames: creating one fails, the session resamples the budget
    once (target_oom_retries), cannot shrink under its own working set and
    reports BUDGET_PRESSURE without poisoning itself; once the memory is back,
    the same session computes the product exactly."""
    size, frame = 16384, 256 * MiB
    s = xv.Session(lib_product, chunk_size_bytes=frame, cache_target_bytes=4 * GiB,
                   budget_poll_ms=1_000_000_000)  # no periodic samples: only forced ones
    taken = None
    try:
        a, b, c = pattern_gemm(s, synth, size)
        plan = make_plan(s, a, b, c, size)
        assert s.telemetry().physical_handles_created == 0  # frames are created lazily
        taken = Taken(hip, free_bytes(hip) - 1280 * MiB)  # room for about five frames
        log(f"taken {sum(1 for _ in taken.ptrs)} pieces; free now {free_bytes(hip) / MiB:.0f} MiB")
        result, message = run(plan)
        t = s.telemetry()
        log(f"with memory taken: result {result} ({message}), oom retries "
            f"{t.target_oom_retries}, handles {t.physical_handles_created}")
        assert result in (abi.BUDGET_PRESSURE, abi.DEVICE_OUT_OF_MEMORY), message
        assert t.target_oom_retries >= 1
        assert t.poisoned == 0
        taken.release()
        taken = None
        plan.release()
        plan = make_plan(s, a, b, c, size)
        result, message = run(plan)
        assert result == abi.SUCCESS, message
        assert exact(c, size, oracle_mod) == 0
        plan.release()
    finally:
        if taken is not None:
            taken.release()
        closed(s)


def test_lru_policy_out_of_core(lib_product, synth, oracle_mod):
    size = 16384
    s = xv.Session(lib_product, chunk_size_bytes=64 * MiB, cache_target_bytes=GiB,
                   cache_policy=abi.CACHE_POLICY_LRU)
    try:
        a, b, c = pattern_gemm(s, synth, size)
        plan = make_plan(s, a, b, c, size)
        t0 = s.telemetry()
        assert run(plan)[0] == abi.SUCCESS
        t1 = s.telemetry()
        assert t1.bytes_h2d - t0.bytes_h2d > 3 * GiB  # out of core
        assert t1.clean_evictions + t1.dirty_evictions > 0
        assert exact(c, size, oracle_mod) == 0
        log(f"LRU: H2D {(t1.bytes_h2d - t0.bytes_h2d) / GiB:.1f} GiB, evictions "
            f"{t1.clean_evictions}+{t1.dirty_evictions}")
        plan.release()
    finally:
        closed(s)


@pytest.fixture(scope="module")
def lib_product():
    return xv.load()
