"""Victim policies and the live device budget.

Policies (CLOCK, the default, and LRU) are driven through a command program
exported by the hostsim library: pinned by the reference's own known answers
(tests/unit/residency_core_tests.cpp:200-250) and, where the reference tree is
mounted, by random programs run side by side against the reference's compiled
policy.cpp (oracle/_ref), whose answers tests/golden/reference_outputs.json
also records for checkouts without the reference tree. The live budget (shrink at once, grow by two frames
after ten samples, one retry after an out-of-memory frame allocation;
reference runtime.cpp:3184-3468) is exercised through hostsim sessions whose
device memory the test changes underneath them."""
import ctypes
import time

import numpy as np
import pytest

import generators
import xvram_amd as xv
from generators import CLEAN, DIRTY, DROP, ERASE, INSERT, NONE, SELECT, SET, TOUCH
from xvram_amd import abi

from gemm_cases import Problem, pattern_operands, uniform

KiB = 1 << 10


@pytest.fixture(scope="module")
def run():
    lib = xv.load(hostsim=True).dll
    generators.declare_policy(lib.xvram_hostsim_policy_run)
    return lambda kind, cmds: generators.run_policy(lib.xvram_hostsim_policy_run, kind, cmds)


def test_clock_kats(run):
    """residency_core_tests.cpp:207-224."""
    out = run(0, [(INSERT, 1, 1, 0, 0), (INSERT, 2, 2, 1, 0), (INSERT, 3, 3, 0, 1),
                  (SET, 1, CLEAN), (SET, 2, CLEAN), (SET, 3, DIRTY),
                  (SELECT,),                       # speculative clean (cost 1) goes first
                  (SET, 2, CLEAN, 0, 1),           # pin it
                  (SELECT,),                       # then the ordinary clean entry
                  (SET, 1, CLEAN, 0, 0, 0, 1),     # in the working set
                  (SELECT,),                       # then the dirty one-touch entry
                  (SET, 3, DIRTY, 0, 0, 1),        # in flight
                  (SELECT,),                       # nothing left
                  (ERASE, 2), (ERASE, 2)])
    assert out[6] == 2 and out[8] == 1 and out[10] == 3 and out[12] == NONE
    assert out[13:] == [1, 0]


def test_lru_kats(run):
    """residency_core_tests.cpp:226-236."""
    out = run(1, [(INSERT, 2, 10), (INSERT, 1, 10), (INSERT, 3, 20),
                  (SET, 1, CLEAN), (SET, 2, DIRTY), (SET, 3, CLEAN),
                  (SELECT,), (TOUCH, 1, 30), (SELECT,), (SET, 2, DIRTY, 0, 1), (SELECT,)])
    assert (out[6], out[8], out[10]) == (1, 2, 3)


@pytest.mark.parametrize("kind", [0, 1], ids=["clock", "lru"])
def test_hot_entries_go_last(run, kind):
    """residency_core_tests.cpp:238-249."""
    out = run(kind, [(INSERT, 1, 1), (INSERT, 2, 2), (SET, 1, CLEAN, 1), (SET, 2, CLEAN), (SELECT,)])
    assert out[4] == 2


def selections(programs, outputs):
    return sum(1 for cmds, out in zip(programs, outputs)
               for c, v in zip(cmds, out) if c[0] == SELECT and v != NONE)


@pytest.mark.parametrize("kind", [0, 1], ids=["clock", "lru"])
def test_policies_match_recorded_reference(run, kind):
    programs = generators.policy_programs(kind, 150)
    want = generators.reference_outputs(("policy_clock", "policy_lru")[kind], programs)
    for cmds, theirs in zip(programs, want):
        mine = [-1 if v == NONE else v for v in run(kind, cmds)]
        assert mine == theirs, cmds
    assert selections(programs, want) > 250


@pytest.mark.parametrize("kind", [0, 1], ids=["clock", "lru"])
def test_policies_match_reference(run, oracle_mod, kind):
    ref = oracle_mod.ref_lib()
    if ref is None:
        pytest.skip("reference tree not built into oracle/_ref")
    generators.declare_policy(ref.ref_policy_run)
    programs = generators.policy_programs(kind, 300)
    outputs = []
    for cmds in programs:
        mine = run(kind, cmds)
        theirs = generators.run_policy(ref.ref_policy_run, kind, cmds)
        assert mine == theirs, cmds
        outputs.append(mine)
    assert selections(programs, outputs) > 500


# ---- live budget ------------------------------------------------------------------------

@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_set_memory.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    lib.dll.xvram_hostsim_inject.argtypes = [ctypes.c_int, ctypes.c_long, ctypes.c_int]
    yield lib
    lib.dll.xvram_hostsim_reset()


F = 16 * KiB


def budget_session(lib, policy=abi.CACHE_POLICY_CLOCK, headroom=0, poll_ms=1):
    return xv.Session(lib, chunk_size_bytes=F, cache_target_bytes=0, workspace_cap_bytes=0,
                      device_headroom_bytes=headroom, budget_poll_ms=poll_ms, cache_policy=policy)


def touch_all(s, alloc, size, mode=abi.ACCESS_READ_WRITE, value=None):
    def cb(view):
        if value is not None:
            for _, off, ln, addr, _ in view.ranges:
                np.ctypeslib.as_array((ctypes.c_uint8 * ln).from_address(addr))[:] = value
    s.execute_transaction([xv.access(alloc, 0, size, mode)], cb)


def test_shrink_writes_back_and_releases(sim):
    sim.dll.xvram_hostsim_set_memory(16 * F, 16 * F)
    s = budget_session(sim)
    try:
        t = s.telemetry()
        assert t.cache_target_bytes == 16 * F
        a = s.allocation(10 * F)
        touch_all(s, a, 10 * F, value=7)            # 10 frames created
        b = s.allocation(2 * F)
        data = np.arange(2 * F, dtype=np.uint8)
        b.write(data)
        sim.dll.xvram_hostsim_set_memory(1 * F, 16 * F)  # someone took memory: 1 free + 10 ours
        time.sleep(0.005)
        touch_all(s, b, 2 * F, mode=abi.ACCESS_READ)
        t = s.telemetry()
        assert t.budget_shrinks == 1
        assert t.cache_target_bytes == 11 * F and t.cache_target_minimum_bytes == 11 * F
        assert t.resident_bytes_peak <= 16 * F
        assert np.array_equal(a.read(), np.full(10 * F, 7, np.uint8))
        assert np.array_equal(b.read(), data)
        s.close()
        t = s.telemetry()
        assert t.physical_handles_created == t.physical_handles_released
        assert t.mappings == t.unmaps and t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    finally:
        s.release()


def test_grow_needs_ten_samples_and_two_frames(sim):
    sim.dll.xvram_hostsim_set_memory(16 * F, 16 * F)
    with budget_session(sim) as s:
        a = s.allocation(F)
        sim.dll.xvram_hostsim_set_memory(4 * F, 16 * F)
        time.sleep(0.005)
        touch_all(s, a, F)
        assert s.telemetry().budget_shrinks == 1
        shrunk = s.telemetry().cache_target_bytes
        sim.dll.xvram_hostsim_set_memory(16 * F, 16 * F)
        grows = []
        for _ in range(25):
            time.sleep(0.003)
            touch_all(s, a, F)
            grows.append(s.telemetry().budget_grows)
        assert grows[8] == 0            # fewer than ten samples: no growth yet
        assert grows[-1] >= 2
        t = s.telemetry()
        assert t.cache_target_bytes == shrunk + 2 * grows[-1] * F
        assert t.cache_target_maximum_bytes == 16 * F  # never above the setup target


def test_out_of_memory_frame_allocation_retries_once(sim):
    sim.dll.xvram_hostsim_set_memory(16 * F, 16 * F)
    # A 1 s poll interval keeps the target stale through the transaction below
    # however slowly the host runs (with 1 ms a delay could resample first).
    with budget_session(sim, poll_ms=1000) as s:
        a = s.allocation(3 * F)
        sim.dll.xvram_hostsim_set_memory(2 * F, 16 * F)  # only two frames can still be created
        # Within the poll interval the target is stale; the third frame's
        # creation runs out of memory, the forced resample shrinks the pool.
        with pytest.raises(xv.XvramError) as e:
            touch_all(s, a, 3 * F)
        assert e.value.status == abi.BUDGET_PRESSURE
        t = s.telemetry()
        assert t.target_oom_retries >= 1 and t.budget_shrinks >= 1
        assert t.poisoned == 0
        touch_all(s, a, 2 * F)  # a working set that fits still runs


def test_gemm_under_a_shrinking_budget(sim, oracle_mod):
    """A GEMM keeps its results correct when the pool shrinks between operations:
    once other users leave less than the headroom free, the pool gives frames
    back until the headroom is free again."""
    sim.dll.xvram_hostsim_set_memory(24 * F, 24 * F)
    m, n, k = 96, 80, 120
    prob = Problem(uniform(oracle_mod, m, k, 61), uniform(oracle_mod, k, n, 62))
    with budget_session(sim, headroom=4 * F) as s:
        a_flat = np.asfortranarray(prob.a_op).T.reshape(-1)
        b_flat = np.asfortranarray(prob.b_op).T.reshape(-1)
        A, B, C = s.allocation(a_flat.nbytes), s.allocation(b_flat.nbytes), s.allocation(m * n * 4)
        A.write(a_flat)
        B.write(b_flat)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k), xv.matrix(C, m, n, m),
                           tile_hints=(32, 32, 32))
        plan.execute()
        first = C.read(dtype=np.float32)
        assert s.telemetry().physical_handles_created == 20
        sim.dll.xvram_hostsim_set_memory(0, 24 * F)   # the 4 free frames were taken
        time.sleep(0.005)
        plan.execute()
        second = C.read(dtype=np.float32)
        plan.release()
        t = s.telemetry()
        assert t.budget_shrinks == 1 and t.cache_target_bytes == 16 * F
        assert t.physical_handles_released == 4
    assert np.array_equal(first, second)
    ref, absab = prob.reference(oracle_mod)
    assert oracle_mod.check_bound(np.asfortranarray(second.reshape(n, m).T), k, ref, absab)[0] == 0


@pytest.mark.parametrize("policy", [abi.CACHE_POLICY_CLOCK, abi.CACHE_POLICY_LRU], ids=["clock", "lru"])
def test_both_policies_give_identical_results_out_of_core(sim, oracle_mod, policy):
    m, n, k = 150, 120, 200
    prob = Problem(uniform(oracle_mod, m, k, 71), uniform(oracle_mod, k, n, 72))
    with xv.Session(sim, chunk_size_bytes=16 * KiB, cache_target_bytes=8 * 16 * KiB,
                    workspace_cap_bytes=0, device_headroom_bytes=0, cache_policy=policy) as s:
        out = prob.run(s, repeat=2)
        t = s.telemetry()
        assert t.clean_evictions > 0 and t.unsafe_transitions == 0
    ref, absab = prob.reference(oracle_mod)
    assert oracle_mod.check_bound(out, k, ref, absab)[0] == 0


def test_out_of_memory_in_a_gemm_then_recovery(sim, oracle_mod):
    """The GPU scenario of tests/test_gpu_budget.py on the host simulation:
    memory runs out while a GEMM creates its frames, the forced resample
    cannot shrink under the frames the GEMM holds (BUDGET_PRESSURE, no
    poison); once memory is back the same session computes the product
    exactly, and the frame whose creation failed is reused through legal
    state transitions only."""
    sim.dll.xvram_hostsim_set_memory(64 * F, 64 * F)
    s = xv.Session(sim, chunk_size_bytes=F, cache_target_bytes=16 * F, workspace_cap_bytes=0,
                   device_headroom_bytes=2 * F, budget_poll_ms=10 ** 9)
    try:
        m = n = k = 256
        a_op, b_op = pattern_operands(m, n, k)
        a, b, c = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        a.write(np.asfortranarray(a_op).T.copy())
        b.write(np.asfortranarray(b_op).T.copy())

        def plan():
            return xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k),
                               xv.matrix(c, m, n, m))

        p = plan()
        assert p.info().tile_count > 8
        sim.dll.xvram_hostsim_set_memory(5 * F, 64 * F)  # room for five frames
        with pytest.raises(xv.XvramError) as e:
            p.execute()
        assert e.value.status == abi.BUDGET_PRESSURE
        t = s.telemetry()
        assert t.target_oom_retries == 1 and t.budget_shrinks == 0 and t.poisoned == 0
        assert t.physical_handles_created == 5
        p.release()
        sim.dll.xvram_hostsim_set_memory(59 * F, 64 * F)  # the memory is back
        p = plan()
        p.execute()
        out = np.asfortranarray(c.read(dtype=np.float32).reshape(n, m).T)
        assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))
        p.release()
        s.close()
        t = s.telemetry()
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        assert t.physical_handles_created == t.physical_handles_released
    finally:
        s.release()
