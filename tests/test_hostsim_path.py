"""CPU tests of the whole ABI -> session -> planner -> panel cache -> executor path,
run over libxvram_hostsim.so (the same host runtime over a host-memory device
simulation; the tile kernel there is a plain loop). Covers operand forms,
beta semantics, out-of-core scheduling and exact cache accounting."""
import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import Problem, pattern_operands, uniform

KiB = 1 << 10
OPS = [(abi.OP_N, abi.OP_N), (abi.OP_N, abi.OP_T), (abi.OP_T, abi.OP_N), (abi.OP_T, abi.OP_T)]
OP_IDS = ["NN", "NT", "TN", "TT"]


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def small_session(lib, frames=12, frame_kib=64, **extra):
    cfg = dict(chunk_size_bytes=frame_kib * KiB, cache_target_bytes=frames * frame_kib * KiB,
               workspace_cap_bytes=0, device_headroom_bytes=0)
    cfg.update(extra)
    return xv.Session(lib, **cfg)


def check(oracle, prob, out):
    ref, absab = prob.reference(oracle)
    bad, max_err, _ = oracle.check_bound(out, prob.k, ref, absab)
    assert bad == 0, f"{bad} elements outside the bound (max err {max_err})"


@pytest.mark.parametrize("layouts", [(1, 1, 1), (0, 0, 0), (1, 0, 1), (0, 1, 0)],
                         ids=["CCC", "RRR", "CRC", "RCR"])
@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_operand_forms_out_of_core(sim, oracle_mod, ops, layouts):
    m, n, k = 150, 97, 211
    prob = Problem(uniform(oracle_mod, m, k, 1), uniform(oracle_mod, k, n, 2),
                   uniform(oracle_mod, m, n, 3), op_a=ops[0], op_b=ops[1], layouts=layouts,
                   alpha=1.5, beta=0.5, ld_pad=(1, 2, 3))
    with small_session(sim, frames=8, frame_kib=16) as s:
        out = prob.run(s)
        assert prob.plan_info.tile_count > 1
    check(oracle_mod, prob, out)


def test_beta_zero_does_not_read_c(sim, oracle_mod):
    m, n, k = 90, 70, 50
    prob = Problem(uniform(oracle_mod, m, k, 4), uniform(oracle_mod, k, n, 5))
    with small_session(sim) as s:
        out = prob.run(s, c_fill=np.float32(np.nan))
    assert np.isfinite(out).all()
    check(oracle_mod, prob, out)


def test_padding_outside_c_is_untouched(sim, oracle_mod):
    m, n, k = 40, 30, 20
    prob = Problem(uniform(oracle_mod, m, k, 6), uniform(oracle_mod, k, n, 7),
                   ld_pad=(0, 0, 5))
    with small_session(sim) as s:
        prob.run(s, c_fill=np.float32(-7.0))
    flat = prob.c_flat_out.reshape(n, m + 5)
    assert (flat[:, m:] == np.float32(-7.0)).all()


@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_pattern_exact(sim, oracle_mod, ops):
    m, n, k = 130, 110, 300
    a_op, b_op = pattern_operands(m, n, k)
    with small_session(sim, frames=10, frame_kib=16) as s:
        out = Problem(a_op, b_op, op_a=ops[0], op_b=ops[1]).run(s)
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_accounting_invariants_and_teardown(sim, oracle_mod):
    m, n, k = 300, 200, 500
    prob = Problem(uniform(oracle_mod, m, k, 8), uniform(oracle_mod, k, n, 9),
                   uniform(oracle_mod, m, n, 10), alpha=1.5, beta=0.5)
    s = small_session(sim, frames=12)
    out = prob.run(s)
    check(oracle_mod, prob, out)
    t = s.telemetry()
    # C tiles of every block but the last were written back and evicted during
    # the operation; the last block's stayed cached, dirty, until the read of C
    # wrote them back (keeping them cached, clean).
    assert 0 < t.dirty_evictions < t.writebacks_completed
    assert t.clean_evictions > 0 and t.handle_reuses > 0
    assert t.mappings == t.set_access_calls == t.physical_handles_created <= 12
    assert t.resident_bytes_peak <= t.cache_target_bytes
    assert t.bytes_d2h == m * n * 4                       # every C element written back once
    assert t.bytes_h2d >= (m * k + k * n + m * n) * 4     # compulsory traffic (beta != 0)
    assert t.transactions_completed == prob.plan_info.tile_count
    assert t.unsafe_remaps == 0 and t.unsafe_transitions == 0
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps
    assert t.physical_handles_created == t.physical_handles_released
    assert t.resident_bytes == 0
    s.release()


def test_accounting_is_reproducible(sim, oracle_mod):
    """The schedule and frame choices do not depend on device timing: two runs
    give identical counters."""
    counters = []
    for _ in range(2):
        prob = Problem(uniform(oracle_mod, 257, 129, 11), uniform(oracle_mod, 129, 300, 12))
        with small_session(sim, frames=9, frame_kib=16) as s:
            prob.run(s, repeat=2)
            t = s.telemetry()
            counters.append({f: getattr(t, f) for f in (
                "bytes_h2d", "bytes_d2h", "cache_hits", "cache_misses", "clean_evictions",
                "dirty_evictions", "writebacks_completed", "mappings", "handle_reuses",
                "event_boundaries")})
    assert counters[0] == counters[1]


def test_repeat_hits_cached_panels(sim, oracle_mod):
    m = n = k = 64
    prob = Problem(uniform(oracle_mod, m, k, 13), uniform(oracle_mod, k, n, 14))
    with small_session(sim, frames=16) as s:
        out = prob.run(s, repeat=3)
        t = s.telemetry()
        assert t.bytes_h2d == 2 * m * k * 4
        # C stays cached (dirty) between executions; only the final read of C
        # writes it back.
        assert t.bytes_d2h == m * n * 4
        assert t.writebacks_completed == 1 and t.dirty_evictions == 0
        assert t.cache_hits == 6   # A, B and C hit on the 2nd and 3rd execution
    check(oracle_mod, prob, out)


def test_write_invalidates_cached_panels(sim, oracle_mod):
    m = n = k = 48
    a1, b1 = uniform(oracle_mod, m, k, 15), uniform(oracle_mod, k, n, 16)
    a2 = uniform(oracle_mod, m, k, 17)
    with small_session(sim, frames=16) as s:
        a = s.allocation(m * k * 4)
        b = s.allocation(k * n * 4)
        c = s.allocation(m * n * 4)
        a.write(np.ascontiguousarray(a1.T))
        b.write(np.ascontiguousarray(b1.T))
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
        plan.execute()
        a.write(np.ascontiguousarray(a2.T))  # must drop the cached A panel
        plan.execute()
        out = np.asfortranarray(c.read(dtype=np.float32).reshape(n, m).T)
        plan.release()
    prob = Problem(a2, b1)
    check(oracle_mod, prob, out)
