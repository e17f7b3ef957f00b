"""CPU tests of the sliced first launch over libxvram_hostsim.so.

An operation's first launch whose panel depth is at least twice the minimum
slice (2048) runs as one kernel per K slice (at most 8, each at least 2048
deep); each of its missing A or B panels is filled by one copy per slice and
each kernel waits only for its own slices. The slicing belongs to the plan: a
first launch whose panels are cached runs the same slices, so C does not
depend on what an earlier operation left in the cache. These cases make the
first launch 4096 or 8192 deep and check: the kernel count (one per slice of
the first launch, one per later launch), bit-exact analytic-pattern results in
all four N/T forms, beta over the slices (the first slice applies the caller's
beta, the later ones accumulate), the epilogue applied once after the last
slice, and unchanged accounting (the slices tile the panels: same H2D bytes;
one retired tile per tile)."""
import json

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import Problem, pattern_operands, uniform

MiB = 1 << 20
OPS = [(abi.OP_N, abi.OP_N), (abi.OP_N, abi.OP_T), (abi.OP_T, abi.OP_N), (abi.OP_T, abi.OP_T)]
OP_IDS = ["NN", "NT", "TN", "TT"]


@pytest.fixture()
def sim(tmp_path, monkeypatch):
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("XVRAM_TRACE_FILE", str(trace))
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib, trace
    lib.dll.xvram_hostsim_reset()


def session(lib, frame_mib=2, frames=10):
    return xv.Session(lib, chunk_size_bytes=frame_mib * MiB,
                      cache_target_bytes=frames * frame_mib * MiB, workspace_cap_bytes=0,
                      device_headroom_bytes=0, max_transaction_ms=600000)


def kernels_per_operation(trace):
    return [len(json.loads(line)["kernels"]) for line in open(trace)]


@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_first_launch_runs_in_k_slices(sim, oracle_mod, ops):
    lib, trace = sim
    # 2 MiB frames: 128 x 4096 panels, so K = 8192 is two 4096-deep launches and
    # the first one runs as two 2048-deep slices.
    m, n, k = 128, 64, 8192
    a_op, b_op = pattern_operands(m, n, k)
    with session(lib) as s:
        prob = Problem(a_op, b_op, op_a=ops[0], op_b=ops[1])
        out = prob.run(s)
        t = s.telemetry()
        info = prob.plan_info
    assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (128, 64, 4096, 2)
    assert kernels_per_operation(trace) == [3]          # 2 slices + the second launch
    assert t.transactions_completed == info.tile_count  # one retired tile per tile
    assert t.bytes_h2d == (m * k + k * n) * 4           # slices tile the panels exactly
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_slices_apply_beta_once(sim, oracle_mod):
    lib, trace = sim
    m, n, k = 128, 64, 8192
    prob = Problem(uniform(oracle_mod, m, k, 21), uniform(oracle_mod, k, n, 22),
                   uniform(oracle_mod, m, n, 23), alpha=-0.75, beta=0.5,
                   layouts=(abi.COLUMN_MAJOR, abi.ROW_MAJOR, abi.COLUMN_MAJOR))
    with session(lib) as s:
        out = prob.run(s)
    assert kernels_per_operation(trace) == [3]
    ref, absab = prob.reference(oracle_mod)
    assert oracle_mod.check_bound(out, k, ref, absab)[0] == 0


def test_cached_panels_keep_the_slicing(sim, oracle_mod):
    """A second execution finds the first launch's panels cached and runs the
    same slices (without waits): C does not depend on the cache state."""
    lib, trace = sim
    m, n, k = 128, 64, 8192
    a_op, b_op = pattern_operands(m, n, k)
    with session(lib, frames=12) as s:
        prob = Problem(a_op, b_op)
        out = prob.run(s, repeat=2)
        t = s.telemetry()
    assert kernels_per_operation(trace) == [3, 3]
    assert t.bytes_h2d == (m * k + k * n) * 4  # the second execution hit every panel
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_epilogue_after_the_last_slice(sim, oracle_mod):
    """One 8192-deep K panel per tile (8 MiB frames, two C tiles): the first
    launch runs as four slices and the bias/ReLU epilogue must apply once, on
    the last slice only."""
    lib, trace = sim
    m, n, k = 256, 128, 8192
    a_op = uniform(oracle_mod, m, k, 31)
    b_op = uniform(oracle_mod, k, n, 32)
    bias_vec = uniform(oracle_mod, 1, n, 33).reshape(n) * np.float32(4.0)
    with session(lib, frame_mib=8, frames=8) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        A.write(np.asfortranarray(a_op).T.copy())
        B.write(np.asfortranarray(b_op).T.copy())
        bias = s.allocation(n * 4)
        bias.write(bias_vec)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k), xv.matrix(C, m, n, m),
                           tile_hints=(128, 0, 8192),
                           epilogue=xv.epilogue(bias, abi.BIAS_PER_COLUMN, relu=True))
        info = plan.info()
        plan.execute()
        out = np.asfortranarray(C.read(dtype=np.float32).reshape(n, m).T)
        plan.release()
    assert info.tile_k == k and info.tile_count == 2
    assert kernels_per_operation(trace) == [5]          # 4 slices + the second tile
    ref, absab = oracle_mod.sgemm_f64(a_op, b_op)
    pre = ref + bias_vec.astype(np.float64)[None, :]
    bound = 4 * k * 2.0 ** -24 * (absab + np.abs(bias_vec)[None, :])
    assert np.all(np.abs(out - np.maximum(pre, 0.0)) <= bound)
