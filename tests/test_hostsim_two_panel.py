"""CPU tests of launches over two K panels, over libxvram_hostsim.so.

Short launches of interior 256 x 256 tiles (a C tile of at least 4096 x 4096
elements; K a multiple of 4 for N/T, of 8 for the other forms) take two K
panels per launch when the schedule's H2D traffic does not grow: the tile kernel then reads and writes the C tile once per two
panels. The simulated device enforces the gfx950 two-panel launch contract
(xvram_amd/csrc/sgemm_launch.hpp) and computes each element's K products in
order, so these cases check the planner's choice, the executor's acquisition
and dispatch of both panels (one dispatch per launch), alpha/beta applied once
per C tile pass, the fused epilogue after the last pass, the accounting (one
retired tile per C tile x K panel, the same H2D bytes as one-panel launches)
and bit-exact analytic-pattern results. The operation's first K pass (its
first block's) runs as one-panel launches: there the link sets the pace and
one panel per launch needs half the new bytes per launch."""
import json

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import pattern_operands, storage, uniform

MiB = 1 << 20
M = N = 4096  # one C tile of 16 x 16 tiles of 256 x 256: the two-panel kernel's minimum


@pytest.fixture()
def sim(tmp_path, monkeypatch):
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("XVRAM_TRACE_FILE", str(trace))
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib, trace
    lib.dll.xvram_hostsim_reset()


def session(lib, frames=12):
    # 64 MiB frames hold the 4096 x 4096 C tile.
    return xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=frames * 64 * MiB,
                      workspace_cap_bytes=0, device_headroom_bytes=0, max_transaction_ms=600000)


def kernels_per_operation(trace):
    return [len(json.loads(line)["kernels"]) for line in open(trace)]


def run_nt(s, a_op, b_op, c0=None, alpha=1.0, beta=0.0, tile_k=32, epilogue=None, bias=None,
           ops=(abi.OP_N, abi.OP_T)):
    """C (column-major) = alpha * op(A) * op(B) + beta * C0 with A and B stored
    for `ops` (default: A op-N, m x k, and B op-T, n x k), tile hints (4096,
    4096, tile_k)."""
    m, k = a_op.shape
    n = b_op.shape[1]
    a_stored = a_op if ops[0] == abi.OP_N else a_op.T
    b_stored = b_op if ops[1] == abi.OP_N else b_op.T
    a_flat, lda = storage(np.ascontiguousarray(a_stored), abi.COLUMN_MAJOR)
    b_flat, ldb = storage(np.ascontiguousarray(b_stored), abi.COLUMN_MAJOR)
    c_flat, ldc = storage(c0 if c0 is not None else np.zeros((m, n), np.float32), abi.COLUMN_MAJOR)
    A, B, C = (s.allocation(x.nbytes) for x in (a_flat, b_flat, c_flat))
    A.write(a_flat)
    B.write(b_flat)
    C.write(c_flat)
    ep = None
    if bias is not None:
        V = s.allocation(bias.nbytes)
        V.write(bias)
        ep = xv.epilogue(V, abi.BIAS_PER_COLUMN, relu=epilogue == "relu")
    plan = xv.GemmPlan(s, xv.matrix(A, *a_stored.shape, lda), xv.matrix(B, *b_stored.shape, ldb),
                       xv.matrix(C, m, n, ldc), ops[0], ops[1], alpha, beta,
                       tile_hints=(4096, 4096, tile_k), epilogue=ep)
    info = plan.info()
    plan.execute()
    out = C.read(dtype=np.float32).reshape(n, ldc)[:, :m].T
    plan.release()
    return np.asfortranarray(out), info


def test_two_panel_launches_are_exact(sim, oracle_mod):
    lib, trace = sim
    k = 192  # six 32-deep K panels: the first pass as two one-panel launches, then two of two
    a_op, b_op = pattern_operands(M, N, k)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op)
        t = s.telemetry()
    assert (info.tile_m, info.tile_n, info.tile_k) == (4096, 4096, 32)
    assert info.tile_count == 6                          # C tiles x K panels
    assert info.maximum_working_set_bytes == 5 * 64 * MiB  # C + two A + two B frames
    assert kernels_per_operation(trace) == [4]           # one dispatch per launch
    assert t.transactions_completed == info.tile_count   # one retired tile per K panel
    assert t.bytes_h2d == (M * k + k * N) * 4            # every panel loaded once
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M, N, k))


@pytest.mark.parametrize("ops", [(abi.OP_N, abi.OP_N), (abi.OP_T, abi.OP_N), (abi.OP_T, abi.OP_T)],
                         ids=["NN", "TN", "TT"])
def test_two_panel_launches_other_forms(sim, oracle_mod, ops):
    """The same schedule for the forms with a k-contiguous operand (K a
    multiple of 8): one dispatch per launch, bit-exact pattern, and seeded
    U[-1,1) data within the FP64 bound on a column subset."""
    lib, trace = sim
    k = 192
    a_op, b_op = pattern_operands(M, N, k)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op, ops=ops)
    assert info.tile_count == 6 and info.maximum_working_set_bytes == 5 * 64 * MiB
    assert kernels_per_operation(trace) == [4]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M, N, k))
    k = 128
    a_op = uniform(oracle_mod, M, k, 41)
    b_op = uniform(oracle_mod, k, N, 42)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op, ops=ops)
    assert kernels_per_operation(trace) == [4, 3]
    cols = np.arange(0, N, 101)
    ref = a_op.astype(np.float64) @ b_op[:, cols].astype(np.float64)
    bound = 4 * k * 2.0 ** -24 * (np.abs(a_op).astype(np.float64) @
                                  np.abs(b_op[:, cols]).astype(np.float64)) + 1e-30
    assert np.all(np.abs(out[:, cols].astype(np.float64) - ref) <= bound)


def test_ragged_pair_of_a_k_contiguous_operand_runs_per_panel(sim, oracle_mod):
    """N/N, K = 112 in 32-deep panels: B's panels hold K inside their lines, so
    the 32-deep and 16-deep panels of the last launch have different leading
    dimensions and that launch runs one dispatch per panel."""
    lib, trace = sim
    k = 112
    a_op, b_op = pattern_operands(M, N, k)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op, ops=(abi.OP_N, abi.OP_N))
    assert info.tile_count == 4
    assert kernels_per_operation(trace) == [4]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M, N, k))


def test_odd_panel_count_ends_with_one_panel(sim, oracle_mod):
    lib, trace = sim
    k = 160  # five panels: two one-panel launches (first pass), one of two, one of one
    a_op, b_op = pattern_operands(M, N, k)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op)
    assert info.tile_count == 5
    assert kernels_per_operation(trace) == [4]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M, N, k))


def test_ragged_second_panel(sim, oracle_mod):
    """K = 112 in 32-deep panels: after the first pass's two one-panel launches,
    the second pass pairs a 32-deep panel with a 16-deep one (k_split 32, k 48)
    in one two-panel dispatch."""
    lib, trace = sim
    k = 112
    a_op, b_op = pattern_operands(M, N, k)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op)
    assert info.tile_count == 4
    assert kernels_per_operation(trace) == [3]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M, N, k))


def test_alpha_beta_and_epilogue_over_two_panel_passes(sim, oracle_mod):
    lib, trace = sim
    k = 128
    a_op = uniform(oracle_mod, M, k, 31)
    b_op = uniform(oracle_mod, k, N, 32)
    c0 = uniform(oracle_mod, M, N, 33)
    bias = (oracle_mod.fill_uniform(N, 34) * 0.25).astype(np.float32)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op, c0, alpha=-0.75, beta=0.5, epilogue="relu", bias=bias)
    assert kernels_per_operation(trace) == [3]
    # FP64 reference of act(alpha A B + beta C0 + bias) on a column subset.
    cols = np.arange(0, N, 97)
    ref = (-0.75 * (a_op.astype(np.float64) @ b_op[:, cols].astype(np.float64))
           + 0.5 * c0[:, cols].astype(np.float64) + bias[cols].astype(np.float64)[None, :])
    ref = np.maximum(ref, 0.0)
    absab = (0.75 * (np.abs(a_op).astype(np.float64) @ np.abs(b_op[:, cols]).astype(np.float64))
             + 0.5 * np.abs(c0[:, cols]).astype(np.float64) + np.abs(bias[cols])[None, :])
    bound = 4 * k * 2.0 ** -24 * absab + 1e-30
    assert np.all(np.abs(out[:, cols].astype(np.float64) - ref) <= bound)


def test_planner_keeps_one_panel_when_frames_are_short(sim, oracle_mod):
    """With too few frames for the two-panel working set the plan keeps one
    panel per launch (same H2D either way here, so only frames decide)."""
    lib, trace = sim
    k = 128
    a_op, b_op = pattern_operands(M, N, k)
    with session(lib, frames=6) as s:
        out, info = run_nt(s, a_op, b_op)
    assert info.maximum_working_set_bytes == 3 * 64 * MiB
    assert kernels_per_operation(trace) == [4]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M, N, k))


def test_one_panel_below_the_two_panel_tile_count(sim, oracle_mod):
    """A 3840 x 4096 C tile is 240 tiles of 256 x 256, under the two-panel
    kernel's minimum of one per CU: one panel per launch."""
    lib, trace = sim
    k = 64
    a_op, b_op = pattern_operands(M - 256, N, k)
    with session(lib) as s:
        out, info = run_nt(s, a_op, b_op)
    assert kernels_per_operation(trace) == [2]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(M - 256, N, k))
