"""GPU parity of the 256 x 256 tile kernel (sgemm_wide.hip).

A launch with at least 256 such tiles (C of 4096 x 4096 or more) and operand
panels under 2^31 bytes runs the wide kernel; these cases cover its four
operation forms (direct-to-LDS and register-staged operands), interior and edge
tiles, the K tail after its three-stage unrolled loop, alpha/beta, the fused
bias/ReLU epilogue, and one out-of-core case whose 4096 x 4096 C tiles
accumulate over several K panels.

N/T launches whose tiles are all interior (m, n multiples of 256) and whose K
is a multiple of 4 run the barrier-free variant (sgemm_ring_kernel: each wave
streams its own operand halves through a private LDS ring); the N/T cases
above with such shapes (interior, bit-exact pattern, beta = 0 over NaN,
out-of-core panels) run it, and the ring cases below add K tails around its
8-pair unrolled loop and 7-pair prefetch distance, alpha/beta and the epilogue.
Launches of the other forms with such tiles and K a multiple of 8 run
sgemm_ring8_kernel (the same scheme with k-contiguous halves loaded straight
into LDS in 8-deep slots): the NN, TN and TT interior and pattern cases above
run it, and the ring8 cases add its slot tails, alpha/beta and the shapes
that fall back to sgemm_wide_kernel.

Ragged launches whose K is a multiple of 4 (N/T) or 8 run whole on the ring
kernels' edge instances (tests/test_gpu_edge_ring.py) or take an edge split
(interior on the ring kernels, strips apart; tests/test_gpu_edge_split.py),
and those whose K is not, with K rounded down at least 512, a K remainder; the
ragged random case here has K = 501 and stays whole on sgemm_wide_kernel, and
the ragged pattern cases of the ring tests below run the edge instances.

Random cases are checked element by element against the FP64 oracle on three
column ranges (first, middle and last tile columns, every row) with the bound
|C - C_ref| <= 4*K*2^-24*(|alpha|(|A||B|)_ij + |beta*C0_ij|); the analytic
integer pattern is checked bit-exactly over the whole matrix (exact in FP32
while 28*K < 2^24)."""
import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import Problem, logical_from_storage, pattern_operands, storage, uniform

pytestmark = pytest.mark.gpu

MiB = 1 << 20
OPS = [(abi.OP_N, abi.OP_N), (abi.OP_N, abi.OP_T), (abi.OP_T, abi.OP_N), (abi.OP_T, abi.OP_T)]
OP_IDS = ["NN", "NT", "TN", "TT"]


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.fixture(scope="module")
def resident(lib):
    s = xv.Session(lib, chunk_size_bytes=256 * MiB)
    yield s
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps == t.set_access_calls
    assert t.physical_handles_created == t.physical_handles_released
    assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    s.release()


def column_ranges(n, width=24):
    mid = n // 2 - width // 2
    return [(0, width), (mid, mid + width), (n - width, n)]


def sampled_check(oracle, prob, out, label):
    worst = 0.0
    for j0, j1 in column_ranges(prob.n):
        ref, absab = prob.reference(oracle, columns=(j0, j1))
        bad, max_err, ratio = oracle.check_bound(np.asfortranarray(out[:, j0:j1]), prob.k,
                                                 ref, absab)
        print(f"{label} cols {j0}:{j1}: violations={bad} max_err={max_err:.3e} "
              f"err/bound={ratio:.3e}", flush=True)
        assert bad == 0, f"{label}: {bad} elements of columns {j0}:{j1} outside the bound"
        worst = max(worst, ratio)
    return worst


@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_wide_interior(resident, oracle_mod, ops):
    """4096 x 4096 x 1040: 256 interior tiles, 65 K stages (unrolled loop + tail)."""
    m, n, k = 4096, 4096, 1040
    prob = Problem(uniform(oracle_mod, m, k, 1101), uniform(oracle_mod, k, n, 1102),
                   op_a=ops[0], op_b=ops[1])
    out = prob.run(resident)
    assert prob.plan_info.tile_count == 1
    sampled_check(oracle_mod, prob, out, f"wide interior {ops}")


@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_wide_edges_alpha_beta(resident, oracle_mod, ops):
    """4000 x 3950 x 501: edge tiles on both sides and a partial last K stage
    (16 x 16 tiles: one round, no edge split; K rounded down to a multiple of 4
    or 8 is below 512, so no K remainder: the launch stays whole on this
    kernel)."""
    m, n, k = 4000, 3950, 501
    prob = Problem(uniform(oracle_mod, m, k, 1201), uniform(oracle_mod, k, n, 1202),
                   uniform(oracle_mod, m, n, 1203), op_a=ops[0], op_b=ops[1],
                   alpha=-1.25, beta=0.75)
    out = prob.run(resident)
    sampled_check(oracle_mod, prob, out, f"wide edges {ops}")


@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_wide_pattern_bit_exact(resident, oracle_mod, ops):
    m, n, k = 4352, 4096, 1104
    a_op, b_op = pattern_operands(m, n, k)
    prob = Problem(a_op, b_op, op_a=ops[0], op_b=ops[1])
    out = prob.run(resident)
    expected = oracle_mod.pattern_expected_matrix(m, n, k)
    assert np.array_equal(out.astype(np.float64), expected)


def test_wide_beta_zero_over_nan(resident, oracle_mod):
    m, n, k = 4096, 4096, 528
    prob = Problem(uniform(oracle_mod, m, k, 1301), uniform(oracle_mod, k, n, 1302),
                   op_b=abi.OP_T)
    out = prob.run(resident, c_fill=np.float32(np.nan))
    assert np.isfinite(out).all()
    sampled_check(oracle_mod, prob, out, "wide beta=0 over NaN C")


@pytest.mark.parametrize("k", [4, 28, 32, 36, 60, 64, 1036])
def test_ring_k_tails_pattern(resident, oracle_mod, k):
    """Barrier-free N/T kernel, bit-exact pattern: fewer pairs than the
    prefetch distance (k = 4, 28), exactly one unrolled block plus tail
    (32 .. 64) and a long loop with a 3-pair tail (1036)."""
    m, n = 4096, 4096
    a_op, b_op = pattern_operands(m, n, k)
    prob = Problem(a_op, b_op, op_b=abi.OP_T)
    out = prob.run(resident)
    assert prob.plan_info.tile_count == 1
    expected = oracle_mod.pattern_expected_matrix(m, n, k)
    assert np.array_equal(out.astype(np.float64), expected)


@pytest.mark.parametrize("m,n,k", [(4096, 4096, 1001), (4000, 4096, 1040), (4096, 4000, 1040)],
                         ids=["k%4-wide", "m%256-edge", "n%256-edge"])
def test_ring_fallback_shapes_pattern(resident, oracle_mod, m, n, k):
    """N/T launches just outside the interior barrier-free kernel's conditions:
    K not a multiple of 4 (one round of interior tiles, which neither a tail
    split nor a K remainder would speed up: sgemm_wide_kernel), or m or n not a
    multiple of 256 (one round of 16 x 16 tiles, which no edge split would
    speed up: the ring kernel's edge instance). Bit-exact pattern."""
    a_op, b_op = pattern_operands(m, n, k)
    prob = Problem(a_op, b_op, op_b=abi.OP_T)
    out = prob.run(resident)
    assert prob.plan_info.tile_count == 1
    expected = oracle_mod.pattern_expected_matrix(m, n, k)
    assert np.array_equal(out.astype(np.float64), expected)


KC_OPS = OPS[:1] + OPS[2:]
KC_IDS = ["NN", "TN", "TT"]


@pytest.mark.parametrize("k", [8, 24, 32, 40, 56, 1048])
@pytest.mark.parametrize("ops", KC_OPS, ids=KC_IDS)
def test_ring8_k_tails_pattern(resident, oracle_mod, ops, k):
    """Barrier-free kernel of the forms with a k-contiguous operand, bit-exact
    pattern: fewer 8-deep slots than the ring (k = 8, 24), exactly one
    unrolled block (32), a block plus a tail (40, 56) and a long loop with a
    3-slot tail (1048)."""
    m, n = 4096, 4096
    a_op, b_op = pattern_operands(m, n, k)
    prob = Problem(a_op, b_op, op_a=ops[0], op_b=ops[1])
    out = prob.run(resident)
    assert prob.plan_info.tile_count == 1
    expected = oracle_mod.pattern_expected_matrix(m, n, k)
    assert np.array_equal(out.astype(np.float64), expected)


@pytest.mark.parametrize("ops", KC_OPS, ids=KC_IDS)
def test_ring8_alpha_beta(resident, oracle_mod, ops):
    m, n, k = 4608, 4096, 1000
    prob = Problem(uniform(oracle_mod, m, k, 1701), uniform(oracle_mod, k, n, 1702),
                   uniform(oracle_mod, m, n, 1703), op_a=ops[0], op_b=ops[1], alpha=-1.25,
                   beta=0.75)
    out = prob.run(resident)
    sampled_check(oracle_mod, prob, out, f"ring8 alpha/beta {ops}")


@pytest.mark.parametrize("ops,m,k", [(OPS[0], 4096, 1004), (OPS[2], 4000, 1040), (OPS[3], 4096, 1020)],
                         ids=["NN-k%8-wide", "TN-m%256-edge", "TT-k%8-wide"])
def test_ring8_fallback_shapes_pattern(resident, oracle_mod, ops, m, k):
    """Launches just outside that kernel's interior conditions in one round of
    16 x 16 tiles: K not a multiple of 8 (sgemm_wide_kernel) or m not a
    multiple of 256 (its edge instance). Bit-exact pattern."""
    n = 4096
    a_op, b_op = pattern_operands(m, n, k)
    prob = Problem(a_op, b_op, op_a=ops[0], op_b=ops[1])
    out = prob.run(resident)
    expected = oracle_mod.pattern_expected_matrix(m, n, k)
    assert np.array_equal(out.astype(np.float64), expected)


def test_ring_alpha_beta(resident, oracle_mod):
    m, n, k = 4608, 4096, 1000
    prob = Problem(uniform(oracle_mod, m, k, 1601), uniform(oracle_mod, k, n, 1602),
                   uniform(oracle_mod, m, n, 1603), op_b=abi.OP_T, alpha=-1.25, beta=0.75)
    out = prob.run(resident)
    sampled_check(oracle_mod, prob, out, "ring alpha/beta")


@pytest.mark.parametrize("n", [4000, 4096], ids=["wide", "ring"])
@pytest.mark.parametrize("axis", [abi.BIAS_PER_ROW, abi.BIAS_PER_COLUMN], ids=["row", "col"])
def test_wide_epilogue(lib, oracle_mod, axis, n):
    m, k = 4096, 800
    a = uniform(oracle_mod, m, k, 1401)
    b = uniform(oracle_mod, k, n, 1402)
    c0 = uniform(oracle_mod, m, n, 1403)
    bias = oracle_mod.fill_uniform(m if axis == abi.BIAS_PER_ROW else n, 1404).astype(np.float32)
    s = xv.Session(lib, chunk_size_bytes=256 * MiB)
    try:
        a_flat, lda = storage(np.ascontiguousarray(a), abi.COLUMN_MAJOR)
        b_flat, ldb = storage(np.ascontiguousarray(b.T), abi.ROW_MAJOR)  # op(B) = T over B^T
        c_flat, ldc = storage(c0, abi.COLUMN_MAJOR)
        A, B, C, V = (s.allocation(x) for x in (a_flat.nbytes, b_flat.nbytes, c_flat.nbytes,
                                                bias.nbytes))
        A.write(a_flat)
        B.write(b_flat)
        C.write(c_flat)
        V.write(bias)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, lda, abi.COLUMN_MAJOR),
                           xv.matrix(B, n, k, ldb, abi.ROW_MAJOR),
                           xv.matrix(C, m, n, ldc, abi.COLUMN_MAJOR), abi.OP_N, abi.OP_T,
                           0.5, 1.5, epilogue=xv.epilogue(V, axis, relu=True))
        plan.execute()
        out = np.asfortranarray(logical_from_storage(C.read(dtype=np.float32), m, n, ldc,
                                                     abi.COLUMN_MAJOR))
        plan.release()
    finally:
        s.close()
        s.release()
    for j0, j1 in column_ranges(n):
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a), np.asfortranarray(b), 0.5, 1.5,
                                          np.asfortranarray(c0), 0, (j0, j1))
        add = bias.astype(np.float64)[:, None] if axis == abi.BIAS_PER_ROW else \
            bias.astype(np.float64)[None, j0:j1]
        ref = np.maximum(ref + add, 0.0)
        bad, max_err, ratio = oracle_mod.check_bound(np.asfortranarray(out[:, j0:j1]), k,
                                                     np.asfortranarray(ref),
                                                     np.asfortranarray(absab + np.abs(add)))
        print(f"wide epilogue axis {axis} cols {j0}:{j1}: violations={bad} "
              f"err/bound={ratio:.3e}", flush=True)
        assert bad == 0


def test_wide_out_of_core_panels(lib, oracle_mod):
    """8192 x 8192 x 6000 under a 9-frame budget of 64 MiB frames: 4096 x 4096 C
    tiles, each accumulated over K panels (beta = 1 after the first) with
    evictions and write-backs in between."""
    m, n, k = 8192, 8192, 6000
    prob = Problem(uniform(oracle_mod, m, k, 1501), uniform(oracle_mod, k, n, 1502),
                   op_b=abi.OP_T)
    with xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=9 * 64 * MiB,
                    workspace_cap_bytes=0, device_headroom_bytes=0) as s:
        out = prob.run(s)
        t = s.telemetry()
        assert prob.plan_info.tile_count > 1
        assert t.clean_evictions + t.dirty_evictions > 0
        assert t.resident_bytes_peak <= t.cache_target_bytes
    sampled_check(oracle_mod, prob, out, "wide out-of-core 8192x8192x6000")


def test_mixed_kernels_out_of_core_pattern(lib, oracle_mod):
    """8192 x 8192 x 6002 N/T on 64 MiB frames: 4096 x 4096 C tiles over a
    4096-deep K panel (barrier-free kernel) and a 1906-deep one (K not a
    multiple of 4: sgemm_wide_kernel), accumulated through C between launches
    (and the first launch sliced): bit-exact pattern."""
    m, n, k = 8192, 8192, 6002
    a_op, b_op = pattern_operands(m, n, k)
    prob = Problem(a_op, b_op, op_b=abi.OP_T)
    with xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=12 * 64 * MiB,
                    workspace_cap_bytes=0, device_headroom_bytes=0) as s:
        out = prob.run(s)
        info = prob.plan_info
    assert (info.tile_m, info.tile_n, info.tile_k) == (4096, 4096, 4096) and info.tile_count == 8
    expected = oracle_mod.pattern_expected_matrix(m, n, k)
    assert np.array_equal(out.astype(np.float64), expected)
