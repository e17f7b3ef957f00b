"""CPU tests of split-K launches over libxvram_hostsim.so.

A launch whose C has fewer 256 x 256 tiles than the chip has CUs cuts its K
into ranges (kernels::split_k_plan: as many as fill one workgroup per CU, each
at least 256 deep, in multiples of 32), accumulates each range into a partial
held in one frame of the pool, and adds the partials in range order before
alpha, beta and the epilogue. The simulated device performs exactly that data
flow (partials written to and read back from the frame, which must be mapped)
and counts the launches that split, so these tests check the planner's
reservation of the frame, the executor's use of it, the split arithmetic
(bit-exact analytic pattern, FP64 bound with K tails, beta and the epilogue)
and that repeated runs give identical bits. The same launches on the GPU are
in tests/test_gpu_split_k.py."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import pattern_operands, storage, uniform

MiB = 1 << 20
FORMS = {"NN": (abi.OP_N, abi.OP_N), "NT": (abi.OP_N, abi.OP_T), "TN": (abi.OP_T, abi.OP_N),
         "TT": (abi.OP_T, abi.OP_T)}


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_split_launches.restype = ctypes.c_uint64
    lib.dll.xvram_hostsim_split_launches.argtypes = [ctypes.POINTER(ctypes.c_int)]
    yield lib
    lib.dll.xvram_hostsim_reset()


def split_stats(lib):
    last = ctypes.c_int(0)
    count = lib.dll.xvram_hostsim_split_launches(ctypes.byref(last))
    return count, last.value


def run(s, a_op, b_op, ops, c0=None, alpha=1.0, beta=0.0, bias=None, relu=False, repeat=1):
    m, k = a_op.shape
    n = b_op.shape[1]
    a_st = a_op if ops[0] == abi.OP_N else a_op.T
    b_st = b_op if ops[1] == abi.OP_N else b_op.T
    a_flat, lda = storage(np.ascontiguousarray(a_st), abi.COLUMN_MAJOR)
    b_flat, ldb = storage(np.ascontiguousarray(b_st), abi.COLUMN_MAJOR)
    c_flat, ldc = storage(c0 if c0 is not None else np.zeros((m, n), np.float32), abi.COLUMN_MAJOR)
    A, B, C = (s.allocation(x.nbytes) for x in (a_flat, b_flat, c_flat))
    A.write(a_flat)
    B.write(b_flat)
    ep = None
    if bias is not None or relu:
        V = None
        if bias is not None:
            V = s.allocation(bias.nbytes)
            V.write(bias)
        ep = xv.epilogue(V, abi.BIAS_PER_COLUMN if V is not None else abi.BIAS_NONE, relu=relu)
    plan = xv.GemmPlan(s, xv.matrix(A, *a_st.shape, lda), xv.matrix(B, *b_st.shape, ldb),
                       xv.matrix(C, m, n, ldc), ops[0], ops[1], alpha, beta, epilogue=ep)
    outs = []
    for _ in range(repeat):
        C.write(c_flat)
        plan.execute()
        outs.append(C.read(dtype=np.float32).reshape(n, ldc)[:, :m].T.copy())
    info = plan.info()
    plan.release()
    return outs, info


def session(lib, frame_mib=16, frames=12):
    return xv.Session(lib, chunk_size_bytes=frame_mib * MiB, cache_target_bytes=frames * frame_mib * MiB,
                      workspace_cap_bytes=0, device_headroom_bytes=0, max_transaction_ms=600000)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_split_pattern_is_exact(sim, oracle_mod, form):
    """512 x 256 x 2048: two tiles, so eight K ranges of 256 (one launch)."""
    m, n, k = 512, 256, 2048
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim) as s:
        (out,), info = run(s, a_op, b_op, FORMS[form])
    assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (m, n, k, 1)
    assert split_stats(sim) == (1, 8)
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


@pytest.mark.parametrize("form", sorted(FORMS))
def test_split_with_k_tail_beta_and_epilogue(sim, oracle_mod, form):
    """K = 1000: three ranges of 352, 352 and 296 (a tail that is no multiple
    of 32); alpha, beta and a per-column bias with ReLU after the reduction.
    Within the FP64 bound, and the same bits on every run."""
    m, n, k = 512, 256, 1000
    a_op = uniform(oracle_mod, m, k, 71)
    b_op = uniform(oracle_mod, k, n, 72)
    c0 = uniform(oracle_mod, m, n, 73)
    bias = (oracle_mod.fill_uniform(n, 74) * 0.5).astype(np.float32)
    with session(sim) as s:
        outs, _ = run(s, a_op, b_op, FORMS[form], c0, alpha=-0.75, beta=0.5, bias=bias,
                      relu=True, repeat=2)
    assert split_stats(sim) == (2, 3)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    a64, b64 = a_op.astype(np.float64), b_op.astype(np.float64)
    ref = np.maximum(-0.75 * (a64 @ b64) + 0.5 * c0 + bias[None, :], 0.0)
    absab = 0.75 * (np.abs(a64) @ np.abs(b64)) + 0.5 * np.abs(c0) + np.abs(bias)[None, :]
    bound = 4 * k * 2.0 ** -24 * absab + 1e-30
    assert np.all(np.abs(outs[0] - ref) <= bound)


def test_split_across_k_panels(sim, oracle_mod):
    """K panels smaller than K (frames of 2 MiB: 512 x 1024 panels): each
    launch splits its own panel; later panels accumulate onto C (beta 1)."""
    m, n, k = 512, 256, 4096
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim, frame_mib=2, frames=16) as s:
        (out,), info = run(s, a_op, b_op, FORMS["NT"])
    assert info.tile_k < k and info.tile_count == k // info.tile_k
    count, last = split_stats(sim)
    assert count == info.tile_count and last >= 2
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_no_split_when_k_is_shallow_or_tiles_fill_the_chip(sim, oracle_mod):
    """K = 384 leaves fewer than two ranges of 256; ragged C (m = 500) is not
    a whole number of 256 x 256 tiles: both run unsplit."""
    for m, n, k in ((512, 256, 384), (500, 256, 2048)):
        a_op, b_op = pattern_operands(m, n, k)
        with session(sim) as s:
            (out,), _ = run(s, a_op, b_op, FORMS["NN"])
        assert split_stats(sim)[0] == 0
        assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_split_frame_is_returned_to_the_pool(sim, oracle_mod):
    """The partials' frame is not a cache entry: the session still tears down
    balanced, and nothing of it is written back."""
    m, n, k = 512, 256, 2048
    a_op, b_op = pattern_operands(m, n, k)
    s = session(sim)
    run(s, a_op, b_op, FORMS["TN"])
    run(s, a_op, b_op, FORMS["TN"])
    s.drain()
    t = s.telemetry()
    assert t.bytes_d2h == 2 * m * n * 4  # the two C results, nothing of the partials
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps and t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    assert t.physical_handles_created == t.physical_handles_released
    s.release()
