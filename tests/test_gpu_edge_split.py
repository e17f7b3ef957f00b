"""Edge splits on the MI355X, through the C ABI, against the oracle.

A launch of at least 256 tiles of 256 x 256 whose m or n is not a multiple of
256 may run as its interior tiles (ring kernels, or their tail split) and two
edge strips, each a launch of its own (kernels::edge_parts):

* 4100 x 4100 x 1024 (17 x 17 tiles: the 16 x 16 interior, a 4096 x 4 right
  strip and a 4 x 4100 bottom strip), all four forms, seeded U[-1,1) operands
  with alpha, beta and ReLU and a per-row or per-column bias (offset into each
  strip's rows or columns): every element within the FP64 bound, and two
  executions bit-identical.
* 5000 x 5000 x 2048 (the interior of 19 x 19 tiles takes a tail split), N/N
  and N/T: the analytic pattern, every element bit-exact.
* 4100 x 4100 x 1024 in a session (resident, 128 MiB frames: the strips'
  partials in one frame of the pool), N/N and T/T: the pattern, bit-exact.

Tolerance: |C - C_ref| <= 4*K*2^-24*(|alpha||A||B| + |beta C0| + |bias|)_ij."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_sgemm_device import FORMS, Hip, desc_for, padded, stored
from test_gpu_tail_split import pattern_stored, synth  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu

MiB = 1 << 20


def log(msg):
    print(f"[edge-split] {msg}", flush=True)


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.fixture()
def hip(lib):
    h = Hip()
    yield h
    h.close()


@pytest.mark.parametrize("axis", [abi.BIAS_PER_ROW, abi.BIAS_PER_COLUMN], ids=["row", "col"])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_edge_split_within_bound_and_deterministic(lib, hip, oracle_mod, form, axis):
    m, n, k = 4100, 4100, 1024
    alpha, beta = 1.25, -0.5
    ops = FORMS[form]
    seed = 801
    a_op = np.asfortranarray(oracle_mod.fill_uniform(m * k, seed).reshape(k, m).T)
    b_op = np.asfortranarray(oracle_mod.fill_uniform(k * n, seed + 1).reshape(n, k).T)
    c0 = np.asfortranarray(oracle_mod.fill_uniform(m * n, seed + 2).reshape(n, m).T)
    length = m if axis == abi.BIAS_PER_ROW else n
    bias = (oracle_mod.fill_uniform(length, seed + 3) * 0.5).astype(np.float32)
    a_flat, lda = stored(a_op, ops[0])
    b_flat, ldb = stored(b_op, ops[1])
    c_flat, ldc = padded(c0)
    pa, pb, pc = hip.alloc(a_flat.nbytes), hip.alloc(b_flat.nbytes), hip.alloc(c_flat.nbytes)
    pbias = hip.alloc(bias.nbytes)
    s = hip.stream()
    outs = []
    try:
        hip.put(pa, a_flat)
        hip.put(pb, b_flat)
        hip.put(pbias, bias)
        d = desc_for((pa, pb, pc), m, n, k, ops, (lda, ldb, ldc), alpha, beta, pbias, axis, True)
        for _ in range(2):
            hip.put(pc, c_flat)
            assert lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(s)) == abi.SUCCESS
            hip.sync(s)
            outs.append(hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T)
    finally:
        for p in (pa, pb, pc, pbias):
            hip.free(p)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    ref, absab = oracle_mod.sgemm_f64(a_op, b_op, alpha, beta, c0)
    badd = bias[:, None] if axis == abi.BIAS_PER_ROW else bias[None, :]
    ref = np.maximum(ref + badd.astype(np.float64), 0.0)
    absab = absab + np.abs(badd)
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"{m}x{n}x{k} {form} bias {'row' if length == m else 'col'} + ReLU: violations {bad}, "
        f"err/bound {ratio:.3e}")
    assert bad == 0


@pytest.mark.parametrize("form", ["NN", "NT"])
def test_edge_split_with_tail_pattern(lib, hip, synth, oracle_mod, form):
    m, n, k = 5000, 5000, 2048
    ops = FORMS[form]
    a_st = pattern_stored(synth, "a", *((m, k) if ops[0] == abi.OP_N else (k, m)),
                          ops[0] == abi.OP_T)
    b_st = pattern_stored(synth, "b", *((k, n) if ops[1] == abi.OP_N else (n, k)),
                          ops[1] == abi.OP_T)
    a_flat, lda = padded(a_st)
    b_flat, ldb = padded(b_st)
    c_flat, ldc = padded(np.zeros((m, n), np.float32))
    pa, pb, pc = hip.alloc(a_flat.nbytes), hip.alloc(b_flat.nbytes), hip.alloc(c_flat.nbytes)
    s = hip.stream()
    try:
        hip.put(pa, a_flat)
        hip.put(pb, b_flat)
        hip.put(pc, c_flat)
        d = desc_for((pa, pb, pc), m, n, k, ops, (lda, ldb, ldc))
        assert lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(s)) == abi.SUCCESS
        hip.sync(s)
        got = hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T
    finally:
        for p in (pa, pb, pc):
            hip.free(p)
    expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
    bad = int(np.count_nonzero(got != expect))
    log(f"pattern {m}x{n}x{k} {form}: {bad} of {m * n} differ")
    assert bad == 0


@pytest.mark.parametrize("form", ["NN", "TT"])
def test_edge_split_in_a_session(lib, synth, oracle_mod, form):
    m, n, k = 4100, 4100, 1024
    ops = FORMS[form]
    a_shape = (m, k) if ops[0] == abi.OP_N else (k, m)
    b_shape = (k, n) if ops[1] == abi.OP_N else (n, k)
    s = xv.Session(lib, chunk_size_bytes=128 * MiB)
    try:
        a = s.allocation(m * k * 4)
        b = s.allocation(k * n * 4)
        c = s.allocation(m * n * 4)
        a.write(np.asfortranarray(pattern_stored(synth, "a", *a_shape, ops[0] == abi.OP_T))
                .T.reshape(-1))
        b.write(np.asfortranarray(pattern_stored(synth, "b", *b_shape, ops[1] == abi.OP_T))
                .T.reshape(-1))
        plan = xv.GemmPlan(s, xv.matrix(a, *a_shape, a_shape[0]), xv.matrix(b, *b_shape, b_shape[0]),
                           xv.matrix(c, m, n, m), ops[0], ops[1])
        info = plan.info()
        assert info.tile_count == 1
        # C, A, B and the partials' frame.
        assert info.maximum_working_set_bytes == 4 * 128 * MiB
        plan.execute()
        got = c.read(dtype=np.float32).reshape(n, m).T
        plan.release()
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps and t.physical_handles_created == t.physical_handles_released
        s.release()
    expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
    bad = int(np.count_nonzero(got != expect))
    log(f"session pattern {m}x{n}x{k} {form}: {bad} of {m * n} differ")
    assert bad == 0


@pytest.mark.parametrize("m,n,k,form", [(4100, 4100, 1028, "NN"), (4352, 4096, 1027, "TT"),
                                        (4100, 4100, 1030, "NT")],
                         ids=["edge-NN", "tail-TT", "edge-NT"])
def test_k_remainder_within_bound(lib, hip, oracle_mod, m, n, k, form):
    """K not a multiple of 8 (N/N, T/T) or 4 (N/T): the launch runs over the
    rounded K (an edge or tail split, no epilogue) and then over the last 2-4
    K rows onto that result (beta 1, the epilogue): alpha, beta, a per-row
    bias and ReLU, every element within the FP64 bound, repeats bit-identical."""
    from test_gpu_sgemm_device import run_device_gemm

    outs, ref, absab = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 811,
                                       alpha=0.75, beta=-1.25, bias_rows=True, relu=True,
                                       repeat=2)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"{m}x{n}x{k} {form} (K remainder): violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0
