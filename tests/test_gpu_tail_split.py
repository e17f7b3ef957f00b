"""Tail splits on the MI355X, through the C ABI, against the oracle.

A launch of at least 256 interior 256 x 256 tiles runs in rounds of one
workgroup per CU; when its last round would fill few CUs, it runs instead as a
head (whole tile rows, unsplit, in full rounds) and a tail (the remaining tile
rows, K split on the ring kernels; kernels::tail_split_shape):

* 4352 x 4096 x 1024 (17 x 16 tiles: a head of 16 rows, one round, and a tail
  of one row of 16 tiles in 5 ranges of 224), all four forms, seeded U[-1,1)
  operands with alpha, beta, a per-row bias (offset into the tail's rows) and
  ReLU: every element within the FP64 bound, and two executions
  bit-identical; with a workspace of the caller's exactly the size the tail
  wants: the same bits.
* 4608 x 4608 x 2048 (18 x 18 tiles: a head of 14 rows, a tail of 4 rows in 7
  ranges of 320, two rounds of the CUs, 126 MiB of partials) N/N and T/N: the
  analytic pattern, every element bit-exact.
* The 4352 x 4096 x 1024 launch in a session (resident, 256 MiB frames: the
  partials in one frame of the pool), N/N and N/T: the pattern, bit-exact.

Tolerance: |C - C_ref| <= 4*K*2^-24*(|alpha||A||B| + |beta C0| + |bias|)_ij."""
import ctypes
import os

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_sgemm_device import FORMS, Hip, desc_for, padded, run_device_gemm

pytestmark = pytest.mark.gpu

MiB = 1 << 20
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP = ctypes.POINTER(ctypes.c_float)


def log(msg):
    print(f"[tail-split] {msg}", flush=True)


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.fixture(scope="module")
def synth():
    s = ctypes.CDLL(os.path.join(ROOT, "xvram_amd", "lib", "libxvram_synth.so"))
    u64 = ctypes.c_uint64
    for name in ("synth_fill_pattern_a", "synth_fill_pattern_b"):
        getattr(s, name).argtypes = [FP, u64, u64, u64, ctypes.c_int]
    return s


@pytest.fixture()
def hip(lib):
    h = Hip()
    yield h
    h.close()


def pattern_stored(synth, which, rows, cols, transposed):
    """The analytic pattern operand as stored (rows x cols column-major)."""
    buf = np.empty(rows * cols, dtype=np.float32)
    getattr(synth, f"synth_fill_pattern_{which}")(buf.ctypes.data_as(FP), rows, cols, 0,
                                                  1 if transposed else 0)
    return buf.reshape(cols, rows).T


@pytest.mark.parametrize("form", sorted(FORMS))
def test_tail_split_within_bound_and_deterministic(lib, hip, oracle_mod, form):
    m, n, k = 4352, 4096, 1024
    outs, ref, absab = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 701,
                                       alpha=-0.5, beta=0.75, bias_rows=True, relu=True,
                                       repeat=2)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"{m}x{n}x{k} {form} + bias/ReLU: violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0
    if form == "NT":
        # Five partials of the tail's 256 x 4096 floats in a workspace of the caller's.
        mine, _, _ = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 701,
                                     alpha=-0.5, beta=0.75, bias_rows=True, relu=True,
                                     workspace_bytes=5 * 256 * 4096 * 4)
        assert np.array_equal(mine[0].view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("form", ["NN", "TN"])
def test_two_round_tail_pattern(lib, hip, synth, oracle_mod, form):
    m, n, k = 4608, 4608, 2048
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


@pytest.mark.parametrize("form", ["NN", "NT"])
def test_tail_split_in_a_session(lib, synth, oracle_mod, form):
    m, n, k = 4352, 4096, 1024
    ops = FORMS[form]
    a_shape = (m, k) if ops[0] == abi.OP_N else (k, m)
    b_shape = (k, n) if ops[1] == abi.OP_N else (n, k)
    s = xv.Session(lib, chunk_size_bytes=256 * MiB)
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
        assert info.maximum_working_set_bytes == 4 * 256 * MiB
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
