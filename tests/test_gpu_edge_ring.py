"""Ragged launches on the ring kernels' edge instances and the thin-K kernel,
on the MI355X through the C ABI (the extension's sgemm_device on device
memory), against the oracle.

A launch of at least 256 tiles of 256 x 256 whose m or n is not a multiple of
256, whose K is a multiple of 4 (N/T) or 8 (the other forms) and whose edge
split would not run faster (kernels::edge_split_rated_faster: here one round
of 16 x 16 tiles) runs whole on the barrier-free ring kernels' edge
instances: a lane whose four elements would start past the operand's last
whole float4 loads that float4 instead, and the predicated store writes only
elements of C. The padding rows (columns) of every operand here hold NaN, so
a load that fed an element of C from past the operand's rows, columns or K
would show in C.

* 4001 x 3999 x 1024 (m and n not multiples of 4), all four forms, seeded
  U[-1,1) operands, alpha, beta, a per-row or per-column bias and ReLU: every
  element within the FP64 bound, and two executions bit-identical.
* 4001 x 4093 x 2048 and 3900 x 4096 x 1000, all four forms: the analytic
  pattern, every element bit-exact.
* A K remainder onto a whole launch: 4001 x 3999 x 1030 (K % 8 = 6, K % 4 =
  2), all four forms, alpha, beta, a per-row bias and ReLU: the rounded K on
  the edge instances, the last K rows on the thin-K kernel; within the bound.
* Thin-K launches (K = 1, 3 and 7; 1001 x 515: a partial row block and a
  partial group of columns), all four forms, alpha, beta, a per-column bias
  and ReLU: within the bound.
* The other kernels under the same NaN padding, whose predicated loads take
  out-of-range rows, columns and k as zeros in both operands (0 x NaN would
  be NaN): the general 256 x 256 kernel on 4001 x 3999 x 501 (edge tiles and
  a K tail; no K remainder below 512) and 4096^2 x 1001 (interior tiles, K
  tail), and the 256 x 128 kernel's split on config 2 (3001 x 2047 x 4099),
  all four forms: within the bound, no NaN.

Tolerance: |C - C_ref| <= 4*K*2^-24*(|alpha||A||B| + |beta C0| + |bias|)_ij."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_sgemm_device import FORMS, Hip, desc_for
from test_gpu_tail_split import pattern_stored, synth  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[edge-ring] {msg}", flush=True)


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.fixture()
def hip(lib):
    h = Hip()
    yield h
    h.close()


def nan_padded(mat):
    """Column-major storage (flat, ld) with ld rounded up to 4 floats and the
    padding rows set to NaN."""
    rows, cols = mat.shape
    ld = (rows + 3) // 4 * 4
    buf = np.full((cols, ld), np.nan, dtype=np.float32)
    buf[:, :rows] = mat.T
    return buf.reshape(-1), ld


def run_gemm(lib, hip, oracle_mod, m, n, k, form, seed, alpha, beta, axis, relu, repeat=2):
    ops = FORMS[form]
    a_op = np.asfortranarray(oracle_mod.fill_uniform(m * k, seed).reshape(k, m).T)
    b_op = np.asfortranarray(oracle_mod.fill_uniform(k * n, seed + 1).reshape(n, k).T)
    c0 = np.asfortranarray(oracle_mod.fill_uniform(m * n, seed + 2).reshape(n, m).T)
    length = m if axis == abi.BIAS_PER_ROW else n
    bias = (oracle_mod.fill_uniform(length, seed + 3) * 0.5).astype(np.float32)
    a_flat, lda = nan_padded(a_op if ops[0] == abi.OP_N else a_op.T)
    b_flat, ldb = nan_padded(b_op if ops[1] == abi.OP_N else b_op.T)
    c_flat, ldc = nan_padded(c0)
    pa, pb, pc = hip.alloc(a_flat.nbytes), hip.alloc(b_flat.nbytes), hip.alloc(c_flat.nbytes)
    pbias = hip.alloc(bias.nbytes)
    s = hip.stream()
    outs = []
    try:
        hip.put(pa, a_flat)
        hip.put(pb, b_flat)
        hip.put(pbias, bias)
        d = desc_for((pa, pb, pc), m, n, k, ops, (lda, ldb, ldc), alpha, beta, pbias, axis, relu)
        for _ in range(repeat):
            hip.put(pc, c_flat)
            assert lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(s)) == abi.SUCCESS
            hip.sync(s)
            outs.append(hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T)
    finally:
        for p in (pa, pb, pc, pbias):
            hip.free(p)
    ref, absab = oracle_mod.sgemm_f64(a_op, b_op, alpha, beta, c0)
    badd = bias[:, None] if axis == abi.BIAS_PER_ROW else bias[None, :]
    ref = ref + badd.astype(np.float64)
    if relu:
        ref = np.maximum(ref, 0.0)
    return outs, ref, absab + np.abs(badd)


def check(oracle_mod, outs, k, ref, absab, what):
    assert not np.isnan(outs[0]).any(), f"{what}: NaN from past the operands reached C"
    for o in outs[1:]:
        assert np.array_equal(outs[0].view(np.uint32), o.view(np.uint32))
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"{what}: violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0


@pytest.mark.parametrize("axis", [abi.BIAS_PER_ROW, abi.BIAS_PER_COLUMN], ids=["row", "col"])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_edge_ring_within_bound(lib, hip, oracle_mod, form, axis):
    m, n, k = 4001, 3999, 1024
    outs, ref, absab = run_gemm(lib, hip, oracle_mod, m, n, k, form, 901, 1.25, -0.5, axis, True)
    check(oracle_mod, outs, k, ref, absab,
          f"{m}x{n}x{k} {form} bias {'row' if axis == abi.BIAS_PER_ROW else 'col'} + ReLU")


@pytest.mark.parametrize("m,n,k", [(4001, 4093, 2048), (3900, 4096, 1000)], ids=["mn", "m"])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_edge_ring_pattern(lib, hip, synth, oracle_mod, form, m, n, k):
    ops = FORMS[form]
    a_st = pattern_stored(synth, "a", *((m, k) if ops[0] == abi.OP_N else (k, m)),
                          ops[0] == abi.OP_T)
    b_st = pattern_stored(synth, "b", *((k, n) if ops[1] == abi.OP_N else (n, k)),
                          ops[1] == abi.OP_T)
    a_flat, lda = nan_padded(a_st)
    b_flat, ldb = nan_padded(b_st)
    c_flat, ldc = nan_padded(np.zeros((m, n), np.float32))
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


@pytest.mark.parametrize("form", sorted(FORMS))
def test_k_remainder_onto_whole_launch(lib, hip, oracle_mod, form):
    m, n, k = 4001, 3999, 1030
    outs, ref, absab = run_gemm(lib, hip, oracle_mod, m, n, k, form, 911, 0.75, 1.5,
                                abi.BIAS_PER_ROW, True)
    check(oracle_mod, outs, k, ref, absab, f"{m}x{n}x{k} {form} (K remainder) bias row + ReLU")


@pytest.mark.parametrize("k", [1, 3, 7])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_thin_k_within_bound(lib, hip, oracle_mod, form, k):
    m, n = 1001, 515
    outs, ref, absab = run_gemm(lib, hip, oracle_mod, m, n, k, form, 921 + k, -1.5, 0.25,
                                abi.BIAS_PER_COLUMN, True)
    check(oracle_mod, outs, k, ref, absab, f"thin {m}x{n}x{k} {form} bias col + ReLU")


@pytest.mark.parametrize("m,n,k", [(4001, 3999, 501), (4096, 4096, 1001), (3001, 2047, 4099)],
                         ids=["wide-edge", "wide-ktail", "narrow-split"])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_other_kernels_ignore_nan_padding(lib, hip, oracle_mod, form, m, n, k):
    outs, ref, absab = run_gemm(lib, hip, oracle_mod, m, n, k, form, 931, 1.5, 0.5,
                                abi.BIAS_PER_COLUMN, False, repeat=1)
    check(oracle_mod, outs, k, ref, absab, f"{m}x{n}x{k} {form} under NaN padding")
