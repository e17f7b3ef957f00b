"""ctypes front end of ``build/libxvram_oracle.so`` (and of ``_ref/``).

Test infrastructure only (see ``xvram_oracle.c`` for what each function
restates and where the reference defines it).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libxvram_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libxvram_ref.so")

_i64 = ctypes.c_int64
_u64 = ctypes.c_uint64
_dbl = ctypes.c_double
_fp = ctypes.POINTER(ctypes.c_float)
_dp = ctypes.POINTER(ctypes.c_double)

_lib = None
_ref = None


def build(reference: bool = False) -> None:
    """Compile the oracle (and, if asked and present, the reference shim)."""
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)
    if reference:
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        l = ctypes.CDLL(LIB_PATH)
        l.oracle_sgemm_f64_columns.argtypes = [
            _i64, _i64, _i64, _dbl, _fp, _i64, _i64, _fp, _i64, _i64, _dbl, _fp, _i64, _i64,
            _dp, _dp, _i64, _i64, _i64, ctypes.c_int]
        l.oracle_sgemm_f64_columns.restype = None
        l.oracle_check_bound.argtypes = [_i64, _i64, _i64, _fp, _i64, _i64, _dp, _dp, _i64,
                                         _dp, _dp]
        l.oracle_check_bound.restype = _i64
        l.oracle_check_example_tolerance.argtypes = [_i64, _i64, _fp, _i64, _i64, _dp, _i64]
        l.oracle_check_example_tolerance.restype = _i64
        for name in ("oracle_pattern_a", "oracle_pattern_b"):
            getattr(l, name).argtypes = [_u64, _u64]
            getattr(l, name).restype = _u64
        l.oracle_pattern_expected.argtypes = [_u64, _u64, _u64]
        l.oracle_pattern_expected.restype = _u64
        l.oracle_pattern_sums.argtypes = [_u64, ctypes.POINTER(_u64), ctypes.POINTER(_u64),
                                          ctypes.POINTER(_u64)]
        l.oracle_fill_uniform.argtypes = [_fp, _u64, _u64, _u64]
        l.oracle_fill_uniform_strided.argtypes = [_fp, _u64, _u64, _u64, _u64, _u64, _u64]
        l.oracle_fill_normal.argtypes = [_fp, _u64, _u64, _u64, _dbl]
        _lib = l
    return _lib


def ref_lib():
    """The reference's own pattern/planner code, or None where it was not built."""
    global _ref
    if _ref is None and os.path.exists(REF_PATH):
        r = ctypes.CDLL(REF_PATH)
        r.ref_pattern_a.argtypes = [_u64, _u64]
        r.ref_pattern_a.restype = _u64
        r.ref_pattern_b.argtypes = [_u64, _u64]
        r.ref_pattern_b.restype = _u64
        r.ref_pattern_expected.argtypes = [_u64, _u64, _u64, ctypes.POINTER(_u64)]
        r.ref_pattern_expected.restype = ctypes.c_int
        r.ref_pattern_sums.argtypes = [_u64] + [ctypes.POINTER(_u64)] * 3
        r.ref_validate_problem.restype = ctypes.c_int
        _ref = r
    return _ref


def _f(a):
    return a.ctypes.data_as(_fp)


def _d(a):
    return a.ctypes.data_as(_dp)


def strides(arr: np.ndarray):
    """Element strides (row, column) of a 2-D float32 numpy view."""
    assert arr.dtype == np.float32
    return arr.strides[0] // 4, arr.strides[1] // 4


def sgemm_f64(a_op, b_op, alpha=1.0, beta=0.0, c0=None, threads=0, columns=None):
    """FP64 reference of alpha*a_op@b_op + beta*c0 over float32 operand views.

    ``a_op`` (m x k) and ``b_op`` (k x n) are the *operated* matrices (numpy
    views carrying the strides of the stored data, so N and T operands and
    row/column-major storage are all expressed by the view). Returns
    ``(ref, absab)`` float64 (m x n_cols) arrays in column-major order; with
    ``columns=(j0, j1)`` only that column range is computed.
    """
    m, k = a_op.shape
    k2, n = b_op.shape
    assert k == k2
    j0, j1 = (0, n) if columns is None else columns
    ref = np.empty((m, j1 - j0), dtype=np.float64, order="F")
    absab = np.empty_like(ref)
    ars, acs = strides(a_op)
    brs, bcs = strides(b_op)
    if c0 is not None and beta != 0.0:
        crs, ccs = strides(c0)
        cptr = _f(c0)
    else:
        crs = ccs = 0
        cptr = None
    lib().oracle_sgemm_f64_columns(m, n, k, alpha, _f(a_op), ars, acs, _f(b_op), brs, bcs, beta,
                                   cptr, crs, ccs, _d(ref), _d(absab), m, j0, j1, threads)
    return ref, absab


def check_bound(c, k, ref, absab):
    """(violations, max_abs_err, max_err/bound) for an FP32 result view ``c``."""
    m, n = ref.shape
    crs, ccs = strides(c)
    me = ctypes.c_double()
    mr = ctypes.c_double()
    bad = lib().oracle_check_bound(m, n, k, _f(c), crs, ccs, _d(ref), _d(absab), m,
                                   ctypes.byref(me), ctypes.byref(mr))
    return int(bad), me.value, mr.value


def check_example_tolerance(c, ref):
    m, n = ref.shape
    crs, ccs = strides(c)
    return int(lib().oracle_check_example_tolerance(m, n, _f(c), crs, ccs, _d(ref), m))


def pattern_a(row, k):
    return int(lib().oracle_pattern_a(row, k))


def pattern_b(k, col):
    return int(lib().oracle_pattern_b(k, col))


def pattern_expected(row, col, k):
    return int(lib().oracle_pattern_expected(row, col, k))


def pattern_sums(k):
    p, q, pq = _u64(), _u64(), _u64()
    lib().oracle_pattern_sums(k, ctypes.byref(p), ctypes.byref(q), ctypes.byref(pq))
    return p.value, q.value, pq.value


def pattern_expected_matrix(m, n, k):
    """Expected C (m x n, float64) of the analytic pattern, vectorised closed form."""
    sp, sq, spq = pattern_sums(k)
    a0 = 1 + (np.arange(m, dtype=np.int64) % 3)
    b0 = 1 + (np.arange(n, dtype=np.int64) % 5)
    return (k * np.outer(a0, b0) + np.outer(a0 * sq, np.ones(n, np.int64))
            + np.outer(np.ones(m, np.int64), b0 * sp) + spq).astype(np.float64)


def fill_uniform(count, seed, first=0):
    out = np.empty(count, dtype=np.float32)
    lib().oracle_fill_uniform(_f(out), count, seed, first)
    return out


def fill_uniform_strided(rows, cols, seed, first, row_stride, col_stride):
    """(rows x cols) Fortran array, element (r, c) = U(first + r*row_stride + c*col_stride)."""
    out = np.empty(rows * cols, dtype=np.float32)
    lib().oracle_fill_uniform_strided(_f(out), rows, cols, seed, first, row_stride, col_stride)
    return np.asfortranarray(out.reshape(cols, rows).T)


def fill_normal(count, seed, sigma, first=0):
    out = np.empty(count, dtype=np.float32)
    lib().oracle_fill_normal(_f(out), count, seed, first, sigma)
    return out
