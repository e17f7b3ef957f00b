"""Shared helpers: build GEMM operands in any layout/operation, run them through
the C ABI, and read C back in logical form. Not a test module."""
from __future__ import annotations

import numpy as np

import xvram_amd as xv
from xvram_amd import abi


def storage(logical: np.ndarray, layout: int, ld_pad: int = 0):
    """Flat float32 storage of a logical r x c matrix and its leading dimension."""
    r, c = logical.shape
    if layout == abi.COLUMN_MAJOR:
        ld = r + ld_pad
        buf = np.zeros((c, ld), dtype=np.float32)
        buf[:, :r] = logical.T
    else:
        ld = c + ld_pad
        buf = np.zeros((r, ld), dtype=np.float32)
        buf[:, :c] = logical
    return buf.reshape(-1), ld


def logical_from_storage(flat: np.ndarray, rows: int, cols: int, ld: int, layout: int):
    if layout == abi.COLUMN_MAJOR:
        return flat.reshape(cols, ld)[:, :rows].T
    return flat.reshape(rows, ld)[:, :cols]


class Problem:
    """op(A) (m x k), op(B) (k x n), C0 (m x n) as logical float32 matrices."""

    def __init__(self, a_op, b_op, c0=None, op_a=abi.OP_N, op_b=abi.OP_N,
                 layouts=(abi.COLUMN_MAJOR,) * 3, alpha=1.0, beta=0.0, ld_pad=(0, 0, 0)):
        self.a_op, self.b_op = a_op, b_op
        self.m, self.k = a_op.shape
        self.n = b_op.shape[1]
        self.c0 = c0
        self.op_a, self.op_b = op_a, op_b
        self.layouts = layouts
        self.alpha, self.beta = alpha, beta
        self.ld_pad = ld_pad

    def run(self, session: xv.Session, c_fill=None, repeat: int = 1):
        a_stored = self.a_op if self.op_a == abi.OP_N else self.a_op.T
        b_stored = self.b_op if self.op_b == abi.OP_N else self.b_op.T
        a_flat, lda = storage(np.ascontiguousarray(a_stored), self.layouts[0], self.ld_pad[0])
        b_flat, ldb = storage(np.ascontiguousarray(b_stored), self.layouts[1], self.ld_pad[1])
        c_logical = self.c0 if self.c0 is not None else np.zeros((self.m, self.n), np.float32)
        c_flat, ldc = storage(c_logical, self.layouts[2], self.ld_pad[2])
        if c_fill is not None:
            c_flat[:] = c_fill
        a = session.allocation(a_flat.nbytes)
        b = session.allocation(b_flat.nbytes)
        c = session.allocation(c_flat.nbytes)
        a.write(a_flat)
        b.write(b_flat)
        c.write(c_flat)
        plan = xv.GemmPlan(
            session,
            xv.matrix(a, a_stored.shape[0], a_stored.shape[1], lda, self.layouts[0]),
            xv.matrix(b, b_stored.shape[0], b_stored.shape[1], ldb, self.layouts[1]),
            xv.matrix(c, self.m, self.n, ldc, self.layouts[2]),
            self.op_a, self.op_b, self.alpha, self.beta)
        self.plan_info = plan.info()
        for _ in range(repeat):
            plan.execute()
        out_flat = c.read(dtype=np.float32)
        plan.release()
        for h in (a, b, c):
            h.release()
        self.c_flat_out = out_flat
        return np.asfortranarray(logical_from_storage(out_flat, self.m, self.n, ldc,
                                                      self.layouts[2]))

    def reference(self, oracle, threads=0, columns=None):
        c0 = self.c0 if self.beta != 0.0 else None
        return oracle.sgemm_f64(np.asfortranarray(self.a_op), np.asfortranarray(self.b_op),
                                self.alpha, self.beta,
                                None if c0 is None else np.asfortranarray(c0), threads, columns)


def uniform(oracle, rows, cols, seed):
    """Seeded U[-1,1) logical matrix (element counter = column-major index)."""
    return np.asfortranarray(oracle.fill_uniform(rows * cols, seed).reshape(cols, rows).T)


def pattern_operands(m, n, k):
    """The reference bench's analytic operands: A(i,p) = 1 + i%3 + p%2,
    B(p,j) = 1 + j%5 + p%3 (src/gemm_bench/pattern.cpp:207-213)."""
    i = np.arange(m)[:, None]
    p = np.arange(k)[None, :]
    a = (1 + i % 3 + p % 2).astype(np.float32)
    p2 = np.arange(k)[:, None]
    j = np.arange(n)[None, :]
    b = (1 + j % 5 + p2 % 3).astype(np.float32)
    return np.asfortranarray(a), np.asfortranarray(b)
