"""Spread sample check of a large GEMM result against the FP64 oracle.

TEST INFRASTRUCTURE ONLY (used by tests/ and by bench.py's check after its
timed region). A full FP64 check of an out-of-core product (up to 5.6e14 FMA)
is out of reach on the host, so the result is checked on a sample chosen to
see every C tile: one full column inside every tile column, one full row
inside every tile row (so every tile row and every tile column of the plan's
C grid is covered, and a panel routed to the wrong C block changes whole
sampled lines), plus seeded random elements; every sampled element with its
full K reduction (oracle_sgemm_f64, the restatement of
examples/preview-gemm/main.cpp:107-119) against the per-element bound
4*K*2^-24*(|A||B|)_ij (oracle_check_bound; tolerance as
src/gemm_bench/executor.cpp:779-783 scaled to K).

Operands are seeded U[-1,1) matrices in the counter-based definition of
``oracle.fill_uniform`` (element counter = column-major storage index), so
the checker regenerates them independently of the product's copies.
"""
from __future__ import annotations

import numpy as np

from . import oracle as _o


class SeededOperand:
    """op(X) of a stored column-major matrix X (stored_rows x stored_cols) whose
    element (r, c) is U(seed, r + c*stored_rows); op T when ``transposed``."""

    def __init__(self, seed: int, stored_rows: int, stored_cols: int, transposed: bool):
        self.seed, self.sr, self.sc, self.t = seed, stored_rows, stored_cols, transposed
        self.shape = (stored_cols, stored_rows) if transposed else (stored_rows, stored_cols)

    def full(self) -> np.ndarray:
        """The whole operated matrix as a float32 view (stored once)."""
        flat = _o.fill_uniform(self.sr * self.sc, self.seed)
        stored = flat.reshape(self.sc, self.sr).T  # Fortran view of the stored matrix
        return stored.T if self.t else stored

    def rows(self, idx) -> np.ndarray:
        """Rows `idx` of op(X), (len(idx) x cols) Fortran."""
        cols = self.shape[1]
        out = np.empty((len(idx), cols), dtype=np.float32, order="F")
        for r, i in enumerate(idx):
            i = int(i)
            # op row i: stored row i (op N) or stored column i (op T).
            first, stride = (i * self.sr, 1) if self.t else (i, self.sr)
            out[r, :] = _o.fill_uniform_strided(1, cols, self.seed, first, 0, stride)[0]
        return out

    def cols(self, idx) -> np.ndarray:
        """Columns `idx` of op(X), (rows x len(idx)) Fortran."""
        rows = self.shape[0]
        out = np.empty((rows, len(idx)), dtype=np.float32, order="F")
        for c, j in enumerate(idx):
            j = int(j)
            first, stride = (j, self.sr) if self.t else (j * self.sr, 1)
            out[:, c] = _o.fill_uniform_strided(rows, 1, self.seed, first, stride, 0)[:, 0]
        return out


def spread_positions(m: int, n: int, tile_m: int, tile_n: int, seed: int = 0,
                     randoms: int = 1024):
    """One column per tile column, one row per tile row (at a seeded offset
    inside the tile), and `randoms` seeded random elements."""
    rng = np.random.default_rng(seed)
    cols = [t * tile_n + int(rng.integers(0, min(tile_n, n - t * tile_n)))
            for t in range(-(-n // tile_n))]
    rows = [t * tile_m + int(rng.integers(0, min(tile_m, m - t * tile_m)))
            for t in range(-(-m // tile_m))]
    ri = rng.integers(0, m, randoms)
    rj = rng.integers(0, n, randoms)
    return rows, cols, ri, rj


def spread_check(a: SeededOperand, b: SeededOperand, read_columns, tile_m: int, tile_n: int,
                 seed: int = 0, randoms: int = 1024, slab_bytes: int = 256 << 20,
                 threads: int = 0) -> dict:
    """Checks C = op(A) op(B) (alpha 1, beta 0) through ``read_columns(j0, j1)``,
    which returns C[:, j0:j1] as an (m x (j1-j0)) float32 array."""
    m, k = a.shape
    n = b.shape[1]
    rows, cols, ri, rj = spread_positions(m, n, tile_m, tile_n, seed, randoms)
    # References: full columns need all of op(A); full rows all of op(B)
    # (as C[rows, :]^T = op(B)^T op(A)[rows, :]^T); one operand at a time.
    a_full = a.full()
    ref_c, abs_c = _o.sgemm_f64(a_full, b.cols(cols), threads=threads)
    del a_full
    b_full = b.full()
    ref_r, abs_r = _o.sgemm_f64(b_full.T, np.asfortranarray(a.rows(rows).T), threads=threads)
    del b_full
    a_ri, b_rj = a.rows(ri), b.cols(rj)
    ref_e = np.empty(len(ri))
    abs_e = np.empty(len(ri))
    for e in range(len(ri)):
        r, s = _o.sgemm_f64(a_ri[e:e + 1, :], b_rj[:, e:e + 1])
        ref_e[e], abs_e[e] = r[0, 0], s[0, 0]
    # The product's values, read a slab of columns at a time.
    got_c = np.empty((m, len(cols)), dtype=np.float32, order="F")
    got_r = np.empty((len(rows), n), dtype=np.float32, order="F")
    got_e = np.empty(len(ri), dtype=np.float32)
    width = max(1, slab_bytes // (4 * m))
    col_at = {j: t for t, j in enumerate(cols)}
    for j0 in range(0, n, width):
        j1 = min(n, j0 + width)
        slab = read_columns(j0, j1)
        got_r[:, j0:j1] = slab[rows, :]
        for j in range(j0, j1):
            if j in col_at:
                got_c[:, col_at[j]] = slab[:, j - j0]
        hit = (rj >= j0) & (rj < j1)
        got_e[hit] = slab[ri[hit], rj[hit] - j0]
    bad_c, _, worst_c = _o.check_bound(got_c, k, ref_c, abs_c)
    bad_r, _, worst_r = _o.check_bound(np.asfortranarray(got_r.T), k, ref_r, abs_r)
    bad_e, _, worst_e = _o.check_bound(got_e.reshape(1, -1), k, ref_e.reshape(1, -1),
                                       abs_e.reshape(1, -1))
    elements = m * len(cols) + n * len(rows) + len(ri)
    return {"elements": int(elements), "violations": int(bad_c + bad_r + bad_e),
            "max_err_over_bound": float(max(worst_c, worst_r, worst_e)),
            "full_columns": [int(j) for j in cols], "full_rows": [int(i) for i in rows],
            "random_elements": int(len(ri)),
            "tile_grid": [-(-m // tile_m), -(-n // tile_n)]}
