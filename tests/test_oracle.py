"""Pins the CPU oracle before anything is checked against it.

- pattern values, closed-form sums and expected C: the reference's own KATs
  (tests/unit/gemm_pattern_tests.cpp:103-153), the answers of the reference's
  compiled pattern code recorded in tests/golden/reference_outputs.json, and,
  where the reference tree is mounted, that compiled code itself (oracle/_ref);
- the FP64 SGEMM: brute-force Python loops (bit-exact, same summation order),
  numpy float64 matmul, the analytic pattern (exact) for all N/T views, and the
  reference example's closed-form inputs (examples/preview-gemm/main.cpp:53-58);
- the bound: planted mistakes (a dropped term, a transposed operand, a wrong
  beta, a NaN) must fail it;
- the input generator: range/representability, determinism, and bit-identity
  with the product-side generator (xvram_amd/lib/libxvram_synth.so).
"""
import ctypes
import itertools
import os

import numpy as np
import pytest

import generators
import oracle


def test_pattern_kats():
    # tests/unit/gemm_pattern_tests.cpp:112-117
    assert oracle.pattern_a(0, 0) == 1
    assert oracle.pattern_a(2, 1) == 4
    assert oracle.pattern_a(4, 7) == 3
    assert oracle.pattern_b(0, 0) == 1
    assert oracle.pattern_b(5, 4) == 7
    assert oracle.pattern_b(8, 6) == 4
    # :140-143 and :152
    assert oracle.pattern_sums(32769) == (16384, 32769, 16384)
    assert oracle.pattern_expected(4, 6, 11) == 78


def test_pattern_sums_brute_force():
    for k in range(0, 301):
        p = sum(t % 2 for t in range(k))
        q = sum(t % 3 for t in range(k))
        pq = sum((t % 2) * (t % 3) for t in range(k))
        assert oracle.pattern_sums(k) == (p, q, pq), k


def test_pattern_expected_brute_force():
    for row, col, k in itertools.product(range(7), range(9), range(1, 24)):
        naive = sum(oracle.pattern_a(row, t) * oracle.pattern_b(t, col) for t in range(k))
        assert oracle.pattern_expected(row, col, k) == naive


def test_pattern_against_recorded_reference():
    """The reference's own pattern.cpp answers, recorded by tests/golden/make_golden.py."""
    pts = generators.pattern_points(1000, 7)
    want = generators.reference_outputs("pattern", pts)
    for (row, col, k), (a, b, expected, p, q, pq) in zip(pts, want):
        assert oracle.pattern_a(row, k) == a
        assert oracle.pattern_b(k, col) == b
        assert oracle.pattern_expected(row, col, k) == expected
        assert oracle.pattern_sums(k) == (p, q, pq)


def test_pattern_against_compiled_reference():
    ref = oracle.ref_lib()
    if ref is None:
        pytest.skip("reference pattern code not built here (oracle/_ref needs /root/reference)")
    out = ctypes.c_uint64()
    p, q, pq = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    for row, col, k in generators.pattern_points(2000, 7):
        assert ref.ref_pattern_a(row, k) == oracle.pattern_a(row, k)
        assert ref.ref_pattern_b(k, col) == oracle.pattern_b(k, col)
        assert ref.ref_pattern_expected(row, col, k, ctypes.byref(out)) == 1
        assert out.value == oracle.pattern_expected(row, col, k)
        ref.ref_pattern_sums(k, ctypes.byref(p), ctypes.byref(q), ctypes.byref(pq))
        assert (p.value, q.value, pq.value) == oracle.pattern_sums(k)


def _brute(a, b, alpha, beta, c0):
    m, k = a.shape
    n = b.shape[1]
    al, be = float(np.float32(alpha)), float(np.float32(beta))
    out = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            s = 0.0
            for t in range(k):
                s += float(a[i, t]) * float(b[t, j])
            out[i, j] = al * s + (be * float(c0[i, j]) if be != 0.0 else 0.0)
    return out


@pytest.mark.parametrize("order_a,order_b", [("F", "F"), ("C", "F"), ("F", "C"), ("C", "C")])
def test_sgemm_bit_exact_against_brute_force(order_a, order_b):
    rng = np.random.default_rng(1)
    m, n, k = 7, 5, 13
    a = np.asarray(rng.uniform(-1, 1, (m, k)), dtype=np.float32, order=order_a)
    b = np.asarray(rng.uniform(-1, 1, (k, n)), dtype=np.float32, order=order_b)
    c0 = np.asfortranarray(rng.uniform(-1, 1, (m, n)).astype(np.float32))
    for alpha, beta in [(1.0, 0.0), (1.5, 0.5), (-0.3, 2.0)]:
        ref, absab = oracle.sgemm_f64(a, b, alpha, beta, c0)
        assert np.array_equal(ref, _brute(a, b, alpha, beta, c0))
        want_abs = np.abs(np.float32(alpha)) * (np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64)))
        if beta:
            want_abs += np.abs(np.float32(beta) * c0.astype(np.float64))
        np.testing.assert_allclose(absab, want_abs, rtol=1e-13)


def test_sgemm_transposed_views_agree():
    """op(A) given as a transposed view of differently stored data gives
    identical results (the oracle reads logical elements through strides)."""
    rng = np.random.default_rng(2)
    a = np.asfortranarray(rng.uniform(-1, 1, (120, 90)).astype(np.float32))
    b = np.asfortranarray(rng.uniform(-1, 1, (90, 70)).astype(np.float32))
    r1, _ = oracle.sgemm_f64(a, b)
    r2, _ = oracle.sgemm_f64(np.ascontiguousarray(a.T).T, np.ascontiguousarray(b.T).T)
    assert np.array_equal(r1, r2)


def test_sgemm_against_numpy():
    rng = np.random.default_rng(3)
    a = np.asfortranarray(rng.uniform(-1, 1, (300, 257)).astype(np.float32))
    b = np.asfortranarray(rng.uniform(-1, 1, (257, 199)).astype(np.float32))
    ref, _ = oracle.sgemm_f64(a, b, 1.25)
    np.testing.assert_allclose(ref, 1.25 * (a.astype(np.float64) @ b.astype(np.float64)),
                               rtol=1e-12, atol=1e-12)


def test_column_range_matches_full():
    rng = np.random.default_rng(4)
    a = np.asfortranarray(rng.uniform(-1, 1, (64, 50)).astype(np.float32))
    b = np.asfortranarray(rng.uniform(-1, 1, (50, 40)).astype(np.float32))
    full, fa = oracle.sgemm_f64(a, b)
    part, pa = oracle.sgemm_f64(a, b, columns=(13, 29))
    assert np.array_equal(part, full[:, 13:29]) and np.array_equal(pa, fa[:, 13:29])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_sgemm_exact_on_pattern(ta, tb):
    m, n, k = 37, 29, 301
    i = np.arange(m)[:, None]
    p = np.arange(k)[None, :]
    a = (1 + i % 3 + p % 2).astype(np.float32)
    b = (1 + np.arange(n)[None, :] % 5 + np.arange(k)[:, None] % 3).astype(np.float32)
    a_view = np.ascontiguousarray(a.T).T if ta else np.asfortranarray(a)
    b_view = np.ascontiguousarray(b.T).T if tb else np.asfortranarray(b)
    ref, _ = oracle.sgemm_f64(a_view, b_view)
    assert np.array_equal(ref, oracle.pattern_expected_matrix(m, n, k))


def test_reference_example_inputs():
    """examples/preview-gemm/main.cpp:14-16,53-58: m=37 n=19 k=67 closed inputs;
    the FP32 rounding of the oracle passes the example's own tolerance."""
    m, n, k = 37, 19, 67
    a = np.array([[((r + 3 * c) % 17 - 8) / 16.0 for c in range(k)] for r in range(m)],
                 dtype=np.float32)
    b = np.array([[((2 * r + c) % 13 - 6) / 16.0 for c in range(n)] for r in range(k)],
                 dtype=np.float32)
    ref, absab = oracle.sgemm_f64(np.asfortranarray(a), np.asfortranarray(b))
    assert np.array_equal(ref, _brute(a, b, 1.0, 0.0, None))
    c32 = np.asfortranarray(ref.astype(np.float32))
    assert oracle.check_example_tolerance(c32, ref) == 0
    assert oracle.check_bound(c32, k, ref, absab)[0] == 0


def _random_problem(seed, m=64, n=48, k=64):
    rng = np.random.default_rng(seed)
    a = np.asfortranarray(rng.uniform(-1, 1, (m, k)).astype(np.float32))
    b = np.asfortranarray(rng.uniform(-1, 1, (k, n)).astype(np.float32))
    c0 = np.asfortranarray(rng.uniform(-1, 1, (m, n)).astype(np.float32))
    return a, b, c0


def test_bound_accepts_fp32_sequential_accumulation():
    a, b, c0 = _random_problem(5)
    ref, absab = oracle.sgemm_f64(a, b, 1.5, 0.5, c0)
    # A plain FP32 loop (the weakest accumulation order) is inside the bound.
    acc = np.zeros((a.shape[0], b.shape[1]), dtype=np.float32)
    for t in range(a.shape[1]):
        acc = acc + np.outer(a[:, t], b[t, :]).astype(np.float32)
    c = np.asfortranarray((np.float32(1.5) * acc + np.float32(0.5) * c0).astype(np.float32))
    assert oracle.check_bound(c, a.shape[1], ref, absab)[0] == 0


@pytest.mark.parametrize("mistake", ["dropped_term", "transposed_b", "wrong_beta", "nan"])
def test_bound_rejects_planted_mistakes(mistake):
    a, b, c0 = _random_problem(6)
    ref, absab = oracle.sgemm_f64(a, b, 1.5, 0.5, c0)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    if mistake == "dropped_term":
        wrong = 1.5 * (a64[:, :-1] @ b64[:-1, :]) + 0.5 * c0
    elif mistake == "transposed_b":
        bt = np.ascontiguousarray(b64[:, :].T)[: b.shape[0], : b.shape[1]] if b.shape[0] == b.shape[1] \
            else np.roll(b64, 1, axis=0)
        wrong = 1.5 * (a64 @ bt) + 0.5 * c0
    elif mistake == "wrong_beta":
        wrong = 1.5 * (a64 @ b64) + 1.0 * c0
    else:
        wrong = ref.copy()
        wrong[3, 4] = np.nan
    c = np.asfortranarray(wrong.astype(np.float32))
    assert oracle.check_bound(c, a.shape[1], ref, absab)[0] > 0


def test_uniform_generator():
    x = oracle.fill_uniform(1 << 16, 42)
    assert x.min() >= -1.0 and x.max() < 1.0
    assert np.array_equal(x, oracle.fill_uniform(1 << 16, 42))
    assert not np.array_equal(x, oracle.fill_uniform(1 << 16, 43))
    # multiples of 2^-23: exactly representable
    assert np.array_equal(np.round(x.astype(np.float64) * 2**23), x.astype(np.float64) * 2**23)
    # counters are positional: a window equals the same slice of a longer fill
    assert np.array_equal(oracle.fill_uniform(100, 42, first=1000), oracle.fill_uniform(1100, 42)[1000:])
    assert abs(float(x.mean())) < 0.02 and abs(float(x.var()) - 1 / 3) < 0.01


def test_normal_generator():
    x = oracle.fill_normal(1 << 18, 9, 0.5).astype(np.float64)
    assert abs(x.mean()) < 0.01 and abs(x.std() - 0.5) < 0.01


def test_product_generator_is_bit_identical():
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "xvram_amd",
                        "lib", "libxvram_synth.so")
    synth = ctypes.CDLL(path)
    fp = ctypes.POINTER(ctypes.c_float)
    u64 = ctypes.c_uint64
    synth.synth_fill_uniform.argtypes = [fp, u64, u64, u64]
    synth.synth_fill_normal.argtypes = [fp, u64, u64, u64, ctypes.c_double]
    synth.synth_fill_uniform_strided.argtypes = [fp, u64, u64, u64, u64, u64, u64]
    out = np.empty(4096, np.float32)
    synth.synth_fill_uniform(out.ctypes.data_as(fp), 4096, 5, 777)
    assert np.array_equal(out, oracle.fill_uniform(4096, 5, first=777))
    synth.synth_fill_normal(out.ctypes.data_as(fp), 4096, 6, 11, ctypes.c_double(0.25))
    assert np.array_equal(out, oracle.fill_normal(4096, 6, 0.25, first=11))
    # strided sample of a column-major 50 x 40 matrix: rows 3..12, columns 5..9
    full = oracle.fill_uniform(50 * 40, 8).reshape(40, 50).T
    blk = np.empty(10 * 5, np.float32)
    synth.synth_fill_uniform_strided(blk.ctypes.data_as(fp), 10, 5, 8, 3 + 5 * 50, 1, 50)
    assert np.array_equal(blk.reshape(5, 10).T, full[3:13, 5:10])


def test_product_pattern_fillers_match_the_oracle():
    """The product-side pattern fillers (used to build full-size pattern
    operands) against the oracle's restatement of pattern.cpp, for both
    storage forms of each operand and a column window that does not start at 0."""
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "xvram_amd",
                        "lib", "libxvram_synth.so")
    synth = ctypes.CDLL(path)
    fp = ctypes.POINTER(ctypes.c_float)
    u64 = ctypes.c_uint64
    for name in ("synth_fill_pattern_a", "synth_fill_pattern_b"):
        getattr(synth, name).argtypes = [fp, u64, u64, u64, ctypes.c_int]
    rows, cols, col0 = 37, 23, 1000
    for transposed in (0, 1):
        a = np.empty(rows * cols, np.float32)
        synth.synth_fill_pattern_a(a.ctypes.data_as(fp), rows, cols, col0, transposed)
        b = np.empty(rows * cols, np.float32)
        synth.synth_fill_pattern_b(b.ctypes.data_as(fp), rows, cols, col0, transposed)
        a, b = a.reshape(cols, rows).T, b.reshape(cols, rows).T  # stored (x, y - col0)
        for x in range(rows):
            for c in range(cols):
                y = col0 + c
                # stored N: A(i=x, k=y), B(k=x, j=y); stored T: A(i=y, k=x), B(k=y, j=x)
                want_a = oracle.pattern_a(y, x) if transposed else oracle.pattern_a(x, y)
                want_b = oracle.pattern_b(y, x) if transposed else oracle.pattern_b(x, y)
                assert a[x, c] == want_a and b[x, c] == want_b, (transposed, x, y)
