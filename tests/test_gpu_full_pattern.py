"""Every element of the benchmark GEMMs at their real shapes, bit-exact.

The analytic pattern of the reference's GEMM benchmark (A(i,k) = 1 + i%3 +
k%2, B(k,j) = 1 + j%5 + k%3; src/gemm_bench/pattern.cpp:207-237) keeps every
partial sum an integer below 2^24 for K = 65536 (at most 28 * K), so the FP32
product is exact in any summation order and C(i,j) depends only on (i%3, j%5):
the oracle's closed form gives the 15 values. The operands are built at full
size in pinned host memory (the product-side pattern fillers, themselves
checked against the oracle on the CPU), the GEMM runs once through the C ABI
with the benchmark's budget, frames and N/T operands, and all of C is read back
and compared -- every element of the north-star 65536^3 product out of core, and
of config 4's 32768^3 product under a 2 GiB budget.

The pattern repeats with period 3 in rows and 5 in columns, so with 8192-wide
tiles a C block routed between tile rows t and t+3 (or tile columns t and
t+5) would still match it. The north-star product is therefore also run on
seeded U[-1,1) operands and checked against the FP64 oracle on one full
column in every tile column, one full row in every tile row and 1024 random
elements, each with its full K (oracle/sample.py), within
|C - C_ref| <= 4*K*2^-24*(|A||B|)_ij (src/gemm_bench/executor.cpp:779-843
checks the reference's runs the same way, on a sample)."""
import ctypes
import os
import time

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

pytestmark = pytest.mark.gpu

MiB, GiB = 1 << 20, 1 << 30
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def log(msg):
    print(f"[full-pattern] {msg}", flush=True)


@pytest.fixture(scope="module")
def synth():
    lib = ctypes.CDLL(os.path.join(ROOT, "xvram_amd", "lib", "libxvram_synth.so"))
    fp = ctypes.POINTER(ctypes.c_float)
    for name in ("synth_fill_pattern_a", "synth_fill_pattern_b"):
        getattr(lib, name).argtypes = [fp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                       ctypes.c_int]
    lib.synth_fill_uniform.argtypes = [fp, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
    return lib


def fill(alloc, filler, rows, cols, transposed, chunk_bytes=GiB):
    step = max(1, chunk_bytes // (rows * 4))
    buf = np.empty(rows * step, dtype=np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    for c0 in range(0, cols, step):
        n = min(step, cols - c0)
        view = buf[:rows * n]
        filler(view.ctypes.data_as(fp), rows, n, c0, transposed)
        alloc.write(view, offset=c0 * rows * 4)


@pytest.mark.parametrize("size,budget,frame", [(65536, 16 * GiB, 1024 * MiB),
                                               (32768, 2 * GiB, 64 * MiB)],
                         ids=["ns65536_nt_16g", "c4_32768_nt_2g"])
def test_every_element_of_the_pattern_product(synth, oracle_mod, size, budget, frame):
    m = n = k = size
    assert 28 * k < (1 << 24)
    lib = xv.load()
    s = xv.Session(lib, chunk_size_bytes=frame, cache_target_bytes=budget)
    try:
        t = time.perf_counter()
        a = s.allocation(m * k * 4)          # A, op N: stored m x k
        b = s.allocation(n * k * 4)          # B, op T: stored n x k
        c = s.allocation(m * n * 4)
        fill(a, synth.synth_fill_pattern_a, m, k, 0)
        fill(b, synth.synth_fill_pattern_b, n, k, 1)
        log(f"{size}^3: operands built ({time.perf_counter() - t:.1f} s)")
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, n, k, n), xv.matrix(c, m, n, m),
                           abi.OP_N, abi.OP_T)
        info = plan.info()
        t0 = s.telemetry()
        t = time.perf_counter()
        plan.execute()
        secs = time.perf_counter() - t
        t1 = s.telemetry()
        log(f"{size}^3: executed {info.tile_count} launches of {info.tile_m}x{info.tile_n}x"
            f"{info.tile_k} in {secs:.2f} s ({2.0 * m * n * k / secs / 1e12:.1f} TFLOP/s), "
            f"H2D {(t1.bytes_h2d - t0.bytes_h2d) / 1e9:.1f} GB, evictions "
            f"{t1.clean_evictions - t0.clean_evictions}+{t1.dirty_evictions - t0.dirty_evictions}")
        assert t1.bytes_h2d - t0.bytes_h2d > 3 * budget  # genuinely out of core
        plan.release()

        # Expected column for each j % 5 class: rows repeat with period 3.
        vals = np.array([[oracle_mod.pattern_expected(r, q, k) for q in range(5)] for r in range(3)],
                        dtype=np.float64)
        assert np.all(vals == vals.astype(np.float32))
        expect = np.stack([np.resize(vals[:, q].astype(np.float32), m) for q in range(5)])
        t = time.perf_counter()
        step = max(1, GiB // (m * 4))
        buf = np.empty(m * step, dtype=np.float32)
        bad = compared = 0
        for j0 in range(0, n, step):
            cols = min(step, n - j0)
            view = c.read_into(buf[:m * cols], offset=j0 * m * 4).reshape(cols, m)
            for q in range(5):
                first = (q - j0) % 5
                block = view[first::5]
                compared += block.size
                if block.shape[0] and not np.array_equal(block, np.broadcast_to(expect[q], block.shape)):
                    wrong = block != expect[q]
                    bad += int(wrong.sum())
                    jj, ii = np.argwhere(wrong)[0]
                    log(f"mismatch at C[{ii}, {j0 + first + 5 * jj}]: {block[jj, ii]} vs "
                        f"{expect[q][ii]}")
        log(f"{size}^3: {compared} of {m * n} elements compared ({time.perf_counter() - t:.1f} s), "
            f"{bad} differ")
        assert compared == m * n and bad == 0
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps and t.physical_handles_created == t.physical_handles_released
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        s.release()


def test_north_star_random_every_tile_row_and_column_sampled(synth):
    from oracle.sample import SeededOperand, spread_check

    m = n = k = 65536
    budget, frame = 16 * GiB, 1024 * MiB
    lib = xv.load()
    s = xv.Session(lib, chunk_size_bytes=frame, cache_target_bytes=budget)
    fp = ctypes.POINTER(ctypes.c_float)
    try:
        t = time.perf_counter()
        a = s.allocation(m * k * 4)          # A, op N: stored m x k
        b = s.allocation(n * k * 4)          # B, op T: stored n x k
        c = s.allocation(m * n * 4)
        buf = np.empty(GiB // 4, dtype=np.float32)
        for alloc, seed in ((a, 11), (b, 12)):
            for e0 in range(0, m * k, buf.size):
                synth.synth_fill_uniform(buf.ctypes.data_as(fp), buf.size, seed, e0)
                alloc.write(buf, offset=e0 * 4)
        log(f"{m}^3 random: operands built ({time.perf_counter() - t:.1f} s)")
        plan = xv.GemmPlan(s, xv.matrix(a, m, k, m), xv.matrix(b, n, k, n), xv.matrix(c, m, n, m),
                           abi.OP_N, abi.OP_T)
        info = plan.info()
        assert (info.tile_m, info.tile_n) == (8192, 8192)
        t = time.perf_counter()
        plan.execute()
        log(f"{m}^3 random: executed in {time.perf_counter() - t:.2f} s")
        plan.release()

        def read_columns(j0, j1):
            out = np.empty((j1 - j0) * m, dtype=np.float32)
            c.read_into(out, offset=j0 * m * 4)
            return out.reshape(j1 - j0, m).T

        t = time.perf_counter()
        res = spread_check(SeededOperand(11, m, k, False), SeededOperand(12, n, k, True),
                           read_columns, info.tile_m, info.tile_n, seed=65536, randoms=1024)
        log(f"{m}^3 random: {res['elements']} elements checked ({time.perf_counter() - t:.1f} s): "
            f"columns {res['full_columns']}, rows {res['full_rows']}, violations "
            f"{res['violations']}, err/bound {res['max_err_over_bound']:.3e}")
        assert len(res["full_columns"]) == m // info.tile_n
        assert len(res["full_rows"]) == m // info.tile_m
        assert res["violations"] == 0
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps and t.physical_handles_created == t.physical_handles_released
        s.release()
