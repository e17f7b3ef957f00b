"""The reference planner's large-K regression fixture on the MI355X, through
the C ABI: 2049 x 2049 x 32769 with every matrix row-major, 64 MiB frames, a
384 MiB target and a 4 MiB workspace cap (tests/unit/gemm_planner_tests.cpp:
265-300). The panel planner runs it as 2049 x 2049 C tiles over nine K panels
of 4096 (the last one 1 deep), out of core: A and B (256 MiB each) stream
through five frames, one of which holds the split-K partials of the ragged
2049 x 2049 x 4096 launches (256 x 128 kernel, 3 ranges). Seeded U[-1,1)
operands; C checked against the FP64 oracle on one full column per 256
columns, one full row per 256 rows and 1024 random elements, every one with
its full K, within |C - C_ref| <= 4*K*2^-24*(|A||B|)_ij."""
import ctypes
import os

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi
from oracle.sample import SeededOperand, spread_check

pytestmark = pytest.mark.gpu

MiB = 1 << 20
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP = ctypes.POINTER(ctypes.c_float)


def log(msg):
    print(f"[large-k] {msg}", flush=True)


@pytest.fixture(scope="module")
def synth():
    lib = ctypes.CDLL(os.path.join(ROOT, "xvram_amd", "lib", "libxvram_synth.so"))
    lib.synth_fill_uniform.argtypes = [FP, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64]
    return lib


def test_reference_large_k_fixture(synth):
    m = n = 2049
    k = 32769
    lib = xv.load()
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=384 * MiB,
                   workspace_cap_bytes=4 * MiB)
    try:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        for alloc, count, seed in ((A, m * k, 701), (B, k * n, 702)):
            buf = np.empty(count, dtype=np.float32)
            synth.synth_fill_uniform(buf.ctypes.data_as(FP), count, seed, 0)
            alloc.write(buf)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, k, abi.ROW_MAJOR),
                           xv.matrix(B, k, n, n, abi.ROW_MAJOR),
                           xv.matrix(C, m, n, n, abi.ROW_MAJOR))
        info = plan.info()
        assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (2049, 2049, 4096, 9)
        t0 = s.telemetry()
        op = plan.submit()
        st, oi = op.wait()
        assert st == abi.SUCCESS and oi.result == abi.SUCCESS, op.error().message.decode()
        op.release()
        h2d = s.telemetry().bytes_h2d - t0.bytes_h2d
        # Row-major C (m x n) is the column-major storage of C^T.
        c = C.read(dtype=np.float32).reshape(m, n)
        # Row-major A (m x k, ld k) is the column-major storage of A^T (k x m):
        # op(A) = its transpose; likewise B.
        res = spread_check(SeededOperand(701, k, m, True), SeededOperand(702, n, k, True),
                           lambda j0, j1: np.asfortranarray(c[:, j0:j1]), 256, 256, seed=7,
                           randoms=1024)
        log(f"{m}x{n}x{k} row-major, 384 MiB: H2D {h2d / MiB:.0f} MiB, {res['elements']} "
            f"elements, violations {res['violations']}, err/bound {res['max_err_over_bound']:.3e}")
        assert h2d >= (m * k + k * n) * 4
        assert res["elements"] >= 35000 and res["violations"] == 0
        plan.release()
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps and t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        assert t.physical_handles_created == t.physical_handles_released
        s.release()
