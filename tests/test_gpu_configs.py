"""BASELINE configs 3, 4 and 5 at their real sizes on the MI355X, through the C
ABI, against the FP64 oracle.

* Config 3, the resident sweep: {4096, 8192, 16384}^3 in N/N and N/T, seeded
  U[-1,1) operands, unrestricted budget with frames that hold whole operands
  (one launch). Checked on one full column in each of 16 column bands, one full
  row in each of 16 row bands and 1024 seeded random elements, each with its
  full K (oracle/sample.py); plus the analytic pattern at the same shapes,
  every element bit-exact. A repeated execution moves no bytes: C stays
  cached (dirty) between executions of the write-back cache.
* The same sweep's 8192^3 and 16384^3 under the reference's default session
  (64 MiB frames, automatic budget): tiled, the operands cached; the sample
  (one full column and row per 2048-wide band, two per 4096-wide tile) and the
  pattern.
* Config 4: 32768^3 N/T under a 2 GiB budget of 64 MiB frames, seeded U[-1,1):
  one full column per tile column, one full row per tile row of the plan's C
  grid, and 1024 random elements -- every C block of the out-of-core schedule
  is sampled (the pattern's mod-3/mod-5 structure cannot see a block routed
  to the wrong place); executed twice, each execution's H2D within the planned
  schedule's 20 GiB.
* Config 5: 8 x [Y = ReLU(X W^T + b)] with X 256 x 16384 ~ N(0,1), W 16384^2
  and b ~ N(0, 1/16384), 2 GiB budget of 64 MiB frames, the layers queued back
  to back. Each layer is checked against an FP64 forward of the input the GPU
  actually consumed, on 8 full batch rows and 16 full output columns, and the
  chain end to end against a pure FP64 forward.

Tolerance: |C - C_ref| <= 4*K*2^-24*(|A||B|)_ij (+|b| for the chain), the
FP32 bound of the north star; the pattern runs are exact."""
import ctypes
import os
import time

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi
from oracle.sample import SeededOperand, spread_check

pytestmark = pytest.mark.gpu

MiB, GiB = 1 << 20, 1 << 30
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP = ctypes.POINTER(ctypes.c_float)


def log(msg):
    print(f"[configs] {msg}", flush=True)


@pytest.fixture(scope="module")
def synth():
    lib = ctypes.CDLL(os.path.join(ROOT, "xvram_amd", "lib", "libxvram_synth.so"))
    u64 = ctypes.c_uint64
    lib.synth_fill_uniform.argtypes = [FP, u64, u64, u64]
    for name in ("synth_fill_pattern_a", "synth_fill_pattern_b"):
        getattr(lib, name).argtypes = [FP, u64, u64, u64, ctypes.c_int]
    return lib


@pytest.fixture(scope="module")
def lib():
    return xv.load()


def closed(s):
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps == t.set_access_calls
    assert t.physical_handles_created == t.physical_handles_released
    assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    s.release()


def fill_uniform(synth, alloc, elements, seed, chunk=256 * MiB):
    """The product-side generator (synth.c) writing U(seed, e) in storage order."""
    buf = np.empty(min(chunk, elements), dtype=np.float32)
    for e0 in range(0, elements, chunk):
        view = buf[:min(chunk, elements - e0)]
        synth.synth_fill_uniform(view.ctypes.data_as(FP), view.size, seed, e0)
        alloc.write(view, offset=e0 * 4)


def fill_pattern(alloc, filler, rows, cols, transposed, chunk_bytes=GiB):
    step = max(1, chunk_bytes // (rows * 4))
    buf = np.empty(rows * step, dtype=np.float32)
    for c0 in range(0, cols, step):
        n = min(step, cols - c0)
        view = buf[:rows * n]
        filler(view.ctypes.data_as(FP), rows, n, c0, transposed)
        alloc.write(view, offset=c0 * rows * 4)


def column_reader(c, m):
    def read(j0, j1):
        out = np.empty((j1 - j0) * m, dtype=np.float32)
        c.read_into(out, offset=j0 * m * 4)
        return out.reshape(j1 - j0, m).T
    return read


def operands(s, m, n, k, op_b):
    a_rows, a_cols = m, k                                   # A op N: stored m x k
    b_rows, b_cols = (k, n) if op_b == abi.OP_N else (n, k)
    a = s.allocation(m * k * 4)
    b = s.allocation(k * n * 4)
    c = s.allocation(m * n * 4)
    plan = xv.GemmPlan(s, xv.matrix(a, a_rows, a_cols, a_rows),
                       xv.matrix(b, b_rows, b_cols, b_rows), xv.matrix(c, m, n, m),
                       abi.OP_N, op_b)
    return a, b, c, plan, (b_rows, b_cols)


def run_op(plan):
    op = plan.submit()
    st, info = op.wait()
    assert st == abi.SUCCESS and info.result == abi.SUCCESS, op.error().message.decode()
    op.release()
    return info


C3 = [(size, frame, op_b) for size, frame in ((4096, 64 * MiB), (8192, 256 * MiB),
                                              (16384, 1024 * MiB))
      for op_b in (abi.OP_N, abi.OP_T)]
C3_IDS = [f"{size}_n{'nt'[op_b]}" for size, _, op_b in C3]


@pytest.mark.parametrize("size,frame,op_b", C3, ids=C3_IDS)
def test_c3_resident_random(lib, synth, size, frame, op_b):
    m = n = k = size
    s = xv.Session(lib, chunk_size_bytes=frame)
    try:
        a, b, c, plan, (b_rows, b_cols) = operands(s, m, n, k, op_b)
        assert plan.info().tile_count == 1  # resident: one launch
        fill_uniform(synth, a, m * k, 301)
        fill_uniform(synth, b, k * n, 302)
        first = run_op(plan)
        again = run_op(plan)
        assert first.bytes_d2h == 0 and again.bytes_d2h == 0 and again.bytes_h2d == 0
        t = time.perf_counter()
        band = size // 16  # 16 full columns and 16 full rows: first, middle and last bands
        res = spread_check(SeededOperand(301, m, k, False),
                           SeededOperand(302, b_rows, b_cols, op_b == abi.OP_T),
                           column_reader(c, m), band, band, seed=size + op_b, randoms=1024)
        log(f"C3 {size}^3 N{'NT'[op_b]}: {res['elements']} elements, violations "
            f"{res['violations']}, err/bound {res['max_err_over_bound']:.3e} "
            f"({time.perf_counter() - t:.1f} s)")
        assert res["elements"] >= 100000 and res["violations"] == 0
        plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("size,frame,op_b", C3, ids=C3_IDS)
def test_c3_resident_pattern_every_element(lib, synth, oracle_mod, size, frame, op_b):
    m = n = k = size
    s = xv.Session(lib, chunk_size_bytes=frame)
    try:
        a, b, c, plan, (b_rows, b_cols) = operands(s, m, n, k, op_b)
        fill_pattern(a, synth.synth_fill_pattern_a, m, k, 0)
        fill_pattern(b, synth.synth_fill_pattern_b, b_rows, b_cols, 1 if op_b == abi.OP_T else 0)
        run_op(plan)
        got = c.read(dtype=np.float32).reshape(n, m).T
        expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
        bad = int(np.count_nonzero(got != expect))
        log(f"C3 pattern {size}^3 N{'NT'[op_b]}: {m * n} elements, {bad} differ")
        assert bad == 0
        plan.release()
    finally:
        closed(s)


# The same sweep under the reference's default session (xvram.h:135-150:
# 64 MiB frames, cache_target_bytes 0 = free memory - headroom), as a drop-in
# caller that never tunes frames gets it: 8192^3 and 16384^3 are tiled into
# 4096 x 4096 C tiles with 4096-deep K panels (two per launch after the first
# pass), the operands stay cached, and a repeated execution moves no bytes.
C3_DEFAULT = [(size, op_b) for size in (8192, 16384) for op_b in (abi.OP_N, abi.OP_T)]
C3_DEFAULT_IDS = [f"{size}_n{'nt'[op_b]}" for size, op_b in C3_DEFAULT]


@pytest.mark.parametrize("size,op_b", C3_DEFAULT, ids=C3_DEFAULT_IDS)
def test_c3_default_session_random(lib, synth, size, op_b):
    m = n = k = size
    s = xv.Session(lib)  # XVRAM_SESSION_CONFIG_V1_INIT
    try:
        assert s.config.chunk_size_bytes == 64 * MiB and s.config.cache_target_bytes == 0
        a, b, c, plan, (b_rows, b_cols) = operands(s, m, n, k, op_b)
        info = plan.info()
        assert (info.tile_m, info.tile_n, info.tile_k) == (4096, 4096, 4096)
        assert info.tile_count == (size // 4096) ** 3
        fill_uniform(synth, a, m * k, 311)
        fill_uniform(synth, b, k * n, 312)
        run_op(plan)
        again = run_op(plan)
        assert again.bytes_h2d == 0 and again.bytes_d2h == 0  # resident: all hits
        t = time.perf_counter()
        res = spread_check(SeededOperand(311, m, k, False),
                           SeededOperand(312, b_rows, b_cols, op_b == abi.OP_T),
                           column_reader(c, m), 2048, 2048, seed=size + 7 + op_b, randoms=1024)
        log(f"C3 default session {size}^3 N{'NT'[op_b]}: {res['elements']} elements, "
            f"violations {res['violations']}, err/bound {res['max_err_over_bound']:.3e} "
            f"({time.perf_counter() - t:.1f} s)")
        assert res["elements"] >= 50000 and res["violations"] == 0
        plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("size,op_b", C3_DEFAULT, ids=C3_DEFAULT_IDS)
def test_c3_default_session_pattern_every_element(lib, synth, oracle_mod, size, op_b):
    m = n = k = size
    s = xv.Session(lib)
    try:
        a, b, c, plan, (b_rows, b_cols) = operands(s, m, n, k, op_b)
        fill_pattern(a, synth.synth_fill_pattern_a, m, k, 0)
        fill_pattern(b, synth.synth_fill_pattern_b, b_rows, b_cols, 1 if op_b == abi.OP_T else 0)
        run_op(plan)
        got = c.read(dtype=np.float32).reshape(n, m).T
        expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
        bad = int(np.count_nonzero(got != expect))
        log(f"C3 default session pattern {size}^3 N{'NT'[op_b]}: {m * n} elements, {bad} differ")
        assert bad == 0
        plan.release()
    finally:
        closed(s)


def test_c4_random_every_block_sampled(lib, synth):
    m = n = k = 32768
    budget = 2 * GiB
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=budget)
    try:
        a, b, c, plan, (b_rows, b_cols) = operands(s, m, n, k, abi.OP_T)
        info = plan.info()
        t = time.perf_counter()
        fill_uniform(synth, a, m * k, 401)
        fill_uniform(synth, b, k * n, 402)
        log(f"C4 operands ready ({time.perf_counter() - t:.1f} s); plan {info.tile_m}x"
            f"{info.tile_n}x{info.tile_k}, {info.tile_count} launches")
        # Twice: the second execution starts from the first one's cache (its
        # last block's C tiles dirty), where a budget this tight once made the
        # schedule evict panels before their last use. Either way the H2D
        # stays within the planned schedule's: 3 C-block rows x |B| + 2 C-block
        # columns x |A| = 20 GiB.
        for run in range(2):
            t0 = s.telemetry()
            t = time.perf_counter()
            run_op(plan)
            secs = time.perf_counter() - t
            t1 = s.telemetry()
            h2d = t1.bytes_h2d - t0.bytes_h2d
            log(f"C4 execution {run}: {secs:.3f} s ({2.0 * m * n * k / secs / 1e12:.1f} TFLOP/s), "
                f"H2D {h2d / 1e9:.2f} GB")
            assert 3 * budget < h2d <= 20 * GiB  # genuinely out of core, no re-loads
        t = time.perf_counter()
        res = spread_check(SeededOperand(401, m, k, False), SeededOperand(402, n, k, True),
                           column_reader(c, m), info.tile_m, info.tile_n, seed=4, randoms=1024)
        log(f"C4 sample: {res['elements']} elements over the {res['tile_grid']} tile grid, "
            f"violations {res['violations']}, err/bound {res['max_err_over_bound']:.3e} "
            f"({time.perf_counter() - t:.1f} s)")
        assert res["tile_grid"] == [m // info.tile_m, n // info.tile_n]
        assert len(res["full_columns"]) == n // info.tile_n
        assert len(res["full_rows"]) == m // info.tile_m
        assert res["elements"] >= 100000 and res["violations"] == 0
        plan.release()
    finally:
        closed(s)


def test_c5_chain_full_size(lib, oracle_mod):
    layers, batch, width = 8, 256, 16384
    std = width ** -0.5
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=2 * GiB)
    try:
        t = time.perf_counter()
        acts = [s.allocation(batch * width * 4) for _ in range(layers + 1)]
        x0 = oracle_mod.fill_normal(batch * width, 5100, 1.0).reshape(batch, width)
        acts[0].write(x0)
        weights, biases, plans = [], [], []
        for l in range(layers):
            w = oracle_mod.fill_normal(width * width, 5200 + l, std)
            bvec = oracle_mod.fill_normal(width, 5300 + l, std)
            W, Bv = s.allocation(w.nbytes), s.allocation(bvec.nbytes)
            W.write(w)
            Bv.write(bvec)
            weights.append(w.reshape(width, width))  # row-major: out x in
            biases.append(bvec)
            plans.append(xv.GemmPlan(
                s, xv.matrix(acts[l], batch, width, width, abi.ROW_MAJOR),
                xv.matrix(W, width, width, width, abi.ROW_MAJOR),
                xv.matrix(acts[l + 1], batch, width, width, abi.ROW_MAJOR), abi.OP_N, abi.OP_T,
                epilogue=xv.epilogue(Bv, abi.BIAS_PER_COLUMN, relu=True)))
        log(f"C5 chain ready ({time.perf_counter() - t:.1f} s)")
        t0 = s.telemetry()
        t = time.perf_counter()
        ops = [p.submit() for p in plans]  # queued back to back
        for op in ops:
            st, info = op.wait()
            assert st == abi.SUCCESS and info.result == abi.SUCCESS, op.error().message.decode()
            op.release()
        secs = time.perf_counter() - t
        t1 = s.telemetry()
        h2d = t1.bytes_h2d - t0.bytes_h2d
        log(f"C5 forward {secs * 1e3:.1f} ms, H2D {h2d / 1e9:.2f} GB")
        assert h2d >= layers * width * width * 4  # every weight streamed
        ys = [a.read(dtype=np.float32).reshape(batch, width) for a in acts]
        for p in plans:
            p.release()
    finally:
        closed(s)

    rows = list(range(8))
    cols = sorted(np.random.default_rng(55).choice(width, 16, replace=False).tolist())
    factor = 4 * width * 2.0 ** -24
    worst = 0.0
    for l in range(layers):
        xin = ys[l]                   # the FP32 input this layer consumed
        wt = weights[l].T             # (in x out) view of the row-major weights: op T
        # 8 full batch rows: Y[rows, :] = ReLU(X[rows, :] W^T + b).
        x_rows = np.asfortranarray(xin[rows, :])
        bias_rows = np.asfortranarray(np.broadcast_to(biases[l], (len(rows), width)))
        ref, absab = oracle_mod.sgemm_f64(x_rows, wt, 1.0, 1.0, bias_rows)
        bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(ys[l + 1][rows, :]), width,
                                               np.asfortranarray(np.maximum(ref, 0.0)), absab)
        assert bad == 0, (l, "rows", ratio)
        worst = max(worst, ratio)
        # 16 full output columns over the whole batch.
        w_cols = np.asfortranarray(wt[:, cols])
        bias_cols = np.asfortranarray(np.broadcast_to(biases[l][cols], (batch, len(cols))))
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(xin), w_cols, 1.0, 1.0, bias_cols)
        got = np.asfortranarray(ys[l + 1][:, cols])
        bad, _, ratio = oracle_mod.check_bound(got, width, np.asfortranarray(np.maximum(ref, 0.0)),
                                               absab)
        assert bad == 0, (l, "columns", ratio)
        worst = max(worst, ratio)
        assert factor > 0
    # End to end on the sampled rows against a pure FP64 forward.
    y = x0[rows, :].astype(np.float64)
    for l in range(layers):
        y = np.maximum(y @ weights[l].astype(np.float64).T + biases[l], 0.0)
    rel = float(np.abs(ys[-1][rows, :] - y).max() / np.abs(y).max())
    log(f"C5 per-layer worst err/bound {worst:.3e}; end to end max|Y - Y64|/max|Y64| = {rel:.3e}")
    assert rel < 1e-4
