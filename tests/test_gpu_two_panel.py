"""Launches over two K panels on the MI355X, through the C ABI.

A 4096 x 4096 x 16384 product under 64 MiB frames plans 4096 x 4096 x 4096
tiles, four K panels per C tile, two panels per launch (the two-panel
barrier-free kernels: one C-tile read and write per two panels; N/T runs
sgemm_ring_kernel, the other forms sgemm_ring8_kernel). The first K
pass runs as two one-panel launches (the operation's first pass is
link-bound), the first of them as two 2048-deep slices waiting for their
panels slice by slice; the last launch is one two-panel dispatch (beta 1 over
the first pass's C, then the epilogue). A repeated execution finds every panel
cached and runs the same dispatches.

* Analytic pattern, every element bit for bit (exact in FP32: 28 * 16384 <
  2^24) -- a panel routed to the wrong half of the launch, a skipped panel or
  a wrong k_split changes whole columns.
* Seeded U[-1,1) with alpha = -0.75, beta = 0.5, per-column bias and ReLU,
  executed twice (C1 = act(alpha A B + beta C0 + b), C2 from C1), each checked
  against the FP64 oracle on 16 full columns and 16 full rows (one at a seeded
  offset in each sixteenth of C) with the bound |C - C_ref| <=
  4*K*2^-24*(|alpha||A||B| + |beta C| + |b|)."""
import json

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_configs import FP, closed, fill_pattern, fill_uniform, synth  # noqa: F401

pytestmark = pytest.mark.gpu

MiB = 1 << 20
M = N = 4096
K = 16384


def log(msg):
    print(f"[two-panel] {msg}", flush=True)


@pytest.fixture()
def traced(tmp_path, monkeypatch):
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("XVRAM_TRACE_FILE", str(trace))
    return trace


def kernels(trace):
    return [len(json.loads(line)["kernels"]) for line in open(trace)]


def session(lib):
    return xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=16 * 64 * MiB)


OPS = {"NT": (abi.OP_N, abi.OP_T), "NN": (abi.OP_N, abi.OP_N), "TN": (abi.OP_T, abi.OP_N),
       "TT": (abi.OP_T, abi.OP_T)}


def pattern_plan(s, synth, ops, k):
    """A (op(A) M x k) and B (op(B) k x N) filled with the analytic pattern,
    stored for `ops` (column-major); C M x N."""
    a, b, c = s.allocation(M * k * 4), s.allocation(N * k * 4), s.allocation(M * N * 4)
    a_t, b_t = ops[0] == abi.OP_T, ops[1] == abi.OP_T
    fill_pattern(a, synth.synth_fill_pattern_a, k if a_t else M, M if a_t else k, int(a_t))
    fill_pattern(b, synth.synth_fill_pattern_b, N if b_t else k, k if b_t else N, int(b_t))
    am = xv.matrix(a, k, M, k) if a_t else xv.matrix(a, M, k, M)
    bm = xv.matrix(b, N, k, N) if b_t else xv.matrix(b, k, N, k)
    return xv.GemmPlan(s, am, bm, xv.matrix(c, M, N, M), ops[0], ops[1]), c


@pytest.mark.parametrize("form", list(OPS))
def test_two_panel_pattern_every_element(traced, synth, oracle_mod, form):
    """Every form: N/T runs sgemm_ring_kernel<true>, the others the two-panel
    instance of sgemm_ring8_kernel."""
    lib = xv.load()
    s = session(lib)
    try:
        plan, c = pattern_plan(s, synth, OPS[form], K)
        info = plan.info()
        log(f"{form}: plan {info.tile_m}x{info.tile_n}x{info.tile_k}, {info.tile_count} tiles, "
            f"working set {info.maximum_working_set_bytes >> 20} MiB")
        assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (4096, 4096, 4096, 4)
        assert info.maximum_working_set_bytes == 5 * 64 * MiB  # two panels per launch
        expect = oracle_mod.pattern_expected_matrix(M, N, K).astype(np.float32)
        for run in range(2):
            plan.execute()
            got = c.read(dtype=np.float32).reshape(N, M).T
            bad = int(np.count_nonzero(got != expect))
            log(f"{form} execution {run}: {bad} elements differ; kernels {kernels(traced)}")
            assert bad == 0
        assert kernels(traced) == [4, 4]  # 2 slices + 1 + one two-panel dispatch, each time
        plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("form", ["NT", "NN"])
def test_two_panel_ragged_second_panel(traced, synth, oracle_mod, form):
    """K = 14336: panels 4096, 4096, 4096, 2048; after the first pass's two
    one-panel launches, the last launch pairs a 4096-deep panel with the
    2048-deep one: for N/T one two-panel dispatch (k_split 4096, k 6144); for
    N/N, whose B panels hold K inside their lines, the two panels' leading
    dimensions differ and the launch runs one dispatch per panel."""
    k = 14336
    lib = xv.load()
    s = session(lib)
    try:
        plan, c = pattern_plan(s, synth, OPS[form], k)
        info = plan.info()
        assert (info.tile_k, info.tile_count) == (4096, 4)
        plan.execute()
        got = c.read(dtype=np.float32).reshape(N, M).T
        expect = oracle_mod.pattern_expected_matrix(M, N, k).astype(np.float32)
        bad = int(np.count_nonzero(got != expect))
        log(f"{form} ragged second panel: {bad} elements differ; kernels {kernels(traced)}")
        assert bad == 0
        assert kernels(traced) == ([4] if form == "NT" else [5])
        plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("form", ["NT", "NN"])
def test_two_panel_alpha_beta_epilogue(traced, synth, oracle_mod, form):
    from oracle.sample import SeededOperand

    b_t = form == "NT"

    lib = xv.load()
    s = session(lib)
    rng = np.random.default_rng(5)
    try:
        a, b, c = s.allocation(M * K * 4), s.allocation(N * K * 4), s.allocation(M * N * 4)
        fill_uniform(synth, a, M * K, 501)
        fill_uniform(synth, b, N * K, 502)
        fill_uniform(synth, c, M * N, 503)
        bias = (oracle_mod.fill_uniform(N, 504) * 0.5).astype(np.float32)
        v = s.allocation(N * 4)
        v.write(bias)
        alpha, beta = -0.75, 0.5
        bm = xv.matrix(b, N, K, N) if b_t else xv.matrix(b, K, N, K)
        plan = xv.GemmPlan(s, xv.matrix(a, M, K, M), bm, xv.matrix(c, M, N, M),
                           abi.OP_N, OPS[form][1], alpha, beta,
                           epilogue=xv.epilogue(v, abi.BIAS_PER_COLUMN, relu=True))
        A = SeededOperand(501, M, K, False).full().astype(np.float64)   # M x K
        B = (SeededOperand(502, N, K, True) if b_t else SeededOperand(502, K, N, False)) \
            .full().astype(np.float64)                                   # K x N
        prev = c.read(dtype=np.float32).reshape(N, M).T.astype(np.float64)
        cols = np.arange(16) * (N // 16) + rng.integers(0, N // 16, 16)
        rows = np.arange(16) * (M // 16) + rng.integers(0, M // 16, 16)
        for run in range(2):
            plan.execute()
            got = c.read(dtype=np.float32).reshape(N, M).T.astype(np.float64)
            worst, violations = 0.0, 0
            for sel_r, sel_c in ((slice(None), cols), (rows, slice(None))):
                ab = A[sel_r] @ B[:, sel_c]
                absab = np.abs(A[sel_r]) @ np.abs(B[:, sel_c])
                ref = np.maximum(alpha * ab + beta * prev[sel_r][:, sel_c] + bias[sel_c], 0.0)
                bound = 4 * K * 2.0 ** -24 * (abs(alpha) * absab + abs(beta) * np.abs(prev[sel_r][:, sel_c])
                                              + np.abs(bias[sel_c]))
                err = np.abs(got[sel_r][:, sel_c] - ref)
                violations += int(np.count_nonzero(err > bound))
                worst = max(worst, float(np.max(err / (bound + 1e-300))))
            log(f"{form} execution {run}: {len(cols)} columns + {len(rows)} rows, violations {violations}, "
                f"err/bound {worst:.3e}; kernels {kernels(traced)}")
            assert violations == 0
            prev = got
        assert kernels(traced) == [4, 4]
        plan.release()
    finally:
        closed(s)
