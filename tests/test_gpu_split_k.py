"""Split-K launches on the MI355X, through the C ABI, against the oracle.

Launches that would leave workgroup slots idle split K (kernels::split_k_plan):
each K range of each tile is one workgroup (of the ring kernels for interior
256 x 256 tiles, else of the 256 x 128 kernel), writing raw partial sums into
one frame of the pool, and a second kernel adds the partials in range order
and applies alpha, beta and the epilogue.

* The config-5 launch shape (4096 x 256 x 4096 under 64 MiB frames: 16 tiles,
  16 ranges of 256, the partials filling the frame exactly), all four forms:
  the analytic pattern, every element bit-exact.
* A K tail (4096 x 256 x 4000: 16 ranges of 256, the last 160) with alpha,
  beta and a per-column bias + ReLU, seeded U[-1,1) operands: every element
  within the FP64 bound, and two executions bit-identical (the reduction
  order is fixed).
* A resident config-5 layer with the weights resident (16384 x 256 x 16384
  T/N under 1 GiB frames: 64 tiles, 4 ranges of 4096): pattern bit-exact.
* Config 1's shape (1024^3 N/N: its ring split would take 64-deep ranges, so
  32 tiles of 256 x 128 in 8 ranges of 128): every element within the
  FP64 bound.
* Launches that are not whole 256 x 256 tiles split on the 256 x 128 kernel:
  501 x 200 x 2048 (2 x 2 tiles, 32 ranges; partials of leading dimension 504)
  bit-exact on the pattern in all four forms; 501 x 200 x 1000 (eleven ranges,
  a K tail) with alpha, beta and a per-row or per-column bias + ReLU within the
  bound, two executions bit-identical; config 2's shape (3001 x 2047 x 4099)
  in all four forms with alpha 1.5, beta 0.5 within the bound, under 64 MiB
  frames (the partials' frame holds 2 ranges) and 128 MiB frames (5 ranges,
  two rounds of the kernel's workgroup slots).

Tolerance: |C - C_ref| <= 4*K*2^-24*(|alpha||A||B| + |beta C0| + |bias|)_ij."""
import ctypes
import os

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

pytestmark = pytest.mark.gpu

MiB, GiB = 1 << 20, 1 << 30
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP = ctypes.POINTER(ctypes.c_float)
FORMS = {"NN": (abi.OP_N, abi.OP_N), "NT": (abi.OP_N, abi.OP_T), "TN": (abi.OP_T, abi.OP_N),
         "TT": (abi.OP_T, abi.OP_T)}


def log(msg):
    print(f"[split-k] {msg}", flush=True)


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


class Gemm:
    """op(A) m x k, op(B) k x n, C m x n column-major, stored per `ops`."""

    def __init__(self, s, m, n, k, ops, alpha=1.0, beta=0.0, bias=None, relu=False,
                 axis=abi.BIAS_PER_COLUMN):
        self.m, self.n, self.k, self.ops = m, n, k, ops
        self.a_shape = (m, k) if ops[0] == abi.OP_N else (k, m)
        self.b_shape = (k, n) if ops[1] == abi.OP_N else (n, k)
        self.a = s.allocation(m * k * 4)
        self.b = s.allocation(k * n * 4)
        self.c = s.allocation(m * n * 4)
        ep = None
        if bias is not None or relu:
            v = None
            if bias is not None:
                v = s.allocation(bias.nbytes)
                v.write(bias)
            ep = xv.epilogue(v, axis if v is not None else abi.BIAS_NONE, relu=relu)
        self.plan = xv.GemmPlan(s, xv.matrix(self.a, *self.a_shape, self.a_shape[0]),
                                xv.matrix(self.b, *self.b_shape, self.b_shape[0]),
                                xv.matrix(self.c, m, n, m), ops[0], ops[1], alpha, beta,
                                epilogue=ep)

    def fill_pattern(self, synth):
        for alloc, filler, (rows, cols), t in (
                (self.a, synth.synth_fill_pattern_a, self.a_shape, self.ops[0] == abi.OP_T),
                (self.b, synth.synth_fill_pattern_b, self.b_shape, self.ops[1] == abi.OP_T)):
            buf = np.empty(rows * cols, dtype=np.float32)
            filler(buf.ctypes.data_as(FP), rows, cols, 0, 1 if t else 0)
            alloc.write(buf)

    def fill_uniform(self, synth, seed_a, seed_b):
        for alloc, (rows, cols), seed in ((self.a, self.a_shape, seed_a),
                                          (self.b, self.b_shape, seed_b)):
            buf = np.empty(rows * cols, dtype=np.float32)
            synth.synth_fill_uniform(buf.ctypes.data_as(FP), buf.size, seed, 0)
            alloc.write(buf)
            yield buf.reshape(cols, rows).T  # the stored matrix, logical view

    def execute(self):
        op = self.plan.submit()
        st, info = op.wait()
        assert st == abi.SUCCESS and info.result == abi.SUCCESS, op.error().message.decode()
        op.release()

    def result(self):
        return self.c.read(dtype=np.float32).reshape(self.n, self.m).T


@pytest.mark.parametrize("form", sorted(FORMS))
def test_split_c5_launch_pattern(lib, synth, oracle_mod, form):
    m, n, k = 4096, 256, 4096
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=2 * GiB)
    try:
        g = Gemm(s, m, n, k, FORMS[form])
        info = g.plan.info()
        assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (m, n, k, 1)
        g.fill_pattern(synth)
        g.execute()
        got = g.result()
        expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
        bad = int(np.count_nonzero(got != expect))
        log(f"pattern {m}x{n}x{k} {form}: {bad} of {m * n} differ")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_split_k_tail_beta_epilogue_deterministic(lib, synth, oracle_mod, form):
    m, n, k = 4096, 256, 4000
    alpha, beta = 1.5, 0.5
    bias = (oracle_mod.fill_uniform(n, 94) * 0.5).astype(np.float32)
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=2 * GiB)
    try:
        g = Gemm(s, m, n, k, FORMS[form], alpha, beta, bias=bias, relu=True)
        a_st, b_st = list(g.fill_uniform(synth, 91, 92))
        c0 = np.empty(m * n, dtype=np.float32)
        synth.synth_fill_uniform(c0.ctypes.data_as(FP), c0.size, 93, 0)
        outs = []
        for _ in range(2):
            g.c.write(c0)
            g.execute()
            outs.append(g.result().copy())
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        a_op = a_st if FORMS[form][0] == abi.OP_N else a_st.T
        b_op = b_st if FORMS[form][1] == abi.OP_N else b_st.T
        c0m = c0.reshape(n, m).T
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a_op), np.asfortranarray(b_op),
                                          alpha, beta, np.asfortranarray(c0m))
        ref = np.maximum(ref + bias[None, :].astype(np.float64), 0.0)
        absab = absab + np.abs(bias)[None, :]
        bad, _, ratio = oracle_mod.check_bound(outs[0], k, ref, absab)
        log(f"tail {m}x{n}x{k} {form}: violations {bad}, err/bound {ratio:.3e}")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)


def test_split_resident_c5_layer_pattern(lib, synth, oracle_mod):
    m, n, k = 16384, 256, 16384
    s = xv.Session(lib, chunk_size_bytes=GiB)
    try:
        g = Gemm(s, m, n, k, FORMS["TN"])
        assert g.plan.info().tile_count == 1
        g.fill_pattern(synth)
        g.execute()
        got = g.result()
        expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
        bad = int(np.count_nonzero(got != expect))
        log(f"pattern {m}x{n}x{k} TN: {bad} of {m * n} differ")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)


def test_split_config1_shape(lib, synth, oracle_mod):
    m = n = k = 1024
    s = xv.Session(lib)
    try:
        g = Gemm(s, m, n, k, FORMS["NN"])
        a_st, b_st = list(g.fill_uniform(synth, 95, 96))
        g.execute()
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a_st), np.asfortranarray(b_st))
        bad, _, ratio = oracle_mod.check_bound(g.result(), k, ref, absab)
        log(f"1024^3 NN: violations {bad}, err/bound {ratio:.3e}")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_ragged_split_pattern(lib, synth, oracle_mod, form):
    m, n, k = 501, 200, 2048
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=2 * GiB)
    try:
        g = Gemm(s, m, n, k, FORMS[form])
        g.fill_pattern(synth)
        g.execute()
        got = g.result()
        expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
        bad = int(np.count_nonzero(got != expect))
        log(f"ragged pattern {m}x{n}x{k} {form}: {bad} of {m * n} differ")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("axis", [abi.BIAS_PER_ROW, abi.BIAS_PER_COLUMN], ids=["row", "col"])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_ragged_split_k_tail_beta_epilogue(lib, synth, oracle_mod, form, axis):
    m, n, k = 501, 200, 1000
    alpha, beta = 1.25, -0.5
    length = m if axis == abi.BIAS_PER_ROW else n
    bias = (oracle_mod.fill_uniform(length, 97) * 0.5).astype(np.float32)
    s = xv.Session(lib, chunk_size_bytes=64 * MiB, cache_target_bytes=2 * GiB)
    try:
        g = Gemm(s, m, n, k, FORMS[form], alpha, beta, bias=bias, relu=True, axis=axis)
        a_st, b_st = list(g.fill_uniform(synth, 98, 99))
        c0 = np.empty(m * n, dtype=np.float32)
        synth.synth_fill_uniform(c0.ctypes.data_as(FP), c0.size, 100, 0)
        outs = []
        for _ in range(2):
            g.c.write(c0)
            g.execute()
            outs.append(g.result().copy())
        assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
        a_op = a_st if FORMS[form][0] == abi.OP_N else a_st.T
        b_op = b_st if FORMS[form][1] == abi.OP_N else b_st.T
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a_op), np.asfortranarray(b_op),
                                          alpha, beta, np.asfortranarray(c0.reshape(n, m).T))
        badd = bias[:, None] if axis == abi.BIAS_PER_ROW else bias[None, :]
        ref = np.maximum(ref + badd.astype(np.float64), 0.0)
        absab = absab + np.abs(badd)
        bad, _, ratio = oracle_mod.check_bound(outs[0], k, ref, absab)
        log(f"ragged tail {m}x{n}x{k} {form} bias {'row' if length == m else 'col'}: "
            f"violations {bad}, err/bound {ratio:.3e}")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)


@pytest.mark.parametrize("frame_mib", [64, 128])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_config2_shape_split(lib, synth, oracle_mod, form, frame_mib):
    """Config 2 (3001 x 2047 x 4099, alpha 1.5, beta 0.5) resident: one launch of
    12 x 16 tiles of 256 x 128 that splits K into as many ranges as the
    partials' frame holds up to the rule's 5: 2 under 64 MiB frames, 5 under
    128 MiB."""
    m, n, k = 3001, 2047, 4099
    alpha, beta = 1.5, 0.5
    s = xv.Session(lib, chunk_size_bytes=frame_mib * MiB, cache_target_bytes=2 * GiB)
    try:
        g = Gemm(s, m, n, k, FORMS[form], alpha, beta)
        assert g.plan.info().tile_count == 1
        a_st, b_st = list(g.fill_uniform(synth, 101, 102))
        c0 = np.empty(m * n, dtype=np.float32)
        synth.synth_fill_uniform(c0.ctypes.data_as(FP), c0.size, 103, 0)
        g.c.write(c0)
        g.execute()
        got = g.result()
        a_op = a_st if FORMS[form][0] == abi.OP_N else a_st.T
        b_op = b_st if FORMS[form][1] == abi.OP_N else b_st.T
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(a_op), np.asfortranarray(b_op),
                                          alpha, beta, np.asfortranarray(c0.reshape(n, m).T))
        bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(got), k, ref, absab)
        log(f"config 2 {m}x{n}x{k} {form}, {frame_mib} MiB frames: violations {bad}, "
            f"err/bound {ratio:.3e}")
        assert bad == 0
        g.plan.release()
    finally:
        closed(s)
