"""CPU tests of the fused bias/ReLU epilogue (extension table) through the C ABI
over libxvram_hostsim.so: both bias axes, both C layouts (the row-major swap
moves the bias to the other canonical axis), out-of-core K splits (the epilogue
must apply once, after the last K panel), the linear-layer mapping of config 5,
and the extension's validation rules.

Reference for each result: the oracle's FP64 GEMM, then + bias and ReLU in
FP64; the bound is the GEMM bound with |bias| as one more term of the sum
(ReLU is 1-Lipschitz, so it cannot enlarge an error)."""
import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import logical_from_storage, storage, uniform

KiB = 1 << 10


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def session(lib, frames=10, frame_kib=32):
    return xv.Session(lib, chunk_size_bytes=frame_kib * KiB,
                      cache_target_bytes=frames * frame_kib * KiB, workspace_cap_bytes=0,
                      device_headroom_bytes=0)


def run_epilogue(s, a_op, b_op, c0, bias_vec, axis, relu, op_a=abi.OP_N, op_b=abi.OP_N,
                 layouts=(abi.COLUMN_MAJOR,) * 3, alpha=1.0, beta=0.0, bias_pad=0):
    m, k = a_op.shape
    n = b_op.shape[1]
    a_st = a_op if op_a == abi.OP_N else a_op.T
    b_st = b_op if op_b == abi.OP_N else b_op.T
    a_flat, lda = storage(np.ascontiguousarray(a_st), layouts[0])
    b_flat, ldb = storage(np.ascontiguousarray(b_st), layouts[1])
    c_flat, ldc = storage(c0, layouts[2])
    A, B, C = s.allocation(a_flat.nbytes), s.allocation(b_flat.nbytes), s.allocation(c_flat.nbytes)
    A.write(a_flat)
    B.write(b_flat)
    C.write(c_flat)
    bias = None
    if bias_vec is not None:
        raw = np.concatenate([np.full(bias_pad, np.nan, np.float32), bias_vec.astype(np.float32)])
        bias = s.allocation(raw.nbytes)
        bias.write(raw)
    ep = xv.epilogue(bias, axis, offset=bias_pad * 4, relu=relu)
    plan = xv.GemmPlan(s, xv.matrix(A, a_st.shape[0], a_st.shape[1], lda, layouts[0]),
                       xv.matrix(B, b_st.shape[0], b_st.shape[1], ldb, layouts[1]),
                       xv.matrix(C, m, n, ldc, layouts[2]), op_a, op_b, alpha, beta, epilogue=ep)
    info = plan.info()
    plan.execute()
    out = logical_from_storage(C.read(dtype=np.float32), m, n, ldc, layouts[2])
    plan.release()
    return np.asfortranarray(out), info


def reference(oracle, a_op, b_op, c0, bias_vec, axis, relu, alpha=1.0, beta=0.0):
    ref, absab = oracle.sgemm_f64(np.asfortranarray(a_op), np.asfortranarray(b_op), alpha, beta,
                                  np.asfortranarray(c0) if beta != 0 else None)
    if bias_vec is not None:
        b64 = bias_vec.astype(np.float64)
        add = b64[:, None] if axis == abi.BIAS_PER_ROW else b64[None, :]
        ref = ref + add
        absab = absab + np.abs(add)
    if relu:
        ref = np.where(ref < 0, 0.0, ref)
    return np.asfortranarray(ref), np.asfortranarray(absab)


@pytest.mark.parametrize("c_layout", [abi.COLUMN_MAJOR, abi.ROW_MAJOR], ids=["Ccol", "Crow"])
@pytest.mark.parametrize("axis", [abi.BIAS_PER_ROW, abi.BIAS_PER_COLUMN], ids=["row", "col"])
@pytest.mark.parametrize("relu", [False, True], ids=["id", "relu"])
def test_bias_axes_layouts_out_of_core(sim, oracle_mod, c_layout, axis, relu):
    m, n, k = 70, 90, 300
    a = uniform(oracle_mod, m, k, 31)
    b = uniform(oracle_mod, k, n, 32)
    c0 = uniform(oracle_mod, m, n, 33)
    bias = oracle_mod.fill_uniform(m if axis == abi.BIAS_PER_ROW else n, 34).astype(np.float32)
    with session(sim) as s:
        out, info = run_epilogue(s, a, b, c0, bias, axis, relu, layouts=(1, 0, c_layout),
                                 alpha=1.5, beta=0.5, bias_pad=3)
        assert info.tile_count > 1  # K is split: the epilogue must run once, at the end
    ref, absab = reference(oracle_mod, a, b, c0, bias, axis, relu, 1.5, 0.5)
    bad, max_err, _ = oracle_mod.check_bound(out, k, ref, absab)
    assert bad == 0, max_err
    if relu:
        assert (out >= 0).all() and (out == 0).any()


def test_relu_without_bias(sim, oracle_mod):
    m, n, k = 40, 50, 60
    a, b = uniform(oracle_mod, m, k, 41), uniform(oracle_mod, k, n, 42)
    with session(sim) as s:
        out, _ = run_epilogue(s, a, b, np.zeros((m, n), np.float32), None, abi.BIAS_NONE, True,
                              op_a=abi.OP_T, op_b=abi.OP_T)
    ref, absab = reference(oracle_mod, a, b, None, None, abi.BIAS_NONE, True)
    assert oracle_mod.check_bound(out, k, ref, absab)[0] == 0


def test_linear_layer_mapping(sim, oracle_mod):
    """Config 5's layer: Y = ReLU(X W^T + b) with row-major X (batch x in),
    W (out x in), Y (batch x out): op(A) = X, op(B) = W^T, per-column bias
    (python/xvram/torch_native.py:1907-1970 maps linear the same way)."""
    batch, fin, fout = 24, 96, 80
    rng = np.random.default_rng(5)
    x = rng.standard_normal((batch, fin)).astype(np.float32)
    w = (rng.standard_normal((fout, fin)) / np.sqrt(fin)).astype(np.float32)
    bvec = (rng.standard_normal(fout) / np.sqrt(fin)).astype(np.float32)
    with session(sim, frames=8, frame_kib=8) as s:
        X, W, Y, Bv = (s.allocation(v) for v in (x.nbytes, w.nbytes, batch * fout * 4, bvec.nbytes))
        X.write(x)
        W.write(w)
        Bv.write(bvec)
        plan = xv.GemmPlan(s, xv.matrix(X, batch, fin, fin, abi.ROW_MAJOR),
                           xv.matrix(W, fout, fin, fin, abi.ROW_MAJOR),
                           xv.matrix(Y, batch, fout, fout, abi.ROW_MAJOR), abi.OP_N, abi.OP_T,
                           epilogue=xv.epilogue(Bv, abi.BIAS_PER_COLUMN, relu=True))
        plan.execute()
        y = Y.read(dtype=np.float32).reshape(batch, fout)
        plan.release()
    pre = x.astype(np.float64) @ w.astype(np.float64).T + bvec.astype(np.float64)
    ref = np.maximum(pre, 0.0)
    absab = np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T + np.abs(bvec)
    assert np.all(np.abs(y - ref) <= 4 * fin * 2.0 ** -24 * absab)


def test_epilogue_validation(sim):
    with session(sim, frames=6, frame_kib=16) as s:
        A, B, C = s.allocation(32 * 32 * 4), s.allocation(32 * 32 * 4), s.allocation(32 * 32 * 4)
        bias = s.allocation(31 * 4)
        big = s.allocation(8192 * 4)
        mats = (xv.matrix(A, 32, 32, 32), xv.matrix(B, 32, 32, 32), xv.matrix(C, 32, 32, 32))

        def status(ep, mats=mats):
            with pytest.raises(xv.XvramError) as e:
                xv.GemmPlan(s, *mats, epilogue=ep)
            return e.value.status

        assert status(xv.epilogue(bias, abi.BIAS_PER_ROW)) == abi.INVALID_ARGUMENT  # 31 < 32
        assert status(xv.epilogue(big, abi.BIAS_PER_ROW, offset=2)) == abi.INVALID_ARGUMENT
        assert status(xv.epilogue(None, abi.BIAS_PER_ROW)) == abi.INVALID_ARGUMENT
        assert status(xv.epilogue(big, abi.BIAS_NONE)) == abi.INVALID_ARGUMENT
        assert status(xv.epilogue(big, 7)) == abi.INVALID_ARGUMENT
        ep = xv.epilogue(big, abi.BIAS_PER_ROW)
        ep.activation = 9
        assert status(ep) == abi.INVALID_ARGUMENT
        ep = xv.epilogue(big, abi.BIAS_PER_ROW)
        ep.flags = 1
        assert status(ep) == abi.INVALID_ARGUMENT
        ep = xv.epilogue(big, abi.BIAS_PER_ROW)
        ep.struct_size -= 8
        assert status(ep) == abi.INCOMPATIBLE_ABI
        # A bias inside C's storage.
        assert status(xv.epilogue(C, abi.BIAS_PER_ROW, offset=64)) == abi.INVALID_ARGUMENT
        # A bias longer than one frame (16 KiB) cannot be pinned.
        wide = s.allocation(4 * 8192 * 4)
        mats2 = (xv.matrix(A, 32, 32, 32), xv.matrix(wide, 32, 8192, 32),
                 xv.matrix(big, 1, 8192, 1))
        assert status(xv.epilogue(wide, abi.BIAS_PER_COLUMN), mats2) in (
            abi.BUDGET_PRESSURE, abi.INVALID_ARGUMENT)
        # A valid plan still works afterwards.
        plan = xv.GemmPlan(s, *mats, epilogue=xv.epilogue(big, abi.BIAS_PER_COLUMN, relu=True))
        plan.execute()
        plan.release()
        assert s.telemetry().poisoned == 0
