"""The extension's sgemm_device on the MI355X: the tile kernels on device
memory the caller owns, enqueued on the caller's HIP stream, through the C ABI
(extension table), against the FP64 oracle.

* Config 1's shape (1024^3 N/N: 32 tiles of 256 x 128, K in 8 ranges) with the
  library's stream-ordered workspace and with a workspace of the caller's:
  the same bits both ways, within the FP64 bound.
* The config-5 launch shape in every form (4096 x 256 x 4096, 16 ranges) with
  alpha, beta and a per-row bias + ReLU: within the bound.
* Shapes that do not split (256 tiles; K too shallow for two ranges).
* Config 2's ragged shape (3001 x 2047 x 4099, alpha 1.5, beta 0.5): 12 x 16
  tiles of 256 x 128 split into 5 ranges (960 workgroups: two rounds of the
  kernel's workgroup slots), with the library's workspace and with the
  caller's: the same bits both ways, within the bound.
* Interior 256 x 256 tiles whose operand panel the ring kernels cannot
  address: op-T A with a leading dimension of 2^20 floats (a 2 GiB panel,
  beyond their 32-bit buffer offsets), 512 x 512 x 2048 in 32 ranges on the
  256 x 128 kernel, within the bound.
* Inside a transaction callback, on the resolved addresses of a session's
  allocations and the callback's native_stream (the use the entry point is
  for): C read back through allocation_read.

Device memory comes from the HIP runtime the library itself loaded (ctypes),
not from another runtime instance. Tolerance: |C - C_ref| <=
4*K*2^-24*(|alpha||A||B| + |beta C0| + |bias|)_ij."""
import ctypes
import os

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

pytestmark = pytest.mark.gpu

MiB = 1 << 20
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FP = ctypes.POINTER(ctypes.c_float)
FORMS = {"NN": (abi.OP_N, abi.OP_N), "NT": (abi.OP_N, abi.OP_T), "TN": (abi.OP_T, abi.OP_N),
         "TT": (abi.OP_T, abi.OP_T)}


def log(msg):
    print(f"[sgemm_device] {msg}", flush=True)


class Hip:
    """The few HIP runtime calls the tests need, from the library's runtime."""

    def __init__(self):
        self.rt = ctypes.CDLL("libamdhip64.so")
        self.streams = []

    def ok(self, rc, what):
        assert rc == 0, f"{what}: hipError {rc}"

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        self.ok(self.rt.hipMalloc(ctypes.byref(p), ctypes.c_size_t(max(nbytes, 16))), "hipMalloc")
        return p.value

    def free(self, p):
        self.ok(self.rt.hipFree(ctypes.c_void_p(p)), "hipFree")

    def put(self, p, host):
        host = np.ascontiguousarray(host)
        self.ok(self.rt.hipMemcpy(ctypes.c_void_p(p), host.ctypes.data_as(ctypes.c_void_p),
                                  ctypes.c_size_t(host.nbytes), 1), "hipMemcpy H2D")

    def get(self, p, count):
        out = np.empty(count, dtype=np.float32)
        self.ok(self.rt.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), ctypes.c_void_p(p),
                                  ctypes.c_size_t(out.nbytes), 2), "hipMemcpy D2H")
        return out

    def stream(self):
        s = ctypes.c_void_p()
        self.ok(self.rt.hipStreamCreateWithFlags(ctypes.byref(s), 1), "hipStreamCreate")
        self.streams.append(s.value)
        return s.value

    def sync(self, s):
        self.ok(self.rt.hipStreamSynchronize(ctypes.c_void_p(s)), "hipStreamSynchronize")

    def close(self):
        for s in self.streams:
            self.rt.hipStreamDestroy(ctypes.c_void_p(s))


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.fixture()
def hip(lib):
    h = Hip()
    yield h
    h.close()


def padded(mat):
    """Column-major storage (flat, ld) of a matrix, ld rounded up to 4 floats
    (the entry point's contract); the padding rows are zero."""
    rows, cols = mat.shape
    ld = (rows + 3) // 4 * 4
    buf = np.zeros((cols, ld), dtype=np.float32)
    buf[:, :rows] = mat.T
    return buf.reshape(-1), ld


def stored(op_mat, op):
    """The storage of a logical operated matrix (op T: stored transposed)."""
    return padded(op_mat if op == abi.OP_N else op_mat.T)


def desc_for(ptrs, m, n, k, ops, lds, alpha=1.0, beta=0.0, bias=0, axis=abi.BIAS_NONE, relu=False,
             workspace=0, workspace_bytes=0):
    d = abi.sgemm_device_init()
    d.a, d.b, d.c = ptrs
    d.m, d.n, d.k = m, n, k
    d.lda, d.ldb, d.ldc = lds
    d.operation_a, d.operation_b = ops
    d.alpha, d.beta = alpha, beta
    d.bias, d.bias_axis = (bias or None), axis
    d.activation = abi.ACTIVATION_RELU if relu else abi.ACTIVATION_NONE
    d.workspace, d.workspace_bytes = (workspace or None), workspace_bytes
    return d


def run_device_gemm(lib, hip, oracle_mod, m, n, k, ops, seed, alpha=1.0, beta=0.0, bias_rows=False,
                    relu=False, workspace_bytes=0, repeat=1):
    a_op = np.asfortranarray(oracle_mod.fill_uniform(m * k, seed).reshape(k, m).T)
    b_op = np.asfortranarray(oracle_mod.fill_uniform(k * n, seed + 1).reshape(n, k).T)
    c0 = np.asfortranarray(oracle_mod.fill_uniform(m * n, seed + 2).reshape(n, m).T)
    a_flat, lda = stored(a_op, ops[0])
    b_flat, ldb = stored(b_op, ops[1])
    bias = (oracle_mod.fill_uniform(m, seed + 3) * 0.5).astype(np.float32) if bias_rows else None
    c_flat, ldc = padded(c0)
    pa, pb, pc = hip.alloc(a_flat.nbytes), hip.alloc(b_flat.nbytes), hip.alloc(c_flat.nbytes)
    pbias = hip.alloc(bias.nbytes) if bias is not None else 0
    pws = hip.alloc(workspace_bytes) if workspace_bytes else 0
    s = hip.stream()
    try:
        hip.put(pa, a_flat)
        hip.put(pb, b_flat)
        if bias is not None:
            hip.put(pbias, bias)
        d = desc_for((pa, pb, pc), m, n, k, ops, (lda, ldb, ldc), alpha, beta, pbias,
                     abi.BIAS_PER_ROW if bias is not None else abi.BIAS_NONE, relu, pws,
                     workspace_bytes)
        outs = []
        for _ in range(repeat):
            hip.put(pc, c_flat)
            assert lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(s)) == abi.SUCCESS
            hip.sync(s)
            outs.append(hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T)
    finally:
        for p in (pa, pb, pc, pbias, pws):
            if p:
                hip.free(p)
    ref, absab = oracle_mod.sgemm_f64(a_op, b_op, alpha, beta, c0 if beta else None)
    if bias is not None:
        ref = ref + bias[:, None].astype(np.float64)
        absab = absab + np.abs(bias)[:, None]
    if relu:
        ref = np.maximum(ref, 0.0)
    return outs, ref, absab


def test_config1_shape_library_and_caller_workspace(lib, hip, oracle_mod):
    m = n = k = 1024
    outs, ref, absab = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS["NN"], 501, repeat=2)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"1024^3 NN, library workspace: violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0
    # Eight 4 MiB partials in a workspace of the caller's, exactly their size: the same
    # split, the same bits.
    mine, _, _ = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS["NN"], 501,
                                 workspace_bytes=32 * MiB)
    assert np.array_equal(mine[0].view(np.uint32), outs[0].view(np.uint32))


@pytest.mark.parametrize("form", sorted(FORMS))
def test_config5_launch_shape_with_epilogue(lib, hip, oracle_mod, form):
    m, n, k = 4096, 256, 4096
    outs, ref, absab = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 511,
                                       alpha=-0.5, beta=0.75, bias_rows=True, relu=True)
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"{m}x{n}x{k} {form} + bias/ReLU: violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0


@pytest.mark.parametrize("m,n,k,form", [(4096, 4096, 256, "NT"), (1000, 700, 300, "TN"),
                                        (257, 1031, 500, "TT")])
def test_unsplit_shapes(lib, hip, oracle_mod, m, n, k, form):
    outs, ref, absab = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 521, beta=0.5)
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"{m}x{n}x{k} {form}: violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0


@pytest.mark.parametrize("form", sorted(FORMS))
def test_config2_ragged_split(lib, hip, oracle_mod, form):
    m, n, k = 3001, 2047, 4099
    outs, ref, absab = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 541,
                                       alpha=1.5, beta=0.5)
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(outs[0]), k, ref, absab)
    log(f"config 2 {m}x{n}x{k} {form}, library workspace: violations {bad}, "
        f"err/bound {ratio:.3e}")
    assert bad == 0
    # Five partials of 3004 x 2047 floats in a workspace of the caller's.
    mine, _, _ = run_device_gemm(lib, hip, oracle_mod, m, n, k, FORMS[form], 541, alpha=1.5,
                                 beta=0.5, workspace_bytes=5 * 3004 * 2047 * 4)
    assert np.array_equal(mine[0].view(np.uint32), outs[0].view(np.uint32))


def test_split_on_the_256x128_kernel(lib, hip, oracle_mod):
    """op-T A stored k x m with lda = 2^20: the panel of A spans m * lda * 4 =
    2 GiB, which the ring kernels' 32-bit buffer offsets cannot reach, so the
    launch of 2 x 2 interior 256 x 256 tiles splits on the 256 x 128 kernel
    instead: 2 x 4 of its tiles, K in 32 ranges of 64."""
    m, n, k = 512, 512, 2048
    lda = 1 << 20
    a_op = np.asfortranarray(oracle_mod.fill_uniform(m * k, 551).reshape(k, m).T)
    b_op = np.asfortranarray(oracle_mod.fill_uniform(k * n, 552).reshape(n, k).T)
    a_lines = np.ascontiguousarray(a_op)  # row i of op(A) = line i of the stored A
    b_flat, ldb = stored(b_op, abi.OP_N)
    c_flat, ldc = padded(np.zeros((m, n), np.float32))
    pa = hip.alloc(m * lda * 4)
    pb, pc = hip.alloc(b_flat.nbytes), hip.alloc(c_flat.nbytes)
    s = hip.stream()
    try:
        hip.ok(hip.rt.hipMemset(ctypes.c_void_p(pa), 0, ctypes.c_size_t(m * lda * 4)), "hipMemset")
        hip.ok(hip.rt.hipMemcpy2D(ctypes.c_void_p(pa), ctypes.c_size_t(lda * 4),
                                  a_lines.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(k * 4),
                                  ctypes.c_size_t(k * 4), ctypes.c_size_t(m), 1), "hipMemcpy2D")
        hip.put(pb, b_flat)
        hip.put(pc, c_flat)
        d = desc_for((pa, pb, pc), m, n, k, (abi.OP_T, abi.OP_N), (lda, ldb, ldc))
        assert lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(s)) == abi.SUCCESS
        hip.sync(s)
        got = hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T
    finally:
        for p in (pa, pb, pc):
            hip.free(p)
    ref, absab = oracle_mod.sgemm_f64(a_op, b_op)
    bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(got), k, ref, absab)
    log(f"{m}x{n}x{k} TN, lda 2^20 (256 x 128 kernel): violations {bad}, err/bound {ratio:.3e}")
    assert bad == 0


def test_inside_a_transaction_callback(lib, oracle_mod):
    """C = A B on the working set of a transaction, on its native stream."""
    m, n, k = 1024, 512, 768
    a_op = np.asfortranarray(oracle_mod.fill_uniform(m * k, 531).reshape(k, m).T)
    b_op = np.asfortranarray(oracle_mod.fill_uniform(k * n, 532).reshape(n, k).T)
    s = xv.Session(lib, chunk_size_bytes=64 * MiB)
    try:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        A.write(a_op.reshape(-1, order="F"))
        B.write(b_op.reshape(-1, order="F"))
        status = []
        ids = [x.info().allocation_id for x in (A, B, C)]

        def body(view):
            address = {alloc: addr for alloc, offset, _, addr, _ in view.ranges if offset == 0}
            d = desc_for(tuple(address[i] for i in ids), m, n, k, FORMS["NN"], (m, k, m))
            status.append(lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(view.stream)))

        s.execute_transaction([xv.access(A, 0, m * k * 4, abi.ACCESS_READ),
                               xv.access(B, 0, k * n * 4, abi.ACCESS_READ),
                               xv.access(C, 0, m * n * 4, abi.ACCESS_WRITE_ONLY)], body)
        assert status == [abi.SUCCESS]
        got = C.read(dtype=np.float32).reshape(n, m).T
        ref, absab = oracle_mod.sgemm_f64(a_op, b_op)
        bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(got), k, ref, absab)
        log(f"in a transaction {m}x{n}x{k}: violations {bad}, err/bound {ratio:.3e}")
        assert bad == 0
    finally:
        s.close()
        s.release()
