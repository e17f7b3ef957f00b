"""CPU tests of split-K launches over libxvram_hostsim.so.

A launch that would leave workgroup slots idle cuts its K into ranges
(kernels::split_k_shape: on the ring kernels as many as one round of the CUs
takes when those are at least 256 deep, else on the 256 x 128 kernel the count
its timing model rates fastest; each at least 64 deep, in multiples of 32),
accumulates each range into a partial held in one frame of
the pool (leading dimension m rounded up to 4), and adds the partials in range
order before alpha, beta and the epilogue. Launches of interior 256 x 256 tiles
split on the ring kernels (one workgroup per CU); the others on the 256 x 128
kernel (two per CU). The simulated device performs exactly that data flow
(partials written to and read back from the frame, which must be mapped) and
counts the launches that split, so these tests check the rule itself (through
the library's own split_k_shape), the planner's reservation of the frame, the
executor's use of it, the split arithmetic (bit-exact analytic pattern, FP64
bound with K tails, beta and the epilogue, ragged m and n) and that repeated
runs give identical bits. The same launches on the GPU are in
tests/test_gpu_split_k.py."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import pattern_operands, storage, uniform

MiB = 1 << 20
FORMS = {"NN": (abi.OP_N, abi.OP_N), "NT": (abi.OP_N, abi.OP_T), "TN": (abi.OP_T, abi.OP_N),
         "TT": (abi.OP_T, abi.OP_T)}


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_split_launches.restype = ctypes.c_uint64
    lib.dll.xvram_hostsim_split_launches.argtypes = [ctypes.POINTER(ctypes.c_int)]
    yield lib
    lib.dll.xvram_hostsim_reset()


def narrow_splits(lib):
    lib.dll.xvram_hostsim_narrow_split_launches.restype = ctypes.c_uint64
    return lib.dll.xvram_hostsim_narrow_split_launches()


def split_stats(lib):
    last = ctypes.c_int(0)
    count = lib.dll.xvram_hostsim_split_launches(ctypes.byref(last))
    return count, last.value


def run(s, a_op, b_op, ops, c0=None, alpha=1.0, beta=0.0, bias=None, relu=False, repeat=1,
        axis=abi.BIAS_PER_COLUMN):
    m, k = a_op.shape
    n = b_op.shape[1]
    a_st = a_op if ops[0] == abi.OP_N else a_op.T
    b_st = b_op if ops[1] == abi.OP_N else b_op.T
    a_flat, lda = storage(np.ascontiguousarray(a_st), abi.COLUMN_MAJOR)
    b_flat, ldb = storage(np.ascontiguousarray(b_st), abi.COLUMN_MAJOR)
    c_flat, ldc = storage(c0 if c0 is not None else np.zeros((m, n), np.float32), abi.COLUMN_MAJOR)
    A, B, C = (s.allocation(x.nbytes) for x in (a_flat, b_flat, c_flat))
    A.write(a_flat)
    B.write(b_flat)
    ep = None
    if bias is not None or relu:
        V = None
        if bias is not None:
            V = s.allocation(bias.nbytes)
            V.write(bias)
        ep = xv.epilogue(V, axis if V is not None else abi.BIAS_NONE, relu=relu)
    plan = xv.GemmPlan(s, xv.matrix(A, *a_st.shape, lda), xv.matrix(B, *b_st.shape, ldb),
                       xv.matrix(C, m, n, ldc), ops[0], ops[1], alpha, beta, epilogue=ep)
    outs = []
    for _ in range(repeat):
        C.write(c_flat)
        plan.execute()
        outs.append(C.read(dtype=np.float32).reshape(n, ldc)[:, :m].T.copy())
    info = plan.info()
    plan.release()
    return outs, info


def session(lib, frame_mib=16, frames=12):
    return xv.Session(lib, chunk_size_bytes=frame_mib * MiB, cache_target_bytes=frames * frame_mib * MiB,
                      workspace_cap_bytes=0, device_headroom_bytes=0, max_transaction_ms=600000)


@pytest.mark.parametrize("form", sorted(FORMS))
def test_split_pattern_is_exact(sim, oracle_mod, form):
    """512 x 256 x 2048: two 256 x 256 tiles, whose ring split would take
    64-deep ranges, so the 256 x 128 kernel's 2 x 2 tiles split K into 32
    ranges of 64 (one launch)."""
    m, n, k = 512, 256, 2048
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim) as s:
        (out,), info = run(s, a_op, b_op, FORMS[form])
    assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (m, n, k, 1)
    assert info.maximum_working_set_bytes == 4 * 16 * MiB  # C, A, B and the partials' frame
    assert split_stats(sim) == (1, 32) and narrow_splits(sim) == 1
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))



@pytest.mark.parametrize("form", ["NN", "NT"])
def test_ring_split_pattern_is_exact(sim, oracle_mod, form):
    """1024 x 512 x 8192 under 64 MiB frames: eight 256 x 256 tiles whose K
    splits into 32 ranges of 256 on the ring kernels (one round of the CUs;
    the 32 partials of 2 MiB fill the partials' frame)."""
    m, n, k = 1024, 512, 8192
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim, frame_mib=64, frames=8) as s:
        (out,), info = run(s, a_op, b_op, FORMS[form])
    assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (m, n, k, 1)
    assert split_stats(sim) == (1, 32) and narrow_splits(sim) == 0
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))

@pytest.mark.parametrize("form", sorted(FORMS))
def test_split_with_k_tail_beta_and_epilogue(sim, oracle_mod, form):
    """K = 1000: eleven ranges, ten of 96 and a tail of 40 (no multiple of
    32); alpha, beta and a per-column bias with ReLU after the reduction.
    Within the FP64 bound, and the same bits on every run."""
    m, n, k = 512, 256, 1000
    a_op = uniform(oracle_mod, m, k, 71)
    b_op = uniform(oracle_mod, k, n, 72)
    c0 = uniform(oracle_mod, m, n, 73)
    bias = (oracle_mod.fill_uniform(n, 74) * 0.5).astype(np.float32)
    with session(sim) as s:
        outs, _ = run(s, a_op, b_op, FORMS[form], c0, alpha=-0.75, beta=0.5, bias=bias,
                      relu=True, repeat=2)
    assert split_stats(sim) == (2, 11)
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    a64, b64 = a_op.astype(np.float64), b_op.astype(np.float64)
    ref = np.maximum(-0.75 * (a64 @ b64) + 0.5 * c0 + bias[None, :], 0.0)
    absab = 0.75 * (np.abs(a64) @ np.abs(b64)) + 0.5 * np.abs(c0) + np.abs(bias)[None, :]
    bound = 4 * k * 2.0 ** -24 * absab + 1e-30
    assert np.all(np.abs(outs[0] - ref) <= bound)


def test_split_across_k_panels(sim, oracle_mod):
    """K panels smaller than K (frames of 2 MiB: 512 x 1024 panels): each
    launch splits its own panel; later panels accumulate onto C (beta 1)."""
    m, n, k = 512, 256, 4096
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim, frame_mib=2, frames=16) as s:
        (out,), info = run(s, a_op, b_op, FORMS["NT"])
    assert info.tile_k < k and info.tile_count == k // info.tile_k
    count, last = split_stats(sim)
    assert count == info.tile_count and last >= 2
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_no_split_when_k_is_shallow(sim, oracle_mod):
    """K = 120 leaves fewer than two ranges of 64: unsplit."""
    m, n, k = 512, 256, 120
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim) as s:
        (out,), info = run(s, a_op, b_op, FORMS["NN"])
    assert split_stats(sim)[0] == 0 and info.maximum_working_set_bytes == 3 * 16 * MiB
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


MiB_ = 1 << 20


@pytest.mark.parametrize("m,n,k,nt,ring,ws,expect", [
    # the C5 chain's launch: 16 tiles of 256 x 256 -> 16 ranges of 256 (ring kernels,
    # one round of the CUs)
    (4096, 256, 4096, False, True, 64 * MiB_, (16, 256, 0)),
    # the resident C5 layer: 64 tiles -> 4 ranges of 4096
    (16384, 256, 16384, False, True, 1 << 30, (4, 4096, 0)),
    # config 1: 16 tiles, whose ring split would take 16 ranges of 64: the 256 x 128
    # kernel's 32 tiles in 8 ranges of 128 instead
    (1024, 1024, 1024, False, True, 64 * MiB_, (8, 128, 1)),
    # 8 tiles, 32 ranges of 256 in one round: the ring kernels
    (1024, 512, 8192, True, True, 64 * MiB_, (32, 256, 0)),
    # config 2: ragged, 12 x 16 tiles of 256 x 128 on the 256 x 128 kernel: 5 ranges
    # (960 workgroups, two rounds of its 512 slots); 64 MiB hold only 2 partials
    (3001, 2047, 4099, False, True, 128 * MiB_, (5, 832, 1)),
    (3001, 2047, 4099, False, True, 64 * MiB_, (2, 2080, 1)),
    # 16 x 24 tiles of 256 x 128 fill 3/4 of the slots unsplit; 2 ranges run faster
    (4000, 3000, 2000, True, True, 1 << 30, (2, 1024, 1)),
    # 256 tiles of 256 x 256 fill the chip
    (4096, 4096, 4096, True, True, 64 * MiB_, (1, 0, 0)),
    # ragged, but 17 x 16 tiles of 256 x 256: no split K (an edge split, if any, is its own rule)
    (4100, 4096, 4096, True, True, 64 * MiB_, (1, 0, 0)),
    # interior but K not a multiple of 8 (N/N): the 256 x 128 kernel; N/T splits on the ring
    (1024, 1024, 1004, False, True, 64 * MiB_, (8, 128, 1)),
    (1024, 1024, 1004, True, True, 64 * MiB_, (8, 128, 1)),
    # operand panels the ring kernels cannot address: the 256 x 128 kernel
    (1024, 1024, 1024, False, False, 64 * MiB_, (8, 128, 1)),
    # K below two ranges of 64: unsplit
    (1024, 1024, 120, False, True, 64 * MiB_, (1, 0, 0)),
    # the workspace holds 3 partials: 3 ranges; 1 partial: unsplit
    (4096, 256, 4096, False, True, 12 * MiB_, (3, 1376, 0)),
    (4096, 256, 4096, False, True, 4 * MiB_, (1, 0, 0)),
    # partials of m rounded up to 4: 501 x 200 -> ld 504
    (501, 200, 2048, False, True, 8 * 504 * 200 * 4, (8, 256, 1)),
    (501, 200, 2048, False, True, 8 * 504 * 200 * 4 - 1, (7, 320, 1)),
])
def test_split_rule(sim, m, n, k, nt, ring, ws, expect):
    fn = sim.dll.xvram_hostsim_split_shape
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                   ctypes.c_uint64, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    depth, narrow = ctypes.c_int(0), ctypes.c_int(0)
    splits = fn(m, n, k, int(nt), int(ring), ws, ctypes.byref(depth), ctypes.byref(narrow))
    assert (splits, depth.value, narrow.value) == expect


@pytest.mark.parametrize("form", sorted(FORMS))
def test_ragged_split_pattern_is_exact(sim, oracle_mod, form):
    """501 x 200 x 2048: not whole 256 x 256 tiles, so the 256 x 128 kernel's
    2 x 2 tiles split K into 32 ranges of 64; the partials' leading dimension
    is 504 (m rounded up to 4) and the reduction's last quad of each column
    holds one row."""
    m, n, k = 501, 200, 2048
    a_op, b_op = pattern_operands(m, n, k)
    with session(sim) as s:
        (out,), info = run(s, a_op, b_op, FORMS[form])
    assert info.tile_count == 1
    assert split_stats(sim) == (1, 32) and narrow_splits(sim) == 1
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


@pytest.mark.parametrize("axis", [abi.BIAS_PER_ROW, abi.BIAS_PER_COLUMN], ids=["row", "col"])
@pytest.mark.parametrize("form", sorted(FORMS))
def test_ragged_split_with_k_tail_beta_and_epilogue(sim, oracle_mod, form, axis):
    """501 x 200 x 1000 on the 256 x 128 kernel: eleven ranges (ten of 96, 40),
    alpha, beta and a per-row or per-column bias with ReLU after the
    reduction. Within the FP64 bound, and the same bits on every run."""
    m, n, k = 501, 200, 1000
    a_op = uniform(oracle_mod, m, k, 81)
    b_op = uniform(oracle_mod, k, n, 82)
    c0 = uniform(oracle_mod, m, n, 83)
    length = m if axis == abi.BIAS_PER_ROW else n
    bias = (oracle_mod.fill_uniform(length, 84) * 0.5).astype(np.float32)
    with session(sim) as s:
        outs, _ = run(s, a_op, b_op, FORMS[form], c0, alpha=1.25, beta=-0.5, bias=bias,
                      relu=True, repeat=2, axis=axis)
    assert split_stats(sim) == (2, 11) and narrow_splits(sim) == 2
    assert np.array_equal(outs[0].view(np.uint32), outs[1].view(np.uint32))
    a64, b64 = a_op.astype(np.float64), b_op.astype(np.float64)
    badd = bias[:, None] if axis == abi.BIAS_PER_ROW else bias[None, :]
    ref = np.maximum(1.25 * (a64 @ b64) - 0.5 * c0 + badd, 0.0)
    absab = 1.25 * (np.abs(a64) @ np.abs(b64)) + 0.5 * np.abs(c0) + np.abs(badd)
    bound = 4 * k * 2.0 ** -24 * absab + 1e-30
    assert np.all(np.abs(outs[0] - ref) <= bound)


def test_split_frame_is_returned_to_the_pool(sim, oracle_mod):
    """The partials' frame is not a cache entry: the session still tears down
    balanced, and nothing of it is written back."""
    m, n, k = 512, 256, 2048
    a_op, b_op = pattern_operands(m, n, k)
    s = session(sim)
    run(s, a_op, b_op, FORMS["TN"])
    run(s, a_op, b_op, FORMS["TN"])
    s.drain()
    t = s.telemetry()
    assert t.bytes_d2h == 2 * m * n * 4  # the two C results, nothing of the partials
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps and t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    assert t.physical_handles_created == t.physical_handles_released
    s.release()


def test_split_rule_properties(sim):
    """Over a grid of shapes, forms and panel limits: every split covers K with
    ranges of at least 64 in multiples of 32, keeps to one round of the CUs
    (ring kernels: partials <= 64 MiB) or two rounds of the 256 x 128 kernel's
    slots (partials <= 128 MiB), and a launch given exactly the workspace its
    split wants (split_k_bytes_wanted) takes the same split, family included;
    one byte less takes fewer ranges on the same family."""
    fn = sim.dll.xvram_hostsim_split_shape
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                   ctypes.c_uint64, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]

    def split(m, n, k, nt, ring, ws):
        depth, narrow = ctypes.c_int(0), ctypes.c_int(0)
        s = fn(m, n, k, int(nt), int(ring), ws, ctypes.byref(depth), ctypes.byref(narrow))
        return s, depth.value, narrow.value

    checked = 0
    dims = [200, 256, 501, 512, 768, 1000, 1024, 2048, 3001, 4096, 5000]
    for m in dims:
        for n in dims:
            for k in (96, 128, 500, 1024, 2048, 4099, 8192, 16384):
                for nt in (False, True):
                    for ring in (False, True):
                        s, depth, narrow = split(m, n, k, nt, ring, (1 << 64) - 1)
                        if s == 1:
                            continue
                        checked += 1
                        assert depth % 32 == 0 and depth >= 64 and (s - 1) * depth < k <= s * depth
                        partial = (m + 3) // 4 * 4 * n * 4
                        if narrow:
                            tiles = -(-m // 256) * -(-n // 128)
                            assert tiles * s <= 1024 and s * partial <= 128 * MiB
                        else:
                            assert m % 256 == 0 and n % 256 == 0 and ring
                            assert (m // 256) * (n // 256) * s <= 256 and s * partial <= 64 * MiB
                        assert split(m, n, k, nt, ring, s * partial) == (s, depth, narrow)
                        s2, _, narrow2 = split(m, n, k, nt, ring, s * partial - 1)
                        assert s2 < s and (s2 == 1 or narrow2 == narrow)
    assert checked > 500


def tail_rule(lib):
    fn = lib.dll.xvram_hostsim_tail_split_shape
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                   ctypes.c_uint64, ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int)]

    def tail(m, n, k, nt, ring, ws):
        head, depth = ctypes.c_int64(0), ctypes.c_int(0)
        s = fn(m, n, k, int(nt), int(ring), ws, ctypes.byref(head), ctypes.byref(depth))
        return s, head.value, depth.value
    return tail


ANY = (1 << 64) - 1


@pytest.mark.parametrize("m,n,k,nt,ring,ws,expect", [
    # 17 x 17 tiles: 2 rounds for 289 tiles -> a head of 15 rows (255 tiles, one round)
    # and a tail of 2 rows in 7 ranges of 640
    (4352, 4352, 4352, True, True, ANY, (7, 3840, 640)),
    # 17 x 16: a head of 16 rows, the last row in 5 ranges of 224
    (4352, 4096, 1024, False, True, ANY, (5, 4096, 224)),
    # 20 x 20: a head of 12 rows, 8 rows in 3 ranges (two rounds of the CUs); 64 MiB
    # hold only 1 partial of the tail: no tail split
    (5120, 5120, 5120, True, True, ANY, (3, 3072, 1728)),
    (5120, 5120, 5120, True, True, 64 * MiB_, (1, 0, 0)),
    # whole rounds already; too shallow to gain; ragged; panels the ring kernels
    # cannot address; K not a multiple of 8 (N/N)
    (4096, 4096, 4096, True, True, ANY, (1, 0, 0)),
    (4352, 4352, 512, True, True, ANY, (1, 0, 0)),
    (4353, 4352, 4352, True, True, ANY, (1, 0, 0)),
    (4352, 4352, 4352, True, False, ANY, (1, 0, 0)),
    (4352, 4352, 4356, False, True, ANY, (1, 0, 0)),
])
def test_tail_split_rule(sim, m, n, k, nt, ring, ws, expect):
    assert tail_rule(sim)(m, n, k, nt, ring, ws) == expect


def test_tail_split_properties(sim):
    """Over a grid of interior shapes of 256 to 1600 tiles: a tail split keeps
    whole tile rows in the head, ranges at least 224 deep in multiples of 32
    covering K, at most two rounds of the CUs in the tail (partials <= 128 MiB),
    never coincides with an ordinary split, and a launch given exactly the
    workspace the tail wants takes the same tail split."""
    tail = tail_rule(sim)
    fn = sim.dll.xvram_hostsim_split_shape
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int, ctypes.c_int,
                   ctypes.c_uint64, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    taken = 0
    for tm in range(16, 41, 3):
        for tn in range(16, 41, 5):
            for k in (512, 1024, 2048, 4096, 8192):
                m, n = 256 * tm, 256 * tn
                for nt in (False, True):
                    s, head, depth = tail(m, n, k, nt, True, ANY)
                    assert fn(m, n, k, int(nt), 1, ANY, None, None) == 1
                    if s == 1:
                        assert head == 0
                        continue
                    taken += 1
                    assert head % 256 == 0 and 0 < head < m
                    assert depth % 32 == 0 and depth >= 224 and (s - 1) * depth < k <= s * depth
                    assert (m - head) // 256 * tn * s <= 512
                    wanted = s * (m - head) * n * 4
                    assert wanted <= 128 * MiB
                    assert tail(m, n, k, nt, True, wanted) == (s, head, depth)
    assert taken > 100


@pytest.mark.parametrize("m,frames", [(4352, 4), (4096, 3)])
def test_planner_reserves_a_frame_for_a_tail_split(sim, m, frames):
    """4352 x 4096 x 1024 under 256 MiB frames is one launch whose last tile
    row runs as a split tail: the plan counts the partials' frame in its
    working set (C, A, B and the partials); 4096 x 4096 x 1024 fills whole
    rounds and needs none. Planned only (nothing executes)."""
    n, k = 4096, 1024
    with session(sim, frame_mib=256, frames=8) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k), xv.matrix(C, m, n, m))
        info = plan.info()
        plan.release()
        for h in (A, B, C):
            h.release()
    assert info.tile_count == 1
    assert info.maximum_working_set_bytes == frames * 256 * MiB


def edge_rule(lib):
    fn = lib.dll.xvram_hostsim_edge_split_shape
    fn.restype = ctypes.c_int
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_int)]

    def edge(m, n, k, nt):
        wants = ctypes.c_int(0)
        return fn(m, n, k, int(nt), ctypes.byref(wants)), wants.value
    return edge


@pytest.mark.parametrize("m,n,k,nt,expect", [
    # ragged, a last round that would fill few CUs: the interior (20 x 20 tiles: 19 x 19 with
    # a tail split) and two strips, which split
    (5000, 5000, 5000, True, (1, 1)),
    (7000, 7000, 7000, False, (1, 1)),
    (4100, 4100, 1024, False, (1, 1)),
    (4100, 4100, 240, False, (1, 1)),
    (5000, 5000, 2048, False, (1, 1)),
    (6312, 6275, 2176, False, (1, 1)),
    # whole rounds (nearly) full: the whole launch on the ring kernels' edge instances
    (8191, 8191, 2048, True, (0, 0)),
    (8191, 8191, 8192, False, (0, 0)),
    (8100, 8100, 4096, False, (0, 0)),
    (4000, 4000, 12000, True, (0, 0)),
    (4001, 3999, 1024, False, (0, 0)),
    (4001, 4093, 2048, True, (0, 0)),
    (3900, 4096, 1000, False, (0, 0)),
    (6981, 4328, 3928, True, (0, 0)),
    (11500, 11000, 1024, False, (0, 0)),
    # K not a multiple of 8 (N/N; N/T takes it), fewer than 256 tiles, interior
    (4500, 4500, 4500, False, (0, 0)),
    (4500, 4500, 4500, True, (1, 1)),
    (2000, 2000, 2000, True, (0, 0)),
    (4096, 4096, 4096, True, (0, 0)),
])
def test_edge_split_rule(sim, m, n, k, nt, expect):
    assert edge_rule(sim)(m, n, k, nt) == expect


def test_edge_split_pattern_is_exact(sim, oracle_mod):
    """4100 x 4100 x 248 under 128 MiB frames, one launch of 17 x 17 ragged
    tiles: it runs as the 16 x 16 interior tiles, the right strip (4096 x 4)
    and the bottom strip (4 x 4100), each a launch of its own (the strips
    split K in the partials' frame the planner reserved); every element of C
    bit-exact on the analytic pattern."""
    m, n, k = 4100, 4100, 248
    a_op, b_op = pattern_operands(m, n, k)
    sim.dll.xvram_hostsim_edge_split_launches.restype = ctypes.c_uint64
    sim.dll.xvram_hostsim_kernel_launches.restype = ctypes.c_uint64
    with session(sim, frame_mib=128, frames=8) as s:
        (out,), info = run(s, a_op, b_op, FORMS["NN"])
    assert info.tile_count == 1
    assert info.maximum_working_set_bytes == 4 * 128 * MiB  # C, A, B and the partials' frame
    assert sim.dll.xvram_hostsim_edge_split_launches() == 1
    assert sim.dll.xvram_hostsim_kernel_launches() == 3
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


@pytest.mark.parametrize("m,n,k,nt,expect", [
    # K % 8 = 4 (N/N): the rounded 4096 takes an edge split -> a K remainder
    (5000, 5000, 4100, False, 4096),
    # the same K for N/T is a multiple of 4: no remainder needed
    (5000, 5000, 4100, True, 0),
    # interior 17 x 17 tiles, K % 8 = 3: the rounded K takes a tail split
    (4352, 4352, 4099, False, 4096),
    # ragged tiles, whole rounds full: the rounded K runs whole on the ring kernels' edge
    # instances instead of the general kernel's predicated edge tiles
    (8191, 8191, 8190, False, 8184),
    (8191, 8191, 8190, True, 8188),
    (4001, 3999, 1030, False, 1024),
    (4001, 3999, 1030, True, 1028),
    # interior tiles in whole rounds (the general kernel's interior loop), too shallow, or
    # fewer than 256 tiles
    (4096, 4096, 4099, False, 0),
    (5000, 5000, 507, False, 0),
    (3001, 2047, 4099, False, 0),
])
def test_k_remainder_rule(sim, m, n, k, nt, expect):
    fn = sim.dll.xvram_hostsim_k_remainder_shape
    fn.restype = ctypes.c_int64
    fn.argtypes = [ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int]
    assert fn(m, n, k, int(nt)) == expect


def test_k_remainder_pattern_is_exact(sim, oracle_mod):
    """4100 x 4100 x 516 N/N under 128 MiB frames: K % 8 = 4, and the rounded
    512 takes an edge split, so the launch runs as the 512-deep edge split
    (no epilogue) and a 4-deep launch onto its result; every element of C
    bit-exact on the analytic pattern."""
    m, n, k = 4100, 4100, 516
    a_op, b_op = pattern_operands(m, n, k)
    sim.dll.xvram_hostsim_k_remainder_launches.restype = ctypes.c_uint64
    sim.dll.xvram_hostsim_edge_split_launches.restype = ctypes.c_uint64
    with session(sim, frame_mib=128, frames=8) as s:
        (out,), info = run(s, a_op, b_op, FORMS["NN"])
    assert info.tile_count == 1 and info.maximum_working_set_bytes == 4 * 128 * MiB
    assert sim.dll.xvram_hostsim_k_remainder_launches() == 1
    assert sim.dll.xvram_hostsim_edge_split_launches() == 1
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))


def test_partials_never_exceed_the_allocation_free_scratch(sim):
    """Over seeded random launch shapes (small to 16384 wide, ragged or not, K
    down to 1, every form, panels near and past the ring kernels' 2^31-byte
    limit): the partials any launch wants -- its split, tail split, the
    largest part of its edge split or the first part of its K remainder --
    fit the allocation-free entry's 128 MiB scratch."""
    fn = sim.dll.xvram_hostsim_bytes_wanted
    fn.restype = ctypes.c_uint64
    fn.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                   ctypes.c_int64, ctypes.c_int64]
    rng = np.random.default_rng(97)
    most, split = 0, 0
    for _ in range(20000):
        scale = int(rng.choice([512, 4096, 16384]))
        m, n = (int(v) for v in rng.integers(1, scale + 1, 2))
        k = int(rng.integers(1, 3 * scale))
        if rng.random() < 0.5:
            m, n = 256 * max(1, m // 256), 256 * max(1, n // 256)
        ak, bn = (bool(v) for v in rng.integers(0, 2, 2))
        lda = (k if ak else m) + 4 * int(rng.integers(0, 3))
        ldb = (n if bn else k) + 4 * int(rng.integers(0, 3))
        lda, ldb = (lda + 3) // 4 * 4, (ldb + 3) // 4 * 4
        wanted = fn(m, n, k, int(ak), int(bn), lda, ldb)
        most = max(most, wanted)
        split += wanted > 0
        assert wanted <= 128 * MiB, (m, n, k, ak, bn, wanted)
    assert split > 1000 and most > 64 * MiB
