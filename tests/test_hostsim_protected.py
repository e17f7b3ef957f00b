"""CPU test of the executor's protected panels, over libxvram_hostsim.so.

Before each launch's acquisition the executor declares the A, B and C panels
of the launches up to one pass of a C block ahead; victim selection passes
over them while it has another choice. The case is config 4's schedule at
1/32 scale: 1024^3 N/T in 128 x 128 x 128 tiles (8 x 8 C tiles, 8 K panels)
under 31 frames of 64 KiB, so C blocks of 3 x 4 tiles fill 27 of the 31
frames. Every execution loads exactly 286 panels (the planned schedule, 3 x |B|
+ 2 x |A| = 320 panels, less those the serpentine and the previous execution
leave cached); without the protection the policy evicts panels of the running
pass before their last use and 303 are loaded. The accounting is reproducible
(frame choice depends only on the schedule), so the count is exact."""
import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import pattern_operands

KiB = 1 << 10


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def test_no_panel_is_loaded_twice_in_a_block(sim, oracle_mod):
    m = n = k = 1024
    frame = 64 * KiB
    a_op, b_op = pattern_operands(m, n, k)
    with xv.Session(sim, chunk_size_bytes=frame, cache_target_bytes=31 * frame, workspace_cap_bytes=0,
                    device_headroom_bytes=0, max_transaction_ms=600000) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(n * k * 4), s.allocation(m * n * 4)
        A.write(np.ascontiguousarray(a_op.T).reshape(-1))  # column-major m x k
        B.write(np.ascontiguousarray(b_op).reshape(-1))    # column-major n x k (op T)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, n, k, n), xv.matrix(C, m, n, m),
                           abi.OP_N, abi.OP_T)
        info = plan.info()
        assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (128, 128, 128, 512)
        for _ in range(3):
            t0 = s.telemetry()
            plan.execute()
            t1 = s.telemetry()
            assert t1.bytes_h2d - t0.bytes_h2d == 286 * frame
        out = C.read(dtype=np.float32).reshape(n, m).T
        plan.release()
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))
