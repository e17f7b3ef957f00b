"""CPU tests of the panel planner's tile shapes for large frames, over
libxvram_hostsim.so (plans only: the operands are allocated, never multiplied).

- The starting square stops at 8192 (1024 workgroups of the 256 x 256 kernel)
  and the rest of a large frame goes to K: with 1 GiB frames a 16384 x 16384 x
  32768 problem plans 8192 x 8192 x 32768 launches (1 GiB A and B panels), not
  16384^3 ones.
- A and B panels stay below 2^31 bytes (the 256 x 256 kernels' 32-bit buffer
  offsets): with 2 GiB frames an 8192 x 8192 x 65536 problem, whose whole A
  would fill one frame, plans two 32768-deep launches instead of one.
- Frames of 512 MiB and below keep their shapes: 8192 x 8192 x 16384 launches
  at 512 MiB, 4096^3 at 64 MiB.
- The reference planner's large-K regression fixture (row-major 2049 x 2049 x
  32769 under 64 MiB chunks) plans under both of its targets.

Each case allocates its operands in host memory (zero-filled): at most 5 GiB."""
import pytest

import xvram_amd as xv
from xvram_amd import abi

MiB, GiB = 1 << 20, 1 << 30


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def plan_shape(lib, m, n, k, frame, frames, op_b=abi.OP_T):
    with xv.Session(lib, chunk_size_bytes=frame, cache_target_bytes=frames * frame,
                    workspace_cap_bytes=0, device_headroom_bytes=0) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        b_desc = xv.matrix(B, n, k, n) if op_b == abi.OP_T else xv.matrix(B, k, n, k)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), b_desc, xv.matrix(C, m, n, m), abi.OP_N, op_b)
        info = plan.info()
        plan.release()
        for h in (A, B, C):
            h.release()
    return info.tile_m, info.tile_n, info.tile_k, info.tile_count


def test_large_frames_grow_k_not_the_c_tile(sim):
    assert plan_shape(sim, 16384, 16384, 32768, GiB, 16) == (8192, 8192, 32768, 4)


def test_panels_stay_below_two_gib(sim):
    assert plan_shape(sim, 8192, 8192, 65536, 2 * GiB, 8) == (8192, 8192, 32768, 2)


@pytest.mark.parametrize("frame,k,expected", [(512 * MiB, 32768, (8192, 8192, 16384, 2)),
                                              (64 * MiB, 8192, (4096, 4096, 4096, 8))],
                         ids=["512MiB", "64MiB"])
def test_smaller_frames_keep_their_shapes(sim, frame, k, expected):
    assert plan_shape(sim, 8192, 8192, k, frame, 31) == expected


@pytest.mark.parametrize("target_mib", [256, 384])
def test_reference_large_k_fixture(sim, target_mib):
    """The reference planner's large-K regression fixture
    (tests/unit/gemm_planner_tests.cpp:265-300): 2049 x 2049 x 32769 with every
    matrix row-major, 64 MiB chunks, a 4 MiB workspace cap. The reference's
    chunk planner needs five resident chunks (a 384 MiB target; 256 MiB is
    working_set_too_large) and plans 165 tiles of 512 x 2049 x 1024. The panel
    planner needs three frames, so both targets plan: 2049 x 2049 C tiles and
    4096-deep K panels, 9 per tile (the last one 1 deep), three frames at most
    in use (A, B and C panels of 32.8 MiB, 32.8 MiB and 16 MiB), and under the
    larger target one more for the split-K partials."""
    m = n = 2049
    k = 32769
    with xv.Session(sim, chunk_size_bytes=64 * MiB, cache_target_bytes=target_mib * MiB,
                    workspace_cap_bytes=4 * MiB, device_headroom_bytes=0) as s:
        A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
        plan = xv.GemmPlan(s, xv.matrix(A, m, k, k, abi.ROW_MAJOR),
                           xv.matrix(B, k, n, n, abi.ROW_MAJOR),
                           xv.matrix(C, m, n, n, abi.ROW_MAJOR))
        info = plan.info()
        assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (2049, 2049, 4096, 9)
        # Five frames leave one for the split-K partials of the ragged
        # 2049 x 2049 x 4096 launches (three ranges); three frames do not.
        frames = 4 if target_mib == 384 else 3
        assert info.maximum_working_set_bytes == frames * 64 * MiB
        assert info.workspace_bytes == 0
        plan.release()
        for h in (A, B, C):
            h.release()
