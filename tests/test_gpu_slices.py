"""GPU check of the sliced first launch in all four N/T forms.

With 32 MiB frames a 4096 x 4096 x 8192 product plans 2048 x 2048 x 4096
launches (8 of them); the first one finds its A and B panels missing and runs
as two 2048-deep K slices, each waiting only for its own slices of the panels
(filled by separate copies). The analytic pattern makes the product exact in
FP32 (28 * 8192 < 2^24), so every element is compared bit for bit with the
oracle's closed form; the kernel count is read from the library's trace."""
import json

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import Problem, pattern_operands

pytestmark = pytest.mark.gpu

MiB = 1 << 20
OPS = [(abi.OP_N, abi.OP_N), (abi.OP_N, abi.OP_T), (abi.OP_T, abi.OP_N), (abi.OP_T, abi.OP_T)]
OP_IDS = ["NN", "NT", "TN", "TT"]


@pytest.mark.parametrize("ops", OPS, ids=OP_IDS)
def test_sliced_first_launch_is_exact(tmp_path, monkeypatch, oracle_mod, ops):
    trace = tmp_path / "trace.jsonl"
    monkeypatch.setenv("XVRAM_TRACE_FILE", str(trace))
    lib = xv.load()
    m = n = 4096
    k = 8192
    a_op, b_op = pattern_operands(m, n, k)
    s = xv.Session(lib, chunk_size_bytes=32 * MiB, cache_target_bytes=12 * 32 * MiB + 4 * MiB)
    try:
        prob = Problem(a_op, b_op, op_a=ops[0], op_b=ops[1])
        out = prob.run(s)
        info = prob.plan_info
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps and t.physical_handles_created == t.physical_handles_released
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        s.release()
    kernels = [len(json.loads(line)["kernels"]) for line in open(trace)]
    print(f"{OP_IDS[OPS.index(ops)]}: {info.tile_count} launches of {info.tile_m}x{info.tile_n}x"
          f"{info.tile_k}, kernels {kernels}", flush=True)
    assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (2048, 2048, 4096, 8)
    assert kernels == [9]
    assert np.array_equal(out.astype(np.float64), oracle_mod.pattern_expected_matrix(m, n, k))
