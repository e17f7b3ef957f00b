"""The xvram.gemm_bench v1 report from a real out-of-core run on the MI355X:
the analytic pattern verified exactly, and the completed-report semantics of
tests/contract/gemm_contract.py:333-355 (less the device-oversubscription
clause, which 288 GB of HBM cannot meet at test sizes). The schema itself is
checked on the CPU (tests/test_gemm_report.py): the reference tree is not on
the GPU box."""
import json

import pytest

import xvram_amd as xv
from xvram_amd import gemm_report

from test_gemm_report import completed_semantics

pytestmark = pytest.mark.gpu

MiB = 1 << 20


def test_out_of_core_pattern_report():
    report = gemm_report.run_report(xv.load(), 4096, 4096, 4096, "n", "t", chunk_bytes=16 * MiB,
                                    cache_target_bytes=128 * MiB)
    print(json.dumps({k: report[k] for k in ("workloads", "numerics")})[:2000], flush=True)
    assert report["outcome"]["status"] == "completed", report["outcome"]
    assert report["numerics"]["mismatch_count"] == 0
    assert report["plans"][0]["tile_count"] > 1
    assert report["proof"]["cache_smaller_than_logical"]
    assert report["workloads"][0]["dirty_evictions"] > 0
    assert report["device"]["compute_capability_major"] == 9
    assert report["device"]["total_memory_bytes"] > 200 * 1024 * MiB
    completed_semantics(report, oversubscribed=False)
