"""The xvram.gemm_bench v1 report of xvram_amd.gemm_report: validated against the
reference's own schema (schemas/gemm-bench-report-v1.schema.json, read from the
reference tree where it is mounted) and against the completed-report semantics
of tests/contract/gemm_contract.py:333-355, on an oversubscribed hostsim run.
The schema checker itself is pinned by planted mistakes that must fail it."""
import copy
import json
import os

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import gemm_report

from schema_check import errors

SCHEMA = "/root/reference/schemas/gemm-bench-report-v1.schema.json"
KiB = 1 << 10

RAW_ADDRESS_KEYS = {"base_address", "device_address", "device_pointer", "native_stream", "raw_va",
                    "virtual_address", "virtual_address_base", "workspace_device_address"}


def completed_semantics(report, oversubscribed=True):
    """tests/contract/gemm_contract.py:333-355, restated."""
    device, proof, cache = report["device"], report["proof"], report["cache"]
    workload, plan = report["workloads"][0], report["plans"][0]
    assert device is not None
    assert workload["plan_id"] == plan["plan_id"]
    assert workload["tiles_retired"] == workload["tiles_total"] == plan["tile_count"]
    if oversubscribed:
        assert proof["logical_allocation_bytes"] > device["total_memory_bytes"]
        assert proof["maximum_cache_target_bytes"] < proof["logical_allocation_bytes"]
    assert plan["maximum_working_set_bytes"] <= proof["maximum_cache_target_bytes"]
    assert plan["workspace_bytes"] <= proof["workspace_cap_bytes"]
    assert cache["resident_bytes_peak"] <= cache["target_bytes_maximum"]
    assert cache["workspace_bytes_peak"] <= proof["workspace_cap_bytes"]
    assert cache["mapping_count"] == cache["set_access_count"] == cache["unmap_count"]
    # gemm_contract.py:349 asserts equality. Both builds count every write-back
    # (reference src/sdk/runtime.cpp:535 <- residency/runtime.cpp:4253) and the
    # verifying allocation_read writes back C tiles still cached dirty without
    # evicting them (residency/runtime.cpp:931-945), so the write-backs exceed
    # the dirty evictions by exactly those flushes; each dirty eviction is
    # still one write-back.
    assert cache["dirty_evictions"] <= cache["writebacks_completed"]
    assert cache["unsafe_remap_count"] == 0
    assert cache["unsafe_transition_count"] == 0
    assert workload["cache_hits"] + workload["cache_misses"] > 0
    assert workload["output_digest128"] == report["numerics"]["output_digest128"]
    assert report["numerics"]["expected_digest128"] == report["numerics"]["output_digest128"]

    def no_raw(value):
        if isinstance(value, dict):
            assert RAW_ADDRESS_KEYS.isdisjoint(value)
            for child in value.values():
                no_raw(child)
        elif isinstance(value, list):
            for child in value:
                no_raw(child)
    no_raw(report)


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


@pytest.fixture(scope="module")
def schema():
    if not os.path.exists(SCHEMA):
        pytest.skip("the reference tree (and its report schema) is not mounted")
    return json.load(open(SCHEMA))


def test_pattern_closed_form():
    m, n, k = 7, 11, 13
    ref = gemm_report.pattern_a(m, k).astype(np.float64) @ gemm_report.pattern_b(k, n)
    assert np.array_equal(gemm_report.pattern_c(m, n, k), ref.astype(np.float32))
    # The reference's own known answer: expected(4, 6, 11) = 78
    # (tests/unit/gemm_pattern_tests.cpp:103-153).
    assert gemm_report.pattern_c(5, 7, 11)[4, 6] == 78


@pytest.mark.parametrize("ops", [("n", "t"), ("t", "n")])
def test_oversubscribed_report_is_schema_valid(sim, schema, ops):
    sim.dll.xvram_hostsim_set_memory(128 * KiB, 128 * KiB)  # device smaller than the data
    report = gemm_report.run_report(sim, 128, 96, 160, ops[0], ops[1], chunk_bytes=16 * KiB,
                                    workspace_cap_bytes=0, device_headroom_bytes=0)
    assert errors(schema, report) == []
    assert report["outcome"]["status"] == "completed"
    assert report["plans"][0]["tile_count"] > 1
    assert report["workloads"][0]["dirty_evictions"] > 0
    completed_semantics(report)
    json.dumps(report)  # serialisable as is


def test_schema_checker_rejects_planted_mistakes(sim, schema):
    sim.dll.xvram_hostsim_set_memory(128 * KiB, 128 * KiB)
    good = gemm_report.run_report(sim, 64, 64, 64, chunk_bytes=16 * KiB, workspace_cap_bytes=0,
                                  device_headroom_bytes=0)
    assert errors(schema, good) == []
    plants = [
        ("outcome", "exit_code", 5),                      # not an allowed exit code
        ("numerics", "mismatch_count", 1),                # completed requires 0 mismatches
        ("cache", "unsafe_remap_count", 2),               # completed requires zero unsafe activity
        ("configuration", "a_operation", "N"),            # enum is lower case
        ("numerics", "output_digest128", "xyz"),          # not a 128-bit hex digest
        ("build", "cuda_headers_version", 12000),         # below the minimum
    ]
    for section, field, value in plants:
        bad = copy.deepcopy(good)
        bad[section][field] = value
        assert errors(schema, bad), (section, field)
    bad = copy.deepcopy(good)
    bad["workloads"][0]["unexpected"] = 1
    assert errors(schema, bad)
    bad = copy.deepcopy(good)
    del bad["telemetry"]["tile_timing"]
    assert errors(schema, bad)
