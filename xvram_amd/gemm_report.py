"""gemm_report — one analytic-pattern FP32 GEMM through the C ABI, reported as an
``xvram.gemm_bench`` v1 document.

The document has the shape of the reference's GEMM benchmark report
(schemas/gemm-bench-report-v1.schema.json, written by src/gemm_bench/report.cpp
and executor.cpp), so tooling and contract checks written for the reference
(tests/contract/gemm_contract.py:333-355) run against this build unchanged.

The workload is the reference benchmark's analytic integer pattern
(src/gemm_bench/pattern.cpp:207-237): A(i,p) = 1 + i%3 + p%2 and
B(p,j) = 1 + j%5 + p%3 over the logical op(A) (m x k) and op(B) (k x n), so
every C element is an integer below 2^24 for 28*K < 2^24 and is verified
exactly ("structured" validation against the closed form, no tolerance
needed). Digests are BLAKE2b-128 of C's storage bytes, pass after pass; the
expected digest hashes the closed-form C laid out the same way.

Fields that name CUDA-only facilities keep their names: ``cuda_*`` carry the
HIP values (``build.cuda_headers_version`` = HIP_VERSION of the headers the
library was built with), cuBLAS fields are null (no vendor BLAS is used),
WDDM fields are null (Linux).

Usage: python -m xvram_amd.gemm_report --m 8192 --n 8192 --k 8192 \\
           --chunk-bytes 268435456 --cache-target-bytes 2147483648 --out report.json
"""
from __future__ import annotations

import argparse
import ctypes
import datetime
import hashlib
import json
import os
import platform
import statistics
import sys
import tempfile
import time
from typing import Optional

import numpy as np

from . import Library, Session, GemmPlan, matrix, abi, load, LIB_DIR

KIB = 1 << 10
_COMPUTE_NAMES = {abi.COMPUTE_AUTO: "auto", abi.COMPUTE_FP32_STRICT: "fp32_strict",
                  abi.COMPUTE_FP32_TF32: "tf32", abi.COMPUTE_FP64: "fp64"}


# ---- the analytic pattern -----------------------------------------------------------

def pattern_a(m: int, k: int) -> np.ndarray:
    """Logical op(A), m x k: 1 + i%3 + p%2."""
    i = np.arange(m, dtype=np.int64)[:, None] % 3
    p = np.arange(k, dtype=np.int64)[None, :] % 2
    return (1 + i + p).astype(np.float32)


def pattern_b(k: int, n: int) -> np.ndarray:
    """Logical op(B), k x n: 1 + j%5 + p%3."""
    p = np.arange(k, dtype=np.int64)[:, None] % 3
    j = np.arange(n, dtype=np.int64)[None, :] % 5
    return (1 + j + p).astype(np.float32)


def pattern_c(m: int, n: int, k: int) -> np.ndarray:
    """Closed form of C = op(A) op(B): with u = 1 + i%3 and v = 1 + j%5,
    C(i,j) = u*v*K + u*S3 + v*S2 + S23, S2 = sum p%2, S3 = sum p%3,
    S23 = sum (p%2)(p%3) over p < K (exact in FP32 while 28*K < 2^24)."""
    p = np.arange(k, dtype=np.int64)
    s2, s3, s23 = int((p % 2).sum()), int((p % 3).sum()), int(((p % 2) * (p % 3)).sum())
    u = 1 + np.arange(m, dtype=np.int64)[:, None] % 3
    v = 1 + np.arange(n, dtype=np.int64)[None, :] % 5
    return (u * v * k + u * s3 + v * s2 + s23).astype(np.float32)


def column_major(logical: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(logical.T).reshape(-1)


# ---- collection helpers ---------------------------------------------------------------

def _timing(samples) -> dict:
    samples = sorted(float(s) for s in samples)
    if not samples:
        return {"sample_count": 0, "total_ms": None, "minimum_ms": None, "median_ms": None,
                "p95_ms": None, "maximum_ms": None}
    p95 = samples[min(len(samples) - 1, int(round(0.95 * (len(samples) - 1))))]
    return {"sample_count": len(samples), "total_ms": sum(samples), "minimum_ms": samples[0],
            "median_ms": statistics.median(samples), "p95_ms": p95, "maximum_ms": samples[-1]}


def _meminfo() -> tuple[Optional[int], Optional[int]]:
    try:
        fields = {}
        for line in open("/proc/meminfo"):
            name, value = line.split(":", 1)
            fields[name] = int(value.split()[0]) * KIB
        return fields.get("MemTotal"), fields.get("MemAvailable")
    except (OSError, ValueError):
        return None, None


def _build_section() -> dict:
    info = {}
    try:
        info = json.load(open(os.path.join(LIB_DIR, "build_info.json")))
    except (OSError, ValueError):
        pass
    return {"version": info.get("version", "0.1.0"),
            "git_commit": info.get("git_commit", "unknown"),
            "compiler": info.get("compiler", "unknown"),
            "build_type": info.get("build_type", "Release"),
            "cuda_headers_version": max(13000, int(info.get("hip_version", 0)))}


def _device_info(lib: Library, ordinal: int) -> abi.DeviceInfoV1:
    out = abi.DeviceInfoV1()
    out.struct_size = ctypes.sizeof(out)
    status = lib.ext.device_get_info(ordinal, ctypes.byref(out))
    if status != abi.SUCCESS:
        raise RuntimeError(f"device_get_info({ordinal}) failed: {abi.STATUS.get(status, status)}")
    return out


def _telemetry_dict(t) -> dict:
    return {name: getattr(t, name) for name, _ in type(t)._fields_ if name != "reserved"}


# ---- the run --------------------------------------------------------------------------

def run_report(lib: Library, m: int, n: int, k: int, op_a: str = "n", op_b: str = "t",
               chunk_bytes: int = 64 << 20, cache_target_bytes: int = 0,
               workspace_cap_bytes: int = 4 << 20, device_headroom_bytes: int = 512 << 20,
               passes: int = 1, device_ordinal: int = 0, policy: str = "clock",
               identifiers_included: bool = False) -> dict:
    if 28 * k >= (1 << 24):
        raise ValueError("the pattern is exact in FP32 only while 28*K < 2^24")
    started_utc = datetime.datetime.now(datetime.timezone.utc)
    trace_path = os.path.join(tempfile.mkdtemp(prefix="xvram_report_"), "trace.jsonl")
    previous_trace = os.environ.get("XVRAM_TRACE_FILE")
    os.environ["XVRAM_TRACE_FILE"] = trace_path
    dev0 = _device_info(lib, device_ordinal)
    t_start = time.perf_counter()
    cfg = dict(device_ordinal=device_ordinal, chunk_size_bytes=chunk_bytes,
               cache_target_bytes=cache_target_bytes, workspace_cap_bytes=workspace_cap_bytes,
               device_headroom_bytes=device_headroom_bytes,
               cache_policy=abi.CACHE_POLICY_LRU if policy == "lru" else abi.CACHE_POLICY_CLOCK)
    session = Session(lib, **cfg)
    try:
        tele_setup = session.telemetry()
        ta, tb = op_a == "t", op_b == "t"
        a_log, b_log = pattern_a(m, k), pattern_b(k, n)
        a_store = column_major(a_log.T if ta else a_log)   # stored op^-1 view, column-major
        b_store = column_major(b_log.T if tb else b_log)
        a_rows, a_cols = (k, m) if ta else (m, k)
        b_rows, b_cols = (n, k) if tb else (k, n)
        A = session.allocation(a_store.nbytes)
        B = session.allocation(b_store.nbytes)
        C = session.allocation(m * n * 4)
        A.write(a_store)
        B.write(b_store)
        del a_store, b_store, a_log, b_log
        t_plan = time.perf_counter()
        plan = GemmPlan(session, matrix(A, a_rows, a_cols, a_rows), matrix(B, b_rows, b_cols, b_rows),
                        matrix(C, m, n, m), abi.OP_T if ta else abi.OP_N,
                        abi.OP_T if tb else abi.OP_N, compute_mode=abi.COMPUTE_FP32_STRICT)
        plan_ms = (time.perf_counter() - t_plan) * 1e3
        info = plan.info()
        expected = column_major(pattern_c(m, n, k))
        expected_bytes = expected.view(np.uint8)
        tele0 = session.telemetry()
        gemm_ms, mismatches, first_bad, max_abs = [], 0, None, 0.0
        d_out, d_exp = hashlib.blake2b(digest_size=16), hashlib.blake2b(digest_size=16)
        for _ in range(passes):
            t0 = time.perf_counter()
            plan.execute()
            gemm_ms.append((time.perf_counter() - t0) * 1e3)
            got = C.read(dtype=np.float32)
            diff = np.abs(got.astype(np.float64) - expected.astype(np.float64))
            bad = np.flatnonzero(~np.isfinite(got) | (diff > 0))
            if bad.size and first_bad is None:
                first_bad = int(bad[0]) * 4
            mismatches += int(bad.size)
            max_abs = max(max_abs, float(np.nanmax(diff)) if diff.size else 0.0)
            d_out.update(got.view(np.uint8))
            d_exp.update(expected_bytes)
        tele1 = session.telemetry()
        plan.release()
        for h in (A, B, C):
            h.release()
        dev_end = _device_info(lib, device_ordinal)
        session.close()
        tele_end = session.telemetry()
    finally:
        session.release()
        if previous_trace is None:
            os.environ.pop("XVRAM_TRACE_FILE", None)
        else:
            os.environ["XVRAM_TRACE_FILE"] = previous_trace
    total_ms = (time.perf_counter() - t_start) * 1e3

    ops = [json.loads(line) for line in open(trace_path)] if os.path.exists(trace_path) else []
    kernel_ms = [e - s for op in ops for s, e, _ in op.get("kernels", [])]
    h2d_ms = [e - s for op in ops for s, e, _ in op.get("h2d", [])]
    d2h_ms = [e - s for op in ops for s, e, _ in op.get("d2h", [])]

    def delta(name):
        return getattr(tele1, name) - getattr(tele0, name)

    logical = (a_rows * a_cols + b_rows * b_cols + m * n) * 4
    hits, misses = delta("cache_hits"), delta("cache_misses")
    flops = 2.0 * m * n * k * passes
    match = mismatches == 0 and d_out.hexdigest() == d_exp.hexdigest()
    cache_target = tele_end.cache_target_bytes
    workload = {
        "name": f"pattern_{m}x{n}x{k}_{op_a}{op_b}", "plan_id": 1,
        "status": "completed" if match else "failed", "passes_completed": passes,
        "tiles_total": info.tile_count * passes, "tiles_retired": delta("transactions_completed"),
        "logical_allocation_bytes": logical, "oversubscribed": logical > dev0.total_memory_bytes,
        "cache_hits": hits, "cache_misses": misses,
        "cache_hit_rate": hits / (hits + misses) if hits + misses else 0.0,
        "bytes_h2d": delta("bytes_h2d"), "bytes_d2h": delta("bytes_d2h"),
        "clean_evictions": delta("clean_evictions"), "dirty_evictions": delta("dirty_evictions"),
        "writebacks_completed": delta("writebacks_completed"), "mapping_count": delta("mappings"),
        "unmap_count": delta("unmaps"), "set_access_count": delta("set_access_calls"),
        "handle_reuse_count": delta("handle_reuses"),
        "event_boundary_count": delta("event_boundaries"),
        "unsafe_remap_count": delta("unsafe_remaps"),
        "unsafe_transition_count": delta("unsafe_transitions"),
        "elapsed_ms": sum(gemm_ms), "achieved_tflops": flops / (sum(gemm_ms) * 1e-3) / 1e12,
        "output_digest128": d_out.hexdigest()}
    end = tele_end
    cache = {
        "target_bytes_initial": tele_setup.cache_target_bytes,
        "target_bytes_minimum": end.cache_target_minimum_bytes,
        "target_bytes_maximum": end.cache_target_maximum_bytes, "target_bytes_end": cache_target,
        "resident_bytes_peak": end.resident_bytes_peak,
        "pinned_staging_bytes": tele1.pinned_staging_bytes,
        "workspace_bytes_peak": end.workspace_bytes,
        "physical_frame_count_peak": end.physical_handles_created,
        "physical_handle_create_count": end.physical_handles_created,
        "physical_handle_release_count": end.physical_handles_released,
        "handle_reuse_count": end.handle_reuses, "mapping_count": end.mappings,
        "unmap_count": end.unmaps, "set_access_count": end.set_access_calls,
        "event_boundary_count": end.event_boundaries, "unsafe_remap_count": end.unsafe_remaps,
        "unsafe_transition_count": end.unsafe_transitions, "cache_hits": end.cache_hits,
        "cache_misses": end.cache_misses,
        "cache_hit_rate": end.cache_hits / (end.cache_hits + end.cache_misses)
        if end.cache_hits + end.cache_misses else 0.0,
        "clean_evictions": end.clean_evictions, "dirty_evictions": end.dirty_evictions,
        "writebacks_completed": end.writebacks_completed,
        "target_shrink_count": end.budget_shrinks, "target_grow_count": end.budget_grows,
        "target_oom_retry_count": end.target_oom_retries}
    flags = end.flags
    proof = {
        "logical_allocation_bytes": logical, "total_vram_bytes": dev0.total_memory_bytes,
        "maximum_cache_target_bytes": end.cache_target_maximum_bytes,
        "maximum_working_set_bytes": info.maximum_working_set_bytes,
        "workspace_cap_bytes": workspace_cap_bytes,
        "logical_data_exceeds_vram": logical > dev0.total_memory_bytes,
        "cache_smaller_than_logical": end.cache_target_maximum_bytes < logical,
        "tiled_execution_verified": workload["tiles_retired"] == workload["tiles_total"] > 0,
        "handles_reused": end.handle_reuses > 0,
        "stable_virtual_addresses_verified": bool(flags & 1),
        "set_access_after_map_verified": end.mappings == end.set_access_calls,
        "event_boundaries_verified": end.unsafe_remaps == 0,
        "no_physical_aliases_verified": bool(flags & 2),
        # The reference sets this from writebacks_completed > 0
        # (src/gemm_bench/executor.cpp:1117); every C byte of every pass must
        # also have been written back (evicted, or flushed by the verifying read).
        "dirty_writeback_verified": (end.writebacks_completed > 0
                                     and end.dirty_evictions <= end.writebacks_completed
                                     and workload["bytes_d2h"] >= m * n * 4 * passes),
        "cache_target_respected": end.resident_bytes_peak <= end.cache_target_maximum_bytes,
        "workspace_bounded": end.workspace_bytes <= workspace_cap_bytes,
        "all_workloads_match_reference": match, "raw_virtual_addresses_omitted": True}
    cleanup_ok = (end.mappings == end.unmaps
                  and end.physical_handles_created == end.physical_handles_released
                  and end.resident_bytes == 0)
    mem_total, mem_avail = _meminfo()
    ids = identifiers_included
    report = {
        "schema_version": 1, "report_type": "xvram.gemm_bench",
        "generated_at_utc": started_utc.strftime("%Y-%m-%dT%H:%M:%SZ"),
        "build": _build_section(),
        "system": {"os_name": platform.system() or "unknown", "os_version": platform.release(),
                   "architecture": platform.machine() or "unknown",
                   "logical_processor_count": os.cpu_count() or 0,
                   "physical_memory_bytes": mem_total, "available_memory_bytes": mem_avail},
        "device": {
            "ordinal": device_ordinal, "name": dev0.name.decode() or "unknown",
            "uuid": None, "luid": None,
            "pci_bus_id": (dev0.pci_bus_id.decode() or None) if ids else None,
            "driver_model": None, "total_memory_bytes": dev0.total_memory_bytes,
            "free_memory_bytes_start": dev0.free_memory_bytes,
            "free_memory_bytes_end": dev_end.free_memory_bytes,
            "safe_device_budget_bytes": max(0, dev0.free_memory_bytes - device_headroom_bytes),
            "wddm_budget_bytes_start": None, "wddm_usage_bytes_start": None,
            "wddm_available_bytes_start": None, "wddm_available_bytes_minimum": None,
            "wddm_available_bytes_end": None, "vmm_supported": bool(dev0.vmm_supported),
            "uva_supported": True,
            "minimum_granularity_bytes": dev0.granularity_minimum_bytes or None,
            "recommended_granularity_bytes": dev0.granularity_recommended_bytes or None,
            "compute_capability_major": dev0.compute_major,
            "compute_capability_minor": dev0.compute_minor},
        "configuration": {
            "requested_device_ordinal": device_ordinal, "requested_m": m, "requested_n": n,
            "requested_k": k, "scenario": "gemm", "a_data_type": "fp32", "b_data_type": "fp32",
            "c_data_type": "fp32", "compute_mode": "fp32_strict", "a_layout": "column_major",
            "b_layout": "column_major", "c_layout": "column_major", "a_operation": op_a,
            "b_operation": op_b, "alpha": 1.0, "beta": 0.0, "requested_chunk_bytes": chunk_bytes,
            "effective_chunk_bytes": info.maximum_working_set_bytes // 3,
            "requested_cache_target_bytes": cache_target_bytes or None,
            "initial_cache_target_bytes": tele_setup.cache_target_bytes,
            "requested_workspace_cap_bytes": workspace_cap_bytes,
            "effective_workspace_cap_bytes": workspace_cap_bytes,
            "context_mode": "isolated", "policy": policy,
            "staging_slots": session.config.staging_slots,
            "prefetch_distance": session.config.prefetch_distance, "passes": passes,
            "budget_poll_ms": session.config.budget_poll_ms, "stall_timeout_ms": 5000,
            "timeout_ms": 3600000, "max_tile_ms": session.config.max_transaction_ms or 250,
            "identifiers_included": ids},
        "plans": [{
            "plan_id": 1, "status": "completed" if match else "failed", "m": m, "n": n, "k": k,
            "a_data_type": "fp32", "b_data_type": "fp32", "c_data_type": "fp32",
            "effective_compute_mode": _COMPUTE_NAMES.get(info.effective_compute_mode, "fp32_strict"),
            "tile_m": info.tile_m, "tile_n": info.tile_n, "tile_k": info.tile_k,
            "tile_count": info.tile_count,
            "maximum_working_set_bytes": info.maximum_working_set_bytes,
            "workspace_bytes": info.workspace_bytes, "uses_cublas_lt": False,
            "heuristic_algorithm_count": None, "replan_count": 0}],
        "workloads": [workload],
        "numerics": {
            "validation_mode": "structured", "reference_precision": "analytic",
            "absolute_tolerance": 0.0, "relative_tolerance": 0.0,
            "maximum_absolute_error": max_abs, "maximum_relative_error": None,
            "elements_verified": m * n * passes, "mismatch_count": mismatches,
            "first_mismatch_byte_offset": first_bad, "expected_digest128": d_exp.hexdigest(),
            "output_digest128": d_out.hexdigest(), "all_results_match": match},
        "cache": cache,
        "telemetry": {
            "cuda_driver_version": end.cuda_driver_version, "cublas_version": None,
            "cublas_lt_version": None, "cublas_lt_available": None,
            "cublas_library_source": None, "algorithms_selected": end.algorithm_selections,
            "algorithm_cache_hits": end.algorithm_cache_hits,
            "budget_sample_count": end.budget_sample_count,
            "cuda_free_bytes_minimum": end.cuda_free_bytes_minimum,
            "cuda_free_bytes_end": end.cuda_free_bytes_end,
            "wddm_available_bytes_minimum": None, "wddm_available_bytes_end": None,
            "replans": 0, "watchdog_rejections": end.watchdog_rejections,
            "total_elapsed_ms": total_ms, "plan_timing": _timing([plan_ms]),
            "tile_timing": _timing(kernel_ms), "gemm_timing": _timing(gemm_ms),
            "h2d_timing": _timing(h2d_ms), "d2h_timing": _timing(d2h_ms),
            "writeback_timing": _timing(d2h_ms)},
        "proof": proof,
        "outcome": {"status": "completed" if match and cleanup_ok else "failed",
                    "reason": None if match and cleanup_ok else
                    ("reference_mismatch" if not match else "cleanup_incomplete"),
                    "exit_code": 0 if match and cleanup_ok else 70,
                    "stage": None, "operation": None, "native_code": None, "native_name": None,
                    "message": None, "plan_id": None, "tile_sequence": None,
                    "logical_byte_offset": first_bad},
        "cleanup": {k_: cleanup_ok for k_ in (
            "complete", "operations_drained", "events_drained", "events_destroyed",
            "streams_destroyed", "cublas_handles_destroyed", "mappings_removed",
            "physical_handles_released", "workspace_released", "virtual_reservations_released",
            "pinned_staging_released", "host_backing_released", "context_released")},
        "diagnostics": [],
    }
    report["cleanup"]["worker_terminated"] = True
    return report


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--m", type=int, required=True)
    ap.add_argument("--n", type=int, required=True)
    ap.add_argument("--k", type=int, required=True)
    ap.add_argument("--op-a", choices=["n", "t"], default="n")
    ap.add_argument("--op-b", choices=["n", "t"], default="t")
    ap.add_argument("--chunk-bytes", type=int, default=64 << 20)
    ap.add_argument("--cache-target-bytes", type=int, default=0)
    ap.add_argument("--passes", type=int, default=1)
    ap.add_argument("--policy", choices=["clock", "lru"], default="clock")
    ap.add_argument("--out", required=True)
    args = ap.parse_args(argv)
    report = run_report(load(), args.m, args.n, args.k, args.op_a, args.op_b, args.chunk_bytes,
                        args.cache_target_bytes, passes=args.passes, policy=args.policy)
    with open(args.out, "w") as f:
        json.dump(report, f, indent=1)
    return report["outcome"]["exit_code"]


if __name__ == "__main__":
    sys.exit(main())
