#!/usr/bin/env python3
"""bench.py — out-of-core FP32 SGEMM through the xVRAM C ABI on one MI355X.

Default workload (BASELINE.json metric "out-of-core FP32 SGEMM TFLOP/s at 3x
VRAM budget; H2D GB/s vs link peak"): the north-star GEMM, C = A * B^T with
M = N = K = 65536 (A, B, C = 3 x 16 GiB of pinned host memory) under a 16 GiB
VRAM budget of 1 GiB frames (operands = 3x the budget). A "step" is one
complete gemm_execute: every A/B panel streamed from host RAM, every C tile
written back (by the next step, or by the drain that ends the timed region).

Prints one JSON line. ``value`` = 2MNK / wall time per step (inputs resident in
host memory, as the ABI defines them). A step is one gemm_execute; the timed
region of the K steps ends with one session_drain, so every C byte is back in
host memory when the clock stops (the cache is write-back: a GEMM leaves its
last C tiles resident and dirty, the next execution writes them back while it
runs -- the resident config-3 workloads keep C cached between executions, as a
caller repeating a resident GEMM sees it -- and the drain writes back the
rest). ``ms_per_step`` = the timed region / K. ``roofline`` describes the dominant
kernel (the FP32-MFMA tile kernel): algorithmic FLOPs of its launches divided
by the time the kernels ran (the union of their intervals, from the HIP events
attached to every kernel dispatch on the library's compute lanes; trace file
written by the library). Launches of a few ms alternate between two compute
lanes and overlap at their ends, so there the union, not the sum of the
per-launch durations, is the kernels' time (``kernel_overlap_ms`` reports the
difference); ``kernel_ms_per_tile`` is that time per tile of the plan (one C
tile x one K panel; a launch covers one or two K panels, and the launches of
an operation's first K pass may run as several K-slice kernels). Other workloads:
``--workload`` (config 3's resident sweep, config 4, the config-5 chain, and
configs 1 and 2 as single GEMMs on device memory through the extension's
sgemm_device, timed with HIP events on the caller's stream).
``cpu_baseline`` times the FP64 reference loop (the oracle's restatement of
the reference's CPU GEMM) on a bounded sample of the same product, on all host
cores and, faithful to the reference example, on one thread. ``sample_check``
verifies the GPU result against the per-element bound on one full column per
tile column, one full row per tile row and seeded random elements
(oracle/sample.py), every element with its full K.
"""
from __future__ import annotations

import argparse
import ctypes
import glob
import json
import os
import sys
import tempfile
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

GiB = 1 << 30
MiB = 1 << 20
FP32_MFMA_PEAK_TFLOPS = 157.3     # 256 CU x 2.4 GHz x 256 FLOP/clk
PCIE5_X16_THEORETICAL_GBPS = 63.0  # per direction

OP_N, OP_T = 0, 1
WORKLOADS = {
    # name: (m, n, k, op_a, op_b, budget, frame, description)
    # 1 GiB frames: 8192 x 8192 C tiles with 32768-deep K panels (each C tile
    # passes through HBM twice, against 4 times with 512 MiB frames' 16384-deep
    # panels and 8 with 256 MiB frames); the 15 frames still hide the larger
    # A/B re-streaming (about 126 GB of H2D per step) under compute.
    "ns65536_nt_16g": (65536, 65536, 65536, OP_N, OP_T, 16 * GiB, 1024 * MiB,
                       "FP32 SGEMM N/T 65536^3, 3 x 16 GiB operands in pinned host RAM, "
                       "16 GiB VRAM budget (3x)"),
    "c4_32768_nt_2g": (32768, 32768, 32768, OP_N, OP_T, 2 * GiB, 64 * MiB,
                       "FP32 SGEMM N/T 32768^3, 3 x 4 GiB operands, 2 GiB VRAM budget"),
}
# Config 3, the resident sweep: N/N and N/T at 4096^3, 8192^3, 16384^3 (and the
# T/N and T/T forms beside them), one launch each (frames large enough for whole
# operands, budget unrestricted).
for _s, _frame in ((4096, 64 * MiB), (8192, 256 * MiB), (16384, 1024 * MiB)):
    for _oa, _ob in ((OP_N, OP_N), (OP_N, OP_T), (OP_T, OP_N), (OP_T, OP_T)):
        WORKLOADS[f"resident_{_s}_{'nt'[_oa]}{'nt'[_ob]}"] = (
            _s, _s, _s, _oa, _ob, 0, _frame,
            f"FP32 SGEMM {'NT'[_oa]}/{'NT'[_ob]} {_s}^3, fully resident (one launch)")
# One config-5 layer with its weights resident (Y^T = W X^T as the chain's
# T/N launch: 16384 x 256 x 16384, 1 GiB frames): 64 tiles of 256 x 256, so the
# launch splits K into 4 ranges (a single round of 256 workgroups).
WORKLOADS["resident_c5_layer_tn"] = (
    16384, 256, 16384, OP_T, OP_N, 0, 1024 * MiB,
    "FP32 SGEMM T/N 16384 x 256 x 16384 (one config-5 layer, weights resident; split K)")
# Single GEMMs on device memory through the extension's
# sgemm_device (the library's tile-kernel dispatch on the caller's buffers and
# stream): config 1 = 1024^3 N/N, alpha 1, beta 0; config 2 = 3001 x 2047 x
# 4099 in each form, alpha 1.5, beta 0.5. Both have fewer tiles than the chip
# has CUs, so their launches split K (the partials in a stream-ordered
# workspace of the library's).
DEVICE = {"device_c1_nn": (1024, 1024, 1024, OP_N, OP_N, 1.0, 0.0)}
for _oa, _ob in ((OP_N, OP_N), (OP_N, OP_T), (OP_T, OP_N), (OP_T, OP_T)):
    DEVICE[f"device_c2_{'nt'[_oa]}{'nt'[_ob]}"] = (3001, 2047, 4099, _oa, _ob, 1.5, 0.5)
# Square GEMMs whose 256 x 256 tiles leave a last round of the CUs mostly
# idle (4352^3: 289 tiles; 4608^3: 324; 6144^3: 576), which run as a head and
# a split tail, beside 4096^3 (256 tiles, whole rounds); and ragged ones
# (5000^3, 7000^3), which run as their interior tiles and two edge strips.
for _s in (4096, 4352, 4608, 6144, 5000, 7000):
    DEVICE[f"device_{_s}_nt"] = (_s, _s, _s, OP_N, OP_T, 1.0, 0.0)
# 4500^3 N/N and T/N: K not a multiple of 8, so the launch runs over K = 4496
# (an edge split) and then the last 4 K rows (thin-K kernel).
DEVICE["device_4500_nn"] = (4500, 4500, 4500, OP_N, OP_N, 1.0, 0.0)
DEVICE["device_4500_tn"] = (4500, 4500, 4500, OP_T, OP_N, 1.0, 0.0)
# Ragged with whole rounds of 256 x 256 tiles (32 x 32 tiles: 4 rounds): the
# whole launch on the ring kernels' edge instances; with K = 8190 (N/N) first
# over K = 8184, then the last 6 K rows.
DEVICE["device_8191_nt"] = (8191, 8191, 8192, OP_N, OP_T, 1.0, 0.0)
DEVICE["device_8191k_nn"] = (8191, 8191, 8190, OP_N, OP_N, 1.0, 0.0)
DEFAULT = "ns65536_nt_16g"
# Config 5: 8 x [Y = ReLU(X W^T + b)], X 256 x 16384 ~ N(0,1), W 16384 x 16384 and
# b ~ N(0, 1/16384), 2 GiB budget of 64 MiB frames; one step = one 8-layer forward.
CHAIN = {"name": "c5_chain_2g", "layers": 8, "batch": 256, "width": 16384,
         "budget": 2 * GiB, "frame": 64 * MiB}


def wall_roofline(flops: float, operand_bytes: int, c_bytes: int, resident: bool, steps: int,
                  link: dict) -> dict:
    """The time one step cannot beat: max(FLOP / FP32 MFMA peak, compulsory
    H2D / measured H2D peak, compulsory D2H / measured D2H peak). Out of
    core every step loads A and B and writes C back; a resident workload
    (the timed steps loaded nothing: its operands stayed cached) loads
    nothing and writes C back once, in the drain that ends the timed region."""
    terms = {"mfma": flops / (FP32_MFMA_PEAK_TFLOPS * 1e12),
             "h2d link": 0.0 if resident else operand_bytes / (link["h2d_gbps"] * 1e9),
             "d2h link": c_bytes / (steps if resident else 1) / (link["d2h_gbps"] * 1e9)}
    bound = max(terms, key=terms.get)
    return {"t_roof_s": terms[bound], "bound": bound, "resident": resident, "frac": None}


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# ---- host-link peak (pinned hipMemcpyAsync, measured in the same run) ------------

def link_peak(bytes_per_copy: int = 512 * MiB, repeats: int = 8) -> dict:
    hip = ctypes.CDLL("libamdhip64.so")
    vp = ctypes.c_void_p
    f = ctypes.c_float()
    h1, h2, d1, d2 = vp(), vp(), vp(), vp()
    s1, s2 = vp(), vp()
    ev = [vp() for _ in range(4)]

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: {rc}")

    ok(hip.hipSetDevice(0), "hipSetDevice")
    for p in (h1, h2):
        ok(hip.hipHostMalloc(ctypes.byref(p), ctypes.c_size_t(bytes_per_copy), 0), "hipHostMalloc")
    for p in (d1, d2):
        ok(hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(bytes_per_copy)), "hipMalloc")
    for s in (s1, s2):
        ok(hip.hipStreamCreateWithFlags(ctypes.byref(s), 1), "hipStreamCreate")
    for e in ev:
        ok(hip.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
    n = ctypes.c_size_t(bytes_per_copy)

    def timed(pairs):
        # pairs: list of (stream, dst, src, kind, start_event, stop_event)
        for s, dst, src, kind, e0, e1 in pairs:
            ok(hip.hipMemcpyAsync(dst, src, n, kind, s), "warmup copy")
        ok(hip.hipDeviceSynchronize(), "sync")
        for s, dst, src, kind, e0, e1 in pairs:
            ok(hip.hipEventRecord(e0, s), "record")
        for _ in range(repeats):
            for s, dst, src, kind, e0, e1 in pairs:
                ok(hip.hipMemcpyAsync(dst, src, n, kind, s), "copy")
        for s, dst, src, kind, e0, e1 in pairs:
            ok(hip.hipEventRecord(e1, s), "record")
        ok(hip.hipDeviceSynchronize(), "sync")
        out = []
        for s, dst, src, kind, e0, e1 in pairs:
            ok(hip.hipEventElapsedTime(ctypes.byref(f), e0, e1), "elapsed")
            out.append(repeats * bytes_per_copy / (f.value * 1e-3) / 1e9)
        return out

    h2d = timed([(s1, d1, h1, 1, ev[0], ev[1])])[0]
    d2h = timed([(s1, h1, d1, 2, ev[0], ev[1])])[0]
    duplex = timed([(s1, d1, h1, 1, ev[0], ev[1]), (s2, h2, d2, 2, ev[2], ev[3])])
    for p in (d1, d2):
        hip.hipFree(p)
    for p in (h1, h2):
        hip.hipHostFree(p)
    for e in ev:
        hip.hipEventDestroy(e)
    for s in (s1, s2):
        hip.hipStreamDestroy(s)
    return {"h2d_gbps": round(h2d, 2), "d2h_gbps": round(d2h, 2),
            "duplex_h2d_gbps": round(duplex[0], 2), "duplex_d2h_gbps": round(duplex[1], 2),
            "theoretical_gbps": PCIE5_X16_THEORETICAL_GBPS, "bytes_per_copy": bytes_per_copy}


def copy_calibration(nbytes: int) -> None:
    """Four device-to-device hipMemcpy calls of nbytes (HIP runs them as a copy kernel)."""
    hip = ctypes.CDLL("libamdhip64.so")
    src, dst = ctypes.c_void_p(), ctypes.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(ctypes.byref(p), ctypes.c_size_t(nbytes)) != 0:
            raise RuntimeError("hipMalloc failed")
    hip.hipMemset(src, 1, ctypes.c_size_t(nbytes))
    for _ in range(4):
        if hip.hipMemcpy(dst, src, ctypes.c_size_t(nbytes), 3) != 0:
            raise RuntimeError("hipMemcpy failed")
    hip.hipDeviceSynchronize()
    hip.hipFree(src)
    hip.hipFree(dst)
    log(f"copy calibration: 4 x {nbytes} bytes device-to-device")


# ---- trace analysis ------------------------------------------------------------------

def _union(intervals):
    total, cur_s, cur_e = 0.0, None, None
    merged = []
    for s, e in sorted(intervals):
        if cur_e is None or s > cur_e:
            if cur_e is not None:
                merged.append((cur_s, cur_e))
            cur_s, cur_e = s, e
        else:
            cur_e = max(cur_e, e)
    if cur_e is not None:
        merged.append((cur_s, cur_e))
    for s, e in merged:
        total += e - s
    return merged, total


def _intersection(a, b):
    i = j = 0
    total = 0.0
    while i < len(a) and j < len(b):
        s = max(a[i][0], b[j][0])
        e = min(a[i][1], b[j][1])
        if e > s:
            total += e - s
        if a[i][1] < b[j][1]:
            i += 1
        else:
            j += 1
    return total


def analyse(ops):
    """Busy times per operation (each operation's times are relative to its own
    start event, so intervals of different operations are never merged)."""
    k_busy = h_busy = d_busy = copy_busy = hidden = kernel_ms = 0.0
    span = first_kernel = host_enqueued = host_drained = 0.0
    launches = h2d_bytes = d2h_bytes = 0
    for op in ops:
        kernels = [(s, e) for s, e, _ in op["kernels"]]
        h2d = [(s, e) for s, e, _ in op["h2d"]]
        d2h = [(s, e) for s, e, _ in op["d2h"]]
        h2d_bytes += sum(b for _, _, b in op["h2d"])
        d2h_bytes += sum(b for _, _, b in op["d2h"])
        launches += len(kernels)
        kernel_ms += sum(e - s for s, e in kernels)
        k_union, kb = _union(kernels)
        hb = _union(h2d)[1]
        db = _union(d2h)[1]
        copies_union, cb = _union(h2d + d2h)
        k_busy += kb
        h_busy += hb
        d_busy += db
        copy_busy += cb
        hidden += _intersection(copies_union, k_union)
        span += max(e for s, e in kernels + h2d + d2h)
        first_kernel += min(s for s, e in kernels)
        host = op.get("host") or [0.0, 0.0]
        host_enqueued += host[0]
        host_drained += host[1]
    n = max(1, len(ops))
    return {
        # Per operation, averaged: the device timeline (from the operation's
        # start event to its last kernel or copy), the first kernel's start,
        # and host time from begin_operation to the last enqueue and to the
        # device drained.
        "op_timeline_ms": {"device_span": span / n, "first_kernel_start": first_kernel / n,
                           "kernel_idle_in_span": (span - k_busy) / n,
                           "host_last_enqueue": host_enqueued / n,
                           "host_drained": host_drained / n},
        "launches": launches,
        "kernel_ms_total": kernel_ms,
        "kernel_busy_ms": k_busy,
        "h2d_bytes": h2d_bytes, "d2h_bytes": d2h_bytes,
        "h2d_busy_ms": h_busy, "d2h_busy_ms": d_busy,
        "h2d_gbps_while_copying": h2d_bytes / (h_busy * 1e-3) / 1e9 if h_busy else None,
        "d2h_gbps_while_copying": d2h_bytes / (d_busy * 1e-3) / 1e9 if d_busy else None,
        "copy_time_hidden_fraction": hidden / copy_busy if copy_busy else None,
    }


# ---- operands ------------------------------------------------------------------------

def synth_lib():
    lib = ctypes.CDLL(os.path.join(ROOT, "xvram_amd", "lib", "libxvram_synth.so"))
    fp = ctypes.POINTER(ctypes.c_float)
    u64 = ctypes.c_uint64
    lib.synth_fill_uniform.argtypes = [fp, u64, u64, u64]
    lib.synth_fill_uniform_strided.argtypes = [fp, u64, u64, u64, u64, u64, u64]
    lib.synth_fill_normal.argtypes = [fp, u64, u64, u64, ctypes.c_double]
    return lib


def normal(synth, count: int, seed: int, sigma: float) -> np.ndarray:
    out = np.empty(count, dtype=np.float32)
    synth.synth_fill_normal(out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), count, seed, 0,
                            sigma)
    return out


def fill_allocation(synth, alloc, elements: int, seed: int, chunk_elems: int = 256 * MiB):
    buf = np.empty(min(chunk_elems, elements), dtype=np.float32)
    done = 0
    while done < elements:
        n = min(chunk_elems, elements - done)
        view = buf[:n]
        synth.synth_fill_uniform(view.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), n, seed, done)
        alloc.write(view, offset=done * 4)
        done += n


# ---- CPU baseline ----------------------------------------------------------------------

def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(a_seeded, b_seeded, m, n, k, seconds):
    """The oracle's FP64 loop (examples/preview-gemm/main.cpp:107-119 restated)
    on C[0:r, 0:cols] of the same product with full K: on every host thread
    (cols scaled to about `seconds`) and, as the reference example runs it, on
    one thread (a narrower sample scaled to about `seconds` / 2). Rates are
    2 r cols K / time."""
    import oracle

    threads = os.cpu_count() or 1
    r = min(m, 1024)
    a_s = a_seeded.rows(range(r))

    def timed(cols, nthreads):
        b_s = b_seeded.cols(range(cols))
        t = time.perf_counter()
        oracle.sgemm_f64(a_s, b_s, threads=nthreads)
        return time.perf_counter() - t

    out = {"unit": "TFLOP/s", "kind": "port", "cores": threads, "nproc": os.cpu_count(),
           "cpu_model": cpu_model()}
    probe_cols = min(n, 2 * threads)
    probe = timed(probe_cols, threads)
    cols = int(min(n, max(probe_cols, probe_cols * seconds / max(probe, 1e-3))))
    secs = timed(cols, threads)
    out["value"] = round(2.0 * r * cols * k / secs / 1e12, 6)
    out["sample"] = (f"C[0:{r}, 0:{cols}] of the same {m}x{n}x{k} product with full K (FP64 "
                     f"accumulation over FP32 inputs, {secs:.1f} s on {threads} threads)")
    probe1 = timed(1, 1)
    cols1 = int(min(n, max(1, (seconds / 2) / max(probe1, 1e-3))))
    secs1 = timed(cols1, 1)
    out["single_thread"] = {
        "value": round(2.0 * r * cols1 * k / secs1 / 1e12, 6), "unit": "TFLOP/s", "cores": 1,
        "sample": f"C[0:{r}, 0:{cols1}] with full K ({secs1:.1f} s on one thread)"}
    log(f"cpu baseline: {out['value']} TFLOP/s on {threads} threads, "
        f"{out['single_thread']['value']} on one ({out['cpu_model']})")
    return out


def cpu_sweep(seconds: float) -> dict:
    """The reference's CPU GEMM (examples/preview-gemm/main.cpp:107-119, the
    oracle's FP64 loop) on every BASELINE configuration, in its two forms: all
    host threads and one thread. A form whose full problem would take more
    than about `seconds` is timed on a leading column subset of the same
    product and extrapolated linearly in the column count (labelled so)."""
    import oracle
    from oracle.sample import SeededOperand

    threads = os.cpu_count() or 1
    configs = [("C1 1024^3 NN", 1024, 1024, 1024, OP_N, OP_N, 1.0, 0.0)]
    for oa, ob in ((OP_N, OP_N), (OP_N, OP_T), (OP_T, OP_N), (OP_T, OP_T)):
        configs.append((f"C2 3001x2047x4099 {'NT'[oa]}{'NT'[ob]}", 3001, 2047, 4099, oa, ob, 1.5,
                        0.5))
    for size in (4096, 8192, 16384):
        for ob in (OP_N, OP_T):
            configs.append((f"C3 {size}^3 N{'NT'[ob]}", size, size, size, OP_N, ob, 1.0, 0.0))
    configs.append(("C4 32768^3 NT", 32768, 32768, 32768, OP_N, OP_T, 1.0, 0.0))
    configs.append(("NS 65536^3 NT", 65536, 65536, 65536, OP_N, OP_T, 1.0, 0.0))
    out = {"cpu_model": cpu_model(), "nproc": os.cpu_count(), "threads_all": threads,
           "unit": "TFLOP/s", "configs": []}
    for name, m, n, k, oa, ob, alpha, beta in configs:
        a = SeededOperand(11, *((m, k) if oa == OP_N else (k, m)), oa == OP_T)
        b = SeededOperand(12, *((k, n) if ob == OP_N else (n, k)), ob == OP_T)
        rows = min(m, 1024) if m * k > (1 << 28) else m   # large A: a row block
        a_s = a.rows(range(rows)) if rows < m else a.full()
        c0 = None
        if beta != 0.0:
            c0 = SeededOperand(13, m, n, False).full()[:rows, :]
        entry = {"config": name}
        for label, nthreads in (("all_threads", threads), ("one_thread", 1)):
            cols = min(n, 2 * nthreads)
            t = time.perf_counter()
            oracle.sgemm_f64(a_s, b.cols(range(cols)), alpha, beta,
                             None if c0 is None else np.asfortranarray(c0[:, :cols]),
                             threads=nthreads)
            probe = max(time.perf_counter() - t, 1e-4)
            full_cols = n if rows == m else None
            want = int(min(n, max(cols, cols * seconds / probe)))
            if want > cols:
                t = time.perf_counter()
                oracle.sgemm_f64(a_s, b.cols(range(want)), alpha, beta,
                                 None if c0 is None else np.asfortranarray(c0[:, :want]),
                                 threads=nthreads)
                secs, cols = time.perf_counter() - t, want
            else:
                secs = probe
            rate = 2.0 * rows * cols * k / secs / 1e12
            whole = full_cols is not None and cols == n
            entry[label] = {"value": round(rate, 6), "threads": nthreads,
                            "sample": f"C[0:{rows}, 0:{cols}] with full K ({secs:.2f} s)",
                            "extrapolated": not whole,
                            "full_problem_s": round(2.0 * m * n * k / (rate * 1e12), 1)}
        log(f"cpu sweep {name}: {entry['all_threads']['value']} TFLOP/s on {threads} threads, "
            f"{entry['one_thread']['value']} on one")
        out["configs"].append(entry)
    return out


# ---- config 5: the inference chain ---------------------------------------------------

def run_chain(args, xv, lib, synth, link) -> int:
    """One step = one forward of CHAIN["layers"] x [Y = ReLU(X W^T + b)]: each
    layer is one GEMM plan with a fused bias+ReLU epilogue (extension table),
    the 8 operations are submitted back to back, weights stream from pinned host
    memory through the 2 GiB budget, and the step ends with the output read
    back to the host."""
    import oracle

    L, batch, width = CHAIN["layers"], CHAIN["batch"], CHAIN["width"]
    std = width ** -0.5
    session = xv.Session(lib, chunk_size_bytes=CHAIN["frame"], cache_target_bytes=CHAIN["budget"])
    t0 = time.time()
    acts = [session.allocation(batch * width * 4) for _ in range(L + 1)]
    x0 = normal(synth, batch * width, 5000, 1.0)
    acts[0].write(x0)
    weights, biases, plans = [], [], []
    for l in range(L):
        w_alloc = session.allocation(width * width * 4)
        w_alloc.write(normal(synth, width * width, 6000 + l, std))
        b_alloc = session.allocation(width * 4)
        b_alloc.write(normal(synth, width, 7000 + l, std))
        weights.append(w_alloc)
        biases.append(b_alloc)
        plans.append(xv.GemmPlan(
            session, xv.matrix(acts[l], batch, width, width, xv.abi.ROW_MAJOR),
            xv.matrix(w_alloc, width, width, width, xv.abi.ROW_MAJOR),
            xv.matrix(acts[l + 1], batch, width, width, xv.abi.ROW_MAJOR), OP_N, OP_T,
            epilogue=xv.epilogue(b_alloc, xv.abi.BIAS_PER_COLUMN, relu=True)))
    info = plans[0].info()
    log(f"chain ready: {L} x {width * width * 4 / GiB:.0f} GiB weights ({time.time() - t0:.1f}s); "
        f"layer plan tiles {info.tile_m}x{info.tile_n}x{info.tile_k}, {info.tile_count} tiles")

    y_out = np.empty(batch * width, dtype=np.float32)

    def forward():
        """The 8 layers submitted back to back, then the output read back
        (intermediate activations stay in the device cache: each layer's C
        tiles are the next layer's input panels)."""
        ops = [p.submit() for p in plans]
        for op in ops:
            st, res = op.wait()
            if st != 0 or res.result != 0:
                raise RuntimeError(f"layer failed: {st} {res.result} {op.error().message}")
            op.release()
        acts[L].read_into(y_out)

    trace_path = os.environ["XVRAM_TRACE_FILE"]
    for i in range(args.warmup):
        t = time.perf_counter()
        forward()
        log(f"warmup {i}: {time.perf_counter() - t:.3f}s")
    with open(trace_path, "a"):
        pass
    before = sum(1 for _ in open(trace_path))
    tele0 = session.telemetry()
    times = []
    flops = 2.0 * L * batch * width * width
    for i in range(args.steps):
        t = time.perf_counter()
        forward()
        times.append(time.perf_counter() - t)
        log(f"step {i}: {times[-1]:.3f}s = {flops / times[-1] / 1e12:.1f} TFLOP/s")
    tele1 = session.telemetry()
    ops = [json.loads(line) for line in open(trace_path).readlines()[before:]]
    if args.trace_out:
        with open(args.trace_out, "w") as out:
            out.writelines(json.dumps(op) + "\n" for op in ops)
    stats = analyse(ops)
    step_s = sum(times) / len(times)

    # Per-layer check on the first `rows` batch rows (rows are independent through
    # the chain): FP64 forward of the FP32 input each layer actually consumed.
    rows = 8
    worst = 0.0
    violations = 0
    y64 = x0.reshape(batch, width)[:rows].astype(np.float64)
    for l in range(L):
        xin = acts[l].read(rows * width * 4, dtype=np.float32).reshape(rows, width).astype(np.float64)
        got = acts[l + 1].read(rows * width * 4, dtype=np.float32).reshape(rows, width)
        w = normal(synth, width * width, 6000 + l, std).reshape(width, width).astype(np.float64)
        bvec = normal(synth, width, 7000 + l, std).astype(np.float64)
        pre = xin @ w.T + bvec
        absab = np.abs(xin) @ np.abs(w).T + np.abs(bvec)
        bound = 4 * width * 2.0 ** -24 * absab
        err = np.abs(got - np.maximum(pre, 0.0))
        violations += int(np.count_nonzero(err > bound))
        worst = max(worst, float((err / np.maximum(bound, 1e-300)).max()))
        y64 = np.maximum(y64 @ w.T + bvec, 0.0)
        del w, absab
    final = acts[L].read(rows * width * 4, dtype=np.float32).reshape(rows, width)
    e2e = float(np.abs(final - y64).max() / max(np.abs(y64).max(), 1e-300))
    log(f"chain check rows 0:{rows}: violations={violations} err/bound={worst:.3e} "
        f"end-to-end rel={e2e:.3e}")

    cpu = None
    if not args.no_cpu_baseline:
        # The oracle's FP64 loop on layer 0: Y[0:r, 0:width] with full K, r scaled
        # from a probe so the timed work is about --cpu-seconds (at most the batch).
        threads = os.cpu_count() or 1
        w0t = np.asfortranarray(normal(synth, width * width, 6000, std).reshape(width, width).T)
        x_all = x0.reshape(batch, width)
        t = time.perf_counter()
        oracle.sgemm_f64(np.asfortranarray(x_all[:1]), w0t, threads=threads)
        probe = time.perf_counter() - t
        r = int(min(batch, max(1, args.cpu_seconds / max(probe, 1e-3))))
        t = time.perf_counter()
        oracle.sgemm_f64(np.asfortranarray(x_all[:r]), w0t, threads=threads)
        cpu_s = time.perf_counter() - t
        cpu = {"value": round(2.0 * r * width * width / cpu_s / 1e12, 6), "unit": "TFLOP/s",
               "cores": threads, "kind": "port", "nproc": os.cpu_count(),
               "cpu_model": cpu_model(),
               "sample": f"layer 0, Y[0:{r}, 0:{width}] with full K={width} (FP64 accumulation "
                         f"over FP32 inputs, {cpu_s:.1f} s on {threads} threads)"}
        # One thread, as the reference example runs: one batch row.
        t = time.perf_counter()
        oracle.sgemm_f64(np.asfortranarray(x_all[:1]), w0t, threads=1)
        cpu_1 = time.perf_counter() - t
        cpu["single_thread"] = {"value": round(2.0 * width * width / cpu_1 / 1e12, 6),
                                "unit": "TFLOP/s", "cores": 1,
                                "sample": f"layer 0, Y[0:1, 0:{width}] ({cpu_1:.1f} s on one thread)"}
        del w0t

    # Weights and biases of every layer and the input; the output comes back.
    h2d_compulsory = L * (width * width * 4 + width * 4) + batch * width * 4
    d2h_compulsory = batch * width * 4
    t_roof = max(flops / (FP32_MFMA_PEAK_TFLOPS * 1e12), h2d_compulsory / (link["h2d_gbps"] * 1e9),
                 d2h_compulsory / (link["d2h_gbps"] * 1e9))
    kernel_tflops = flops * args.steps / (stats["kernel_busy_ms"] * 1e-3) / 1e12
    h2d_gbps = stats["h2d_gbps_while_copying"]
    result = {
        "metric": "config-5 inference chain FP32 TFLOP/s (8 x Linear 16384 + bias + ReLU, "
                  "2 GiB budget); H2D GB/s vs link peak",
        "value": round(flops / step_s / 1e12, 3), "unit": "TFLOP/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "fp32",
        "data": "synthetic (seeded N(0,1) input, N(0,1/16384) weights and biases)",
        "config": {"workload": CHAIN["name"], "layers": L, "batch": batch, "width": width,
                   "vram_budget_bytes": CHAIN["budget"], "frame_bytes": CHAIN["frame"],
                   "tile": [info.tile_m, info.tile_n, info.tile_k],
                   "tiles_per_step": L * info.tile_count,
                   "kernels_per_step": stats["launches"] / args.steps,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(kernel_tflops, 3),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(kernel_tflops / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": None},
        "roofline_wall": {"t_roof_s": t_roof, "bound": "h2d link", "frac": round(t_roof / step_s, 4)},
        "cpu_baseline": cpu,
        "link": {
            "h2d_gbps_while_copying": round(h2d_gbps, 2) if h2d_gbps else None,
            "measured_peak": link,
            "h2d_frac_of_measured_peak": round(h2d_gbps / link["h2d_gbps"], 4) if h2d_gbps else None,
            "h2d_bytes_per_step": stats["h2d_bytes"] // args.steps,
            "h2d_compulsory_bytes_per_step": h2d_compulsory,
            "d2h_bytes_per_step": stats["d2h_bytes"] // args.steps,
            "copy_time_hidden_fraction": round(stats["copy_time_hidden_fraction"], 4)
            if stats["copy_time_hidden_fraction"] is not None else None,
        },
        "cache": {f: getattr(tele1, f) - getattr(tele0, f) for f in (
            "bytes_h2d", "bytes_d2h", "cache_hits", "cache_misses", "clean_evictions",
            "dirty_evictions", "writebacks_completed", "handle_reuses")},
        "sample_check": {"rows": rows, "elements": rows * width * L, "violations": violations,
                         "max_err_over_bound": worst, "end_to_end_rel_vs_fp64": e2e},
    }
    for p in plans:
        p.release()
    session.close()
    t = session.telemetry()
    result["teardown"] = {"mappings": t.mappings, "unmaps": t.unmaps,
                          "handles_created": t.physical_handles_created,
                          "handles_released": t.physical_handles_released,
                          "unsafe_transitions": t.unsafe_transitions,
                          "unsafe_remaps": t.unsafe_remaps}
    session.release()
    print(json.dumps(result), flush=True)
    return 0 if violations == 0 else 1


def run_device(args, xv, lib, synth) -> int:
    """One GEMM per step on device memory through sgemm_device; the K steps
    are enqueued back to back on one stream and timed with HIP events on it.
    The result of one more launch from the initial C is checked on every
    element against the FP64 oracle after the timed region."""
    import ctypes

    from xvram_amd import abi

    m, n, k, op_a, op_b, alpha, beta = DEVICE[args.workload]
    rt = ctypes.CDLL("libamdhip64.so")

    def ok(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed: hipError {rc}")

    def stored(rows, cols, seed):
        # Element (r, c) is draw c * rows + r of the seeded stream whatever the
        # padding (so the spread check can regenerate it); padding rows are 0.
        ld = (rows + 3) // 4 * 4
        vals = np.empty(rows * cols, dtype=np.float32)
        synth.synth_fill_uniform(vals.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                 vals.size, seed, 0)
        host = np.zeros((cols, ld), dtype=np.float32)
        host[:, :rows] = vals.reshape(cols, rows)
        host = host.reshape(-1)
        ptr = ctypes.c_void_p()
        ok(rt.hipMalloc(ctypes.byref(ptr), ctypes.c_size_t(host.nbytes)), "hipMalloc")
        ok(rt.hipMemcpy(ptr, host.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(host.nbytes),
                        1), "hipMemcpy")
        return ptr, ld, host

    a_rows, a_cols = (m, k) if op_a == OP_N else (k, m)
    b_rows, b_cols = (k, n) if op_b == OP_N else (n, k)
    pa, lda, a_host = stored(a_rows, a_cols, 1)
    pb, ldb, b_host = stored(b_rows, b_cols, 2)
    pc, ldc, c_host = stored(m, n, 3)
    stream = ctypes.c_void_p()
    ok(rt.hipStreamCreateWithFlags(ctypes.byref(stream), 1), "hipStreamCreateWithFlags")
    events = [ctypes.c_void_p(), ctypes.c_void_p()]
    for e in events:
        ok(rt.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
    d = abi.sgemm_device_init()
    d.a, d.b, d.c = pa.value, pb.value, pc.value
    d.m, d.n, d.k, d.lda, d.ldb, d.ldc = m, n, k, lda, ldb, ldc
    d.operation_a, d.operation_b = op_a, op_b
    d.alpha, d.beta = alpha, beta

    def launch():
        status = lib.ext.sgemm_device(ctypes.byref(d), stream)
        if status != abi.SUCCESS:
            raise RuntimeError(f"sgemm_device returned {status}")

    for _ in range(args.warmup):
        launch()
    ok(rt.hipStreamSynchronize(stream), "hipStreamSynchronize")
    ok(rt.hipEventRecord(events[0], stream), "hipEventRecord")
    for _ in range(args.steps):
        launch()
    ok(rt.hipEventRecord(events[1], stream), "hipEventRecord")
    ok(rt.hipEventSynchronize(events[1]), "hipEventSynchronize")
    elapsed = ctypes.c_float()
    ok(rt.hipEventElapsedTime(ctypes.byref(elapsed), events[0], events[1]), "hipEventElapsedTime")
    step_s = elapsed.value * 1e-3 / args.steps
    flops = 2.0 * m * n * k
    value = flops / step_s / 1e12
    log(f"{args.steps} launches: {step_s * 1e6:.1f} us each = {value:.1f} TFLOP/s")

    # One launch from the initial C, checked on every element.
    ok(rt.hipMemcpy(pc, c_host.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(c_host.nbytes), 1),
       "hipMemcpy")
    launch()
    ok(rt.hipStreamSynchronize(stream), "hipStreamSynchronize")
    out = np.empty_like(c_host)
    ok(rt.hipMemcpy(out.ctypes.data_as(ctypes.c_void_p), pc, ctypes.c_size_t(out.nbytes), 2),
       "hipMemcpy")
    for ptr in (pa, pb, pc):
        ok(rt.hipFree(ptr), "hipFree")
    for e in events:
        ok(rt.hipEventDestroy(e), "hipEventDestroy")
    ok(rt.hipStreamDestroy(stream), "hipStreamDestroy")

    import oracle

    if flops <= 6e10 or (alpha, beta) != (1.0, 0.0):
        # Every element against the FP64 oracle (configs 1 and 2 among them).
        def logical(host, rows, cols, ld, op):
            st = host.reshape(cols, ld)[:, :rows].T
            return np.asfortranarray(st if op == OP_N else st.T)

        c0 = np.asfortranarray(c_host.reshape(n, ldc)[:, :m].T)
        ref, absab = oracle.sgemm_f64(logical(a_host, a_rows, a_cols, lda, op_a),
                                      logical(b_host, b_rows, b_cols, ldb, op_b), alpha, beta, c0)
        bad, _, ratio = oracle.check_bound(np.asfortranarray(out.reshape(n, ldc)[:, :m].T), k,
                                           ref, absab)
        elements = m * n
    else:
        # The spread sample (one full column per tile column, one full row per
        # tile row, seeded random elements) of an alpha 1, beta 0 product.
        from oracle.sample import SeededOperand, spread_check

        assert alpha == 1.0 and beta == 0.0
        check = spread_check(SeededOperand(1, a_rows, a_cols, op_a == OP_T),
                             SeededOperand(2, b_rows, b_cols, op_b == OP_T),
                             lambda j0, j1: out.reshape(n, ldc)[j0:j1, :m].T, 256, 256, seed=7,
                             randoms=1024)
        bad, ratio, elements = check["violations"], check["max_err_over_bound"], check["elements"]
    log(f"check: {elements} elements, violations={bad} err/bound={ratio:.3e}")
    frac = value / FP32_MFMA_PEAK_TFLOPS
    result = {
        "metric": "out-of-core FP32 SGEMM TFLOP/s at 3x VRAM budget; H2D GB/s vs link peak",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded U[-1,1) operands, counter-based generator)",
        "config": {"workload": args.workload, "m": m, "n": n, "k": k, "op_a": "NT"[op_a],
                   "op_b": "NT"[op_b], "alpha": alpha, "beta": beta,
                   "description": "one GEMM on device memory through sgemm_device",
                   "step": "one sgemm_device call; the K calls are enqueued back to back on "
                           "one stream and timed with HIP events on it",
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(value, 3), "peak": FP32_MFMA_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(frac, 4), "traffic": None},
        "cpu_baseline": None,
        "check": {"elements": elements, "violations": bad, "max_err_over_bound": ratio},
    }
    print(json.dumps(result), flush=True)
    return 0 if bad == 0 else 1


# ---- main ----------------------------------------------------------------------------

def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(WORKLOADS) + [CHAIN["name"]] + sorted(DEVICE),
                    default=DEFAULT)
    ap.add_argument("--cpu-seconds", type=float, default=15.0,
                    help="target CPU time of the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--frame-mib", type=int, default=0,
                    help="cache frame (chunk_size_bytes) in MiB instead of the workload's")
    ap.add_argument("--tile-hints", default="0,0,0", metavar="M,N,K",
                    help="tile_m/n/k hints of the GEMM plan (0 = the planner's choice)")
    ap.add_argument("--trace-out", default=None,
                    help="also keep the library's per-operation trace (JSON lines) here")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run 4 device-to-device copies of BYTES (a plain copy kernel of "
                         "known size, used to scale rocprofv3 FETCH_SIZE/WRITE_SIZE) and exit")
    ap.add_argument("--cpu-sweep", action="store_true",
                    help="only time the CPU reference GEMM (both forms) on every BASELINE "
                         "configuration and print it as one JSON line (no GPU)")
    args = ap.parse_args()
    if args.cpu_sweep:
        print(json.dumps(cpu_sweep(args.cpu_seconds)), flush=True)
        return 0
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one MI355X: the out-of-core path runs on a single GPU "
              f"(--gpus {args.gpus} is not supported; multi-GPU sharding is a design note only).",
              file=sys.stderr)
        return 2

    if args.workload in DEVICE:
        import xvram_amd as xv

        log(f"workload {args.workload}")
        return run_device(args, xv, xv.load(), synth_lib())
    trace_path = os.path.join(tempfile.mkdtemp(prefix="xvram_bench_"), "trace.jsonl")
    os.environ["XVRAM_TRACE_FILE"] = trace_path

    import xvram_amd as xv

    t0 = time.time()
    link = link_peak()
    log(f"link peak {link} ({time.time() - t0:.1f}s)")
    synth = synth_lib()
    lib = xv.load()
    if args.workload == CHAIN["name"]:
        log(f"workload {args.workload}")
        return run_chain(args, xv, lib, synth, link)
    m, n, k, op_a, op_b, budget, frame, desc = WORKLOADS[args.workload]
    if args.frame_mib:
        frame = args.frame_mib * MiB
        desc += f"; frames of {args.frame_mib} MiB instead of the workload's"
    log(f"workload {args.workload}: {desc}")
    cfg = dict(chunk_size_bytes=frame)
    if budget:
        cfg["cache_target_bytes"] = budget
    session = xv.Session(lib, **cfg)
    a_rows, a_cols = (m, k) if op_a == OP_N else (k, m)
    b_rows, b_cols = (k, n) if op_b == OP_N else (n, k)
    t0 = time.time()
    a = session.allocation(a_rows * a_cols * 4)
    b = session.allocation(b_rows * b_cols * 4)
    c = session.allocation(m * n * 4)
    fill_allocation(synth, a, a_rows * a_cols, 1)
    fill_allocation(synth, b, b_rows * b_cols, 2)
    log(f"operands ready: {3 * m * n * 4 / GiB:.1f} GiB pinned host ({time.time() - t0:.1f}s)")
    plan = xv.GemmPlan(session, xv.matrix(a, a_rows, a_cols, a_rows),
                       xv.matrix(b, b_rows, b_cols, b_rows), xv.matrix(c, m, n, m), op_a, op_b,
                       tile_hints=tuple(int(v) for v in args.tile_hints.split(",")))
    info = plan.info()
    log(f"plan: tiles {info.tile_m}x{info.tile_n}x{info.tile_k}, {info.tile_count} tiles")
    # The timed region ends with session_drain: every C byte is back in host
    # memory when the clock stops (the write-back cache leaves a GEMM's last C
    # tiles dirty on the device; the next execution writes them back while it
    # runs, and the drain writes back the last ones).
    for i in range(args.warmup):
        t = time.perf_counter()
        plan.execute()
        log(f"warmup {i}: {time.perf_counter() - t:.3f}s")
    session.drain()
    with open(trace_path, "a"):
        pass
    trace_lines_before = sum(1 for _ in open(trace_path))
    tele0 = session.telemetry()
    times = []
    t_start = time.perf_counter()
    for i in range(args.steps):
        t = time.perf_counter()
        plan.execute()
        times.append(time.perf_counter() - t)
        log(f"step {i}: {times[-1]:.3f}s = {2.0 * m * n * k / times[-1] / 1e12:.1f} TFLOP/s")
    t = time.perf_counter()
    session.drain()
    drain_s = time.perf_counter() - t
    total_s = time.perf_counter() - t_start
    log(f"final drain {drain_s * 1e3:.1f} ms")
    tele1 = session.telemetry()
    ops = [json.loads(line) for line in open(trace_path).readlines()[trace_lines_before:]]
    if args.trace_out:
        with open(args.trace_out, "w") as out:
            out.writelines(json.dumps(op) + "\n" for op in ops)
    stats = analyse(ops)

    flops = 2.0 * m * n * k
    step_s = total_s / args.steps  # the final drain is shared by the steps
    value = flops / step_s / 1e12
    kernel_tflops = flops * args.steps / (stats["kernel_busy_ms"] * 1e-3) / 1e12
    # Tiles of the plan (C tile x K panel); a launch covers one or two K panels
    # and the first pass's launches may run as several K-slice kernels
    # (cache-miss start), so kernels per step can differ.
    tiles_per_step = info.tile_count
    kernels_per_step = stats["launches"] / args.steps

    # Sample check: one full column per tile column, one full row per tile row
    # and seeded random elements, all with full K, against the FP64 oracle.
    from oracle.sample import SeededOperand, spread_check

    a_seeded = SeededOperand(1, a_rows, a_cols, op_a == OP_T)
    b_seeded = SeededOperand(2, b_rows, b_cols, op_b == OP_T)

    def read_columns(j0, j1):
        out = np.empty((j1 - j0) * m, dtype=np.float32)
        c.read_into(out, offset=j0 * m * 4)
        return out.reshape(j1 - j0, m).T

    t = time.perf_counter()
    check = spread_check(a_seeded, b_seeded, read_columns, info.tile_m, info.tile_n, seed=7,
                         randoms=1024)
    log(f"sample check: {check['elements']} elements ({len(check['full_columns'])} full columns, "
        f"{len(check['full_rows'])} full rows, {check['random_elements']} random), "
        f"violations={check['violations']} err/bound={check['max_err_over_bound']:.3e} "
        f"({time.perf_counter() - t:.1f}s)")
    bad = check["violations"]
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(a_seeded, b_seeded, m, n, k, args.cpu_seconds)

    # HBM traffic per launch from the committed rocprofv3 --pmc summary of this
    # workload's tile kernel (profiles/traffic_<kernel>_<workload>.txt), if any;
    # that summary describes the workload's own launch shape, so a run with a
    # different frame size or tile hints reports none.
    traffic = None
    overridden = bool(args.frame_mib) or any(int(v) for v in args.tile_hints.split(","))
    for traffic_file in sorted(glob.glob(os.path.join(ROOT, "profiles",
                                                      f"traffic_*_{args.workload}.txt"))):
        if overridden:
            break
        for line in open(traffic_file):
            if line.startswith("traffic_bytes_per_launch:"):
                traffic = int(float(line.split(":", 1)[1]))

    h2d_gbps = stats["h2d_gbps_while_copying"]
    result = {
        "metric": "out-of-core FP32 SGEMM TFLOP/s at 3x VRAM budget; H2D GB/s vs link peak",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic (seeded U[-1,1) operands, counter-based generator)",
        "config": {"workload": args.workload, "description": desc, "m": m, "n": n, "k": k,
                   "op_a": "NT"[op_a], "op_b": "NT"[op_b], "vram_budget_bytes": budget,
                   "frame_bytes": frame, "tile": [info.tile_m, info.tile_n, info.tile_k],
                   "tiles_per_step": tiles_per_step, "kernels_per_step": kernels_per_step,
                   "parallelism": "single GPU"},
        "roofline": {"bound": "mfma", "achieved": round(kernel_tflops, 3),
                     "peak": FP32_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(kernel_tflops / FP32_MFMA_PEAK_TFLOPS, 4), "traffic": traffic},
        "cpu_baseline": cpu,
        "link": {
            "h2d_gbps_while_copying": round(h2d_gbps, 2) if h2d_gbps else None,
            "d2h_gbps_while_copying": round(stats["d2h_gbps_while_copying"], 2)
            if stats["d2h_gbps_while_copying"] else None,
            "measured_peak": link,
            "h2d_frac_of_measured_peak": round(h2d_gbps / link["h2d_gbps"], 4) if h2d_gbps else None,
            "h2d_bytes_per_step": stats["h2d_bytes"] // args.steps,
            "d2h_bytes_per_step": stats["d2h_bytes"] // args.steps,
            "copy_time_hidden_fraction": round(stats["copy_time_hidden_fraction"], 4)
            if stats["copy_time_hidden_fraction"] is not None else None,
        },
        "roofline_wall": wall_roofline(flops, (a_rows * a_cols + b_rows * b_cols) * 4,
                                       m * n * 4, stats["h2d_bytes"] == 0, args.steps, link),
        "kernel_ms_per_tile": round(stats["kernel_busy_ms"] / max(1, tiles_per_step * args.steps), 4),
        "kernel_overlap_ms_per_step": round((stats["kernel_ms_total"] - stats["kernel_busy_ms"]) / args.steps, 3),
        "op_timeline_ms": {key: round(v, 3) for key, v in stats["op_timeline_ms"].items()},
        "cache": {f: getattr(tele1, f) - getattr(tele0, f) for f in (
            "bytes_h2d", "bytes_d2h", "cache_hits", "cache_misses", "clean_evictions",
            "dirty_evictions", "writebacks_completed", "handle_reuses", "event_boundaries")},
        "sample_check": check,
    }
    result["config"]["step"] = ("gemm_execute; the timed region ends with one session_drain "
                                f"({drain_s * 1e3:.1f} ms)")
    result["roofline_wall"]["frac"] = round(result["roofline_wall"]["t_roof_s"] / step_s, 4)
    plan.release()
    session.close()
    t = session.telemetry()
    result["teardown"] = {"mappings": t.mappings, "unmaps": t.unmaps,
                          "handles_created": t.physical_handles_created,
                          "handles_released": t.physical_handles_released}
    session.release()
    print(json.dumps(result), flush=True)
    return 0 if bad == 0 else 1


if __name__ == "__main__":
    sys.exit(main())
