"""CPU tests of cross-operation fills over libxvram_hostsim.so: while one GEMM's
last launches run, the session starts the first panel fills of the GEMM queued
next (carried past the running operation's end), so the host link does not idle
between queued operations.

The chains here are queued behind a transaction whose callback holds the
worker until every GEMM is submitted, so each operation's tail deterministically
sees the next one and the accounting is exact. Every layer reads the previous
layer's output, which is still cached (dirty) when the carry runs: those panels
are never carried (a fill from host memory would hold stale bytes); here they
are the previous layer's C tiles themselves, found in the cache."""
import threading

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import uniform

KiB = 1 << 10


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    yield lib
    lib.dll.xvram_hostsim_reset()


def run_chain(lib, oracle_mod, prefetch_distance, layers=4, m=96, n=40, cancel_last=False):
    """act[l+1] (m x n) = W[l] (m x m) @ act[l], column-major, all queued at once.
    Returns the activations read back and the telemetry delta of the chain."""
    s = xv.Session(lib, chunk_size_bytes=16 * KiB, cache_target_bytes=14 * 16 * KiB,
                   workspace_cap_bytes=0, device_headroom_bytes=0,
                   prefetch_distance=prefetch_distance)
    x0 = uniform(oracle_mod, m, n, 40)
    ws = [uniform(oracle_mod, m, m, 41 + l) * np.float32(0.125) for l in range(layers)]
    acts = [s.allocation(m * n * 4) for _ in range(layers + 1)]
    acts[0].write(np.asfortranarray(x0).T.copy())
    plans = []
    for l in range(layers):
        w = s.allocation(m * m * 4)
        w.write(np.asfortranarray(ws[l]).T.copy())
        plans.append(xv.GemmPlan(s, xv.matrix(w, m, m, m), xv.matrix(acts[l], m, n, m),
                                 xv.matrix(acts[l + 1], m, n, m)))
    plan_info = plans[0].info()
    assert plan_info.tile_count > 1
    gate = threading.Event()
    scratch = s.allocation(4 * KiB)

    def hold(_view):
        gate.wait(30)

    t0 = s.telemetry()
    held = s.transaction([xv.access(scratch, 0, 4 * KiB)], hold)
    ops = [p.submit() for p in plans]
    if cancel_last:
        assert ops[-1].cancel() == abi.SUCCESS
    gate.set()
    st, _ = held.wait()
    assert st == abi.SUCCESS
    held.release()
    for i, op in enumerate(ops):
        st, info = op.wait()
        assert st == abi.SUCCESS
        expect = abi.CANCELLED if cancel_last and i == len(ops) - 1 else abi.SUCCESS
        assert info.result == expect, (i, info.result)
        op.release()
    t1 = s.telemetry()
    done = layers - 1 if cancel_last else layers
    out = [np.asfortranarray(a.read(dtype=np.float32).reshape(n, m).T) for a in acts[:done + 1]]
    for p in plans:
        p.release()
    s.close()
    t = s.telemetry()
    assert t.mappings == t.unmaps == t.set_access_calls
    assert t.physical_handles_created == t.physical_handles_released
    assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
    assert t.resident_bytes == 0
    s.release()
    delta = {f: getattr(t1, f) - getattr(t0, f)
             for f in ("bytes_h2d", "bytes_d2h", "cache_hits", "cache_misses",
                       "writebacks_completed", "dirty_evictions")}
    return out, ws, delta, plan_info


def test_carried_fills_keep_results_and_bytes(sim, oracle_mod):
    layers = 4
    plain, ws, d0, info = run_chain(sim, oracle_mod, prefetch_distance=0, layers=layers)
    carried, _, d1, _ = run_chain(sim, oracle_mod, prefetch_distance=2, layers=layers)
    # Same launches on the same bytes: identical results, layer by layer.
    for a, b in zip(plain, carried):
        assert np.array_equal(a, b)
    # And each layer within the FP64 bound of the input it consumed.
    for l, w in enumerate(ws):
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(w), np.asfortranarray(carried[l]))
        bad, _, _ = oracle_mod.check_bound(carried[l + 1], w.shape[1], ref, absab)
        assert bad == 0, l
    # Carried panels are the ones the next operation loads first anyway: no
    # extra H2D bytes and no extra misses, only hits where the next operation
    # finds its first panels already filled.
    assert d1["bytes_h2d"] == d0["bytes_h2d"]
    assert d1["cache_misses"] == d0["cache_misses"]
    # Geometry of each layer (16 KiB frames): 64 x 40 C tiles, 64-deep K panels,
    # so 2 tiles x 2 K panels = 4 launches, each with its own W panel, all four
    # inside the next operation's first lookahead window (14 frames: lookahead 3).
    # The B panels of the next layer are this layer's output: its C tiles, the
    # very same rectangles, still cached (dirty) from this layer, so there is
    # nothing to carry for them. Hence exactly 4 carried panels per boundary.
    assert (info.tile_m, info.tile_n, info.tile_k, info.tile_count) == (64, 40, 64, 4)
    assert d1["cache_hits"] - d0["cache_hits"] == (layers - 1) * 4
    # Write-backs are the cache's business (activations stay cached, dirty, and
    # are written back when the pool needs their frames, which carrying can
    # change): at most every activation once, before the final reads.
    act_bytes = layers * 96 * 40 * 4
    assert d0["bytes_d2h"] <= act_bytes and d1["bytes_d2h"] <= act_bytes
    assert d1["dirty_evictions"] <= d1["writebacks_completed"]


def test_carry_into_a_cancelled_operation(sim, oracle_mod):
    """The last GEMM is cancelled while queued: the fills carried for it stay
    cached, unused, and the session still tears down balanced."""
    out, ws, _, _ = run_chain(sim, oracle_mod, prefetch_distance=2, cancel_last=True)
    for l in range(len(out) - 1):
        ref, absab = oracle_mod.sgemm_f64(np.asfortranarray(ws[l]), np.asfortranarray(out[l]))
        bad, _, _ = oracle_mod.check_bound(out[l + 1], ws[l].shape[1], ref, absab)
        assert bad == 0, l


def test_carried_frames_can_be_evicted_by_a_later_operation(sim, oracle_mod):
    """The GEMM a fill was carried for is cancelled; the next operation, a
    transaction whose working set needs every frame, must be able to evict the
    carried entries (their reuse waits for the fill, like any other frame's)."""
    frames, frame = 14, 16 * KiB
    s = xv.Session(sim, chunk_size_bytes=frame, cache_target_bytes=frames * frame,
                   workspace_cap_bytes=0, device_headroom_bytes=0, prefetch_distance=2)
    try:
        m, n = 96, 40
        x = s.allocation(m * n * 4)
        x.write(np.asfortranarray(uniform(oracle_mod, m, n, 50)).T.copy())
        ys = [s.allocation(m * n * 4) for _ in range(2)]
        plans = []
        for l in range(2):
            w = s.allocation(m * m * 4)
            w.write(np.asfortranarray(uniform(oracle_mod, m, m, 51 + l)).T.copy())
            plans.append(xv.GemmPlan(s, xv.matrix(w, m, m, m), xv.matrix(x, m, n, m),
                                     xv.matrix(ys[l], m, n, m)))
        big = s.allocation(frames * frame)
        big.write(np.arange(frames * frame // 4, dtype=np.float32))
        gate = threading.Event()
        scratch = s.allocation(4 * KiB)

        def hold(_view):
            gate.wait(30)

        held = s.transaction([xv.access(scratch, 0, 4 * KiB)], hold)
        first = plans[0].submit()
        second = plans[1].submit()
        seen = []
        whole = s.transaction([xv.access(big, 0, frames * frame)],
                              lambda view: seen.append(len(view.ranges)))
        assert second.cancel() == abi.SUCCESS
        gate.set()
        results = []
        for op in (held, first, second, whole):
            st, info = op.wait()
            assert st == abi.SUCCESS
            results.append((info.result, op.error().message))
            op.release()
        assert [r for r, _ in results] == [abi.SUCCESS, abi.SUCCESS, abi.CANCELLED, abi.SUCCESS], \
            results
        assert seen == [1]
        for p in plans:
            p.release()
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps and t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        s.release()
