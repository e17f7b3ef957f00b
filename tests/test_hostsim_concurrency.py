"""Several caller threads on one session (the ABI lets any thread call; every
device operation is serialised on the session worker; reference
src/sdk/runtime.cpp:857-930). Over libxvram_hostsim.so: four threads each
allocate, write, plan, submit, poll, cancel and wait on GEMMs of their own
while a fifth runs transactions and prefetches on other allocations. Every
completed GEMM must be within the FP64 bound, cancelled ones must report
CANCELLED without touching C, and the session must tear down balanced."""
import random
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


def test_threads_share_one_session(sim, oracle_mod):
    s = xv.Session(sim, chunk_size_bytes=16 * KiB, cache_target_bytes=24 * 16 * KiB,
                   workspace_cap_bytes=0, device_headroom_bytes=0)
    failures = []
    results = {"gemm": 0, "cancelled": 0, "transactions": 0}
    lock = threading.Lock()

    def gemm_worker(tid):
        rng = random.Random(100 + tid)
        try:
            for it in range(6):
                m, n, k = rng.randint(20, 120), rng.randint(20, 120), rng.randint(20, 160)
                a_op = uniform(oracle_mod, m, k, 1000 * tid + 3 * it)
                b_op = uniform(oracle_mod, k, n, 1000 * tid + 3 * it + 1)
                A, B, C = s.allocation(m * k * 4), s.allocation(k * n * 4), s.allocation(m * n * 4)
                A.write(a_op.T.copy())
                B.write(b_op.T.copy())
                C.write(np.full(m * n, 7.0, np.float32))
                plan = xv.GemmPlan(s, xv.matrix(A, m, k, m), xv.matrix(B, k, n, k),
                                   xv.matrix(C, m, n, m))
                op = plan.submit()
                cancelled = False
                if rng.random() < 0.3:
                    status = op.cancel()
                    assert status in (abi.SUCCESS, abi.BUSY), status
                op.poll()
                st, info = op.wait()
                assert st == abi.SUCCESS
                if info.result == abi.CANCELLED:
                    cancelled = True
                else:
                    assert info.result == abi.SUCCESS, op.error().message
                op.release()
                out = np.asfortranarray(C.read(dtype=np.float32).reshape(n, m).T)
                if cancelled:
                    assert (out == 7.0).all()
                else:
                    ref, absab = oracle_mod.sgemm_f64(a_op, b_op)
                    bad = oracle_mod.check_bound(out, k, ref, absab)[0]
                    assert bad == 0, (tid, it, bad)
                plan.release()
                for h in (A, B, C):
                    h.release()
                with lock:
                    results["cancelled" if cancelled else "gemm"] += 1
        except Exception as exc:  # reported by the main thread
            failures.append((tid, repr(exc)))

    def transaction_worker():
        try:
            big = s.allocation(6 * 16 * KiB)
            data = np.arange(6 * 16 * KiB // 4, dtype=np.float32)
            big.write(data)
            for it in range(12):
                off = (it % 4) * 16 * KiB
                if it % 3 == 0:
                    op = s.prefetch([xv.access(big, off, 32 * KiB)])
                else:
                    seen = []
                    op = s.transaction([xv.access(big, off, 32 * KiB)],
                                       lambda view: seen.append(view.ranges[0][2]))
                st, info = op.wait()
                assert st == abi.SUCCESS and info.result == abi.SUCCESS, op.error().message
                op.release()
                with lock:
                    results["transactions"] += 1
            assert np.array_equal(big.read(dtype=np.float32), data)
            big.release()
        except Exception as exc:
            failures.append(("tx", repr(exc)))

    threads = [threading.Thread(target=gemm_worker, args=(t,)) for t in range(4)]
    threads.append(threading.Thread(target=transaction_worker))
    for t in threads:
        t.start()
    for t in threads:
        t.join(120)
    try:
        assert not any(t.is_alive() for t in threads), "a caller thread did not finish"
        assert not failures, failures
        assert results["gemm"] + results["cancelled"] == 24
        assert results["transactions"] == 12
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps == t.set_access_calls
        assert t.physical_handles_created == t.physical_handles_released
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        # Evictions of dirty entries are a subset of the write-backs (reads of C
        # and close write back entries that stay cached).
        assert t.dirty_evictions <= t.writebacks_completed
        assert t.resident_bytes == 0
        assert t.resident_bytes == 0
        s.release()
