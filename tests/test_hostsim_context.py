"""XVRAM_CONTEXT_ATTACH_CURRENT on the host simulation: the session runs on the
device current on the creating thread and ignores device_ordinal; with no
device current, creation fails with INVALID_ARGUMENT (reference
src/sdk/runtime.cpp:1369-1383, src/residency/runtime.cpp:230-245)."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

KiB = 1 << 10


@pytest.fixture()
def sim():
    lib = xv.load(hostsim=True)
    lib.dll.xvram_hostsim_reset()
    lib.dll.xvram_hostsim_last_init_ordinal.restype = ctypes.c_int
    yield lib
    lib.dll.xvram_hostsim_reset()


def config(**extra):
    cfg = dict(chunk_size_bytes=64 * KiB, cache_target_bytes=8 * 64 * KiB, workspace_cap_bytes=0,
               device_headroom_bytes=0)
    cfg.update(extra)
    return cfg


def small_gemm(session):
    m = n = k = 40
    rng = np.random.default_rng(3)
    a_h = rng.integers(-3, 4, (m, k)).astype(np.float32)
    b_h = rng.integers(-3, 4, (k, n)).astype(np.float32)
    a = session.allocation(a_h.nbytes)
    b = session.allocation(b_h.nbytes)
    c = session.allocation(m * n * 4)
    a.write(np.asfortranarray(a_h).T.copy())
    b.write(np.asfortranarray(b_h).T.copy())
    plan = xv.GemmPlan(session, xv.matrix(a, m, k, m), xv.matrix(b, k, n, k), xv.matrix(c, m, n, m))
    plan.execute()
    out = c.read(dtype=np.float32).reshape(n, m).T
    plan.release()
    np.testing.assert_array_equal(out, a_h @ b_h)


def test_attach_uses_the_current_device_not_the_ordinal(sim):
    sim.dll.xvram_hostsim_set_devices(3, 2)
    # device_ordinal names a device that does not exist: attach mode must not use it.
    with xv.Session(sim, **config(context_mode=abi.CONTEXT_ATTACH_CURRENT,
                                  device_ordinal=7)) as s:
        assert sim.dll.xvram_hostsim_last_init_ordinal() == 2
        small_gemm(s)


def test_isolated_uses_the_ordinal(sim):
    sim.dll.xvram_hostsim_set_devices(3, 2)
    with xv.Session(sim, **config(context_mode=abi.CONTEXT_ISOLATED, device_ordinal=1)) as s:
        assert sim.dll.xvram_hostsim_last_init_ordinal() == 1
        small_gemm(s)
    with pytest.raises(xv.XvramError) as err:
        xv.Session(sim, **config(context_mode=abi.CONTEXT_ISOLATED, device_ordinal=7))
    assert err.value.status == abi.CUDA_ERROR


def test_attach_with_no_current_device_is_invalid(sim):
    sim.dll.xvram_hostsim_set_devices(1, -1)
    with pytest.raises(xv.XvramError) as err:
        xv.Session(sim, **config(context_mode=abi.CONTEXT_ATTACH_CURRENT))
    assert err.value.status == abi.INVALID_ARGUMENT
    assert sim.dll.xvram_hostsim_last_init_ordinal() == -1  # no worker set up


def test_attach_default_device(sim):
    with xv.Session(sim, **config(context_mode=abi.CONTEXT_ATTACH_CURRENT)) as s:
        assert sim.dll.xvram_hostsim_last_init_ordinal() == 0
        small_gemm(s)
