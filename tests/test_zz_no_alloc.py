"""sgemm_device_no_alloc (extension table) on the MI355X: the allocation-free
variant of sgemm_device, whose split-K partials go to the library's static
per-GPU scratch instead of an allocation. Through the C ABI, on two calls in a
row (the second with a smaller input, over what the first left in the
scratch), each against sgemm_device on the same inputs: the same split, so
the same bits, and within the FP64 bound
|C - C_ref| <= 4*K*2^-24*(|A||B|)_ij. After the first call (which loads the
scratch's code object on the GPU), calls leave the device's free memory
unchanged."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_sgemm_device import FORMS, Hip, desc_for, padded, stored

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[no_alloc] {msg}", flush=True)


@pytest.fixture(scope="module")
def lib():
    return xv.load()


def free_bytes(hip):
    free, total = ctypes.c_size_t(), ctypes.c_size_t()
    hip.ok(hip.rt.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)), "hipMemGetInfo")
    return free.value


def test_no_alloc_matches_sgemm_device(lib, oracle_mod):
    hip = Hip()
    s = hip.stream()
    try:
        # 16 tiles x 16 ranges on the ring kernels (64 MiB of partials), then
        # 16 tiles of 256 x 128 x 16 ranges (32 MiB) over what the first call
        # left there, then a ragged launch
        # (2 x 2 tiles of 256 x 128, 32 ranges, partials of leading dimension
        # 504), then config 2's shape (192 tiles of 256 x 128, 5 ranges: 117
        # MiB of partials, most of the 128 MiB scratch), then a tail split
        # (17 x 16 tiles: 16 rows unsplit, the last row in 5 ranges), then an
        # edge split (4100 x 4100: the 16 x 16 interior and two split strips).
        for call, (m, n, k, form, seed) in enumerate([(4096, 256, 4096, "NN", 601),
                                                      (1024, 512, 2048, "NT", 602),
                                                      (501, 200, 2048, "TN", 603),
                                                      (3001, 2047, 4099, "NN", 604),
                                                      (4352, 4096, 1024, "TT", 605),
                                                      (4100, 4100, 1024, "NT", 606)]):
            ops = FORMS[form]
            a_op = np.asfortranarray(oracle_mod.fill_uniform(m * k, seed).reshape(k, m).T)
            b_op = np.asfortranarray(oracle_mod.fill_uniform(k * n, seed + 1).reshape(n, k).T)
            a_flat, lda = stored(a_op, ops[0])
            b_flat, ldb = stored(b_op, ops[1])
            c_flat, ldc = padded(np.zeros((m, n), np.float32))
            pa, pb = hip.alloc(a_flat.nbytes), hip.alloc(b_flat.nbytes)
            pc_ref, pc = hip.alloc(c_flat.nbytes), hip.alloc(c_flat.nbytes)
            try:
                hip.put(pa, a_flat)
                hip.put(pb, b_flat)
                hip.put(pc_ref, c_flat)
                hip.put(pc, c_flat)
                ref_desc = desc_for((pa, pb, pc_ref), m, n, k, ops, (lda, ldb, ldc))
                assert lib.ext.sgemm_device(ctypes.byref(ref_desc), ctypes.c_void_p(s)) == \
                    abi.SUCCESS
                hip.sync(s)
                before = free_bytes(hip)
                desc = desc_for((pa, pb, pc), m, n, k, ops, (lda, ldb, ldc))
                assert lib.ext.sgemm_device_no_alloc(ctypes.byref(desc), ctypes.c_void_p(s)) == \
                    abi.SUCCESS
                hip.sync(s)
                after = free_bytes(hip)
                want = hip.get(pc_ref, c_flat.size).reshape(n, ldc)[:, :m].T
                got = hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T
            finally:
                for p in (pa, pb, pc_ref, pc):
                    hip.free(p)
            same = np.array_equal(got.view(np.uint32), want.view(np.uint32))
            ref, absab = oracle_mod.sgemm_f64(a_op, b_op)
            bad, _, ratio = oracle_mod.check_bound(np.asfortranarray(got), k, ref, absab)
            log(f"call {call}: {m}x{n}x{k} {form}: identical to sgemm_device {same}, "
                f"violations {bad}, err/bound {ratio:.3e}, free memory {before} -> {after}")
            assert same and bad == 0
            if call > 0:
                assert after == before
    finally:
        hip.close()
