"""Seeded random shapes across the launch rules, on the MI355X through the C
ABI (the extension's sgemm_device on device memory), every element checked.

The shapes are drawn so that each of the dispatch rules of sgemm_launch.hpp
fires several times: split K on the ring kernels and on the 256 x 128 kernel
(fewer tiles than CUs, one or two rounds of ranges), the tail split (interior
launches of at least 256 tiles whose last round would leave CUs idle), the
edge split (ragged launches of at least 256 tiles: interior, right strip,
bottom strip) and the whole ragged launch on the ring kernels' edge instances
(6981 x 4328 x 3928 here), in random N/T forms, with K a multiple of 8 and,
for some, not.
Operands are the analytic pattern (examples' gemm_bench pattern: exact in FP32
for these K), so every element of C must equal its closed form bit for bit,
whichever split, order of ranges or part computed it."""
import ctypes

import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from test_gpu_sgemm_device import FORMS, Hip, desc_for, padded
from test_gpu_tail_split import pattern_stored, synth  # noqa: F401  (fixture)

pytestmark = pytest.mark.gpu


def log(msg):
    print(f"[dispatch] {msg}", flush=True)


def make_cases(seed=4242):
    rng = np.random.default_rng(seed)
    cases = []
    kinds = ["small", "small", "narrow", "narrow", "tail", "tail", "edge", "edge", "edge", "edge"]
    for i, kind in enumerate(kinds):
        if kind == "small":     # interior, fewer tiles than CUs: ring or 256 x 128 split
            m, n = (256 * int(v) for v in rng.integers(2, 12, 2))
            k = 8 * int(rng.integers(64, 1024))
        elif kind == "narrow":  # ragged, fewer than 256 tiles: 256 x 128 split
            m, n = (int(v) for v in rng.integers(300, 3500, 2))
            k = int(rng.integers(300, 6000))
        elif kind == "tail":    # interior, 257..400 tiles
            tm = int(rng.integers(16, 21))
            tn = int(rng.integers(max(16, -(-257 // tm)), 21))
            m, n = 256 * tm, 256 * tn
            k = 8 * int(rng.integers(128, 512))
        else:                   # ragged, at least 256 tiles
            tm, tn = (int(v) for v in rng.choice([16, 19, 24, 27], 2))
            m, n = (256 * t + int(rng.integers(1, 256)) for t in (tm, tn))
            k = 8 * int(rng.integers(256, 640))
        form = sorted(FORMS)[int(rng.integers(0, 4))]
        if kind == "edge" and i == len(kinds) - 1:
            k, form = k + 4, "NT"  # K a multiple of 4 only: N/T takes the edge split
        cases.append((kind, m, n, k, form))
    return cases


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.mark.parametrize("kind,m,n,k,form", make_cases(),
                         ids=[f"{c[0]}-{c[1]}x{c[2]}x{c[3]}-{c[4]}" for c in make_cases()])
def test_dispatch_pattern_exact(lib, synth, oracle_mod, kind, m, n, k, form):
    ops = FORMS[form]
    a_st = pattern_stored(synth, "a", *((m, k) if ops[0] == abi.OP_N else (k, m)),
                          ops[0] == abi.OP_T)
    b_st = pattern_stored(synth, "b", *((k, n) if ops[1] == abi.OP_N else (n, k)),
                          ops[1] == abi.OP_T)
    a_flat, lda = padded(a_st)
    b_flat, ldb = padded(b_st)
    c_flat, ldc = padded(np.full((m, n), np.nan, np.float32))  # beta 0: C is never read
    hip = Hip()
    pa, pb, pc = hip.alloc(a_flat.nbytes), hip.alloc(b_flat.nbytes), hip.alloc(c_flat.nbytes)
    s = hip.stream()
    try:
        hip.put(pa, a_flat)
        hip.put(pb, b_flat)
        hip.put(pc, c_flat)
        d = desc_for((pa, pb, pc), m, n, k, ops, (lda, ldb, ldc))
        assert lib.ext.sgemm_device(ctypes.byref(d), ctypes.c_void_p(s)) == abi.SUCCESS
        hip.sync(s)
        got = hip.get(pc, c_flat.size).reshape(n, ldc)[:, :m].T
    finally:
        for p in (pa, pb, pc):
            hip.free(p)
        hip.close()
    expect = oracle_mod.pattern_expected_matrix(m, n, k).astype(np.float32)
    bad = int(np.count_nonzero(got != expect))
    log(f"{kind} {m}x{n}x{k} {form}: {bad} of {m * n} differ")
    assert bad == 0
