"""Access normalisation and the entry-state table of the runtime (pure host
logic, exported by the hostsim library for tests), pinned by the reference's
own known-answer tests (tests/unit/residency_core_tests.cpp:38-147) and, where
the reference tree is mounted, by a differential test against the reference's
compiled core.cpp (oracle/_ref)."""
import ctypes
import random

import numpy as np
import pytest

import xvram_amd as xv

U64 = ctypes.c_uint64
R, RW, WO = 0, 1, 2
STATES = ["host_clean", "prefetch_queued", "mapping", "h2d_in_flight", "resident_clean",
          "resident_dirty", "writeback_queued", "d2h_in_flight", "evicting", "poisoned"]
S = {name: i for i, name in enumerate(STATES)}
# This design's one extra edge: a failed operation's dirty entry is discarded
# (the host copy stays authoritative) instead of being poisoned.
EXTRA_EDGES = {(S["resident_dirty"], S["evicting"])}


@pytest.fixture(scope="module")
def sim():
    lib = xv.load(hostsim=True).dll
    lib.xvram_hostsim_legal_transition.argtypes = [ctypes.c_int, ctypes.c_int]
    lib.xvram_hostsim_legal_transition.restype = ctypes.c_int
    _declare(lib.xvram_hostsim_normalize)
    return lib


def _declare(fn):
    p = ctypes.POINTER(U64)
    fn.argtypes = [p, U64, p, U64, U64, p, p, p, p, ctypes.c_char_p, U64]
    fn.restype = ctypes.c_int


def normalize(fn, allocs, ranges, chunk):
    a = np.array([v for pair in allocs for v in pair] or [0], dtype=np.uint64)
    r = np.array([v for q in ranges for v in q] or [0], dtype=np.uint64)
    cap = 4 * len(ranges) + 64
    out_r = np.zeros(4 * cap, np.uint64)
    out_c = np.zeros(5 * 64 * cap, np.uint64)
    n_r, n_c = U64(cap), U64(64 * cap)
    err = ctypes.create_string_buffer(64)
    ptr = lambda x: x.ctypes.data_as(ctypes.POINTER(U64))
    rc = fn(ptr(a), len(allocs), ptr(r), len(ranges), chunk, ptr(out_r), ctypes.byref(n_r),
            ptr(out_c), ctypes.byref(n_c), err, 64)
    assert rc in (0, 1), rc
    if rc == 1:
        return err.value.decode()
    rng = [tuple(int(v) for v in out_r[4 * i:4 * i + 4]) for i in range(n_r.value)]
    chk = [tuple(int(v) for v in out_c[5 * i:5 * i + 5]) for i in range(n_c.value)]
    return rng, chk


def test_reference_access_plan_kats(sim):
    """residency_core_tests.cpp:38-122 with the reference's 8-byte chunks."""
    first, second = 1, 2
    layouts = [(second, 8), (first, 20)]
    ranges = [(first, 0, 16, WO), (first, 4, 4, R), (first, 16, 4, WO), (second, 0, 4, WO),
              (second, 4, 4, WO)]
    got, chunks = normalize(sim.xvram_hostsim_normalize, layouts, ranges, 8)
    assert got == [(first, 0, 4, WO), (first, 4, 4, RW), (first, 8, 12, WO), (second, 0, 8, WO)]
    # (id, index, valid bytes, requires_h2d, marks_dirty)
    assert chunks == [(first, 0, 8, 1, 1), (first, 1, 8, 0, 1), (first, 2, 4, 0, 1),
                      (second, 0, 8, 0, 1)]
    got, chunks = normalize(sim.xvram_hostsim_normalize, layouts, [(first, 2, 4, WO)], 8)
    assert chunks == [(first, 0, 8, 1, 1)]
    f = sim.xvram_hostsim_normalize
    assert normalize(f, layouts, [(9, 0, 1, R)], 8) == "unknown_allocation"
    assert normalize(f, layouts, [(first, 0, 0, R)], 8) == "zero_length"
    assert normalize(f, layouts, [(first, (1 << 64) - 2, 4, R)], 8) == "range_overflow"
    assert normalize(f, layouts, [(first, 19, 2, R)], 8) == "range_out_of_bounds"
    assert normalize(f, layouts, [(first, 0, 1, 77)], 8) == "invalid_access_mode"


def test_reference_state_machine_kats(sim):
    """residency_core_tests.cpp:126-147."""
    legal = lambda a, b: sim.xvram_hostsim_legal_transition(S[a], S[b]) == 1
    path = ["host_clean", "mapping", "resident_clean", "resident_dirty", "writeback_queued",
            "d2h_in_flight", "resident_clean"]
    for a, b in zip(path, path[1:]):
        assert legal(a, b), (a, b)
    assert not legal("resident_clean", "host_clean")
    assert legal("resident_clean", "poisoned")
    assert not legal("poisoned", "host_clean")
    assert legal("host_clean", "mapping") and legal("mapping", "host_clean")


def test_state_table_matches_reference(sim, oracle_mod):
    ref = oracle_mod.ref_lib()
    if ref is None:
        pytest.skip("reference tree not built into oracle/_ref")
    ref.ref_legal_transition.argtypes = [ctypes.c_int, ctypes.c_int]
    diff = set()
    for a in range(len(STATES)):
        for b in range(len(STATES)):
            mine = sim.xvram_hostsim_legal_transition(a, b)
            theirs = ref.ref_legal_transition(a, b)
            if mine != theirs:
                diff.add((a, b))
                assert mine == 1 and theirs == 0
    assert diff == EXTRA_EDGES


def random_case(rng: random.Random):
    n_alloc = rng.randint(1, 3)
    ids = rng.sample(range(1, 8), n_alloc)
    allocs = [(i, rng.choice([1, 7, 8, 9, 20, 33, 64, 100])) for i in ids]
    ranges = []
    for _ in range(rng.randint(1, 6)):
        aid, size = rng.choice(allocs)
        roll = rng.random()
        if roll < 0.03:
            ranges.append((rng.choice([99, 0]), 0, 1, R))
        elif roll < 0.06:
            ranges.append((aid, rng.randrange(size), 0, R))
        elif roll < 0.08:
            ranges.append((aid, (1 << 64) - rng.randint(1, 3), rng.randint(4, 9), R))
        elif roll < 0.11:
            ranges.append((aid, rng.randrange(size), size, R))
        elif roll < 0.13:
            ranges.append((aid, 0, 1, rng.choice([3, 7])))
        else:
            off = rng.randrange(size)
            ranges.append((aid, off, rng.randint(1, size - off), rng.choice([R, RW, WO])))
    return allocs, ranges, rng.choice([1, 3, 4, 8, 16])


def test_normalization_matches_reference(sim, oracle_mod):
    ref = oracle_mod.ref_lib()
    if ref is None:
        pytest.skip("reference tree not built into oracle/_ref")
    _declare(ref.ref_normalize)
    rng = random.Random(2024)
    outcomes = set()
    for _ in range(4000):
        allocs, ranges, chunk = random_case(rng)
        mine = normalize(sim.xvram_hostsim_normalize, allocs, ranges, chunk)
        theirs = normalize(ref.ref_normalize, allocs, ranges, chunk)
        assert mine == theirs, (allocs, ranges, chunk)
        outcomes.add(mine if isinstance(mine, str) else "ok")
    assert outcomes >= {"ok", "unknown_allocation", "zero_length", "range_overflow",
                        "range_out_of_bounds", "invalid_access_mode"}
