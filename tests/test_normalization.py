"""Access normalisation and the entry-state table of the runtime (pure host
logic, exported by the hostsim library for tests), pinned by the reference's
own known-answer tests (tests/unit/residency_core_tests.cpp:38-147), by the
answers of the reference's compiled core.cpp recorded in
tests/golden/reference_outputs.json, and, where the reference tree is mounted,
by a differential test against that compiled code (oracle/_ref)."""
import ctypes

import pytest

import generators
import xvram_amd as xv
from generators import R, RW, WO, normalize

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
    generators.declare_normalize(lib.xvram_hostsim_normalize)
    return lib


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


def check_state_table(sim, table):
    diff = set()
    for a in range(len(STATES)):
        for b in range(len(STATES)):
            mine = sim.xvram_hostsim_legal_transition(a, b)
            if mine != table[a][b]:
                diff.add((a, b))
                assert mine == 1 and table[a][b] == 0
    assert diff == EXTRA_EDGES


def test_state_table_matches_recorded_reference(sim):
    check_state_table(sim, generators.reference_outputs("state_table"))


def test_state_table_matches_reference(sim, oracle_mod):
    ref = oracle_mod.ref_lib()
    if ref is None:
        pytest.skip("reference tree not built into oracle/_ref")
    ref.ref_legal_transition.argtypes = [ctypes.c_int, ctypes.c_int]
    table = [[ref.ref_legal_transition(a, b) for b in range(len(STATES))] for a in range(len(STATES))]
    assert table == generators.reference_outputs("state_table")
    check_state_table(sim, table)


NORMALIZATION_OUTCOMES = {"ok", "unknown_allocation", "zero_length", "range_overflow",
                          "range_out_of_bounds", "invalid_access_mode"}


def test_normalization_matches_recorded_reference(sim):
    cases = generators.normalization_cases(1000, 2024)
    want = generators.reference_outputs("normalization", cases)
    outcomes = set()
    for case, theirs in zip(cases, want):
        mine = generators.as_json(normalize(sim.xvram_hostsim_normalize, *case))
        assert mine == theirs, case
        outcomes.add(mine if isinstance(mine, str) else "ok")
    assert outcomes >= NORMALIZATION_OUTCOMES


def test_normalization_matches_reference(sim, oracle_mod):
    ref = oracle_mod.ref_lib()
    if ref is None:
        pytest.skip("reference tree not built into oracle/_ref")
    generators.declare_normalize(ref.ref_normalize)
    outcomes = set()
    for allocs, ranges, chunk in generators.normalization_cases(4000, 2024):
        mine = normalize(sim.xvram_hostsim_normalize, allocs, ranges, chunk)
        theirs = normalize(ref.ref_normalize, allocs, ranges, chunk)
        assert mine == theirs, (allocs, ranges, chunk)
        outcomes.add(mine if isinstance(mine, str) else "ok")
    assert outcomes >= NORMALIZATION_OUTCOMES
