#!/usr/bin/env python3
"""Records the reference's own answers for the differential tests into
reference_outputs.json (run here, where /root/reference is mounted; the GPU box
and any checkout without the reference tree then test against the fixture).

The answers come from the reference's sources compiled as they lie
(oracle/Makefile `ref` target -> oracle/_ref/libxvram_ref.so):
  src/gemm_bench/pattern.cpp   analytic pattern values and sums
  src/residency/core.cpp       entry-state transition table, access normalisation
  src/residency/policy.cpp     CLOCK and LRU victim choices
  src/gemm/planner.cpp         validate_problem
Inputs are the seeded generators of generators.py; the fixture stores each
input set's digest next to the outputs.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import ctypes
import json
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import generators as g  # noqa: E402
import oracle  # noqa: E402

OUT = os.path.join(HERE, "reference_outputs.json")
# Fixture sizes (the live differential tests may run more cases).
N_PATTERN, N_NORMALIZE, N_POLICY, N_VALIDATE = 1000, 1000, 150, 1500


def main() -> int:
    if not os.path.isdir("/root/reference"):
        print("the reference tree is not mounted: nothing to record", file=sys.stderr)
        return 1
    oracle.build(reference=True)
    ref = oracle.ref_lib()
    out = {"source": "reference sources compiled by oracle/Makefile (target ref)"}

    pts = g.pattern_points(N_PATTERN, 7)
    res = []
    e, p, q, pq = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    for row, col, k in pts:
        assert ref.ref_pattern_expected(row, col, k, ctypes.byref(e)) == 1
        ref.ref_pattern_sums(k, ctypes.byref(p), ctypes.byref(q), ctypes.byref(pq))
        res.append([ref.ref_pattern_a(row, k), ref.ref_pattern_b(k, col), e.value, p.value,
                    q.value, pq.value])
    out["pattern"] = {"seed": 7, "count": N_PATTERN, "inputs_sha256": g.digest(pts),
                      "outputs": res}

    ref.ref_legal_transition.argtypes = [ctypes.c_int, ctypes.c_int]
    out["state_table"] = [[ref.ref_legal_transition(a, b) for b in range(10)] for a in range(10)]

    g.declare_normalize(ref.ref_normalize)
    cases = g.normalization_cases(N_NORMALIZE, 2024)
    res = [g.normalize(ref.ref_normalize, *c) for c in cases]
    out["normalization"] = {"seed": 2024, "count": N_NORMALIZE, "inputs_sha256": g.digest(cases),
                            "outputs": res}

    g.declare_policy(ref.ref_policy_run)
    for kind, name in ((0, "policy_clock"), (1, "policy_lru")):
        progs = g.policy_programs(kind, N_POLICY)
        res = [[-1 if v == g.NONE else v for v in g.run_policy(ref.ref_policy_run, kind, prog)]
               for prog in progs]
        out[name] = {"seed": 77 + kind, "count": N_POLICY, "inputs_sha256": g.digest(progs),
                     "outputs": res}

    ref.ref_validate_problem.argtypes = [ctypes.POINTER(g.RefMatrix)] * 3 + [
        ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_double]
    cases = g.validation_cases(N_VALIDATE, 2024)
    res = []
    for c in cases:
        mats = [g.ref_matrix(m) for m in c["mats"]]
        rc = g.reference_compute_mode(c["compute"], c["mats"][0][6])
        res.append(ref.ref_validate_problem(*(ctypes.byref(m) for m in mats), c["op_a"], c["op_b"],
                                            rc, c["beta"]))
    out["validation"] = {"seed": 2024, "count": N_VALIDATE, "inputs_sha256": g.digest(cases),
                         "outputs": res}

    with open(OUT, "w") as f:
        json.dump(out, f, separators=(",", ":"))
        f.write("\n")
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")
    return 0


if __name__ == "__main__":
    sys.exit(main())
