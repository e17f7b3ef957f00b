"""Seeded input generators shared by the differential tests and by
make_golden.py (which records the reference's answers for them). Not a test
module. Each generator is deterministic for its seed; the recorded fixtures
also carry a digest of the generated inputs, so a change here (or in the RNG
streams underneath) fails loudly instead of comparing different inputs."""
from __future__ import annotations

import hashlib
import json
import random

import numpy as np

# Access modes (xvram_access_mode) and policy program opcodes / entry states
# as the hostsim and reference shims take them.
R, RW, WO = 0, 1, 2
INSERT, TOUCH, ERASE, SET, DROP, SELECT = range(6)
CLEAN, DIRTY, H2D = 4, 5, 3
NONE = (1 << 64) - 1


def digest(obj) -> str:
    return hashlib.sha256(json.dumps(obj, sort_keys=True, separators=(",", ":")).encode()).hexdigest()


def pattern_points(n: int = 2000, seed: int = 7):
    """(row, col, k) points for the analytic pattern."""
    rng = np.random.default_rng(seed)
    return [(int(r), int(c), int(k)) for r, c, k in zip(rng.integers(0, 10**6, n),
                                                        rng.integers(0, 10**6, n),
                                                        rng.integers(1, 10**7, n))]


def normalization_case(rng: random.Random):
    """One random access list: (allocations [(id, size)], ranges [(id, offset,
    length, mode)], chunk bytes), with a few invalid ranges mixed in."""
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


def normalization_cases(n: int = 4000, seed: int = 2024):
    rng = random.Random(seed)
    return [normalization_case(rng) for _ in range(n)]


def policy_program(rng: random.Random, length: int = 120):
    """A random command program for the victim-policy drivers."""
    cmds, seq, ids = [], 0, list(range(1, 9))
    for _ in range(length):
        r = rng.random()
        i = rng.choice(ids)
        seq += rng.choice([0, 1, 1, 2])
        if r < 0.25:
            cmds.append((INSERT, i, seq, int(rng.random() < 0.3), int(rng.random() < 0.2)))
        elif r < 0.45:
            cmds.append((TOUCH, i, seq, int(rng.random() < 0.2)))
        elif r < 0.5:
            cmds.append((ERASE, i))
        elif r < 0.75:
            cmds.append((SET, i, rng.choice([CLEAN, CLEAN, DIRTY, H2D]), int(rng.random() < 0.2),
                         int(rng.random() < 0.15), int(rng.random() < 0.1), int(rng.random() < 0.1)))
        elif r < 0.8:
            cmds.append((DROP, i))
        else:
            cmds.append((SELECT,))
    return cmds


def policy_programs(kind: int, n: int = 300):
    rng = random.Random(77 + kind)
    return [policy_program(rng) for _ in range(n)]


# Allocation sizes the validation cases draw from (allocation index 0..2).
VALIDATION_SIZES = [4096, 8192, 20000]
_ROW_MAJOR = 0


def validation_cases(n: int = 1500, seed: int = 2024):
    """Random GEMM descriptors. Each case: matrices [(allocation index, offset,
    rows, columns, ld, layout, element type)] for A, B, C, then op_a, op_b, the
    compute mode, beta. Shapes are made consistent most of the time so that
    every later validation rule is reached."""
    rng = np.random.default_rng(seed)
    cases = []
    for _ in range(n):
        ids = rng.integers(0, 3, 3)
        mats = []
        for slot in range(3):
            al = int(ids[slot])
            rows = int(rng.integers(1, 40))
            cols = int(rng.integers(1, 40))
            layout = int(rng.integers(0, 2))
            dtype = int(rng.choice([0, 1, 2, 2, 2, 3]))
            need = cols if layout == _ROW_MAJOR else rows
            ld = int(need + rng.integers(-2, 4)) if rng.random() < 0.9 else int(rng.integers(1, 1 << 33))
            ld = max(ld, 1)
            offset = [0, 0, 64, 1000, 4096, 30000, (1 << 64) - 8][int(rng.integers(0, 7))]
            mats.append([al, offset, rows, cols, ld, layout, dtype])
        op_a, op_b = int(rng.integers(0, 2)), int(rng.integers(0, 2))
        if rng.random() < 0.7:
            a = mats[0]
            m = a[3] if op_a else a[2]
            k = a[2] if op_a else a[3]
            nn = int(rng.integers(1, 40))
            mats[1][2], mats[1][3] = (nn, k) if op_b else (k, nn)
            mats[2][2], mats[2][3] = m, nn
            for slot in (1, 2):
                d = mats[slot]
                need = d[3] if d[5] == _ROW_MAJOR else d[2]
                if d[4] < need and rng.random() < 0.8:
                    d[4] = need
        compute = int(rng.integers(0, 4))
        beta = float(rng.choice([0.0, 0.5]))
        cases.append({"mats": mats, "op_a": op_a, "op_b": op_b, "compute": compute, "beta": beta})
    return cases


# ---- ctypes drivers shared by the tests and make_golden.py --------------------------------

import ctypes  # noqa: E402

U64 = ctypes.c_uint64


def declare_normalize(fn):
    p = ctypes.POINTER(U64)
    fn.argtypes = [p, U64, p, U64, U64, p, p, p, p, ctypes.c_char_p, U64]
    fn.restype = ctypes.c_int


def normalize(fn, allocs, ranges, chunk):
    """Runs one normalisation through `fn` (hostsim or reference shim): the
    error name, or (resolved ranges, chunk plans) as tuples."""
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


def declare_policy(fn):
    fn.argtypes = [ctypes.c_int, ctypes.POINTER(U64), U64, ctypes.POINTER(U64)]
    fn.restype = ctypes.c_int


def run_policy(fn, kind, cmds):
    """Runs a command program through `fn`; one output word per command."""
    words = []
    for c in cmds:
        words += list(c) + [0] * (7 - len(c))
    prog = np.array(words, dtype=np.uint64)
    out = np.zeros(len(cmds), dtype=np.uint64)
    assert fn(kind, prog.ctypes.data_as(ctypes.POINTER(U64)), len(cmds),
              out.ctypes.data_as(ctypes.POINTER(U64))) == 0
    return [int(v) for v in out]


class RefMatrix(ctypes.Structure):
    """The reference shim's matrix view (allocation id, bytes, offset, rows,
    columns, ld, layout, element type)."""
    _fields_ = [("allocation_id", ctypes.c_uint64), ("allocation_bytes", ctypes.c_uint64),
                ("offset_bytes", ctypes.c_uint64), ("rows", ctypes.c_uint64),
                ("columns", ctypes.c_uint64), ("leading_dimension", ctypes.c_uint64),
                ("layout", ctypes.c_uint32), ("element_type", ctypes.c_uint32)]


def ref_matrix(mat):
    al, offset, rows, cols, ld, layout, dtype = mat
    return RefMatrix(al + 1, VALIDATION_SIZES[al], offset, rows, cols, ld, layout, dtype)


def reference_compute_mode(compute: int, a_type: int) -> int:
    """The reference's compute-mode resolution (src/sdk/runtime.cpp:119-135):
    AUTO -> FP64 for FP64 data, strict for FP16/BF16, TF32 for FP32; the shim
    takes 0 = strict, 1 = TF32, 2 = FP64."""
    if compute == 0:
        return 2 if a_type == 3 else (0 if a_type in (0, 1) else 1)
    return {1: 0, 2: 1, 3: 2}[compute]


# ---- recorded reference answers -------------------------------------------------------------

import os  # noqa: E402

FIXTURE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "reference_outputs.json")


def reference_outputs(section: str, inputs=None):
    """The recorded reference answers of one fixture section. With `inputs`,
    first checks that they are the inputs the answers were recorded for and
    returns the answers alone."""
    with open(FIXTURE) as f:
        data = json.load(f)[section]
    if inputs is None:
        return data
    assert data["count"] == len(inputs) and data["inputs_sha256"] == digest(inputs), (
        f"{section}: the generated inputs differ from the recorded ones "
        f"(regenerate with tests/golden/make_golden.py)")
    return data["outputs"]


def as_json(obj):
    """`obj` as it reads back from the fixture (tuples become lists)."""
    return json.loads(json.dumps(obj))
