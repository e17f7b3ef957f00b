"""Seeded random GEMMs through the C ABI on the MI355X, every element checked.

Each case draws m, n, k, the N/T forms, the storage layout of A, B and C
(row-major C exercises the operand swap), leading-dimension padding, alpha and
beta, and a cache configuration: resident (whole operands in one frame) or
out of core (small frames, so the planner tiles C and splits K and the panels
stream through a few frames). A quarter of the cases are large enough that
their launches run a 256 x 256 kernel (ragged ones of more than one round of
tiles as an edge split: ring interior, strips on the 256 x 128 kernel, and
with K not a multiple of 8 possibly a K remainder); the rest run the 256 x
128 kernel,
many with ragged edges in every dimension. Six more cases are N/T with m and n
multiples of 256, so their large launches run the barrier-free N/T kernel, and
six are N/N, T/N or T/T with such m and n and K a multiple of 8 (the
barrier-free kernel of those forms). With beta = 0, C is filled with NaN
first (it must never be read).

Every element is compared with the FP64 oracle (the reference's CPU GEMM,
examples/preview-gemm/main.cpp:107-119) under
|C - C_ref| <= 4*K*2^-24*(|alpha|(|A||B|)_ij + |beta*C0_ij|)."""
import numpy as np
import pytest

import xvram_amd as xv
from xvram_amd import abi

from gemm_cases import Problem, uniform

pytestmark = pytest.mark.gpu

MiB = 1 << 20
OPS = [(abi.OP_N, abi.OP_N), (abi.OP_N, abi.OP_T), (abi.OP_T, abi.OP_N), (abi.OP_T, abi.OP_T)]


def make_cases(count=24, seed=2026):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        wide = i % 4 == 0
        resident = rng.random() < 0.4
        if wide:
            # 256 x 256 kernel; out of core: 64 MiB frames, 4096 x 4096 C tiles + ragged edges
            m, n = (int(v) for v in rng.integers(4097, 4700, 2))
            k = int(rng.integers(1, 600))
            cache = (0, 0) if resident else (64, 12)
        elif resident:
            m, n = (int(v) for v in rng.integers(1, 1400, 2))
            k = int(rng.integers(1, 2500))
            cache = (0, 0)
        else:
            # 2 MiB frames; A alone exceeds one, so the planner must tile
            m, n = int(rng.integers(520, 1400)), int(rng.integers(1, 1400))
            k = int(rng.integers(1030, 2500))
            cache = (2, 10)
        cases.append(dict(
            m=m, n=n, k=k, ops=OPS[int(rng.integers(0, 4))],
            layouts=tuple(int(v) for v in rng.integers(0, 2, 3)),
            ld_pad=tuple(int(v) for v in rng.integers(0, 8, 3)),
            alpha=float(rng.choice([1.0, -0.75, 2.5])), beta=float(rng.choice([0.0, 1.0, 0.5])),
            cache=cache,  # (frame MiB, frames); (0, 0) = resident, one frame per operand
            seed=1000 + 3 * i))
    return cases


def make_ring_cases(count=6, seed=2027):
    """N/T with column-major storage, m and n multiples of 256 from 4096 and K a
    multiple of 4: the 4096 x 4096 (and resident) launches run the barrier-free
    kernel, the narrower edge launches of the out-of-core cases the others."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        resident = i % 2 == 0
        cases.append(dict(
            m=256 * int(rng.integers(16, 21)), n=256 * int(rng.integers(16, 21)),
            k=4 * int(rng.integers(1, 300)), ops=(abi.OP_N, abi.OP_T), layouts=(1, 1, 1),
            ld_pad=tuple(int(v) for v in rng.integers(0, 8, 3)),
            alpha=float(rng.choice([1.0, -0.75, 2.5])), beta=float(rng.choice([0.0, 1.0, 0.5])),
            cache=(0, 0) if resident else (64, 12), seed=5000 + 3 * i))
    return cases


def make_ring8_cases(count=6, seed=2028):
    """N/N, T/N and T/T with m and n multiples of 256 from 4096 and K a multiple
    of 8, every storage layout (a row-major C turns the product into its
    transpose, so the canonical form of a case may be any of the four): the
    4096 x 4096 (and resident) launches run a barrier-free kernel, mostly
    sgemm_ring8_kernel."""
    rng = np.random.default_rng(seed)
    forms = [OPS[0], OPS[2], OPS[3]]
    cases = []
    for i in range(count):
        resident = i % 2 == 0
        cases.append(dict(
            m=256 * int(rng.integers(16, 21)), n=256 * int(rng.integers(16, 21)),
            k=8 * int(rng.integers(1, 150)), ops=forms[i % 3],
            layouts=tuple(int(v) for v in rng.integers(0, 2, 3)),
            ld_pad=tuple(int(v) for v in rng.integers(0, 8, 3)),
            alpha=float(rng.choice([1.0, -0.75, 2.5])), beta=float(rng.choice([0.0, 1.0, 0.5])),
            cache=(0, 0) if resident else (64, 12), seed=7000 + 3 * i))
    return cases


CASES = make_cases() + make_ring_cases() + make_ring8_cases()


def case_id(c):
    kind = "resident" if c["cache"][0] == 0 else f"{c['cache'][1]}x{c['cache'][0]}MiB"
    return (f"{c['m']}x{c['n']}x{c['k']}-{'NT'[c['ops'][0]]}{'NT'[c['ops'][1]]}-"
            f"{''.join('RC'[v] for v in c['layouts'])}-a{c['alpha']}-b{c['beta']}-{kind}")


@pytest.fixture(scope="module")
def lib():
    return xv.load()


@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_random_gemm(lib, oracle_mod, case):
    m, n, k = case["m"], case["n"], case["k"]
    seed = case["seed"]
    a_op = uniform(oracle_mod, m, k, seed)
    b_op = uniform(oracle_mod, k, n, seed + 1)
    c0 = uniform(oracle_mod, m, n, seed + 2)
    prob = Problem(a_op, b_op, c0, op_a=case["ops"][0], op_b=case["ops"][1],
                   layouts=case["layouts"], alpha=case["alpha"], beta=case["beta"],
                   ld_pad=case["ld_pad"])
    frame_mib, frames = case["cache"]
    if frame_mib == 0:
        s = xv.Session(lib, chunk_size_bytes=256 * MiB)
    else:
        s = xv.Session(lib, chunk_size_bytes=frame_mib * MiB,
                       cache_target_bytes=frames * frame_mib * MiB + 4 * MiB)
    try:
        out = prob.run(s, c_fill=np.float32(np.nan) if case["beta"] == 0.0 else None)
        info = prob.plan_info
    finally:
        s.close()
        t = s.telemetry()
        assert t.mappings == t.unmaps == t.set_access_calls
        assert t.physical_handles_created == t.physical_handles_released
        assert t.unsafe_transitions == 0 and t.unsafe_remaps == 0
        s.release()
    if frame_mib:
        assert info.tile_count > 1, "an out-of-core case must tile"
    ref, absab = prob.reference(oracle_mod)
    bad, max_err, ratio = oracle_mod.check_bound(out, k, ref, absab)
    print(f"{case_id(case)}: {info.tile_count} launches of {info.tile_m}x{info.tile_n}x"
          f"{info.tile_k}, violations={bad} max_err={max_err:.3e} err/bound={ratio:.3e}",
          flush=True)
    assert np.isfinite(out).all()
    assert bad == 0
